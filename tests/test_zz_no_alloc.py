"""The allocation-free layer entry point (dgm_megamoe_fused_launch_noalloc: the persistent kernel's
workspace in a file-scope device array instead of the caller's buffer) against the buffered entry
point dgm_megamoe_fused_launch on the same inputs, both through the C ABI: y, top-k, top-k
weights and recv stats bit for bit, on two calls in a row (the second with fewer tokens), for the
in-prologue selection (<= 8 tokens) and the selection launch (> 8 tokens), at the array's route
limit (512) for MXFP8 and NVFP4, and on eight seeded random shapes (every format, each of the
kernel's three (H, I), EP shares, top-1 to top-16); and its size limit, which is refused on the
host with a clear message."""
import ctypes

import numpy as np
import pytest
import torch

from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16

pytestmark = pytest.mark.gpu

H, I, TOPK = 3072, 1280, 8


def _weights(fmt, E_LOCAL):
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_mxfp4_fused as qf
    from hopper_megamoe_basedondeepgemm_amd import quantization_nvfp4 as qn
    from hopper_megamoe_basedondeepgemm_amd import quantization_qoq_fused as qq
    g = torch.Generator(device="cuda")
    g.manual_seed(1301)
    w1 = (torch.randn((E_LOCAL, 2 * I, H), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((E_LOCAL, H, I), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    if fmt == "qoq":
        return dgm.transform_qoq_weights_for_mega_moe_fused(qq.quantize_to_qoq(w1), qq.quantize_to_qoq(w2))
    if fmt == "nvfp4":
        return dgm.transform_nvfp4_weights_for_mega_moe_fused(qn.quantize_to_nvfp4(w1), qn.quantize_to_nvfp4(w2))
    return dgm.transform_mxfp4_weights_for_mega_moe_fused(qf.quantize_to_mxfp4(w1), qf.quantize_to_mxfp4(w2))


def _launch(entry, args):
    from hopper_megamoe_basedondeepgemm_amd import _lib
    return getattr(_lib.load(), entry)(ctypes.byref(args), _lib.stream())


@pytest.mark.parametrize("fmt,sizes,E,ep_size", [("mxfp8", (16, 5), 384, 8), ("qoq", (16, 5), 384, 8),
                                                   # the array's limit: 64 tokens x top-8 = 512 local routes
                                                   ("mxfp8", (64, 40), 48, 1), ("nvfp4", (64, 40), 48, 1)])
def test_noalloc_matches_buffered_entry_point(fmt, sizes, E, ep_size):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import _lib, mega
    e_local = E // ep_size
    t1, t2 = _weights(fmt, e_local)
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, max(sizes), TOPK, H, I, act_format=fmt, ep_size=ep_size,
                                                 ep_rank=1 % ep_size)
    rng = np.random.default_rng(1300)
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    for M in sizes:                        # two calls in a row, the second with fewer tokens
        print(f"no-alloc vs buffered: fmt={fmt} M={M} E={E} E_local={e_local} (EP rank {1 % ep_size} of {ep_size})",
              flush=True)
        x = bf16_cpu(randn_bf16(rng, (M, H))).cuda()
        dgm.fable_router_quant_topk_frontend(x, rw, buf, select_in_mega=True)
        out = {}
        for entry in ("dgm_megamoe_fused_launch", "dgm_megamoe_fused_launch_noalloc"):
            y = torch.full((M, H), 3.0, dtype=torch.bfloat16, device="cuda")
            stats = torch.zeros(e_local, dtype=torch.int32, device="cuda")
            args = mega._moe_args(y, t1, t2, buf, stats, 10.0, fmt=fmt)
            _lib.check(_launch(entry, args))
            torch.cuda.synchronize()
            assert buf.host_error() == 0 and buf.kernel_error() == 0
            out[entry] = (y.view(torch.int16).cpu(), stats.cpu(), buf.topk_idx[:M].cpu().clone(),
                          buf.topk_weights[:M].cpu().clone().view(torch.int32))
        a, b = out.values()
        for u, v in zip(a, b):
            assert torch.equal(u, v)
        assert int(a[1].sum()) > 0                 # some routes were local


def test_noalloc_size_limit():
    """More than 512 routes: refused on the host (no launch) with the array's limit named."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import _lib, mega
    M = 65                                         # 65 * 8 = 520 routes
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, 64, M, TOPK, 512, 256, act_format="mxfp4")
    w1 = (torch.zeros((64, 32, 4, 64, 16), dtype=torch.uint8, device="cuda"),
          torch.zeros((64, 32, 1, 64, 4), dtype=torch.uint8, device="cuda"), None)
    w2 = (torch.zeros((64, 32, 2, 64, 16), dtype=torch.uint8, device="cuda"),
          torch.zeros((64, 32, 1, 64, 4), dtype=torch.uint8, device="cuda"), None)
    y = torch.empty((M, 512), dtype=torch.bfloat16, device="cuda")
    args = mega._moe_args(y, w1, w2, buf, None, 10.0, fmt="mxfp4")
    st = _launch("dgm_megamoe_fused_launch_noalloc", args)
    assert st == -1
    assert b"num_tokens * topk must be <= 512" in _lib.load().dgm_last_error()


def _random_noalloc_cases(n=8, seed=2031):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        H_, I_ = [(512, 256), (1024, 512), (3072, 1280)][int(rng.integers(3))]
        fmt = ["mxfp4", "mxfp8", "qoq", "nvfp4"][i % 4]
        ep = [1, 2, 4][int(rng.integers(3))]
        e_local = int(rng.integers(2, 33))
        topk = int(rng.integers(1, min(16, e_local * ep) + 1))
        sizes = tuple(int(v) for v in rng.integers(1, 512 // topk + 1, 2))
        out.append((i, H_, I_, fmt, e_local * ep, ep, topk, sizes))
    return out


@pytest.mark.parametrize("case", _random_noalloc_cases(), ids=lambda c: f"case{c[0]}")
def test_noalloc_random_shapes(case):
    """Seeded random shapes on both entry points (each of the kernel's three shapes, every
    format, EP shares, top-1 to top-16, up to the array's 512 routes), two calls each: y,
    top-k and stats bit for bit."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import _lib, mega
    from tests.test_gpu_one_launch import weights_for
    i, H_, I_, fmt, E, ep, topk, sizes = case
    e_local = E // ep
    t1, t2 = weights_for(fmt, e_local, H_, I_, 1400 + i)
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, max(sizes), topk, H_, I_, act_format=fmt, ep_size=ep,
                                                 ep_rank=(i % ep))
    rng = np.random.default_rng(1410 + i)
    rw = bf16_cpu(randn_bf16(rng, (E, H_), 0.02)).cuda()
    for M in sizes:
        print(f"no-alloc random {i}: {fmt} H={H_} I={I_} M={M} E={E} local={e_local}@rank{i % ep} topk={topk}",
              flush=True)
        x = bf16_cpu(randn_bf16(rng, (M, H_))).cuda()
        dgm.fable_router_quant_topk_frontend(x, rw, buf, select_in_mega=bool(i % 2))
        out = {}
        for entry in ("dgm_megamoe_fused_launch", "dgm_megamoe_fused_launch_noalloc"):
            y = torch.full((M, H_), 3.0, dtype=torch.bfloat16, device="cuda")
            stats = torch.zeros(e_local, dtype=torch.int32, device="cuda")
            args = mega._moe_args(y, t1, t2, buf, stats, 10.0, fmt=fmt)
            _lib.check(_launch(entry, args))
            torch.cuda.synchronize()
            assert buf.host_error() == 0 and buf.kernel_error() == 0
            out[entry] = (y.view(torch.int16).cpu(), stats.cpu(), buf.topk_idx[:M].cpu().clone(),
                          buf.topk_weights[:M].cpu().clone().view(torch.int32))
        a, b = out.values()
        for u, v in zip(a, b):
            assert torch.equal(u, v)
