"""GPU checks of the ``_C`` module (the reference's positional ``deep_gemm._C`` calls,
csrc/apis/mega_fused.hpp:101-105, csrc/apis/mega.hpp:378, 744): a buffer sized and sliced the
reference's way, filled as tests/test_four_api_correctness.py fills it, gives the same y bit for
bit as the named API on the same inputs; the frontend writes the fp32-scale-per-128 cast and,
with select_in_mega, the key array where the reference's wrapper reads it."""
import numpy as np
import pytest
import torch

from oracle import packers as pk
from oracle import moe
from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16

pytestmark = pytest.mark.gpu


def _mx_weights(E, H, I, seed):
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_mxfp4 as qs
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w1 = (torch.randn((E, 2 * I, H), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((E, H, I), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    return dgm.transform_mxfp4_weights_for_mega_moe_fused(qs.quantize_to_mxfp4(w1), qs.quantize_to_mxfp4(w2))


def _routing(rng, M, E, topk):
    idx = np.stack([rng.choice(E, topk, replace=False) for _ in range(M)]).astype(np.int64)
    w = rng.random((M, topk)).astype(np.float32)
    return idx, (w / w.sum(1, keepdims=True)).astype(np.float32)


def test_c_fused_matches_named_split_api():
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import _C
    M, E, H, I, topk = 8, 32, 1024, 512, 8
    print(f"_C fused M={M} E={E} H={H} I={I}", flush=True)
    (v1, s1, r1), (v2, s2, r2) = _mx_weights(E, H, I, 11)
    rng = np.random.default_rng(12)
    x = randn_bf16(rng, (M, H))
    xq, xs = pk.per_token_cast_to_fp8_f32sf(x, 128)
    idx, w = _routing(rng, M, E, topk)
    n, slice_fn = _C.get_symm_buffer_size_for_fused_mega_moe(1, E, M, topk, H, I)
    raw = torch.zeros(n, dtype=torch.int8, device="cuda")
    bx, bxs, bidx, bw, a1, a1s, a2, a2s, comb = slice_fn(raw)
    assert bx.dtype == torch.float8_e4m3fn and bxs.dtype == torch.float32 and tuple(comb.shape) == (topk, M, H)
    bx[:M].copy_(torch.from_numpy(xq).view(torch.float8_e4m3fn).cuda())
    bxs[:M].copy_(torch.from_numpy(xs).cuda())
    bidx[:M].copy_(torch.from_numpy(idx).cuda())
    bw[:M].copy_(torch.from_numpy(w).cuda())
    y = torch.zeros((M, H), dtype=torch.bfloat16, device="cuda")
    stats = torch.zeros(E, dtype=torch.int32, device="cuda")
    _C.mxfp4_mega_moe_fused(y, (v1, s1), (v2, s2), stats, r1, r2, raw, [raw.data_ptr()], 0, M, E, topk, 10.0, True,
                            None, None)
    # the named API on its own buffer with the same inputs
    buf = dgm.get_symm_buffer_for_mega_moe(None, E, M, topk, H, I, mma_type="fp8xmxfp4")
    buf.x[:M].copy_(bx[:M])
    buf.x_sf[:M].copy_(bxs[:M])
    buf.topk_idx[:M].copy_(bidx[:M])
    buf.topk_weights[:M].copy_(bw[:M])
    y2 = torch.zeros_like(y)
    dgm.mxfp4_mega_moe(y2, (v1, s1), (v2, s2), buf, activation_clamp=10.0)
    torch.cuda.synchronize()
    assert y.float().abs().max() > 0
    np.testing.assert_array_equal(y.view(torch.int16).cpu().numpy(), y2.view(torch.int16).cpu().numpy())
    np.testing.assert_array_equal(stats.cpu().numpy(), moe.dispatch(idx, 0, E)[0])
    np.testing.assert_array_equal(comb.view(torch.int16).cpu().numpy(),
                                  buf.combine_partials.view(torch.int16).cpu().numpy())


def test_c_qoq_fused_matches_named_api():
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import _C
    from hopper_megamoe_basedondeepgemm_amd import quantization_qoq_fused as qq
    M, E, H, I, topk = 6, 16, 1024, 512, 8
    g = torch.Generator(device="cuda")
    g.manual_seed(21)
    w1 = (torch.randn((E, 2 * I, H), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((E, H, I), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    (v1, m1, r1), (v2, m2, r2) = dgm.transform_qoq_weights_for_mega_moe_fused(qq.quantize_to_qoq(w1),
                                                                            qq.quantize_to_qoq(w2))
    rng = np.random.default_rng(22)
    x = randn_bf16(rng, (M, H))
    q8, s8 = pk.per_token_cast_to_int8(x)
    idx, w = _routing(rng, M, E, topk)
    n, slice_fn = _C.get_symm_buffer_size_for_fused_mega_moe(1, E, M, topk, H, I)
    raw = torch.zeros(n, dtype=torch.int8, device="cuda")
    bx, bxs, bidx, bw = slice_fn(raw)[:4]
    bx[:M].copy_(torch.from_numpy(q8).view(torch.float8_e4m3fn).cuda())
    bxs[:M].copy_(torch.from_numpy(np.repeat(s8[:, None], H // 128, 1)).cuda())
    bidx[:M].copy_(torch.from_numpy(idx).cuda())
    bw[:M].copy_(torch.from_numpy(w).cuda())
    y = torch.zeros((M, H), dtype=torch.bfloat16, device="cuda")
    _C.qoq_mega_moe_fused(y, (v1, m1), (v2, m2), None, r1, r2, raw, [raw.data_ptr()], 0, M, E, topk, 10.0, True)
    fb = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format="qoq")
    fb.x[:M].copy_(torch.from_numpy(q8).cuda())
    fb.x_sf[:M].copy_(bxs[:M])
    fb.topk_idx[:M].copy_(bidx[:M])
    fb.topk_weights[:M].copy_(bw[:M])
    y2 = torch.zeros_like(y)
    dgm.qoq_mega_moe_fused(y2, (v1, m1, r1), (v2, m2, r2), fb, activation_clamp=10.0)
    torch.cuda.synchronize()
    assert y.float().abs().max() > 0
    np.testing.assert_array_equal(y.view(torch.int16).cpu().numpy(), y2.view(torch.int16).cpu().numpy())


def test_c_frontend_cast_and_select_in_mega_keys():
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import _C
    M, E, H, I, topk = 4, 48, 1024, 512, 8
    rng = np.random.default_rng(31)
    x = randn_bf16(rng, (M, H))
    rw = randn_bf16(rng, (E, H), 0.02)
    n, slice_fn = _C.get_symm_buffer_size_for_fused_mega_moe(1, E, M, topk, H, I)
    raw = torch.zeros(n, dtype=torch.int8, device="cuda")
    bx, bxs, bidx, bw = slice_fn(raw)[:4]
    ws = torch.zeros(256 + 64 * 1024 + 4 * 64 * E, dtype=torch.uint8, device="cuda")
    xg, rg = bf16_cpu(x).cuda(), bf16_cpu(rw).cuda()
    _C.fable_router_quant_topk_frontend(xg, rg, bx[:M], bxs[:M], bidx[:M], bw[:M], ws, 0, 0, 0, 0, 0, 1)
    torch.cuda.synchronize()
    xq, xs = pk.per_token_cast_to_fp8_f32sf(x, 128)
    np.testing.assert_array_equal(bx[:M].view(torch.uint8).cpu().numpy(), xq)
    np.testing.assert_array_equal(bxs[:M].cpu().numpy().view(np.uint32), xs.view(np.uint32))
    idx, w, _ = moe.topk_softmax(moe.router_logits_f32(x, rw), topk)
    np.testing.assert_array_equal(bidx[:M].cpu().numpy(), idx)
    np.testing.assert_allclose(bw[:M].cpu().numpy(), w, rtol=1e-6, atol=0)
    # select_in_mega: the keys land at workspace + 256 + 64 KB as well
    _C.fable_router_quant_topk_frontend(xg, rg, bx[:M], bxs[:M], bidx[:M], bw[:M], ws, 0, 0, 0, 0, 1, 1)
    torch.cuda.synchronize()
    keys = moe.topk_keys(np_bf16_bits(moe.router_logits_f32(x, rw)), E)
    off = 256 + 64 * 1024
    got = ws[off:off + 4 * M * E].view(torch.int32).cpu().numpy().view(np.uint32).reshape(M, E)
    np.testing.assert_array_equal(got, keys)


def np_bf16_bits(a):
    from oracle import numerics as nu
    return nu.f32_to_bf16_bits(a)


def test_c_buffer_cache_follows_the_callers_tensor():
    """A sliced buffer is remembered per (address, rank, format) for as long as the caller's
    tensor lives: slicing the same memory for another shape replaces the wrapper (the later
    layer calls then use the new shape), and dropping the tensor drops the entry (and the view
    that kept its memory)."""
    need_gpu()
    import gc
    from hopper_megamoe_basedondeepgemm_amd import _C
    n, slice_fn = _C.get_symm_buffer_size_for_fused_mega_moe(1, 32, 8, 8, 1024, 512)
    n2, slice_fn2 = _C.get_symm_buffer_size_for_fused_mega_moe(1, 32, 4, 8, 1024, 512)
    assert n2 < n
    raw = torch.zeros(n, dtype=torch.int8, device="cuda")
    key = (raw.data_ptr(), 0, "fp8f128")
    slice_fn(raw)
    assert _C._lookup(raw, 0).num_max_tokens_per_rank == 8
    views = slice_fn2(raw)
    assert _C._lookup(raw, 0).num_max_tokens_per_rank == 4 and tuple(views[2].shape) == (4, 8)
    assert key in _C._BUFFERS
    del raw, views
    gc.collect()
    assert key not in _C._BUFFERS
