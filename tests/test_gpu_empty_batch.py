"""An empty batch (no tokens): the frontend and every layer entry point return without launching
work, leave the recv stats and the buffer's counters as they were, and the next call on the
same buffer gives the fresh buffer's result bit for bit."""
import numpy as np
import pytest
import torch

from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16

pytestmark = pytest.mark.gpu

E, H, I, TOPK, MAXM = 16, 512, 256, 4, 8


@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4", "qoq", "nvfp4"])
def test_empty_batch_then_normal_call(fmt):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from tests.test_gpu_l2_halves import _weights, _fused
    print(f"empty batch fmt={fmt}", flush=True)
    rng = np.random.default_rng(7500 + len(fmt))
    t1, t2 = _weights(fmt, E, 7501)
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    x = bf16_cpu(randn_bf16(rng, (MAXM, H))).cuda()
    shared = dgm.get_fused_symm_buffer_for_mega_moe(None, E, MAXM, TOPK, H, I, act_format=fmt)
    stats = torch.full((E,), 3, dtype=torch.int32, device="cuda")
    for select in (True, False):
        y0 = torch.empty((0, H), dtype=torch.bfloat16, device="cuda")
        dgm.fable_router_quant_topk_frontend(x[:0], rw, shared, select_in_mega=select)
        _fused(dgm, fmt, y0, t1, t2, shared, stats)
        if fmt in ("mxfp8", "mxfp4"):
            dgm.mxfp4_mega_moe_split(y0, t1, t2, shared, cumulative_local_expert_recv_stats=stats)
    torch.cuda.synchronize()
    assert shared.kernel_error() == 0 and shared.host_error() == 0
    assert (stats == 3).all()
    # then a normal call on the same buffer, against a fresh buffer
    ys = []
    for b in (shared, dgm.get_fused_symm_buffer_for_mega_moe(None, E, MAXM, TOPK, H, I, act_format=fmt)):
        y = torch.empty((MAXM, H), dtype=torch.bfloat16, device="cuda")
        st = torch.zeros(E, dtype=torch.int32, device="cuda")
        dgm.fable_router_quant_topk_frontend(x, rw, b, select_in_mega=True)
        _fused(dgm, fmt, y, t1, t2, b, st)
        torch.cuda.synchronize()
        assert b.kernel_error() == 0
        ys.append((y, st))
    assert torch.equal(ys[0][0].view(torch.int16), ys[1][0].view(torch.int16))
    assert torch.equal(ys[0][1], ys[1][1])


@pytest.mark.parametrize("fmt,flags", [("mxfp8", 0), ("mxfp4", 8), ("qoq", 0), ("nvfp4", 0)])
def test_no_local_route_then_normal_call(fmt, flags):
    """Tokens but no local route (every top-k slot on another EP rank's experts, or unrouted): the
    persistent kernel runs with no active expert (no L1 or L2 unit), writes y = 0 and leaves the
    recv stats alone; its counter sets stay consistent, so the next call on the same buffer
    gives a fresh buffer's result bit for bit. (flags 8: the early-streaming form.)"""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from tests.test_gpu_l2_halves import _weights, _fused
    print(f"no local route fmt={fmt} flags={flags}", flush=True)
    rng = np.random.default_rng(7700 + len(fmt) + flags)
    t1, t2 = _weights(fmt, E, 7701)
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    x = bf16_cpu(randn_bf16(rng, (MAXM, H))).cuda()
    # EP rank 1 of 2: local experts 8..15 of 16 (the weights cover the 8 local ones)
    shared = dgm.get_fused_symm_buffer_for_mega_moe(None, E, MAXM, TOPK, H, I, act_format=fmt, ep_size=2,
                                                    ep_rank=1)
    shared._debug_flags = flags
    t1l = tuple(t[:E // 2] if t is not None else None for t in t1)
    t2l = tuple(t[:E // 2] if t is not None else None for t in t2)
    dgm.fable_router_quant_topk_frontend(x, rw, shared)
    idx = np.tile(np.arange(TOPK, dtype=np.int64), (MAXM, 1))       # experts 0..3: rank 0's
    idx[2] = -1                                                     # and one unrouted token
    shared.topk_idx.copy_(torch.from_numpy(idx).cuda())
    shared.topk_weights.fill_(0.25)
    stats = torch.full((E // 2,), 3, dtype=torch.int32, device="cuda")
    for _ in range(2):
        y = torch.full((MAXM, H), 5.0, dtype=torch.bfloat16, device="cuda")
        _fused(dgm, fmt, y, t1l, t2l, shared, stats)
        torch.cuda.synchronize()
        assert shared.kernel_error() == 0 and shared.host_error() == 0
        assert (y.float() == 0).all()
        assert (stats == 3).all()
        assert int(shared.pool_table()[0].sum()) == 0
    ys = []
    for b in (shared, dgm.get_fused_symm_buffer_for_mega_moe(None, E, MAXM, TOPK, H, I, act_format=fmt, ep_size=2,
                                                             ep_rank=1)):
        b._debug_flags = flags
        y = torch.empty((MAXM, H), dtype=torch.bfloat16, device="cuda")
        st = torch.zeros(E // 2, dtype=torch.int32, device="cuda")
        dgm.fable_router_quant_topk_frontend(x, rw, b, select_in_mega=True)
        _fused(dgm, fmt, y, t1l, t2l, b, st)
        torch.cuda.synchronize()
        assert b.kernel_error() == 0
        ys.append((y, st))
    assert torch.equal(ys[0][0].view(torch.int16), ys[1][0].view(torch.int16))
    assert torch.equal(ys[0][1], ys[1][1])
