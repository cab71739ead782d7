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
