"""L2 items of one 128-row block (halves of the 256-row units, used when the units fill at most
half the grid) against whole units (debug flag bit 2) on the same inputs: each route's output
rows come from the same K-order accumulation either way, so y, the route outputs and the recv
stats must agree bit for bit, in every activation format, with one and with several 16-route
slabs per expert. Parity with the oracle of the half-item path itself is covered by every
small-shape layer test, which runs it by default."""
import numpy as np
import pytest
import torch

from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16

pytestmark = pytest.mark.gpu

H, I, TOPK = 512, 256, 4


def _weights(fmt, E, seed):
    if fmt == "qoq":
        from tests.test_gpu_qoq import make_qoq_weights
        return make_qoq_weights(E, H, I, seed)[0]
    if fmt == "nvfp4":
        from tests.test_gpu_nvfp4 import make_nvfp4_weights
        return make_nvfp4_weights(E, H, I, seed)[0]
    from tests.test_gpu_layer import make_weights
    return make_weights(E, H, I, seed)[0]


def _fused(dgm, fmt, y, t1, t2, b, stats):
    if fmt == "qoq":
        dgm.qoq_mega_moe_fused(y, t1, t2, b, cumulative_local_expert_recv_stats=stats)
    elif fmt == "nvfp4":
        dgm.fp4_fp4_mega_moe(y, t1, t2, b, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)
    else:
        dgm.mxfp4_mega_moe_fused(y, t1, t2, b, cumulative_local_expert_recv_stats=stats)


@pytest.mark.parametrize("M,E", [(6, 16), (40, 8)])
@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4", "qoq", "nvfp4"])
def test_half_items_match_whole_units(fmt, M, E):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    print(f"L2 halves vs whole units fmt={fmt} M={M} E={E}", flush=True)
    rng = np.random.default_rng(7100 + M + len(fmt))
    t1, t2 = _weights(fmt, E, 7101 + M)
    x = bf16_cpu(randn_bf16(rng, (M, H))).cuda()
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    out = []
    for flags in (0, 4):
        b = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, TOPK, H, I, act_format=fmt)
        b._debug_flags = flags
        y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
        stats = torch.zeros(E, dtype=torch.int32, device="cuda")
        dgm.fable_router_quant_topk_frontend(x, rw, b, select_in_mega=True)
        _fused(dgm, fmt, y, t1, t2, b, stats)
        torch.cuda.synchronize()
        assert b.kernel_error() == 0 and b.host_error() == 0
        counts = b.pool_table()[0]
        out.append((y.clone(), b.combine_partials[:, :M].clone(), stats.clone(), counts))
    (y0, p0, s0, c0), (y1, p1, s1, c1) = out
    if M == 40:
        assert int(c0.max()) > 16, "several slabs per expert"
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    assert torch.equal(s0, s1)
    # route outputs (slot-major bf16 rows) of the routes that were computed, both ways
    assert torch.equal(p0.view(torch.int16), p1.view(torch.int16))


@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
def test_half_items_past_one_round(fmt):
    """A-MXFP also runs halves when the units fill more than one round of the grid and at most
    1.5 (the last round half full or less): 160 experts forced-balanced at H=512 give 320 units,
    640 half items, so items are claimed beyond the first two per workgroup. Bit for bit equal
    to whole units."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    M, E = 40, 160
    print(f"L2 halves past one round fmt={fmt} M={M} E={E}", flush=True)
    rng = np.random.default_rng(7200 + len(fmt))
    t1, t2 = _weights(fmt, E, 7201)
    x = bf16_cpu(randn_bf16(rng, (M, H))).cuda()
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    out = []
    for flags in (0, 4):
        b = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, TOPK, H, I, act_format=fmt)
        b._debug_flags = flags
        y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
        stats = torch.zeros(E, dtype=torch.int32, device="cuda")
        dgm.fable_router_quant_topk_frontend(x, rw, b, select_in_mega=True, force_balanced=True)
        _fused(dgm, fmt, y, t1, t2, b, stats)
        torch.cuda.synchronize()
        assert b.kernel_error() == 0 and b.host_error() == 0
        n_active = int((b.pool_table()[0] > 0).sum())
        out.append((y.clone(), b.combine_partials[:, :M].clone(), stats.clone(), n_active))
    (y0, p0, s0, na), (y1, p1, s1, _) = out
    units = na * (H // 256)
    assert 256 < units <= 384, (units, "more than one round, at most 1.5")
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    assert torch.equal(s0, s1)
    assert torch.equal(p0.view(torch.int16), p1.view(torch.int16))
