"""The persistent kernel's tail-half-unit form (opt-in, debug flag bit 4; A-MXFP4 / A-MXFP8 at
H = 3072, up to 32 routes):
when the last round of L1 units fills at most half the grid, each of its units runs as two
half items of 32 features, each 16-row weight block's K split over two waves whose sums the
gate wave adds from LDS in the order a whole unit sums its two K chains. Against the default
(plain) form on the same inputs: y, the route outputs, the intermediate rows and their
scales and the recv stats bit for bit; y also against the oracle at the north star's tolerance
(cos >= 0.9999, rel-RMSE <= 0.5 %). Covered: every unit as half items (units <= half the grid),
whole units then half items (M=2 on 48 experts: ~300 units on 256 workgroups), half items of
several 16-route slabs, unrouted tokens, an EP rank's share, the top-k selected in the kernel's
prologue and read from the buffer, and the form present with no partial round to split."""
import numpy as np
import pytest
import torch

from oracle import moe
from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16
from tests.test_gpu_layer import make_weights
from tests.test_gpu_early_streaming import _routing, _run

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
REL_RMSE_MAX = 0.005
H, I = 3072, 1280
TAIL_FORM, PLAIN_FORM = 3, 0
TAIL_FLAG = 16


@pytest.mark.parametrize("fmt", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("M,E,E_local,topk,kind", [
    (2, 48, 48, 8, "select"),        # ~15 experts: ~300 units, whole units then half items
    (24, 4, 4, 1, "skew"),           # 80 units, all half items; expert 0 has 20 routes (2 slabs)
    (6, 16, 16, 4, "zero"),          # all half items, unrouted tokens
    (4, 384, 48, 8, "frontend"),     # one EP rank's share (config 1 at M=4): 4 local routes
    (1, 48, 48, 8, "frontend"),      # 8 experts: 160 units, a round more than half full (no halves)
])
def test_tail_halves_match_plain(fmt, M, E, E_local, topk, kind):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    print(f"tail halves vs plain fmt={fmt} M={M} E={E} E_local={E_local} topk={topk} routing={kind}", flush=True)
    rng = np.random.default_rng(9100 + M + E)
    weights = make_weights(E_local, H, I, 9101 + M + E)
    (t1, t2), W1, W2 = weights
    x = randn_bf16(rng, (M, H))
    rw = randn_bf16(rng, (E, H), 0.02)
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format=fmt, ep_size=E // E_local,
                                                 ep_rank=0)
    xs, rws = bf16_cpu(x).cuda(), bf16_cpu(rw).cuda()
    balanced = kind == "frontend" and E == 384
    dgm.fable_router_quant_topk_frontend(xs, rws, buf, force_balanced=balanced, select_in_mega=kind == "select")
    if kind in ("skew", "zero"):
        idx, w = _routing(kind, M, E, topk, rng)
        buf.topk_idx[:M].copy_(torch.from_numpy(idx).cuda())
        buf.topk_weights[:M].copy_(torch.from_numpy(w).cuda())
    elif balanced:
        idx, w = moe.balanced_routing(M, E, topk)
    else:
        idx, w, _ = moe.topk_softmax(moe.router_logits_f32(x, rw), topk)
    res = {}
    for flags in (0, TAIL_FLAG):      # plain first: the select path's top-k is written by the call
        res[flags] = _run(dgm, buf, fmt, t1, t2, M, E_local, flags)
    assert res[0][0] == PLAIN_FORM and res[TAIL_FLAG][0] == TAIL_FORM
    np.testing.assert_array_equal(buf.topk_idx[:M].cpu().numpy(), idx)
    counts = buf.pool_table()[0]
    if kind == "skew":
        assert int(counts.max()) == 20
    units = int((counts > 0).sum()) * (I // 64)
    print(f"  {units} L1 units on {dgm.mega.fused_workgroups(buf)} workgroups", flush=True)
    for name, u, v in zip(("y", "stats", "partials", "mid", "mid_sf"), res[0][1], res[TAIL_FLAG][1]):
        assert torch.equal(u, v), name
    _, _, x_dq = moe.quant_act(x, fmt)
    ref, _ = moe.moe_forward(x_dq, idx, w, W1, W2, 0, fmt)
    yv = res[TAIL_FLAG][1][0].view(torch.bfloat16).float().numpy()
    keep = [t for t in range(M) if ((idx[t] >= 0) & (idx[t] < E_local)).any()]
    m = moe.metrics(yv[keep], ref[keep])
    assert m["cos_min"] >= COS_MIN and m["rel_rmse"] <= REL_RMSE_MAX, m
    for t in range(M):
        if t not in keep:
            assert (res[TAIL_FLAG][1][0][t] == 0).all()
    print(f"  y {m}", flush=True)


def test_tail_form_rule():
    """With flag bit 4 the form runs for up to 32 routes (A-MXFP, H = 3072), not beyond; without
    it, the plain form."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    (t1, t2), _, _ = make_weights(16, H, I, 9201)
    rng = np.random.default_rng(9200)
    rw = bf16_cpu(randn_bf16(rng, (16, H), 0.02)).cuda()
    for M, flags, want in ((4, TAIL_FLAG, TAIL_FORM), (5, TAIL_FLAG, PLAIN_FORM), (4, 0, PLAIN_FORM)):   # 32, 40 routes
        buf = dgm.get_fused_symm_buffer_for_mega_moe(None, 16, M, 8, H, I, act_format="mxfp4")
        buf._debug_flags = flags
        x = bf16_cpu(randn_bf16(rng, (M, H))).cuda()
        dgm.fable_router_quant_topk_frontend(x, rw, buf)
        y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
        dgm.mxfp4_mega_moe_fused(y, t1, t2, buf, activation_clamp=10.0)
        torch.cuda.synchronize()
        assert buf.kernel_error() == 0
        assert dgm.mega.fused_last_form(buf) == want, (M, flags)
