"""The persistent kernel's early-weight-streaming form (opt-in, debug flag bit 3; small routed
sets, A-MXFP4 / A-MXFP8: the workgroup's first L1 unit is found from a mask of the active experts
while the top-k is read, and its slab, scales and tile ring are requested before the pool table
exists) against the default (plain) form on the same inputs: both run the same item order and the same
K-order accumulation, so y, the route outputs, the intermediate rows and the recv stats must
agree bit for bit; y also against the oracle at the north star's tolerance (cos >= 0.9999,
rel-RMSE <= 0.5 %). Covered: a first item of several 16-route slabs (the first slab requested
early, the second after the pool table), unrouted tokens, an EP rank's share (config 1: routes
of other ranks in the top-k), the top-k selected in the kernel's prologue and read from the
buffer, K-tile counts 4 (H = 512), 8 (H = 1024) and 24 (H = 3072), and the rule that picks the
form (the flag is not honoured beyond 32 expected local routes)."""
import numpy as np
import pytest
import torch

from oracle import moe
from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16
from tests.test_gpu_layer import make_weights

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
REL_RMSE_MAX = 0.005
EARLY_FORM, PLAIN_FORM = 2, 0
EARLY_FLAG = 8


def _routing(kind, M, E, topk, rng):
    """Explicit routing: 'skew' puts 20 of the tokens' (top-1) routes on expert 0 (two slabs);
    'zero' routes uniformly at random without repeats and leaves tokens 1 and 3 unrouted."""
    if kind == "skew":
        idx = np.where(np.arange(M)[:, None] < 20, 0, 1 + np.arange(M)[:, None] % (E - 1)).astype(np.int64)
    else:
        idx = np.stack([rng.permutation(E)[:topk] for _ in range(M)]).astype(np.int64)
    w = rng.uniform(0.05, 1.0, size=(M, topk)).astype(np.float32)
    if kind == "zero":
        idx[[1, 3]] = -1
        w[[1, 3]] = 0.0
    return idx, w


def _run(dgm, buf, fmt, t1, t2, M, E_local, flags):
    buf._debug_flags = flags
    y = torch.full((M, buf.hidden), 5.0, dtype=torch.bfloat16, device="cuda")
    stats = torch.zeros(E_local, dtype=torch.int32, device="cuda")
    dgm.mxfp4_mega_moe_fused(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)
    torch.cuda.synchronize()
    assert buf.kernel_error() == 0 and buf.host_error() == 0
    form = dgm.mega.fused_last_form(buf)
    n = int(buf.pool_table()[0].sum())
    out = (y.view(torch.int16).cpu(), stats.cpu(), buf.combine_partials[:, :M].view(torch.int16).cpu().clone(),
           buf.l2_acts[:n].view(torch.uint8).cpu().clone(), buf.l2_acts_sf[:n].view(torch.uint8).cpu().clone())
    return form, out


@pytest.mark.parametrize("fmt", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("M,E,E_local,topk,H,I,kind", [
    (24, 4, 4, 1, 512, 256, "skew"),          # 20 routes on expert 0: its first item is 2 slabs
    (6, 16, 16, 4, 512, 256, "zero"),          # unrouted tokens
    (4, 48, 48, 8, 1024, 512, "zero"),         # 8 K-tiles, 32 routes (the rule's limit)
    (8, 384, 48, 8, 3072, 1280, "frontend"),   # config 1: one EP rank's share, 8 local routes
    (2, 48, 48, 8, 3072, 1280, "select"),      # config 0's shape, top-k selected in the prologue
])
def test_early_streaming_matches_plain(fmt, M, E, E_local, topk, H, I, kind):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    print(f"early vs plain fmt={fmt} M={M} E={E} E_local={E_local} topk={topk} H={H} routing={kind}", flush=True)
    rng = np.random.default_rng(8100 + M + E + H)
    weights = make_weights(E_local, H, I, 8101 + M + H)
    (t1, t2), W1, W2 = weights
    x = randn_bf16(rng, (M, H))
    rw = randn_bf16(rng, (E, H), 0.02)
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format=fmt, ep_size=E // E_local,
                                                 ep_rank=0)
    xs, rws = bf16_cpu(x).cuda(), bf16_cpu(rw).cuda()
    dgm.fable_router_quant_topk_frontend(xs, rws, buf, force_balanced=kind == "frontend",
                                         select_in_mega=kind == "select")
    if kind in ("skew", "zero"):
        idx, w = _routing(kind, M, E, topk, rng)
        buf.topk_idx[:M].copy_(torch.from_numpy(idx).cuda())
        buf.topk_weights[:M].copy_(torch.from_numpy(w).cuda())
    elif kind == "frontend":
        idx, w = moe.balanced_routing(M, E, topk)
    else:
        idx, w, _ = moe.topk_softmax(moe.router_logits_f32(x, rw), topk)
    res = {}
    for flags in (0, EARLY_FLAG):      # plain first: the select path's top-k is written by the call
        res[flags] = _run(dgm, buf, fmt, t1, t2, M, E_local, flags)
    assert res[0][0] == PLAIN_FORM and res[EARLY_FLAG][0] == EARLY_FORM
    np.testing.assert_array_equal(buf.topk_idx[:M].cpu().numpy(), idx)
    counts = buf.pool_table()[0]
    if kind == "skew":
        assert int(counts.max()) == 20
    for name, u, v in zip(("y", "stats", "partials", "mid", "mid_sf"), res[0][1], res[EARLY_FLAG][1]):
        assert torch.equal(u, v), name
    _, _, x_dq = moe.quant_act(x, fmt)
    ref, _ = moe.moe_forward(x_dq, idx, w, W1, W2, 0, fmt)
    yv = res[EARLY_FLAG][1][0].view(torch.bfloat16).float().numpy()
    keep = [t for t in range(M) if (idx[t] >= 0).any()]
    m = moe.metrics(yv[keep], ref[keep])
    assert m["cos_min"] >= COS_MIN and m["rel_rmse"] <= REL_RMSE_MAX, m
    for t in range(M):
        if t not in keep:
            assert (res[EARLY_FLAG][1][0][t] == 0).all()
    print(f"  y {m}", flush=True)


def test_form_rule():
    """With the flag, early streaming is the form for at most 32 expected local routes (A-MXFP4 /
    A-MXFP8, the frontend run before the launch), the plain form beyond; without it, always the
    plain form."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    H, I, topk = 512, 256, 4
    (t1, t2), _, _ = make_weights(16, H, I, 8201)
    rng = np.random.default_rng(8200)
    rw = bf16_cpu(randn_bf16(rng, (16, H), 0.02)).cuda()
    for M, flags, want in ((8, EARLY_FLAG, EARLY_FORM), (9, EARLY_FLAG, PLAIN_FORM),   # 32 and 36 routes
                           (8, 0, PLAIN_FORM)):
        buf = dgm.get_fused_symm_buffer_for_mega_moe(None, 16, M, topk, H, I, act_format="mxfp8")
        buf._debug_flags = flags
        x = bf16_cpu(randn_bf16(rng, (M, H))).cuda()
        dgm.fable_router_quant_topk_frontend(x, rw, buf)
        y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
        dgm.mxfp4_mega_moe_fused(y, t1, t2, buf, activation_clamp=10.0)
        torch.cuda.synchronize()
        assert buf.kernel_error() == 0
        assert dgm.mega.fused_last_form(buf) == want, (M, flags)
    # the one-launch layer (in-kernel frontend) keeps its own form
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, 16, 4, topk, H, I, act_format="mxfp8")
    buf._debug_flags = EARLY_FLAG
    x = bf16_cpu(randn_bf16(rng, (4, H))).cuda()
    y = torch.empty((4, H), dtype=torch.bfloat16, device="cuda")
    dgm.mxfp4_mega_moe_from_bf16(y, x, rw, t1, t2, buf, one_launch=True)
    torch.cuda.synchronize()
    assert buf.kernel_error() == 0
    assert dgm.mega.fused_last_form(buf) == 1
