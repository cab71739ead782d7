"""The reference's fused recipe on the persistent kernel: E4M3 activations with one fp32 scale per
128 K (the buffer of csrc/apis/mega_fused.hpp:31-76, filled as tests/test_four_api_correctness.py:
215 fills it), MXFP4 weights, fp32 gate / up, a power-of-two E4M3 intermediate per 64 features,
routes rounded to bf16, slot-order fp32 combine (T4:54-62, 419-446).

The one-launch layer (``mxfp4_mega_moe_fused`` / ``_C.mxfp4_mega_moe_fused`` on that buffer)
against the split path's kernels on the same buffer and inputs, bit for bit: y, the intermediate
codes and scales of every pool row, the route outputs and the recv stats (both accumulate each
K-tile's product promoted by its scale in K order, and requantise per 64 features the same
way); and y against the oracle at the north star's tolerance (cos >= 0.9999, rel-RMSE <= 0.5 %).
Covered: several slabs per expert, unrouted tokens (top-k -1), the top-k selected from the
frontend's keys in the prologue, the in-kernel frontend (one launch from bf16), and the
reference's positional ``_C`` call."""
import numpy as np
import pytest
import torch

from oracle import packers as pk
from oracle import moe
from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16
from tests.test_gpu_split_api import _split_weights, _oracle, _random_routing

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
REL_RMSE_MAX = 0.005
TOPK = 8


def _fill(buf, x, idx, w):
    M = x.shape[0]
    xq, xs = pk.per_token_cast_to_fp8_f32sf(x, 128)
    buf.x[:M].copy_(torch.from_numpy(xq).view(torch.float8_e4m3fn).cuda())
    buf.x_sf[:M].copy_(torch.from_numpy(xs).cuda())
    buf.topk_idx[:M].copy_(torch.from_numpy(idx).cuda())
    buf.topk_weights[:M].copy_(torch.from_numpy(w).cuda())
    return pk.dequant_fp8_rows(xq, xs, 128)


def _run(dgm, fused, buf, t1, t2, M, H, E):
    y = torch.full((M, H), 7.0, dtype=torch.bfloat16, device="cuda")
    stats = torch.zeros(E, dtype=torch.int32, device="cuda")
    if fused:
        dgm.mxfp4_mega_moe_fused(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)
    else:
        dgm.mxfp4_mega_moe(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)
    torch.cuda.synchronize()
    assert buf.kernel_error() == 0 and buf.host_error() == 0
    n = int(buf.pool_table()[0].sum())
    return (y.view(torch.int16).cpu(), stats.cpu(), buf.l2_acts[:n].view(torch.uint8).cpu().clone(),
            buf.l2_acts_sf[:n].cpu().clone(), buf.combine_partials[:, :M].view(torch.int16).cpu().clone())


@pytest.mark.parametrize("M,E,H,I,zero_rows", [(5, 16, 512, 256, ()), (40, 8, 512, 256, (3, 17)),
                                               (16, 48, 1024, 512, (0,)), (8, 48, 3072, 1280, ()),
                                               (64, 48, 3072, 1280, (9,))])
def test_fused_fp8f128_equals_split(M, E, H, I, zero_rows):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    print(f"fp8f128 fused vs split M={M} E={E} H={H} I={I} zero_rows={zero_rows}", flush=True)
    (t1, t2), q1, q2 = _split_weights(E, H, I, 1500 + M)
    rng = np.random.default_rng(1501 + M)
    x = randn_bf16(rng, (M, H))
    x[1, :128] = 0.0                       # an all-zero 128-group (scale floor 1e-4)
    idx, w = _random_routing(rng, M, E, TOPK)
    for r in zero_rows:
        idx[r] = -1
        w[r] = 0.0
    buf = dgm.get_symm_buffer_for_mega_moe(None, E, M, TOPK, H, I, mma_type="fp8xmxfp4")
    x_dq = _fill(buf, x, idx, w)
    split = _run(dgm, False, buf, t1, t2, M, H, E)
    buf.l2_acts.zero_()
    buf.combine_partials.zero_()
    fused = _run(dgm, True, buf, t1, t2, M, H, E)
    assert dgm.mega.fused_workgroups(buf) > 0           # the persistent kernel ran
    for name, u, v in zip(("y", "stats", "mid", "mid_sf", "partials"), split, fused):
        assert torch.equal(u, v), name
    ref, _ = _oracle(x_dq, idx, w, q1, q2, I, "fp8f128")
    m = moe.metrics(fused[0].view(torch.bfloat16).float().numpy(), ref)
    assert m["cos_min"] >= COS_MIN and m["rel_rmse"] <= REL_RMSE_MAX, m
    for r in zero_rows:
        assert (fused[0][r] == 0).all()
    print(f"  y {m}", flush=True)


def test_fused_fp8f128_frontend_paths():
    """The frontend's fp32-scale-per-128 cast with the top-k left to the fused kernel
    (select_in_mega: selected in the prologue up to 8 tokens, by a selection launch beyond), and
    the in-kernel frontend (one launch from bf16): the same y as the frontend + split path."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    E, H, I = 48, 3072, 1280
    (t1, t2), q1, q2 = _split_weights(E, H, I, 1600)
    rng = np.random.default_rng(1601)
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    for M in (6, 24):
        print(f"fp8f128 frontend paths M={M}", flush=True)
        x = bf16_cpu(randn_bf16(rng, (M, H))).cuda()
        outs = []
        for mode in ("split", "select_in_mega", "one_launch"):
            buf = dgm.get_symm_buffer_for_mega_moe(None, E, M, TOPK, H, I, mma_type="fp8xmxfp4")
            y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
            if mode == "split":
                dgm.fable_router_quant_topk_frontend(x, rw, buf)
                dgm.mxfp4_mega_moe(y, t1, t2, buf, activation_clamp=10.0)
            elif mode == "select_in_mega":
                dgm.mxfp4_mega_moe_from_bf16(y, x, rw, t1, t2, buf, one_launch=False)
            else:
                dgm.mxfp4_mega_moe_from_bf16(y, x, rw, t1, t2, buf, one_launch=True)
            torch.cuda.synchronize()
            assert buf.kernel_error() == 0 and buf.host_error() == 0
            outs.append((y.view(torch.int16).cpu(), buf.topk_idx[:M].cpu().clone(), buf.x[:M].view(torch.uint8).cpu(),
                         buf.x_sf[:M].cpu().clone()))
        for o in outs[1:]:
            for u, v in zip(outs[0], o):
                assert torch.equal(u, v)


def test_c_fused_fp8f128_is_one_launch():
    """``_C.mxfp4_mega_moe_fused`` on the reference's fused buffer runs the persistent kernel
    (one launch; its workgroup count is recorded) with the split path's y bit for bit."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import _C, _lib
    M, E, H, I = 8, 32, 1024, 512
    (t1, t2), q1, q2 = _split_weights(E, H, I, 1700)
    (v1, s1), (v2, s2) = t1[:2], t2[:2]
    r1 = r2 = None
    rng = np.random.default_rng(1701)
    x = randn_bf16(rng, (M, H))
    idx, w = _random_routing(rng, M, E, TOPK)
    n, slice_fn = _C.get_symm_buffer_size_for_fused_mega_moe(1, E, M, TOPK, H, I)
    raw = torch.zeros(n, dtype=torch.int8, device="cuda")
    bx, bxs, bidx, bw = slice_fn(raw)[:4]
    xq, xs = pk.per_token_cast_to_fp8_f32sf(x, 128)
    bx[:M].copy_(torch.from_numpy(xq).view(torch.float8_e4m3fn).cuda())
    bxs[:M].copy_(torch.from_numpy(xs).cuda())
    bidx[:M].copy_(torch.from_numpy(idx).cuda())
    bw[:M].copy_(torch.from_numpy(w).cuda())
    y = torch.zeros((M, H), dtype=torch.bfloat16, device="cuda")
    st = torch.zeros((1024, 8), dtype=torch.int64, device="cuda")
    _C.mxfp4_mega_moe_fused(y, (v1, s1), (v2, s2), None, r1, r2, raw, [raw.data_ptr()], 0, M, E, TOPK, 10.0, True,
                            st, None)
    torch.cuda.synchronize()
    # the persistent kernel's workgroups stamped their rows (the split kernels write no stamps)
    G = _lib.load().dgm_fused_workgroups(H, I, _lib.ACT_FORMATS["fp8f128"])
    a = st.cpu().numpy()
    assert 0 < G <= 1024 and (a[:G, 0] > 0).all() and (a[:G, 5] >= a[:G, 0]).all()
    buf = dgm.get_symm_buffer_for_mega_moe(None, E, M, TOPK, H, I, mma_type="fp8xmxfp4")
    _fill(buf, x, idx, w)
    y2 = torch.zeros((M, H), dtype=torch.bfloat16, device="cuda")
    dgm.mxfp4_mega_moe(y2, t1, t2, buf, activation_clamp=10.0)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
