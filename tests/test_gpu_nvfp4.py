"""GPU parity of the NVFP4 W4A4 layer (fp4_fp4_mega_moe / nvfp4_mega_moe on an "nvfp4" buffer).

Bit-exact: the NVFP4 activation codes and E4M3 scale bytes of the frontend (the W4A4 row cast of
sm100_b200/test_mega_moe.py:68-93), the pool, the weight transform (dequant(transform(q)) ==
interleave(dequant(q))). Tolerance (the north star's bar): per-row cos >= 0.9999 and rel-RMSE
<= 0.5 % of the bf16 output against the fp32 oracle of the reference's W4A4 test
(sm100_b200/test_mega_moe.py:411-486: dequantised NVFP4 weights and activations, fp32 gate/up
rounded to bf16, clamp, SiLU * up * w, per-16 NVFP4 requant, fp32 down projection and sum).
Weights are packed with ``quantize_to_nvfp4`` (deep_gemm/quantization_nvfp4.py:62, UE4M3 ceil
scales, Marlin order); the kernel's numerics depend only on the decoded values."""
import numpy as np
import pytest
import torch

from oracle import packers as pk
from oracle import moe
from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16, decode_native_nvfp4, interleave16

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
REL_RMSE_MAX = 0.005


def make_nvfp4_weights(E, H, I, seed, scale=0.02):
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_nvfp4 as qn
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w1 = (torch.randn((E, 2 * I, H), generator=g, device="cuda", dtype=torch.float32) * scale).to(torch.bfloat16)
    q1 = qn.quantize_to_nvfp4(w1)
    del w1
    w2 = (torch.randn((E, H, I), generator=g, device="cuda", dtype=torch.float32) * scale).to(torch.bfloat16)
    q2 = qn.quantize_to_nvfp4(w2)
    del w2
    t = dgm.transform_nvfp4_weights_for_mega_moe_fused(q1, q2)
    W1 = moe.LazyDequant(q1[0].cpu().numpy(), q1[1].cpu().numpy(), fn=pk.dequantize_nvfp4)
    W2 = moe.LazyDequant(q2[0].cpu().numpy(), q2[1].cpu().numpy(), fn=pk.dequantize_nvfp4)
    return t, W1, W2


def run_nvfp4(M, E, E_local, expert_begin, H, I, topk, seed, force_balanced=False, zero_rows=(),
              select_in_mega=False, global_scales=False):
    import hopper_megamoe_basedondeepgemm_amd as dgm
    print(f"nvfp4 layer M={M} E={E} E_local={E_local} H={H} I={I} topk={topk} seed={seed} "
          f"balanced={force_balanced} select_in_mega={select_in_mega} global_scales={global_scales}", flush=True)
    rng = np.random.default_rng(seed)
    x = randn_bf16(rng, (M, H))
    for r in zero_rows:
        x[r] = 0.0
    rw = randn_bf16(rng, (E, H), 0.02)
    (t1, t2), W1, W2 = make_nvfp4_weights(E_local, H, I, seed + 1)
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format="nvfp4",
                                                 ep_size=E // E_local, ep_rank=expert_begin // E_local)
    xs, rws = bf16_cpu(x).cuda(), bf16_cpu(rw).cuda()
    stats = torch.zeros(E_local, dtype=torch.int32, device="cuda")
    y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    dgm.fable_router_quant_topk_frontend(xs, rws, buf, force_balanced=force_balanced, select_in_mega=select_in_mega)
    gs1 = gs2 = None
    if global_scales:
        gs1 = (rng.random(E_local).astype(np.float32) * 1.5 + 0.25).astype(np.float32)
        gs2 = (rng.random(E_local).astype(np.float32) * 1.5 + 0.25).astype(np.float32)
        dgm.nvfp4_mega_moe(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0,
                           l1_global_scales=torch.from_numpy(gs1).cuda(), l2_global_scales=torch.from_numpy(gs2).cuda())
    else:
        dgm.fp4_fp4_mega_moe(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)
    torch.cuda.synchronize()
    logits = moe.router_logits_f32(x, rw)
    idx, w, _ = moe.topk_softmax(logits, topk)
    if force_balanced:
        idx, w = moe.balanced_routing(M, E, topk)
    for r in zero_rows:
        idx[r] = -1
        w[r] = 0.0
    codes, sfb, x_dq = moe.quant_act(x, "nvfp4")
    ref, _ = moe.moe_forward(x_dq, idx, w, W1, W2, expert_begin, "nvfp4", gs1=gs1, gs2=gs2)
    return dict(buf=buf, y=y.float().cpu().numpy(), ref=ref, idx=idx, codes=codes, sfb=sfb,
                stats=stats.cpu().numpy(), E_local=E_local, expert_begin=expert_begin, t=(t1, t2), gs=(gs1, gs2))


def check_frontend(r, M):
    b = r["buf"]
    np.testing.assert_array_equal(b.topk_idx[:M].cpu().numpy(), r["idx"])
    np.testing.assert_array_equal(b.x[:M].cpu().numpy(), r["codes"])
    np.testing.assert_array_equal(b.x_sf[:M].cpu().numpy(), r["sfb"])


def check_pool(r):
    counts, active, offsets, routes = r["buf"].pool_table()
    rc, ra, ro, rr = moe.dispatch(r["idx"], r["expert_begin"], r["E_local"])
    np.testing.assert_array_equal(counts.numpy(), rc)
    np.testing.assert_array_equal(routes.numpy(), rr)
    np.testing.assert_array_equal(r["stats"], rc)


def check_y(r, zero_rows=()):
    assert r["buf"].kernel_error() == 0
    for zr in zero_rows:
        assert (r["y"][zr] == 0).all()
    keep = [i for i in range(r["y"].shape[0]) if i not in zero_rows]
    m = moe.metrics(r["y"][keep], r["ref"][keep])
    assert m["cos_min"] >= COS_MIN and m["rel_rmse"] <= REL_RMSE_MAX, m
    return m


def test_transform_nvfp4_invariant():
    """dequant(transform(q)) == interleave(dequant(q)) for L1 and L2, both source orders."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_nvfp4 as qn
    rng = np.random.default_rng(41)
    w1 = randn_bf16(rng, (2, 64, 384), 0.05)
    w2 = randn_bf16(rng, (2, 32, 256), 0.05)
    q1 = qn.quantize_to_nvfp4(bf16_cpu(w1).cuda())
    q2 = qn.quantize_to_nvfp4(bf16_cpu(w2).cuda())
    (v1, s1), (v2, s2) = dgm.transform_nvfp4_weights_for_mega_moe_fused(q1, q2)
    d1 = pk.dequantize_nvfp4(q1[0].cpu().numpy(), q1[1].cpu().numpy())
    d2 = pk.dequantize_nvfp4(q2[0].cpu().numpy(), q2[1].cpu().numpy())
    np.testing.assert_array_equal(decode_native_nvfp4(v1.cpu().numpy(), s1.cpu().numpy()), interleave16(d1))
    np.testing.assert_array_equal(decode_native_nvfp4(v2.cpu().numpy(), s2.cpu().numpy()), d2)
    # low-nibble-first source (the W4A4 row cast)
    p3, _, sb3 = pk.cast_to_nvfp4_rows(w2)
    (_, _), (v3, s3) = dgm.transform_nvfp4_weights_for_mega_moe_fused(
        q1, (torch.from_numpy(p3).cuda(), torch.from_numpy(sb3).cuda()), src_order="low_first")
    from oracle import numerics as nu
    d3 = pk.dequant_fp4_rows(p3, nu.e4m3_decode(sb3), 16)
    np.testing.assert_array_equal(decode_native_nvfp4(v3.cpu().numpy(), s3.cpu().numpy()), d3)
    # the sm100 name picks the format from the scale count per row (K/16: NVFP4, K/32: MXFP4)
    p1, _, sb1 = pk.cast_to_nvfp4_rows(w1)
    lf1 = (torch.from_numpy(p1).cuda(), torch.from_numpy(sb1).cuda())
    lf2 = (torch.from_numpy(p3).cuda(), torch.from_numpy(sb3).cuda())
    got = dgm.transform_weights_for_mega_moe(lf1, lf2)
    want = dgm.transform_nvfp4_weights_for_mega_moe_fused(lf1, lf2, src_order="low_first")
    for g, w in zip(got, want):
        for a, b in zip(g, w):
            assert torch.equal(a, b)
    m1 = pk.cast_to_fp4_rows(w1)
    m2 = pk.cast_to_fp4_rows(w2)
    mx1 = (torch.from_numpy(m1[0]).cuda(), torch.from_numpy(m1[2]).cuda())
    mx2 = (torch.from_numpy(m2[0]).cuda(), torch.from_numpy(m2[2]).cuda())
    got = dgm.transform_weights_for_mega_moe(mx1, mx2)
    want = dgm.transform_mxfp4_weights_for_mega_moe_fused(mx1, mx2, src_order="low_first")
    for g, w in zip(got, want):
        assert torch.equal(g[0], w[0]) and torch.equal(g[1], w[1])


def test_nvfp4_small_layer():
    need_gpu()
    r = run_nvfp4(6, 16, 16, 0, 512, 256, 4, seed=800)
    check_frontend(r, 6)
    check_pool(r)
    print(check_y(r))


def test_nvfp4_config0_shape():
    need_gpu()
    r = run_nvfp4(2, 48, 48, 0, 3072, 1280, 8, seed=810)
    check_frontend(r, 2)
    check_pool(r)
    print(check_y(r))


def test_nvfp4_m128_unbalanced_ep_share():
    """Config 4's largest M: 128 tokens, seeded unbalanced routing over E=384, one EP rank's 48
    experts (several experts get more than 16 routes: multi-slab items)."""
    need_gpu()
    r = run_nvfp4(128, 384, 48, 96, 3072, 1280, 8, seed=820)
    check_frontend(r, 128)
    check_pool(r)
    print(check_y(r))


def test_nvfp4_global_scales_zero_rows_select_in_mega():
    need_gpu()
    r = run_nvfp4(40, 8, 8, 0, 1024, 512, 4, seed=830, zero_rows=(5, 21), select_in_mega=True,
                  global_scales=True)
    check_frontend(r, 40)
    check_pool(r)
    print(check_y(r, zero_rows=(5, 21)))


def test_nvfp4_limits_raise_before_launch():
    """NVFP4 runs only on the persistent kernel: beyond 1024 routes (tokens x topk) or 256
    tokens every entry (fp4_fp4_mega_moe, nvfp4_mega_moe fused / split / auto) raises
    RuntimeError with no launch (y keeps its sentinel); a call within the limits on the same
    buffer still runs."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    E, H, I = 8, 512, 256
    (t1, t2), _, _ = make_nvfp4_weights(E, H, I, 961)
    for M, topk, what in ((160, 8, "1280 routes"), (300, 2, "300 tokens")):
        print(f"nvfp4 limits: M={M} topk={topk} ({what}) must raise", flush=True)
        buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format="nvfp4")
        y = torch.full((M, H), 3.0, dtype=torch.bfloat16, device="cuda")
        calls = [lambda: dgm.fp4_fp4_mega_moe(y, t1, t2, buf)]
        calls += [lambda f=f: dgm.nvfp4_mega_moe(y, t1, t2, buf, kernel_family=f) for f in ("fused", "split", "auto")]
        for call in calls:
            with pytest.raises(RuntimeError, match="at most 1024 routes"):
                call()
        torch.cuda.synchronize()
        assert bool((y == 3.0).all()), "a refused call wrote y"
        assert buf.kernel_error() == 0
        rng = np.random.default_rng(962)
        m = 1024 // topk // 2
        x = bf16_cpu(randn_bf16(rng, (m, H))).cuda()
        rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
        dgm.fable_router_quant_topk_frontend(x, rw, buf)
        ys = torch.full((m, H), 3.0, dtype=torch.bfloat16, device="cuda")
        dgm.fp4_fp4_mega_moe(ys, t1, t2, buf)
        torch.cuda.synchronize()
        assert buf.kernel_error() == 0 and bool(torch.isfinite(ys.float()).all()) and not bool((ys == 3.0).all())


def test_nvfp4_split_family_matches_fused():
    """kernel_family="split" (dispatch + L1, then L2 + combine: two launches) and "auto" above
    family_threshold give the fused launch's output, intermediate rows and recv stats bit for
    bit, with per-expert global scales, zero rows and the top-k selected in the first launch."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    M, E, H, I, topk = 40, 8, 1024, 512, 4
    print(f"nvfp4 split vs fused M={M} E={E} H={H} I={I}", flush=True)
    rng = np.random.default_rng(840)
    x = randn_bf16(rng, (M, H))
    x[7] = 0.0
    rw = randn_bf16(rng, (E, H), 0.02)
    (t1, t2), _, _ = make_nvfp4_weights(E, H, I, 841)
    gs1 = torch.from_numpy((rng.random(E) * 1.5 + 0.25).astype(np.float32)).cuda()
    gs2 = torch.from_numpy((rng.random(E) * 1.5 + 0.25).astype(np.float32)).cuda()
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format="nvfp4")
    xs, rws = bf16_cpu(x).cuda(), bf16_cpu(rw).cuda()
    R = M * topk
    outs = []
    for family, thr, sel in (("fused", 256, False), ("split", 256, False), ("auto", 16, True)):
        y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
        stats = torch.zeros(E, dtype=torch.int32, device="cuda")
        dgm.fable_router_quant_topk_frontend(xs, rws, buf, select_in_mega=sel)
        dgm.nvfp4_mega_moe(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0,
                           l1_global_scales=gs1, l2_global_scales=gs2, kernel_family=family, family_threshold=thr)
        torch.cuda.synchronize()
        assert buf.kernel_error() == 0
        outs.append((y.clone(), stats.clone(), buf.l2_acts[:R].clone(), buf.l2_acts_sf[:R].clone(),
                     buf.topk_idx[:M].clone()))
    for o in outs[1:]:
        for a, b in zip(outs[0], o):
            assert torch.equal(a, b)
    assert (outs[0][0][7] == 0).all()
