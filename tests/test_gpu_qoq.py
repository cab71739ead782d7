"""GPU parity of the QoQ W4A8 layer (qoq_mega_moe_fused) against the oracle.

Bit-exact: the per-token int8 activation codes and scales of the frontend, the pool, and the
L1 int32 accumulators of every route (dumped by the kernel's debug hook) against the exact
integer product of the weights' (code - z) * s2 with the int8 activations.
Integer path: the intermediate int8 codes and per-64 scales the kernel hands from L1 to L2
are checked against an exact-integer restatement of L1 (int64 group sums
sum_k (code - z) * s2 * x8, then float(Q) * s1 * sx): scales within 1e-5 relative error,
codes equal except for rare +-1 flips where SiLU's hardware exp2 / reciprocal or the fp32
product order moves a value across a rounding boundary.
Tolerance (the north star's bar): per-row cos >= 0.9999 and rel-RMSE <= 0.5 % of the bf16
output against the fp32 oracle of the reference's QoQ test (tests/test_four_api_correctness.py:
421-446: dequantised weights and activations, fp32 gate / up, per-64 int8 requant, per-route
bf16)."""
import numpy as np
import pytest
import torch

from oracle import packers as pk
from oracle import moe
from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
REL_RMSE_MAX = 0.005


class LazyQoQ:
    """Per-expert dequantisation of quantize_to_qoq outputs (``W[e]`` -> f32 [N, K])."""

    def __init__(self, q):
        self.p, self.s2, self.z, self.s1 = q
        E, N, Kh = self.p.shape
        self.shape = (E, N, 2 * Kh)

    def __getitem__(self, e):
        return pk.dequantize_qoq(self.p[e:e + 1], self.s2[e:e + 1], self.z[e:e + 1], self.s1[e:e + 1])[0]


def make_qoq_weights(E, H, I, seed, scale=0.02):
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_qoq_fused as qq
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w1 = (torch.randn((E, 2 * I, H), generator=g, device="cuda", dtype=torch.float32) * scale).to(torch.bfloat16)
    q1 = qq.quantize_to_qoq(w1)
    del w1
    w2 = (torch.randn((E, H, I), generator=g, device="cuda", dtype=torch.float32) * scale).to(torch.bfloat16)
    q2 = qq.quantize_to_qoq(w2)
    del w2
    t = dgm.transform_qoq_weights_for_mega_moe_fused(q1, q2)
    h1 = tuple(a.cpu().numpy() for a in q1)
    h2 = tuple(a.cpu().numpy() for a in q2)
    return t, h1, h2


def run_qoq(M, E, E_local, expert_begin, H, I, topk, seed, force_balanced=False, zero_rows=(),
            weights=None, select_in_mega=False):
    import hopper_megamoe_basedondeepgemm_amd as dgm
    print(f"qoq layer M={M} E={E} E_local={E_local} H={H} I={I} topk={topk} seed={seed} "
          f"balanced={force_balanced} select_in_mega={select_in_mega}", flush=True)
    rng = np.random.default_rng(seed)
    x = randn_bf16(rng, (M, H))
    for r in zero_rows:
        x[r] = 0.0
    rw = randn_bf16(rng, (E, H), 0.02)
    if weights is None:
        weights = make_qoq_weights(E_local, H, I, seed + 1)
    (t1, t2), h1, h2 = weights
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format="qoq",
                                                 ep_size=E // E_local, ep_rank=expert_begin // E_local)
    xs, rws = bf16_cpu(x).cuda(), bf16_cpu(rw).cuda()
    stats = torch.zeros(E_local, dtype=torch.int32, device="cuda")
    y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    dgm.fable_router_quant_topk_frontend(xs, rws, buf, force_balanced=force_balanced, select_in_mega=select_in_mega)
    dgm.qoq_mega_moe_fused(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats)
    torch.cuda.synchronize()
    # ---- oracle
    logits = moe.router_logits_f32(x, rw)
    idx, w, _ = moe.topk_softmax(logits, topk)
    if force_balanced:
        idx, w = moe.balanced_routing(M, E, topk)
    for r in zero_rows:
        idx[r] = -1
        w[r] = 0.0
    codes, sf, x_dq = moe.quant_act(x, "qoq")
    ref, _ = moe.moe_forward_qoq(x_dq, idx, w, LazyQoQ(h1), LazyQoQ(h2), expert_begin)
    return dict(buf=buf, y=y.float().cpu().numpy(), ref=ref, idx=idx, w=w, codes=codes, sf=sf,
                stats=stats.cpu().numpy(), h1=h1, E_local=E_local, expert_begin=expert_begin, I=I, topk=topk)


def check_frontend(r, M):
    b = r["buf"]
    np.testing.assert_array_equal(b.topk_idx[:M].cpu().numpy(), r["idx"])
    np.testing.assert_array_equal(b.x[:M].cpu().numpy(), r["codes"])
    sf = b.x_sf[:M].cpu().numpy()
    np.testing.assert_array_equal(sf.view(np.uint32), np.repeat(r["sf"][:, None], sf.shape[1], 1).view(np.uint32))


def check_pool(r):
    counts, active, offsets, routes = r["buf"].pool_table()
    rc, ra, ro, rr = moe.dispatch(r["idx"], r["expert_begin"], r["E_local"])
    np.testing.assert_array_equal(counts.numpy(), rc)
    np.testing.assert_array_equal(routes.numpy(), rr)
    np.testing.assert_array_equal(r["stats"], rc)
    return ra, ro, rr


def check_mid(r, max_flip_frac=0.01):
    """Intermediate codes / scales of every route against the exact-integer L1 restatement."""
    ra, ro, rr = check_pool(r)
    b, I, topk = r["buf"], r["I"], r["topk"]
    p, s2, z, s1 = r["h1"]
    codes_w = pk.unpack_marlin(p)                                      # [E, 2I, H] 0..15
    total = int(ro[-1])
    got_q = b.l2_acts[:total].cpu().numpy().astype(np.int64)
    got_s = b.l2_acts_sf[:total].cpu().numpy()
    x8 = r["codes"].astype(np.int64)
    flips = 0
    for a, e in enumerate(ra):
        rows = rr[ro[a]:ro[a + 1]]
        t = rows // topk
        H = codes_w.shape[2]
        G = H // 128
        c = codes_w[e].reshape(2 * I, G, 128).astype(np.int64)
        acc = np.zeros((2 * I, len(rows)), np.int64)
        for gi in range(G):
            acc += s2[e][:, gi, None].astype(np.int64) * moe.qoq_group_acc(c[:, gi], z[e][:, gi], x8[t, gi * 128:(gi + 1) * 128])
        h = (acc.astype(np.float32) * s1[e][:, None]).astype(np.float32) * r["sf"][t][None, :]
        gate = np.minimum(h[:I].T, np.float32(10.0))
        up = np.clip(h[I:].T, -10.0, 10.0).astype(np.float32)
        act = (moe.silu(gate) * up).astype(np.float32) * r["w"].reshape(-1)[rows][:, None]
        q, sc, _ = moe.requant_mid_qoq(act.astype(np.float32))
        gs = got_s[ro[a]:ro[a + 1]]
        np.testing.assert_allclose(gs, sc, rtol=1e-5, atol=0)
        d = got_q[ro[a]:ro[a + 1]] - q.astype(np.int64)
        assert np.abs(d).max() <= 1, (e, np.abs(d).max())
        flips += int((d != 0).sum())
    n = total * I
    assert flips <= max_flip_frac * n, (flips, n)
    return flips, n


def check_y(r, zero_rows=()):
    assert r["buf"].kernel_error() == 0
    for zr in zero_rows:
        assert (r["y"][zr] == 0).all()
    keep = [i for i in range(r["y"].shape[0]) if i not in zero_rows]
    m = moe.metrics(r["y"][keep], r["ref"][keep])
    assert m["cos_min"] >= COS_MIN and m["rel_rmse"] <= REL_RMSE_MAX, m
    return m


def test_qoq_small_layer():
    need_gpu()
    r = run_qoq(6, 16, 16, 0, 512, 256, 4, seed=700)
    check_frontend(r, 6)
    print("mid flips", check_mid(r))
    print(check_y(r))


def test_qoq_config0_shape():
    """benchmark config 0 shape (E=48, H=3072, I=1280, top-8, M=2) on the QoQ path."""
    need_gpu()
    r = run_qoq(2, 48, 48, 0, 3072, 1280, 8, seed=710)
    check_frontend(r, 2)
    print("mid flips", check_mid(r))
    print(check_y(r))


def test_qoq_ep_share_balanced():
    """384-way router, forced-balanced, one EP rank's 48 experts, M=16 (config 3's layout)."""
    need_gpu()
    r = run_qoq(16, 384, 48, 48, 3072, 1280, 8, seed=720, force_balanced=True)
    check_frontend(r, 16)
    print("mid flips", check_mid(r))
    print(check_y(r))


def test_qoq_zero_rows_multi_slab_select_in_mega():
    """Zero rows unrouted (y == 0), > 16 routes per expert (several slabs), top-k selected in
    the fused kernel's prologue."""
    need_gpu()
    r = run_qoq(40, 8, 8, 0, 1024, 512, 4, seed=730, zero_rows=(3, 17), select_in_mega=True)
    check_frontend(r, 40)
    print("mid flips", check_mid(r))
    print(check_y(r, zero_rows=(3, 17)))


def test_qoq_buffer_format_guard():
    """The MXFP entry points refuse a qoq buffer and the QoQ entry points an MXFP buffer."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    b = dgm.get_fused_symm_buffer_for_mega_moe(None, 16, 4, 4, 512, 256, act_format="qoq")
    y = torch.empty((4, 512), dtype=torch.bfloat16, device="cuda")
    dummy = (torch.empty(1, device="cuda"),) * 3
    with pytest.raises(ValueError):
        dgm.mxfp4_mega_moe_fused(y, dummy, dummy, b)
    bm = dgm.get_fused_symm_buffer_for_mega_moe(None, 16, 4, 4, 512, 256, act_format="mxfp4")
    with pytest.raises(ValueError):
        dgm.qoq_mega_moe_split(y, dummy, dummy, bm)
    with pytest.raises(ValueError):
        dgm.qoq_mega_moe_fused(y, dummy, dummy, bm)


def test_qoq_limits_raise_before_launch():
    """QoQ runs only on the persistent kernel: a call beyond 1024 routes (tokens x topk) or 256
    tokens raises RuntimeError from both entry points, with no launch (y keeps its sentinel),
    and a call within the limits on the same buffer still runs."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    E, H, I = 8, 512, 256
    (t1, t2), _, _ = make_qoq_weights(E, H, I, 951)
    for M, topk, what in ((160, 8, "1280 routes"), (300, 2, "300 tokens")):
        print(f"qoq limits: M={M} topk={topk} ({what}) must raise", flush=True)
        buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format="qoq")
        y = torch.full((M, H), 3.0, dtype=torch.bfloat16, device="cuda")
        for fn in (dgm.qoq_mega_moe_fused, dgm.qoq_mega_moe_split):
            with pytest.raises(RuntimeError, match="at most 1024 routes"):
                fn(y, t1, t2, buf)
        torch.cuda.synchronize()
        assert bool((y == 3.0).all()), "a refused call wrote y"
        assert buf.kernel_error() == 0
        rng = np.random.default_rng(952)
        m = 1024 // topk // 2
        x = bf16_cpu(randn_bf16(rng, (m, H))).cuda()
        rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
        dgm.fable_router_quant_topk_frontend(x, rw, buf)
        ys = torch.full((m, H), 3.0, dtype=torch.bfloat16, device="cuda")
        dgm.qoq_mega_moe_fused(ys, t1, t2, buf)
        torch.cuda.synchronize()
        assert buf.kernel_error() == 0 and bool(torch.isfinite(ys.float()).all()) and not bool((ys == 3.0).all())


def test_qoq_int4_packer_and_split_matches_fused():
    """The split path: quantize_to_qoq_int4 (int32 coefficient plane) bit-exact against the
    oracle; transform_qoq_int4_weights_for_mega_moe_sm90 equal to the fused packer's transform of
    the same weights; qoq_mega_moe_split (dispatch + L1, then L2 + combine) equal to
    qoq_mega_moe_fused bit for bit (y, intermediate codes and scales, recv stats), with the
    frontend run from router_input / router_weight and with the top-k selected in the first
    launch; y within tolerance of the oracle."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_mxfp4 as qm
    from hopper_megamoe_basedondeepgemm_amd import quantization_qoq_fused as qq
    M, E, H, I, topk = 40, 16, 512, 256, 4
    print(f"qoq int4 packer + split vs fused M={M} E={E} H={H} I={I}", flush=True)
    rng = np.random.default_rng(740)
    w1 = randn_bf16(rng, (E, 2 * I, H), 0.02)
    w2 = randn_bf16(rng, (E, H, I), 0.02)
    w1d, w2d = bf16_cpu(w1).cuda(), bf16_cpu(w2).cuda()
    i1, i2 = qm.quantize_to_qoq_int4(w1d), qm.quantize_to_qoq_int4(w2d)
    for got, w in ((i1, w1), (i2, w2)):
        rp, rpl = pk.quantize_to_qoq_int4(w)
        np.testing.assert_array_equal(got[0].cpu().numpy(), rp)
        np.testing.assert_array_equal(got[1].cpu().numpy(), rpl)
    t4 = dgm.transform_qoq_int4_weights_for_mega_moe_sm90(i1, i2)
    tf = dgm.transform_qoq_weights_for_mega_moe_fused(qq.quantize_to_qoq(w1d), qq.quantize_to_qoq(w2d))
    for a, b in zip(t4, tf):
        for u, v in zip(a, b):
            assert torch.equal(u, v)
    x = randn_bf16(rng, (M, H))
    x[9] = 0.0
    rw = randn_bf16(rng, (E, H), 0.02)
    xs, rws = bf16_cpu(x).cuda(), bf16_cpu(rw).cuda()
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format="qoq")
    R = M * topk
    outs = []
    for mode in ("fused", "split_router_input", "split_select_in_mega"):
        y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
        stats = torch.zeros(E, dtype=torch.int32, device="cuda")
        if mode == "fused":
            dgm.fable_router_quant_topk_frontend(xs, rws, buf)
            dgm.qoq_mega_moe_fused(y, t4[0], t4[1], buf, cumulative_local_expert_recv_stats=stats)
        elif mode == "split_router_input":
            dgm.qoq_mega_moe_split(y, t4[0], t4[1], buf, stats, activation_clamp=10.0,
                                   router_input=xs, router_weight=rws)
        else:
            dgm.fable_router_quant_topk_frontend(xs, rws, buf, select_in_mega=True)
            dgm.qoq_mega_moe_split(y, t4[0], t4[1], buf, cumulative_local_expert_recv_stats=stats,
                                   activation_clamp=10.0)
        torch.cuda.synchronize()
        assert buf.kernel_error() == 0
        outs.append((y.clone(), stats.clone(), buf.l2_acts[:R].clone(), buf.l2_acts_sf[:R].clone(),
                     buf.topk_idx[:M].clone()))
    for o in outs[1:]:
        for a, b in zip(outs[0], o):
            assert torch.equal(a, b)
    # y against the oracle
    logits = moe.router_logits_f32(x, rw)
    idx, w, _ = moe.topk_softmax(logits, topk)
    idx[9] = -1
    w[9] = 0.0
    _, _, x_dq = moe.quant_act(x, "qoq")
    h1 = pk.qoq_int4_to_fused(*(a.cpu().numpy() for a in i1))
    h2 = pk.qoq_int4_to_fused(*(a.cpu().numpy() for a in i2))
    ref, _ = moe.moe_forward_qoq(x_dq, idx, w, LazyQoQ(h1), LazyQoQ(h2), 0)
    yv = outs[0][0].float().cpu().numpy()
    assert (yv[9] == 0).all()
    keep = [i for i in range(M) if i != 9]
    m = moe.metrics(yv[keep], ref[keep])
    assert m["cos_min"] >= COS_MIN and m["rel_rmse"] <= REL_RMSE_MAX, m
    print(m)


@pytest.mark.parametrize("M,E,H,I", [(12, 16, 1024, 512), (8, 48, 3072, 1280)])
def test_qoq_l1_int_accumulators_bit_exact(M, E, H, I):
    """The W4A8 L1 accumulator of each (route, W1 row), sum over K128 groups g of
    s2_g * sum_k (code - z_g) * x8_k, is exact int32 arithmetic in the kernel (int8 matrix-core
    sums, integer zero-point correction and scale promotion): equal to the oracle's int64
    product, element for element (the north star's 'int GEMM accumulators bit-exact')."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    topk = 8
    print(f"qoq int accumulators M={M} E={E} H={H} I={I}", flush=True)
    t, h1, h2 = make_qoq_weights(E, H, I, 600 + M)
    rng = np.random.default_rng(601 + M)
    x = randn_bf16(rng, (M, H))
    rw = randn_bf16(rng, (E, H), 0.02)
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format="qoq")
    dgm.fable_router_quant_topk_frontend(bf16_cpu(x).cuda(), bf16_cpu(rw).cuda(), buf)
    R = M * topk
    dump = torch.zeros(R * I, dtype=torch.int64, device="cuda")         # int32 [R][2I]
    y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    buf._debug_flags = 2
    try:
        dgm.qoq_mega_moe_fused(y, t[0], t[1], buf, activation_clamp=10.0, phase_stamps=dump)
        torch.cuda.synchronize()
    finally:
        buf._debug_flags = 0
    assert buf.kernel_error() == 0
    got = dump.view(torch.int32).cpu().numpy().reshape(R, 2 * I).astype(np.int64)
    _, active, offsets, routes = buf.pool_table()
    idx = buf.topk_idx[:M].cpu().numpy()
    x8 = buf.x[:M].cpu().numpy().astype(np.int64)
    n_checked = 0
    for a, e in enumerate(active.tolist()):
        wint = pk.qoq_int_codes(h1[0][e:e + 1], h1[1][e:e + 1], h1[2][e:e + 1])[0]    # [2I, H]
        for pr in range(int(offsets[a]), int(offsets[a + 1])):
            rid = int(routes[pr])
            tok = rid // topk
            assert idx[tok, rid % topk] == e
            np.testing.assert_array_equal(got[pr], wint @ x8[tok])
            n_checked += 1
    assert n_checked == R
