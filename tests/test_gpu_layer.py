"""GPU parity of the frontend and the fused layer against the oracle.

Bit-exact: fp32 router logits (fixed accumulation order), top-k indices and slot order,
activation codes and scales, pool membership and order, recv stats. Tolerance (the bar the
north star states): per-row cos >= 0.9999 and rel-RMSE <= 0.5 % of the bf16 output against
the fp32-accumulated oracle (the intermediate requant codes depend on the fp32 order)."""
import numpy as np
import pytest
import torch

from oracle import numerics as nu
from oracle import packers as pk
from oracle import moe
from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
REL_RMSE_MAX = 0.005


def make_weights(E, H, I, seed, scale=0.02):
    """bf16 weights drawn on the GPU (seeded), packed on the GPU by the HIP packer; returns
    the transformed weights and lazily dequantised oracle views of the packed bytes."""
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_mxfp4_fused as qf
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w1 = (torch.randn((E, 2 * I, H), generator=g, device="cuda", dtype=torch.float32) * scale).to(torch.bfloat16)
    q1 = qf.quantize_to_mxfp4(w1)
    del w1
    w2 = (torch.randn((E, H, I), generator=g, device="cuda", dtype=torch.float32) * scale).to(torch.bfloat16)
    q2 = qf.quantize_to_mxfp4(w2)
    del w2
    t = dgm.transform_mxfp4_weights_for_mega_moe_fused(q1, q2)
    W1 = moe.LazyDequant(q1[0].cpu().numpy(), q1[1].cpu().numpy())
    W2 = moe.LazyDequant(q2[0].cpu().numpy(), q2[1].cpu().numpy())
    return t, W1, W2


def run_layer(M, E, E_local, expert_begin, H, I, topk, fmt, seed, force_balanced=False, zero_rows=(),
              max_tokens=None, weights=None, ep=None, select_in_mega=False, split=False):
    import hopper_megamoe_basedondeepgemm_amd as dgm
    rng = np.random.default_rng(seed)
    x = randn_bf16(rng, (M, H))
    for r in zero_rows:
        x[r] = 0.0
    rw = randn_bf16(rng, (E, H), 0.02)
    if weights is None:
        weights = make_weights(E_local, H, I, seed + 1)
    (t1, t2), W1, W2 = weights
    ep_size, ep_rank = ep if ep else (E // E_local, expert_begin // E_local)
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, max_tokens or M, topk, H, I, act_format=fmt,
                                                 ep_size=ep_size, ep_rank=ep_rank)
    xs, rws = bf16_cpu(x).cuda(), bf16_cpu(rw).cuda()
    stats = torch.arange(E_local, dtype=torch.int32, device="cuda")
    y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    dgm.fable_router_quant_topk_frontend(xs, rws, buf, force_balanced=force_balanced, select_in_mega=select_in_mega)
    layer = dgm.mxfp4_mega_moe_split if split else dgm.mxfp4_mega_moe_fused
    layer(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)
    torch.cuda.synchronize()
    # ---- oracle
    logits = moe.router_logits_f32(x, rw)
    idx, w, _ = moe.topk_softmax(logits, topk)
    if force_balanced:
        idx, w = moe.balanced_routing(M, E, topk)
    for r in zero_rows:
        idx[r] = -1
        w[r] = 0.0
    codes, sfb, x_dq = moe.quant_act(x, fmt)
    ref, _ = moe.moe_forward(x_dq, idx, w, W1, W2, expert_begin, fmt)
    return dict(buf=buf, y=y.float().cpu().numpy(), ref=ref, logits=logits, idx=idx, w=w, codes=codes,
                sfb=sfb, stats=stats.cpu().numpy(), x=x)


def check_frontend(r, fmt, M, force_balanced=False, zero_rows=()):
    b = r["buf"]
    if not force_balanced:
        got = b.logits[:M].cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint32), r["logits"].view(np.uint32))
    keys = moe.topk_keys(nu.f32_to_bf16_bits(r["logits"]), b.num_experts)
    keys[list(zero_rows)] = 0                  # all-zero rows: unrouted (zero keys)
    np.testing.assert_array_equal(b.fe_keys[:M].cpu().numpy().view(np.uint32), keys)
    np.testing.assert_array_equal(b.topk_idx[:M].cpu().numpy(), r["idx"])
    np.testing.assert_allclose(b.topk_weights[:M].cpu().numpy(), r["w"], rtol=1e-6, atol=0)
    np.testing.assert_array_equal(b.x[:M].cpu().numpy(), r["codes"])
    np.testing.assert_array_equal(b.x_sf[:M].cpu().numpy(), r["sfb"])


def check_pool(r, E_local, expert_begin):
    counts, active, offsets, routes = r["buf"].pool_table()
    rc, ra, ro, rr = moe.dispatch(r["idx"], expert_begin, E_local)
    np.testing.assert_array_equal(counts.numpy(), rc)
    np.testing.assert_array_equal(active.numpy(), ra)
    np.testing.assert_array_equal(offsets.numpy(), ro)
    np.testing.assert_array_equal(routes.numpy(), rr)
    np.testing.assert_array_equal(r["stats"], np.arange(E_local) + rc)


def check_y(r, zero_rows=()):
    assert r["buf"].kernel_error() == 0
    for zr in zero_rows:
        assert (r["y"][zr] == 0).all()
    keep = [i for i in range(r["y"].shape[0]) if i not in zero_rows]
    m = moe.metrics(r["y"][keep], r["ref"][keep])
    assert m["cos_min"] >= COS_MIN and m["rel_rmse"] <= REL_RMSE_MAX, m
    return m


@pytest.mark.parametrize("fmt", ["mxfp4", "mxfp8"])
def test_small_layer(fmt):
    need_gpu()
    M, E, H, I, topk = 6, 16, 512, 256, 4
    r = run_layer(M, E, E, 0, H, I, topk, fmt, seed=100)
    check_frontend(r, fmt, M)
    check_pool(r, E, 0)
    print(fmt, check_y(r))


@pytest.mark.parametrize("fmt", ["mxfp4", "mxfp8"])
def test_config0_shape(fmt):
    """benchmark config 0: E=48, H=3072, I=1280, top-8, M=2, real (unbalanced) routing."""
    need_gpu()
    r = run_layer(2, 48, 48, 0, 3072, 1280, 8, fmt, seed=200)
    check_frontend(r, fmt, 2)
    check_pool(r, 48, 0)
    print(fmt, check_y(r))


def test_config1_ep_share():
    """benchmark config 1: 384-way router, forced-balanced, one EP rank's share (experts 0..47)
    on one GPU, M=8 -> 8 rows over 48 local experts, output = the local partial."""
    need_gpu()
    r = run_layer(8, 384, 48, 0, 3072, 1280, 8, "mxfp4", seed=300, force_balanced=True)
    check_frontend(r, "mxfp4", 8, force_balanced=True)
    check_pool(r, 48, 0)
    assert int((r["buf"].pool_table()[0] > 0).sum()) == 8
    print(check_y(r))


def test_zero_rows_and_multi_slab():
    """All-zero rows are unrouted and give y == 0 exactly; 40 tokens on 8 experts put > 16
    routes on an expert (several 16-token slabs)."""
    need_gpu()
    r = run_layer(40, 8, 8, 0, 512, 256, 4, "mxfp4", seed=400, zero_rows=(3, 17))
    check_frontend(r, "mxfp4", 40, zero_rows=(3, 17))
    check_pool(r, 8, 0)
    assert r["buf"].pool_table()[0].max() > 16
    print(check_y(r, zero_rows=(3, 17)))


def test_second_ep_rank_and_replay():
    """A rank other than 0 (experts 16..31 of 64) and two calls in a row (stats accumulate,
    the result is identical)."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    weights = make_weights(16, 512, 256, 501)
    r = run_layer(5, 64, 16, 16, 512, 256, 4, "mxfp8", seed=500, weights=weights)
    check_pool(r, 16, 16)
    check_y(r)
    (t1, t2), _, _ = weights
    y2 = torch.empty((5, 512), dtype=torch.bfloat16, device="cuda")
    dgm.mxfp4_mega_moe_fused(y2, t1, t2, r["buf"])
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y2.float().cpu().numpy(), r["y"])
    assert r["buf"].kernel_error() == 0


@pytest.mark.parametrize("fmt", ["mxfp4", "mxfp8"])
def test_split_matches_fused(fmt):
    """The split API (separate launches) gives the fused kernel's result bit for bit."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    weights = make_weights(48, 3072, 1280, 601)
    r = run_layer(3, 48, 48, 0, 3072, 1280, 8, fmt, seed=600, weights=weights)
    check_y(r)
    (t1, t2), _, _ = weights
    y2 = torch.empty((3, 3072), dtype=torch.bfloat16, device="cuda")
    dgm.mxfp4_mega_moe_split(y2, t1, t2, r["buf"], activation_clamp=10.0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y2.float().cpu().numpy(), r["y"])


@pytest.mark.parametrize("fmt", ["mxfp4", "mxfp8"])
def test_select_in_mega(fmt):
    """Top-k selected in the fused kernel's prologue (frontend with select_in_mega): the same
    routing, weights and output; topk_idx / topk_weights are written by the fused call."""
    need_gpu()
    M, E, H, I, topk = 6, 16, 512, 256, 4
    r = run_layer(M, E, E, 0, H, I, topk, fmt, seed=100, select_in_mega=True)
    check_frontend(r, fmt, M)
    check_pool(r, E, 0)
    print(fmt, check_y(r))


def test_select_in_mega_zero_rows_multi_slab_and_split():
    """select_in_mega with zero rows and > 16 routes per expert; and through the split API
    (which materialises the top-k in a separate launch first)."""
    need_gpu()
    for split in (False, True):
        r = run_layer(40, 8, 8, 0, 512, 256, 4, "mxfp4", seed=400, zero_rows=(3, 17), select_in_mega=True,
                      split=split)
        check_frontend(r, "mxfp4", 40, zero_rows=(3, 17))
        check_pool(r, 8, 0)
        print(split, check_y(r, zero_rows=(3, 17)))


@pytest.mark.parametrize("M", [8, 16])
def test_select_in_mega_config1_balanced(M):
    """benchmark config 1 with the forced-balanced rule applied in the fused kernel's prologue
    (forced-balanced routing is selected there up to 16 tokens, real top-k up to 8)."""
    need_gpu()
    print(f"select_in_mega config 1 balanced M={M}", flush=True)
    r = run_layer(M, 384, 48, 0, 3072, 1280, 8, "mxfp4", seed=300 + M, force_balanced=True, select_in_mega=True)
    check_frontend(r, "mxfp4", M, force_balanced=True)
    check_pool(r, 48, 0)
    print(check_y(r))


@pytest.mark.parametrize("M,E,H", [(64, 48, 3072), (77, 48, 3072), (130, 20, 512)])
def test_frontend_router_tiles(M, E, H):
    """From 64 tokens on the frontend's router workgroups stage 8 hidden rows in LDS and share
    them over four experts: logits and keys bit-exact against the oracle as on the one-wave
    path, including a ragged last tile (rows past M clamped, not written), zero rows and an
    expert count that is not a multiple of four; top-k, weights and activation codes too."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    print(f"frontend router tiles M={M} E={E} H={H}", flush=True)
    rng = np.random.default_rng(5100 + M)
    x = randn_bf16(rng, (M, H))
    zero_rows = (0, M - 1, M // 2)
    for r in zero_rows:
        x[r] = 0.0
    rw = randn_bf16(rng, (E, H), 0.02)
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, 8, H, 256, act_format="mxfp4")
    dgm.fable_router_quant_topk_frontend(bf16_cpu(x).cuda(), bf16_cpu(rw).cuda(), buf)
    torch.cuda.synchronize()
    logits = moe.router_logits_f32(x, rw)
    idx, w, _ = moe.topk_softmax(logits, 8)
    for r in zero_rows:
        idx[r] = -1
        w[r] = 0.0
    codes, sfb, _ = moe.quant_act(x, "mxfp4")
    check_frontend(dict(buf=buf, logits=logits, idx=idx, w=w, codes=codes, sfb=sfb), "mxfp4", M,
                   zero_rows=zero_rows)


@pytest.mark.parametrize("select_in_mega", [False, True])
def test_maximum_router_width_and_topk(select_in_mega):
    """The router's limits: 1024 experts and top-16 (an EP rank's 64 local experts of them),
    12 tokens (the top-k of a separate selection launch either way above 8 tokens): logits,
    keys, top-k and weights bit-exact, pool table, y within tolerance."""
    need_gpu()
    print(f"max router width E=1024 topk=16 select_in_mega={select_in_mega}", flush=True)
    r = run_layer(12, 1024, 64, 64, 512, 256, 16, "mxfp8", seed=960, zero_rows=(5,), select_in_mega=select_in_mega)
    check_frontend(r, "mxfp8", 12, zero_rows=(5,))
    check_pool(r, 64, 64)
    print(check_y(r, zero_rows=(5,)))


@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
def test_persistent_kernel_at_its_limits(fmt):
    """256 tokens at top-4: exactly the persistent kernel's 1024 routes and 256 tokens (its LDS
    tables full), unbalanced routing with zero rows: frontend, pool table and y as elsewhere."""
    need_gpu()
    print(f"persistent kernel limits fmt={fmt} M=256 topk=4", flush=True)
    r = run_layer(256, 16, 16, 0, 512, 256, 4, fmt, seed=970, zero_rows=(0, 255))
    check_frontend(r, fmt, 256, zero_rows=(0, 255))
    check_pool(r, 16, 0)
    print(check_y(r, zero_rows=(0, 255)))


def test_large_batch_beyond_fused_limits():
    """200 tokens at top-8: 1600 routes exceed the persistent kernel's 1024, so the fused entry
    point runs the split path (dispatch, L1, L2, combine kernels); frontend, pool and y as
    everywhere else."""
    need_gpu()
    r = run_layer(200, 16, 16, 0, 512, 256, 8, "mxfp4", seed=950, zero_rows=(7,))
    check_frontend(r, "mxfp4", 200, zero_rows=(7,))
    check_pool(r, 16, 0)
    print(check_y(r, zero_rows=(7,)))


def test_fe_keys_honoured():
    """A caller's key array (the reference's fe_keys: orderable bf16 << 16 | 0xFFFF - e, a zero
    first key = unrouted) is what the fused layer selects from: keys of other logits than the
    router's give that routing (top-k, weights, pool, y), and a zero key row gives y == 0.
    fable_frontend_keys is the buffer's own key array (bit-exact against the oracle)."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    M, E, H, I, topk = 6, 16, 512, 256, 4
    weights = make_weights(E, H, I, 1101)
    (t1, t2), W1, W2 = weights
    rng = np.random.default_rng(1100)
    x = randn_bf16(rng, (M, H))
    rw = randn_bf16(rng, (E, H), 0.02)
    other = randn_bf16(rng, (M, E))                        # logits of another router
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format="mxfp8")
    xs, rws = bf16_cpu(x).cuda(), bf16_cpu(rw).cuda()
    dgm.fable_router_quant_topk_frontend(xs, rws, buf, select_in_mega=True)
    torch.cuda.synchronize()
    own = moe.topk_keys(nu.f32_to_bf16_bits(moe.router_logits_f32(x, rw)), E)
    np.testing.assert_array_equal(dgm.fable_frontend_keys(buf).view(M, E).cpu().numpy().view(np.uint32), own)
    keys = moe.topk_keys(nu.f32_to_bf16_bits(other), E).astype(np.uint32)
    keys[2] = 0                                             # token 2 unrouted
    fk = torch.from_numpy(keys.view(np.int32)).cuda()
    y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    dgm.mxfp4_mega_moe_fused(y, t1, t2, buf, fe_keys=fk)
    torch.cuda.synchronize()
    assert buf.kernel_error() == 0
    idx, w, _ = moe.topk_softmax(other, topk)
    idx[2] = -1
    w[2] = 0.0
    np.testing.assert_array_equal(buf.topk_idx[:M].cpu().numpy(), idx)
    np.testing.assert_allclose(buf.topk_weights[:M].cpu().numpy(), w, rtol=1e-6, atol=0)
    _, _, x_dq = moe.quant_act(x, "mxfp8")
    ref, _ = moe.moe_forward(x_dq, idx, w, W1, W2, 0, "mxfp8")
    yv = y.float().cpu().numpy()
    assert (yv[2] == 0).all()
    keep = [i for i in range(M) if i != 2]
    m = moe.metrics(yv[keep], ref[keep])
    assert m["cos_min"] >= COS_MIN and m["rel_rmse"] <= REL_RMSE_MAX, m


def test_expired_wait_is_reported(monkeypatch):
    """A bounded wait that expires (forced by the test hook: a wait on a counter nothing sets,
    with a zero spin limit) sets the buffer's error counter and its host-visible word; the next
    call on the buffer raises without synchronising; DG_CHECK_ERRORS=1 raises at once;
    clear_error() makes the buffer usable again with unchanged results."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    weights = make_weights(16, 512, 256, 1201)
    r = run_layer(5, 16, 16, 0, 512, 256, 4, "mxfp4", seed=1200, weights=weights)
    check_y(r)
    b = r["buf"]
    (t1, t2), _, _ = weights
    y = torch.empty((5, 512), dtype=torch.bfloat16, device="cuda")
    b._debug_flags = 1
    dgm.mxfp4_mega_moe_fused(y, t1, t2, b)
    torch.cuda.synchronize()
    assert b.kernel_error() == 1 and b.host_error() == 1
    b._debug_flags = 0
    with pytest.raises(RuntimeError, match="bounded wait"):
        dgm.mxfp4_mega_moe_fused(y, t1, t2, b)
    b.clear_error()
    assert b.kernel_error() == 0 and b.host_error() == 0
    monkeypatch.setenv("DG_CHECK_ERRORS", "1")
    b._debug_flags = 1
    with pytest.raises(RuntimeError, match="bounded wait"):
        dgm.mxfp4_mega_moe_fused(y, t1, t2, b)
    b._debug_flags = 0
    b.clear_error()
    dgm.mxfp4_mega_moe_fused(y, t1, t2, b)
    torch.cuda.synchronize()
    assert b.kernel_error() == 0
    np.testing.assert_array_equal(y.float().cpu().numpy(), r["y"])


@pytest.mark.parametrize("fmt", ["mxfp8", "qoq", "nvfp4"])
def test_cooperative_launch_matches_plain(fmt):
    """The opt-in cooperative launch of the persistent kernel (``buffer.cooperative`` /
    DG_MEGA_COOPERATIVE=1: co-residency guaranteed for callers sharing the GPU) gives the plain
    launch's y and recv stats bit for bit, on the same grid."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from tests.test_gpu_l2_halves import _weights, _fused
    M, E, H, I = 12, 16, 512, 256
    print(f"cooperative vs plain launch fmt={fmt}", flush=True)
    rng = np.random.default_rng(7600 + len(fmt))
    t1, t2 = _weights(fmt, E, 7601)
    x = bf16_cpu(randn_bf16(rng, (M, H))).cuda()
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    b = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, 4, H, I, act_format=fmt)
    out = []
    for coop in (False, True):
        b.cooperative = coop
        assert dgm.mega.cooperative_launch(b) == coop
        dgm.fable_router_quant_topk_frontend(x, rw, b, select_in_mega=True)
        y = torch.full((M, H), 9.0, dtype=torch.bfloat16, device="cuda")
        stats = torch.zeros(E, dtype=torch.int32, device="cuda")
        _fused(dgm, fmt, y, t1, t2, b, stats)
        torch.cuda.synchronize()
        assert b.kernel_error() == 0 and b.host_error() == 0
        out.append((y.view(torch.int16).cpu(), stats.cpu(), dgm.mega.fused_workgroups(b)))
    (y0, s0, g0), (y1, s1, g1) = out
    assert torch.equal(y0, y1) and torch.equal(s0, s1) and g0 == g1 > 0
