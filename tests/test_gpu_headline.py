"""GPU parity at every workload the bench times, at full size: benchmark config 2 (all 384
experts resident, W-MXFP4 x A-MXFP8 and x A-MXFP4, M=2/4/8/16 forced-balanced and M=16 seeded
unbalanced routing), config 3 (QoQ W4A8, M=2/4/8/16 forced-balanced) and config 4 (NVFP4 W4A4,
M=16, 64 and 128 seeded unbalanced; 128 tokens are the persistent kernel's 1024-route limit),
through the calls the bench makes: ``fable_router_quant_topk_frontend(...,
select_in_mega=True)`` then the fused layer. These shapes run the persistent kernel's dynamic
claim path (more L1 and L2 units than twice the grid) and its L1 -> L2 hand-off at the size the
bench times.

Bit-exact: the frontend's fp32 logits and top-k keys, top-k indices and slot order, activation
codes and scales, the pool table, the recv stats. Tolerance (the north star's bar): per-row
cos >= 0.9999 and rel-RMSE <= 0.5 % of y against the oracle (tests/test_four_api_correctness.py:
419-446; sm100_b200/test_mega_moe.py:411-488); the local routes' bf16 outputs
(``combine_partials``) against the oracle's per-route outputs: min cos >= 0.999, rel-RMSE <= 0.5 %."""
import numpy as np
import pytest
import torch

from oracle import numerics as nu
from oracle import packers as pk
from oracle import moe
from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16, oracle_routes_parallel, active_local_experts

pytestmark = pytest.mark.gpu

E, H, I, TOPK = 384, 3072, 1280, 8
COS_MIN = 0.9999
REL_RMSE_MAX = 0.005
ROUTE_COS_MIN = 0.999


def _chunked(fill, seed, shapes, chunk=32):
    """Seeded bf16 ~N(0, 0.02) weights of every shape in `shapes`, drawn on the GPU in chunks of
    experts and handed to fill(i_shape, e0, e1, w_bf16)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    for i, (N, K) in enumerate(shapes):
        for e0 in range(0, E, chunk):
            e1 = min(E, e0 + chunk)
            w = (torch.randn((e1 - e0, N, K), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
            fill(i, e0, e1, w)
            del w


@pytest.fixture(scope="module")
def mxfp4_weights():
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_mxfp4_fused as qf
    q = [(torch.empty((E, N, K // 2), dtype=torch.uint8, device="cuda"),
          torch.empty((E, N, K // 32), dtype=torch.uint8, device="cuda")) for N, K in ((2 * I, H), (H, I))]

    def fill(i, e0, e1, w):
        q[i][0][e0:e1], q[i][1][e0:e1] = qf.quantize_to_mxfp4(w)
    _chunked(fill, 1234, ((2 * I, H), (H, I)))
    t = dgm.transform_mxfp4_weights_for_mega_moe_fused(q[0], q[1])
    torch.cuda.synchronize()
    return t, q


@pytest.fixture(scope="module")
def qoq_weights():
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_qoq_fused as qq
    q = [(torch.empty((E, N, K // 2), dtype=torch.uint8, device="cuda"),
          torch.empty((E, N, K // 128), dtype=torch.uint8, device="cuda"),
          torch.empty((E, N, K // 128), dtype=torch.uint8, device="cuda"),
          torch.empty((E, N), dtype=torch.float32, device="cuda")) for N, K in ((2 * I, H), (H, I))]

    def fill(i, e0, e1, w):
        for dst, src in zip(q[i], qq.quantize_to_qoq(w)):
            dst[e0:e1] = src
    _chunked(fill, 4321, ((2 * I, H), (H, I)))
    t = dgm.transform_qoq_weights_for_mega_moe_fused(q[0], q[1])
    torch.cuda.synchronize()
    return t, q


@pytest.fixture(scope="module")
def nvfp4_weights():
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_nvfp4 as qn
    q = [(torch.empty((E, N, K // 2), dtype=torch.uint8, device="cuda"),
          torch.empty((E, N, K // 16), dtype=torch.uint8, device="cuda")) for N, K in ((2 * I, H), (H, I))]

    def fill(i, e0, e1, w):
        q[i][0][e0:e1], q[i][1][e0:e1] = qn.quantize_to_nvfp4(w)
    _chunked(fill, 5678, ((2 * I, H), (H, I)))
    t = dgm.transform_nvfp4_weights_for_mega_moe_fused(q[0], q[1])
    torch.cuda.synchronize()
    return t, q


def _fetch(q, experts):
    """The packed bytes of the given experts of every tensor of q (W1's, then W2's), as numpy
    arrays per expert."""
    sel = torch.tensor(experts, dtype=torch.long, device="cuda")
    host = [t.index_select(0, sel).cpu().numpy() for mat in q for t in mat]
    return {e: tuple(h[i] for h in host) for i, e in enumerate(experts)}


def _deq_qoq(p, s2, z, s1):
    return pk.dequantize_qoq(p[None], s2[None], z[None], s1[None])[0]


def run_headline(fmt, M, balanced, seed, weights):
    import hopper_megamoe_basedondeepgemm_amd as dgm
    print(f"headline parity: fmt={fmt} E={E} (all resident) M={M} balanced={balanced} seed={seed}", flush=True)
    (t1, t2), q = weights
    rng = np.random.default_rng(seed)
    x = randn_bf16(rng, (M, H))
    rw = randn_bf16(rng, (E, H), 0.02)
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, TOPK, H, I, act_format=fmt)
    stats = torch.zeros(E, dtype=torch.int32, device="cuda")
    y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    xs, rws = bf16_cpu(x).cuda(), bf16_cpu(rw).cuda()
    dgm.fable_router_quant_topk_frontend(xs, rws, buf, force_balanced=balanced, select_in_mega=True)
    fused = {"qoq": dgm.qoq_mega_moe_fused, "nvfp4": dgm.fp4_fp4_mega_moe}.get(fmt, dgm.mxfp4_mega_moe_fused)
    if fmt == "nvfp4":
        fused(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)
    else:
        fused(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats)
    torch.cuda.synchronize()
    assert buf.kernel_error() == 0 and buf.host_error() == 0
    # ---- frontend and routing, bit-exact
    logits = moe.router_logits_f32(x, rw)
    np.testing.assert_array_equal(buf.logits[:M].cpu().numpy().view(np.uint32), logits.view(np.uint32))
    keys = moe.topk_keys(nu.f32_to_bf16_bits(logits), E)
    np.testing.assert_array_equal(buf.fe_keys[:M].cpu().numpy().view(np.uint32), keys)
    idx, w, _ = moe.topk_softmax(logits, TOPK)
    if balanced:
        idx, w = moe.balanced_routing(M, E, TOPK)
    np.testing.assert_array_equal(buf.topk_idx[:M].cpu().numpy(), idx)
    np.testing.assert_allclose(buf.topk_weights[:M].cpu().numpy(), w, rtol=1e-6, atol=0)
    codes, sf, x_dq = moe.quant_act(x, fmt)
    np.testing.assert_array_equal(buf.x[:M].cpu().numpy().view(np.uint8), np.asarray(codes).view(np.uint8))
    if fmt == "qoq":
        got_sf = buf.x_sf[:M].cpu().numpy()
        np.testing.assert_array_equal(got_sf.view(np.uint32), np.repeat(sf[:, None], got_sf.shape[1], 1).view(np.uint32))
    else:
        np.testing.assert_array_equal(buf.x_sf[:M].cpu().numpy(), sf)
    counts, active, offsets, routes = buf.pool_table()
    rc, ra, ro, rr = moe.dispatch(idx, 0, E)
    np.testing.assert_array_equal(counts.numpy(), rc)
    np.testing.assert_array_equal(active.numpy(), ra)
    np.testing.assert_array_equal(offsets.numpy(), ro)
    np.testing.assert_array_equal(routes.numpy(), rr)
    np.testing.assert_array_equal(stats.cpu().numpy(), rc)
    # ---- y and the route outputs against the oracle
    experts = active_local_experts(idx, 0, E)
    host = _fetch(q, experts)
    if fmt == "qoq":
        ex = {e: (v[0:4], v[4:8]) for e, v in host.items()}
        ref, ref_routes = oracle_routes_parallel(x_dq, idx, w, ex, _deq_qoq, _deq_qoq, 0, E, I, "qoq",
                                                 bf16_gate_up=False)
    else:
        deq = pk.dequantize_nvfp4 if fmt == "nvfp4" else pk.dequantize_mxfp4_marlin
        ex = {e: (v[0:2], v[2:4]) for e, v in host.items()}
        ref, ref_routes = oracle_routes_parallel(x_dq, idx, w, ex, deq, deq, 0, E, I, fmt)
    yv = y.float().cpu().numpy()
    m = moe.metrics(yv, ref)
    assert m["cos_min"] >= COS_MIN and m["rel_rmse"] <= REL_RMSE_MAX, m
    part = buf.combine_partials[:, :M].float().cpu().numpy()        # [slot, token, H]
    rids = sorted(ref_routes)
    got_r = np.stack([part[r % TOPK, r // TOPK] for r in rids])
    want_r = np.stack([ref_routes[r] for r in rids])
    mr = moe.metrics(got_r, want_r)
    assert mr["cos_min"] >= ROUTE_COS_MIN and mr["rel_rmse"] <= REL_RMSE_MAX, mr
    print(f"  active experts {len(experts)}  y {m}  routes {mr}", flush=True)
    return m


@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
def test_config2_m8_balanced(mxfp4_weights, fmt):
    """The headline step (config 2, M=8 forced-balanced: 64 active experts, 1280 L1 and 768 L2
    units), both activation formats."""
    run_headline(fmt, 8, True, 508, mxfp4_weights)


@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
def test_config2_m16_unbalanced(mxfp4_weights, fmt):
    """Config 2's unbalanced run (M=16, seeded N(0,1) hidden states through the router: > 8
    tokens, so the top-k is selected by its own launch before the fused kernel)."""
    run_headline(fmt, 16, False, 777, mxfp4_weights)


def test_config2_m2_m4_balanced(mxfp4_weights):
    """The small-M end of the sweep (the claim counters start beyond the first units only from
    M=4 on; M=2 runs every unit from the workgroups' first two)."""
    run_headline("mxfp8", 2, True, 502, mxfp4_weights)
    run_headline("mxfp4", 4, True, 504, mxfp4_weights)


@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
def test_config2_small_m_kernel_forms_match(mxfp4_weights, fmt):
    """At the bench's M=2 and M=4 (forced-balanced, 384 resident experts: 320 and 640 L1 units on
    256 workgroups), the default form and the opt-in early-weight-streaming (debug flag bit 3) and
    tail-half-unit (bit 4) forms give the same y, route outputs, intermediate rows and recv stats
    bit for bit."""
    import hopper_megamoe_basedondeepgemm_amd as dgm
    (t1, t2), _ = mxfp4_weights
    for M in (2, 4):
        print(f"kernel forms at full size: fmt={fmt} M={M}", flush=True)
        rng = np.random.default_rng(520 + M)
        x = bf16_cpu(randn_bf16(rng, (M, H))).cuda()
        rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
        buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, TOPK, H, I, act_format=fmt)
        outs = []
        for flags in (0, 8, 16):
            buf._debug_flags = flags
            dgm.fable_router_quant_topk_frontend(x, rw, buf, force_balanced=True, select_in_mega=True)
            y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
            stats = torch.zeros(E, dtype=torch.int32, device="cuda")
            dgm.mxfp4_mega_moe_fused(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats)
            torch.cuda.synchronize()
            assert buf.kernel_error() == 0 and buf.host_error() == 0
            assert dgm.mega.fused_last_form(buf) == {0: 0, 8: 2, 16: 3}[flags]
            n = int(buf.pool_table()[0].sum())
            outs.append((y.view(torch.int16).cpu(), stats.cpu(), buf.combine_partials[:, :M].view(torch.int16).cpu(),
                         buf.l2_acts[:n].view(torch.uint8).cpu(), buf.l2_acts_sf[:n].cpu()))
        for o in outs[1:]:
            for name, u, v in zip(("y", "stats", "partials", "mid", "mid_sf"), outs[0], o):
                assert torch.equal(u, v), name


def test_config3_qoq_m8_balanced(qoq_weights):
    """Config 3: the QoQ W4A8 layer with 384 resident experts, M=8 forced-balanced."""
    run_headline("qoq", 8, True, 508, qoq_weights)


@pytest.mark.parametrize("M", [16, 64])
def test_config4_nvfp4_unbalanced(nvfp4_weights, M):
    """Config 4: the NVFP4 W4A4 layer with 384 resident experts and seeded unbalanced routing."""
    run_headline("nvfp4", M, False, 900 + M, nvfp4_weights)


@pytest.mark.parametrize("fmt", ["mxfp8", "mxfp4"])
def test_config2_m16_balanced(mxfp4_weights, fmt):
    """Config 2 at M=16 forced-balanced (128 active experts, 2560 L1 and 1536 L2 units: the
    sweep's best-fraction point), both activation formats. Forced-balanced routing at 16 tokens
    is selected in the fused kernel's prologue."""
    run_headline(fmt, 16, True, 516, mxfp4_weights)


@pytest.mark.parametrize("M", [2, 4, 16])
def test_config3_qoq_sweep_balanced(qoq_weights, M):
    """Config 3's other timed points: QoQ W4A8 with 384 resident experts at M=2, 4 and 16
    forced-balanced."""
    run_headline("qoq", M, True, 600 + M, qoq_weights)


def test_config4_nvfp4_m128_unbalanced(nvfp4_weights):
    """Config 4 at M=128 (seeded unbalanced routing over 384 resident experts): 1024 routes, the
    persistent kernel's limit, with the most active experts of any timed point."""
    run_headline("nvfp4", 128, False, 1028, nvfp4_weights)
