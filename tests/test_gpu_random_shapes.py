"""Seeded random layer shapes through the persistent kernel: expert counts, EP shares and ranks,
top-k from 1 to 16, token counts from 1 to 64, both A-MXFP formats, real or forced-balanced
routing, all-zero rows, the top-k selected in the frontend or in the kernel's prologue. Each case
is checked as the fixed-shape tests are: frontend keys, top-k and activation codes and the pool
table bit-exact against the oracle, recv stats, y within the north star's tolerance; and the
split launches give the fused kernel's y bit for bit."""
import numpy as np
import pytest
import torch

from tests.gpu_common import need_gpu
from tests.test_gpu_layer import make_weights, run_layer, check_frontend, check_pool, check_y

pytestmark = pytest.mark.gpu


def _cases(n=40, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        H, I = [(512, 256), (1024, 512)][int(rng.integers(2))]
        ep = [1, 2, 4][int(rng.integers(3))]
        e_local = int(rng.integers(2, 41))
        E = e_local * ep
        topk = int(rng.integers(1, min(16, E) + 1))
        M = int(rng.integers(1, 65))
        while M * topk > 512:
            M //= 2
        fmt = ["mxfp4", "mxfp8"][i % 2]
        balanced = E % topk == 0 and rng.random() < 0.5
        zero_rows = () if balanced or M < 3 else tuple(sorted(set(int(v) for v in rng.integers(0, M, int(rng.integers(0, 3))))))
        select = bool(rng.integers(2))
        rank = int(rng.integers(ep))
        out.append((i, M, E, e_local, rank * e_local, H, I, topk, fmt, balanced, zero_rows, select))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"case{c[0]}")
def test_random_shape(case):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    i, M, E, e_local, begin, H, I, topk, fmt, balanced, zero_rows, select = case
    print(f"random shape {i}: M={M} E={E} local={e_local}@{begin} H={H} I={I} topk={topk} {fmt} "
          f"balanced={balanced} zero_rows={zero_rows} select_in_mega={select}", flush=True)
    weights = make_weights(e_local, H, I, 9000 + i)
    r = run_layer(M, E, e_local, begin, H, I, topk, fmt, seed=9100 + i, force_balanced=balanced,
                  zero_rows=zero_rows, weights=weights, select_in_mega=select)
    check_frontend(r, fmt, M, force_balanced=balanced, zero_rows=zero_rows)
    check_pool(r, e_local, begin)
    check_y(r, zero_rows=zero_rows)
    (t1, t2), _, _ = weights
    y2 = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    dgm.mxfp4_mega_moe_split(y2, t1, t2, r["buf"], activation_clamp=10.0)
    torch.cuda.synchronize()
    assert r["buf"].kernel_error() == 0
    np.testing.assert_array_equal(y2.float().cpu().numpy(), r["y"])


@pytest.mark.parametrize("case", _cases(12, seed=2027), ids=lambda c: f"case{c[0]}")
def test_random_shape_qoq(case):
    """QoQ W4A8: the same random shapes (the format column ignored): frontend codes and scales,
    pool and stats bit-exact, intermediate codes against the exact-integer L1 restatement,
    y within tolerance."""
    need_gpu()
    from tests import test_gpu_qoq as tq
    i, M, E, e_local, begin, H, I, topk, _, balanced, zero_rows, select = case
    r = tq.run_qoq(M, E, e_local, begin, H, I, topk, seed=9300 + i, force_balanced=balanced, zero_rows=zero_rows,
                   select_in_mega=select)
    tq.check_frontend(r, M)
    tq.check_mid(r)
    tq.check_y(r, zero_rows=zero_rows)


@pytest.mark.parametrize("case", _cases(12, seed=2028), ids=lambda c: f"case{c[0]}")
def test_random_shape_nvfp4(case):
    """NVFP4 W4A4 (per-expert global scales on odd cases): frontend codes and scales, pool and
    stats bit-exact, y within tolerance; the split family (two launches) gives the fused
    launch's y bit for bit."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from tests import test_gpu_nvfp4 as tn
    i, M, E, e_local, begin, H, I, topk, _, balanced, zero_rows, select = case
    r = tn.run_nvfp4(M, E, e_local, begin, H, I, topk, seed=9500 + i, force_balanced=balanced, zero_rows=zero_rows,
                     select_in_mega=select, global_scales=bool(i % 2))
    tn.check_frontend(r, M)
    tn.check_pool(r)
    tn.check_y(r, zero_rows=zero_rows)
    (t1, t2), (gs1, gs2) = r["t"], r["gs"]
    gs = {} if gs1 is None else dict(l1_global_scales=torch.from_numpy(gs1).cuda(),
                                     l2_global_scales=torch.from_numpy(gs2).cuda())
    y2 = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    dgm.nvfp4_mega_moe(y2, t1, t2, r["buf"], activation_clamp=10.0, kernel_family="split", **gs)
    torch.cuda.synchronize()
    assert r["buf"].kernel_error() == 0
    np.testing.assert_array_equal(y2.float().cpu().numpy(), r["y"])


@pytest.mark.parametrize("case", _cases(16, seed=2029), ids=lambda c: f"case{c[0]}")
def test_random_shape_one_launch(case):
    """The one-launch layer (router, zero-row flags and cast in the fused kernel) against the
    two launches on the same inputs, every activation format in turn: frontend outputs, pool
    table and y bit for bit."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from tests.gpu_common import bf16_cpu, randn_bf16
    from tests.test_gpu_one_launch import weights_for, layer_two_launch, snapshot
    i, M, E, e_local, begin, H, I, topk, _, balanced, zero_rows, _ = case
    fmt = ["mxfp8", "mxfp4", "qoq", "nvfp4"][i % 4]
    print(f"one-launch random shape {i}: {fmt} M={M} E={E} local={e_local}@{begin} H={H} I={I} topk={topk} "
          f"balanced={balanced} zero_rows={zero_rows}", flush=True)
    rng = np.random.default_rng(9700 + i)
    x = randn_bf16(rng, (M, H))
    for r in zero_rows:
        x[r] = 0.0
    rw = randn_bf16(rng, (E, H), 0.02)
    xs, rws = bf16_cpu(x).cuda(), bf16_cpu(rw).cuda()
    t1, t2 = weights_for(fmt, e_local, H, I, 9701 + i)
    bufs = [dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format=fmt, ep_size=E // e_local,
                                                   ep_rank=begin // e_local) for _ in range(2)]
    y2 = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    layer_two_launch(dgm, fmt, y2, xs, rws, t1, t2, bufs[0], balanced)
    y1 = torch.full((M, H), 7.0, dtype=torch.bfloat16, device="cuda")
    dgm.mxfp4_mega_moe_from_bf16(y1, xs, rws, t1, t2, bufs[1], activation_clamp=10.0, force_balanced=balanced,
                                 one_launch=True)
    torch.cuda.synchronize()
    assert bufs[0].kernel_error() == 0 and bufs[1].kernel_error() == 0
    ref, got = snapshot(bufs[0], M), snapshot(bufs[1], M)
    for k in ref:
        a, r = got[k].cpu(), ref[k].cpu()
        if a.dtype == torch.float32:
            a, r = a.view(torch.int32), r.view(torch.int32)
        assert torch.equal(a, r), k
    for a, r in zip(bufs[1].pool_table(), bufs[0].pool_table()):
        assert torch.equal(a, r)
    assert torch.equal(y1.view(torch.int16).cpu(), y2.view(torch.int16).cpu())


def _form_cases(n=8, seed=2030):
    """Shapes where the opt-in forms apply: H = 3072, I = 1280, at most 32 routes."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        ep = [1, 2, 8][int(rng.integers(3))]
        e_local = int(rng.integers(4, 25))
        E = e_local * ep
        topk = int(rng.integers(1, min(8, E) + 1))
        M = int(rng.integers(1, 32 // topk + 1))
        out.append((i, M, E, e_local, int(rng.integers(ep)) * e_local, topk, ["mxfp4", "mxfp8"][i % 2]))
    return out


@pytest.mark.parametrize("case", _form_cases(), ids=lambda c: f"case{c[0]}")
def test_random_shape_opt_in_forms(case):
    """The opt-in kernel forms (early weight streaming, debug bit 3; tail half units, bit 4)
    against the default form on random small routed sets at H = 3072: y, recv stats and the
    intermediate rows bit for bit, and each form reported as the one that ran when its rule
    applies."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from tests.gpu_common import bf16_cpu, randn_bf16
    i, M, E, e_local, begin, topk, fmt = case
    H, I = 3072, 1280
    print(f"forms random shape {i}: {fmt} M={M} E={E} local={e_local}@{begin} topk={topk}", flush=True)
    rng = np.random.default_rng(9900 + i)
    x = bf16_cpu(randn_bf16(rng, (M, H))).cuda()
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    (t1, t2), _, _ = make_weights(e_local, H, I, 9901 + i)
    outs = {}
    for flags in (0, 8, 16):
        b = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format=fmt, ep_size=E // e_local,
                                                   ep_rank=begin // e_local)
        b._debug_flags = flags
        dgm.fable_router_quant_topk_frontend(x, rw, b)
        y = torch.full((M, H), 5.0, dtype=torch.bfloat16, device="cuda")
        stats = torch.zeros(e_local, dtype=torch.int32, device="cuda")
        dgm.mxfp4_mega_moe_fused(y, t1, t2, b, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)
        torch.cuda.synchronize()
        assert b.kernel_error() == 0 and b.host_error() == 0
        n = int(b.pool_table()[0].sum())
        outs[flags] = (dgm.mega.fused_last_form(b), y.view(torch.int16).cpu(), stats.cpu(),
                       b.l2_acts[:n].view(torch.uint8).cpu().clone(), b.l2_acts_sf[:n].view(torch.uint8).cpu().clone())
    R = M * topk
    assert outs[0][0] == 0
    if R <= 64 and R * e_local <= 32 * E:
        assert outs[8][0] == 2
    assert outs[16][0] == 3
    for flags in (8, 16):
        for a, r in zip(outs[flags][1:], outs[0][1:]):
            assert torch.equal(a, r), flags


@pytest.mark.parametrize("fmt", ["mxfp4", "mxfp8", "qoq", "nvfp4"])
def test_random_call_sequence(fmt):
    """One buffer through 30 calls of random token count (zero rows included) and random launch
    form: the fused launch with the top-k from the frontend or selected in its prologue, the
    split launches, the one-launch layer, and (A-MXFP) the early-streaming form and a
    cooperative launch. Every call equals a fresh buffer's fused launch bit for bit (y and the
    accumulated recv stats), with no device error: the buffer's two counter sets stay
    consistent whatever the sequence."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from tests.gpu_common import bf16_cpu, randn_bf16
    from tests.test_gpu_one_launch import weights_for
    E, H, I, topk, maxm = 24, 512, 256, 4, 24
    rng = np.random.default_rng(4300 + len(fmt))
    t1, t2 = weights_for(fmt, E, H, I, 4301)
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    fused = {"qoq": dgm.qoq_mega_moe_fused, "nvfp4": dgm.fp4_fp4_mega_moe}.get(fmt, dgm.mxfp4_mega_moe_fused)

    def split(y, b, stats):
        if fmt == "qoq":
            dgm.qoq_mega_moe_split(y, t1, t2, b, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)
        elif fmt == "nvfp4":
            dgm.nvfp4_mega_moe(y, t1, t2, b, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0,
                               kernel_family="split")
        else:
            dgm.mxfp4_mega_moe_split(y, t1, t2, b, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)

    def run(mode, y, x, b, stats):
        b._debug_flags = 8 if mode == "early" else 0
        b.cooperative = mode == "coop"
        if mode == "one":
            dgm.mxfp4_mega_moe_from_bf16(y, x, rw, t1, t2, b, cumulative_local_expert_recv_stats=stats,
                                         activation_clamp=10.0, one_launch=True)
        elif mode == "split":
            dgm.fable_router_quant_topk_frontend(x, rw, b)
            split(y, b, stats)
        else:
            dgm.fable_router_quant_topk_frontend(x, rw, b, select_in_mega=(mode == "select"))
            fused(y, t1, t2, b, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)

    modes = ["fused", "select", "split", "one"] + (["early", "coop"] if fmt in ("mxfp4", "mxfp8") else [])
    shared = dgm.get_fused_symm_buffer_for_mega_moe(None, E, maxm, topk, H, I, act_format=fmt)
    stats = torch.zeros(E, dtype=torch.int32, device="cuda")
    want = torch.zeros(E, dtype=torch.int32, device="cuda")
    for i in range(30):
        M = int(rng.integers(1, maxm + 1))
        mode = modes[int(rng.integers(len(modes)))]
        print(f"sequence {fmt} call {i}: M={M} mode={mode}", flush=True)
        xh = randn_bf16(rng, (M, H))
        if M > 3 and rng.random() < 0.5:
            xh[int(rng.integers(M))] = 0.0
        x = bf16_cpu(xh).cuda()
        fresh = dgm.get_fused_symm_buffer_for_mega_moe(None, E, maxm, topk, H, I, act_format=fmt)
        y_ref = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
        run("fused", y_ref, x, fresh, want)
        y = torch.full((M, H), 7.0, dtype=torch.bfloat16, device="cuda")
        run(mode, y, x, shared, stats)
        torch.cuda.synchronize()
        assert fresh.kernel_error() == 0 and shared.kernel_error() == 0 and shared.host_error() == 0, (i, M, mode)
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), (i, M, mode)
        assert torch.equal(stats, want), (i, M, mode)
