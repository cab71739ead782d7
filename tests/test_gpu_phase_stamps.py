"""The fused kernel's phase stamps (the reference's phase_stamps facility: per workgroup, 100 MHz
wall clock at entry, dispatch table ready, L1 units done, the first L1 arrival the L2 phase
waited for, L2 units done, exit; then the wall ticks of the L1 K loops and of the L1
epilogues). Every workgroup of the launch writes its row; the stamps of a row are in phase
order, the two tick sums fit inside the row's span, and stamping does not change the output
(y and the recv stats bit for bit against the same call without stamps)."""
import numpy as np
import pytest
import torch

from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16

pytestmark = pytest.mark.gpu

H, I, TOPK = 512, 256, 4


@pytest.mark.parametrize("M,E", [(12, 16), (40, 160)])
@pytest.mark.parametrize("fmt", ["mxfp8", "qoq"])
def test_phase_stamps_ordered_and_harmless(fmt, M, E):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from tests.test_gpu_l2_halves import _weights, _fused
    print(f"phase stamps fmt={fmt} M={M} E={E}", flush=True)
    rng = np.random.default_rng(7400 + M + len(fmt))
    t1, t2 = _weights(fmt, E, 7401 + M)
    x = bf16_cpu(randn_bf16(rng, (M, H))).cuda()
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    out = []
    for stamped in (False, True):
        b = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, TOPK, H, I, act_format=fmt)
        y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
        stats = torch.zeros(E, dtype=torch.int32, device="cuda")
        dgm.fable_router_quant_topk_frontend(x, rw, b, select_in_mega=True)
        st = torch.zeros((2048, 8), dtype=torch.int64, device="cuda") if stamped else None
        if fmt == "qoq":
            dgm.qoq_mega_moe_fused(y, t1, t2, b, cumulative_local_expert_recv_stats=stats, phase_stamps=st)
        else:
            dgm.mxfp4_mega_moe_fused(y, t1, t2, b, cumulative_local_expert_recv_stats=stats, phase_stamps=st)
        torch.cuda.synchronize()
        assert b.kernel_error() == 0 and b.host_error() == 0
        out.append((y.clone(), stats.clone(), st, dgm.mega.fused_workgroups(b)))
    (y0, s0, _, _), (y1, s1, st, G) = out
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    assert torch.equal(s0, s1)
    a = st.cpu().numpy()
    assert 0 < G <= a.shape[0]
    rows, rest = a[:G], a[G:]
    assert (rest == 0).all(), "rows past the grid are left alone"
    entry, ready, l1, seen, l2, ex = (rows[:, i] for i in range(6))
    assert (entry > 0).all()
    assert (ready >= entry).all() and (l1 >= ready).all() and (l2 >= l1).all() and (ex >= l2).all()
    w = seen > 0
    assert ((seen[w] >= ready[w]) & (seen[w] <= ex[w])).all()
    span = ex - entry
    assert (rows[:, 6] >= 0).all() and (rows[:, 7] >= 0).all()
    assert (rows[:, 6] + rows[:, 7] <= span).all()
    # every workgroup enters before the launch's last exit (a short launch's workgroups need not
    # all be dispatched before the first exits: a few have entered 6-8 us late on some boxes)
    assert entry.max() <= ex.max()


def test_one_launch_stamps():
    """The one-launch layer (frontend in the fused kernel) stamps its frontend in [6] (this
    workgroup's router and cast work done) and [7] (the grid-wide arrival passed): in order
    with entry and the dispatch, and no workgroup passes the arrival before every workgroup has
    done its frontend work."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from tests.test_gpu_l2_halves import _weights
    M, E = 6, 16
    t1, t2 = _weights("mxfp8", E, 7501)
    rng = np.random.default_rng(7500)
    x = bf16_cpu(randn_bf16(rng, (M, H))).cuda()
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    b = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, TOPK, H, I, act_format="mxfp8")
    y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    st = torch.zeros((2048, 8), dtype=torch.int64, device="cuda")
    dgm.mxfp4_mega_moe_from_bf16(y, x, rw, t1, t2, b, one_launch=True, phase_stamps=st)
    torch.cuda.synchronize()
    assert b.kernel_error() == 0 and dgm.mega.fused_last_form(b) == 1
    G = dgm.mega.fused_workgroups(b)
    r = st.cpu().numpy()[:G]
    entry, ready, ex, fe, arr = r[:, 0], r[:, 1], r[:, 5], r[:, 6], r[:, 7]
    assert ((entry > 0) & (fe >= entry) & (arr >= fe) & (ready >= arr) & (ex >= ready)).all()
    assert arr.min() >= fe.max()


@pytest.mark.parametrize("M,act", [(8, "mxfp8"), (3, "qoq"), (64, "nvfp4")])
def test_frontend_stamps(M, act):
    """fable_frontend_stamps (deep_gemm/mega/__init__.py:743-756) after a frontend call with
    stamps=1: one row per frontend workgroup (router rows, then cast rows), entry <= the phase
    stamp <= exit in ns, the hardware position recorded, and the stamped call writes the same
    logits, keys and activation codes bit for bit as the call without stamps; no stamped call
    yet raises."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import _lib
    E, Hh = 384, 3072
    print(f"frontend stamps M={M} act={act}", flush=True)
    rng = np.random.default_rng(7500 + M)
    x = bf16_cpu(randn_bf16(rng, (M, Hh))).cuda()
    rw = bf16_cpu(randn_bf16(rng, (E, Hh), 0.02)).cuda()
    outs = []
    for stamps in (0, 1):
        b = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, 8, Hh, 1280, act_format=act)
        if not stamps:
            with pytest.raises(RuntimeError, match="stamps=1"):
                dgm.fable_frontend_stamps(b, E)
        dgm.fable_router_quant_topk_frontend(x, rw, b, select_in_mega=True, stamps=stamps)
        torch.cuda.synchronize()
        outs.append((b.logits[:M].clone(), b.fe_keys[:M].clone(), b.x[:M].clone(), b.x_sf[:M].clone(), b))
    for u, v in zip(outs[0][:4], outs[1][:4]):
        assert torch.equal(u.view(torch.uint8), v.view(torch.uint8))
    b = outs[1][4]
    st = dgm.fable_frontend_stamps(b, E).cpu().numpy()
    n_router = dgm.fable_frontend_router_ctas(M, E, Hh)
    assert st.shape[0] == _lib.load().dgm_frontend_workgroups(M, Hh, E, b.act_code, _lib.FE_SELECT_IN_MEGA |
                                                             _lib.FE_ZERO_ROW_UNROUTED, 1) > n_router
    entry, ex = st[:, 0], st[:, 7]
    assert (entry > 0).all() and (ex >= entry).all()
    r, c = st[:n_router], st[n_router:]
    assert ((r[:, 3] >= r[:, 0]) & (r[:, 3] <= r[:, 7]) & (r[:, 5] == 0)).all()
    assert ((c[:, 5] >= c[:, 0]) & (c[:, 5] <= c[:, 7]) & (c[:, 3] == 0)).all()
    assert (ex.max() - entry.min()) < 10_000_000          # one launch: well under 10 ms
    assert len(np.unique(st[:, 6])) > 1                    # workgroups on more than one CU / wave slot
