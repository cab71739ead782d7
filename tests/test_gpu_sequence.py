"""One layer buffer driven through a sequence of calls that differ in token count and launch
form: the fused launch (top-k selected in its prologue, by a selection launch, or by the
frontend), the split launches and the one-launch layer, back to back. Each launch uses one of
the buffer's two counter sets, clears the other for the next launch and hands it over at its end,
so every call's output must equal a fresh buffer's bit for bit (y and the recv stats, which
accumulate over the sequence), with no device error. Bit-exact against the fresh buffer's fused
launch, whose own parity with the oracle the layer tests check."""
import numpy as np
import pytest
import torch

from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16

pytestmark = pytest.mark.gpu

E, H, I, TOPK, MAXM = 16, 512, 256, 4, 12
SEQUENCE = [(12, "fused"), (3, "split"), (8, "one"), (1, "fused"), (12, "split"), (5, "one"),
            (9, "fused_fe"), (7, "fused"), (12, "one"), (2, "split"), (10, "fused")]


def _weights(fmt, seed):
    if fmt == "qoq":
        from tests.test_gpu_qoq import make_qoq_weights
        return make_qoq_weights(E, H, I, seed)[0]
    from tests.test_gpu_layer import make_weights
    return make_weights(E, H, I, seed)[0]


def _entries(dgm, fmt):
    if fmt == "qoq":
        return dgm.qoq_mega_moe_fused, dgm.qoq_mega_moe_split
    return dgm.mxfp4_mega_moe_fused, dgm.mxfp4_mega_moe_split


def _call(dgm, fmt, mode, y, x, rw, t1, t2, b, stats):
    fused, split = _entries(dgm, fmt)
    if mode == "one":
        dgm.mxfp4_mega_moe_from_bf16(y, x, rw, t1, t2, b, cumulative_local_expert_recv_stats=stats, one_launch=True)
    elif mode == "split":
        dgm.fable_router_quant_topk_frontend(x, rw, b)
        split(y, t1, t2, b, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)
    else:
        dgm.fable_router_quant_topk_frontend(x, rw, b, select_in_mega=(mode == "fused"))
        fused(y, t1, t2, b, cumulative_local_expert_recv_stats=stats)


@pytest.mark.parametrize("fmt", ["mxfp8", "qoq"])
def test_mixed_launch_sequence_on_one_buffer(fmt):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    rng = np.random.default_rng(4242 + len(fmt))
    t1, t2 = _weights(fmt, 4243)
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    shared = dgm.get_fused_symm_buffer_for_mega_moe(None, E, MAXM, TOPK, H, I, act_format=fmt)
    stats = torch.zeros(E, dtype=torch.int32, device="cuda")
    want_stats = torch.zeros(E, dtype=torch.int32, device="cuda")
    for i, (M, mode) in enumerate(SEQUENCE):
        print(f"sequence fmt={fmt} call {i}: M={M} mode={mode}", flush=True)
        xh = randn_bf16(rng, (M, H))
        if M > 4:
            xh[i % M] = 0.0                   # a zero row: unrouted
        x = bf16_cpu(xh).cuda()
        fresh = dgm.get_fused_symm_buffer_for_mega_moe(None, E, MAXM, TOPK, H, I, act_format=fmt)
        y_ref = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
        _call(dgm, fmt, "fused_fe", y_ref, x, rw, t1, t2, fresh, want_stats)
        y = torch.full((M, H), 7.0, dtype=torch.bfloat16, device="cuda")
        _call(dgm, fmt, mode, y, x, rw, t1, t2, shared, stats)
        torch.cuda.synchronize()
        assert fresh.kernel_error() == 0 and shared.kernel_error() == 0, (i, M, mode)
        assert shared.host_error() == 0, (i, M, mode)
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), (i, M, mode)
        assert torch.equal(stats, want_stats), (i, M, mode)
