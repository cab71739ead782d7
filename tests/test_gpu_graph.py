"""HIP graph capture of the layer (the reference's tests capture it in a CUDA graph:
tests/profile_four_api_h20.py:216-221). The frontend and fused launches are captured once and
replayed with new inputs copied into the captured tensors; every replay must give the eager
result bit for bit (y, recv stats), and eager calls on the same buffer between replays must
too: the workspace counters return to zero at the end of every launch, and nothing on the call
path allocates, synchronises or writes memory with memset."""
import numpy as np
import pytest
import torch

from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16

pytestmark = pytest.mark.gpu


def _weights(fmt, E, H, I, seed):
    if fmt == "nvfp4":
        from tests.test_gpu_nvfp4 import make_nvfp4_weights
        return make_nvfp4_weights(E, H, I, seed)[0]
    if fmt == "qoq":
        from tests.test_gpu_qoq import make_qoq_weights
        return make_qoq_weights(E, H, I, seed)[0]
    from tests.test_gpu_layer import make_weights      # (MXFP4 weights, for either MXFP activation format)
    return make_weights(E, H, I, seed)[0]


@pytest.mark.parametrize("M", [6, 12])
@pytest.mark.parametrize("fmt", ["mxfp8", "nvfp4", "qoq"])
def test_graph_capture_replay(fmt, M):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    E, H, I, topk = 16, 512, 256, 4
    print(f"graph capture fmt={fmt} M={M} E={E} H={H} I={I}", flush=True)
    rng = np.random.default_rng(900 + M)
    t1, t2 = _weights(fmt, E, H, I, 901 + M)
    fused = {"qoq": dgm.qoq_mega_moe_fused, "nvfp4": dgm.fp4_fp4_mega_moe}.get(fmt, dgm.mxfp4_mega_moe_fused)
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format=fmt)
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    x = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    stats = torch.zeros(E, dtype=torch.int32, device="cuda")
    inputs = []
    for i in range(3):
        xi = randn_bf16(rng, (M, H))
        xi[i] = 0.0                       # a zero row (unrouted) in each input
        inputs.append(bf16_cpu(xi).cuda())

    def layer():
        dgm.fable_router_quant_topk_frontend(x, rw, buf, select_in_mega=True)
        fused(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)

    refs = []
    for xi in inputs:
        x.copy_(xi)
        stats.zero_()
        layer()
        torch.cuda.synchronize()
        assert buf.kernel_error() == 0
        refs.append((y.clone(), stats.clone()))
    x.copy_(inputs[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        layer()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer()
    torch.cuda.synchronize()
    for rep in range(6):
        i = rep % 3
        x.copy_(inputs[i])
        stats.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert buf.kernel_error() == 0
        assert torch.equal(y, refs[i][0]), (rep, i)
        assert torch.equal(stats, refs[i][1]), (rep, i)
        # an eager call on the same buffer between replays
        j = (i + 1) % 3
        x.copy_(inputs[j])
        stats.zero_()
        layer()
        torch.cuda.synchronize()
        assert torch.equal(y, refs[j][0]), (rep, j)
    print("replays match the eager results", flush=True)
