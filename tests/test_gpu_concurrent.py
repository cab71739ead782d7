"""The persistent kernel launched while another stream's kernel holds part of the GPU: the fused
kernel's workgroups that cannot start yet are waited for (bounded waits of seconds), so a layer
call that overlaps finite work elsewhere is only delayed: y and the recv stats equal the same
call run alone, bit for bit, with no device error."""
import numpy as np
import pytest
import torch

from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16

pytestmark = pytest.mark.gpu

E, H, I, TOPK = 48, 3072, 1280, 8


@pytest.mark.parametrize("fmt", ["mxfp8", "nvfp4"])
def test_layer_overlapping_another_streams_kernels(fmt):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from tests.test_gpu_one_launch import weights_for
    print(f"concurrent streams fmt={fmt}", flush=True)
    rng = np.random.default_rng(5100 + len(fmt))
    t1, t2 = weights_for(fmt, E, H, I, 5101)
    rw = bf16_cpu(randn_bf16(rng, (E, H), 0.02)).cuda()
    M = 8
    x = bf16_cpu(randn_bf16(rng, (M, H))).cuda()
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, TOPK, H, I, act_format=fmt)
    fused = dgm.fp4_fp4_mega_moe if fmt == "nvfp4" else dgm.mxfp4_mega_moe_fused

    def layer(y, stats):
        dgm.fable_router_quant_topk_frontend(x, rw, buf, select_in_mega=True)
        fused(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats, activation_clamp=10.0)

    y_ref = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    s_ref = torch.zeros(E, dtype=torch.int32, device="cuda")
    layer(y_ref, s_ref)
    torch.cuda.synchronize()
    assert buf.kernel_error() == 0
    other = torch.cuda.Stream()                  # default priority
    big = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    for rep in range(4):
        y = torch.full((M, H), 3.0, dtype=torch.bfloat16, device="cuda")
        stats = torch.zeros(E, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        with torch.cuda.stream(other):
            for _ in range(4):                   # ~1 GiB elementwise passes, many short workgroups
                big.mul_(1.0)
        layer(y, stats)                          # on the current stream, while `other` runs
        torch.cuda.synchronize()
        assert buf.kernel_error() == 0 and buf.host_error() == 0, rep
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), rep
        assert torch.equal(stats, s_ref), rep
