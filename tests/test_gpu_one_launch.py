"""The one-launch layer (``mxfp4_mega_moe_from_bf16(one_launch=True)``, up to 64 tokens: router, zero-row flags and
activation cast inside the fused kernel, before its top-k prologue) against the two-launch path
(``fable_router_quant_topk_frontend`` + the fused layer) on the same inputs: logits, top-k keys,
activation codes and scales, routing, pool and y must agree bit for bit (same device
arithmetic, same order), for every activation format, with zero rows and forced-balanced
routing, and on a second call (counters return to zero)."""
import numpy as np
import pytest
import torch

from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16

pytestmark = pytest.mark.gpu


def weights_for(fmt, E, H, I, seed):
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_mxfp4_fused as qf
    from hopper_megamoe_basedondeepgemm_amd import quantization_nvfp4 as qn
    from hopper_megamoe_basedondeepgemm_amd import quantization_qoq_fused as qq
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w1 = (torch.randn((E, 2 * I, H), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((E, H, I), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    if fmt == "qoq":
        return dgm.transform_qoq_weights_for_mega_moe_fused(qq.quantize_to_qoq(w1), qq.quantize_to_qoq(w2))
    if fmt == "nvfp4":
        return dgm.transform_nvfp4_weights_for_mega_moe_fused(qn.quantize_to_nvfp4(w1), qn.quantize_to_nvfp4(w2))
    return dgm.transform_mxfp4_weights_for_mega_moe_fused(qf.quantize_to_mxfp4(w1), qf.quantize_to_mxfp4(w2))


def layer_two_launch(dgm, fmt, y, x, rw, t1, t2, b, balanced):
    dgm.fable_router_quant_topk_frontend(x, rw, b, force_balanced=balanced, select_in_mega=True)
    if fmt == "qoq":
        dgm.qoq_mega_moe_fused(y, t1, t2, b)
    elif fmt == "nvfp4":
        dgm.fp4_fp4_mega_moe(y, t1, t2, b, activation_clamp=10.0)
    else:
        dgm.mxfp4_mega_moe_fused(y, t1, t2, b)


def snapshot(b, M):
    return {k: getattr(b, k)[:M].clone() for k in ("x", "x_sf", "topk_idx", "topk_weights", "logits",
                                                   "fe_keys")}


@pytest.mark.parametrize("fmt,balanced", [("mxfp8", True), ("mxfp4", False), ("qoq", False), ("nvfp4", True)])
def test_one_launch_matches_two_launch(fmt, balanced):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    M, E, H, I, topk = 12, 64, 1024, 512, 8
    print(f"one-launch fmt={fmt} balanced={balanced} M={M} E={E}", flush=True)
    rng = np.random.default_rng(900 + len(fmt))
    x = randn_bf16(rng, (M, H))
    x[4] = 0.0                                  # a zero row: unrouted
    rw = randn_bf16(rng, (E, H), 0.02)
    xs, rws = bf16_cpu(x).cuda(), bf16_cpu(rw).cuda()
    (t1, t2) = weights_for(fmt, E, H, I, 77)
    b2 = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format=fmt)
    b1 = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format=fmt)
    y2 = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    layer_two_launch(dgm, fmt, y2, xs, rws, t1, t2, b2, balanced)
    torch.cuda.synchronize()
    ref = snapshot(b2, M)
    for call in range(2):
        y1 = torch.full((M, H), 7.0, dtype=torch.bfloat16, device="cuda")
        clamp = 10.0
        dgm.mxfp4_mega_moe_from_bf16(y1, xs, rws, t1, t2, b1, activation_clamp=clamp, force_balanced=balanced,
                                     one_launch=True)
        torch.cuda.synchronize()
        assert b1.kernel_error() == 0
        got = snapshot(b1, M)
        for k in ref:
            a, r = got[k].cpu(), ref[k].cpu()
            if a.dtype in (torch.float32,):
                a, r = a.view(torch.int32), r.view(torch.int32)
            assert torch.equal(a, r), (call, k)
        for t1_, t2_ in zip(b1.pool_table(), b2.pool_table()):
            assert torch.equal(t1_, t2_), call
        assert torch.equal(y1.view(torch.int16).cpu(), y2.view(torch.int16).cpu()), call
        assert (y1[4] == 0).all()
