"""GPU parity of the split API on the reference's own buffer and weights (deep_gemm/mega/__init__.py:
20-127 SymmBuffer / get_symm_buffer_for_mega_moe, :257 transform_mxfp4_weights_for_mega_moe_sm90,
:340-448 mxfp4_mega_moe / int4_mega_moe), driven the way tests/test_four_api_correctness.py drives
it: x / x_sf from ``per_token_cast_to_fp8(x, use_ue8m0=False, gran_k=128)`` (QoQ:
``per_token_cast_to_int8``) and the routing copied into the buffer, or the router inputs.

Bit-exact: the activation cast of ``hidden_input``, the routing from ``router_logits`` (both
weight rules) and from ``router_input``, the pool table, QoQ through ``int4_mega_moe`` against
``qoq_mega_moe_fused``. Tolerance (the north star's bar, as T4:419-446): y per-row cos >= 0.9999
and rel-RMSE <= 0.5 % against the oracle (fp32 gate / up, per-64 power-of-two FP8 intermediate,
routes rounded to bf16, slot-order fp32 sum); routes: min cos >= 0.999."""
import numpy as np
import pytest
import torch

from oracle import numerics as nu
from oracle import packers as pk
from oracle import moe
from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16, oracle_routes_parallel, active_local_experts

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
REL_RMSE_MAX = 0.005


def _split_weights(E, H, I, seed, scale=0.02):
    """bf16 weights drawn on the GPU, packed by the split packer (deep_gemm/quantization_mxfp4.py:52,
    Marlin order), transformed by transform_mxfp4_weights_for_mega_moe_sm90."""
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_mxfp4 as qs
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w1 = (torch.randn((E, 2 * I, H), generator=g, device="cuda") * scale).to(torch.bfloat16)
    q1 = qs.quantize_to_mxfp4(w1)
    del w1
    w2 = (torch.randn((E, H, I), generator=g, device="cuda") * scale).to(torch.bfloat16)
    q2 = qs.quantize_to_mxfp4(w2)
    del w2
    t = dgm.transform_mxfp4_weights_for_mega_moe_sm90(q1, q2)
    torch.cuda.synchronize()
    return t, q1, q2


def _oracle(x_dq, idx, w, q1, q2, I, act):
    experts = active_local_experts(idx, 0, q1[0].shape[0])
    sel = torch.tensor(experts, dtype=torch.long, device="cuda")
    host = [t.index_select(0, sel).cpu().numpy() for t in (q1[0], q1[1], q2[0], q2[1])]
    ex = {e: ((host[0][i], host[1][i]), (host[2][i], host[3][i])) for i, e in enumerate(experts)}
    deq = pk.dequantize_mxfp4_marlin
    return oracle_routes_parallel(x_dq, idx, w, ex, deq, deq, 0, q1[0].shape[0], I, act, bf16_gate_up=False)


def _random_routing(rng, M, E, topk):
    idx = np.stack([rng.choice(E, topk, replace=False) for _ in range(M)]).astype(np.int64)
    w = rng.random((M, topk)).astype(np.float32)
    return idx, (w / w.sum(1, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("M,E,H,I,balanced", [(5, 16, 512, 256, False), (16, 48, 1024, 512, False),
                                              (8, 48, 3072, 1280, True)])
def test_mxfp4_mega_moe_fp8xmxfp4(M, E, H, I, balanced):
    """T4's split call: x / x_sf / topk written into the buffer, then the layer."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    topk = 8
    print(f"split api fp8xmxfp4 M={M} E={E} H={H} I={I} balanced={balanced}", flush=True)
    (t1, t2), q1, q2 = _split_weights(E, H, I, 100 + M)
    rng = np.random.default_rng(7 + M)
    x = randn_bf16(rng, (M, H))
    xq, xs = pk.per_token_cast_to_fp8_f32sf(x, 128)
    idx, w = moe.balanced_routing(M, E, topk) if balanced else _random_routing(rng, M, E, topk)
    buf = dgm.get_symm_buffer_for_mega_moe(None, E, M, topk, H, I, mma_type="fp8xmxfp4", activation="swiglu")
    assert buf.x.dtype == torch.float8_e4m3fn and buf.x_sf.dtype == torch.float32
    assert tuple(buf.x_sf.shape) == (M, H // 128)
    buf.x[:M].copy_(torch.from_numpy(xq).view(torch.float8_e4m3fn).cuda())
    buf.x_sf[:M].copy_(torch.from_numpy(xs).cuda())
    buf.topk_idx[:M].copy_(torch.from_numpy(idx).cuda())
    buf.topk_weights[:M].copy_(torch.from_numpy(w).cuda())
    y = torch.zeros((M, H), dtype=torch.bfloat16, device="cuda")
    stats = torch.zeros(E, dtype=torch.int32, device="cuda")
    dgm.mxfp4_mega_moe(y, t1, t2, buf, cumulative_local_expert_recv_stats=stats, recipe=(128, 128, 128),
                       activation_clamp=10.0)
    torch.cuda.synchronize()
    counts, active, offsets, routes = buf.pool_table()
    rc, ra, ro, rr = moe.dispatch(idx, 0, E)
    np.testing.assert_array_equal(counts.numpy(), rc)
    np.testing.assert_array_equal(routes.numpy(), rr)
    np.testing.assert_array_equal(stats.cpu().numpy(), rc)
    x_dq = pk.dequant_fp8_rows(xq, xs, 128)
    ref, ref_routes = _oracle(x_dq, idx, w, q1, q2, I, "fp8f128")
    m = moe.metrics(y.float().cpu().numpy(), ref)
    assert m["cos_min"] >= COS_MIN and m["rel_rmse"] <= REL_RMSE_MAX, m
    part = buf.combine_partials[:, :M].float().cpu().numpy()
    rids = sorted(ref_routes)
    mr = moe.metrics(np.stack([part[r % topk, r // topk] for r in rids]), np.stack([ref_routes[r] for r in rids]))
    assert mr["cos_min"] >= 0.999 and mr["rel_rmse"] <= REL_RMSE_MAX, mr
    print(f"  y {m}  routes {mr}", flush=True)


def test_hidden_input_cast_and_router_logits():
    """hidden_input: the buffer's x / x_sf are the fp32-scale-per-128 cast, bit for bit;
    router_logits (bf16): top-k by value (ties: the lower expert), softmax weights or (no
    renormalisation) the logits themselves; then the layer as with the cast written by hand."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    M, E, H, I, topk = 12, 32, 1024, 512, 8
    (t1, t2), q1, q2 = _split_weights(E, H, I, 301)
    rng = np.random.default_rng(302)
    x = randn_bf16(rng, (M, H))
    x[3, :128] = 0.0                           # an all-zero 128-group: amax floor 1e-4
    logits = randn_bf16(rng, (M, E))
    logits[5, 7] = logits[5, 9] = np.float32(4.0)      # a tie between two top logits
    buf = dgm.get_symm_buffer_for_mega_moe(None, E, M, topk, H, I, mma_type="fp8xmxfp4")
    y = torch.zeros((M, H), dtype=torch.bfloat16, device="cuda")
    xg, lg = bf16_cpu(x).cuda(), bf16_cpu(logits).cuda()
    for renorm in (True, False):
        dgm.mxfp4_mega_moe(y, t1, t2, buf, router_logits=lg, router_renormalize=renorm, hidden_input=xg,
                           activation_clamp=10.0)
        torch.cuda.synchronize()
        xq, xs = pk.per_token_cast_to_fp8_f32sf(x, 128)
        np.testing.assert_array_equal(buf.x[:M].view(torch.uint8).cpu().numpy(), xq)
        np.testing.assert_array_equal(buf.x_sf[:M].cpu().numpy().view(np.uint32), xs.view(np.uint32))
        idx, w, _ = moe.topk_softmax(logits, topk)
        assert idx[5, 0] == 7 and idx[5, 1] == 9
        if not renorm:
            w = np.take_along_axis(logits, idx, 1).astype(np.float32)
        np.testing.assert_array_equal(buf.topk_idx[:M].cpu().numpy(), idx)
        np.testing.assert_allclose(buf.topk_weights[:M].cpu().numpy(), w, rtol=1e-6, atol=0)
        if renorm:
            ref, _ = _oracle(pk.dequant_fp8_rows(xq, xs, 128), idx, w, q1, q2, I, "fp8f128")
            m = moe.metrics(y.float().cpu().numpy(), ref)
            assert m["cos_min"] >= COS_MIN and m["rel_rmse"] <= REL_RMSE_MAX, m


def test_router_input_leaves_x():
    """router_input + router_weight: the router and top-k alone (the frontend's fixed-order fp32
    logits, top-k of their bf16 keys, softmax); x / x_sf stay as written."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    M, E, H, I, topk = 6, 16, 512, 256, 8
    (t1, t2), q1, q2 = _split_weights(E, H, I, 401)
    rng = np.random.default_rng(402)
    x = randn_bf16(rng, (M, H))
    ri = randn_bf16(rng, (M, H))
    rw = randn_bf16(rng, (E, H), 0.02)
    xq, xs = pk.per_token_cast_to_fp8_f32sf(x, 128)
    buf = dgm.get_symm_buffer_for_mega_moe(None, E, M, topk, H, I, mma_type="fp8xmxfp4")
    buf.x[:M].copy_(torch.from_numpy(xq).view(torch.float8_e4m3fn).cuda())
    buf.x_sf[:M].copy_(torch.from_numpy(xs).cuda())
    y = torch.zeros((M, H), dtype=torch.bfloat16, device="cuda")
    dgm.mxfp4_mega_moe(y, t1, t2, buf, router_input=bf16_cpu(ri).cuda(), router_weight=bf16_cpu(rw).cuda(),
                       activation_clamp=10.0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(buf.x[:M].view(torch.uint8).cpu().numpy(), xq)
    idx, w, _ = moe.topk_softmax(moe.router_logits_f32(ri, rw), topk)
    np.testing.assert_array_equal(buf.topk_idx[:M].cpu().numpy(), idx)
    np.testing.assert_allclose(buf.topk_weights[:M].cpu().numpy(), w, rtol=1e-6, atol=0)
    ref, _ = _oracle(pk.dequant_fp8_rows(xq, xs, 128), idx, w, q1, q2, I, "fp8f128")
    m = moe.metrics(y.float().cpu().numpy(), ref)
    assert m["cos_min"] >= COS_MIN and m["rel_rmse"] <= REL_RMSE_MAX, m


def test_int4_mega_moe_on_split_buffer():
    """int4_mega_moe (the same entry) with QoQ int4 weights on the fp8xmxfp4 buffer, x written as
    T4 writes it (per_token_cast_to_int8 bytes, the token's scale repeated): y equals
    qoq_mega_moe_fused on a QoQ fused buffer bit for bit."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_mxfp4 as qq
    M, E, H, I, topk = 8, 16, 1024, 512, 8
    g = torch.Generator(device="cuda")
    g.manual_seed(501)
    w1 = (torch.randn((E, 2 * I, H), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((E, H, I), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    t = dgm.transform_qoq_int4_weights_for_mega_moe_sm90(qq.quantize_to_qoq_int4(w1), qq.quantize_to_qoq_int4(w2))
    rng = np.random.default_rng(502)
    x = randn_bf16(rng, (M, H))
    idx, w = _random_routing(rng, M, E, topk)
    q8, s8 = pk.per_token_cast_to_int8(x)
    buf = dgm.get_symm_buffer_for_mega_moe(None, E, M, topk, H, I, mma_type="fp8xmxfp4")
    buf.x[:M].copy_(torch.from_numpy(q8).view(torch.float8_e4m3fn).cuda())
    buf.x_sf[:M].copy_(torch.from_numpy(np.repeat(s8[:, None], H // 128, 1)).cuda())
    buf.topk_idx[:M].copy_(torch.from_numpy(idx).cuda())
    buf.topk_weights[:M].copy_(torch.from_numpy(w).cuda())
    y = torch.zeros((M, H), dtype=torch.bfloat16, device="cuda")
    dgm.int4_mega_moe(y, *t, buf, recipe=(128, 128, 128), activation_clamp=10.0)
    fb = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, topk, H, I, act_format="qoq")
    fb.x[:M].copy_(torch.from_numpy(q8).cuda())
    fb.x_sf[:M].copy_(torch.from_numpy(np.repeat(s8[:, None], H // 128, 1)).cuda())
    fb.topk_idx[:M].copy_(torch.from_numpy(idx).cuda())
    fb.topk_weights[:M].copy_(torch.from_numpy(w).cuda())
    y2 = torch.zeros_like(y)
    dgm.qoq_mega_moe_fused(y2, t[0], t[1], fb, activation_clamp=10.0)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and y.float().abs().max() > 0
    np.testing.assert_array_equal(y.view(torch.int16).cpu().numpy(), y2.view(torch.int16).cpu().numpy())


def test_fp8xfp4_buffer_views():
    """mma_type="fp8xfp4": x E4M3 with the UE8M0 scales of each 32 packed four to an int32
    (x_sf int32 [tokens, H/128]); the layer is the MXFP8 one."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    M, E, H, I, topk = 4, 16, 512, 256, 8
    buf = dgm.get_symm_buffer_for_mega_moe(None, E, M, topk, H, I, mma_type="fp8xfp4")
    assert buf.x.dtype == torch.float8_e4m3fn and buf.x_sf.dtype == torch.int32
    assert tuple(buf.x_sf.shape) == (M, H // 128)
    with pytest.raises(ValueError):
        dgm.get_symm_buffer_for_mega_moe(None, E, M, topk, H, I, mma_type="bf16xbf16")
