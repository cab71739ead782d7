"""GPU parity: matrix-core lane layout, packers and the weight-layout transform (bit-exact)."""
import numpy as np
import pytest
import torch

from oracle import numerics as nu
from oracle import packers as pk
from tests.gpu_common import need_gpu, bf16_cpu, randn_bf16, decode_native, interleave16

pytestmark = pytest.mark.gpu


def _probe(fa, fb, seed, sel=None):
    from hopper_megamoe_basedondeepgemm_amd import _lib
    rng = np.random.default_rng(seed)
    nbytes_a = 16 if fa == 4 else 32
    nbytes_b = 16 if fb == 4 else 32
    a = np.zeros((64, 32), np.uint8)
    b = np.zeros((64, 32), np.uint8)
    if fa == 4:
        a[:, :16] = rng.integers(0, 256, (64, 16), dtype=np.uint8)
    else:
        a[:, :] = nu.e4m3_encode(rng.standard_normal((64, 32)).astype(np.float32))
    if fb == 4:
        b[:, :16] = rng.integers(0, 256, (64, 16), dtype=np.uint8)
    else:
        b[:, :] = nu.e4m3_encode(rng.standard_normal((64, 32)).astype(np.float32))
    sa = rng.integers(120, 134, 64).astype(np.int32)
    sb = rng.integers(120, 134, 64).astype(np.int32)
    dev = torch.device("cuda")
    ta, tb = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    tsa, tsb = torch.from_numpy(sa).to(dev), torch.from_numpy(sb).to(dev)
    out = torch.zeros(64 * 4, dtype=torch.float32, device=dev)
    if sel is None:
        _lib.check(_lib.load_probe().dgm_probe_mfma_scale(_lib.ptr(ta), _lib.ptr(tb), _lib.ptr(tsa), _lib.ptr(tsb),
                                                    _lib.ptr(out), fa, fb, _lib.stream()))
    else:
        # the scale sits in byte `sel` of each word; the other bytes hold other (wrong) codes
        noise = rng.integers(100, 150, (2, 64, 4)).astype(np.int64)
        noise[0, :, sel] = sa
        noise[1, :, sel] = sb
        wa = (noise[0] << np.array([0, 8, 16, 24])).sum(-1).astype(np.uint32).view(np.int32)
        wb = (noise[1] << np.array([0, 8, 16, 24])).sum(-1).astype(np.uint32).view(np.int32)
        tsa, tsb = torch.from_numpy(wa).to(dev), torch.from_numpy(wb).to(dev)
        _lib.check(_lib.load_probe().dgm_probe_mfma_scale_sel(_lib.ptr(ta), _lib.ptr(tb), _lib.ptr(tsa), _lib.ptr(tsb),
                                                        _lib.ptr(out), sel, _lib.stream()))
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(64, 4)

    def vals(x, f):
        if f == 4:
            nib = np.stack([x[:, :16] & 0xF, x[:, :16] >> 4], -1).reshape(64, 32)
            return nu.e2m1_decode(nib).astype(np.float64)
        return nu.e4m3_decode(x).astype(np.float64)
    A = np.zeros((16, 128))
    B = np.zeros((128, 16))

    def kmap(f, l):
        g = l // 16
        if f == 4:                      # E2M1: 32 consecutive K per lane
            return np.arange(32 * g, 32 * g + 32)
        return np.concatenate([np.arange(16 * g, 16 * g + 16), np.arange(64 + 16 * g, 80 + 16 * g)])
    for l in range(64):
        A[l % 16, kmap(fa, l)] = vals(a, fa)[l]
        B[kmap(fb, l), l % 16] = vals(b, fb)[l]
    # the scale of lane l applies to row/column l%16 over the 32-block 32*(l//16)
    for l in range(64):
        A[l % 16, 32 * (l // 16):32 * (l // 16) + 32] *= nu.e8m0_to_f32(sa[l])
        B[32 * (l // 16):32 * (l // 16) + 32, l % 16] *= nu.e8m0_to_f32(sb[l])
    D = A @ B
    exp = np.zeros((64, 4))
    for l in range(64):
        for i in range(4):
            exp[l, i] = D[4 * (l // 16) + i, l % 16]
    return got, exp


@pytest.mark.parametrize("fa,fb", [(4, 4), (4, 0)])
def test_mfma_scale_lane_layout(fa, fb):
    need_gpu()
    for seed in range(3):
        got, exp = _probe(fa, fb, seed)
        np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-6 * np.abs(exp).max())


@pytest.mark.parametrize("sel", [0, 1, 2, 3])
def test_mfma_scale_byte_select(sel):
    """op_sel of the block-scale operands picks byte `sel` of the 32-bit scale word."""
    need_gpu()
    got, exp = _probe(4, 4, 10 + sel, sel=sel)
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-6 * np.abs(exp).max())


def test_packers_bit_exact():
    need_gpu()
    from hopper_megamoe_basedondeepgemm_amd import quantization_mxfp4_fused as qf, quantization_mxfp4 as qs
    from hopper_megamoe_basedondeepgemm_amd import quantization_nvfp4 as qn, quantization_qoq_fused as qq
    from hopper_megamoe_basedondeepgemm_amd import utils as du
    rng = np.random.default_rng(11)
    w = randn_bf16(rng, (3, 64, 512), 0.02)
    w[0, 0, :32] = 0.0
    w[0, 1, :32] = np.float32(-1e-3)
    w[0, 1, 5] = np.float32(0.75)
    w[0, 2] = np.tile(np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5, 6], np.float32) / 8, 64)
    tw = bf16_cpu(w).cuda()
    for fn, ref in ((qf.quantize_to_mxfp4, pk.quantize_to_mxfp4_fused),
                    (qs.quantize_to_mxfp4, pk.quantize_to_mxfp4_split),
                    (qn.quantize_to_nvfp4, pk.quantize_to_nvfp4)):
        p, s = fn(tw)
        rp, rs = ref(w)
        np.testing.assert_array_equal(s.cpu().numpy(), rs)
        np.testing.assert_array_equal(p.cpu().numpy(), rp)
    p, s2, z, s1 = qq.quantize_to_qoq(tw)
    rp, rs2, rz, rs1 = pk.quantize_to_qoq(w)
    np.testing.assert_array_equal(s1.cpu().numpy(), rs1)
    np.testing.assert_array_equal(s2.cpu().numpy(), rs2)
    np.testing.assert_array_equal(z.cpu().numpy(), rz)
    np.testing.assert_array_equal(p.cpu().numpy(), rp)

    x = randn_bf16(rng, (5, 3072))
    x[0, :32] = 0
    tx = bf16_cpu(x).cuda()
    q, sf = qq.per_token_cast_to_int8(tx)
    rq, rsf = pk.per_token_cast_to_int8(x)
    np.testing.assert_array_equal(q.cpu().numpy(), rq)
    np.testing.assert_array_equal(sf[:, 0].cpu().numpy(), rsf)
    p4, sf4 = du.per_token_cast_to_fp4(tx)
    rp4, rsf4 = pk.per_token_cast_to_fp4(x)
    np.testing.assert_array_equal(p4.cpu().numpy(), rp4)
    np.testing.assert_array_equal(sf4.cpu().numpy(), rsf4)
    p4, sf4 = du.per_token_cast_to_fp4(tx, amax_floor=1e-30)
    rp4, rsf4, _ = pk.cast_to_fp4_rows(x)
    np.testing.assert_array_equal(p4.cpu().numpy(), rp4)
    np.testing.assert_array_equal(sf4.cpu().numpy(), rsf4)
    q8, sf8 = du.per_token_cast_to_fp8(tx)
    rq8, rsf8 = pk.per_token_cast_to_fp8_ue8m0(x)
    np.testing.assert_array_equal(q8.view(torch.uint8).cpu().numpy(), rq8)
    np.testing.assert_array_equal(sf8.cpu().numpy(), rsf8)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_packers_take_fp32_and_fp16_weights(dtype):
    """The weight packers read bf16, fp16 or fp32 weights at their fp32 value, as the reference's
    do (weight.to(torch.float32): deep_gemm/quantization_mxfp4_fused.py:36, quantization_mxfp4.py:54,
    quantization_nvfp4.py:62, quantization_qoq_fused.py:20): codes and scales bit-exact against the
    oracle on the same values, with values that bf16 cannot hold, an all-zero group, an amax a
    hair above 6 * 2^k (where the log2 rule keeps 2^k) and E2M1 midpoints."""
    need_gpu()
    from hopper_megamoe_basedondeepgemm_amd import quantization_mxfp4_fused as qf, quantization_mxfp4 as qs
    from hopper_megamoe_basedondeepgemm_amd import quantization_nvfp4 as qn, quantization_qoq_fused as qq
    rng = np.random.default_rng(17)
    w = (rng.standard_normal((3, 64, 512)) * 0.02).astype(np.float32)
    w[0, 0, :32] = 0.0
    w[0, 1, 3] = np.float32(6.0 * 2.0 ** -9) * np.float32(1 + 2 ** -22)      # amax / 6 a hair above 2^-9
    w[0, 2] = np.tile(np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5, 6], np.float32) / 8, 64)
    if dtype == torch.float16:
        w = w.astype(np.float16).astype(np.float32)
    else:
        assert (nu.round_bf16(w) != w).mean() > 0.9          # mostly values bf16 cannot hold
    tw = torch.from_numpy(w).to(dtype).cuda()
    print(f"packers from {dtype}", flush=True)
    for fn, ref in ((qf.quantize_to_mxfp4, pk.quantize_to_mxfp4_fused),
                    (qs.quantize_to_mxfp4, pk.quantize_to_mxfp4_split),
                    (qn.quantize_to_nvfp4, pk.quantize_to_nvfp4)):
        p, s = fn(tw)
        rp, rs = ref(w)
        np.testing.assert_array_equal(s.cpu().numpy(), rs)
        np.testing.assert_array_equal(p.cpu().numpy(), rp)
    p, s2, z, s1 = qq.quantize_to_qoq(tw)
    rp, rs2, rz, rs1 = pk.quantize_to_qoq(w)
    np.testing.assert_array_equal(s1.cpu().numpy(), rs1)
    np.testing.assert_array_equal(s2.cpu().numpy(), rs2)
    np.testing.assert_array_equal(z.cpu().numpy(), rz)
    np.testing.assert_array_equal(p.cpu().numpy(), rp)
    p, plane = qs.quantize_to_qoq_int4(tw)
    rp, rplane = pk.quantize_to_qoq_int4(w)
    np.testing.assert_array_equal(plane.cpu().numpy(), rplane)
    np.testing.assert_array_equal(p.cpu().numpy(), rp)
    with pytest.raises(TypeError, match="bf16, fp16 or fp32"):
        qf.quantize_to_mxfp4(tw.double())


def test_transform_dequant_invariant():
    """dequant(transform(q)) == interleave(dequant(q)) (the reference's transform check,
    tests/test_mxfp4_mega_moe_sm90_correctness.py:153-182), for L1 (interleaved) and L2."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_mxfp4_fused as qf
    rng = np.random.default_rng(12)
    w1 = randn_bf16(rng, (2, 64, 640), 0.05)      # K = 640: 5 K-tiles, padded scale group
    w2 = randn_bf16(rng, (2, 32, 256), 0.05)
    q1 = qf.quantize_to_mxfp4(bf16_cpu(w1).cuda())
    q2 = qf.quantize_to_mxfp4(bf16_cpu(w2).cuda())
    (v1, s1, _), (v2, s2, _) = dgm.transform_mxfp4_weights_for_mega_moe_fused(q1, q2)
    torch.cuda.synchronize()
    d1 = pk.dequantize_mxfp4_marlin(q1[0].cpu().numpy(), q1[1].cpu().numpy())
    d2 = pk.dequantize_mxfp4_marlin(q2[0].cpu().numpy(), q2[1].cpu().numpy())
    np.testing.assert_array_equal(decode_native(v1.cpu().numpy(), s1.cpu().numpy()), interleave16(d1))
    np.testing.assert_array_equal(decode_native(v2.cpu().numpy(), s2.cpu().numpy()), d2)
    # padding scale bytes of the last (partial) group are 2^0
    assert (s1.cpu().numpy()[:, :, -1, :, 1:] == 127).all()
    # low-nibble-first sources give the same layout
    lf = pk.pack_low_first(pk.unpack_marlin(q2[0].cpu().numpy()))
    (u1, t1, _), (u2, t2, _) = dgm.transform_mxfp4_weights_for_mega_moe_fused(
        (q1[0], q1[1]), (torch.from_numpy(lf).cuda(), q2[1]), src_order="low_first")
    np.testing.assert_array_equal(u2.cpu().numpy(), v2.cpu().numpy())


def _i8_kmap(layout, l):
    g = l // 16
    if layout == "contiguous":                 # lane bytes j -> K = 16 g + j
        return np.arange(16 * g, 16 * g + 16)
    # split halves: bytes 0-7 -> K = 8 g .. +8, bytes 8-15 -> K = 32 + 8 g .. +8
    return np.concatenate([np.arange(8 * g, 8 * g + 8), np.arange(32 + 8 * g, 40 + 8 * g)])


def test_mfma_i8_lane_layout():
    """V_MFMA_I32_16X16X64_I8 (the W4A8 path): lane l supplies A row l%16 / B column l%16,
    16 int8 K values; result register i of lane l is D[4*(l/16)+i][l%16], exact int32. The
    K order of a lane's 16 bytes is the one the W4A8 kernels assume (``I8_KMAP``)."""
    need_gpu()
    from hopper_megamoe_basedondeepgemm_amd import _lib
    rng = np.random.default_rng(21)
    a = rng.integers(-128, 128, (64, 16), dtype=np.int64).astype(np.int8)
    b = rng.integers(-128, 128, (64, 16), dtype=np.int64).astype(np.int8)
    ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    out = torch.zeros(64 * 4, dtype=torch.int32, device="cuda")
    _lib.check(_lib.load_probe().dgm_probe_mfma_i8(_lib.ptr(ta), _lib.ptr(tb), _lib.ptr(out), _lib.stream()))
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(64, 4)
    res = {}
    for layout in ("contiguous", "split"):
        A = np.zeros((16, 64), np.int64)
        B = np.zeros((64, 16), np.int64)
        for l in range(64):
            A[l % 16, _i8_kmap(layout, l)] = a[l]
            B[_i8_kmap(layout, l), l % 16] = b[l]
        D = A @ B
        exp = np.array([[D[4 * (l // 16) + i, l % 16] for i in range(4)] for l in range(64)])
        res[layout] = bool((exp == got).all())
    print(res)
    assert res[I8_KMAP], res


I8_KMAP = "contiguous"


def test_transform_qoq_invariant():
    """QoQ: dequant(transform(q)) == interleave(dequant(q)) for L1 (interleaved) and L2, bit
    for bit ((code - z) * s2 * s1 is exact in fp32)."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_qoq_fused as qq
    from tests.gpu_common import decode_native_qoq
    rng = np.random.default_rng(31)
    w1 = randn_bf16(rng, (2, 64, 384), 0.05)
    w2 = randn_bf16(rng, (2, 32, 256), 0.05)
    q1 = qq.quantize_to_qoq(bf16_cpu(w1).cuda())
    q2 = qq.quantize_to_qoq(bf16_cpu(w2).cuda())
    (v1, m1, r1), (v2, m2, r2) = dgm.transform_qoq_weights_for_mega_moe_fused(q1, q2)
    torch.cuda.synchronize()
    d1 = pk.dequantize_qoq(*[t.cpu().numpy() for t in q1])
    d2 = pk.dequantize_qoq(*[t.cpu().numpy() for t in q2])
    np.testing.assert_array_equal(decode_native_qoq(v1.cpu().numpy(), m1.cpu().numpy(), r1.cpu().numpy()),
                                  interleave16(d1))
    np.testing.assert_array_equal(decode_native_qoq(v2.cpu().numpy(), m2.cpu().numpy(), r2.cpu().numpy(), l1=False),
                                  d2)


def test_mfma_f16_lane_layout():
    """V_MFMA_F32_16X16X32_F16 (the NVFP4 path): lane l supplies A row l%16 / B column l%16 with
    8 halves of K = 8 (l/16) .. +8; result register i of lane l is D[4 (l/16) + i][l%16]. Inputs
    are small integers, so the fp32 sums are exact."""
    need_gpu()
    from hopper_megamoe_basedondeepgemm_amd import _lib
    rng = np.random.default_rng(23)
    a = rng.integers(-8, 9, (64, 8)).astype(np.float16)
    b = rng.integers(-8, 9, (64, 8)).astype(np.float16)
    ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    out = torch.zeros(64 * 4, dtype=torch.float32, device="cuda")
    _lib.check(_lib.load_probe().dgm_probe_mfma_f16(_lib.ptr(ta), _lib.ptr(tb), _lib.ptr(out), _lib.stream()))
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(64, 4)
    A = np.zeros((16, 32))
    B = np.zeros((32, 16))
    for l in range(64):
        A[l % 16, 8 * (l // 16):8 * (l // 16) + 8] = a[l]
        B[8 * (l // 16):8 * (l // 16) + 8, l % 16] = b[l]
    D = A @ B
    exp = np.array([[D[4 * (l // 16) + i, l % 16] for i in range(4)] for l in range(64)])
    np.testing.assert_array_equal(got, exp)


def test_cvt_fp4_f16_and_fp8():
    """V_CVT_SCALEF32_PK_F16_FP4 on every byte with scales that are UE4M3 values (normal and
    subnormal, non-power-of-two mantissas): low nibble -> first half, high nibble -> second, and
    the scale's power-of-two part only is applied: value = E2M1(code) * 2^floor(log2(scale)),
    exactly (a non-power-of-two scale's mantissa is dropped, so the NVFP4 kernels convert with
    scale 1.0 and multiply by the E4M3 block scale afterwards). V_CVT_F32_FP8 = the E4M3 value
    of every byte except NaN."""
    need_gpu()
    from hopper_megamoe_basedondeepgemm_amd import _lib
    from oracle import numerics as nu
    codes = np.arange(256, dtype=np.uint32)
    sc_codes = np.array([0x38, 0x39, 0x3F, 0x01, 0x05, 0x07, 0x08, 0x0B, 0x7E, 0x55, 0x2A], np.uint8)
    scales = nu.e4m3_decode(sc_codes).astype(np.float32)
    src = np.repeat(codes * 0x01010101, len(scales)).astype(np.uint32)
    sc = np.tile(scales, len(codes)).astype(np.float32)
    n = src.size
    ts, tsc = torch.from_numpy(src.view(np.int32)).cuda(), torch.from_numpy(sc).cuda()
    oh = torch.zeros(4 * n, dtype=torch.int32, device="cuda")
    of = torch.zeros(4 * n, dtype=torch.float32, device="cuda")
    _lib.check(_lib.load_probe().dgm_probe_cvt_fp4(_lib.ptr(ts), _lib.ptr(tsc), _lib.ptr(oh), _lib.ptr(of), n,
                                             _lib.stream()))
    torch.cuda.synchronize()
    h = oh.cpu().numpy().view(np.uint32).reshape(n, 4)
    lo = (h & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
    hi = (h >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
    byte = (src & 0xFF)
    exp_lo = nu.e2m1_decode(byte & 0xF) * sc
    exp_hi = nu.e2m1_decode(byte >> 4) * sc
    ok_scaled = bool((lo[:, 0] == exp_lo).all() and (hi[:, 0] == exp_hi).all())
    pow2 = np.exp2(np.floor(np.log2(sc))).astype(np.float32)
    ok_exp = bool((lo[:, 0] == nu.e2m1_decode(byte & 0xF) * pow2).all() and
                  (hi[:, 0] == nu.e2m1_decode(byte >> 4) * pow2).all())
    print("full-float scale:", ok_scaled, "exponent only:", ok_exp)
    assert ok_exp and not ok_scaled
    one = sc == 1.0                              # (the kernels' use: scale 1.0, exact codes)
    np.testing.assert_array_equal(lo[one, 0], nu.e2m1_decode(byte[one] & 0xF))
    np.testing.assert_array_equal(hi[one, 0], nu.e2m1_decode(byte[one] >> 4))
    f = of.cpu().numpy().reshape(n, 4)[:, 0]
    ref = nu.e4m3_decode(byte.astype(np.uint8))
    keep = ~np.isnan(ref)
    np.testing.assert_array_equal(f[keep], ref[keep])


def test_global_load_lds_lane_layout():
    """GLOBAL_LOAD_LDS_DWORDX4 (the L2 phase's prefetch of weight tiles into LDS): lane l of a
    wave lands its 16 bytes at the wave's LDS base + 16 l, so a 1 KB tile keeps its order."""
    need_gpu()
    from hopper_megamoe_basedondeepgemm_amd import _lib
    src = torch.randint(0, 256, (4096,), dtype=torch.uint8, device="cuda")
    out = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    _lib.check(_lib.load_probe().dgm_probe_global_load_lds(_lib.ptr(src), _lib.ptr(out), _lib.stream()))
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), src.cpu())
