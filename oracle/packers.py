"""CPU restatement of the reference's offline packers and activation casts (test infrastructure).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
this module. Each function cites the reference rule it restates. All arithmetic is fp32
numpy, operation for operation, so the packed codes are bit-exact references.
"""
import numpy as np

from .numerics import (as_f32, ceil_to_ue8m0, ue8m0_byte, e2m1_code_ties_down,
                       e2m1_nibble_bucketize, e2m1_decode, e8m0_to_f32, ceil_log2_f32,
                       e4m3_encode, e4m3_decode, fp32_to_ue4m3_ceil, ue4m3_to_f32,
                       round_bf16, f32_to_bf16_bits, bf16_bits_to_f32)

FP4_MAX = np.float32(6.0)


# ----------------------------------------------------------------------------- nibble packing
def pack_marlin(nibbles):
    """Marlin order (deep_gemm/quantization_mxfp4.py:66-70): every 8 K nibbles -> 4 bytes,
    byte b = K[b] << 4 | K[b+4]."""
    *outer, K = nibbles.shape
    ch = nibbles.reshape(*outer, K // 8, 8).astype(np.uint8)
    return (ch[..., 4:8] | (ch[..., 0:4] << 4)).reshape(*outer, K // 2).astype(np.uint8)


def unpack_marlin(packed):
    """Inverse of ``pack_marlin`` (deep_gemm/quantization_mxfp4_fused.py:143-152)."""
    *outer, Kh = packed.shape
    p = packed.reshape(*outer, Kh // 4, 4)
    return np.concatenate([(p >> 4) & 0xF, p & 0xF], axis=-1).reshape(*outer, Kh * 2).astype(np.uint8)


def pack_low_first(nibbles):
    """OCP order (deep_gemm/utils/math.py:99-100; sm100_b200/test_mega_moe.py:91):
    byte j = K[2j] | K[2j+1] << 4."""
    n = nibbles.astype(np.uint8)
    return ((n[..., 0::2] & 0xF) | ((n[..., 1::2] & 0xF) << 4)).astype(np.uint8)


def unpack_low_first(packed):
    p = packed.astype(np.uint8)
    return np.stack([p & 0xF, p >> 4], axis=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)


# ----------------------------------------------------------------------------- MXFP4 weight packers
def quantize_to_mxfp4_fused(w):
    """``quantization_mxfp4_fused.quantize_to_mxfp4`` (deep_gemm/quantization_mxfp4_fused.py:29-52):
    exp = ceil(log2(max(amax,1e-38)/6)), -127 for an all-zero group, clamp [-127,127];
    nibbles by bucketize of (w/2^exp) clamped to +-6; Marlin byte order.
    Returns (packed uint8 [..., K/2], scale_e8m0 uint8 [..., K/32])."""
    w = as_f32(w)
    *outer, K = w.shape
    g = w.reshape(*outer, K // 32, 32)
    amax = np.abs(g).max(axis=-1)
    q = np.maximum(amax, np.float32(1e-38)) / FP4_MAX
    exp = ceil_log2_f32(q)
    exp = np.where(amax > 0, exp, np.float32(-127.0))
    exp = np.clip(exp, -127, 127)
    scale = np.ldexp(np.float64(1.0), exp.astype(np.int64)).astype(np.float32)
    x = np.clip(g / scale[..., None], -FP4_MAX, FP4_MAX)
    nib = e2m1_nibble_bucketize(x).reshape(*outer, K)
    return pack_marlin(nib), (exp.astype(np.int64) + 127).astype(np.uint8)


def quantize_to_mxfp4_split(w):
    """``quantization_mxfp4.quantize_to_mxfp4`` (deep_gemm/quantization_mxfp4.py:33-71):
    amax clamped to >= 1e-30, desired = amax/6 clamped to [2^-126, 2^127],
    code = clamp(ceil(log2) + 127, 1, 254), scale = 2^(max(code,1)-127); Marlin order."""
    w = as_f32(w)
    *outer, K = w.shape
    g = w.reshape(*outer, K // 32, 32)
    amax = np.maximum(np.abs(g).max(axis=-1), np.float32(1e-30))
    d = np.clip(amax / FP4_MAX, np.float32(2.0 ** -126), np.float32(2.0 ** 127))
    code = np.clip(ceil_log2_f32(d).astype(np.int64) + 127, 1, 254).astype(np.uint8)
    scale = e8m0_to_f32(np.maximum(code, 1))
    x = np.clip(g / scale[..., None], -FP4_MAX, FP4_MAX)
    nib = e2m1_nibble_bucketize(x).reshape(*outer, K)
    return pack_marlin(nib), code


def dequantize_mxfp4_marlin(packed, scale_e8m0):
    """``dequantize_mxfp4_to_fp32`` (deep_gemm/quantization_mxfp4_fused.py:155-161):
    exact E2M1 x 2^(code-127)."""
    vals = e2m1_decode(unpack_marlin(packed))
    *outer, K = vals.shape
    s = e8m0_to_f32(scale_e8m0)
    return (vals.reshape(*outer, K // 32, 32) * s[..., None]).reshape(*outer, K).astype(np.float32)


# ----------------------------------------------------------------------------- per-row MXFP4 / MXFP8 casts
def cast_to_fp4_rows(x, vec=32):
    """W4A4 row cast (sm100_b200/test_mega_moe.py:68-93 with act_format 'mxfp4'):
    amax per vec clamped >= 1e-30, sf = ceil_to_ue8m0(amax/6), codes = ties-down E2M1 of
    x/sf (no -0), low-nibble-first packing, sf byte = exponent bits.
    Returns (packed uint8 [M, K/2], sf_f32 [M, K/vec], sf_byte uint8 [M, K/vec])."""
    x = as_f32(x)
    *outer, K = x.shape
    g = x.reshape(*outer, K // vec, vec)
    amax = np.maximum(np.abs(g).max(axis=-1), np.float32(1e-30))
    sf = ceil_to_ue8m0(amax / FP4_MAX)
    codes = e2m1_code_ties_down(g / sf[..., None]).reshape(*outer, K)
    return pack_low_first(codes), sf, ue8m0_byte(sf)


def per_token_cast_to_fp4(x, gran_k=32):
    """``per_token_cast_to_fp4(use_ue8m0=True)`` (deep_gemm/utils/math.py:85-111): like
    ``cast_to_fp4_rows`` but amax clamped to >= 1e-4 and x * (1/sf)."""
    x = as_f32(x)
    *outer, K = x.shape
    g = x.reshape(*outer, K // gran_k, gran_k)
    amax = np.maximum(np.abs(g).max(axis=-1), np.float32(1e-4))
    sf = ceil_to_ue8m0(amax / FP4_MAX)
    codes = e2m1_code_ties_down(g * (np.float32(1.0) / sf)[..., None]).reshape(*outer, K)
    return pack_low_first(codes), sf


def dequant_fp4_rows(packed, sf_f32, vec=32):
    vals = e2m1_decode(unpack_low_first(packed))
    *outer, K = vals.shape
    return (vals.reshape(*outer, K // vec, vec) * as_f32(sf_f32)[..., None]).reshape(*outer, K)


def per_token_cast_to_fp8_ue8m0(x, gran_k=32):
    """``per_token_cast_to_fp8(use_ue8m0=True, gran_k=32)`` (deep_gemm/utils/math.py:26-38):
    amax clamped >= 1e-4, sf = ceil_to_ue8m0(amax/448), e4m3(x * (1/sf)).
    Returns (e4m3 bytes [M, K], sf_f32 [M, K/gran_k])."""
    x = as_f32(x)
    *outer, K = x.shape
    g = x.reshape(*outer, K // gran_k, gran_k)
    amax = np.maximum(np.abs(g).max(axis=-1), np.float32(1e-4))
    sf = ceil_to_ue8m0(amax / np.float32(448.0))
    q = e4m3_encode(g * (np.float32(1.0) / sf)[..., None]).reshape(*outer, K)
    return q, sf


def per_token_cast_to_fp8_f32sf(x, gran_k=128):
    """``per_token_cast_to_fp8(use_ue8m0=False)`` (deep_gemm/utils/math.py:26-38): plain fp32
    sf = amax/448 (amax >= 1e-4)."""
    x = as_f32(x)
    *outer, K = x.shape
    g = x.reshape(*outer, K // gran_k, gran_k)
    amax = np.maximum(np.abs(g).max(axis=-1), np.float32(1e-4))
    sf = amax / np.float32(448.0)
    q = e4m3_encode(g * (np.float32(1.0) / sf)[..., None]).reshape(*outer, K)
    return q, sf


def dequant_fp8_rows(q, sf_f32, gran_k=32):
    v = e4m3_decode(q)
    *outer, K = v.shape
    return (v.reshape(*outer, K // gran_k, gran_k) * as_f32(sf_f32)[..., None]).reshape(*outer, K)


# ----------------------------------------------------------------------------- NVFP4
def quantize_to_nvfp4(w):
    """``quantize_to_nvfp4`` (deep_gemm/quantization_nvfp4.py:62-82): per-16 UE4M3 ceil
    scale of amax/6 (amax >= 1e-30), nibbles by bucketize of w/scale clamped to +-6,
    Marlin order. Returns (packed uint8 [..., K/2], scale_ue4m3 uint8 [..., K/16])."""
    w = as_f32(w)
    *outer, K = w.shape
    g = w.reshape(*outer, K // 16, 16)
    amax = np.maximum(np.abs(g).max(axis=-1), np.float32(1e-30))
    code = fp32_to_ue4m3_ceil(amax / FP4_MAX)
    scale = ue4m3_to_f32(code)
    x = np.clip(g / scale[..., None], -FP4_MAX, FP4_MAX)
    nib = e2m1_nibble_bucketize(x).reshape(*outer, K)
    return pack_marlin(nib), code


def dequantize_nvfp4(packed, scale_ue4m3):
    """``dequantize_nvfp4_to_fp32`` (deep_gemm/quantization_nvfp4.py:155-189), row-major."""
    vals = e2m1_decode(unpack_marlin(packed))
    *outer, K = vals.shape
    s = ue4m3_to_f32(scale_ue4m3)
    return (vals.reshape(*outer, K // 16, 16) * s[..., None]).reshape(*outer, K).astype(np.float32)


def cast_to_nvfp4_rows(x):
    """W4A4 NVFP4 row cast (sm100_b200/test_mega_moe.py:68-93 with act_format 'nvfp4'):
    amax per 16 (>= 1e-30), sf = e4m3(amax/6) (RNE cast, not ceil), ties-down E2M1 of x/sf,
    low-nibble-first packing. Returns (packed, sf_f32, sf_byte)."""
    x = as_f32(x)
    *outer, K = x.shape
    g = x.reshape(*outer, K // 16, 16)
    amax = np.maximum(np.abs(g).max(axis=-1), np.float32(1e-30))
    sfb = e4m3_encode(amax / FP4_MAX)
    sf = e4m3_decode(sfb)
    with np.errstate(divide="ignore", invalid="ignore"):     # sf 0: x / 0 -> code 7 or 0
        codes = e2m1_code_ties_down(g / sf[..., None]).reshape(*outer, K)
    return pack_low_first(codes), sf, sfb


# ----------------------------------------------------------------------------- QoQ W4A8
def quantize_to_qoq(w):
    """``quantize_to_qoq`` (deep_gemm/quantization_qoq_fused.py:18-38):
    s1 = bf16(max(amax_row/120, 1e-30)); w8 = clamp(rne(w/s1), +-112);
    per K128: s2 = clamp(ceil((mx-mn)/15), 1, 15), z = clamp(rne(-mn/s2), 0, 15),
    code = clamp(rne(w8/s2 + z), 0, 15); Marlin order.
    Returns (packed [E,N,K/2], s2 u8 [E,N,K/128], z u8 [E,N,K/128], s1 f32 [E,N])."""
    w = as_f32(w)
    E, N, K = w.shape
    s1 = np.maximum(np.abs(w).max(axis=-1, keepdims=True) / np.float32(120.0), np.float32(1e-30))
    s1 = round_bf16(s1)
    w8 = np.clip(np.rint(w / s1), -112, 112).astype(np.float32)
    g = w8.reshape(E, N, K // 128, 128)
    mn = g.min(axis=-1, keepdims=True)
    mx = g.max(axis=-1, keepdims=True)
    s2 = np.clip(np.ceil((mx - mn) / np.float32(15.0)), 1, 15).astype(np.float32)
    z = np.clip(np.rint(-mn / s2), 0, 15).astype(np.float32)
    code = np.clip(np.rint((g / s2 + z).astype(np.float32)), 0, 15).reshape(E, N, K)
    return (pack_marlin(code.astype(np.uint8)), s2[..., 0].astype(np.uint8),
            z[..., 0].astype(np.uint8), s1[..., 0].astype(np.float32))


def dequantize_qoq(packed, s2, z, s1):
    """``dequantize_qoq_to_fp32`` (deep_gemm/quantization_qoq_fused.py:68-75)."""
    codes = unpack_marlin(packed).astype(np.float32)
    E, N, K = codes.shape
    c = codes.reshape(E, N, K // 128, 128)
    wv = (c - z.astype(np.float32)[..., None]) * s2.astype(np.float32)[..., None]
    return (wv.reshape(E, N, K) * as_f32(s1)[..., None]).astype(np.float32)


def quantize_to_qoq_int4(w):
    """``quantize_to_qoq_int4`` (deep_gemm/quantization_mxfp4.py:323-353), the split path's QoQ
    packer: the same s1 / w8 / z / code chain as quantize_to_qoq except s2 = clamp(ceil((mx-mn)/15),
    1, 127); Marlin-packed codes and an int32 plane per (row, K128 group) with bytes
    [s2, z, s1 as bf16 (high half)]. Returns (packed [E,N,K/2], plane int32 [E,N,K/128])."""
    w = as_f32(w)
    E, N, K = w.shape
    s1 = round_bf16(np.maximum(np.abs(w).max(axis=-1, keepdims=True) / np.float32(120.0), np.float32(1e-30)))
    w8 = np.clip(np.rint(w / s1), -112, 112).astype(np.float32)
    g = w8.reshape(E, N, K // 128, 128)
    mn = g.min(axis=-1, keepdims=True)
    mx = g.max(axis=-1, keepdims=True)
    s2 = np.clip(np.ceil((mx - mn) / np.float32(15.0)), 1, 127).astype(np.float32)
    z = np.clip(np.rint(-mn / s2), 0, 15).astype(np.float32)
    code = np.clip(np.rint((g / s2 + z).astype(np.float32)), 0, 15).reshape(E, N, K)
    s1w = (s1.astype(np.float32).view(np.uint32) & np.uint32(0xFFFF0000)).astype(np.uint32)
    plane = (np.broadcast_to(s1w, (E, N, K // 128)) | (z[..., 0].astype(np.uint32) << 8)
             | s2[..., 0].astype(np.uint32)).view(np.int32)
    return pack_marlin(code.astype(np.uint8)), np.ascontiguousarray(plane)


def dequantize_qoq_int4(packed, plane):
    """``dequantize_qoq_int4`` (deep_gemm/quantization_mxfp4.py:365-383):
    (code - z) * s2 * s1 with s2 = byte 0, z = byte 1, s1 = the plane's high half as fp32."""
    codes = unpack_marlin(packed).astype(np.float32)
    E, N, K = codes.shape
    u = np.ascontiguousarray(plane).view(np.uint32)
    s2 = (u & 0xFF).astype(np.float32)
    z = ((u >> 8) & 0xFF).astype(np.float32)
    s1 = (u & np.uint32(0xFFFF0000)).view(np.float32)
    c = codes.reshape(E, N, K // 128, 128)
    return ((c - z[..., None]) * s2[..., None] * s1[..., None]).reshape(E, N, K).astype(np.float32)


def qoq_int4_to_fused(packed, plane):
    """The int4 packer's output in quantize_to_qoq's form (packed, s2, z, s1): the same codes;
    s2, z and the row's s1 read back from the plane (s1 is the same in every group of a row)."""
    u = np.ascontiguousarray(plane).view(np.uint32)
    s2 = (u & 0xFF).astype(np.uint8)
    z = ((u >> 8) & 0xFF).astype(np.uint8)
    s1 = (u[..., 0] & np.uint32(0xFFFF0000)).view(np.float32)
    return packed, s2, z, s1


def qoq_int_codes(packed, s2, z):
    """Integer weight (code - z) * s2 per element (exact, |.| <= 225)."""
    codes = unpack_marlin(packed).astype(np.int64)
    E, N, K = codes.shape
    c = codes.reshape(E, N, K // 128, 128)
    return ((c - z.astype(np.int64)[..., None]) * s2.astype(np.int64)[..., None]).reshape(E, N, K)


def per_token_cast_to_int8(x):
    """``per_token_cast_to_int8`` (deep_gemm/quantization_qoq_fused.py:78-91):
    sf = max(amax_row, 1e-30)/127, q = clamp(rne(x/sf), +-127). Returns (int8 [M,K], sf [M])."""
    x = as_f32(x)
    amax = np.maximum(np.abs(x).max(axis=-1, keepdims=True), np.float32(1e-30))
    sf = amax / np.float32(127.0)
    q = np.clip(np.rint(x / sf), -127, 127).astype(np.int8)
    return q, sf[..., 0].astype(np.float32)


# ----------------------------------------------------------------------------- checkpoint formats
# The fused kernel's FP4 tile layouts (the layouts dgm_packers.hip's transform writes), restated
# with numpy reshapes, and the nibble-order conversions between OCP checkpoints (low nibble =
# even K, deep_gemm/utils/math.py:99-100) and the reference's Marlin order
# (deep_gemm/quantization_mxfp4.py:66-70).
def marlin_to_low_first(packed):
    """Marlin bytes -> OCP low-nibble-first bytes of the same codes."""
    return pack_low_first(unpack_marlin(np.asarray(packed)))


def low_first_to_marlin(packed):
    return pack_marlin(unpack_low_first(np.asarray(packed)))


def native_src_rows(N, l1_mode):
    """Source row of each native row (block q = i // 16, row r = i % 16). l1_mode 0: identity;
    1: W1 as [gate rows; up rows] -> block 2p = gate rows 16p.., block 2p+1 = up rows N/2 + 16p..;
    2: W1 with gate / up interleaved by row (row 2i = gate i, row 2i+1 = up i) -> the same blocks."""
    i = np.arange(N)
    q, r = i // 16, i % 16
    if l1_mode == 1:
        return np.where(q % 2 == 1, N // 2 + 16 * (q // 2) + r, 16 * (q // 2) + r)
    if l1_mode == 2:
        return 2 * (16 * (q // 2) + r) + q % 2
    return i


def _to_low_first(packed, order):
    return np.asarray(packed) if order in ("low_first", "ocp") else marlin_to_low_first(packed)


def _from_low_first(packed, order):
    return packed if order in ("low_first", "ocp") else low_first_to_marlin(packed)


def fp4_to_tile(packed, scale, order="marlin", l1_mode=0):
    """MXFP4 [E, N, K/2] codes + E8M0 [E, N, K/32] -> values [E, N/16, K/128, 64, 16] (lane l =
    row l % 16 of the block, its 32 codes K = 128 kt + 32 (l // 16) .. +32, low nibble first) and
    scales [E, N/16, ceil(K/512), 64, 4] (byte j = the scale of K-tile 4 g + j of the lane's
    (row, 32-group); 127 = 2^0 past the last K-tile)."""
    lf = _to_low_first(packed, order)
    scale = np.asarray(scale)
    E, N, Kh = lf.shape
    K = 2 * Kh
    KT, NB = K // 128, N // 16
    KG = (KT + 3) // 4
    rows = native_src_rows(N, l1_mode)
    lf, sc = lf[:, rows], scale[:, rows]
    vals = lf.reshape(E, NB, 16, KT, 4, 16).transpose(0, 1, 3, 4, 2, 5).reshape(E, NB, KT, 64, 16)
    s = sc.reshape(E, NB, 16, KT, 4).transpose(0, 1, 3, 4, 2).reshape(E, NB, KT, 64)
    out = np.full((E, NB, KG * 4, 64), 127, np.uint8)
    out[:, :, :KT] = s
    out = out.reshape(E, NB, KG, 4, 64).transpose(0, 1, 2, 4, 3)
    return np.ascontiguousarray(vals), np.ascontiguousarray(out)


def fp4_from_tile(values, scales, order="marlin", l1_mode=0):
    """Inverse of ``fp4_to_tile`` (the padding scale bytes are dropped)."""
    values, scales = np.asarray(values), np.asarray(scales)
    E, NB, KT = values.shape[:3]
    N, K = NB * 16, KT * 128
    lf = values.reshape(E, NB, KT, 4, 16, 16).transpose(0, 1, 4, 2, 3, 5).reshape(E, N, K // 2)
    s = scales.transpose(0, 1, 2, 4, 3).reshape(E, NB, -1, 64)[:, :, :KT]
    s = s.reshape(E, NB, KT, 4, 16).transpose(0, 1, 4, 2, 3).reshape(E, N, K // 32)
    rows = native_src_rows(N, l1_mode)
    packed, sc = np.empty_like(lf), np.empty_like(s)
    packed[:, rows], sc[:, rows] = lf, s
    return _from_low_first(packed, order), sc


def nvfp4_to_tile(packed, scale, order="marlin", l1_mode=0):
    """NVFP4 [E, N, K/2] codes + E4M3 [E, N, K/16] -> values [E, N/16, K/128, 64, 16] (lane l =
    row l % 16; dword j = the eight codes K = 128 kt + 32 j + 8 (l // 16) .. +8, low nibble first)
    and scales [E, N/16, K/128, 2, 16, 4] (dword (p, r) byte j = the scale of 16-block 8 kt + 2 j + p
    of row r)."""
    lf = _to_low_first(packed, order)
    scale = np.asarray(scale)
    E, N, Kh = lf.shape
    K = 2 * Kh
    KT, NB = K // 128, N // 16
    rows = native_src_rows(N, l1_mode)
    lf, sc = lf[:, rows], scale[:, rows]
    vals = lf.reshape(E, NB, 16, KT, 4, 4, 4).transpose(0, 1, 3, 5, 2, 4, 6).reshape(E, NB, KT, 64, 16)
    s = sc.reshape(E, NB, 16, KT, 4, 2).transpose(0, 1, 3, 5, 2, 4)
    return np.ascontiguousarray(vals), np.ascontiguousarray(s)


def nvfp4_from_tile(values, scales, order="marlin", l1_mode=0):
    """Inverse of ``nvfp4_to_tile``."""
    values, scales = np.asarray(values), np.asarray(scales)
    E, NB, KT = values.shape[:3]
    N, K = NB * 16, KT * 128
    lf = values.reshape(E, NB, KT, 4, 16, 4, 4).transpose(0, 1, 4, 2, 5, 3, 6).reshape(E, N, K // 2)
    s = scales.transpose(0, 1, 4, 2, 5, 3).reshape(E, N, K // 16)
    rows = native_src_rows(N, l1_mode)
    packed, sc = np.empty_like(lf), np.empty_like(s)
    packed[:, rows], sc[:, rows] = lf, s
    return _from_low_first(packed, order), sc
