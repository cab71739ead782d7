"""CPU restatement of the reference's scalar number formats (test infrastructure only).

This module is the checker, never the product: only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s CPU-baseline leg may import it.

Every function restates one rule of the reference with numpy integer/float32 arithmetic.
Citations are ``path:line`` into the reference tree (DeepGEMM fork, MegaMoE branch).

Pinning (what checks each function against something other than itself):
  * ``f32_to_bf16`` / ``bf16_to_f32``: exhaustive over all 65536 bf16 patterns and
    random fp32 against ``torch.Tensor.to(torch.bfloat16)`` (library).
  * ``e4m3_encode`` / ``e4m3_decode``: exhaustive round trip over the 256 codes and
    2^20 random / tie inputs against ``torch.float8_e4m3fn`` casts (library).
  * ``e2m1_code_ties_down`` / ``e2m1_nibble_bucketize``: brute force over all 65536 bf16
    inputs against the textbook rule written as a nearest-value search with the tie rule,
    plus the reference's own known-answer table (nibble -> value, -0 handling).
  * ``ceil_to_ue8m0``: closed form (smallest power of two >= x) over all exponents and
    mantissas; ``ceil_log2_f32``: diff-tested against ``torch.log2`` in the CPU tests.
  * ``fp32_to_ue4m3_ceil``: brute force "smallest UE4M3 code whose value >= x" except
    the reference's documented -1e-6 fudge, which the golden vectors pin.
"""
import numpy as np

FP4_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)
FP4_SIGNED = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6],
                      dtype=np.float32)
FP4_BOUNDARIES = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=np.float32)


def as_f32(x):
    return np.asarray(x, dtype=np.float32)


# ----------------------------------------------------------------------------- bf16
def f32_to_bf16_bits(x):
    """fp32 -> bf16 bits, round to nearest even; NaN stays NaN (quiet bit set)."""
    u = as_f32(x).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x):
    """fp32 -> bf16 -> fp32 (the ``.to(torch.bfloat16).float()`` of the reference)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ----------------------------------------------------------------------------- E2M1
def e2m1_code_ties_down(x):
    """``_quantize_to_fp4_e2m1`` (deep_gemm/utils/math.py:73-82): code = #{b : |x| > b}
    over the midpoints (ties go to the smaller magnitude); sign bit only when code != 0
    (no -0 code). Returns uint8 nibbles 0..15."""
    ax = np.abs(as_f32(x))
    code = np.zeros(ax.shape, dtype=np.uint8)
    for b in FP4_BOUNDARIES:
        code += (ax > b).astype(np.uint8)
    sign = (as_f32(x) < 0) & (code != 0)
    return code | (sign.astype(np.uint8) << 3)


def e2m1_nibble_bucketize(x):
    """``fp32_to_fp4_nibble`` (deep_gemm/quantization_mxfp4.py:21-30,
    deep_gemm/quantization_nvfp4.py:17-28): magnitude clamped to 6, bucketize with
    right=False (= #{b : mag > b}, ties to the smaller magnitude); the sign bit is set
    for every x < 0, so a negative value that rounds to 0 gives the -0 nibble 0x8."""
    xf = as_f32(x)
    mag = np.minimum(np.abs(xf), np.float32(6.0))
    idx = np.zeros(mag.shape, dtype=np.uint8)
    for b in FP4_BOUNDARIES:
        idx += (mag > b).astype(np.uint8)
    return idx | ((xf < 0).astype(np.uint8) << 3)


def e2m1_decode(nib):
    return FP4_SIGNED[np.asarray(nib, dtype=np.uint8) & 0xF]


# ----------------------------------------------------------------------------- E8M0
def ceil_to_ue8m0(x):
    """``ceil_to_ue8m0`` (deep_gemm/utils/math.py:13-16): smallest power of two >= |x|
    by exponent bits (+1 when the mantissa is non-zero), exponent clamped to [1, 254].
    Returns the fp32 power of two."""
    bits = np.abs(as_f32(x)).view(np.uint32).astype(np.int64)
    exp = ((bits >> 23) & 0xFF) + ((bits & 0x7FFFFF) != 0).astype(np.int64)
    exp = np.clip(exp, 1, 254)
    return (exp.astype(np.uint32) << 23).view(np.float32)


def ue8m0_byte(pow2_f32):
    """Power-of-two fp32 scale -> its E8M0 byte (biased exponent)."""
    return ((as_f32(pow2_f32).view(np.uint32) >> 23) & 0xFF).astype(np.uint8)


def e8m0_to_f32(code):
    """E8M0 byte -> 2^(code-127) as fp32 (codes 0..254; 0 gives the subnormal 2^-127)."""
    c = np.asarray(code, dtype=np.int64)
    return np.ldexp(np.float64(1.0), c - 127).astype(np.float32)


def ceil_log2_f32(x):
    """``torch.ceil(torch.log2(x))`` for positive normal fp32 x, with log2 correctly
    rounded to fp32 (computed in float64, then rounded). This is how the reference's
    log2-based scale rules behave (deep_gemm/quantization_mxfp4.py:41-42,
    deep_gemm/quantization_mxfp4_fused.py:43, sm100_b200/test_mega_moe.py:428): a value a
    hair above a power of two can round down to the integer, so the 'ceil' keeps that
    power of two (and the quotient later saturates at the format maximum)."""
    xf = as_f32(x).astype(np.float64)
    l2 = np.log2(xf).astype(np.float32)
    return np.ceil(l2).astype(np.float32)


# ----------------------------------------------------------------------------- E4M3
def e4m3_encode(x):
    """fp32 -> float8_e4m3fn byte with round-to-nearest-even, as torch's cast
    (``.to(torch.float8_e4m3fn)``): |x| whose rounding exceeds 448 -> NaN (0x7F|sign)."""
    xf = as_f32(x)
    sign = (np.signbit(xf)).astype(np.uint8) << 7
    ax = np.abs(xf).astype(np.float64)
    out = np.zeros(xf.shape, dtype=np.uint8)
    nan = np.isnan(xf)
    sub = ax < 2.0 ** -6
    # subnormals (and zero): multiples of 2^-9, RNE
    q = np.rint(ax * 512.0)
    code_sub = q.astype(np.int64)               # q == 8 -> 0x08 = 2^-6, the smallest normal
    m, e = np.frexp(np.where(sub, 1.0, ax))     # ax = m * 2^e, m in [0.5, 1)
    e = e - 1                                   # ax = (2m) * 2^e, 2m in [1, 2)
    frac = (2.0 * m - 1.0) * 8.0
    qn = np.rint(frac).astype(np.int64)
    carry = qn == 8
    e = np.where(carry, e + 1, e)
    qn = np.where(carry, 0, qn)
    code_norm = (e + 7) * 8 + qn
    code = np.where(sub, code_sub, code_norm)
    code = np.where(code > 0x7E, 0x7F, code)
    code = np.where(nan | np.isinf(xf), 0x7F, code)
    out[...] = code.astype(np.uint8)
    return out | sign


def e4m3_decode(b):
    b = np.asarray(b, dtype=np.uint8)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.ldexp(1.0, e.astype(np.int64) - 7))
    val = np.where((b & 0x7F) == 0x7F, np.nan, val)
    return (s * val).astype(np.float32)


# ----------------------------------------------------------------------------- UE4M3 (NVFP4 scales)
UE4M3_MIN_DENORM = 2.0 ** -9
UE4M3_MAX_DENORM = 7.0 * UE4M3_MIN_DENORM
UE4M3_MIN_NORMAL = 2.0 ** -6
UE4M3_MAX_FINITE = 448.0


def fp32_to_ue4m3_ceil(x):
    """``fp32_to_ue4m3_ceil`` (deep_gemm/quantization_nvfp4.py:31-48), step for step in
    fp32: clamp to [2^-9, 448]; denormal code ceil(x / 2^-9) in [1, 7]; normal code from
    floor(log2 x), base 2^e, mantissa ceil((x/base - 1) * 8 - 1e-6) with carry."""
    xf = np.clip(as_f32(x), np.float32(UE4M3_MIN_DENORM), np.float32(UE4M3_MAX_FINITE))
    denorm = np.clip(np.ceil(xf / np.float32(UE4M3_MIN_DENORM)).astype(np.int64), 1, 7)
    xn = np.maximum(xf, np.float32(UE4M3_MIN_NORMAL))
    # floor(log2(xn)) of a correctly rounded fp32 log2: for normal xn this is the exponent
    # unless xn is a hair below a power of two and log2 rounds up to the integer.
    l2 = np.log2(xn.astype(np.float64)).astype(np.float32)
    e = np.floor(l2)
    exp_bits = (e + 7).astype(np.int64)
    base = np.exp2(e).astype(np.float32)
    t = (xn / base - np.float32(1.0)) * np.float32(8.0) - np.float32(1e-6)
    mant = np.ceil(t.astype(np.float32)).astype(np.int64)
    over = mant > 7
    exp_bits = np.where(over, exp_bits + 1, exp_bits)
    mant = np.clip(np.where(over, 0, mant), 0, 7)
    normal = np.clip(exp_bits * 8 + mant, 8, 0x7E)
    code = np.where(xf <= np.float32(UE4M3_MAX_DENORM), denorm, normal)
    return code.astype(np.uint8)


def ue4m3_to_f32(code):
    """``ue4m3_to_fp32`` (deep_gemm/quantization_nvfp4.py:51-59)."""
    c = np.asarray(code, dtype=np.int64) & 0x7F
    eb = c >> 3
    m = c & 7
    den = m.astype(np.float32) * np.float32(UE4M3_MIN_DENORM)
    nor = (np.float32(1.0) + m.astype(np.float32) * np.float32(0.125)) * \
        np.exp2((eb - 7).astype(np.float32))
    v = np.where(eb == 0, den, nor).astype(np.float32)
    return np.where(c == 0x7F, np.float32(UE4M3_MAX_FINITE), v).astype(np.float32)


# ----------------------------------------------------------------------------- rounding helpers
def round_half_even_f32(x):
    """``torch.round`` on fp32 (half to even)."""
    return np.rint(as_f32(x)).astype(np.float32)
