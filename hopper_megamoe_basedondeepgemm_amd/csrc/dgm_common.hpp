// Device-side number formats and CDNA4 matrix-core wrappers shared by every kernel.
// Target: gfx950 (MI355X) only. All helpers are exact integer/bit manipulations or
// IEEE fp32 operations, so every rounding rule here has a bit-exact CPU counterpart.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <utility>

#define DGM_DEV __device__ __forceinline__

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

namespace dgm {

// Compile-time unrolled loop: f(std::integral_constant<int, i>) for i = 0 .. N-1.
template <class F, int... Is>
DGM_DEV void static_for_impl(F& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
DGM_DEV void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// ---------------------------------------------------------------- bf16
DGM_DEV float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet.
DGM_DEV uint16_t f32_to_bf16(float f) {
  // (a select, not a branch: a branch costs an exec-mask round per call)
  const uint32_t u = __float_as_uint(f);
  const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? (u >> 16) | 0x40u : r);
}
DGM_DEV float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// ---------------------------------------------------------------- E2M1
// Midpoint count rule: code = #{b in {.25,.75,1.25,1.75,2.5,3.5,5} : mag > b}; ties go to
// the smaller magnitude.
DGM_DEV uint32_t e2m1_mag_code(float a) {
  return (uint32_t)(a > 0.25f) + (uint32_t)(a > 0.75f) + (uint32_t)(a > 1.25f) +
         (uint32_t)(a > 1.75f) + (uint32_t)(a > 2.5f) + (uint32_t)(a > 3.5f) + (uint32_t)(a > 5.0f);
}
// Activation rule: sign bit only when the magnitude code is non-zero (no -0 code).
DGM_DEV uint32_t e2m1_ties_down(float x) {
  uint32_t c = e2m1_mag_code(fabsf(x));
  return c | ((x < 0.f && c != 0u) ? 8u : 0u);
}
// Packer rule: magnitude clamped to 6, sign bit for every negative input (-0 code possible).
DGM_DEV uint32_t e2m1_bucketize(float x) {
  uint32_t c = e2m1_mag_code(fminf(fabsf(x), 6.0f));
  return c | (x < 0.f ? 8u : 0u);
}
DGM_DEV float e2m1_value(uint32_t nib) {
  const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
  float v = mag[nib & 7u];
  return (nib & 8u) ? -v : v;
}

// ---------------------------------------------------------------- E8M0
// Smallest power of two >= |x| by exponent bits, exponent clamped to [1, 254].
DGM_DEV uint32_t ceil_ue8m0_code(float x) {
  uint32_t b = __float_as_uint(x) & 0x7fffffffu;
  uint32_t e = ((b >> 23) & 0xffu) + ((b & 0x7fffffu) != 0u ? 1u : 0u);
  return e < 1u ? 1u : (e > 254u ? 254u : e);
}
DGM_DEV float e8m0_value(uint32_t code) { return __uint_as_float(code << 23); }   // code >= 1
// 2^(code-127) including code 0 (2^-127, subnormal).
DGM_DEV float e8m0_value_any(uint32_t code) {
  return code == 0u ? __uint_as_float(0x00400000u) : __uint_as_float(code << 23);
}
// 2^(127 - code): the exact reciprocal of the E8M0 value (code 254 gives the subnormal 2^-127),
// so x * e8m0_inv(code) == x / e8m0_value_any(code) bit for bit.
DGM_DEV float e8m0_inv(uint32_t code) {
  return code >= 254u ? __uint_as_float(0x00400000u) : __uint_as_float((254u - code) << 23);
}
// ceil(fp32(log2(x))) with log2 evaluated in double and rounded once to fp32: the
// behaviour of the log2-based scale rules near powers of two.
DGM_DEV float ceil_log2_f32(float x) { return ceilf((float)log2((double)x)); }

// ---------------------------------------------------------------- E4M3 (OCP fn)
// fp32 -> e4m3fn byte, round to nearest even; anything rounding above 448 -> 0x7F (NaN).
DGM_DEV uint32_t e4m3_encode(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return sign | 0x7fu;
  float ax = __uint_as_float(a);
  uint32_t code;
  if (ax < 0.015625f) {                     // < 2^-6: multiples of 2^-9
    code = (uint32_t)rintf(ax * 512.0f);
  } else {
    int e = (int)(a >> 23) - 127;
    uint32_t mant = a & 0x7fffffu;
    uint32_t m3 = mant >> 20, rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (m3 & 1u))) m3++;
    if (m3 == 8u) { m3 = 0u; e++; }
    int c = ((e + 7) << 3) | (int)m3;
    code = c > 0x7e ? 0x7fu : (uint32_t)c;
  }
  return sign | code;
}

// ---------------------------------------------------------------- SwiGLU
// sigmoid(g) = 1 / (1 + e^-g). fast: e^-g = 2^(-g log2 e) on the hardware exp2 and the
// hardware reciprocal (the reference's fast_math=True path is an approximate exp and an
// approximate reciprocal too); otherwise IEEE expf and a correctly rounded division.
template <bool FAST>
DGM_DEV float sigmoid(float g) {
  if (FAST) return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
  return 1.0f / (1.0f + expf(-g));
}

// ---------------------------------------------------------------- top-k selection
// Key order of the router top-k: orderable(bf16(logit)) << 16 | (0xFFFF - e), -0 -> +0, so
// larger keys are larger values and, on ties, lower expert ids.
DGM_DEV uint32_t topk_key(float logit, int e) {
  uint32_t b = f32_to_bf16(logit);
  b = b == 0x8000u ? 0u : b;
  const uint32_t o = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
  return (o << 16) | (0xffffu - (uint32_t)e);
}
DGM_DEV float key_value(uint32_t key) {
  uint32_t o = key >> 16;
  uint32_t b = (o & 0x8000u) ? (o & 0x7fffu) : (~o & 0xffffu);
  return bf16_to_f32((uint16_t)b);
}

// Wave-wide max, uniform result: DPP within rows of 16 lanes (quad xor 1, quad xor 2, half
// mirror, mirror), then the 4 row results via readlane.
DGM_DEV uint32_t wave_max_u32(uint32_t v) {
  auto mx = [](uint32_t a, int b) { return a > (uint32_t)b ? a : (uint32_t)b; };
  v = mx(v, __builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false));    // quad_perm [1,0,3,2]
  v = mx(v, __builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false));    // quad_perm [2,3,0,1]
  v = mx(v, __builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false));   // row_half_mirror
  v = mx(v, __builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false));   // row_mirror
  const uint32_t a = __builtin_amdgcn_readlane((int)v, 15), b = __builtin_amdgcn_readlane((int)v, 31);
  const uint32_t c = __builtin_amdgcn_readlane((int)v, 47), d = __builtin_amdgcn_readlane((int)v, 63);
  const uint32_t ab = a > b ? a : b, cd = c > d ? c : d;
  return ab > cd ? ab : cd;
}

// Top-k of one token's key row (E <= 1024, topk <= 16) by one wave; load(e) returns the
// token's key of expert e (topk_key of its logit). Lane l holds the keys of experts l + 64 i
// (i < NK), sorted descending; each of the k rounds takes the wave-wide maximum of the lanes'
// first keys (keys are distinct: they carry the expert id) and the winning lane shifts its list
// by one. Lane k keeps slot k. Weights: w_k = exp(v_k - v_0) / sum_k, the sum taken
// sequentially in slot order.
template <int NK, class LoadKey>
DGM_DEV void select_topk_wave_nk(LoadKey load, int E, int topk, int lane, int& idx, float& wt) {
  // every key is read before any is used (one memory round trip, not one per key)
  uint32_t key[NK];
#pragma unroll
  for (int i = 0; i < NK; ++i) key[i] = load(lane + 64 * i < E ? lane + 64 * i : E - 1);
#pragma unroll
  for (int i = 0; i < NK; ++i) key[i] = lane + 64 * i < E ? key[i] : 0u;
  // odd-even transposition sort, descending
#pragma unroll
  for (int r = 0; r < NK; ++r)
#pragma unroll
    for (int i = r & 1; i + 1 < NK; i += 2) {
      const uint32_t a = key[i], b = key[i + 1];
      key[i] = a > b ? a : b;
      key[i + 1] = a > b ? b : a;
    }
  float myv = 0.f, v0 = 0.f;
  int mye = -1;
  for (int k = 0; k < topk; ++k) {
    const uint32_t m = wave_max_u32(key[0]);
    if (key[0] == m) {         // the lane holding the winner
#pragma unroll
      for (int i = 0; i + 1 < NK; ++i) key[i] = key[i + 1];
      key[NK - 1] = 0u;
    }
    const float v = key_value(m);
    if (k == 0) v0 = v;
    if (lane == k) {
      myv = v;
      mye = (int)(0xffffu - (m & 0xffffu));
    }
  }
  const float ex = lane < topk ? expf(myv - v0) : 0.f;
  float sum = 0.f;
  for (int k = 0; k < topk; ++k) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), k));
  if (lane < topk) {
    idx = mye;
    wt = ex / sum;
  }
}

// The key row of an unrouted token (an all-zero hidden row under DGM_FE_ZERO_ROW_UNROUTED) starts
// with a zero key: every slot -1 / 0 (a real key is never zero: its low half is 0xFFFF - e).
// balanced: slot s -> s G + (g + 7 s) % G with G = E / topk, weight 1 / topk (g = the token's
// global index).
template <class LoadKey>
DGM_DEV void select_topk_wave(LoadKey load, int E, int topk, bool balanced, int g, int lane, int& idx, float& wt) {
  idx = -1;
  wt = 0.f;
  if (load(0) == 0u) return;
  if (balanced) {
    const int G = E / topk;
    if (lane < topk) {
      idx = lane * G + (g + 7 * lane) % G;
      wt = 1.0f / (float)topk;
    }
    return;
  }
  const int nk = (E + 63) >> 6;         // keys per lane (wave-uniform)
  if (nk <= 1) select_topk_wave_nk<1>(load, E, topk, lane, idx, wt);
  else if (nk <= 2) select_topk_wave_nk<2>(load, E, topk, lane, idx, wt);
  else if (nk <= 4) select_topk_wave_nk<4>(load, E, topk, lane, idx, wt);
  else if (nk <= 6) select_topk_wave_nk<6>(load, E, topk, lane, idx, wt);
  else if (nk <= 8) select_topk_wave_nk<8>(load, E, topk, lane, idx, wt);
  else select_topk_wave_nk<16>(load, E, topk, lane, idx, wt);
}

// ---------------------------------------------------------------- scopes / atomics
DGM_DEV int atomic_add_acqrel_agent(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
DGM_DEV int atomic_load_acquire_agent(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- matrix cores
// D(16x16 f32) += A(16x128) * B(128x16) with per-32 E8M0 block scales.
// fmt: 0 = E4M3, 4 = E2M1. Lane l supplies A row l%16 / B column l%16. E2M1 operands
// (4 dwords): K = 32*(l/16) .. +32, low nibble first. E4M3 operands (8 dwords): bytes 0-15
// hold K = 16*(l/16) .. +16 and bytes 16-31 hold K = 64 + 16*(l/16) .. +16. In both cases
// the scale byte of lane l applies to row/column l%16 over the 32-block K = 32*(l/16) .. +32.
// Result register i of lane l is D[4*(l/16) + i][l%16]. (Pinned by the probe test.)
template <int FMT_A, int FMT_B>
DGM_DEV v4f mfma_scale_16x16x128(v8i a, v8i b, v4f c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FMT_A, FMT_B, 0, sa, 0, sb);
}
// Same, with the scale bytes selected from 4-byte scale words: byte OPA of sa, byte OPB of sb.
template <int FMT_A, int FMT_B, int OPA, int OPB>
DGM_DEV v4f mfma_scale_16x16x128_sel(v8i a, v8i b, v4f c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FMT_A, FMT_B, OPA, sa, OPB, sb);
}

// Keeps the scale registers of a chain of block-scaled matrix-core ops allocated until the chain's
// last op has issued (the result `acc` is an input here), so that no instruction inside the chain
// writes a register a later op of the chain reads as its scale. With the scale operands taken
// from loaded dwords (never computed by VALU ops between the ops), the chain's scales are written
// only by memory loads.
template <int N>
DGM_DEV void keep_scales_until(const uint32_t (&r)[N], v4f acc) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" ::"v"(acc[0]), "v"(r[i]));
}

// D(16x16 i32) += A(16x64 int8) * B(64x16 int8), exact. Lane l supplies A row l%16 / B column
// l%16 with 16 K values (lane group l/16 of both operands pairs byte for byte); result
// register i of lane l is D[4*(l/16) + i][l%16]. (Pinned by the probe test.)
DGM_DEV v4i mfma_i8_16x16x64(v4i a, v4i b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0); }

// QoQ codes: dword d holds K j = b (low nibble of byte b) and 4 + b (high nibble); as int8
// bytes: (d & 0x0F0F0F0F, (d >> 4) & 0x0F0F0F0F).
DGM_DEV v4i qoq_codes(uint32_t d0, uint32_t d1) {
  v4i r = {(int)(d0 & 0x0F0F0F0Fu), (int)((d0 >> 4) & 0x0F0F0F0Fu), (int)(d1 & 0x0F0F0F0Fu),
           (int)((d1 >> 4) & 0x0F0F0F0Fu)};
  return r;
}

// sum of the 16 int8 values of a 16-byte fragment (exact)
DGM_DEV int i8_sum16(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  int s = __builtin_amdgcn_sdot4((int)a, 0x01010101, 0, false);
  s = __builtin_amdgcn_sdot4((int)b, 0x01010101, s, false);
  s = __builtin_amdgcn_sdot4((int)c, 0x01010101, s, false);
  return __builtin_amdgcn_sdot4((int)d, 0x01010101, s, false);
}

}  // namespace dgm
