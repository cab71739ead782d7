// Router GEMV and activation casts of the frontend, shared by the frontend kernel
// (dgm_megamoe.hip) and the fused kernel's in-kernel frontend (dgm_fused.hip). AGENT selects
// write-through agent-scope stores, for data that other workgroups of the same launch read.
#pragma once
#include "dgm_common.hpp"
#include "../../include/dgm_megamoe.h"

namespace dgm {

template <bool AGENT>
DGM_DEV void put8(uint8_t* p, uint32_t v) {
  if (AGENT) __hip_atomic_store(p, (uint8_t)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = (uint8_t)v;
}
template <bool AGENT>
DGM_DEV void put16(uint16_t* p, uint32_t v) {
  if (AGENT) __hip_atomic_store(p, (uint16_t)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = (uint16_t)v;
}
template <bool AGENT>
DGM_DEV void put32(uint32_t* p, uint32_t v) {
  if (AGENT) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}
template <bool AGENT>
DGM_DEV void put64(uint64_t* p, uint64_t v) {
  if (AGENT) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}

// Router: one wave computes the logits of expert e for tokens t0 .. t0 + 3 (rows past M are
// clamped and not written). Lane l accumulates K = 512 j + 8 l + i (j, then i ascending) with
// fp32 FMAs of exact bf16 products, then an xor butterfly (32..1) reduces the 64 lane sums: a
// fixed order, so the fp32 logits are reproducible bit for bit. Writes the fp32 logit and the
// top-k key (topk_key: orderable bf16 << 16 | 0xFFFF - e); with zero_unrouted, the keys of an
// all-zero hidden row are 0 (the token is unrouted).
// The logits of expert e (its router row wv, lane l holding K = 512 j + 8 l .. +7) for the four
// token rows xv (laid out the same way), in the order stated above; rows t0 + tt >= M are not
// written.
template <int J, bool AGENT>
DGM_DEV void router_dot4(const uint4 (&wv)[J], const uint4 (&xv)[4][J], int M, int E, int e, int t0, int lane,
                         float* __restrict__ logits, uint32_t* __restrict__ keys, bool zero_unrouted) {
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    float acc = 0.f;
    uint32_t any = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t xa[4] = {xv[tt][j].x, xv[tt][j].y, xv[tt][j].z, xv[tt][j].w};
      const uint32_t wa[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        acc = fmaf(__uint_as_float(xa[qq] << 16), __uint_as_float(wa[qq] << 16), acc);
        acc = fmaf(__uint_as_float(xa[qq] & 0xffff0000u), __uint_as_float(wa[qq] & 0xffff0000u), acc);
        any |= xa[qq] & 0x7fff7fffu;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc = acc + __shfl_xor(acc, off);
    const bool unrouted = zero_unrouted && !__any(any != 0u);
    if (lane == 0 && t0 + tt < M && e < E) {
      const size_t o = (size_t)(t0 + tt) * E + e;
      put32<AGENT>(reinterpret_cast<uint32_t*>(logits) + o, __float_as_uint(acc));
      put32<AGENT>(keys + o, unrouted ? 0u : topk_key(acc, e));
    }
  }
}

template <int J, bool AGENT>
DGM_DEV void router_wave(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int M, int E, int e,
                         int t0, int lane, float* __restrict__ logits, uint32_t* __restrict__ keys,
                         bool zero_unrouted) {
  constexpr int H = J * 512;
  uint4 wv[J];
  const int ee = e < E ? e : E - 1;
#pragma unroll
  for (int j = 0; j < J; ++j) wv[j] = *reinterpret_cast<const uint4*>(w + (size_t)ee * H + 512 * j + 8 * lane);
  uint4 xv[4][J];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const int t = t0 + tt < M ? t0 + tt : M - 1;
#pragma unroll
    for (int j = 0; j < J; ++j) xv[tt][j] = *reinterpret_cast<const uint4*>(x + (size_t)t * H + 512 * j + 8 * lane);
  }
  router_dot4<J, AGENT>(wv, xv, M, E, e, t0, lane, logits, keys, zero_unrouted);
}

// Router tile of a 256-thread workgroup for larger batches: the hidden rows of tokens
// t0 .. t0 + RT - 1 (clamped to M - 1) are staged in LDS once (xs: RT * J * 64 uint4) and wave w
// computes expert e0 + w for all of them from its router row in registers, four tokens at a
// time: each router row is read once per RT tokens and each hidden row once per four experts
// (the one-wave path reads the hidden rows once per expert). Same order of operations as
// router_wave, so the same bits.
template <int J, int RT, bool AGENT>
DGM_DEV void router_tile(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int M, int E, int e0,
                         int t0, float* __restrict__ logits, uint32_t* __restrict__ keys, bool zero_unrouted,
                         uint4* __restrict__ xs) {
  constexpr int H = J * 512, RV = RT * J * 64;       // uint4 per tile
  static_assert(RT % 4 == 0 && RV % 256 == 0, "tile of 4-token groups, whole rounds of 256 threads");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int e = e0 + wave, ee = e < E ? e : E - 1;
  uint4 wv[J];
#pragma unroll
  for (int j = 0; j < J; ++j) wv[j] = *reinterpret_cast<const uint4*>(w + (size_t)ee * H + 512 * j + 8 * lane);
  uint4 st[RV / 256];
#pragma unroll
  for (int i = 0; i < RV / 256; ++i) {
    const int v = 256 * i + tid, tt = v / (J * 64), c = v % (J * 64);
    const int t = t0 + tt < M ? t0 + tt : M - 1;
    st[i] = *reinterpret_cast<const uint4*>(x + (size_t)t * H + 8 * c);
  }
#pragma unroll
  for (int i = 0; i < RV / 256; ++i) xs[256 * i + tid] = st[i];
  __syncthreads();
#pragma unroll
  for (int g = 0; g < RT / 4; ++g) {
    uint4 xv[4][J];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
      for (int j = 0; j < J; ++j) xv[tt][j] = xs[(4 * g + tt) * (J * 64) + 64 * j + lane];
    }
    router_dot4<J, AGENT>(wv, xv, M, E, e, t0 + 4 * g, lane, logits, keys, zero_unrouted);
  }
}

// Cast lanes. MXFP4 / MXFP8: lane i of 8 per 32-element group g = i / 8 (4 elements each;
// MXFP4 rows with amax floor 1e-30, MXFP8 rows with amax floor 1e-4: the rules of
// dgm_cast_fp4_rows / dgm_cast_fp8_rows). NVFP4: 4 lanes per 16-element group (the W4A4 row
// cast: E4M3 (round to nearest even) of max(amax, 1e-30) / 6, ties-down E2M1 of x / sf). The
// lanes of a group must be adjacent and all active.
template <bool AGENT>
DGM_DEV void cast_lane_mx(const uint16_t* __restrict__ x, int act, int64_t i, uint8_t* __restrict__ q,
                          uint8_t* __restrict__ sf) {
  const int64_t g = i >> 3;
  const int part = (int)(i & 7);            // elements 4 part .. +3 of the group
  const uint2 raw = *reinterpret_cast<const uint2*>(x + g * 32 + 4 * part);
  const float v[4] = {__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                      __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u)};
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  amax = fmaxf(amax, __shfl_xor(amax, 4));
  if (act == DGM_ACT_MXFP4) {
    const uint32_t code = ceil_ue8m0_code(fmaxf(amax, 1e-30f) / 6.0f);
    const float sc = e8m0_value(code);
    uint32_t o = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) o |= e2m1_ties_down(v[k] / sc) << (4 * k);
    put16<AGENT>(reinterpret_cast<uint16_t*>(q) + g * 8 + part, o);
    if (part == 0) put8<AGENT>(sf + g, code);
  } else {
    const uint32_t code = ceil_ue8m0_code(fmaxf(amax, 1e-4f) / 448.0f);
    const float inv = 1.0f / e8m0_value(code);
    uint32_t o = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) o |= e4m3_encode(v[k] * inv) << (8 * k);
    put32<AGENT>(reinterpret_cast<uint32_t*>(q) + g * 8 + part, o);
    if (part == 0) put8<AGENT>(sf + g, code);
  }
}

template <bool AGENT>
DGM_DEV void cast_lane_nvfp4(const uint16_t* __restrict__ x, int64_t i, uint8_t* __restrict__ q,
                             uint8_t* __restrict__ sf) {
  const int64_t g = i >> 2;
  const int part = (int)(i & 3);
  const uint2 raw = *reinterpret_cast<const uint2*>(x + g * 16 + 4 * part);
  const float v[4] = {__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                      __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u)};
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  const uint32_t code = e4m3_encode(fmaxf(amax, 1e-30f) / 6.0f);
  const float sc = __builtin_amdgcn_cvt_f32_fp8((int)code, 0);
  uint32_t o = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) o |= e2m1_ties_down(v[k] / sc) << (4 * k);
  put16<AGENT>(reinterpret_cast<uint16_t*>(q) + g * 4 + part, o);
  if (part == 0) put8<AGENT>(sf + g, code);
}

// FP8 rows with one fp32 scale per 128 (per_token_cast_to_fp8(use_ue8m0=False, gran_k=128),
// deep_gemm/utils/math.py:26-38): 32 adjacent lanes per 128-element group, 4 elements each;
// sf = max(amax, 1e-4) / 448, E4M3 (round to nearest even) of x * (1 / sf) (IEEE division).
template <bool AGENT>
DGM_DEV void cast_lane_fp8f128(const uint16_t* __restrict__ x, int64_t i, uint8_t* __restrict__ q,
                               uint8_t* __restrict__ sf) {
  const int64_t g = i >> 5;
  const int part = (int)(i & 31);
  const uint2 raw = *reinterpret_cast<const uint2*>(x + g * 128 + 4 * part);
  const float v[4] = {__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                      __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u)};
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
  for (int off = 1; off < 32; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float s = fmaxf(amax, 1e-4f) / 448.0f;
  const float inv = 1.0f / s;
  uint32_t o = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) o |= e4m3_encode(v[k] * inv) << (8 * k);
  put32<AGENT>(reinterpret_cast<uint32_t*>(q) + g * 32 + part, o);
  if (part == 0) put32<AGENT>(reinterpret_cast<uint32_t*>(sf) + g, __float_as_uint(s));
}

// QoQ per-token int8 cast (per_token_cast_to_int8) of token t by one wave: lane l holds
// elements 512 j + 8 l .. +7; sf = max(amax, 1e-30) / 127 (fp32), q = clamp(rne(x / sf),
// +-127); the scale is repeated over the row's H / 128 slots.
template <int J, bool AGENT>
DGM_DEV void cast_qoq_token(const uint16_t* __restrict__ x, int t, int lane, uint8_t* __restrict__ q,
                            uint8_t* __restrict__ sf) {
  constexpr int H = J * 512;
  uint4 xv[J];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    xv[j] = *reinterpret_cast<const uint4*>(x + (size_t)t * H + 512 * j + 8 * lane);
    const uint32_t d[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
      amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(d[k] << 16)), fabsf(__uint_as_float(d[k] & 0xffff0000u))));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float scale = fmaxf(amax, 1e-30f) / 127.0f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint32_t d[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
    uint32_t o[2] = {0u, 0u};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t bits = (k & 1) ? (d[k >> 1] & 0xffff0000u) : (d[k >> 1] << 16);
      const float v = fminf(fmaxf(rintf(__uint_as_float(bits) / scale), -127.f), 127.f);
      o[k >> 2] |= ((uint32_t)(int)v & 0xffu) << (8 * (k & 3));
    }
    put64<AGENT>(reinterpret_cast<uint64_t*>(q + (size_t)t * H + 512 * j + 8 * lane), (uint64_t)o[0] | ((uint64_t)o[1] << 32));
  }
  if (lane < H / 128) put32<AGENT>(reinterpret_cast<uint32_t*>(sf) + (size_t)t * (H / 128) + lane, __float_as_uint(scale));
}

}  // namespace dgm
