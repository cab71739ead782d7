// Weight packers, activation casts and the weight-layout transform (gfx950).
//
// Every kernel restates one reference packer rule bit for bit (citations on each
// extern "C" entry in include/dgm_megamoe.h). They are memory-bound byte/integer passes:
// one thread owns one scale group, reads its elements with vector loads and writes the
// packed bytes with vector stores; no LDS, no matrix cores.
#include "dgm_common.hpp"
#include "dgm_abi_internal.hpp"

using namespace dgm;

namespace {

struct alignas(16) U4 { uint32_t x, y, z, w; };

// Load 32 bf16 (64 B) of one group starting at p (16-byte aligned).
DGM_DEV void load32_bf16(const uint16_t* p, float* v) {
  const U4* q = reinterpret_cast<const U4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    U4 r = q[i];
    uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[i * 8 + 2 * j] = __uint_as_float(w[j] << 16);
      v[i * 8 + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
}

// Source element types of the weight packers (the reference packers take any float tensor and
// compute on its fp32 value: weight.to(torch.float32)); every one converts to fp32 exactly.
enum SrcType { SRC_BF16 = 0, SRC_F16 = 1, SRC_F32 = 2 };

DGM_DEV float half_bits_to_f32(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// N (a multiple of 8) consecutive elements starting at element `off` of a SRC array (16-byte
// aligned there) as fp32.
template <int SRC, int N>
DGM_DEV void load_vals(const void* base, int64_t off, float* v) {
  static_assert(N % 8 == 0, "whole 16-byte loads");
  if constexpr (SRC == SRC_F32) {
    const U4* q = reinterpret_cast<const U4*>(reinterpret_cast<const float*>(base) + off);
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const U4 r = q[i];
      v[4 * i] = __uint_as_float(r.x);
      v[4 * i + 1] = __uint_as_float(r.y);
      v[4 * i + 2] = __uint_as_float(r.z);
      v[4 * i + 3] = __uint_as_float(r.w);
    }
  } else {
    const U4* q = reinterpret_cast<const U4*>(reinterpret_cast<const uint16_t*>(base) + off);
#pragma unroll
    for (int i = 0; i < N / 8; ++i) {
      const U4 r = q[i];
      const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (SRC == SRC_BF16) {
          v[i * 8 + 2 * j] = __uint_as_float(w[j] << 16);
          v[i * 8 + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        } else {
          v[i * 8 + 2 * j] = half_bits_to_f32(w[j] & 0xffffu);
          v[i * 8 + 2 * j + 1] = half_bits_to_f32(w[j] >> 16);
        }
      }
    }
  }
}

// Element i of a SRC array as fp32.
template <int SRC>
DGM_DEV float load_one(const void* base, int64_t i) {
  if constexpr (SRC == SRC_F32) return reinterpret_cast<const float*>(base)[i];
  else if constexpr (SRC == SRC_F16) return half_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[i]);
  else return bf16_to_f32(reinterpret_cast<const uint16_t*>(base)[i]);
}

// Marlin byte order of 8 nibbles n[0..7]: byte b = n[b] << 4 | n[b+4]  -> one u32.
DGM_DEV uint32_t marlin8(const uint32_t* n) {
  uint32_t w = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) w |= ((n[b] << 4) | n[b + 4]) << (8 * b);
  return w;
}
// Low-nibble-first order of 8 nibbles: byte j = n[2j] | n[2j+1] << 4.
DGM_DEV uint32_t lowfirst8(const uint32_t* n) {
  uint32_t w = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) w |= (n[2 * j] | (n[2 * j + 1] << 4)) << (8 * j);
  return w;
}

// ------------------------------------------------------------------ MXFP4 weight packers
// rule 0: quantization_mxfp4_fused.quantize_to_mxfp4; rule 1: quantization_mxfp4.quantize_to_mxfp4.
template <int SRC>
__global__ void k_quantize_mxfp4(const void* __restrict__ w, int64_t groups, int rule,
                                 uint32_t* __restrict__ packed, uint8_t* __restrict__ scale) {
  int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= groups) return;
  float v[32];
  load_vals<SRC, 32>(w, g * 32, v);
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  float sc;
  uint32_t code;
  if (rule == 0) {
    float e = amax > 0.f ? ceil_log2_f32(fmaxf(amax, 1e-38f) / 6.0f) : -127.f;
    e = fminf(fmaxf(e, -127.f), 127.f);
    code = (uint32_t)((int)e + 127);
    sc = e8m0_value_any(code);
  } else {
    float d = fminf(fmaxf(fmaxf(amax, 1e-30f) / 6.0f, 0x1p-126f), 0x1p127f);
    int c = (int)ceil_log2_f32(d) + 127;
    c = c < 1 ? 1 : (c > 254 ? 254 : c);
    code = (uint32_t)c;
    sc = e8m0_value(code);
  }
  uint32_t out[4];
#pragma unroll
  for (int c8 = 0; c8 < 4; ++c8) {
    uint32_t n[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) n[i] = e2m1_bucketize(fminf(fmaxf(v[c8 * 8 + i] / sc, -6.f), 6.f));
    out[c8] = marlin8(n);
  }
  reinterpret_cast<U4*>(packed)[g] = U4{out[0], out[1], out[2], out[3]};
  scale[g] = (uint8_t)code;
}

// ------------------------------------------------------------------ row casts (activations)
// MXFP4 rows: amax >= floor, sf = ceil_ue8m0(amax/6), ties-down E2M1 of x/sf, low-nibble-first.
__global__ void k_cast_fp4_rows(const uint16_t* __restrict__ x, int64_t groups, float amax_floor,
                                uint32_t* __restrict__ packed, uint8_t* __restrict__ sf) {
  int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= groups) return;
  float v[32];
  load32_bf16(x + g * 32, v);
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  uint32_t code = ceil_ue8m0_code(fmaxf(amax, amax_floor) / 6.0f);
  float s = e8m0_value(code);
  uint32_t out[4];
#pragma unroll
  for (int c8 = 0; c8 < 4; ++c8) {
    uint32_t n[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) n[i] = e2m1_ties_down(v[c8 * 8 + i] / s);
    out[c8] = lowfirst8(n);
  }
  reinterpret_cast<U4*>(packed)[g] = U4{out[0], out[1], out[2], out[3]};
  sf[g] = (uint8_t)code;
}

// MXFP8 rows: amax >= 1e-4, sf = ceil_ue8m0(amax/448), e4m3(x * (1/sf)).
__global__ void k_cast_fp8_rows(const uint16_t* __restrict__ x, int64_t groups,
                                uint32_t* __restrict__ q, uint8_t* __restrict__ sf) {
  int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= groups) return;
  float v[32];
  load32_bf16(x + g * 32, v);
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  uint32_t code = ceil_ue8m0_code(fmaxf(amax, 1e-4f) / 448.0f);
  float inv = 1.0f / e8m0_value(code);
  uint32_t out[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t w = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) w |= e4m3_encode(v[j * 4 + b] * inv) << (8 * b);
    out[j] = w;
  }
  U4* dst = reinterpret_cast<U4*>(q) + g * 2;
  dst[0] = U4{out[0], out[1], out[2], out[3]};
  dst[1] = U4{out[4], out[5], out[6], out[7]};
  sf[g] = (uint8_t)code;
}

// ------------------------------------------------------------------ NVFP4 packer
DGM_DEV uint32_t ue4m3_ceil(float x) {
  x = fminf(fmaxf(x, 0x1p-9f), 448.0f);
  int den = (int)ceilf(x / 0x1p-9f);
  den = den < 1 ? 1 : (den > 7 ? 7 : den);
  float xn = fmaxf(x, 0x1p-6f);
  float e = floorf((float)log2((double)xn));
  int eb = (int)e + 7;
  float base = exp2f(e);
  float t = (xn / base - 1.0f) * 8.0f - 1e-6f;
  int mant = (int)ceilf(t);
  if (mant > 7) { eb += 1; mant = 0; }
  mant = mant < 0 ? 0 : (mant > 7 ? 7 : mant);
  int normal = eb * 8 + mant;
  normal = normal < 8 ? 8 : (normal > 0x7e ? 0x7e : normal);
  return x <= 7.0f * 0x1p-9f ? (uint32_t)den : (uint32_t)normal;
}
DGM_DEV float ue4m3_value(uint32_t c) {
  c &= 0x7fu;
  uint32_t eb = c >> 3, m = c & 7u;
  if (c == 0x7fu) return 448.0f;
  if (eb == 0) return (float)m * 0x1p-9f;
  return (1.0f + (float)m * 0.125f) * exp2f((float)((int)eb - 7));
}

template <int SRC>
__global__ void k_quantize_nvfp4(const void* __restrict__ w, int64_t groups16,
                                 uint32_t* __restrict__ packed, uint8_t* __restrict__ scale) {
  int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= groups16) return;
  float v[16];
  load_vals<SRC, 16>(w, g * 16, v);
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
  uint32_t code = ue4m3_ceil(fmaxf(amax, 1e-30f) / 6.0f);
  float s = ue4m3_value(code);
  uint32_t out[2];
#pragma unroll
  for (int c8 = 0; c8 < 2; ++c8) {
    uint32_t n[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) n[i] = e2m1_bucketize(fminf(fmaxf(v[c8 * 8 + i] / s, -6.f), 6.f));
    out[c8] = marlin8(n);
  }
  packed[g * 2] = out[0];
  packed[g * 2 + 1] = out[1];
  scale[g] = (uint8_t)code;
}

// ------------------------------------------------------------------ QoQ W4A8 packer
// One wave per weight row: row amax -> s1 (bf16), then lane-per-K128-group codes.
// plane != null: the split path's int4 form (s2 clamped to 127 instead of 15, which |w8| <= 112
// never reaches; s2 | z << 8 | bf16(s1) << 16 per (row, K128 group) instead of s2o / zo / s1o)
template <int SRC>
__global__ void k_quantize_qoq(const void* __restrict__ w, int64_t rows, int K,
                               uint8_t* __restrict__ packed, uint8_t* __restrict__ s2o,
                               uint8_t* __restrict__ zo, float* __restrict__ s1o, uint32_t* __restrict__ plane) {
  int lane = threadIdx.x & 63;
  int64_t row = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t src = row * K;        // the row's first element
  float amax = 0.f;
  for (int k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(load_one<SRC>(w, src + k)));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  float s1 = round_bf16(fmaxf(amax / 120.0f, 1e-30f));
  if (lane == 0 && !plane) s1o[row] = s1;
  int G = K / 128;
  for (int g = lane; g < G; g += 64) {
    const int64_t p = src + g * 128;
    float mn = 1e30f, mx = -1e30f;
    for (int i = 0; i < 128; ++i) {
      float w8 = fminf(fmaxf(rintf(load_one<SRC>(w, p + i) / s1), -112.f), 112.f);
      mn = fminf(mn, w8);
      mx = fmaxf(mx, w8);
    }
    float s2 = fminf(fmaxf(ceilf((mx - mn) / 15.0f), 1.f), plane ? 127.f : 15.f);
    float z = fminf(fmaxf(rintf(-mn / s2), 0.f), 15.f);
    uint32_t* dst = reinterpret_cast<uint32_t*>(packed + row * (K / 2) + g * 64);
    for (int c8 = 0; c8 < 16; ++c8) {
      uint32_t n[8];
      for (int i = 0; i < 8; ++i) {
        float w8 = fminf(fmaxf(rintf(load_one<SRC>(w, p + c8 * 8 + i) / s1), -112.f), 112.f);
        n[i] = (uint32_t)fminf(fmaxf(rintf(w8 / s2 + z), 0.f), 15.f);
      }
      dst[c8] = marlin8(n);
    }
    if (plane) {
      plane[row * G + g] = (__float_as_uint(s1) & 0xFFFF0000u) | ((uint32_t)z << 8) | (uint32_t)s2;
    } else {
      s2o[row * G + g] = (uint8_t)s2;
      zo[row * G + g] = (uint8_t)z;
    }
  }
}

// Per-token int8: sf = max(amax, 1e-30)/127, q = clamp(rne(x/sf), +-127). One wave per row.
__global__ void k_cast_int8_rows(const uint16_t* __restrict__ x, int64_t rows, int K,
                                 int8_t* __restrict__ q, float* __restrict__ sf) {
  int lane = threadIdx.x & 63;
  int64_t row = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* src = x + row * K;
  float amax = 0.f;
  for (int k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(bf16_to_f32(src[k])));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  float s = fmaxf(amax, 1e-30f) / 127.0f;
  if (lane == 0) sf[row] = s;
  for (int k = lane; k < K; k += 64)
    q[row * K + k] = (int8_t)fminf(fmaxf(rintf(bf16_to_f32(src[k]) / s), -127.f), 127.f);
}

// Source row of row r of native block q (16 rows each). l1_interleave 0: rows as they are;
// 1: W1 with gate rows [0, N/2) then up rows [N/2, N) -> block 2p = gate rows 16p.., block
// 2p+1 = up rows N/2 + 16p..; 2: W1 with gate and up rows interleaved (row 2i = gate row i,
// row 2i+1 = up row i) -> the same native blocks.
DGM_DEV int native_src_row(int q, int r, int N, int l1_interleave) {
  if (l1_interleave == 1) return (q & 1) ? (N / 2 + 16 * (q >> 1) + r) : (16 * (q >> 1) + r);
  if (l1_interleave == 2) return 2 * (16 * (q >> 1) + r) + (q & 1);
  return 16 * q + r;
}

// ------------------------------------------------------------------ FP4 weight-layout transform
// Source: packed [E][N][K/2] (Marlin or low-first order), scale [E][N][K/32] E8M0 bytes.
// Destination (matrix-core fragment order, see dgm_layout in dgm_abi_internal.hpp):
//   values [E][N/16][K/128][64 lanes][16 B]: lane l = row l%16 of the 16-row block,
//          K = 128*kt + 32*(l/16) .. +32, byte j = K[2j] | K[2j+1] << 4.
//   scales [E][N/16][ceil(K/512)][64 lanes][4 B]: byte j = scale of K-tile 4*g + j.
// l1_interleave (native_src_row): native block q holds the gate rows of features 16*(q/2)..
// (q even) or the up rows of the same features (q odd), so a (gate, up) pair of blocks covers
// the same 16 features.
__global__ void k_transform_fp4(const uint8_t* __restrict__ src, const uint8_t* __restrict__ ssrc,
                                int E, int N, int K, int src_order, int l1_interleave,
                                uint8_t* __restrict__ dst, uint8_t* __restrict__ sdst) {
  int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int KT = K / 128, NB = N / 16, KG = (KT + 3) / 4;
  int64_t total = (int64_t)E * NB * KT * 64;
  if (tid >= total) return;
  int lane = (int)(tid & 63);
  int64_t t = tid >> 6;
  int kt = (int)(t % KT); t /= KT;
  int q = (int)(t % NB);
  int e = (int)(t / NB);
  int r = lane & 15, kq = lane >> 4;
  const int src_row = native_src_row(q, r, N, l1_interleave);
  const uint8_t* s = src + ((int64_t)e * N + src_row) * (K / 2) + kt * 64 + kq * 16;
  U4 in = *reinterpret_cast<const U4*>(s);
  uint32_t w[4] = {in.x, in.y, in.z, in.w};
  uint32_t o[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint32_t n[8];
    if (src_order == 0) {        // Marlin: byte b = K[b] << 4 | K[b+4]
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        uint32_t byte = (w[c] >> (8 * b)) & 0xffu;
        n[b] = byte >> 4;
        n[b + 4] = byte & 0xfu;
      }
      o[c] = lowfirst8(n);
    } else {
      o[c] = w[c];
    }
  }
  int64_t tile = ((int64_t)e * NB + q) * KT + kt;
  *reinterpret_cast<U4*>(dst + tile * 1024 + lane * 16) = U4{o[0], o[1], o[2], o[3]};
  uint8_t sc = ssrc[((int64_t)e * N + src_row) * (K / 32) + kt * 4 + kq];
  sdst[((((int64_t)e * NB + q) * KG + kt / 4) * 64 + lane) * 4 + (kt & 3)] = sc;
}

// NVFP4 weights -> the fused kernel's layout for the f16 matrix core (one thread per (expert,
// 16-row block, K-tile, lane)). Source: packed [E][N][K/2] (Marlin or low-first order), scales
// [E][N][K/16] E4M3 bytes. Values [E][N/16][K/128][64 lanes][16 B]: lane l = row l%16; dword j
// holds op j's eight codes K = 128 kt + 32 j + 8 (l/16) .. +8, byte b = K[2b] | K[2b+1] << 4.
// Scales [E][N/16][K/128][2][16][4 B]: dword (p, r) byte j = the scale of row r, 16-block
// 8 kt + 2 j + p, so lane l reads dword (l/32, l%16) for the four blocks its ops touch.
__global__ void k_transform_nvfp4(const uint8_t* __restrict__ src, const uint8_t* __restrict__ ssrc,
                                  int E, int N, int K, int src_order, int l1_interleave,
                                  uint8_t* __restrict__ dst, uint8_t* __restrict__ sdst) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int KT = K / 128, NB = N / 16;
  const int64_t total = (int64_t)E * NB * KT * 64;
  if (tid >= total) return;
  const int lane = (int)(tid & 63);
  int64_t t = tid >> 6;
  const int kt = (int)(t % KT); t /= KT;
  const int q = (int)(t % NB);
  const int e = (int)(t / NB);
  const int r = lane & 15, g = lane >> 4;
  const int src_row = native_src_row(q, r, N, l1_interleave);
  const uint8_t* row = src + ((int64_t)e * N + src_row) * (K / 2) + kt * 64;
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(row + 16 * j + 4 * g);   // K 32 j + 8 g .. +8
    if (src_order == 0) {        // Marlin: byte b = K[b] << 4 | K[b+4]
      uint32_t n[8];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t byte = (w >> (8 * b)) & 0xffu;
        n[b] = byte >> 4;
        n[b + 4] = byte & 0xfu;
      }
      o[j] = lowfirst8(n);
    } else {
      o[j] = w;
    }
  }
  const int64_t tile = ((int64_t)e * NB + q) * KT + kt;
  *reinterpret_cast<U4*>(dst + tile * 1024 + lane * 16) = U4{o[0], o[1], o[2], o[3]};
  if ((g & 1) == 0) {
    const int p = g >> 1;
    const uint8_t* sr = ssrc + ((int64_t)e * N + src_row) * (K / 16) + 8 * kt + p;
    const uint32_t sd = (uint32_t)sr[0] | ((uint32_t)sr[2] << 8) | ((uint32_t)sr[4] << 16) | ((uint32_t)sr[6] << 24);
    *reinterpret_cast<uint32_t*>(sdst + tile * 128 + (16 * p + r) * 4) = sd;
  }
}

// ------------------------------------------------------------------ checkpoint formats
// Nibble order of one 4-byte word of packed E2M1 codes (8 codes): Marlin (byte b = n[b] << 4 |
// n[b+4]) <-> low-nibble-first (OCP: byte j = n[2j] | n[2j+1] << 4).
DGM_DEV uint32_t marlin_to_lowfirst32(uint32_t w) {
  uint32_t n[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint32_t byte = (w >> (8 * b)) & 0xffu;
    n[b] = byte >> 4;
    n[b + 4] = byte & 0xfu;
  }
  return lowfirst8(n);
}
DGM_DEV uint32_t lowfirst_to_marlin32(uint32_t w) {
  uint32_t n[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) n[k] = (w >> (4 * k)) & 0xfu;
  return marlin8(n);
}
DGM_DEV uint32_t reorder32(uint32_t w, int from, int to) {
  if (from == to) return w;
  return from == 0 ? marlin_to_lowfirst32(w) : lowfirst_to_marlin32(w);
}

// One thread per 16 bytes (the last thread may own fewer whole words); in place is allowed.
// (src == dst converts in place: each thread reads its words before it writes them, so no
// __restrict__ here)
__global__ void k_reorder_fp4(const uint8_t* src, uint8_t* dst, int64_t words,
                              int from, int to) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= words) return;
  if (i + 4 <= words) {
    const U4 v = *reinterpret_cast<const U4*>(src + 4 * i);
    *reinterpret_cast<U4*>(dst + 4 * i) = U4{reorder32(v.x, from, to), reorder32(v.y, from, to),
                                             reorder32(v.z, from, to), reorder32(v.w, from, to)};
  } else {
    for (int64_t j = i; j < words; ++j) {
      const uint32_t v = reinterpret_cast<const uint32_t*>(src)[j];
      reinterpret_cast<uint32_t*>(dst)[j] = reorder32(v, from, to);
    }
  }
}

// Inverse of k_transform_fp4: the tile layout back to packed [E][N][K/2] (dst_order 0 Marlin,
// 1 low-nibble-first) and E8M0 scales [E][N][K/32], rows in checkpoint order (gate rows, then
// up rows, when l1_interleave). Same thread mapping as the forward pass.
__global__ void k_untransform_fp4(const uint8_t* __restrict__ vals, const uint8_t* __restrict__ svals, int E, int N,
                                  int K, int dst_order, int l1_interleave, uint8_t* __restrict__ dst,
                                  uint8_t* __restrict__ sdst) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int KT = K / 128, NB = N / 16, KG = (KT + 3) / 4;
  const int64_t total = (int64_t)E * NB * KT * 64;
  if (tid >= total) return;
  const int lane = (int)(tid & 63);
  int64_t t = tid >> 6;
  const int kt = (int)(t % KT); t /= KT;
  const int q = (int)(t % NB);
  const int e = (int)(t / NB);
  const int r = lane & 15, kq = lane >> 4;
  const int row = native_src_row(q, r, N, l1_interleave);
  const int64_t tile = ((int64_t)e * NB + q) * KT + kt;
  const U4 in = *reinterpret_cast<const U4*>(vals + tile * 1024 + lane * 16);
  *reinterpret_cast<U4*>(dst + ((int64_t)e * N + row) * (K / 2) + kt * 64 + kq * 16) =
      U4{reorder32(in.x, 1, dst_order), reorder32(in.y, 1, dst_order), reorder32(in.z, 1, dst_order),
         reorder32(in.w, 1, dst_order)};
  sdst[((int64_t)e * N + row) * (K / 32) + kt * 4 + kq] =
      svals[((((int64_t)e * NB + q) * KG + kt / 4) * 64 + lane) * 4 + (kt & 3)];
}

// Inverse of k_transform_nvfp4: packed [E][N][K/2] (dst_order as above) and E4M3 scales
// [E][N][K/16]. Lanes of groups 0 and 2 also write their row's eight scale bytes of the tile.
__global__ void k_untransform_nvfp4(const uint8_t* __restrict__ vals, const uint8_t* __restrict__ svals, int E,
                                    int N, int K, int dst_order, int l1_interleave, uint8_t* __restrict__ dst,
                                    uint8_t* __restrict__ sdst) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int KT = K / 128, NB = N / 16;
  const int64_t total = (int64_t)E * NB * KT * 64;
  if (tid >= total) return;
  const int lane = (int)(tid & 63);
  int64_t t = tid >> 6;
  const int kt = (int)(t % KT); t /= KT;
  const int q = (int)(t % NB);
  const int e = (int)(t / NB);
  const int r = lane & 15, g = lane >> 4;
  const int row = native_src_row(q, r, N, l1_interleave);
  const int64_t tile = ((int64_t)e * NB + q) * KT + kt;
  const U4 in = *reinterpret_cast<const U4*>(vals + tile * 1024 + lane * 16);
  const uint32_t o[4] = {in.x, in.y, in.z, in.w};
  uint8_t* drow = dst + ((int64_t)e * N + row) * (K / 2) + kt * 64;
#pragma unroll
  for (int j = 0; j < 4; ++j) *reinterpret_cast<uint32_t*>(drow + 16 * j + 4 * g) = reorder32(o[j], 1, dst_order);
  if ((g & 1) == 0) {
    const int p = g >> 1;
    const uint32_t sd = *reinterpret_cast<const uint32_t*>(svals + tile * 128 + (16 * p + r) * 4);
    uint8_t* sr = sdst + ((int64_t)e * N + row) * (K / 16) + 8 * kt + p;
#pragma unroll
    for (int j = 0; j < 4; ++j) sr[2 * j] = (uint8_t)(sd >> (8 * j));
  }
}

// QoQ (W4A8) weights -> the fused kernel's layout (one thread per (expert, 16-row block,
// K-tile, lane)). Values [E][N/16][K/128][64][16 B]: lane l = row l%16; its 16 bytes hold the
// two K=64 int8 operands (op h: codes n[h][j] of K = 64 h + 16 (l/16) + j, j = 0..15) as
// nibbles. L1 (l1_interleave = 1), paired: dword 2h byte b = n[h][b] | n[h][4+b] << 4, dword
// 2h+1 byte b = n[h][8+b] | n[h][12+b] << 4, so op h's codes come out as (d & 0x0F0F0F0F,
// (d >> 4) & 0x0F0F0F0F) of its two dwords. L2 (l1_interleave = 0), chunk-split: dword q byte
// b = n[0][4q+b] | (n[1][4q+b] ^ 8) << 4, so op 0 is (d & 0x0F0F0F0F) and op 1 is
// (d & 0xF0F0F0F0) = 16 code - 128 as int8, one mask per dword. Meta [E][N/16][K/128]
// [16 B]: byte r = z | s2 << 4 of row r (both are 4-bit by construction: z 0..15, s2 1..15),
// so dword kq holds the four rows 4 kq .. +3 that lane group kq accumulates. s1 [E][N] in the
// same row order. l1_interleave as for the MXFP4 transform.
// plane != null: s2, z and s1 come from the int4 packer's coefficient plane (bytes 0, 1 and the
// bf16 high half of each (row, K128 group) word) instead of s2 / z / s1
__global__ void k_transform_qoq(const uint8_t* __restrict__ src, const uint8_t* __restrict__ s2,
                                const uint8_t* __restrict__ z, const float* __restrict__ s1,
                                const uint32_t* __restrict__ plane, int E, int N,
                                int K, int l1_interleave, uint8_t* __restrict__ dst, uint8_t* __restrict__ mdst,
                                float* __restrict__ s1dst) {
  int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int KT = K / 128, NB = N / 16;
  const int64_t total = (int64_t)E * NB * KT * 64;
  if (tid >= total) return;
  const int lane = (int)(tid & 63);
  int64_t t = tid >> 6;
  const int kt = (int)(t % KT); t /= KT;
  const int q = (int)(t % NB);
  const int e = (int)(t / NB);
  const int r = lane & 15, g = lane >> 4;
  const int src_row = native_src_row(q, r, N, l1_interleave);
  const uint8_t* row = src + ((int64_t)e * N + src_row) * (K / 2);
  uint32_t n[2][16];       // codes of K = 128 kt + 64 h + 16 g + j
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // two Marlin chunks of 8 (byte b = K[b] << 4 | K[b+4])
    const uint8_t* c = row + (128 * kt + 64 * h + 16 * g) / 2;
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t byte = c[4 * ch + b];
        n[h][8 * ch + b] = byte >> 4;
        n[h][8 * ch + b + 4] = byte & 0xfu;
      }
  }
  uint32_t o[4] = {0u, 0u, 0u, 0u};
  if (l1_interleave) {
    // paired: dword 2h byte b = n[h][b] | n[h][4+b] << 4, dword 2h+1 byte b = n[h][8+b] | n[h][12+b] << 4
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        o[2 * h] |= (n[h][b] | (n[h][4 + b] << 4)) << (8 * b);
        o[2 * h + 1] |= (n[h][8 + b] | (n[h][12 + b] << 4)) << (8 * b);
      }
  } else {
    // chunk-split: dword q byte b = n[0][4q+b] | (n[1][4q+b] ^ 8) << 4
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int b = 0; b < 4; ++b) o[q] |= (n[0][4 * q + b] | ((n[1][4 * q + b] ^ 8u) << 4)) << (8 * b);
  }
  const int64_t tile = ((int64_t)e * NB + q) * KT + kt;
  *reinterpret_cast<U4*>(dst + tile * 1024 + lane * 16) = U4{o[0], o[1], o[2], o[3]};
  if (g == 0) {
    const int64_t mi = ((int64_t)e * N + src_row) * KT + kt;
    const uint32_t zv = plane ? (plane[mi] >> 8) & 0xffu : z[mi], sv = plane ? plane[mi] & 0xffu : s2[mi];
    mdst[tile * 16 + r] = (uint8_t)((zv & 15u) | (sv << 4));
    if (kt == 0)
      s1dst[((int64_t)e * NB + q) * 16 + r] = plane ? __uint_as_float(plane[mi] & 0xFFFF0000u) : s1[(int64_t)e * N + src_row];
  }
}

// Fill the padding bytes of the last scale group (K-tiles KT..4*KG-1) with 127 (= 2^0).
__global__ void k_fill_scale_pad(uint8_t* sdst, int64_t blocks, int KT, int KG) {
  int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int pad = KG * 4 - KT;
  if (pad == 0) return;
  int64_t total = blocks * 64 * pad;
  if (tid >= total) return;
  int p = (int)(tid % pad);
  int64_t t = tid / pad;
  int lane = (int)(t & 63);
  int64_t b = t >> 6;
  int kt = KT + p;
  sdst[((b * KG + kt / 4) * 64 + lane) * 4 + (kt & 3)] = 127;
}

inline int grid_for(int64_t n, int bs) { return (int)((n + bs - 1) / bs); }

}  // namespace

// ==================================================================== C ABI
extern "C" {

int dgm_quantize_mxfp4(const void* w_bf16, int64_t rows, int64_t K, int rule,
                       void* packed, void* scale_e8m0, hipStream_t stream) {
  return dgm_quantize_mxfp4_typed(w_bf16, DGM_SRC_BF16, rows, K, rule, packed, scale_e8m0, stream);
}

int dgm_quantize_mxfp4_typed(const void* w_bf16, int src_dtype, int64_t rows, int64_t K, int rule,
                             void* packed, void* scale_e8m0, hipStream_t stream) {
  DGM_CHECK_ARG(w_bf16 && packed && scale_e8m0, "null pointer");
  DGM_CHECK_ARG(src_dtype >= DGM_SRC_BF16 && src_dtype <= DGM_SRC_F32, "src_dtype 0 bf16, 1 fp16, 2 fp32");
  DGM_CHECK_ARG(rows >= 0 && K > 0 && K % 32 == 0, "K must be a positive multiple of 32");
  DGM_CHECK_ARG(rule == 0 || rule == 1, "rule must be 0 (fused) or 1 (split)");
  DGM_CHECK_ARG(((uintptr_t)w_bf16 & 15) == 0 && ((uintptr_t)packed & 15) == 0, "16-byte alignment");
  int64_t groups = rows * (K / 32);
  if (groups == 0) return 0;
  const dim3 gd(grid_for(groups, 256));
  if (src_dtype == DGM_SRC_F32)
    hipLaunchKernelGGL(k_quantize_mxfp4<SRC_F32>, gd, dim3(256), 0, stream, w_bf16, groups, rule, (uint32_t*)packed,
                       (uint8_t*)scale_e8m0);
  else if (src_dtype == DGM_SRC_F16)
    hipLaunchKernelGGL(k_quantize_mxfp4<SRC_F16>, gd, dim3(256), 0, stream, w_bf16, groups, rule, (uint32_t*)packed,
                       (uint8_t*)scale_e8m0);
  else
    hipLaunchKernelGGL(k_quantize_mxfp4<SRC_BF16>, gd, dim3(256), 0, stream, w_bf16, groups, rule, (uint32_t*)packed,
                       (uint8_t*)scale_e8m0);
  return dgm_last_launch_status();
}

int dgm_cast_fp4_rows(const void* x_bf16, int64_t rows, int64_t K, float amax_floor,
                      void* packed, void* sf_e8m0, hipStream_t stream) {
  DGM_CHECK_ARG(x_bf16 && packed && sf_e8m0, "null pointer");
  DGM_CHECK_ARG(rows >= 0 && K > 0 && K % 32 == 0, "K must be a positive multiple of 32");
  DGM_CHECK_ARG(((uintptr_t)x_bf16 & 15) == 0 && ((uintptr_t)packed & 15) == 0, "16-byte alignment");
  int64_t groups = rows * (K / 32);
  if (groups == 0) return 0;
  hipLaunchKernelGGL(k_cast_fp4_rows, dim3(grid_for(groups, 256)), dim3(256), 0, stream,
                     (const uint16_t*)x_bf16, groups, amax_floor, (uint32_t*)packed, (uint8_t*)sf_e8m0);
  return dgm_last_launch_status();
}

int dgm_cast_fp8_rows(const void* x_bf16, int64_t rows, int64_t K, void* q_e4m3, void* sf_e8m0,
                      hipStream_t stream) {
  DGM_CHECK_ARG(x_bf16 && q_e4m3 && sf_e8m0, "null pointer");
  DGM_CHECK_ARG(rows >= 0 && K > 0 && K % 32 == 0, "K must be a positive multiple of 32");
  DGM_CHECK_ARG(((uintptr_t)x_bf16 & 15) == 0 && ((uintptr_t)q_e4m3 & 15) == 0, "16-byte alignment");
  int64_t groups = rows * (K / 32);
  if (groups == 0) return 0;
  hipLaunchKernelGGL(k_cast_fp8_rows, dim3(grid_for(groups, 256)), dim3(256), 0, stream,
                     (const uint16_t*)x_bf16, groups, (uint32_t*)q_e4m3, (uint8_t*)sf_e8m0);
  return dgm_last_launch_status();
}

int dgm_quantize_nvfp4(const void* w_bf16, int64_t rows, int64_t K, void* packed, void* scale_ue4m3,
                       hipStream_t stream) {
  return dgm_quantize_nvfp4_typed(w_bf16, DGM_SRC_BF16, rows, K, packed, scale_ue4m3, stream);
}

int dgm_quantize_nvfp4_typed(const void* w_bf16, int src_dtype, int64_t rows, int64_t K, void* packed,
                             void* scale_ue4m3, hipStream_t stream) {
  DGM_CHECK_ARG(w_bf16 && packed && scale_ue4m3, "null pointer");
  DGM_CHECK_ARG(src_dtype >= DGM_SRC_BF16 && src_dtype <= DGM_SRC_F32, "src_dtype 0 bf16, 1 fp16, 2 fp32");
  DGM_CHECK_ARG(rows >= 0 && K > 0 && K % 16 == 0, "K must be a positive multiple of 16");
  DGM_CHECK_ARG(((uintptr_t)w_bf16 & 15) == 0 && ((uintptr_t)packed & 7) == 0, "alignment");
  int64_t groups = rows * (K / 16);
  if (groups == 0) return 0;
  const dim3 gd(grid_for(groups, 256));
  if (src_dtype == DGM_SRC_F32)
    hipLaunchKernelGGL(k_quantize_nvfp4<SRC_F32>, gd, dim3(256), 0, stream, w_bf16, groups, (uint32_t*)packed,
                       (uint8_t*)scale_ue4m3);
  else if (src_dtype == DGM_SRC_F16)
    hipLaunchKernelGGL(k_quantize_nvfp4<SRC_F16>, gd, dim3(256), 0, stream, w_bf16, groups, (uint32_t*)packed,
                       (uint8_t*)scale_ue4m3);
  else
    hipLaunchKernelGGL(k_quantize_nvfp4<SRC_BF16>, gd, dim3(256), 0, stream, w_bf16, groups, (uint32_t*)packed,
                       (uint8_t*)scale_ue4m3);
  return dgm_last_launch_status();
}

}  // extern "C"

// The QoQ packer over a source of src_dtype: s2 / z / s1 planes, or (plane non-null) the int32
// coefficient plane of the split path's int4 form.
static int quantize_qoq_any(const void* w, int src_dtype, int64_t rows, int64_t K, void* packed, void* s2, void* z,
                            void* s1, void* plane, hipStream_t stream) {
  DGM_CHECK_ARG(src_dtype >= DGM_SRC_BF16 && src_dtype <= DGM_SRC_F32, "src_dtype 0 bf16, 1 fp16, 2 fp32");
  DGM_CHECK_ARG(rows >= 0 && K > 0 && K % 128 == 0, "K must be a positive multiple of 128");
  if (rows == 0) return 0;
  const dim3 gd(grid_for(rows, 4));
#define DGM_QOQ(SRC)                                                                                             \
  hipLaunchKernelGGL(k_quantize_qoq<SRC>, gd, dim3(256), 0, stream, w, rows, (int)K, (uint8_t*)packed, (uint8_t*)s2, \
                     (uint8_t*)z, (float*)s1, (uint32_t*)plane)
  if (src_dtype == DGM_SRC_F32) DGM_QOQ(SRC_F32);
  else if (src_dtype == DGM_SRC_F16) DGM_QOQ(SRC_F16);
  else DGM_QOQ(SRC_BF16);
#undef DGM_QOQ
  return dgm_last_launch_status();
}

extern "C" {

int dgm_quantize_qoq(const void* w_bf16, int64_t rows, int64_t K, void* packed, void* s2, void* z,
                     void* s1_f32, hipStream_t stream) {
  return dgm_quantize_qoq_typed(w_bf16, DGM_SRC_BF16, rows, K, packed, s2, z, s1_f32, stream);
}

int dgm_quantize_qoq_typed(const void* w_bf16, int src_dtype, int64_t rows, int64_t K, void* packed, void* s2,
                           void* z, void* s1_f32, hipStream_t stream) {
  DGM_CHECK_ARG(w_bf16 && packed && s2 && z && s1_f32, "null pointer");
  return quantize_qoq_any(w_bf16, src_dtype, rows, K, packed, s2, z, s1_f32, nullptr, stream);
}

int dgm_quantize_qoq_int4(const void* w_bf16, int64_t rows, int64_t K, void* packed, void* plane_i32,
                          hipStream_t stream) {
  return dgm_quantize_qoq_int4_typed(w_bf16, DGM_SRC_BF16, rows, K, packed, plane_i32, stream);
}

int dgm_quantize_qoq_int4_typed(const void* w_bf16, int src_dtype, int64_t rows, int64_t K, void* packed,
                                void* plane_i32, hipStream_t stream) {
  DGM_CHECK_ARG(w_bf16 && packed && plane_i32, "null pointer");
  return quantize_qoq_any(w_bf16, src_dtype, rows, K, packed, nullptr, nullptr, nullptr, plane_i32, stream);
}

int dgm_cast_int8_rows(const void* x_bf16, int64_t rows, int64_t K, void* q_i8, void* sf_f32,
                       hipStream_t stream) {
  DGM_CHECK_ARG(x_bf16 && q_i8 && sf_f32, "null pointer");
  DGM_CHECK_ARG(rows >= 0 && K > 0, "bad shape");
  if (rows == 0) return 0;
  hipLaunchKernelGGL(k_cast_int8_rows, dim3(grid_for(rows, 4)), dim3(256), 0, stream,
                     (const uint16_t*)x_bf16, rows, (int)K, (int8_t*)q_i8, (float*)sf_f32);
  return dgm_last_launch_status();
}

int dgm_transform_fp4_weights(const void* packed, const void* scale_e8m0, int E, int N, int K,
                              int src_order, int l1_interleave, void* dst_values, void* dst_scales,
                              hipStream_t stream) {
  DGM_CHECK_ARG(packed && scale_e8m0 && dst_values && dst_scales, "null pointer");
  DGM_CHECK_ARG(E > 0 && N > 0 && K > 0 && N % 32 == 0 && K % 128 == 0, "N % 32, K % 128");
  DGM_CHECK_ARG(src_order == 0 || src_order == 1, "src_order 0 = Marlin, 1 = low-nibble-first");
  DGM_CHECK_ARG(l1_interleave >= 0 && l1_interleave <= 2, "l1_interleave 0, 1 or 2");
  DGM_CHECK_ARG(((uintptr_t)packed & 15) == 0 && ((uintptr_t)dst_values & 15) == 0, "16-byte alignment");
  int KT = K / 128, NB = N / 16, KG = (KT + 3) / 4;
  int64_t total = (int64_t)E * NB * KT * 64;
  hipLaunchKernelGGL(k_transform_fp4, dim3(grid_for(total, 256)), dim3(256), 0, stream,
                     (const uint8_t*)packed, (const uint8_t*)scale_e8m0, E, N, K, src_order,
                     l1_interleave, (uint8_t*)dst_values, (uint8_t*)dst_scales);
  int st = dgm_last_launch_status();
  if (st) return st;
  int64_t pad_total = (int64_t)E * NB * 64 * (KG * 4 - KT);
  if (pad_total > 0)
    hipLaunchKernelGGL(k_fill_scale_pad, dim3(grid_for(pad_total, 256)), dim3(256), 0, stream,
                       (uint8_t*)dst_scales, (int64_t)E * NB, KT, KG);
  return dgm_last_launch_status();
}

int dgm_transform_nvfp4_weights(const void* packed, const void* scale_e4m3, int E, int N, int K, int src_order,
                                int l1_interleave, void* dst_values, void* dst_scales, hipStream_t stream) {
  DGM_CHECK_ARG(packed && scale_e4m3 && dst_values && dst_scales, "null pointer");
  DGM_CHECK_ARG(E > 0 && N > 0 && K > 0 && N % 32 == 0 && K % 128 == 0, "N % 32, K % 128");
  DGM_CHECK_ARG(src_order == 0 || src_order == 1, "src_order 0 = Marlin, 1 = low-nibble-first");
  DGM_CHECK_ARG(l1_interleave >= 0 && l1_interleave <= 2, "l1_interleave 0, 1 or 2");
  DGM_CHECK_ARG(((uintptr_t)packed & 3) == 0 && ((uintptr_t)dst_values & 15) == 0 && ((uintptr_t)dst_scales & 3) == 0,
                "alignment");
  const int64_t total = (int64_t)E * (N / 16) * (K / 128) * 64;
  hipLaunchKernelGGL(k_transform_nvfp4, dim3(grid_for(total, 256)), dim3(256), 0, stream, (const uint8_t*)packed,
                     (const uint8_t*)scale_e4m3, E, N, K, src_order, l1_interleave, (uint8_t*)dst_values,
                     (uint8_t*)dst_scales);
  return dgm_last_launch_status();
}

int dgm_reorder_fp4_nibbles(const void* src, void* dst, int64_t n_bytes, int src_order, int dst_order,
                            hipStream_t stream) {
  DGM_CHECK_ARG(src && dst, "null pointer");
  DGM_CHECK_ARG(n_bytes >= 0 && n_bytes % 4 == 0, "n_bytes % 4 == 0 (8 codes per word)");
  DGM_CHECK_ARG((src_order == 0 || src_order == 1) && (dst_order == 0 || dst_order == 1),
                "order 0 = Marlin, 1 = low-nibble-first");
  DGM_CHECK_ARG(((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0, "16-byte alignment");
  const uint8_t* s8 = (const uint8_t*)src;
  uint8_t* d8 = (uint8_t*)dst;
  DGM_CHECK_ARG(s8 == d8 || s8 + n_bytes <= d8 || d8 + n_bytes <= s8, "src and dst overlap partially");
  if (n_bytes == 0) return 0;
  const int64_t words = n_bytes / 4;
  hipLaunchKernelGGL(k_reorder_fp4, dim3(grid_for((words + 3) / 4, 256)), dim3(256), 0, stream, s8, d8, words,
                     src_order, dst_order);
  return dgm_last_launch_status();
}

int dgm_untransform_fp4_weights(const void* values, const void* scales, int E, int N, int K, int dst_order,
                                int l1_interleave, void* packed, void* scale_e8m0, hipStream_t stream) {
  DGM_CHECK_ARG(values && scales && packed && scale_e8m0, "null pointer");
  DGM_CHECK_ARG(E > 0 && N > 0 && K > 0 && N % 32 == 0 && K % 128 == 0, "N % 32, K % 128");
  DGM_CHECK_ARG(dst_order == 0 || dst_order == 1, "dst_order 0 = Marlin, 1 = low-nibble-first");
  DGM_CHECK_ARG(l1_interleave >= 0 && l1_interleave <= 2, "l1_interleave 0, 1 or 2");
  DGM_CHECK_ARG(((uintptr_t)values & 15) == 0 && ((uintptr_t)packed & 15) == 0, "16-byte alignment");
  const int64_t total = (int64_t)E * (N / 16) * (K / 128) * 64;
  hipLaunchKernelGGL(k_untransform_fp4, dim3(grid_for(total, 256)), dim3(256), 0, stream, (const uint8_t*)values,
                     (const uint8_t*)scales, E, N, K, dst_order, l1_interleave, (uint8_t*)packed,
                     (uint8_t*)scale_e8m0);
  return dgm_last_launch_status();
}

int dgm_untransform_nvfp4_weights(const void* values, const void* scales, int E, int N, int K, int dst_order,
                                  int l1_interleave, void* packed, void* scale_e4m3, hipStream_t stream) {
  DGM_CHECK_ARG(values && scales && packed && scale_e4m3, "null pointer");
  DGM_CHECK_ARG(E > 0 && N > 0 && K > 0 && N % 32 == 0 && K % 128 == 0, "N % 32, K % 128");
  DGM_CHECK_ARG(dst_order == 0 || dst_order == 1, "dst_order 0 = Marlin, 1 = low-nibble-first");
  DGM_CHECK_ARG(l1_interleave >= 0 && l1_interleave <= 2, "l1_interleave 0, 1 or 2");
  DGM_CHECK_ARG(((uintptr_t)values & 15) == 0 && ((uintptr_t)scales & 3) == 0 && ((uintptr_t)packed & 3) == 0,
                "alignment");
  const int64_t total = (int64_t)E * (N / 16) * (K / 128) * 64;
  hipLaunchKernelGGL(k_untransform_nvfp4, dim3(grid_for(total, 256)), dim3(256), 0, stream, (const uint8_t*)values,
                     (const uint8_t*)scales, E, N, K, dst_order, l1_interleave, (uint8_t*)packed,
                     (uint8_t*)scale_e4m3);
  return dgm_last_launch_status();
}

int dgm_transform_qoq_weights(const void* packed, const void* s2, const void* z, const void* s1, int E, int N,
                              int K, int l1_interleave, void* dst_values, void* dst_meta, void* dst_s1,
                              hipStream_t stream) {
  DGM_CHECK_ARG(packed && s2 && z && s1 && dst_values && dst_meta && dst_s1, "null pointer");
  DGM_CHECK_ARG(E > 0 && N > 0 && K > 0 && N % 16 == 0 && K % 128 == 0, "E, N, K (N % 16, K % 128)");
  DGM_CHECK_ARG(!l1_interleave || N % 32 == 0, "l1_interleave needs N % 32 == 0");
  DGM_CHECK_ARG(l1_interleave >= 0 && l1_interleave <= 2, "l1_interleave 0, 1 or 2");
  const int64_t total = (int64_t)E * (N / 16) * (K / 128) * 64;
  hipLaunchKernelGGL(k_transform_qoq, dim3(grid_for(total, 256)), dim3(256), 0, stream, (const uint8_t*)packed,
                     (const uint8_t*)s2, (const uint8_t*)z, (const float*)s1, (const uint32_t*)nullptr, E, N, K,
                     l1_interleave, (uint8_t*)dst_values, (uint8_t*)dst_meta, (float*)dst_s1);
  return dgm_last_launch_status();
}

int dgm_transform_qoq_int4_weights(const void* packed, const void* plane_i32, int E, int N, int K, int l1_interleave,
                                   void* dst_values, void* dst_meta, void* dst_s1, hipStream_t stream) {
  DGM_CHECK_ARG(packed && plane_i32 && dst_values && dst_meta && dst_s1, "null pointer");
  DGM_CHECK_ARG(E > 0 && N > 0 && K > 0 && N % 16 == 0 && K % 128 == 0, "E, N, K (N % 16, K % 128)");
  DGM_CHECK_ARG(!l1_interleave || N % 32 == 0, "l1_interleave needs N % 32 == 0");
  DGM_CHECK_ARG(l1_interleave >= 0 && l1_interleave <= 2, "l1_interleave 0, 1 or 2");
  const int64_t total = (int64_t)E * (N / 16) * (K / 128) * 64;
  hipLaunchKernelGGL(k_transform_qoq, dim3(grid_for(total, 256)), dim3(256), 0, stream, (const uint8_t*)packed,
                     (const uint8_t*)nullptr, (const uint8_t*)nullptr, (const float*)nullptr,
                     (const uint32_t*)plane_i32, E, N, K, l1_interleave, (uint8_t*)dst_values, (uint8_t*)dst_meta,
                     (float*)dst_s1);
  return dgm_last_launch_status();
}

}  // extern "C"
