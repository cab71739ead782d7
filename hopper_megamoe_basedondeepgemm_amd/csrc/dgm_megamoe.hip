// MegaMoE layer kernels for MI355X (gfx950): router/top-k frontend, dispatch, L1 and L2
// grouped block-scaled GEMMs on the matrix cores, and the top-k combine.
//
// Data layout in HBM (one GPU's share of the EP layer):
//  * weights: matrix-core fragment order written by dgm_transform_fp4_weights. A 16-row x
//    128-K tile is 1 KB and lane l of a wave loads bytes [16 l, 16 l + 16) of it with one
//    16-byte load: the whole wave reads the tile as one contiguous 1 KB run. Per-32 E8M0
//    scales of 4 consecutive K-tiles sit in one dword per lane.
//  * activations x: [tokens, H/2] E2M1 (low nibble = even K) or [tokens, H] E4M3, scales
//    [tokens, H/32]. Routed rows are read in place through the pool table (on one GPU the
//    per-expert pool is the list of routes; no row copies).
//  * intermediate (L1 -> L2): [pool row, I/2 | I] codes + [pool row, I/32] scales, pool rows
//    in (expert asc, token asc, slot asc) order.
//  * route outputs: fp32 [token * topk + slot, H]; the combine sums valid slots in slot order.
//
// Matrix-core use: swap-AB. The weight tile is the 16-row A operand, up to 16 routed tokens
// form the narrow B operand (one 16-token slab), V_MFMA_SCALE_F32_16X16X128_F8F6F4 applies
// the E8M0 block scales of both operands in hardware (no dequantisation on the VALU).
#include "dgm_common.hpp"
#include "dgm_abi_internal.hpp"
#include "dgm_fused.hpp"
#include "dgm_frontend.hpp"

using namespace dgm;

namespace {

struct alignas(16) U4 { uint32_t x, y, z, w; };

DGM_DEV v8i u4_to_v8i(U4 a) { v8i r = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0}; return r; }
DGM_DEV v8i u8_to_v8i(U4 a, U4 b) {
  v8i r = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
  return r;
}

// ------------------------------------------------------------------ pool table
struct Pool {
  int* meta;      // [0] n_active, [1] total routes
  int* counts;    // [E_local]
  int* active;    // [n_active] local expert ids, ascending
  int* offsets;   // [n_active + 1] first pool row of each active expert
  int* routes;    // [total] route id (token * topk + slot) of each pool row
};

__host__ __device__ inline size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }

__host__ __device__ inline Pool pool_view(uint8_t* base, int E_local) {
  Pool p;
  p.meta = (int*)base;
  p.counts = (int*)(base + 256);
  p.active = (int*)(base + 256 + a256((size_t)E_local * 4));
  p.offsets = (int*)(base + 256 + 2 * a256((size_t)E_local * 4));
  p.routes = (int*)(base + 256 + 2 * a256((size_t)E_local * 4) + a256((size_t)(E_local + 1) * 4));
  return p;
}

// ------------------------------------------------------------------ frontend
// Router rows of the grid (by < ceil(M / RTOK)): workgroup (bx, by) computes the logits and
// top-k keys of experts 4 bx .. +3 for tokens RTOK by .. +RTOK - 1 (fixed accumulation order,
// bit-reproducible fp32 logits; zero keys for an all-zero row when zero_unrouted): RT = 0, one
// wave per expert over 4 tokens (router_wave, RTOK = 4); RT > 0, the RT tokens' hidden rows
// staged in LDS and shared by the four waves (router_tile, RTOK = RT; the same bits). Cast rows
// (the rest of the grid, running beside the router rows rather than after them): MXFP4 / MXFP8
// 8 lanes per 32-element group, NVFP4 4 lanes per 16-element group, QoQ one wave per token
// (dgm_frontend.hpp).
// Tiled router rows from 64 tokens on (MI355X, E384 H3072, kernel + launch by events: 64 tokens
// 13.7 us against 15.2, 128 tokens 24.0 against 26.8; at 16 and 32 tokens the LDS staging and
// its barrier cost 1.1-1.7 us more than the hidden-row reads they save).
constexpr int FE_ROUTER_TILE = 8;         // tokens per router workgroup in the tiled form
constexpr int FE_TILE_MIN_TOKENS = 64;
// Phase stamps (the reference's DG_FE_STAMPS, deep_gemm/mega/__init__.py:743-756): with stamps
// non-null, workgroup b = blockIdx.y * gridDim.x + blockIdx.x < stamp_rows writes row b of 8
// int64: [0] entry, [3] (router rows) keys and logits stored by all four waves, [5] (cast rows)
// cast stored, [6] the hardware position (HW_ID | XCC_ID << 32), [7] exit; wall clock at 100 MHz.
DGM_DEV long long fe_clock() { return (long long)__builtin_amdgcn_s_memrealtime(); }
DGM_DEV long long fe_hw_position() {
  uint32_t hw, xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  return (long long)hw | ((long long)(xcc & 0xffffu) << 32);
}

template <int J, int RT>
__global__ void __launch_bounds__(256) k_frontend(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                  int M, int E, int act_format, float* __restrict__ logits,
                                                  uint32_t* __restrict__ keys, int zero_unrouted,
                                                  uint8_t* __restrict__ q, uint8_t* __restrict__ sf, int router,
                                                  long long* __restrict__ stamps, int stamp_rows) {
  constexpr int H = J * 512, RTOK = RT > 0 ? RT : 4;
  __shared__ uint4 xs[RT > 0 ? RT * J * 64 : 1];
  // every argument (and the grid size) requested at entry behind one wait: left to the compiler,
  // the loads came in four dependent rounds, two of them misses on the two argument lines
  // (0.16-0.36 us of this kernel at 2-8 tokens)
  asm volatile("" ::"s"(x), "s"(w), "s"(M), "s"(E), "s"(act_format), "s"(logits), "s"(keys), "s"(zero_unrouted),
               "s"(q), "s"(sf), "s"(router), "s"(stamps), "s"(stamp_rows), "s"(gridDim.x), "s"(gridDim.y));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ry = router ? (M + RTOK - 1) / RTOK : 0;
  const int brow = (int)(blockIdx.y * gridDim.x + blockIdx.x);
  long long* st = stamps != nullptr && brow < stamp_rows ? stamps + (size_t)brow * 8 : nullptr;
  const long long t_entry = st ? fe_clock() : 0;
  if ((int)blockIdx.y < ry) {
    if constexpr (RT > 0)
      router_tile<J, RT, false>(x, w, M, E, blockIdx.x * 4, blockIdx.y * RT, logits, keys, zero_unrouted != 0, xs);
    else
      router_wave<J, false>(x, w, M, E, blockIdx.x * 4 + wave, blockIdx.y * 4, lane, logits, keys, zero_unrouted != 0);
    if (st) {
      __syncthreads();
      if (tid == 0) {
        const long long t = fe_clock();
        st[0] = t_entry; st[1] = 0; st[2] = 0; st[3] = t; st[4] = 0; st[5] = 0;
        st[6] = fe_hw_position(); st[7] = fe_clock();
      }
    }
    return;
  }
  const int cy = (int)gridDim.y - ry, by = (int)blockIdx.y - ry;
  const int64_t lane0 = ((int64_t)by * gridDim.x + blockIdx.x) * 256 + tid;
  const int64_t nl = (int64_t)gridDim.x * cy * 256;
  if (act_format == DGM_ACT_QOQ) {
    const int nwaves = gridDim.x * cy * 4;
    for (int t = (by * (int)gridDim.x + (int)blockIdx.x) * 4 + wave; t < M; t += nwaves)
      cast_qoq_token<J, false>(x, t, lane, q, sf);
  } else if (act_format == DGM_ACT_NVFP4) {
    for (int64_t i = lane0; i < (int64_t)M * (H / 16) * 4; i += nl) cast_lane_nvfp4<false>(x, i, q, sf);
  } else if (act_format == DGM_ACT_FP8F128) {
    for (int64_t i = lane0; i < (int64_t)M * (H / 128) * 32; i += nl) cast_lane_fp8f128<false>(x, i, q, sf);
  } else {
    for (int64_t i = lane0; i < (int64_t)M * (H / 32) * 8; i += nl) cast_lane_mx<false>(x, act_format, i, q, sf);
  }
  if (st) {
    __syncthreads();
    if (tid == 0) {
      const long long t = fe_clock();
      st[0] = t_entry; st[1] = 0; st[2] = 0; st[3] = 0; st[4] = 0; st[5] = t;
      st[6] = fe_hw_position(); st[7] = fe_clock();
    }
  }
}

// ------------------------------------------------------------------ top-k + softmax
// One wave per token over its key row (orderable(bf16(logit)) << 16 | (0xFFFF - e), -0 -> +0):
// k rounds of a wave-wide max select; softmax w_k = exp(v_k - v_0) / sum (sequential sum).
// Unrouted tokens (a zero first key) get idx -1 / weight 0; forced-balanced routing
// (DGM_FE_FORCE_BALANCED) gives slot s -> s G + (g + 7 s) % G with weight 1 / topk.
constexpr int SELECT_TPB = 4;           // tokens (waves) per workgroup
__global__ void __launch_bounds__(256) k_select(const uint32_t* __restrict__ keys, int M, int E, int topk, int flags,
                                                int token_offset, int64_t* __restrict__ topk_idx,
                                                float* __restrict__ topk_w) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * SELECT_TPB + (threadIdx.x >> 6);
  if (t >= M) return;
  int idx = -1;
  float wt = 0.f;
  const uint32_t* row = keys + (size_t)t * E;
  select_topk_wave([row](int e) { return row[e]; }, E, topk, (flags & DGM_FE_FORCE_BALANCED) != 0,
                   token_offset + t, lane, idx, wt);
  // (DGM_FE_RAW_WEIGHTS: the selected logit itself, no softmax)
  if ((flags & DGM_FE_RAW_WEIGHTS) && !(flags & DGM_FE_FORCE_BALANCED) && lane < topk && idx >= 0) wt = key_value(row[idx]);
  if (lane < topk) {
    topk_idx[(size_t)t * topk + lane] = idx;
    topk_w[(size_t)t * topk + lane] = wt;
  }
}

// Top-k keys of bf16 router logits [M, E] (the frontend's key of each logit, topk_key).
__global__ void __launch_bounds__(256) k_keys_bf16(const uint16_t* __restrict__ logits, int64_t n, int E,
                                                   uint32_t* __restrict__ keys) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  keys[i] = topk_key(bf16_to_f32(logits[i]), (int)(i % E));
}

// ------------------------------------------------------------------ dispatch
// One workgroup: per-expert counts, canonical pool order (token asc, slot asc) by rank of
// the route id among the routes of its expert, exclusive scans over experts, stats update.
constexpr int DISPATCH_THREADS = 1024;
constexpr int MAX_ROUTES_DISPATCH = 4096;
constexpr int MAX_LOCAL_EXPERTS = 1024;

__global__ void __launch_bounds__(DISPATCH_THREADS) k_dispatch(const int64_t* __restrict__ topk_idx, int routes_n,
                                                               int expert_begin, int E_local,
                                                               uint8_t* __restrict__ pool_base,
                                                               int* __restrict__ recv_stats) {
  __shared__ int s_exp[MAX_ROUTES_DISPATCH];
  __shared__ int s_cnt[MAX_LOCAL_EXPERTS];
  __shared__ int s_off[MAX_LOCAL_EXPERTS];
  __shared__ int s_act[MAX_LOCAL_EXPERTS];
  __shared__ int s_wave[DISPATCH_THREADS / 64][2];
  Pool P = pool_view(pool_base, E_local);
  const int tid = threadIdx.x;
  for (int e = tid; e < E_local; e += DISPATCH_THREADS) s_cnt[e] = 0;
  for (int r = tid; r < routes_n; r += DISPATCH_THREADS) {
    int64_t g = topk_idx[r];
    int64_t l = g - expert_begin;
    s_exp[r] = (g >= 0 && l >= 0 && l < E_local) ? (int)l : -1;
  }
  __syncthreads();
  for (int r = tid; r < routes_n; r += DISPATCH_THREADS)
    if (s_exp[r] >= 0) atomicAdd(&s_cnt[s_exp[r]], 1);
  __syncthreads();
  // exclusive scans of counts and of the active flags over experts (E_local <= 1024)
  int c = 0, a = 0;
  if (tid < E_local) { c = s_cnt[tid]; a = c > 0 ? 1 : 0; }
  int lane = tid & 63, wv = tid >> 6;
  int ic = c, ia = a;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int oc = __shfl_up(ic, off), oa = __shfl_up(ia, off);
    if (lane >= off) { ic += oc; ia += oa; }
  }
  if (lane == 63) { s_wave[wv][0] = ic; s_wave[wv][1] = ia; }
  __syncthreads();
  int bc = 0, ba = 0;
  for (int i = 0; i < wv; ++i) { bc += s_wave[i][0]; ba += s_wave[i][1]; }
  int exc = bc + ic - c, exa = ba + ia - a;
  if (tid < E_local) {
    s_off[tid] = exc;
    P.counts[tid] = c;
    if (a) { s_act[exa] = tid; P.active[exa] = tid; P.offsets[exa] = exc; }
    if (recv_stats) recv_stats[tid] += c;
  }
  __syncthreads();
  if (tid == 0) {
    int tot = 0, na = 0;
    for (int i = 0; i < DISPATCH_THREADS / 64; ++i) { tot += s_wave[i][0]; na += s_wave[i][1]; }
    P.meta[0] = na;
    P.meta[1] = tot;
    P.offsets[na] = tot;
  }
  for (int r = tid; r < routes_n; r += DISPATCH_THREADS) {
    int e = s_exp[r];
    if (e < 0) continue;
    int rank = 0;
    for (int q = 0; q < r; ++q) rank += (s_exp[q] == e) ? 1 : 0;
    P.routes[s_off[e] + rank] = r;
  }
}

// ------------------------------------------------------------------ L1: gate/up + SwiGLU + requant
// Workgroup = NWV waves; item = (active expert a, 16 NWV intermediate features q). Wave w owns
// the (gate, up) block pair p = NWV q + w (16 features). Both weight tiles of every K-tile are
// loaded into registers up front (one 1 KB coalesced run per tile), the 16-token B slab is
// staged once per workgroup in LDS in fragment order, then 2 * KT matrix-core ops run.
// Epilogue: clamp, silu(g)*u*w, requant of the item's features across its waves.
// MXFP4 / MXFP8 (2 waves): gate/up rounded to bf16, per-32 E8M0 requant.
// FP8F128 (4 waves): the activation's fp32 scale of each (token, K-tile) multiplies that
// K-tile's product (the op runs with a unit activation scale into a zero accumulator, then
// acc += s * part), fp32 gate/up, per-64 power-of-two FP8 requant stored as two equal per-32
// E8M0 bytes (so the MXFP8 L2 reads it).
template <int ACT> constexpr int l1_waves() { return ACT == DGM_ACT_FP8F128 ? 4 : 2; }

template <int KT, int ACT>
struct L1Smem {
  static constexpr int BYTES = ACT == DGM_ACT_MXFP4 ? 16 : 32;
  static constexpr int KG = (KT + 3) / 4;
  U4 b[KT][64][BYTES / 16];
  uint32_t bs[KG][64];
  float bsf[ACT == DGM_ACT_FP8F128 ? KT : 1][16];    // FP8F128: per (K-tile, slab column) scale
  float amax[l1_waves<ACT>()][16];
};

template <int KT, int ACT>
__global__ void __launch_bounds__(64 * l1_waves<ACT>()) k_l1(const uint8_t* __restrict__ w1v,
                                                           const uint32_t* __restrict__ w1s,
                                                           const uint8_t* __restrict__ x, const uint8_t* __restrict__ xsf,
                                                           const float* __restrict__ topk_w, uint8_t* __restrict__ pool_base,
                                                           int E_local, int I, int topk, float clamp, int fast_math,
                                                           uint8_t* __restrict__ mid, uint8_t* __restrict__ mid_sf) {
  constexpr int NWV = l1_waves<ACT>(), NT = 64 * NWV;
  constexpr bool F128 = ACT == DGM_ACT_FP8F128;
  constexpr int KG = (KT + 3) / 4;
  constexpr int XB = ACT == DGM_ACT_MXFP4 ? KT * 64 : KT * 128;   // x row bytes (H/2 or H)
  constexpr int H = KT * 128;
  __shared__ L1Smem<KT, ACT> sm;
  Pool P = pool_view(pool_base, E_local);
  const int n_active = P.meta[0];
  const int QN = I / (16 * NWV);
  const int NB1 = I / 8;            // 16-row blocks of the 2I-row L1 weight
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int midb = ACT == DGM_ACT_MXFP4 ? I / 2 : I;
  const int items = n_active * QN;
  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    const int a = item / QN, q = item % QN;
    const int e = P.active[a];
    const int r0 = P.offsets[a], n = P.offsets[a + 1] - r0;
    const int p = NWV * q + wv;
    // ---- A operands: gate tile (block 2p) and up tile (block 2p+1) for every K-tile
    const uint8_t* gbase = w1v + ((size_t)(e * NB1 + 2 * p) * KT) * 1024 + lane * 16;
    const uint8_t* ubase = gbase + (size_t)KT * 1024;
    U4 ag[KT], au[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      ag[kt] = *reinterpret_cast<const U4*>(gbase + kt * 1024);
      au[kt] = *reinterpret_cast<const U4*>(ubase + kt * 1024);
    }
    uint32_t sg[KG], su[KG];
    const uint32_t* gs = w1s + ((size_t)(e * NB1 + 2 * p) * KG) * 64 + lane;
#pragma unroll
    for (int g = 0; g < KG; ++g) { sg[g] = gs[g * 64]; su[g] = gs[(KG + g) * 64]; }

    for (int s0 = 0; s0 < n; s0 += 16) {
      // ---- stage the B slab (routes s0..s0+15 of this expert) in fragment order
      __syncthreads();
      for (int f = threadIdx.x; f < KT * 64; f += NT) {
        int kt = f >> 6, l = f & 63, c = l & 15;
        U4 v0 = {0, 0, 0, 0}, v1 = {0, 0, 0, 0};
        if (s0 + c < n) {
          int t = P.routes[r0 + s0 + c] / topk;
          if (ACT == DGM_ACT_MXFP4) {
            v0 = *reinterpret_cast<const U4*>(x + (size_t)t * XB + kt * 64 + (l >> 4) * 16);
          } else {
            // E4M3 operand: lane group g holds K = 16 g .. +16 (bytes 0-15) and
            // K = 64 + 16 g .. +16 (bytes 16-31) of the 128-wide K-tile.
            const uint8_t* src = x + (size_t)t * XB + kt * 128 + (l >> 4) * 16;
            v0 = *reinterpret_cast<const U4*>(src);
            v1 = *reinterpret_cast<const U4*>(src + 64);
          }
        }
        sm.b[kt][l][0] = v0;
        if (ACT != DGM_ACT_MXFP4) sm.b[kt][l][ACT != DGM_ACT_MXFP4 ? 1 : 0] = v1;
      }
      for (int f = threadIdx.x; f < KG * 64; f += NT) {
        int g = f >> 6, l = f & 63, c = l & 15;
        uint32_t w = 0x7f7f7f7fu;
        if (!F128 && s0 + c < n) {
          int t = P.routes[r0 + s0 + c] / topk;
          w = 0;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            int kt = 4 * g + j;
            uint32_t b = kt < KT ? xsf[(size_t)t * (H / 32) + kt * 4 + (l >> 4)] : 127u;
            w |= b << (8 * j);
          }
        }
        sm.bs[g][l] = w;
      }
      if constexpr (F128) {
        for (int f = threadIdx.x; f < KT * 16; f += NT) {
          const int kt = f >> 4, c = f & 15;
          float v = 0.f;
          if (s0 + c < n) v = reinterpret_cast<const float*>(xsf)[(size_t)(P.routes[r0 + s0 + c] / topk) * KT + kt];
          sm.bsf[kt][c] = v;
        }
      }
      __syncthreads();
      // ---- matrix cores. Scale bytes are selected from the loaded scale dwords by the op's
      // byte select (no VALU writes to a scale operand inside the chain of matrix-core ops)
      v4f accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
      v4f accg1 = {0.f, 0.f, 0.f, 0.f}, accu1 = {0.f, 0.f, 0.f, 0.f};
      uint32_t bsw[KG];
#pragma unroll
      for (int g = 0; g < KG; ++g) bsw[g] = sm.bs[g][lane];
      const int c = lane & 15;
      static_for<KT>([&](auto kc) {
        constexpr int kt = decltype(kc)::value;
        v8i bop;
        if (ACT == DGM_ACT_MXFP4) bop = u4_to_v8i(sm.b[kt][lane][0]);
        else bop = u8_to_v8i(sm.b[kt][lane][0], sm.b[kt][lane][ACT != DGM_ACT_MXFP4 ? 1 : 0]);
        constexpr int FB = ACT == DGM_ACT_MXFP4 ? 4 : 0;
        constexpr int SEL = kt & 3;
        if constexpr (F128) {
          // this K-tile's products with a unit activation scale, promoted by the token's scale
          const v4f z = {0.f, 0.f, 0.f, 0.f};
          const v4f tg = mfma_scale_16x16x128_sel<4, FB, SEL, SEL>(u4_to_v8i(ag[kt]), bop, z, (int)sg[kt >> 2], (int)bsw[kt >> 2]);
          const v4f tu = mfma_scale_16x16x128_sel<4, FB, SEL, SEL>(u4_to_v8i(au[kt]), bop, z, (int)su[kt >> 2], (int)bsw[kt >> 2]);
          const float sx = sm.bsf[kt][c];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            accg[i] = fmaf(sx, tg[i], accg[i]);
            accu[i] = fmaf(sx, tu[i], accu[i]);
          }
        } else if constexpr (kt < KT / 2) {
          accg = mfma_scale_16x16x128_sel<4, FB, SEL, SEL>(u4_to_v8i(ag[kt]), bop, accg, (int)sg[kt >> 2], (int)bsw[kt >> 2]);
          accu = mfma_scale_16x16x128_sel<4, FB, SEL, SEL>(u4_to_v8i(au[kt]), bop, accu, (int)su[kt >> 2], (int)bsw[kt >> 2]);
        } else {
          accg1 = mfma_scale_16x16x128_sel<4, FB, SEL, SEL>(u4_to_v8i(ag[kt]), bop, accg1, (int)sg[kt >> 2], (int)bsw[kt >> 2]);
          accu1 = mfma_scale_16x16x128_sel<4, FB, SEL, SEL>(u4_to_v8i(au[kt]), bop, accu1, (int)su[kt >> 2], (int)bsw[kt >> 2]);
        }
      });
      if constexpr (F128) {
        keep_scales_until(sg, accg);
        keep_scales_until(su, accu);
        keep_scales_until(bsw, accg);
        keep_scales_until(bsw, accu);
      } else {
        keep_scales_until(sg, accg1);
        keep_scales_until(su, accu1);
        keep_scales_until(bsw, accg1);
        keep_scales_until(bsw, accu1);
        accg += accg1;
        accu += accu1;
      }
      // ---- epilogue: lane holds features 16p + 4(l/16) + i for slab column c = l % 16
      const bool valid = s0 + c < n;
      float act[4];
      float am = 0.f;
      float wt = 0.f;
      if (valid) wt = topk_w[P.routes[r0 + s0 + c]];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float g = fminf(F128 ? accg[i] : round_bf16(accg[i]), clamp);
        float u = fminf(fmaxf(F128 ? accu[i] : round_bf16(accu[i]), -clamp), clamp);
        float sg1 = fast_math ? sigmoid<true>(g) : sigmoid<false>(g);
        act[i] = valid ? ((g * sg1) * u) * wt : 0.f;
        am = fmaxf(am, fabsf(act[i]));
      }
      am = fmaxf(am, __shfl_xor(am, 16));
      am = fmaxf(am, __shfl_xor(am, 32));
      if (lane < 16) sm.amax[wv][lane] = am;
      __syncthreads();
      am = sm.amax[0][c];
#pragma unroll
      for (int w = 1; w < NWV; ++w) am = fmaxf(am, sm.amax[w][c]);
      if (valid) {
        const int row = r0 + s0 + c;
        const int f0 = 16 * p + 4 * (lane >> 4);
        if (ACT == DGM_ACT_MXFP4) {
          uint32_t code = ceil_ue8m0_code(fmaxf(am, 1e-30f) / 6.0f);
          float is = e8m0_inv(code);
          uint32_t w = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) w |= e2m1_ties_down(act[i] * is) << (4 * i);
          *reinterpret_cast<uint16_t*>(mid + (size_t)row * midb + f0 / 2) = (uint16_t)w;
          if (wv == 0 && lane < 16) mid_sf[(size_t)row * (I / 32) + q] = (uint8_t)code;
        } else {
          // MXFP8: 2^ceil(log2(max(amax, 1e-30) / 448)); FP8F128: 2^ceil(log2(max(amax / 448,
          // FLT_MIN)))
          float ex = F128 ? ceil_log2_f32(fmaxf(am / 448.0f, 1.17549435e-38f))
                          : ceil_log2_f32(fmaxf(am, 1e-30f) / 448.0f);
          int code = (int)ex + 127;
          float is = e8m0_inv((uint32_t)code);
          uint32_t w = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) w |= e4m3_encode(act[i] * is) << (8 * i);
          *reinterpret_cast<uint32_t*>(mid + (size_t)row * midb + f0) = w;
          if (wv == 0 && lane < 16) {
            if (F128) {
              mid_sf[(size_t)row * (I / 32) + 2 * q] = (uint8_t)code;
              mid_sf[(size_t)row * (I / 32) + 2 * q + 1] = (uint8_t)code;
            } else {
              mid_sf[(size_t)row * (I / 32) + q] = (uint8_t)code;
            }
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------------ L2: down projection
// One wave per item (active expert a, 16 output rows b). A: KT2 tiles in registers; B: the
// 16-route slab of intermediate rows read straight from L2-resident memory.
template <int KT, int ACT>
__global__ void __launch_bounds__(256) k_l2(const uint8_t* __restrict__ w2v, const uint32_t* __restrict__ w2s,
                                            const uint8_t* __restrict__ mid, const uint8_t* __restrict__ mid_sf,
                                            uint8_t* __restrict__ pool_base, int E_local, int H, int topk,
                                            int part_rows, uint16_t* __restrict__ partials) {
  constexpr int KG = (KT + 3) / 4;
  constexpr int I = KT * 128;
  constexpr int MB = ACT == DGM_ACT_MXFP4 ? I / 2 : I;
  Pool P = pool_view(pool_base, E_local);
  const int n_active = P.meta[0];
  const int NB2 = H / 16;
  const int lane = threadIdx.x & 63;
  const int items = n_active * NB2;
  const int waves = gridDim.x * 4;
  for (int item = blockIdx.x * 4 + (threadIdx.x >> 6); item < items; item += waves) {
    const int a = item / NB2, b = item % NB2;
    const int e = P.active[a];
    const int r0 = P.offsets[a], n = P.offsets[a + 1] - r0;
    const uint8_t* base = w2v + ((size_t)(e * NB2 + b) * KT) * 1024 + lane * 16;
    U4 av[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) av[kt] = *reinterpret_cast<const U4*>(base + kt * 1024);
    uint32_t sa[KG];
    const uint32_t* sp = w2s + ((size_t)(e * NB2 + b) * KG) * 64 + lane;
#pragma unroll
    for (int g = 0; g < KG; ++g) sa[g] = sp[g * 64];
    const int c = lane & 15, kq = lane >> 4;
    for (int s0 = 0; s0 < n; s0 += 16) {
      const bool valid = s0 + c < n;
      const int row = r0 + s0 + (valid ? c : 0);
      v4f acc = {0.f, 0.f, 0.f, 0.f};
      // the activation scale bytes of every K-tile, loaded before the chain of matrix-core ops
      // into registers of their own (a lane without a route reads its slab's first row: its B
      // operand is zero, and a real scale byte is finite); the weight scale bytes are selected
      // from the loaded dwords by the op's byte select, so no VALU op writes a scale operand
      // inside the chain
      uint32_t sbv[KT];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) sbv[kt] = mid_sf[(size_t)row * (I / 32) + kt * 4 + kq];
      static_for<KT>([&](auto kc) {
        constexpr int kt = decltype(kc)::value;
        v8i bop;
        if (ACT == DGM_ACT_MXFP4) {
          U4 v = {0, 0, 0, 0};
          if (valid) v = *reinterpret_cast<const U4*>(mid + (size_t)row * MB + kt * 64 + kq * 16);
          bop = u4_to_v8i(v);
        } else {
          U4 v0 = {0, 0, 0, 0}, v1 = {0, 0, 0, 0};
          if (valid) {
            const uint8_t* s = mid + (size_t)row * MB + kt * 128 + kq * 16;
            v0 = *reinterpret_cast<const U4*>(s);
            v1 = *reinterpret_cast<const U4*>(s + 64);
          }
          bop = u8_to_v8i(v0, v1);
        }
        constexpr int FB = ACT == DGM_ACT_MXFP4 ? 4 : 0;
        acc = mfma_scale_16x16x128_sel<4, FB, kt & 3, 0>(u4_to_v8i(av[kt]), bop, acc, (int)sa[kt >> 2], (int)sbv[kt]);
      });
      keep_scales_until(sa, acc);
      keep_scales_until(sbv, acc);
      if (valid) {
        // the route's output rounded to bf16, slot-major [topk][part_rows][H]
        const int rid = P.routes[row];
        const int t = rid / topk, sl = rid - t * topk;
        const uint2 o = make_uint2((uint32_t)f32_to_bf16(acc[0]) | ((uint32_t)f32_to_bf16(acc[1]) << 16),
                                   (uint32_t)f32_to_bf16(acc[2]) | ((uint32_t)f32_to_bf16(acc[3]) << 16));
        *reinterpret_cast<uint2*>(partials + ((size_t)sl * part_rows + t) * H + b * 16 + 4 * kq) = o;
      }
    }
  }
}

// ------------------------------------------------------------------ combine
// y[t, n] = bf16(sum over valid local slots s ascending of float(partials[s, t, n])) (bf16 route
// outputs, fp32 sum).
__global__ void k_combine(const uint16_t* __restrict__ partials, int part_rows, const int64_t* __restrict__ topk_idx,
                          int M, int H, int topk, int expert_begin, int E_local, uint16_t* __restrict__ y) {
  const int t = blockIdx.y;
  const int n = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (t >= M || n >= H) return;
  // every local route's values are loaded first (one round trip), then summed in slot order
  // (fp32; a route of another rank adds nothing)
  constexpr int MAXK = 16;                         // (topk <= 16, checked on the host)
  uint2 v[MAXK];
  uint32_t use = 0;
#pragma unroll
  for (int s = 0; s < MAXK; ++s) {
    v[s] = make_uint2(0u, 0u);
    if (s < topk) {
      const int64_t g = topk_idx[(size_t)t * topk + s];
      const int64_t l = g - expert_begin;
      if (g >= 0 && l >= 0 && l < E_local) {
        use |= 1u << s;
        v[s] = *reinterpret_cast<const uint2*>(partials + ((size_t)s * part_rows + t) * H + n);
      }
    }
  }
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
  for (int s = 0; s < MAXK; ++s)
    if ((use >> s) & 1u) {
      s0 += __uint_as_float(v[s].x << 16);
      s1 += __uint_as_float(v[s].x & 0xffff0000u);
      s2 += __uint_as_float(v[s].y << 16);
      s3 += __uint_as_float(v[s].y & 0xffff0000u);
    }
  uint32_t lo = (uint32_t)f32_to_bf16(s0) | ((uint32_t)f32_to_bf16(s1) << 16);
  uint32_t hi = (uint32_t)f32_to_bf16(s2) | ((uint32_t)f32_to_bf16(s3) << 16);
  *reinterpret_cast<uint2*>(y + (size_t)t * H + n) = make_uint2(lo, hi);
}

int g_cu_count = 0;

int cu_count() {
  if (g_cu_count == 0) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess) g_cu_count = prop.multiProcessorCount;
    if (g_cu_count <= 0) g_cu_count = 256;
  }
  return g_cu_count;
}

template <int KT1, int KT2, int ACT>
int launch_experts(const DgmMoeArgs* A, uint8_t* buf, const DgmBufferLayout* L, hipStream_t stream) {
  const int cus = cu_count();
  uint8_t* pool = buf + L->pool;
  int items1 = A->num_local_experts * (A->intermediate / (16 * l1_waves<ACT>()));
  int grid1 = items1 < cus * 4 ? items1 : cus * 4;
  hipLaunchKernelGGL((k_l1<KT1, ACT>), dim3(grid1), dim3(64 * l1_waves<ACT>()), 0, stream, (const uint8_t*)A->w1_values,
                     (const uint32_t*)A->w1_scales, buf + L->x, buf + L->x_sf,
                     (const float*)(buf + L->topk_weights), pool, A->num_local_experts, A->intermediate,
                     A->topk, A->activation_clamp, A->fast_math, buf + L->mid, buf + L->mid_sf);
  int st = dgm_last_launch_status();
  if (st) return st;
  int items2 = A->num_local_experts * (A->hidden / 16);
  int grid2 = (items2 + 3) / 4 < cus * 4 ? (items2 + 3) / 4 : cus * 4;
  // (FP8F128: the intermediate is FP8 with E8M0 bytes per 32, as MXFP8's)
  constexpr int ACT2 = ACT == DGM_ACT_FP8F128 ? DGM_ACT_MXFP8 : ACT;
  hipLaunchKernelGGL((k_l2<KT2, ACT2>), dim3(grid2), dim3(256), 0, stream, (const uint8_t*)A->w2_values,
                     (const uint32_t*)A->w2_scales, buf + L->mid, buf + L->mid_sf, pool, A->num_local_experts,
                     A->hidden, A->topk, L->max_tokens, (uint16_t*)(buf + L->partials));
  return dgm_last_launch_status();
}

}  // namespace

// ==================================================================== C ABI
static thread_local char g_err[512];
void dgm_set_error(const char* msg) {
  strncpy(g_err, msg, sizeof(g_err) - 1);
  g_err[sizeof(g_err) - 1] = 0;
}

static bool fused_fits(const DgmMoeArgs* A);
static int fused_launch_phases(const DgmMoeArgs* A, int phases, hipStream_t stream);

extern "C" {

int dgm_version(void) { return 1; }
const char* dgm_last_error(void) { return g_err; }

int dgm_device_cu_count(void) { return cu_count(); }

int dgm_abi_struct_sizes(size_t* moe_args, size_t* buffer_layout) {
  DGM_CHECK_ARG(moe_args && buffer_layout, "null pointer");
  *moe_args = sizeof(DgmMoeArgs);
  *buffer_layout = sizeof(DgmBufferLayout);
  return 0;
}

int dgm_host_device_pointer(const void* host, void** device) {
  DGM_CHECK_ARG(host && device, "null pointer");
  hipError_t e = hipHostGetDevicePointer(device, const_cast<void*>(host), 0);
  if (e != hipSuccess) {
    dgm_set_error("hipHostGetDevicePointer failed: not pinned host memory");
    return (int)e;
  }
  return 0;
}

int dgm_fused_workgroups(int hidden, int intermediate, int act_format) {
  return dgm_fused_grid_blocks(hidden, intermediate, act_format);
}

int dgm_fused_last_form(int hidden, int intermediate, int act_format) {
  return dgm_fused_form(hidden, intermediate, act_format);
}

int dgm_fused_buffer_layout(int max_tokens, int num_experts, int num_local_experts, int topk,
                            int hidden, int intermediate, int act_format, DgmBufferLayout* out) {
  DGM_CHECK_ARG(out != nullptr, "null layout");
  DGM_CHECK_ARG(max_tokens > 0 && topk > 0 && topk <= 16, "max_tokens > 0, 0 < topk <= 16");
  DGM_CHECK_ARG(num_experts > 0 && num_experts <= 1024, "num_experts in (0, 1024]");
  DGM_CHECK_ARG(num_local_experts > 0 && num_local_experts <= num_experts, "num_local_experts");
  DGM_CHECK_ARG(hidden % 512 == 0 && intermediate % 128 == 0, "hidden % 512, intermediate % 128");
  DGM_CHECK_ARG(act_format >= DGM_ACT_MXFP4 && act_format <= DGM_ACT_FP8F128, "act_format");
  DGM_CHECK_ARG((int64_t)max_tokens * topk <= MAX_ROUTES_DISPATCH, "max_tokens * topk <= 4096");
  // scales: E8M0 bytes per 32 (MXFP); QoQ: fp32 per token repeated over H / 128 slots (the
  // same H / 32 bytes) and fp32 per 64 intermediate features (I / 16 bytes); NVFP4: E4M3
  // bytes per 16; FP8F128: fp32 per 128 K (H / 32 bytes) and E8M0 bytes per 32 intermediate
  // features, sized as QoQ's (so one buffer serves both layers of the split recipe)
  const DgmRowBytes rb = dgm_row_bytes(act_format, hidden, intermediate);
  const size_t xb = rb.x, mb = rb.mid, xsfb = rb.x_sf, msfb = rb.mid_sf;
  const int R = max_tokens * topk;
  size_t off = 0;
  memset(out, 0, sizeof(*out));
  out->x = off; off += dgm_align256((size_t)max_tokens * xb);
  out->x_sf = off; off += dgm_align256((size_t)max_tokens * xsfb);
  out->topk_idx = off; off += dgm_align256((size_t)R * 8);
  out->topk_weights = off; off += dgm_align256((size_t)R * 4);
  out->logits = off; off += dgm_align256((size_t)max_tokens * num_experts * 4);
  out->fe_keys = off; off += dgm_align256((size_t)max_tokens * num_experts * 4);
  out->pool = off; off += dgm_align256(dgm_pool_bytes(num_local_experts, R));
  out->mid = off; off += dgm_align256((size_t)R * mb);
  out->mid_sf = off; off += dgm_align256((size_t)R * msfb);
  out->partials = off; off += dgm_align256((size_t)R * hidden * 2);     // bf16 [topk][max_tokens][H]
  out->counters = off; off += dgm_align256((size_t)CNT_ALL * 4);
  out->total_bytes = off;
  out->x_row_bytes = (int32_t)xb;
  out->mid_row_bytes = (int32_t)mb;
  out->max_routes = R;
  out->max_tokens = max_tokens;
  out->topk = topk;
  out->num_experts = num_experts;
  out->num_local_experts = num_local_experts;
  out->hidden = hidden;
  out->intermediate = intermediate;
  out->act_format = act_format;
  out->x_sf_row_bytes = (int32_t)xsfb;
  out->mid_sf_row_bytes = (int32_t)msfb;
  return 0;
}

}  // extern "C"

int dgm_check_layout_call(const DgmBufferLayout* L, int num_tokens, int topk, int num_experts, int num_local_experts,
                          int hidden, int intermediate, int act_format) {
  DGM_CHECK_ARG(L != nullptr, "null layout");
  DGM_CHECK_ARG(L->max_routes == L->max_tokens * L->topk && L->topk > 0,
                "the layout was not made by dgm_fused_buffer_layout");
  DGM_CHECK_ARG(num_tokens >= 0 && num_tokens <= L->max_tokens, "num_tokens exceeds the buffer's max_tokens");
  DGM_CHECK_ARG(topk > 0 && topk <= L->topk, "topk exceeds the buffer's topk (route outputs are [topk][max_tokens][H])");
  DGM_CHECK_ARG(num_experts > 0 && num_experts <= L->num_experts, "num_experts exceeds the buffer's");
  DGM_CHECK_ARG(num_local_experts < 0 || num_local_experts <= L->num_local_experts,
                "num_local_experts exceeds the buffer's (dispatch table)");
  DGM_CHECK_ARG(hidden == L->hidden, "hidden differs from the buffer's");
  DGM_CHECK_ARG(intermediate < 0 || intermediate == L->intermediate, "intermediate differs from the buffer's");
  const DgmRowBytes rb = dgm_row_bytes(act_format, hidden, intermediate < 0 ? L->intermediate : intermediate);
  DGM_CHECK_ARG(rb.x <= (size_t)L->x_row_bytes && rb.x_sf <= (size_t)L->x_sf_row_bytes,
                "the activation format needs wider x / x_sf rows than the buffer's");
  DGM_CHECK_ARG(intermediate < 0 || (rb.mid <= (size_t)L->mid_row_bytes && rb.mid_sf <= (size_t)L->mid_sf_row_bytes),
                "the activation format needs wider intermediate rows than the buffer's");
  return 0;
}

extern "C" {

}  // extern "C"

// The frontend launch's grid: router rows (4 experts x 4 tokens per workgroup, 8 tokens from
// FE_TILE_MIN_TOKENS on) and, beside them, cast rows of one cast lane per thread (QoQ: one wave
// per token).
static dim3 fe_grid(int num_tokens, int hidden, int num_experts, int act_format, int flags, bool router) {
  const int rx = (num_experts + 3) / 4;
  const int64_t cast_threads = act_format == DGM_ACT_QOQ       ? (int64_t)num_tokens * 64
                               : act_format == DGM_ACT_NVFP4   ? (int64_t)num_tokens * (hidden / 16) * 4
                               : act_format == DGM_ACT_FP8F128 ? (int64_t)num_tokens * (hidden / 128) * 32
                                                               : (int64_t)num_tokens * (hidden / 32) * 8;
  const int64_t cast_rows = (flags & DGM_FE_NO_CAST) ? 0 : (cast_threads + (int64_t)rx * 256 - 1) / ((int64_t)rx * 256);
  const int rtok = num_tokens >= FE_TILE_MIN_TOKENS ? FE_ROUTER_TILE : 4;
  return dim3(rx, (router ? (num_tokens + rtok - 1) / rtok : 0) + (int)cast_rows);
}

extern "C" {

int dgm_frontend_workgroups(int num_tokens, int hidden, int num_experts, int act_format, int flags, int router) {
  if (num_tokens <= 0 || hidden <= 0 || num_experts <= 0) return 0;
  const dim3 g = fe_grid(num_tokens, hidden, num_experts, act_format, flags, router != 0);
  return (int)(g.x * g.y);
}

int dgm_router_topk_launch(const void* hidden_bf16, const void* router_weight_bf16, int num_tokens,
                           int hidden, int num_experts, int topk, int act_format, int flags,
                           int token_offset, void* buffer, const DgmBufferLayout* L, hipStream_t stream) {
  return dgm_router_topk_launch_stamped(hidden_bf16, router_weight_bf16, num_tokens, hidden, num_experts, topk,
                                        act_format, flags, token_offset, buffer, L, nullptr, 0, stream);
}

int dgm_router_topk_launch_stamped(const void* hidden_bf16, const void* router_weight_bf16, int num_tokens,
                                   int hidden, int num_experts, int topk, int act_format, int flags,
                                   int token_offset, void* buffer, const DgmBufferLayout* L, int64_t* stamps,
                                   int stamp_rows, hipStream_t stream) {
  DGM_CHECK_ARG(buffer && L && (hidden_bf16 || num_tokens == 0), "null pointer");   // (no tokens: no rows)
  DGM_CHECK_ARG(topk > 0 && topk <= 16 && topk <= num_experts, "topk");
  DGM_CHECK_ARG(act_format >= DGM_ACT_MXFP4 && act_format <= DGM_ACT_FP8F128, "act_format");
  {
    const int chk = dgm_check_layout_call(L, num_tokens, topk, num_experts, -1, hidden, -1, act_format);
    if (chk) return chk;
  }
  DGM_CHECK_ARG(num_experts <= 1024, "num_experts <= 1024");
  DGM_CHECK_ARG(hidden % 512 == 0, "hidden % 512 == 0");
  DGM_CHECK_ARG(!(flags & DGM_FE_FORCE_BALANCED) || num_experts % topk == 0, "forced-balanced needs E % topk == 0");
  DGM_CHECK_ARG(act_format >= DGM_ACT_MXFP4 && act_format <= DGM_ACT_FP8F128, "act_format");
  DGM_CHECK_ARG(((uintptr_t)hidden_bf16 & 15) == 0 && ((uintptr_t)router_weight_bf16 & 15) == 0, "16-byte alignment");
  DGM_CHECK_ARG(router_weight_bf16 || !(flags & (DGM_FE_FORCE_BALANCED | DGM_FE_ZERO_ROW_UNROUTED | DGM_FE_SELECT_IN_MEGA)),
                "cast only (router_weight NULL): no routing flags");
  DGM_CHECK_ARG(router_weight_bf16 || !(flags & DGM_FE_NO_CAST), "DGM_FE_NO_CAST needs the router weight");
  if (num_tokens == 0) return 0;
  DGM_CHECK_ARG(stamp_rows >= 0 && (stamps != nullptr || stamp_rows == 0), "stamps / stamp_rows");
  uint8_t* buf = (uint8_t*)buffer;
  const int J = hidden / 512;
  const int router = router_weight_bf16 ? 1 : 0;
  const bool tiled = num_tokens >= FE_TILE_MIN_TOKENS;
  const dim3 rg = fe_grid(num_tokens, hidden, num_experts, act_format, flags, router != 0);
  long long* stamp_ptr = (long long*)stamps;
  const uint16_t* x = (const uint16_t*)hidden_bf16;
  const uint16_t* w = (const uint16_t*)router_weight_bf16;
  float* logits = (float*)(buf + L->logits);
  uint32_t* keys = (uint32_t*)(buf + L->fe_keys);
  const int zero_unrouted = (flags & DGM_FE_ZERO_ROW_UNROUTED) ? 1 : 0;
#define DGM_FE(JJ)                                                                                           \
  if (tiled)                                                                                                 \
    hipLaunchKernelGGL((k_frontend<JJ, FE_ROUTER_TILE>), rg, dim3(256), 0, stream, x, w, num_tokens, num_experts, \
                       act_format, logits, keys, zero_unrouted, buf + L->x, buf + L->x_sf, router, stamp_ptr, \
                       stamp_rows);                                                                          \
  else                                                                                                       \
    hipLaunchKernelGGL((k_frontend<JJ, 0>), rg, dim3(256), 0, stream, x, w, num_tokens, num_experts,            \
                       act_format, logits, keys, zero_unrouted, buf + L->x, buf + L->x_sf, router, stamp_ptr,   \
                       stamp_rows)
  switch (J) {
    case 1: DGM_FE(1); break;
    case 2: DGM_FE(2); break;
    case 4: DGM_FE(4); break;
    case 6: DGM_FE(6); break;
    case 8: DGM_FE(8); break;
    default: DGM_CHECK_ARG(false, "hidden must be 512, 1024, 2048, 3072 or 4096");
  }
#undef DGM_FE
  int st = dgm_last_launch_status();
  if (st || (flags & DGM_FE_SELECT_IN_MEGA) || !router) return st;
  hipLaunchKernelGGL(k_select, dim3((num_tokens + SELECT_TPB - 1) / SELECT_TPB), dim3(256), 0, stream, keys, num_tokens,
                     num_experts, topk, flags, token_offset, (int64_t*)(buf + L->topk_idx),
                     (float*)(buf + L->topk_weights));
  return dgm_last_launch_status();
}

int dgm_router_logits_topk_launch(const void* logits_bf16, int num_tokens, int num_experts, int topk, int flags,
                                  int token_offset, void* buffer, const DgmBufferLayout* L, hipStream_t stream) {
  DGM_CHECK_ARG(buffer && L && (logits_bf16 || num_tokens == 0), "null pointer");
  DGM_CHECK_ARG(topk > 0 && topk <= 16 && topk <= num_experts, "topk");
  {
    // (no activation rows are written: the buffer's own format and hidden size)
    const int chk = dgm_check_layout_call(L, num_tokens, topk, num_experts, -1, L->hidden, -1, L->act_format);
    if (chk) return chk;
  }
  DGM_CHECK_ARG(num_experts > 0 && num_experts <= 1024, "num_experts <= 1024");
  DGM_CHECK_ARG(!(flags & DGM_FE_FORCE_BALANCED) || num_experts % topk == 0, "forced-balanced needs E % topk == 0");
  DGM_CHECK_ARG(!(flags & DGM_FE_ZERO_ROW_UNROUTED), "zero-row unrouting needs the hidden rows (dgm_router_topk_launch)");
  if (num_tokens == 0) return 0;
  uint8_t* buf = (uint8_t*)buffer;
  uint32_t* keys = (uint32_t*)(buf + L->fe_keys);
  const int64_t n = (int64_t)num_tokens * num_experts;
  hipLaunchKernelGGL(k_keys_bf16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, (const uint16_t*)logits_bf16, n,
                     num_experts, keys);
  int st = dgm_last_launch_status();
  if (st || (flags & DGM_FE_SELECT_IN_MEGA)) return st;
  hipLaunchKernelGGL(k_select, dim3((num_tokens + SELECT_TPB - 1) / SELECT_TPB), dim3(256), 0, stream, keys, num_tokens,
                     num_experts, topk, flags, token_offset, (int64_t*)(buf + L->topk_idx),
                     (float*)(buf + L->topk_weights));
  return dgm_last_launch_status();
}

// The key array the top-k is selected from under select_in_mega: the caller's, else the buffer's
// (written by a DGM_FE_SELECT_IN_MEGA frontend call).
static const uint32_t* select_keys(const DgmMoeArgs* A, uint8_t* buf, const DgmBufferLayout* L) {
  return A->fe_keys ? (const uint32_t*)A->fe_keys : (const uint32_t*)(buf + L->fe_keys);
}

// Writes topk_idx / topk_weights from the select keys for the paths that read them.
static int materialize_topk(const DgmMoeArgs* A, uint8_t* buf, const DgmBufferLayout* L, hipStream_t stream) {
  hipLaunchKernelGGL(k_select, dim3((A->num_tokens + SELECT_TPB - 1) / SELECT_TPB), dim3(256), 0, stream,
                     select_keys(A, buf, L), A->num_tokens, A->num_experts, A->topk, A->fe_flags,
                     A->token_offset, (int64_t*)(buf + L->topk_idx), (float*)(buf + L->topk_weights));
  return dgm_last_launch_status();
}

// Every workgroup of the fused kernel reads all tokens' logits when it selects the top-k; that
// costs ~1 us of SIMD time per token and workgroup (the selection rounds are sequential), so
// above SELECT_IN_MEGA_FAST_TOKENS a separate selection launch (one wave per token over the
// whole GPU) comes first and the fused kernel reads the result. Forced-balanced routing scans
// no keys, so it is selected in the kernel up to SELECT_IN_MEGA_FAST_BALANCED tokens (at 16
// tokens 0.5-1.4 us less than the extra launch; at 32 and 64 no gain). The in-kernel frontend
// (fe_in_mega) selects in the kernel up to SELECT_IN_MEGA_MAX_TOKENS.
constexpr int SELECT_IN_MEGA_MAX_TOKENS = 64;
constexpr int SELECT_IN_MEGA_FAST_TOKENS = 8;     // (one token per wave)
constexpr int SELECT_IN_MEGA_FAST_BALANCED = 16;

int dgm_megamoe_fused_launch(const DgmMoeArgs* A, hipStream_t stream) {
  const int chk = dgm_check_fused_args(A);
  if (chk) return chk;
  if (A->num_tokens == 0) return 0;
  if (fused_fits(A)) return fused_launch_phases(A, 3, stream);
  DGM_CHECK_ARG(A->act_format != DGM_ACT_QOQ && A->act_format != DGM_ACT_NVFP4,
                "QoQ / NVFP4 layer: at most 1024 routes (tokens x topk), 256 tokens and 512 local experts per call");
  DGM_CHECK_ARG(!A->fe_in_mega, "fe_in_mega: the fused kernel's limits (tokens, routes, local experts) are exceeded");
  return dgm_megamoe_split_launch(A, stream);
}

}  // extern "C"

int dgm_check_fused_args(const DgmMoeArgs* A) {
  DGM_CHECK_ARG(A && A->buffer && A->layout && (A->y || A->num_tokens == 0), "null pointer");
  DGM_CHECK_ARG(A->w1_values && A->w1_scales && A->w2_values && A->w2_scales, "null weights");
  const DgmBufferLayout* L = A->layout;
  DGM_CHECK_ARG(A->topk > 0 && A->topk <= 16, "topk");
  DGM_CHECK_ARG(A->act_format >= DGM_ACT_MXFP4 && A->act_format <= DGM_ACT_FP8F128, "act_format");
  {
    const int chk = dgm_check_layout_call(L, A->num_tokens, A->topk, A->num_experts, A->num_local_experts, A->hidden,
                                          A->intermediate, A->act_format);
    if (chk) return chk;
  }
  DGM_CHECK_ARG(A->num_local_experts > 0 && A->num_local_experts <= MAX_LOCAL_EXPERTS, "num_local_experts");
  DGM_CHECK_ARG(A->expert_begin >= 0 && A->expert_begin + A->num_local_experts <= A->num_experts, "expert range");
  DGM_CHECK_ARG(A->act_format >= DGM_ACT_MXFP4 && A->act_format <= DGM_ACT_FP8F128, "act_format");
  DGM_CHECK_ARG(A->act_format != DGM_ACT_QOQ || (A->w1_row_scales && A->w2_row_scales),
                "QoQ needs the row scales s1 of both matrices");
  DGM_CHECK_ARG(A->topk > 0 && A->topk <= 16, "topk");
  DGM_CHECK_ARG(A->hidden % 128 == 0 && A->intermediate % 32 == 0, "shape");
  DGM_CHECK_ARG(A->intermediate % 128 == 0, "intermediate % 128 == 0");
  if (A->fe_in_mega) {
    DGM_CHECK_ARG(A->hidden_states && A->router_weight, "fe_in_mega: null hidden_states / router_weight");
    DGM_CHECK_ARG(((uintptr_t)A->hidden_states & 15) == 0 && ((uintptr_t)A->router_weight & 15) == 0, "16-byte alignment");
    DGM_CHECK_ARG(A->num_tokens <= SELECT_IN_MEGA_MAX_TOKENS, "fe_in_mega: num_tokens <= 64");
    DGM_CHECK_ARG(A->hidden % 512 == 0, "fe_in_mega: hidden % 512 == 0");
    DGM_CHECK_ARG(A->topk <= A->num_experts && A->num_experts <= 1024, "fe_in_mega: topk, num_experts");
    DGM_CHECK_ARG(!(A->fe_flags & DGM_FE_FORCE_BALANCED) || A->num_experts % A->topk == 0,
                  "forced-balanced needs E % topk == 0");
  }
  return 0;
}

// The persistent kernel's limits (route, token, expert and combine-block counts of its LDS tables)
static bool fused_fits(const DgmMoeArgs* A) {
  return A->num_tokens * A->topk <= FUSED_MAX_ROUTES && A->num_local_experts <= FUSED_MAX_LOCAL &&
         A->num_tokens <= FUSED_MAX_TOKENS && A->hidden / 64 <= FUSED_MAX_NB64;
}

// One launch of the persistent kernel running `phases` (FusedParams::phases) of the layer, with
// the buffer's own workspace views.
static int fused_launch_phases(const DgmMoeArgs* A, int phases, hipStream_t stream) {
  const DgmBufferLayout* L = A->layout;
  uint8_t* buf = (uint8_t*)A->buffer;
  DgmWorkspace w;
  w.pool = buf + L->pool;
  w.mid = buf + L->mid;
  w.mid_sf = buf + L->mid_sf;
  w.partials = (uint16_t*)(buf + L->partials);
  w.part_rows = L->max_tokens;
  w.counters = (int*)(buf + L->counters);
  return dgm_fused_launch_ws(A, phases, w, stream);
}

int dgm_fused_launch_ws(const DgmMoeArgs* A, int phases, const DgmWorkspace& w, hipStream_t stream) {
  const DgmBufferLayout* L = A->layout;
  uint8_t* buf = (uint8_t*)A->buffer;
  {
    const int fast = (A->fe_flags & DGM_FE_FORCE_BALANCED) ? SELECT_IN_MEGA_FAST_BALANCED : SELECT_IN_MEGA_FAST_TOKENS;
    const bool sel = (A->fe_in_mega || (A->select_in_mega && A->num_tokens <= fast)) && (phases & 1);
    if (A->select_in_mega && !sel && (phases & 1)) {
      int st = materialize_topk(A, buf, L, stream);
      if (st) return st;
    }
    FusedParams p;
    p.w1v = (const uint8_t*)A->w1_values;
    p.w1s = (const uint32_t*)A->w1_scales;
    p.w2v = (const uint8_t*)A->w2_values;
    p.w2s = (const uint32_t*)A->w2_scales;
    p.w1r = A->act_format == DGM_ACT_QOQ ? (const float*)A->w1_row_scales : nullptr;
    p.w2r = A->act_format == DGM_ACT_QOQ ? (const float*)A->w2_row_scales : nullptr;
    p.gs1 = A->act_format == DGM_ACT_NVFP4 ? A->l1_global_scales : nullptr;
    p.gs2 = A->act_format == DGM_ACT_NVFP4 ? A->l2_global_scales : nullptr;
    p.x = buf + L->x;
    p.xsf = buf + L->x_sf;
    p.topk_idx = (int64_t*)(buf + L->topk_idx);
    p.topk_w = (float*)(buf + L->topk_weights);
    // (the in-kernel frontend writes the buffer's own keys and logits)
    p.keys = A->fe_in_mega ? (const uint32_t*)(buf + L->fe_keys) : select_keys(A, buf, L);
    p.logits = (float*)(buf + L->logits);
    p.select = sel ? 1 : 0;
    p.fe_in = A->fe_in_mega ? 1 : 0;
    p.hidden = (const uint16_t*)A->hidden_states;
    p.router_w = (const uint16_t*)A->router_weight;
    p.fe_flags = A->fe_flags;
    p.token_offset = A->token_offset;
    p.E = A->num_experts;
    p.mid = w.mid;
    p.mid_sf = w.mid_sf;
    p.partials = w.partials;
    p.part_rows = w.part_rows;
    p.y = (uint16_t*)A->y;
    p.pool_out = w.pool;
    p.recv_stats = A->recv_stats;
    p.counters = w.counters;
    p.host_err = A->host_error;
    p.M = A->num_tokens;
    p.topk = A->topk;
    p.expert_begin = A->expert_begin;
    p.E_local = A->num_local_experts;
    p.clamp = A->activation_clamp;
    p.fast_math = A->fast_math;
    p.spin_limit = 1 << 22;
    p.stamps = (long long*)A->phase_stamps;
    // (debug bit 1: phase_stamps receives the QoQ L1 accumulators instead of stamps)
    p.stamp_rows = A->phase_stamps && !(A->debug_flags & 2) ? A->phase_stamp_rows : 0;
    p.phases = phases;
    p.debug = (int16_t)(A->debug_flags & 31);
    return launch_fused(p, A->hidden, A->intermediate, A->act_format, stream,
                        (A->launch_flags & DGM_LAUNCH_COOPERATIVE) != 0);
  }
}

extern "C" {

int dgm_megamoe_split_launch(const DgmMoeArgs* A, hipStream_t stream) {
  DGM_CHECK_ARG(A && A->buffer && A->layout && (A->y || A->num_tokens == 0), "null pointer");
  DGM_CHECK_ARG(A->act_format >= DGM_ACT_MXFP4 && A->act_format <= DGM_ACT_FP8F128, "act_format");
  DGM_CHECK_ARG(!A->fe_in_mega, "split path: fe_in_mega is a fused-launch option");
  DGM_CHECK_ARG(A->topk > 0 && A->topk <= 16, "topk");
  {
    const int chk = dgm_check_layout_call(A->layout, A->num_tokens, A->topk, A->num_experts, A->num_local_experts,
                                          A->hidden, A->intermediate, A->act_format);
    if (chk) return chk;
  }
  if (A->act_format == DGM_ACT_QOQ || A->act_format == DGM_ACT_NVFP4) {
    // two launches of the persistent kernel: dispatch + L1, then L2 + combine
    DGM_CHECK_ARG(A->w1_values && A->w1_scales && A->w2_values && A->w2_scales, "null weights");
    DGM_CHECK_ARG(A->act_format != DGM_ACT_QOQ || (A->w1_row_scales && A->w2_row_scales),
                  "QoQ needs the row scales s1 of both matrices");
    DGM_CHECK_ARG(A->num_tokens >= 0 && (int64_t)A->num_tokens * A->topk <= A->layout->max_routes,
                  "num_tokens exceeds the buffer");
    DGM_CHECK_ARG(A->topk > 0 && A->topk <= 16, "topk");
    DGM_CHECK_ARG(A->num_local_experts > 0 && A->expert_begin >= 0 &&
                  A->expert_begin + A->num_local_experts <= A->num_experts, "expert range");
    DGM_CHECK_ARG(A->hidden % 128 == 0 && A->intermediate % 128 == 0, "shape");
    if (A->num_tokens == 0) return 0;
    DGM_CHECK_ARG(fused_fits(A), "QoQ / NVFP4 layer: at most 1024 routes (tokens x topk), 256 tokens and 512 local experts per call");
    int st = fused_launch_phases(A, 1, stream);
    if (st) return st;
    return fused_launch_phases(A, 2, stream);
  }
  const DgmBufferLayout* L = A->layout;
  DGM_CHECK_ARG(A->num_tokens >= 0 && (int64_t)A->num_tokens * A->topk <= L->max_routes, "num_tokens exceeds the buffer");
  if (A->num_tokens == 0) return 0;
  uint8_t* buf = (uint8_t*)A->buffer;
  const int routes_n = A->num_tokens * A->topk;
  if (A->select_in_mega) {
    int st0 = materialize_topk(A, buf, L, stream);
    if (st0) return st0;
  }
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(DISPATCH_THREADS), 0, stream,
                     (const int64_t*)(buf + L->topk_idx), routes_n, A->expert_begin, A->num_local_experts,
                     buf + L->pool, A->recv_stats);
  int st = dgm_last_launch_status();
  if (st) return st;
  const int KT1 = A->hidden / 128, KT2 = A->intermediate / 128;
#define DGM_SPLIT(K1, K2)                                                                       \
  (A->act_format == DGM_ACT_MXFP4   ? launch_experts<K1, K2, DGM_ACT_MXFP4>(A, buf, L, stream)   \
   : A->act_format == DGM_ACT_MXFP8 ? launch_experts<K1, K2, DGM_ACT_MXFP8>(A, buf, L, stream)   \
                                    : launch_experts<K1, K2, DGM_ACT_FP8F128>(A, buf, L, stream))
  if (KT1 == 24 && KT2 == 10) {
    st = DGM_SPLIT(24, 10);
  } else if (KT1 == 4 && KT2 == 2) {
    st = DGM_SPLIT(4, 2);
  } else if (KT1 == 8 && KT2 == 4) {
    st = DGM_SPLIT(8, 4);
  } else {
    DGM_CHECK_ARG(false, "supported (hidden, intermediate): (3072, 1280), (512, 256), (1024, 512)");
  }
#undef DGM_SPLIT
  if (st) return st;
  dim3 cg((A->hidden / 4 + 255) / 256, A->num_tokens);
  hipLaunchKernelGGL(k_combine, cg, dim3(256), 0, stream, (const uint16_t*)(buf + L->partials), L->max_tokens,
                     (const int64_t*)(buf + L->topk_idx), A->num_tokens, A->hidden, A->topk, A->expert_begin,
                     A->num_local_experts, (uint16_t*)A->y);
  return dgm_last_launch_status();
}

}  // extern "C"
