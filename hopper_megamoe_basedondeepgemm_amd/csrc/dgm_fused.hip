// One persistent kernel for one GPU's share of the MegaMoE layer (gfx950):
// dispatch -> L1 (gate/up, SwiGLU, requant) -> L2 (down) -> top-k combine.
//
// Schedule. The grid is sized to what the device keeps resident at once. Work units are
// L1 units (active expert a, 32 intermediate features q), then L2 units (active expert a,
// 128 output rows b); workgroups claim them two at a time from one atomic counter per phase
// (the next claim is issued before the current chunk runs) and move to the L2 phase only
// when the L1 counter ran out. L1 units never wait, so an L2 unit's wait (on the L1 arrival
// counter of its expert) is only on units claimed earlier by running workgroups. Every wait
// is a bounded spin; on expiry the
// kernel raises an error flag and carries on, so every wave always reaches the end. Units
// of a chunk share an expert, so the 16-column B slab (routed activations or intermediate
// rows) is staged in LDS once.
//
// Streaming. A wave keeps one unit's weight tiles in registers (one 1 KB coalesced load per
// 16x128 tile, <= 12 KB per wave). The next unit's tiles are issued into the same registers
// right after the current unit's matrix-core ops, so the epilogue, barriers, stores and
// hand-offs of a unit overlap the next unit's HBM traffic; 8-wave workgroups at 4 waves per
// SIMD overlap the rest across workgroups.
//
// Dispatch. Every workgroup derives the same pool table from topk_idx in LDS (a few hundred
// routes): per-expert counts, the active-expert list (ascending) and the canonical pool
// order (token asc, slot asc). Workgroup 0 also publishes it, the recv stats and the zero
// rows of unrouted tokens.
//
// Hand-offs between workgroups go through HBM with agent-coherent accesses only: the data
// (intermediate codes and scales, fp32 route outputs) is written with relaxed agent-scope
// atomic stores (write-through, "sc1") and read with agent-scope atomic loads, and the
// producer waits for its stores to complete (s_waitcnt) before bumping the arrival counter.
// No agent-scope release/acquire fence is used: on this GPU those write back / invalidate a
// whole L2 and cost tens of microseconds each.
//   L1 unit -> mid codes + scales of its 32 features, then l1_done[a] += 1
//   L2 unit waits l1_done[a] == I/32, writes fp32 route outputs, then comb[t][b] += 1 per
//   route; the arrival that completes token t's block b sums the token's slots in slot order
//   and writes y (bf16).
// The last workgroup to finish clears all counters, so the next launch starts from zero.
#include "dgm_common.hpp"
#include "dgm_abi_internal.hpp"
#include "dgm_fused.hpp"

using namespace dgm;

namespace {

struct alignas(16) U4 { uint32_t x, y, z, w; };

DGM_DEV v8i as_v8i(U4 a) { v8i r = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0}; return r; }
DGM_DEV v8i as_v8i(U4 a, U4 b) {
  v8i r = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
  return r;
}

// agent-coherent (write-through / L2-bypassing) accesses for cross-workgroup hand-offs
DGM_DEV void st_agent64(void* p, uint64_t v) {
  __hip_atomic_store((uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DGM_DEV void st_agent8(uint8_t* p, uint8_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DGM_DEV uint64_t ld_agent64(const void* p) {
  return __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DGM_DEV uint32_t ld_agent8(const uint8_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DGM_DEV float ld_agent_f32(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// all of this wave's memory operations have completed (stores acknowledged)
DGM_DEV void wait_mem() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

constexpr int FT = 512;        // threads per workgroup (8 waves)
constexpr int NW = FT / 64;

template <int KT1, int KT2, int ACT>
struct FusedSmem {
  static constexpr int BV = ACT == DGM_ACT_MXFP4 ? 1 : 2;          // U4 per lane per K-tile
  static constexpr int KTM = KT1 > KT2 ? KT1 : KT2;
  int exp_of_route[FUSED_MAX_ROUTES];
  int routes[FUSED_MAX_ROUTES];
  int act[FUSED_MAX_LOCAL];
  int aoff[FUSED_MAX_LOCAL + 1];
  int nslot[FUSED_MAX_TOKENS];
  int wsum[NW][2];
  int meta[4];
  union {
    struct {                           // dispatch only
      int cnt[FUSED_MAX_LOCAL];
      int eoff[FUSED_MAX_LOCAL];
    };
    U4 bst[KTM][64][BV];               // B slab in matrix-core fragment order
  };
  uint32_t bsc[(KTM + 3) / 4][64];     // its E8M0 scales, 4 K-tiles per dword
  float slab_w[16];                    // routing weights of the staged slab's routes (L1)
  float red[2][2][64][4];              // L1: second-K-half sums [pair][gate/up][lane][i]
  float upv[2][64][4];                 // L1: reduced up values for the gate waves
  float amax[2][16];
  int last[FUSED_MAX_TOKENS];
  int nlast;
  int is_last;
  int claim;
};

// Exclusive scan of (count, active flag) over n <= FUSED_MAX_LOCAL experts.
template <class S>
DGM_DEV void scan_experts(S& s, int n) {
  constexpr int PER = (FUSED_MAX_LOCAL + FT - 1) / FT;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  int c[PER], a[PER], sc = 0, sa = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    int e = tid * PER + j;
    c[j] = e < n ? s.cnt[e] : 0;
    a[j] = c[j] > 0 ? 1 : 0;
    sc += c[j];
    sa += a[j];
  }
  int ic = sc, ia = sa;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int oc = __shfl_up(ic, off), oa = __shfl_up(ia, off);
    if (lane >= off) { ic += oc; ia += oa; }
  }
  if (lane == 63) { s.wsum[wv][0] = ic; s.wsum[wv][1] = ia; }
  __syncthreads();
  int bc = 0, ba = 0;
  for (int i = 0; i < wv; ++i) { bc += s.wsum[i][0]; ba += s.wsum[i][1]; }
  int xc = bc + ic - sc, xa = ba + ia - sa;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    int e = tid * PER + j;
    if (e < n) {
      s.eoff[e] = xc;
      if (a[j]) { s.act[xa] = e; s.aoff[xa] = xc; }
    }
    xc += c[j];
    xa += a[j];
  }
  if (tid == FT - 1) {
    int tc = 0, ta = 0;
    for (int i = 0; i < NW; ++i) { tc += s.wsum[i][0]; ta += s.wsum[i][1]; }
    s.meta[0] = ta;
    s.meta[1] = tc;
    s.aoff[ta] = tc;
  }
  __syncthreads();
}

DGM_DEV bool spin_until(const int* p, int target, int limit, int* err) {
  int n = 0;
  while (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
    if (++n > limit) {
      __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

// Stage the B slab (16 columns = rows row_of(c) of a [rows, KT*128] activation matrix with
// row_bytes and per-32 E8M0 scales) into LDS in fragment order. Column c >= n is zero.
// COHERENT: the rows were written by other workgroups of this launch (agent-scope loads).
template <int KT, int ACT, bool COHERENT, class S, class RowOf>
DGM_DEV void stage_slab(S& s, const uint8_t* __restrict__ src, const uint8_t* __restrict__ ssrc,
                        int row_bytes, int n, RowOf row_of) {
  const int tid = threadIdx.x;
  for (int f = tid; f < KT * 64; f += FT) {
    const int kt = f >> 6, l = f & 63, c = l & 15;
    uint4 v0 = make_uint4(0, 0, 0, 0), v1 = make_uint4(0, 0, 0, 0);
    if (c < n) {
      const size_t r = (size_t)row_of(c);
      // E2M1: 16 bytes at K = 32 g; E4M3: K = 16 g .. +16 and K = 64 + 16 g .. +16 (g = l / 16)
      const uint8_t* q = ACT == DGM_ACT_MXFP4 ? src + r * row_bytes + kt * 64 + (l >> 4) * 16
                                              : src + r * row_bytes + kt * 128 + (l >> 4) * 16;
      if (COHERENT) {
        uint64_t a0 = ld_agent64(q), a1 = ld_agent64(q + 8);
        v0 = make_uint4((uint32_t)a0, (uint32_t)(a0 >> 32), (uint32_t)a1, (uint32_t)(a1 >> 32));
        if (ACT != DGM_ACT_MXFP4) {
          uint64_t b0 = ld_agent64(q + 64), b1 = ld_agent64(q + 72);
          v1 = make_uint4((uint32_t)b0, (uint32_t)(b0 >> 32), (uint32_t)b1, (uint32_t)(b1 >> 32));
        }
      } else {
        v0 = *reinterpret_cast<const uint4*>(q);
        if (ACT != DGM_ACT_MXFP4) v1 = *reinterpret_cast<const uint4*>(q + 64);
      }
    }
    uint4* dst = reinterpret_cast<uint4*>(&s.bst[kt][l][0]);
    dst[0] = v0;
    if (ACT != DGM_ACT_MXFP4) dst[S::BV - 1] = v1;
  }
  for (int f = tid; f < ((KT + 3) / 4) * 64; f += FT) {
    const int g = f >> 6, l = f & 63, c = l & 15;
    uint32_t w = 0x7f7f7f7fu;
    if (c < n) {
      const size_t r = (size_t)row_of(c);
      w = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kt = 4 * g + j;
        uint32_t b = 127u;
        if (kt < KT) {
          const uint8_t* q = ssrc + r * (KT * 4) + kt * 4 + (l >> 4);
          b = COHERENT ? ld_agent8(q) : (uint32_t)*q;
        }
        w |= b << (8 * j);
      }
    }
    s.bsc[g][l] = w;
  }
}

// Phase stamps (the reference's phase_stamps facility): per workgroup, 100 MHz wall clock at
// [0] entry, [1] dispatch table ready, [2] L1 units done, [3] first L1 arrival observed,
// [4] L2 units done, [5] exit; [6] wall ticks spent waiting on L1 arrivals, [7] reserved.
DGM_DEV long long wall_clock() { return (long long)__builtin_amdgcn_s_memrealtime(); }

template <int KT1, int KT2, int ACT>
__global__ void __launch_bounds__(FT) k_megamoe(FusedParams p) {
  using Smem = FusedSmem<KT1, KT2, ACT>;
  __shared__ Smem s;
  constexpr int FB = ACT == DGM_ACT_MXFP4 ? 4 : 0;        // B operand format
  constexpr int KH = KT1 / 2;                               // L1 K-tiles per wave (K halves)
  constexpr int KG1 = (KT1 + 3) / 4, KG2 = (KT2 + 3) / 4;
  constexpr int H = KT1 * 128, I = KT2 * 128;
  constexpr int XB = ACT == DGM_ACT_MXFP4 ? H / 2 : H;     // activation row bytes
  constexpr int MB = ACT == DGM_ACT_MXFP4 ? I / 2 : I;     // intermediate row bytes
  constexpr int QN = I / 32, NB1 = I / 8, NB2 = H / 16, NBL2 = H / (16 * NW);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index: scalar
  const int R = p.M * p.topk;
  int* exit_cnt = p.counters + CNT_EXIT;
  int* err = p.counters + CNT_ERROR;
  int* l1_done = p.counters + CNT_L1;
  int* comb = p.counters + CNT_L1 + FUSED_MAX_LOCAL;
  long long* st = (p.stamps && (int)blockIdx.x < p.stamp_rows) ? p.stamps + (size_t)blockIdx.x * 8 : nullptr;
  long long wait_ticks = 0;
  if (st && tid == 0) st[0] = wall_clock();

  // ---------------------------------------------------------------- dispatch (every WG)
  for (int e = tid; e < p.E_local; e += FT) s.cnt[e] = 0;
  for (int t = tid; t < p.M; t += FT) s.nslot[t] = 0;
  if (tid == 0) s.nlast = 0;
  for (int r = tid; r < R; r += FT) {
    int64_t g = p.topk_idx[r];
    int64_t l = g - p.expert_begin;
    s.exp_of_route[r] = (g >= 0 && l >= 0 && l < p.E_local) ? (int)l : -1;
  }
  __syncthreads();
  for (int r = tid; r < R; r += FT) {
    int e = s.exp_of_route[r];
    if (e >= 0) { atomicAdd(&s.cnt[e], 1); atomicAdd(&s.nslot[r / p.topk], 1); }
  }
  __syncthreads();
  scan_experts(s, p.E_local);
  for (int r = tid; r < R; r += FT) {
    int e = s.exp_of_route[r];
    if (e < 0) continue;
    int rank = 0;
    for (int q = 0; q < r; ++q) rank += s.exp_of_route[q] == e ? 1 : 0;
    s.routes[s.eoff[e] + rank] = r;
  }
  __syncthreads();
  const int n_active = s.meta[0];
  if (st && tid == 0) st[1] = wall_clock();
  if (blockIdx.x == 0) {
    int* meta = (int*)p.pool_out;
    int* gcnt = (int*)(p.pool_out + 256);
    int* gact = (int*)(p.pool_out + 256 + a256i(p.E_local * 4));
    int* goff = (int*)(p.pool_out + 256 + 2 * a256i(p.E_local * 4));
    int* grt = (int*)(p.pool_out + 256 + 2 * a256i(p.E_local * 4) + a256i((p.E_local + 1) * 4));
    if (tid == 0) { meta[0] = n_active; meta[1] = s.meta[1]; }
    for (int e = tid; e < p.E_local; e += FT) {
      gcnt[e] = s.cnt[e];
      if (p.recv_stats) p.recv_stats[e] += s.cnt[e];
    }
    for (int a = tid; a <= n_active; a += FT) {
      goff[a] = s.aoff[a];
      if (a < n_active) gact[a] = s.act[a];
    }
    for (int r = tid; r < s.meta[1]; r += FT) grt[r] = s.routes[r];
    // tokens without a local route: y row = 0
    for (int i = tid; i < p.M * (H / 8); i += FT) {
      int t = i / (H / 8);
      if (s.nslot[t] == 0) reinterpret_cast<U4*>(p.y + (size_t)t * H)[i % (H / 8)] = U4{0, 0, 0, 0};
    }
  }
  __syncthreads();        // s.cnt / s.eoff (union with the B slab) are dead from here on

  // Units are claimed dynamically, CH at a time: L1 units (active expert a, 32 features q)
  // from one counter, then L2 units (active expert a, 128 output rows b) from another. A
  // workgroup starts on L2 units only after the L1 counter ran out, so an L2 unit's wait is
  // only on L1 units already claimed by running workgroups, which never wait.
  const int U1 = n_active * QN, U2 = n_active * NBL2;
  constexpr int CH = 2;
  const int c = lane & 15, kq = lane >> 4;
  // L1 wave roles: pair pp = w & 1 (16 of the unit's 32 features), tile gu = (w >> 1) & 1
  // (gate or up), K half kh = w >> 2. L2: wave w owns rows 16 (NW b + w) .. +16, full K.
  const int pp = wv & 1, gu = (wv >> 1) & 1, kh = wv >> 2;
  constexpr int NSD = (KH + 3) / 4 + 1;                     // L1 scale dwords per K half
  int staged = -1;          // (phase, a, slab) currently in s.bst
  {
    int* claim = p.counters + CNT_CLAIM + 0;
    int next_claim = 0;
    if (tid == 0) next_claim = __hip_atomic_fetch_add(claim, CH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (;;) {
      if (tid == 0) s.claim = next_claim;
      __syncthreads();
      const int base = __builtin_amdgcn_readfirstlane(s.claim);   // uniform: keep it scalar
      __syncthreads();
      if (base >= U1) break;
      // claim the next chunk now; its value is needed only after this chunk
      if (tid == 0) next_claim = base + CH < U1 ? __hip_atomic_fetch_add(claim, CH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : U1;
      const int top = base + CH < U1 ? base + CH : U1;
      for (int u = base; u < top; ++u) {
      // ============================================================ L1 unit
      const int a = u / QN, q = u % QN;
      U4 wt[KH];
      uint32_t sd[NSD];
      {
        const size_t blk = (size_t)s.act[a] * NB1 + 2 * (2 * q + pp) + gu;
        const uint8_t* base_w = p.w1v + (blk * KT1 + kh * KH) * 1024 + lane * 16;
#pragma unroll
        for (int k = 0; k < KH; ++k) wt[k] = *reinterpret_cast<const U4*>(base_w + k * 1024);
        const int g_lo = (kh * KH) >> 2;
        const uint32_t* sb = p.w1s + (blk * KG1 + g_lo) * 64 + lane;
#pragma unroll
        for (int j = 0; j < NSD; ++j) sd[j] = g_lo + j < KG1 ? sb[j * 64] : 0u;
      }
      const int r0 = s.aoff[a], n = s.aoff[a + 1] - r0;
      const int pr = 2 * q + pp;                       // (gate, up) block pair of this wave
      const int g_lo = (kh * KH) >> 2;
      for (int s0 = 0; s0 < n; s0 += 16) {
        const int key = (a << 16) | s0;
        if (key != staged) {
          __syncthreads();
          const int topk = p.topk;
          const int* rts = s.routes + r0 + s0;
          stage_slab<KT1, ACT, false>(s, p.x, p.xsf, XB, n - s0, [rts, topk](int cc) { return rts[cc] / topk; });
          if (tid < 16) s.slab_w[tid] = s0 + tid < n ? p.topk_w[rts[tid]] : 0.f;
          staged = key;
          __syncthreads();
        }
        const bool valid = s0 + c < n;
        v4f acc = {0.f, 0.f, 0.f, 0.f};
        static_for<KH>([&](auto kc) {
          constexpr int k = decltype(kc)::value;
          const int kt = kh * KH + k;
          v8i bop;
          if (ACT == DGM_ACT_MXFP4) bop = as_v8i(s.bst[kt][lane][0]);
          else bop = as_v8i(s.bst[kt][lane][0], s.bst[kt][lane][Smem::BV - 1]);
          const int bsw = (int)s.bsc[kt >> 2][lane];
          if constexpr (KH % 4 == 0) {
            // the K half starts on a scale dword: byte k & 3 of dword k / 4 (hardware select)
            acc = mfma_scale_16x16x128_sel<4, FB, k & 3, k & 3>(as_v8i(wt[k]), bop, acc, (int)sd[k >> 2], bsw);
          } else {       // small shapes
            const int j = (kt >> 2) - g_lo, sh = 8 * (kt & 3);
            uint32_t wsa = sd[0];
#pragma unroll
            for (int jj = 1; jj < NSD; ++jj) wsa = j == jj ? sd[jj] : wsa;
            acc = mfma_scale_16x16x128<4, FB>(as_v8i(wt[k]), bop, acc, (int)(wsa >> sh), bsw >> sh);
          }
          // keep the LDS reads of the B operand at most a few K-tiles ahead (register budget)
          if constexpr ((k & (ACT == DGM_ACT_MXFP4 ? 3 : 1)) == (ACT == DGM_ACT_MXFP4 ? 3 : 1))
            __builtin_amdgcn_sched_barrier(0);
        });

        if (kh == 1) {
  #pragma unroll
          for (int i = 0; i < 4; ++i) s.red[pp][gu][lane][i] = acc[i];
        }
        __syncthreads();
        if (kh == 0) {
  #pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] = acc[i] + s.red[pp][gu][lane][i];
          if (gu == 1) {
  #pragma unroll
            for (int i = 0; i < 4; ++i) s.upv[pp][lane][i] = acc[i];
          }
        }
        __syncthreads();
        float act[4];
        if (kh == 0 && gu == 0) {
          const float wt_r = s.slab_w[c];
          float am = 0.f;
  #pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float g = fminf(round_bf16(acc[i]), p.clamp);
            const float uu = fminf(fmaxf(round_bf16(s.upv[pp][lane][i]), -p.clamp), p.clamp);
            const float sgm = 1.0f / (1.0f + expf(-g));
            act[i] = valid ? ((g * sgm) * uu) * wt_r : 0.f;
            am = fmaxf(am, fabsf(act[i]));
          }
          am = fmaxf(am, __shfl_xor(am, 16));
          am = fmaxf(am, __shfl_xor(am, 32));
          if (lane < 16) s.amax[pp][lane] = am;
        }
        __syncthreads();
        if (kh == 0 && gu == 0) {
          const float am = fmaxf(s.amax[0][c], s.amax[1][c]);
          const int row = r0 + s0 + c;
          // lane group kq holds features 16 pr + 4 kq .. +3 of column c
          if (ACT == DGM_ACT_MXFP4) {
            const uint32_t code = ceil_ue8m0_code(fmaxf(am, 1e-30f) / 6.0f);
            const float sc = e8m0_value(code);
            uint32_t w = 0;
  #pragma unroll
            for (int i = 0; i < 4; ++i) w |= e2m1_ties_down(act[i] / sc) << (4 * i);
            // gather the 4 lane groups: 16 features = 8 bytes of the intermediate row
            const uint64_t w64 = (uint64_t)(w & 0xffffu) | ((uint64_t)(__shfl(w, c + 16) & 0xffffu) << 16) |
                                 ((uint64_t)(__shfl(w, c + 32) & 0xffffu) << 32) |
                                 ((uint64_t)(__shfl(w, c + 48) & 0xffffu) << 48);
            if (valid && lane < 16) {
              st_agent64(p.mid + (size_t)row * MB + 8 * pr, w64);
              if (pp == 0) st_agent8(p.mid_sf + (size_t)row * (I / 32) + q, (uint8_t)code);
            }
          } else {
            const int code = (int)ceil_log2_f32(fmaxf(am, 1e-30f) / 448.0f) + 127;
            const float sc = e8m0_value_any((uint32_t)code);
            uint32_t w = 0;
  #pragma unroll
            for (int i = 0; i < 4; ++i) w |= e4m3_encode(act[i] / sc) << (8 * i);
            // lanes 0-15: features 0-7 (groups 0, 1); lanes 16-31: features 8-15 (groups 2, 3)
            const int src_lo = lane < 16 ? c : c + 32, src_hi = lane < 16 ? c + 16 : c + 48;
            const uint64_t w64 = (uint64_t)__shfl(w, src_lo) | ((uint64_t)__shfl(w, src_hi) << 32);
            if (valid && lane < 32) {
              st_agent64(p.mid + (size_t)row * MB + 16 * pr + (lane < 16 ? 0 : 8), w64);
              if (pp == 0 && lane < 16) st_agent8(p.mid_sf + (size_t)row * (I / 32) + q, (uint8_t)code);
            }
          }
        }
      }
      // arrival: this unit's intermediate stores have completed (the wait also covers the
      // next task's tiles issued above, which the next iteration needs first anyway)
      wait_mem();
      __syncthreads();
      if (tid == 0) __hip_atomic_fetch_add(&l1_done[a], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  {
    int* claim = p.counters + CNT_CLAIM + 1;
    int next_claim = 0;
    if (tid == 0) next_claim = __hip_atomic_fetch_add(claim, CH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (st && tid == 0) st[2] = wall_clock();
    int ready = -1;         // active expert whose L1 arrival has been observed
    for (;;) {
      if (tid == 0) s.claim = next_claim;
      __syncthreads();
      const int base = __builtin_amdgcn_readfirstlane(s.claim);   // uniform: keep it scalar
      __syncthreads();
      if (base >= U2) break;
      // claim the next chunk now; its value is needed only after this chunk
      if (tid == 0) next_claim = base + CH < U2 ? __hip_atomic_fetch_add(claim, CH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : U2;
      const int top = base + CH < U2 ? base + CH : U2;
      for (int v = base; v < top; ++v) {
      const int a = v / NBL2, b = v % NBL2;
      U4 wt[KT2];
      uint32_t sd[KG2];
      {
        const size_t blk = (size_t)s.act[a] * NB2 + NW * b + wv;
        const uint8_t* base_w = p.w2v + blk * KT2 * 1024 + lane * 16;
#pragma unroll
        for (int k = 0; k < KT2; ++k) wt[k] = *reinterpret_cast<const U4*>(base_w + k * 1024);
#pragma unroll
        for (int g = 0; g < KG2; ++g) sd[g] = p.w2s[(blk * KG2 + g) * 64 + lane];
      }
      const int r0 = s.aoff[a], n = s.aoff[a + 1] - r0;
      if (a != ready) {
        long long w0 = st ? wall_clock() : 0;
        if (tid == 0) spin_until(&l1_done[a], QN, p.spin_limit, err);
        __syncthreads();
        if (st) {
          wait_ticks += wall_clock() - w0;
          if (tid == 0 && ready == -1) st[3] = wall_clock();
        }
        ready = a;
      }
      for (int s0 = 0; s0 < n; s0 += 16) {
        const int key = (1 << 30) | (a << 16) | s0;
        if (key != staged) {
          __syncthreads();
          const int rb = r0 + s0;
          stage_slab<KT2, ACT, true>(s, p.mid, p.mid_sf, MB, n - s0, [rb](int cc) { return rb + cc; });
          staged = key;
          __syncthreads();
        }
        v4f acc = {0.f, 0.f, 0.f, 0.f};
        static_for<KT2>([&](auto kc) {
          constexpr int k = decltype(kc)::value;
          v8i bop;
          if (ACT == DGM_ACT_MXFP4) bop = as_v8i(s.bst[k][lane][0]);
          else bop = as_v8i(s.bst[k][lane][0], s.bst[k][lane][Smem::BV - 1]);
          acc = mfma_scale_16x16x128_sel<4, FB, k & 3, k & 3>(as_v8i(wt[k]), bop, acc, (int)sd[k >> 2],
                                                              (int)s.bsc[k >> 2][lane]);
          if constexpr ((k & (ACT == DGM_ACT_MXFP4 ? 3 : 1)) == (ACT == DGM_ACT_MXFP4 ? 3 : 1))
            __builtin_amdgcn_sched_barrier(0);
        });
        __builtin_amdgcn_sched_barrier(0);
        
        if (s0 + c < n) {
          const int rid = s.routes[r0 + s0 + c];
          float* dst = p.partials + (size_t)rid * H + (NW * b + wv) * 16 + 4 * kq;
          st_agent64(dst, (uint64_t)__float_as_uint(acc[0]) | ((uint64_t)__float_as_uint(acc[1]) << 32));
          st_agent64(dst + 2, (uint64_t)__float_as_uint(acc[2]) | ((uint64_t)__float_as_uint(acc[3]) << 32));
        }
      }
      // ---- combine: the arrival that completes (token, row block b) writes y
      wait_mem();
      __syncthreads();
      for (int r = tid; r < n; r += FT) {
        const int tk = s.routes[r0 + r] / p.topk;
        const int old = __hip_atomic_fetch_add(&comb[tk * NBL2 + b], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == s.nslot[tk] - 1) s.last[atomicAdd(&s.nlast, 1)] = tk;
      }
      __syncthreads();
      const int nl = s.nlast;
      constexpr int RB = 16 * NW;
      for (int i = tid; i < nl * RB; i += FT) {
        const int tk = s.last[i / RB], row = b * RB + (i % RB);
        float sum = 0.f;
        for (int sl = 0; sl < p.topk; ++sl)
          if (s.exp_of_route[tk * p.topk + sl] >= 0) sum += ld_agent_f32(p.partials + ((size_t)tk * p.topk + sl) * H + row);
        p.y[(size_t)tk * H + row] = f32_to_bf16(sum);
      }
      __syncthreads();
      if (tid == 0) s.nlast = 0;
      }
    }
  }

  // ---------------------------------------------------------------- teardown
  if (st && tid == 0) {
    st[4] = wall_clock();
    st[6] = wait_ticks;
    st[7] = 0;
  }
  wait_mem();
  __syncthreads();
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(exit_cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s.is_last = old == (int)gridDim.x - 1;
  }
  __syncthreads();
  if (s.is_last) {
    for (int a = tid; a < n_active; a += FT) __hip_atomic_store(&l1_done[a], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int i = tid; i < p.M * NBL2; i += FT) __hip_atomic_store(&comb[i], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid < 2) __hip_atomic_store(p.counters + CNT_CLAIM + tid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wait_mem();
    __syncthreads();
    if (tid == 0) __hip_atomic_store(exit_cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (st && tid == 0) st[5] = wall_clock();
}

struct GridCache { int blocks[3][3][2] = {}; };
GridCache g_grid;

template <int KT1, int KT2, int ACT>
int launch_fused_t(const FusedParams& prm, int slot, hipStream_t stream) {
  int& nb = g_grid.blocks[slot][ACT][0];
  if (nb == 0) {
    int per_cu = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_megamoe<KT1, KT2, ACT>, FT, 0);
    if (e != hipSuccess || per_cu < 1) per_cu = 1;
    int dev = 0, cus = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    nb = per_cu * (cus > 0 ? cus : 256);
  }
  hipLaunchKernelGGL((k_megamoe<KT1, KT2, ACT>), dim3(nb), dim3(FT), 0, stream, prm);
  return dgm_last_launch_status();
}

}  // namespace

int dgm_fused_grid_blocks(int hidden, int intermediate, int act_format) {
  int slot = hidden == 3072 ? 0 : (hidden == 512 ? 1 : 2);
  return g_grid.blocks[slot][act_format][0];
}

int launch_fused(const FusedParams& prm, int hidden, int intermediate, int act, hipStream_t stream) {
  if (hidden == 3072 && intermediate == 1280)
    return act == DGM_ACT_MXFP4 ? launch_fused_t<24, 10, DGM_ACT_MXFP4>(prm, 0, stream)
                                : launch_fused_t<24, 10, DGM_ACT_MXFP8>(prm, 0, stream);
  if (hidden == 512 && intermediate == 256)
    return act == DGM_ACT_MXFP4 ? launch_fused_t<4, 2, DGM_ACT_MXFP4>(prm, 1, stream)
                                : launch_fused_t<4, 2, DGM_ACT_MXFP8>(prm, 1, stream);
  if (hidden == 1024 && intermediate == 512)
    return act == DGM_ACT_MXFP4 ? launch_fused_t<8, 4, DGM_ACT_MXFP4>(prm, 2, stream)
                                : launch_fused_t<8, 4, DGM_ACT_MXFP8>(prm, 2, stream);
  dgm_set_error("fused kernel: supported (hidden, intermediate) are (3072, 1280), (512, 256), (1024, 512)");
  return DGM_ERR_INVALID_ARGUMENT;
}
