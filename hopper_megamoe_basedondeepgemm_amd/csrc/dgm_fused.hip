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

// Weight tiles are read exactly once: non-temporal loads ("nt") keep them from allocating in
// the L2 / MALL, which lifts streaming bandwidth from ~5.4 to ~7 TB/s on MI355X.
typedef unsigned v4u __attribute__((ext_vector_type(4)));
DGM_DEV U4 ld_stream(const uint8_t* p) {
  v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
  return U4{v.x, v.y, v.z, v.w};
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
// Compiler-only ordering point: memory operations after it stay after the matrix-core ops
// that produced `acc` (otherwise the next unit's tile loads may be hoisted above them and
// need a second register set).
DGM_DEV void after_mfma(v4f acc) {
  asm volatile("" ::"v"(acc[0]), "v"(acc[1]), "v"(acc[2]), "v"(acc[3]) : "memory");
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
  int claimv[2];
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
// [4] L2 units done, [5] exit; [6] wall ticks from L1 unit start to its matrix-core ops done
// (weights landed), [7] wall ticks in L1 arrival signalling (store completion + barrier).
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
  long long wait_ticks = 0, l1_load_ticks = 0, l1_sig_ticks = 0;
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
  //
  // Software pipeline: right after a unit's last matrix-core ops the next unit's weight tiles
  // are issued into the same registers (dead by then), so they stream in
  // while the unit's epilogue, stores and hand-offs run. A unit's arrival signal (L1) or
  // combine arrivals (L2) are sent one unit later, after the next unit's matrix-core ops,
  // when the unit's own stores have long completed (the wait for them is then free).
  const int U1 = n_active * QN, U2 = n_active * NBL2;
  constexpr int CH = 2;
  const int c = lane & 15, kq = lane >> 4;
  // L1 wave roles: pair pp = w & 1 (16 of the unit's 32 features), tile gu = (w >> 1) & 1
  // (gate or up), K half kh = w >> 2. L2: wave w owns rows 16 (NW b + w) .. +16, full K.
  const int pp = wv & 1, gu = (wv >> 1) & 1, kh = wv >> 2;
  constexpr int NSD = (KH + 3) / 4 + 1;                     // L1 scale dwords per K half
  const int g_lo = (kh * KH) >> 2;
  int staged = -1;          // (phase, a, slab) currently in s.bst
  int par = 0;              // LDS slot of the next chunk broadcast (alternates)

  // ================================================================ L1 phase
  {
    int* claim = p.counters + CNT_CLAIM;
    const uint8_t* w1v = p.w1v;
    const uint32_t* w1s = p.w1s;
    auto load1 = [w1v, w1s, lane, pp, gu, kh, g_lo](int u, U4 (&w)[KH], uint32_t (&sw)[NSD]) {
      const int a = u / QN, q = u % QN;
      const size_t blk = (size_t)s.act[a] * NB1 + 2 * (2 * q + pp) + gu;
      const uint8_t* bw = w1v + (blk * KT1 + kh * KH) * 1024 + lane * 16;
#pragma unroll
      for (int k = 0; k < KH; ++k) w[k] = ld_stream(bw + k * 1024);
      const uint32_t* sb = w1s + (blk * KG1 + g_lo) * 64 + lane;
#pragma unroll
      for (int j = 0; j < NSD; ++j) sw[j] = g_lo + j < KG1 ? __builtin_nontemporal_load(sb + j * 64) : 0u;
    };
    if (tid == 0) s.claimv[par] = __hip_atomic_fetch_add(claim, CH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    int cur = __builtin_amdgcn_readfirstlane(s.claimv[par]);
    par ^= 1;
    int top = cur + CH < U1 ? cur + CH : U1;
    int ahead = U1;           // thread 0: the chunk claimed one chunk ahead
    if (tid == 0 && cur + CH < U1) ahead = __hip_atomic_fetch_add(claim, CH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    U4 wt[KH];
    uint32_t sd[NSD];
    if (cur < U1) load1(cur, wt, sd);
    int pending = -1;         // expert slot of the previous unit; its arrival is not sent yet
    while (cur < U1) {
      const int a = cur / QN, q = cur % QN;
      const int r0 = s.aoff[a], n = s.aoff[a + 1] - r0;
      const int pr = 2 * q + pp;                       // (gate, up) block pair of this wave
      int nxt = cur + 1;
      if (nxt >= top) {       // next chunk: the one claimed ahead, broadcast through LDS
        if (tid == 0) s.claimv[par] = ahead;
        __syncthreads();
        nxt = __builtin_amdgcn_readfirstlane(s.claimv[par]);
        par ^= 1;
        top = nxt + CH < U1 ? nxt + CH : U1;
        if (tid == 0) ahead = nxt + CH < U1 ? __hip_atomic_fetch_add(claim, CH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : U1;
      }
      const long long t_u0 = st ? wall_clock() : 0;
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
        after_mfma(acc);
        if (st) l1_load_ticks += wall_clock() - t_u0;
        const bool signal = s0 == 0 && pending >= 0;
        if (signal) wait_mem();                        // the previous unit's stores completed
        // the last slab's matrix-core ops were the last readers: reuse the registers
        if (s0 + 16 >= n && nxt < U1) load1(nxt, wt, sd);
        __builtin_amdgcn_sched_barrier(0);

        if (kh == 1) {
#pragma unroll
          for (int i = 0; i < 4; ++i) s.red[pp][gu][lane][i] = acc[i];
        }
        __syncthreads();
        // every wave waited for its stores before the barrier: the previous unit has arrived
        if (signal && tid == 0) __hip_atomic_fetch_add(&l1_done[pending], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
            const float sgm = p.fast_math ? sigmoid<true>(g) : sigmoid<false>(g);
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
            const float isc = e8m0_inv(code);
            uint32_t w = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) w |= e2m1_ties_down(act[i] * isc) << (4 * i);
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
            const float isc = e8m0_inv((uint32_t)code);
            uint32_t w = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) w |= e4m3_encode(act[i] * isc) << (8 * i);
            // lanes 0-15: features 0-7 (groups 0, 1); lanes 16-31: features 8-15 (groups 2, 3)
            const int src_lo = lane < 16 ? c : c + 32, src_hi = lane < 16 ? c + 16 : c + 48;
            const uint64_t w64 = (uint64_t)__shfl(w, src_lo) | ((uint64_t)__shfl(w, src_hi) << 32);
            if (valid && lane < 32) {
              st_agent64(p.mid + (size_t)row * MB + 16 * pr + (lane < 16 ? 0 : 8), w64);
              if (pp == 0 && lane < 16) st_agent8(p.mid_sf + (size_t)row * (I / 32) + q, (uint8_t)code);
            }
          }
        }
        if (signal) pending = -1;
      }
      pending = a;
      cur = nxt;
    }
    if (pending >= 0) {       // the last unit's arrival
      const long long t_w0 = st ? wall_clock() : 0;
      wait_mem();
      __syncthreads();
      if (tid == 0) __hip_atomic_fetch_add(&l1_done[pending], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (st) l1_sig_ticks += wall_clock() - t_w0;
    }
  }
  if (st && tid == 0) st[2] = wall_clock();

  // ================================================================ L2 phase
  {
    int* claim = p.counters + CNT_CLAIM + 1;
    const uint8_t* w2v = p.w2v;
    const uint32_t* w2s = p.w2s;
    auto load2 = [w2v, w2s, lane, wv](int v, U4 (&w)[KT2], uint32_t (&sw)[KG2]) {
      const int a = v / NBL2, b = v % NBL2;
      const size_t blk = (size_t)s.act[a] * NB2 + NW * b + wv;
      const uint8_t* bw = w2v + blk * KT2 * 1024 + lane * 16;
#pragma unroll
      for (int k = 0; k < KT2; ++k) w[k] = ld_stream(bw + k * 1024);
#pragma unroll
      for (int g = 0; g < KG2; ++g) sw[g] = __builtin_nontemporal_load(w2s + (blk * KG2 + g) * 64 + lane);
    };
    __syncthreads();
    if (tid == 0) s.claimv[par] = __hip_atomic_fetch_add(claim, CH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    int cur = __builtin_amdgcn_readfirstlane(s.claimv[par]);
    par ^= 1;
    int top = cur + CH < U2 ? cur + CH : U2;
    int ahead = U2;
    if (tid == 0 && cur + CH < U2) ahead = __hip_atomic_fetch_add(claim, CH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    U4 wt[KT2];
    uint32_t sd[KG2];
    if (cur < U2) load2(cur, wt, sd);
    int ready = -1;           // active expert whose L1 arrival has been observed
    int pv = -1;              // previous unit; its combine arrivals are not sent yet
    // Combine: per (token, row block) arrival counter; the arrival that completes it sums the
    // token's slots in slot order and writes y. The arrivals of unit `v` are two per-thread
    // atomics at most (an expert holds <= 2 FT routes), issued before the next unit's loads
    // and consumed after them.
    static_assert(FUSED_MAX_ROUTES <= 2 * FT, "combine arrivals: two routes per thread at most");
    auto arrive = [comb, tid](int v, int topk, int& o0, int& o1) {
      const int a = v / NBL2, b = v % NBL2;
      const int r0 = s.aoff[a], n = s.aoff[a + 1] - r0;
      o0 = o1 = -1;
      if (tid < n)
        o0 = __hip_atomic_fetch_add(&comb[(s.routes[r0 + tid] / topk) * NBL2 + b], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (tid + FT < n)
        o1 = __hip_atomic_fetch_add(&comb[(s.routes[r0 + tid + FT] / topk) * NBL2 + b], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    auto finish = [&](int v, int o0, int o1) {
      const int a = v / NBL2, b = v % NBL2;
      const int r0 = s.aoff[a], n = s.aoff[a + 1] - r0;
      if (tid < n) {
        const int tk = s.routes[r0 + tid] / p.topk;
        if (o0 == s.nslot[tk] - 1) s.last[atomicAdd(&s.nlast, 1)] = tk;
      }
      if (tid + FT < n) {
        const int tk = s.routes[r0 + tid + FT] / p.topk;
        if (o1 == s.nslot[tk] - 1) s.last[atomicAdd(&s.nlast, 1)] = tk;
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
      if (tid == 0) s.nlast = 0;   // the next appends follow at least one more barrier
    };
    while (cur < U2) {
      const int a = cur / NBL2, b = cur % NBL2;
      const int r0 = s.aoff[a], n = s.aoff[a + 1] - r0;
      int nxt = cur + 1;
      if (nxt >= top) {
        if (tid == 0) s.claimv[par] = ahead;
        __syncthreads();
        nxt = __builtin_amdgcn_readfirstlane(s.claimv[par]);
        par ^= 1;
        top = nxt + CH < U2 ? nxt + CH : U2;
        if (tid == 0) ahead = nxt + CH < U2 ? __hip_atomic_fetch_add(claim, CH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : U2;
      }
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
        after_mfma(acc);
        const bool send = s0 == 0 && pv >= 0;
        int o0 = -1, o1 = -1;
        if (send) {
          wait_mem();                                  // the previous unit's route outputs landed
          __syncthreads();
          arrive(pv, p.topk, o0, o1);
        }
        if (s0 + 16 >= n && nxt < U2) load2(nxt, wt, sd);
        __builtin_amdgcn_sched_barrier(0);
        if (s0 + c < n) {
          float* dst = p.partials + (size_t)s.routes[r0 + s0 + c] * H + (NW * b + wv) * 16 + 4 * kq;
          st_agent64(dst, (uint64_t)__float_as_uint(acc[0]) | ((uint64_t)__float_as_uint(acc[1]) << 32));
          st_agent64(dst + 2, (uint64_t)__float_as_uint(acc[2]) | ((uint64_t)__float_as_uint(acc[3]) << 32));
        }
        if (send) {
          finish(pv, o0, o1);
          pv = -1;
        }
      }
      pv = cur;
      cur = nxt;
    }
    if (pv >= 0) {            // the last unit's arrivals
      wait_mem();
      __syncthreads();
      int o0, o1;
      arrive(pv, p.topk, o0, o1);
      finish(pv, o0, o1);
    }
  }

  // ---------------------------------------------------------------- teardown
  if (st && tid == 0) {
    st[4] = wall_clock();
    st[6] = l1_load_ticks;
    st[7] = l1_sig_ticks;
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
