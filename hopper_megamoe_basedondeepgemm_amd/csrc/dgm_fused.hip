// One persistent kernel for one GPU's share of the MegaMoE layer (gfx950):
// [top-k] -> dispatch -> L1 (gate/up, SwiGLU, requant) -> L2 (down) -> top-k combine.
//
// Schedule. The grid is what the device keeps resident at once (one 8-wave workgroup per
// CU). Work units: L1 units (active expert a, 64 intermediate features), then L2 units
// (active expert a, 256 output rows). Workgroup g starts with units g and G + g of each
// phase; later units are claimed one at a time from one atomic counter per phase, one unit
// before they are needed (a shared counter at kernel start would serialize every
// workgroup). A workgroup moves to L2 only when it ran out of L1 units; L1 units never wait,
// so an L2 unit's wait (on the L1 arrival counter of its expert) is only on units held by
// running workgroups. Every wait is a bounded spin; on expiry the kernel raises an error flag
// and carries on, so every wave always reaches the end. An item is a unit's share of one
// 16-route slab (units of experts with more than 16 routes have several items).
//
// Streaming. Each wave streams its weight rows through a ring of tile registers (one 1 KB
// coalesced non-temporal load per 16x128 tile): right after the matrix-core op on a tile it
// issues the load of the tile KR positions later, continuing into the next item, so HBM reads
// never pause at item boundaries. The next item's activation slab is loaded into registers
// before the tiles it must not queue behind and stored to LDS between the epilogue's
// barriers. Loads whose values are only combined later (claims, slab bytes) are kept as
// returned: consuming them early would wait for every weight tile issued before them.
//
// Dispatch. Every workgroup derives the same pool table in LDS (a few hundred routes): under
// select_in_mega it first selects the top-k from the router logits itself; then per-expert
// counts, the active-expert list (ascending) and the canonical pool order (token asc, slot
// asc). Workgroup 0 also publishes the routing and the pool, the recv stats and the zero rows
// of tokens without a local route.
//
// Hand-offs between workgroups go through HBM with agent-coherent accesses only: the data
// (intermediate codes and scales, bf16 route outputs) is written with relaxed agent-scope
// atomic stores (write-through, "sc1") and read with agent-scope atomic loads, and the
// producer's stores have completed (s_waitcnt) before it bumps an arrival counter. No
// agent-scope release/acquire fence is used: on this GPU those write back / invalidate a
// whole L2 and cost tens of microseconds each.
//   L1 unit -> mid codes + scales of its 64 features; one item later l1_done[a] += 1
//   L2 item -> bf16 route outputs; one item later comb[t][b] += 1 per route and 128-row block
//   combine -> per (token, block): wait comb == the token's local routes, sum the routes in
//   slot order (fp32) -> bf16 y
// Counters come in two sets picked by a parity word: a launch uses one set and clears the other
// (after its dispatch) for the next launch; the workgroup that counts itself last at entry flips
// the parity at its end. No workgroup clears or waits on counters at the end of a launch.
#include "dgm_common.hpp"
#include "dgm_abi_internal.hpp"
#include "dgm_fused.hpp"
#include "dgm_frontend.hpp"

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

// all but the N youngest of this wave's vector-memory operations have completed (they
// complete in issue order)
template <int N>
DGM_DEV void wait_vm_le() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Streaming tile load issued only after the matrix-core op that produced `acc` (a register
// dependency, so the compiler cannot hoist it above that op and needs no second register
// set for the tile it replaces).
DGM_DEV U4 ld_stream_after(const uint8_t* base, int off, v4f acc) {
  asm("" : "+v"(off) : "v"(acc[0]));
  return ld_stream(base + off);
}
DGM_DEV U4 ld_stream_after(const uint8_t* base, int off, v4i acc) {
  asm("" : "+v"(off) : "v"(acc[0]));
  return ld_stream(base + off);
}
DGM_DEV uint32_t ld_stream32(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}
DGM_DEV uint32_t ld_stream32_after(const uint8_t* base, int off, v4f acc) {
  asm("" : "+v"(off) : "v"(acc[0]));
  return ld_stream32(base + off);
}
// NVFP4 weight operand of op j: the lane's eight E2M1 codes (dword w) -> f16, times the
// E4M3 block scale sv (exact in f16)
DGM_DEV v8h nvfp4_operand(uint32_t w, _Float16 sv) {
  const v2h ss = {sv, sv};
  const v2h h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0) * ss;
  const v2h h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1) * ss;
  const v2h h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2) * ss;
  const v2h h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3) * ss;
  return __builtin_shufflevector(__builtin_shufflevector(h0, h1, 0, 1, 2, 3), __builtin_shufflevector(h2, h3, 0, 1, 2, 3),
                                 0, 1, 2, 3, 4, 5, 6, 7);
}
DGM_DEV v8h as_v8h(U4 u) { return __builtin_bit_cast(v8h, u); }
// one NVFP4 K-tile (four f16 ops): weight codes w, the lane's scale dword sw (byte j = op j's
// block scale), B operands b[4]
DGM_DEV v4f nvfp4_tile(U4 w, uint32_t sw, const U4 (&b)[4], v4f acc) {
  const v2h s01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(sw, 1.0f, false);
  const v2h s23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(sw, 1.0f, true);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(nvfp4_operand(w.x, s01.x), as_v8h(b[0]), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(nvfp4_operand(w.y, s01.y), as_v8h(b[1]), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(nvfp4_operand(w.z, s23.x), as_v8h(b[2]), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(nvfp4_operand(w.w, s23.y), as_v8h(b[3]), acc, 0, 0, 0);
  return acc;
}
DGM_DEV void st_agent32(void* p, uint32_t v) {
  __hip_atomic_store((uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// QoQ: the zero point and group scale of the four accumulator rows 4 kq .. +3 of K-tile u
// (one meta dword per lane group), from the wave's per-item meta registers (dword 4 u + kq of
// the item's meta is held by lane (4 u + kq) % 64 in register (4 u + kq) / 64)
template <int U>
DGM_DEV uint32_t qoq_meta(const uint32_t* md, int kq) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(((4 * U + kq) & 63) * 4, (int)md[U >> 4]);
}
DGM_DEV v4i lo4(v8i v) { return __builtin_shufflevector(v, v, 0, 1, 2, 3); }
// acc += a * b on the low 24 bits of a and b (full-rate VALU). Written out because the
// compiler, seeing only the low 24 bits of a product demanded, rewrites a 24-bit multiply
// into a quarter-rate 32-bit one. The operands are VALU results and the destination is the
// accumulator's own register (never a matrix-core operand), so no matrix-core hazard applies.
DGM_DEV void mad_i24_acc(int& acc, int a, int b) {
  asm("v_mad_i32_i24 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}
// Compiler-only ordering point: the matrix-core ops that use `b` come after the VALU work that
// produced `q` (otherwise the scheduler issues every op of a loop first and keeps all their
// results live until the end)
template <class T>
DGM_DEV void after_values(v8i& b, T q) { asm("" : "+v"(b) : "v"(q)); }
DGM_DEV v4i hi4(v8i v) { return __builtin_shufflevector(v, v, 4, 5, 6, 7); }

constexpr int FT = 512;        // threads per workgroup (8 waves)
constexpr int NW = FT / 64;

template <int KT1, int KT2, int ACT>
struct FusedSmem {
  // U4 per lane per K-tile: E2M1 (32 codes), E4M3 / int8 (two 16-byte halves), NVFP4 as f16
  // (four ops of eight halves)
  static constexpr int BV = ACT == DGM_ACT_MXFP4 ? 1 : ACT == DGM_ACT_NVFP4 ? 4 : 2;
  static constexpr int KTM = KT1 > KT2 ? KT1 : KT2;
  int exp_of_route[FUSED_MAX_ROUTES];
  float route_w[FUSED_MAX_ROUTES];     // routing weight of each route
  int routes[FUSED_MAX_ROUTES];
  int prow[FUSED_MAX_ROUTES];          // per pool row: its route's row in `partials` (slot * part_rows + token)
  static constexpr int PT = ACT == DGM_ACT_NVFP4 ? 1 : FUSED_MAX_ROUTES;
  int ptok[PT];                        // per pool row: its token (not NVFP4)
  float pw[PT];                        // per pool row: its routing weight (not NVFP4)
  int ytok[FUSED_MAX_ROUTES];          // per pool row: its token when that token has no other local
                                       // route (the L2 unit writes y itself), else -1
  int act[FUSED_MAX_LOCAL];
  int aoff[FUSED_MAX_LOCAL + 1];
  int nslot[FUSED_MAX_TOKENS];
  int wsum[NW][2];
  int meta[4];
  uint32_t amask[FUSED_MAX_LOCAL / 32];   // (early streaming) active local experts, bit e
  union {
    struct {                           // dispatch only
      int cnt[FUSED_MAX_LOCAL];
      int eoff[FUSED_MAX_LOCAL];
    };
    U4 bst[KTM][64][BV];               // B slab in matrix-core fragment order
  };
  uint32_t bsc[(KTM + 3) / 4][64];     // its E8M0 scales, 4 K-tiles per dword
  // QoQ slab extras. Input rows (L1): per column and K-tile the sum of the column's int8
  // values (for the zero-point term) and per column the token's scale. Intermediate rows (L2):
  // per column and K-tile (chunks h = 0, 1 of 64 K with scales sm_h and value sums X_h) the
  // promote coefficients {sm_0, sm_1 / 16, 8 X_1 sm_1, -(X_0 sm_0 + X_1 sm_1)}.
  static constexpr int QX = ACT == DGM_ACT_QOQ ? 16 : 1;
  alignas(16) int xsum[QX][ACT == DGM_ACT_QOQ ? KT1 : 1];
  float xsc[QX];
  alignas(16) float4 qc[QX][ACT == DGM_ACT_QOQ ? KT2 : 1];
  // NVFP4: per local expert the L1 / L2 output scales (1 when not given)
  float gsl[2][ACT == DGM_ACT_NVFP4 ? FUSED_MAX_LOCAL : 1];
  // FP8F128 input rows (L1): the token's fp32 activation scale of each K-tile [K-tile][column]
  float xf[ACT == DGM_ACT_FP8F128 ? KT1 : 1][16];
  float slab_w[16];                    // routing weights of the staged slab's routes (L1)
  float upv[4][64][4];                 // L1: up-projection sums for the gate waves [pair][lane][i]
  // L1 half units (TAIL form): per block pair of the half, the K-half-1 sums of its gate and up
  // blocks [pair & 1][gate, up][lane][i]
  static constexpr int HS = (ACT == DGM_ACT_MXFP4 || ACT == DGM_ACT_MXFP8) && KT1 == 24 ? 2 : 1;
  float hsum[HS][2][64][4];
  float amax[4][16];                   // L1: per-token amax of each pair's 16 features
  int claimv[3];            // [0] the claim ahead, [1] prefetch decision, [2] L2: a complete expert
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

// The pool table of R <= 64 routes. Keys = local expert << 16 | route id (routes of other
// ranks sort last), one per lane; sorted, they are the canonical pool order (expert asc, route
// asc = token asc, slot asc), and expert boundaries give the active list, offsets and counts.
// Each key's rank is counted against every key (broadcast by readlane): wave w counts against
// keys 64 / NW * w .. +64 / NW - 1 into part[w][lane] (route_key_ranks, every wave), then one
// wave adds the parts, scatters the keys to their ranks and reads them back in order
// (wave_dispatch). Writes s.routes, s.act, s.aoff, s.meta[0..1], s.cnt (of active experts; the
// rest must be zero) and s.nslot (must be zero).
DGM_DEV uint32_t route_key(int e0, int lane) {
  return ((e0 < 0 ? 0xffffu : (uint32_t)e0) << 16) | (uint32_t)lane;
}

// Position of the n-th set bit (from 0, ascending) of the NWD-word bit string m, or -1 when it
// has fewer than n + 1; the same (scalar) value in every lane of the calling wave. Word i sits
// in lane i; an inclusive prefix of the words' bit counts finds the word, then its lower bits
// are dropped one at a time.
template <int NWD>
DGM_DEV int nth_set_bit(const uint32_t* m, int n, int lane) {
  static_assert(NWD <= 64, "one word per lane");
  const uint32_t w = lane < NWD ? m[lane] : 0u;
  const int cnt = __popc(w);
  int inc = cnt;
#pragma unroll
  for (int off = 1; off < NWD; off <<= 1) {
    const int o = __shfl_up(inc, off);
    if (lane >= off) inc += o;
  }
  const uint64_t hit = __ballot(inc > n && inc - cnt <= n);
  if (hit == 0) return -1;
  const int L = __ffsll((unsigned long long)hit) - 1;
  uint32_t word = (uint32_t)__shfl((int)w, L);
  const int k = n - (__shfl(inc, L) - __shfl(cnt, L));
  for (int i = 0; i < k; ++i) word &= word - 1;
  return __builtin_amdgcn_readfirstlane(32 * L + __ffs((int)word) - 1);
}
template <class S>
DGM_DEV void route_key_ranks(S& s, int R, int lane, int wv, int* part) {
  const uint32_t key = route_key(lane < R ? s.exp_of_route[lane] : -1, lane);
  constexpr int QW = 64 / NW;
  static_assert(64 % NW == 0, "keys per wave");
  int rk = 0;
#pragma unroll
  for (int j = 0; j < QW; ++j) rk += (uint32_t)__builtin_amdgcn_readlane((int)key, QW * wv + j) < key ? 1 : 0;
  part[wv * 64 + lane] = rk;
}
// r / d for 0 <= r < 1024 and 1 <= d <= 16 as a multiply and a shift: with m = ceil(2^20 / d),
// r m / 2^20 exceeds r / d by less than 2^-10 < 1 / d, so the floors agree (also checked for
// every such r and d). A route's token is route / top-k; the generic integer division it
// replaces is a long dependent sequence (M=16 and NVFP4 layer calls: 0.2-1.4 us faster).
DGM_DEV uint32_t div_magic(int d) { return (0x100000u + (uint32_t)d - 1u) / (uint32_t)d; }
DGM_DEV int div_small(int r, uint32_t m) { return (int)(((uint32_t)r * m) >> 20); }
template <class S>
DGM_DEV void wave_dispatch(S& s, int R, uint32_t tkm, int lane, const int* part) {
  uint32_t key = route_key(lane < R ? s.exp_of_route[lane] : -1, lane);
  int rank = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) rank += part[w * 64 + lane];
  // (the route-table slots double as the sort buffer: keys of the routes are unique)
  s.routes[rank] = (int)key;
  key = (uint32_t)s.routes[lane];
  const uint32_t e = key >> 16;
  const bool valid = e != 0xffffu;
  const uint32_t prev = (uint32_t)__shfl_up((int)key, 1);
  const bool first = valid && (lane == 0 || (prev >> 16) != e);
  const uint64_t fb = __ballot(first), vb = __ballot(valid);
  const int a = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(fb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)fb, 0u));
  if (valid) {
    const int r = (int)(key & 0xffffu);
    s.routes[lane] = r;
    atomicAdd(&s.nslot[div_small(r, tkm)], 1);
  }
  if (first) {
    s.act[a] = (int)e;
    s.aoff[a] = lane;
  }
  const int base = __popcll(fb), total = __popcll(vb);
  if (lane == 0) {
    s.aoff[base] = total;
    s.meta[0] = base;
    s.meta[1] = total;
  }
  // per active expert: count = next offset - offset (the wave's LDS stores above come first)
  for (int i = lane; i < base; i += 64) s.cnt[s.act[i]] = s.aoff[i + 1] - s.aoff[i];
}

// A bounded wait expired: the error counter is set (it stays set until the caller clears it),
// and so is the caller's host-visible word when there is one, which the host reads without
// synchronising (vector stores; the host word with system scope).
DGM_DEV void raise_error(int* err, int* herr) {
  __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (herr) __hip_atomic_store(herr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

DGM_DEV bool spin_until(const int* p, int target, int limit, int* err, int* herr) {
  int n = 0;
  while (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
    if (++n > limit) {
      raise_error(err, herr);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}
// The same wait with two reads in flight: each read is issued before the previous one is tested
// (two reads per round, in alternating registers: a register copy would wait for the newer
// read), so a change is seen about half a memory round trip sooner.
DGM_DEV bool spin_until2(const int* p, int target, int limit, int* err, int* herr) {
  int v0 = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int n = 0;; n += 2) {
    const int v1 = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (v0 >= target) return true;
    __builtin_amdgcn_s_sleep(1);
    v0 = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (v1 >= target) return true;
    if (n > limit) {
      raise_error(err, herr);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Stage the B slab (16 columns = rows row_of(c) of a [rows, KT*128] activation matrix with
// row_bytes and per-32 E8M0 scales) into LDS in fragment order. Column c >= n is zero.
// COHERENT: the rows were written by other workgroups of this launch (agent-scope loads).
template <int KT, int ACT, bool COHERENT, class S, class RowOf>
DGM_DEV void stage_slab(S& s, const uint8_t* __restrict__ src, const uint8_t* __restrict__ ssrc,
                        int row_bytes, int n, RowOf row_of) {
  // (the thread index made opaque: the addresses below are computed here, not hoisted out of
  // the item loop and kept live, or spilled, across it)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
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

// A B slab held in registers between its loads and its LDS stores (the loads are issued
// early, ahead of the weight tiles they must not queue behind). Same fragments as stage_slab.
// Values are kept exactly as loaded (vectors, or the 64-bit halves of agent-scope loads) and
// only combined or masked at the store: doing either earlier would wait for every older load.
// Every lane loads (from row 0 when it has no row), so no loaded value crosses a divergent
// branch.
template <int KT, int ACT, bool COHERENT, bool MIDL = COHERENT>
struct SlabRegs {
  static constexpr int FR = (KT * 64 + FT - 1) / FT;
  v4u v0[FR], v1[FR];            // non-coherent fragments
  uint64_t h[FR][4];             // coherent fragments: 64-bit halves (K bytes 0-15, 64-79)
  uint32_t sb[4];                // scale dwords of K-tiles 4g .. 4g+3 (byte l/16 is this lane's)
  uint32_t ok;                   // bit j: fragment j holds a real row; bit 8 + j: scale byte j
  float fsc;                     // QoQ input rows: the token's scale (threads 0-15)
  uint64_t sc2[FR];              // QoQ intermediate rows: fragment j's two chunk scales (lanes 0-15)
  uint32_t s16[FR];              // NVFP4: the dword holding fragment j's two 16-block scales
  float w;
};

// COHERENT: agent-scope loads (rows written by other workgroups of this launch); MIDL: the
// intermediate rows' layout (QoQ: per-chunk scales) rather than the input activations'.
template <int KT, int ACT, bool COHERENT, bool MIDL, class RowOf, class WeightOf>
DGM_DEV void slab_load(SlabRegs<KT, ACT, COHERENT, MIDL>& r, const uint8_t* __restrict__ src, const uint8_t* __restrict__ ssrc,
                       int row_bytes, int n, RowOf row_of, WeightOf weight_of) {
  const int tid = threadIdx.x;
  uint32_t ok = 0;
  // MASK: only the lanes whose column holds a real row load (the slab store zeroes the others):
  // with one route per expert, 15 of 16 columns are empty, and their loads (of row 0) kept the
  // memory pipeline busy for ~0.7 us at each workgroup's first slab (A-MXFP, FP8F128: 0.4-1.7
  // us per layer call). QoQ and NVFP4 keep the unconditional loads: with the branches their
  // kernels spill more registers (5 and 9 values) and measured slower.
  constexpr bool MASK = ACT == DGM_ACT_MXFP4 || ACT == DGM_ACT_MXFP8 || ACT == DGM_ACT_FP8F128;
#pragma unroll
  for (int j = 0; j < SlabRegs<KT, ACT, COHERENT, MIDL>::FR; ++j) {
    const int f = tid + j * FT;
    const int l = f & 63, c = l & 15;
    const bool have = f < KT * 64 && c < n;
    ok |= have ? 1u << j : 0u;
    const int kt = have ? f >> 6 : 0;
    const size_t rr = have ? (size_t)row_of(c) : 0;
    // E2M1 (MXFP4, NVFP4): 16 bytes at K = 32 g; E4M3 / int8: K = 16 g .. +16 and
    // K = 64 + 16 g .. +16 (g = l / 16)
    constexpr bool FP4 = ACT == DGM_ACT_MXFP4 || ACT == DGM_ACT_NVFP4;
    const uint8_t* q = FP4 ? src + rr * row_bytes + kt * 64 + (l >> 4) * 16
                           : src + rr * row_bytes + kt * 128 + (l >> 4) * 16;
    if (COHERENT) {
      r.h[j][0] = r.h[j][1] = r.h[j][2] = r.h[j][3] = 0;
      if (!MASK || have) {
        r.h[j][0] = ld_agent64(q);
        r.h[j][1] = ld_agent64(q + 8);
        if (!FP4) {
          r.h[j][2] = ld_agent64(q + 64);
          r.h[j][3] = ld_agent64(q + 72);
        }
      }
    } else {
      r.v0[j] = r.v1[j] = v4u{0u, 0u, 0u, 0u};
      if (!MASK || have) {
        r.v0[j] = *reinterpret_cast<const v4u*>(q);
        if (!FP4) r.v1[j] = *reinterpret_cast<const v4u*>(q + 64);
      }
    }
    if constexpr (ACT == DGM_ACT_NVFP4) {
      // the two E4M3 scales of the fragment (16-blocks 8 kt + 2 g, +1; row pitch KT * 8 bytes),
      // as the aligned dword holding them
      const uint32_t* sq = reinterpret_cast<const uint32_t*>(ssrc + rr * (KT * 8) + ((8 * kt + 2 * (l >> 4)) & ~3));
      r.s16[j] = COHERENT ? __hip_atomic_load(sq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *sq;
    }
  }
  constexpr int KG = (KT + 3) / 4;
  static_assert(KG * 64 <= FT, "one scale word per thread");
  if constexpr (ACT == DGM_ACT_NVFP4) {
    // (scales loaded with the fragments)
  } else if constexpr (ACT == DGM_ACT_QOQ) {
    if (MIDL) {
      // intermediate rows: fp32 scale per 64-K chunk (row pitch KT * 8 bytes); lane l < 16 of
      // fragment j (K-tile kt, column l) loads the two chunk scales of its tile
#pragma unroll
      for (int j = 0; j < SlabRegs<KT, ACT, COHERENT, MIDL>::FR; ++j) {
        const int f = tid + j * FT;
        const bool have = (ok >> j) & 1u && (f & 63) < 16;
        const size_t rr = have ? (size_t)row_of(f & 15) : 0;
        r.sc2[j] = ld_agent64(ssrc + rr * (KT * 8) + (have ? (f >> 6) * 8 : 0));
      }
    } else {
      // input rows: one fp32 scale per token (row pitch KT * 4 bytes: the reference's
      // [M, K/128] copies), thread c < 16
      const int c = tid & 15;
      const bool have = tid < 16 && c < n;
      const size_t rr = have ? (size_t)row_of(c) : 0;
      const float* fq = reinterpret_cast<const float*>(ssrc + rr * (KT * 4));
      r.fsc = COHERENT ? __hip_atomic_load(fq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *fq;
      ok |= have ? 1u << 8 : 0u;
    }
  } else {
    const int g = tid >> 6, l = tid & 63, c = l & 15;
    const bool have = tid < KG * 64 && c < n;
    const size_t rr = have ? (size_t)row_of(c) : 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kt = 4 * g + j;
      const bool hb = have && kt < KT;
      ok |= hb ? 1u << (8 + j) : 0u;
      const uint32_t* q = reinterpret_cast<const uint32_t*>(ssrc + (hb ? rr * (KT * 4) + kt * 4 : 0));
      r.sb[j] = 0u;
      if (!MASK || hb) r.sb[j] = COHERENT ? __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *q;
    }
  }
  r.ok = ok;
  r.w = tid < n && tid < 16 ? weight_of(tid) : 0.f;
}

template <int KT, int ACT, bool COHERENT, bool MIDL, class S>
DGM_DEV void slab_store(S& s, const SlabRegs<KT, ACT, COHERENT, MIDL>& r) {
  // (the thread index is made opaque so that the LDS addresses below are recomputed here
  // rather than hoisted out of the work loop and kept live, or spilled, across it)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const v4u z = {0u, 0u, 0u, 0u};
  if constexpr (ACT == DGM_ACT_NVFP4) {
    // fragment (K-tile kt, column c, 32-K chunk g') -> f16 operand of op g' for the four lane
    // groups q (K = 32 g' + 8 q .. +8): E2M1 -> f16 exactly, times the E4M3 block scale (the
    // products are exact in f16)
#pragma unroll
    for (int j = 0; j < SlabRegs<KT, ACT, COHERENT, MIDL>::FR; ++j) {
      const int f = tid + j * FT;
      if (f < KT * 64) {
        const bool have = (r.ok >> j) & 1u;
        const int kt = f >> 6, l = f & 63, c = l & 15, gq = l >> 4;
        uint32_t w[4];
        if (COHERENT) {
          w[0] = (uint32_t)r.h[j][0];
          w[1] = (uint32_t)(r.h[j][0] >> 32);
          w[2] = (uint32_t)r.h[j][1];
          w[3] = (uint32_t)(r.h[j][1] >> 32);
        } else {
          w[0] = r.v0[j].x;
          w[1] = r.v0[j].y;
          w[2] = r.v0[j].z;
          w[3] = r.v0[j].w;
        }
        const uint32_t sc2 = r.s16[j] >> ((gq & 1) * 16);      // byte 0: block 2 g', byte 1: 2 g' + 1
        const v2h s01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(sc2, 1.0f, false);
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const _Float16 sv = qd < 2 ? s01.x : s01.y;
          const v2h ss = {sv, sv};
          const v2h h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w[qd], 1.0f, 0) * ss;
          const v2h h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w[qd], 1.0f, 1) * ss;
          const v2h h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w[qd], 1.0f, 2) * ss;
          const v2h h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w[qd], 1.0f, 3) * ss;
          const v4u o = {__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1),
                         __builtin_bit_cast(uint32_t, h2), __builtin_bit_cast(uint32_t, h3)};
          *reinterpret_cast<v4u*>(&s.bst[kt][(qd << 4) | c][gq]) = have ? o : z;
        }
      }
    }
  } else {
#pragma unroll
  for (int j = 0; j < SlabRegs<KT, ACT, COHERENT, MIDL>::FR; ++j) {
    const int f = tid + j * FT;
    if (f < KT * 64) {
      const bool have = (r.ok >> j) & 1u;
      v4u* dst = reinterpret_cast<v4u*>(&s.bst[f >> 6][f & 63][0]);
      if (COHERENT) {
        const uint64_t* h = r.h[j];
        dst[0] = have ? v4u{(uint32_t)h[0], (uint32_t)(h[0] >> 32), (uint32_t)h[1], (uint32_t)(h[1] >> 32)} : z;
        if (ACT != DGM_ACT_MXFP4)
          dst[S::BV - 1] = have ? v4u{(uint32_t)h[2], (uint32_t)(h[2] >> 32), (uint32_t)h[3], (uint32_t)(h[3] >> 32)} : z;
      } else {
        dst[0] = have ? r.v0[j] : z;
        if (ACT != DGM_ACT_MXFP4) dst[S::BV - 1] = have ? r.v1[j] : z;
      }
    }
  }
  }
  constexpr int KG = (KT + 3) / 4;
  if constexpr (ACT == DGM_ACT_NVFP4) {
    // (no scale plane: the scales are folded into the f16 operands)
  } else if constexpr (ACT == DGM_ACT_QOQ) {
#pragma unroll
    for (int j = 0; j < SlabRegs<KT, ACT, COHERENT, MIDL>::FR; ++j) {
      const int f = tid + j * FT;
      if (f < KT * 64) {
        const bool have = (r.ok >> j) & 1u;
        const int kt = f >> 6, l = f & 63;
        int s0, s1;
        if (COHERENT) {
          const uint64_t* h = r.h[j];
          s0 = i8_sum16((uint32_t)h[0], (uint32_t)(h[0] >> 32), (uint32_t)h[1], (uint32_t)(h[1] >> 32));
          s1 = i8_sum16((uint32_t)h[2], (uint32_t)(h[2] >> 32), (uint32_t)h[3], (uint32_t)(h[3] >> 32));
        } else {
          s0 = i8_sum16(r.v0[j].x, r.v0[j].y, r.v0[j].z, r.v0[j].w);
          s1 = i8_sum16(r.v1[j].x, r.v1[j].y, r.v1[j].z, r.v1[j].w);
        }
        s0 = have ? s0 : 0;
        s1 = have ? s1 : 0;
        // (the branch is wave-uniform: a wave's 64 lanes are the 4 lane groups of one K-tile)
        s0 += __shfl_xor(s0, 16);
        s0 += __shfl_xor(s0, 32);
        s1 += __shfl_xor(s1, 16);
        s1 += __shfl_xor(s1, 32);
        if (l < 16) {
          if (MIDL) {            // intermediate rows (L2): the K-tile's promote coefficients
            const float sm0 = have ? __uint_as_float((uint32_t)r.sc2[j]) : 0.f;
            const float sm1 = have ? __uint_as_float((uint32_t)(r.sc2[j] >> 32)) : 0.f;
            const float x0 = (float)s0, x1 = (float)s1;
            s.qc[l][kt] = make_float4(sm0, sm1 * 0.0625f, 8.f * x1 * sm1, -fmaf(x1, sm1, x0 * sm0));
          } else {               // input rows (L1): per K-tile
            s.xsum[l][kt] = s0 + s1;
          }
        }
      }
    }
    if (!MIDL && tid < 16) s.xsc[tid] = (r.ok >> 8) & 1u ? r.fsc : 0.f;
  } else if constexpr (ACT == DGM_ACT_FP8F128) {
    // input rows with one fp32 scale per K-tile (the dword slab_load read for K-tile 4 g + j is
    // that scale: the same row pitch as four E8M0 bytes): per (K-tile, column) to s.xf; the
    // block-scaled op gets unit activation scales
    if (tid < KG * 64) {
      s.bsc[tid >> 6][tid & 63] = 0x7f7f7f7fu;
      if ((tid & 63) < 16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int kt = 4 * (tid >> 6) + j;
          if (kt < KT) s.xf[kt][tid & 63] = (r.ok >> (8 + j)) & 1u ? __uint_as_float(r.sb[j]) : 0.f;
        }
      }
    }
  } else if (tid < KG * 64) {
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w |= ((r.ok >> (8 + j)) & 1u ? (r.sb[j] >> (8 * ((tid & 63) >> 4))) & 0xffu : 127u) << (8 * j);
    s.bsc[tid >> 6][tid & 63] = w;
  }
  if (tid < 16) s.slab_w[tid] = r.w;
}

// Phase stamps (the reference's phase_stamps facility): per workgroup, 100 MHz wall clock at
// [0] entry, [1] dispatch table ready, [2] L1 units done, [3] first L1 arrival observed,
// [4] L2 units done, [5] exit; [6] wall ticks in L1 K loops (matrix-core ops, including the
// waits for their weight tiles), [7] wall ticks in L1 epilogues. With the in-kernel frontend,
// [6] and [7] are instead wall clock at: this workgroup's router and cast work done (its
// stores issued), and the grid-wide arrival passed.
DGM_DEV long long wall_clock() { return (long long)__builtin_amdgcn_s_memrealtime(); }

// FEIN: the router, token flags and activation cast run in this launch (p.fe_in); the rows they
// write are then read with agent-scope loads. Otherwise they were written by an earlier launch
// and are read with ordinary loads, which the L2 caches: every workgroup reads the same few
// activation rows at once, and L2-bypassing loads of them queue at the memory channels.
// EARLY (early weight streaming; small routed sets, one wave's dispatch): the workgroup's first
// L1 unit is found from a mask of the active experts as the top-k is read, and its slab, scales
// and tile ring are requested before the pool table is built. An opt-in form (debug bit 3), not
// the default: measured slower at every size it applies to, since each wave's dispatch code
// then waits behind the acceptance of its own tile requests, and the ring's second half is
// requested no earlier.
// The kernel's forms (one instantiation each; the launch picks one): plain, FEIN, and the
// opt-in EARLY and TAIL (A-MXFP at H = 3072, small routed sets: the last round of L1 units as
// half units).
constexpr int FORM_PLAIN = 0, FORM_FEIN = 1, FORM_EARLY = 2, FORM_TAIL = 3;
template <int KT1, int KT2, int ACT, int FORM>
__global__ void __launch_bounds__(FT) k_megamoe(FusedParams p) {
  constexpr bool FEIN = FORM == FORM_FEIN, EARLY = FORM == FORM_EARLY, TAIL = FORM == FORM_TAIL;
  using Smem = FusedSmem<KT1, KT2, ACT>;
  __shared__ Smem s;
  constexpr int FB = ACT == DGM_ACT_MXFP4 ? 4 : 0;        // B operand format
  constexpr int KH = KT1 / 2;                               // L1 K-tiles per wave (K halves)
  constexpr int KG1 = (KT1 + 3) / 4, KG2 = (KT2 + 3) / 4;
  constexpr int H = KT1 * 128, I = KT2 * 128;
  constexpr bool FP4A = ACT == DGM_ACT_MXFP4 || ACT == DGM_ACT_NVFP4;   // E2M1 activations
  // FP8F128: E4M3 input rows with an fp32 scale per K-tile (each K-tile's product promoted by
  // it); the intermediate is MXFP8's (E4M3, E8M0 per 32), so the L2 phase runs as MXFP8's
  constexpr bool F128 = ACT == DGM_ACT_FP8F128;
  constexpr int ACT2 = F128 ? DGM_ACT_MXFP8 : ACT;
  constexpr int XB = FP4A ? H / 2 : H;     // activation row bytes
  constexpr int MB = FP4A ? I / 2 : I;     // intermediate row bytes
  constexpr int QN1 = I / 64, NB1 = I / 8, NB2 = H / 16, NBL2 = H / (16 * NW);
  static_assert(I % 64 == 0, "L1 units are 64 intermediate features");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index: scalar
  // one field of each 64-byte line of the parameters, read at once: the scalar cache then holds
  // every line, and the later (lazy) parameter reads hit it instead of each paying a round trip
  static_assert(sizeof(FusedParams) <= 256, "four parameter lines");
  asm volatile("" ::"s"(p.w1v), "s"(p.x), "s"(p.partials), "s"(p.router_w));
  const int R = p.M * p.topk;
  const uint32_t tkm = div_magic(p.topk);     // route -> token: div_small(route, tkm)
  // this launch's counter set (the other one is cleared after the dispatch); each workgroup
  // counts itself once it has read the parity: the one that counts last hands the next launch
  // the other set at its end (its count is read only then, long after it has returned).
  // The parity is requested here and taken into a scalar only where it is first needed: after
  // the routing loads (keys or top-k), or (FEIN) at the grid-wide arrival. Taken at once, its
  // round trip came before every later request of the prologue (the scalar copy and the
  // addresses derived from it were hoisted to the load); now the two round trips overlap.
  // (EARLY: counted behind the early requests, which then do not wait for it.)
  int parity_v = __hip_atomic_load(p.counters + CNT_PARITY, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int parity = 0;
  int* cset = nullptr;
  int* l1_done = nullptr;      // expert slot a: l1_done[a * CNT_LINE]
  int* comb = nullptr;         // pair i: comb[i * CNT_LINE]
  auto take_parity = [&]() __attribute__((always_inline)) {
    asm volatile("" : "+v"(parity_v));    // (the wait for the load is placed here)
    parity = __builtin_amdgcn_readfirstlane(parity_v) & 1;
    cset = p.counters + CNT_SET0 + parity * CNT_SET;
    l1_done = cset + CNT_L1;
    comb = cset + CNT_COMB;
  };
  int started = 0;
  auto count_start = [&]() __attribute__((always_inline)) {
    if (tid == 0) started = __hip_atomic_fetch_add(cset + CNT_STARTED, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  int* err = p.counters + CNT_ERROR;
  long long* st = (p.stamps && (int)blockIdx.x < p.stamp_rows) ? p.stamps + (size_t)blockIdx.x * 8 : nullptr;
  long long wait_ticks = 0, l1_load_ticks = 0, l1_sig_ticks = 0;
  if (st && tid == 0) st[0] = wall_clock();

  // ---------------------------------------------------------------- in-kernel frontend
  // (fe_in) router logits and keys and the activation cast, spread over the grid, with
  // write-through stores; then every workgroup waits until all have arrived (the grid is what
  // the device keeps resident, so all workgroups run at once)
  if constexpr (FEIN) {
    constexpr int J = H / 512;
    static_assert(H % 512 == 0, "in-kernel frontend: hidden % 512");
    // router (expert, 4-token group) pairs wave-major from the first wave of every workgroup,
    // cast waves from the last wave down, so both run side by side on all workgroups
    const int G = (int)gridDim.x;
    const int ngrp = (p.M + 3) / 4, npairs = p.E * ngrp;
    for (int pi = wv * G + (int)blockIdx.x; pi < npairs; pi += NW * G) {
      const int e = pi % p.E, tg = pi / p.E;
      router_wave<J, true>(p.hidden, p.router_w, p.M, p.E, e, 4 * tg, lane, p.logits,
                           const_cast<uint32_t*>(p.keys), (p.fe_flags & DGM_FE_ZERO_ROW_UNROUTED) != 0);
    }
    uint8_t* xq = const_cast<uint8_t*>(p.x);
    uint8_t* xsf = const_cast<uint8_t*>(p.xsf);
    const int cw = (NW - 1 - wv) * G + (int)blockIdx.x;          // cast wave index
    if constexpr (ACT == DGM_ACT_QOQ) {
      for (int t = cw; t < p.M; t += NW * G) cast_qoq_token<J, true>(p.hidden, t, lane, xq, xsf);
    } else if constexpr (ACT == DGM_ACT_NVFP4) {
      for (int64_t i = (int64_t)cw * 64 + lane; i < (int64_t)p.M * (H / 16) * 4; i += (int64_t)NW * G * 64)
        cast_lane_nvfp4<true>(p.hidden, i, xq, xsf);
    } else if constexpr (F128) {
      for (int64_t i = (int64_t)cw * 64 + lane; i < (int64_t)p.M * (H / 128) * 32; i += (int64_t)NW * G * 64)
        cast_lane_fp8f128<true>(p.hidden, i, xq, xsf);
    } else {
      for (int64_t i = (int64_t)cw * 64 + lane; i < (int64_t)p.M * (H / 32) * 8; i += (int64_t)NW * G * 64)
        cast_lane_mx<true>(p.hidden, ACT, i, xq, xsf);
    }
    if (st && tid == 0) st[6] = wall_clock();
    wait_mem();                  // this wave's stores have completed
    take_parity();
    __syncthreads();
    if (tid == 0)
      __hip_atomic_fetch_add(cset + CNT_GRID + ((int)blockIdx.x % GRID_SLOTS) * GRID_STRIDE, 1,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (wv == 0) {               // lane k < GRID_SLOTS watches slot k (bounded)
      const int k = lane % GRID_SLOTS;
      const int expect = ((int)gridDim.x - k + GRID_SLOTS - 1) / GRID_SLOTS;
      const int* gc = cset + CNT_GRID + k * GRID_STRIDE;
      for (int it = 0;; ++it) {
        const int v = __hip_atomic_load(gc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__all(v >= expect)) break;
        if (it > p.spin_limit) {
          if (lane == 0) raise_error(err, p.host_err);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    __syncthreads();
    if (st && tid == 0) st[7] = wall_clock();
    count_start();
  }

  // The tile ring (and the NVFP4 scale ring), shared by the two phases: the L1 phase's last
  // item rolls into the first L2 unit's tiles (unit v0), which then stream during the
  // L1 epilogue and the phase change instead of after it.
  constexpr int KR1 = KT1 % 12 == 0 ? 12 : KT1;
  constexpr int RING = KR1 > KT2 ? KR1 : KT2;
  constexpr bool HANDOFF = KR1 >= KT2;
  U4 wr[RING];
  uint32_t sr[ACT == DGM_ACT_NVFP4 ? RING : 1];
  // The L1 phase's wave w streams 16-row block pair pp = w & 3 (16 of a unit's 64 features),
  // tile gu = w >> 2 (gate or up) of local expert e's unit q: block l1_blk(e, q).
  const int pp = wv & 3, gu = wv >> 2;
  auto l1_blk = [pp, gu](int e, int q) __attribute__((always_inline)) {
    return (size_t)e * NB1 + 2 * (4 * q + pp) + gu;
  };
  // per-item L1 scale registers: MXFP: the E8M0 scale dwords of the wave's 16-row block; QoQ:
  // its meta dwords (4 per K-tile, spread over the lanes) and the s1 of the lane's 4 rows
  constexpr int MR1 = (4 * KT1 + 63) / 64;
  constexpr int SW1 = ACT == DGM_ACT_QOQ ? MR1 + 4 : ACT == DGM_ACT_NVFP4 ? 1 : KG1;
  auto load_scales_blk = [w1s = p.w1s, w1r = p.w1r, lane](size_t blk, uint32_t (&sw)[SW1]) __attribute__((always_inline)) {
    if constexpr (ACT == DGM_ACT_QOQ) {
      const uint32_t* mb = w1s + blk * KT1 * 4;
#pragma unroll
      for (int j = 0; j < MR1; ++j)
        sw[j] = __builtin_nontemporal_load(mb + (64 * j + lane < 4 * KT1 ? 64 * j + lane : 4 * KT1 - 1));
      const v4u r = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(w1r + blk * 16 + 4 * (lane >> 4)));
      sw[MR1] = r.x;
      sw[MR1 + 1] = r.y;
      sw[MR1 + 2] = r.z;
      sw[MR1 + 3] = r.w;
    } else if constexpr (ACT == DGM_ACT_NVFP4) {
      sw[0] = 0u;      // (the NVFP4 scales stream with the tiles)
    } else {
#pragma unroll
      for (int g = 0; g < KG1; ++g) sw[g] = __builtin_nontemporal_load(w1s + (blk * KG1 + g) * 64 + lane);
    }
  };
  uint32_t sd[SW1];                        // the current L1 item's scale registers
  SlabRegs<KT1, ACT, FEIN, false> pre;     // an L1 slab on its way to LDS

  // ---------------------------------------------------------------- dispatch (every WG)
  for (int t = tid; t < p.M; t += FT) s.nslot[t] = 0;
  if (EARLY && tid < FUSED_MAX_LOCAL / 32) s.amask[tid] = 0u;
  if (p.select) {
    // top-k from the frontend's keys, as the frontend would have done: the keys of TC tokens at
    // a time go through LDS (the slab area, unused until the L1 phase; one coalesced pass),
    // then one wave selects per token
    uint32_t* lg = reinterpret_cast<uint32_t*>(&s.bst[0][0][0]);
    const int TC = (int)(sizeof(s.bst) / 4) / p.E;
    for (int t0 = 0; t0 < p.M; t0 += TC) {
      const int tn = p.M - t0 < TC ? p.M - t0 : TC;
      // Rounds of SB values per thread, all loaded before any is written, so that a round costs
      // one memory round trip (a load-store loop would pay one per value). The in-kernel
      // frontend's keys (written in this launch) need agent-scope loads; the frontend
      // kernel's are read through the cache.
      const uint32_t* src = p.keys + (size_t)t0 * p.E;
      const int nv = tn * p.E;
      constexpr int SB = 8;
      for (int i0 = 0; i0 < nv; i0 += SB * FT) {
        uint32_t v[SB];
        if constexpr (FEIN) {
#pragma unroll
          for (int j = 0; j < SB; ++j)
            v[j] = __hip_atomic_load(src + min(i0 + j * FT + tid, nv - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
#pragma unroll
          for (int j = 0; j < SB; ++j) v[j] = src[min(i0 + j * FT + tid, nv - 1)];
        }
#pragma unroll
        for (int j = 0; j < SB; ++j)
          if (i0 + j * FT + tid < nv) lg[i0 + j * FT + tid] = v[j];
      }
      __syncthreads();
      for (int tt = wv; tt < tn; tt += NW) {
        const int t = t0 + tt;
        int idx;
        float wt;
        const uint32_t* row = lg + tt * p.E;
        select_topk_wave([row](int e) { return row[e]; }, p.E, p.topk, (p.fe_flags & DGM_FE_FORCE_BALANCED) != 0,
                         p.token_offset + t, lane, idx, wt);
        if (lane < p.topk) {
          const int r = t * p.topk + lane;
          const int l = idx - p.expert_begin;
          const bool mine = idx >= 0 && l >= 0 && l < p.E_local;
          s.exp_of_route[r] = mine ? l : -1;
          if (EARLY && mine) atomicOr(&s.amask[l >> 5], 1u << (l & 31));
          s.route_w[r] = wt;
          if (blockIdx.x == 0) {
            p.topk_idx[r] = idx;
            p.topk_w[r] = wt;
          }
        }
      }
      __syncthreads();
    }
  } else {
    if constexpr (EARLY) __syncthreads();     // (the mask is clear)
    for (int r = tid; r < R; r += FT) {
      int64_t g = p.topk_idx[r];
      int64_t l = g - p.expert_begin;
      const bool mine = g >= 0 && l >= 0 && l < p.E_local;
      s.exp_of_route[r] = mine ? (int)l : -1;
      if (EARLY && mine) atomicOr(&s.amask[l >> 5], 1u << (l & 31));
      s.route_w[r] = p.topk_w[r];
    }
  }
  for (int e = tid; e < p.E_local; e += FT) s.cnt[e] = 0;   // (shares LDS with the key staging)
  if constexpr (!FEIN) take_parity();      // (the routing loads above have returned)
  if constexpr (!EARLY && !FEIN) count_start();
  if constexpr (ACT == DGM_ACT_NVFP4) {
    for (int e = tid; e < p.E_local; e += FT) {
      s.gsl[0][e] = p.gs1 ? p.gs1[e] : 1.f;
      s.gsl[1][e] = p.gs2 ? p.gs2[e] : 1.f;
    }
  }
  __syncthreads();
  if constexpr (EARLY) {
    // The workgroup's first L1 unit is unit blockIdx.x: active expert blockIdx.x / QN1 in
    // ascending order, i.e. the mask's set bit of that index. Its first slab (the expert's
    // first 16 routes in route order, the pool's order within an expert), its scales and its
    // tile ring are requested now, in that order, and arrive while the pool table is built.
    // (R <= 64: the routes are one wave's lanes.)
    const int e0 = (p.phases & 1) ? nth_set_bit<FUSED_MAX_LOCAL / 32>(s.amask, (int)blockIdx.x / QN1, lane) : -1;
    // Nothing older is in flight from here on (the top-k loads were consumed above): without
    // this wait the compiler's wait counting, merging the paths with and without these
    // requests, put full waits (for the whole tile ring) into the dispatch's LDS code.
    wait_mem();
    if (e0 >= 0) {
      const uint64_t m = __ballot(lane < R && s.exp_of_route[lane] == e0);
      uint64_t mc = m;
      for (int i = 0; i < (lane & 15); ++i) mc &= mc - 1;     // drop the first c members
      const int rt = mc ? (int)__builtin_ctzll(mc) : 0;         // the route of slab column c
      slab_load<KT1, ACT, FEIN, false>(pre, p.x, p.xsf, XB, (int)__popcll(m), [rt, tkm](int) { return div_small(rt, tkm); },
                                       [rt](int) { return s.route_w[rt]; });
      const size_t blk = l1_blk(e0, (int)blockIdx.x % QN1);
      load_scales_blk(blk, sd);
      const uint8_t* b = p.w1v + blk * KT1 * 1024 + lane * 16;
#pragma unroll
      for (int k = 0; k < KR1; ++k) wr[k] = ld_stream(b + k * 1024);
    }
    count_start();
  }
  if (R <= 64) {
    // key ranks counted by every wave, then one wave sorts the routes (the other waves wait
    // at the barrier); the parts are staged in the L1 epilogue's up-sum buffer (unused until
    // then)
    int* part = reinterpret_cast<int*>(&s.upv[0][0][0]);
    static_assert(sizeof(s.upv) >= NW * 64 * sizeof(int), "rank parts");
    route_key_ranks(s, R, lane, wv, part);
    __syncthreads();
    if (wv == 0) wave_dispatch(s, R, tkm, lane, part);
    __syncthreads();
  } else {
    // counts, expert offsets, then each route placed in its expert's segment in arrival order
    // (LDS atomics; the staging area `tmp` is the L1 epilogue's up-sum buffer, unused until
    // then) and moved to its canonical position: its rank (route id) within the segment
    for (int r = tid; r < R; r += FT) {
      int e = s.exp_of_route[r];
      if (e >= 0) { atomicAdd(&s.cnt[e], 1); atomicAdd(&s.nslot[div_small(r, tkm)], 1); }
    }
    __syncthreads();
    scan_experts(s, p.E_local);
    int* tmp = reinterpret_cast<int*>(&s.upv[0][0][0]);
    static_assert(sizeof(s.upv) >= FUSED_MAX_ROUTES * sizeof(int), "route staging");
    for (int r = tid; r < R; r += FT) {
      const int e = s.exp_of_route[r];
      if (e >= 0) tmp[atomicAdd(&s.eoff[e], 1)] = r;
    }
    __syncthreads();
    for (int q = tid; q < s.meta[1]; q += FT) {
      const int v = tmp[q], e = s.exp_of_route[v], c = s.cnt[e], b = s.eoff[e] - c;
      int rank = 0;
      for (int j = 0; j < c; ++j) rank += tmp[b + j] < v ? 1 : 0;
      s.routes[b + rank] = v;
    }
    __syncthreads();
  }
  const int n_active = s.meta[0];
  for (int q = tid; q < s.meta[1]; q += FT) {
    const int r = s.routes[q], t = div_small(r, tkm);
    s.prow[q] = (r - t * p.topk) * p.part_rows + t;
    if constexpr (ACT != DGM_ACT_NVFP4) {
      s.ptok[q] = t;
      s.pw[q] = s.route_w[r];
    }
    // (NVFP4: always through the combine; its kernel has no registers to spare for the y store)
    s.ytok[q] = ACT != DGM_ACT_NVFP4 && s.nslot[t] == 1 ? t : -1;
  }
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
      if (p.recv_stats && (p.phases & 1)) {
        // (EARLY: an add with no return value, which does not wait for the requests above)
        if constexpr (EARLY) {
          if (s.cnt[e]) atomicAdd(p.recv_stats + e, s.cnt[e]);
        } else {
          p.recv_stats[e] += s.cnt[e];
        }
      }
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
  // The other counter set, cleared one line per thread, spread over the grid (its last user,
  // the previous launch on this buffer, has completed). (Issued here, behind the routing loads
  // and ahead of the first slab's, which wait about as long as these stores.)
  {
    int* const other = p.counters + CNT_SET0 + (1 - parity) * CNT_SET;
    for (int l = (int)blockIdx.x + (int)gridDim.x * tid; l < CNT_SET / CNT_LINE; l += (int)gridDim.x * FT)
      __hip_atomic_store(other + l * CNT_LINE, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();        // s.cnt / s.eoff (union with the B slab) are dead from here on

  // Units are claimed dynamically from one atomic counter per phase, ahead of their use: L1
  // units (active expert a, 64 intermediate features q), then L2 units (active expert a,
  // 128 output rows b). A workgroup starts on L2 units only after the L1 counter ran out, so
  // an L2 unit's wait is only on L1 units already claimed by running workgroups, which never
  // wait.
  // L2 units span RB2 combine blocks (128 rows each): every wave streams RB2 16-row blocks.
  // Each unit runs as RB2 items of one block instead (halves; debug bit 2 keeps whole units)
  // when the units fill at most half the grid, or (A-MXFP) when they fill more than one round
  // and at most 1.5: the last round, half full or less, then takes half a unit's time (an extra
  // item costs about as much as that saves beyond two rounds). U2 counts the L2 items.
  constexpr int RB2 = NBL2 % 2 == 0 ? 2 : 1, UPE2 = NBL2 / RB2;
  constexpr bool WIDE = ACT == DGM_ACT_MXFP4 || ACT == DGM_ACT_MXFP8 || F128;
  const int u2w = n_active * UPE2, G2 = (int)gridDim.x;
  const bool halves = RB2 == 2 && (2 * u2w <= G2 || (WIDE && u2w > G2 && 2 * (u2w - G2) <= G2)) && !(p.debug & 4);
  const int U1 = n_active * QN1, U2 = n_active * (halves ? NBL2 : UPE2);
  // TAIL: when the last round of L1 units fills at most half the grid, its units run as two
  // half items each (32 features; each 16-row block's K split over two waves, whose sums the
  // gate wave adds in the whole unit's order, so the results are those of whole units bit for
  // bit). Items: the whole units 0 .. Uw - 1, then half j of unit Uw + i as item Uw + 2 i + j.
  // L1 arrivals count half units (a whole unit adds 2).
  constexpr int L1W = TAIL ? 2 : 1;
  const int rem1 = U1 % (int)gridDim.x;
  const bool tail = TAIL && rem1 != 0 && 2 * rem1 <= (int)gridDim.x;
  const int Uw = tail ? U1 - rem1 : U1, UI = tail ? U1 + rem1 : U1;
  // This workgroup's first L2 unit (its second is G + v0)
  const int v0 = (int)blockIdx.x;
  const int c = lane & 15, kq = lane >> 4;
  int staged = -1;          // (phase, a, slab) currently in s.bst
  int l1_pend = -1;         // the L1 phase's last unit's expert slot, signalled in the L2 phase
  int l1_pend_w = 0;        // (and its arrival count)
  bool handed = false;      // wr[0 .. KT2) hold the first L2 unit's tiles 0 .. KT2 - 1
  // L2 item v's first 16-row block for this wave (whole units or halves)
  auto l2_blk = [wv, halves](int v) __attribute__((always_inline)) {
    return halves ? (size_t)s.act[v / NBL2] * NB2 + NW * (v % NBL2) + wv
                  : (size_t)s.act[v / UPE2] * NB2 + (NW * RB2) * (v % UPE2) + RB2 * wv;
  };

  // ================================================================ L1 phase
  // Wave w: block pair pp = w & 3 (16 of the unit's 64 features), tile gu = w >> 2 (gate or
  // up), full K. An L1 item is (unit, 16-route slab); a wave streams its 16-row weight block
  // through a ring of KR tile registers: after the op on tile t it issues tile t + KR of the
  // same item or tile t + KR - KT1 of the next item, so HBM reads never pause at item
  // boundaries. The next item's activation slab (when it differs) is loaded before that
  // item's tiles and stored to LDS between the epilogue's two barriers. An item's
  // intermediate stores have completed when the next item's K loop is done (memory ops
  // complete in order and that loop waited for younger tiles); the unit's arrival is
  // signalled then.
  if (p.phases & 1) {
    constexpr int KR = KT1 % 12 == 0 ? 12 : KT1;   // ring depth: tiles in flight per wave
    static_assert(KT1 % KR == 0, "the ring depth divides the K-tile count");
    int* claim = cset + CNT_CLAIM;
    const uint8_t* w1v = p.w1v;
    const uint32_t* w1s = p.w1s;
    constexpr int KH = KT1 / 2;       // (TAIL) K-tiles per wave of a half item
    static_assert(!TAIL || (KH == KR && KH % 4 == 0), "a half item fills the ring once, whole scale dwords");
    // item q: its unit; (half items) this wave's block pair (of the unit's four) is
    // 2 j + (w & 1), its tile (gate / up) (w >> 1) & 1 and its K half w >> 2
    auto unit_of = [Uw](int q) __attribute__((always_inline)) { return TAIL && q >= Uw ? Uw + ((q - Uw) >> 1) : q; };
    auto item_blk = [Uw, wv, l1_blk](int q) __attribute__((always_inline)) {
      if (TAIL && q >= Uw) {
        const int u = Uw + ((q - Uw) >> 1);
        return (size_t)s.act[u / QN1] * NB1 + 2 * (4 * (u % QN1) + 2 * ((q - Uw) & 1) + (wv & 1)) + ((wv >> 1) & 1);
      }
      return l1_blk(s.act[q / QN1], q % QN1);
    };
    auto tile_base = [w1v, lane, Uw, wv, item_blk](int q) __attribute__((always_inline)) {
      return w1v + item_blk(q) * KT1 * 1024 + (TAIL && q >= Uw ? (size_t)(wv >> 2) * KH * 1024 : 0) + lane * 16;
    };
    // (a half item loads its block's scale dwords of both K halves; it uses its own half's)
    auto load_scales = [load_scales_blk, item_blk](int q, uint32_t (&sw)[SW1]) __attribute__((always_inline)) {
      load_scales_blk(item_blk(q), sw);
    };
    // (TAIL) an item's first K-tile for this wave
    auto k_first = [Uw, wv](int q) __attribute__((always_inline)) { return TAIL && q >= Uw ? (wv >> 2) * KH : 0; };
    // NVFP4: the lane's scale dword of each tile (128 B of E4M3 scales per 16 x 128 tile), in a
    // ring beside the tile ring
    const int slane = (((lane >> 5) << 4) | (lane & 15)) * 4;
    auto stile_base = [w1s, slane, l1_blk](int u) __attribute__((always_inline)) {
      return reinterpret_cast<const uint8_t*>(w1s) + l1_blk(s.act[u / QN1], u % QN1) * KT1 * 128 + slane;
    };
    const uint8_t* xv = p.x;
    const uint8_t* xs = p.xsf;
    // (agent-scope loads when this launch's in-kernel frontend wrote the rows)
    // A slab column's token and weight come from the pool-row tables the dispatch filled: one
    // LDS read each, where route -> token / top-k and route -> weight were a dependent read and
    // an integer division on the first slab's path (0.5-1.7 us per layer call). NVFP4 keeps the
    // route-table reads: with the tables its kernel spills more registers.
    auto load_slab = [xv, xs, tkm](SlabRegs<KT1, ACT, FEIN, false>& r, int a, int s0) __attribute__((always_inline)) {
      if constexpr (ACT == DGM_ACT_NVFP4) {
        const int* rts = s.routes + s.aoff[a] + s0;
        slab_load<KT1, ACT, FEIN, false>(r, xv, xs, XB, s.aoff[a + 1] - s.aoff[a] - s0,
                                         [rts, tkm](int cc) { return div_small(rts[cc], tkm); },
                                         [rts](int cc) { return s.route_w[rts[cc]]; });
      } else {
        const int q0r = s.aoff[a] + s0;
        slab_load<KT1, ACT, FEIN, false>(r, xv, xs, XB, s.aoff[a + 1] - q0r,
                                         [q0r](int cc) { return s.ptok[q0r + cc]; },
                                         [q0r](int cc) { return s.pw[q0r + cc]; });
      }
    };
    // Workgroup g starts with units g and G + g (every workgroup starts at once: claims on
    // one counter would serialize them); later units are claimed one at a time from a counter
    // (offset by 2 G), by thread 0, one item before they are needed.
    const int G = gridDim.x;
    // thread 0: the raw counter value of the claim ahead (unit 2 G + value), -1 for none; it is
    // used as returned (any arithmetic on it here would wait for every load issued before it)
    int ahead = -1;
    int q0 = (int)blockIdx.x < UI ? (int)blockIdx.x : UI;    // current item
    int q1 = G + (int)blockIdx.x < UI ? G + (int)blockIdx.x : UI;   // next item
    int s0 = 0;
    uint32_t sn[SW1];
    int pend = -1;            // expert slot of a finished unit whose arrival is not signalled yet
    int pend_w = 0;           // (and its arrival count)
    if (q0 < UI) {
      // The first item's slab is staged before any tile load is issued: every workgroup
      // starts at once, and tile loads issued first would queue the slab loads (and so the
      // barrier, and every wave's first K loop) behind the whole ring of every wave.
      // (EARLY: all three were requested during the dispatch; q0 < U1 exactly when the mask
      // had an active expert q0 / QN1.)
      if constexpr (!EARLY) {
        load_slab(pre, unit_of(q0) / QN1, 0);
        load_scales(q0, sd);
      }
      slab_store(s, pre);
      staged = (unit_of(q0) / QN1) << 16;
      __syncthreads();
      if constexpr (!EARLY) {
        const uint8_t* b = tile_base(q0);
#pragma unroll
        for (int k = 0; k < KR; ++k) wr[k] = ld_stream(b + k * 1024);
        if constexpr (ACT == DGM_ACT_NVFP4) {
          const uint8_t* sb = stile_base(q0);
#pragma unroll
          for (int k = 0; k < KR; ++k) sr[k] = ld_stream32(sb + k * 128);
        }
      }
    }
    // B operands (the staged slab's fragments) are read from LDS two K-tiles ahead of their
    // matrix-core op. An item's first two, and its first B scale dword, are read at the end of
    // the previous item's epilogue, before its stores: read at the loop's top, they could land
    // in registers of those stores and wait for them (and so for the whole ring).
    auto bfrag = [lane](int t) __attribute__((always_inline)) {
      return ACT == DGM_ACT_MXFP4 ? as_v8i(s.bst[t][lane][0]) : as_v8i(s.bst[t][lane][0], s.bst[t][lane][Smem::BV - 1]);
    };
    v8i bq0 = {}, bq1 = {};
    uint32_t bs0 = 0;
    if (q0 < UI) {
      const int k0 = k_first(q0);
      bq0 = bfrag(k0);
      bq1 = KT1 > 1 ? bfrag(k0 + 1) : bq0;
      bs0 = s.bsc[k0 >> 2][lane];
    }
    bool more = 2 * G < UI;   // the claim counter has not run out
    while (q0 < UI) {
      const int u0 = unit_of(q0);
      const int a = u0 / QN1, q = u0 % QN1;
      const bool hf = TAIL && q0 >= Uw;       // a half item
      const int r0 = s.aoff[a], n = s.aoff[a + 1] - r0;
      const bool last_slab = s0 + 16 >= n;
      const int nq = last_slab ? q1 : q0, ns0 = last_slab ? 0 : s0 + 16;
      const bool has_next = nq < UI;
      const int na = has_next ? unit_of(nq) / QN1 : -1;
      const int nkey = (na << 16) | ns0;
      const bool restage = has_next && nkey != staged;
      const uint8_t* cb = tile_base(q0);
      // no next L1 item: ring slots < KT2 take the first L2 unit's tiles (when that unit is
      // this workgroup's), the rest dummy reads
      const bool hand = HANDOFF && !has_next && (p.phases & 2) && v0 < U2;
      const uint8_t* dummy = w1v + lane * 16;
      const uint8_t* nb = !has_next ? (hand ? p.w2v + l2_blk(v0) * KT2 * 1024 + lane * 16 : dummy)
                                    : nq == q0 ? cb : tile_base(nq);
      const uint8_t* nbd = hand ? dummy : nb;
      if (hand) handed = true;
      const uint8_t* csb = ACT == DGM_ACT_NVFP4 ? stile_base(q0) : nullptr;
      const uint8_t* sdummy = reinterpret_cast<const uint8_t*>(w1s) + slane;
      const uint8_t* nsb = ACT != DGM_ACT_NVFP4 ? nullptr
                           : !has_next ? (hand ? reinterpret_cast<const uint8_t*>(p.w2s) + l2_blk(v0) * KT2 * 128 + slane : sdummy)
                                       : nq == q0 ? csb : stile_base(nq);
      const uint8_t* nsbd = hand ? sdummy : nsb;
      // (MXFP, QoQ: the next item's scale and slab loads are issued in the K loop, after the
      // tile loads of its first KT1 - KR ops, so that the loop starts as soon as its first tile
      // is in)
      if constexpr (ACT == DGM_ACT_NVFP4) {
        if (has_next && nq != q0) load_scales(nq, sn);
        if (restage) load_slab(pre, na, ns0);
      }
      const float wt_r = s.slab_w[c];
      const float sx = ACT == DGM_ACT_QOQ ? s.xsc[c] : 1.f;       // QoQ: the token's activation scale
      // the unit after q1, claimed during the item that finishes q0 (after its loads; the value
      // is read in this item's epilogue, by when it has returned). A-MXFP8 and NVFP4 claim in
      // the K loop, at tile CT (where the refills turn to the next item: the workgroup commits
      // to the unit half an item later, and those kernels' registers come out no worse); the
      // others at the loop's start (A-MXFP4, QoQ, FP8F128: mid-loop claims measured no faster or
      // spilled registers).
      auto claim_ahead = [&]() __attribute__((always_inline)) {
        if (tid == 0 && last_slab && q1 < UI && more) ahead = __hip_atomic_fetch_add(claim, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      };
      constexpr int CT = !TAIL && (ACT == DGM_ACT_MXFP8 || ACT == DGM_ACT_NVFP4) ? KT1 - KR : -1;
      if constexpr (CT < 0) claim_ahead();
      const long long t_k0 = st ? wall_clock() : 0;
      // ---- K loop over the ring
      v4f acc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (ACT == DGM_ACT_QOQ) {
        // per K-tile: two int8 ops on the raw 4-bit codes (exact int32 sums of code * x), then,
        // one tile later (off the matrix-core result's latency), the zero-point correction
        // P = acc - z * sum(x) and the group scale: Q += s2 * P (exact: |Q| < 2^31)
        // (the promote's LDS inputs of a tile are read two ops ahead of their use)
        v4i qa = {0, 0, 0, 0}, prev = {0, 0, 0, 0};
        uint32_t md_c = qoq_meta<0>(sd, kq), md_n = 0;
        int x_c = s.xsum[c][0], x_n = 0;
        auto promote = [&](v4i a, uint32_t md, int X) __attribute__((always_inline)) {
          const int nX = -X;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // 24-bit multiplies (full rate; a 32-bit multiply is quarter rate): z, s2 < 16,
            // |X| <= 128 * 127, |a - z X| <= 128 * 15 * 127 < 2^23
            const int z = (int)((md >> (8 * i)) & 15u), s2 = (int)((md >> (8 * i + 4)) & 15u);
            int q = qa[i];
            mad_i24_acc(q, a[i] + __mul24(z, nX), s2);
            qa[i] = q;
          }
        };
        static_for<KT1>([&](auto tc) {
          constexpr int t = decltype(tc)::value;
          if constexpr (t == CT) claim_ahead();
          v8i bop = bq0;
          bq0 = bq1;
          if constexpr (t + 2 < KT1) bq1 = bfrag(t + 2);
          if constexpr (t >= 2) after_values(bop, qa);      // (tile t - 2 promoted)
          const U4 w = wr[t % KR];
          v4i at = mfma_i8_16x16x64(qoq_codes(w.x, w.y), lo4(bop), v4i{0, 0, 0, 0});
          at = mfma_i8_16x16x64(qoq_codes(w.z, w.w), hi4(bop), at);
          if constexpr (t + KR < KT1) wr[t % KR] = ld_stream_after(cb, (t + KR) * 1024, at);
          else wr[t % KR] = ld_stream_after(t + KR - KT1 < KT2 ? nb : nbd, (t + KR - KT1) * 1024, at);
          if constexpr (t == KT1 - KR) {
            if (has_next && nq != q0) load_scales(nq, sn);
            if (restage) load_slab(pre, na, ns0);
          }
          if constexpr (t > 0) promote(prev, md_n, x_n);         // tile t - 1
          md_n = md_c;
          x_n = x_c;
          if constexpr (t + 1 < KT1) {
            md_c = qoq_meta<t + 1>(sd, kq);
            x_c = s.xsum[c][t + 1];
          }
          prev = at;
        });
        promote(prev, md_n, x_n);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = (float)qa[i] * __uint_as_float(sd[MR1 + i]) * sx;
        if (p.debug & 2) {
          // (tests) the exact int32 accumulators: [pool row][W1 row, gate rows then up rows]
          if (s0 + c < n) {
            int* dq = reinterpret_cast<int*>(p.stamps) + (size_t)(r0 + s0 + c) * (2 * I) + (gu ? I : 0) +
                      16 * (4 * q + pp) + 4 * kq;
#pragma unroll
            for (int i = 0; i < 4; ++i) dq[i] = qa[i];
          }
        }
      } else if constexpr (ACT == DGM_ACT_NVFP4) {
        // four f16 ops per tile: weights E2M1 x E4M3 -> f16 in registers, activations already
        // f16 in LDS (read one tile ahead); scale dwords stream in their own ring
        U4 bn[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bn[j] = s.bst[0][lane][j];
        static_for<KT1>([&](auto tc) {
          constexpr int t = decltype(tc)::value;
          if constexpr (t == CT) claim_ahead();
          U4 bc[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) bc[j] = bn[j];
          if constexpr (t + 1 < KT1) {
#pragma unroll
            for (int j = 0; j < 4; ++j) bn[j] = s.bst[t + 1][lane][j];
          }
          acc = nvfp4_tile(wr[t % KR], sr[t % KR], bc, acc);
          if constexpr (t + KR < KT1) {
            wr[t % KR] = ld_stream_after(cb, (t + KR) * 1024, acc);
            sr[t % KR] = ld_stream32_after(csb, (t + KR) * 128, acc);
          } else {
            wr[t % KR] = ld_stream_after(t + KR - KT1 < KT2 ? nb : nbd, (t + KR - KT1) * 1024, acc);
            sr[t % KR] = ld_stream32_after(t + KR - KT1 < KT2 ? nsb : nsbd, (t + KR - KT1) * 128, acc);
          }
        });
      } else if constexpr (F128) {
        // one chain, as the split path's L1 kernel: per K-tile the block-scaled op with a unit
        // activation scale into a zero accumulator, then acc += s * part with the token's fp32
        // scale s of that K-tile, one tile later (off the op's latency). A compiler ordering
        // point keeps each op after the promote two tiles back (independent ops would otherwise
        // all be issued first, every result kept live).
        uint32_t bs = bs0;
        float xf_c = s.xf[0][c], xf_p = 0.f;
        v4f prev = {0.f, 0.f, 0.f, 0.f};
        static_for<KT1>([&](auto tc) {
          constexpr int t = decltype(tc)::value;
          if constexpr (t == CT) claim_ahead();
          v8i bop = bq0;
          const uint32_t bsw = bs;
          bq0 = bq1;
          if constexpr (t + 2 < KT1) bq1 = bfrag(t + 2);
          if constexpr ((t & 3) == 3 && t + 1 < KT1) bs = s.bsc[(t + 1) >> 2][lane];
          if constexpr (t >= 2) after_values(bop, acc);      // (tile t - 2 promoted)
          const v4f part = mfma_scale_16x16x128_sel<4, FB, t & 3, t & 3>(as_v8i(wr[t % KR]), bop, v4f{0.f, 0.f, 0.f, 0.f},
                                                                         (int)sd[t >> 2], (int)bsw);
          if constexpr (t + KR < KT1) wr[t % KR] = ld_stream_after(cb, (t + KR) * 1024, part);
          else wr[t % KR] = ld_stream_after(t + KR - KT1 < KT2 ? nb : nbd, (t + KR - KT1) * 1024, part);
          if constexpr (t > 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = fmaf(xf_p, prev[i], acc[i]);     // tile t - 1
          }
          xf_p = xf_c;
          if constexpr (t + 1 < KT1) xf_c = s.xf[t + 1][c];
          prev = part;
          if constexpr (t == KT1 - KR) {
            if (has_next && nq != q0) load_scales(nq, sn);
            if (restage) load_slab(pre, na, ns0);
          }
        });
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(xf_p, prev[i], acc[i]);
      } else {
        // two chains, K-tiles 0 .. KT1 / 2 - 1 and KT1 / 2 .., summed after the loop: the split
        // path's L1 kernel sums the same two, so the two paths agree bit for bit for any data.
        // (TAIL, a half item: each wave runs one of the chains, K half w >> 2, and a K half 0
        // wave refills its slots with the next item's tiles: a half item fills the ring once.)
        v4f acc2 = {0.f, 0.f, 0.f, 0.f};
        uint32_t bs = bs0;
        const bool hi_wave = wv >= 4;
        const int ro = TAIL && hf ? 0 : KR * 1024;                     // refill offset of K half 0
        static_for<KT1>([&](auto tc) {
          constexpr int t = decltype(tc)::value;
          if constexpr (t == CT) claim_ahead();
          constexpr bool HI = t >= KT1 / 2;
          if (!TAIL || !hf || HI == hi_wave) {
            const v8i bop = bq0;
            const uint32_t bsw = bs;
            bq0 = bq1;
            if constexpr (t + 2 < KT1) bq1 = bfrag(t + 2);
            if constexpr ((t & 3) == 3 && t + 1 < KT1) bs = s.bsc[(t + 1) >> 2][lane];
            v4f& ac = HI ? acc2 : acc;
            ac = mfma_scale_16x16x128_sel<4, FB, t & 3, t & 3>(as_v8i(wr[t % KR]), bop, ac, (int)sd[t >> 2], (int)bsw);
            if constexpr (t + KR < KT1) {
              // (a half item's K half 0: the next item's tile t, as the second half refills)
              const uint8_t* rb = TAIL && hf ? (t < KT2 ? nb : nbd) : cb;
              wr[t % KR] = ld_stream_after(rb, (TAIL ? ro : KR * 1024) + t * 1024, ac);
            }
            else wr[t % KR] = ld_stream_after(t + KR - KT1 < KT2 ? nb : nbd, (t + KR - KT1) * 1024, ac);
            if constexpr (t == KT1 - KR || (TAIL && t == 0)) {
              if (t == KT1 - KR || (hf && !hi_wave)) {
                if (has_next && nq != q0) load_scales(nq, sn);
                if (restage) load_slab(pre, na, ns0);
              }
            }
          }
        });
        if (TAIL && hf) {
          if (hi_wave) acc = acc2;      // (the K half 1 chain, added by the gate wave)
        } else {
          acc += acc2;
        }
      }
      // all but this loop's KR youngest tile loads (and scale loads) are done: the previous
      // item's stores too
      wait_vm_le<ACT == DGM_ACT_NVFP4 ? 2 * KR : KR>();
      const long long t_e0 = st ? wall_clock() : 0;
      if (st) l1_load_ticks += t_e0 - t_k0;
      if constexpr (ACT == DGM_ACT_NVFP4) {
        const float gsc = s.gsl[0][s.act[a]];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] *= gsc;
      }
      // this wave's block pair (of the unit's four) and tile in the item, and whether it holds
      // K half 1 of a half item (its sum goes to the gate wave through LDS)
      const int ip = hf ? 2 * ((q0 - Uw) & 1) + (wv & 1) : pp;
      const int ig = hf ? (wv >> 1) & 1 : gu;
      const bool khi = hf && wv >= 4;
      if (khi) {
        if constexpr (TAIL) {
#pragma unroll
          for (int i = 0; i < 4; ++i) s.hsum[wv & 1][ig][lane][i] = acc[i];
        }
      } else if (ig == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s.upv[ip][lane][i] = acc[i];
      }
      // the unit after q1 (claimed at this item's start), broadcast here
      const bool bcast = last_slab && q1 < UI;
      if (tid == 0 && bcast) s.claimv[0] = more ? ahead : -1;
      __syncthreads();                                   // (1) up sums visible, slab free
      if (tid == 0 && pend >= 0) __hip_atomic_fetch_add(&l1_done[pend * CNT_LINE], pend_w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      pend = -1;
      int q2 = UI;
      if (bcast) {
        const int raw = __builtin_amdgcn_readfirstlane(s.claimv[0]);
        q2 = raw >= 0 && 2 * G + raw < UI ? 2 * G + raw : UI;
        if (q2 >= UI) more = false;
      }
      if (restage) {
        slab_store(s, pre);
        staged = nkey;
      }
      const bool valid = s0 + c < n;
      const int pr = 4 * q + ip;                         // 16-feature block of this pair
      float act[4];
      if (ig == 0 && !khi) {
        float am = 0.f;
        if constexpr (TAIL) {
          if (hf) {           // the K halves summed as a whole unit sums its two chains
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += s.hsum[wv & 1][0][lane][i];
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // MXFP: gate / up rounded to bf16 (the reference's L1 output); QoQ, FP8F128: fp32
          // (tests/test_four_api_correctness.py:437-442)
          constexpr bool F32GU = ACT == DGM_ACT_QOQ || F128;
          const float g = fminf(F32GU ? acc[i] : round_bf16(acc[i]), p.clamp);
          float uv = s.upv[ip][lane][i];
          if constexpr (TAIL) {
            if (hf) uv += s.hsum[wv & 1][1][lane][i];
          }
          const float uu = fminf(fmaxf(F32GU ? uv : round_bf16(uv), -p.clamp), p.clamp);
          const float sgm = p.fast_math ? sigmoid<true>(g) : sigmoid<false>(g);
          act[i] = valid ? ((g * sgm) * uu) * wt_r : 0.f;
          am = fmaxf(am, fabsf(act[i]));
        }
        am = fmaxf(am, __shfl_xor(am, 16));
        am = fmaxf(am, __shfl_xor(am, 32));
        if (lane < 16) s.amax[ip][lane] = am;
      }
      __syncthreads();                                   // (2) amax visible, next slab staged
      if (has_next) {
        const int k0 = k_first(nq);
        bq0 = bfrag(k0);
        bq1 = KT1 > 1 ? bfrag(k0 + 1) : bq0;
        bs0 = s.bsc[k0 >> 2][lane];
      }
      if (ig == 0 && !khi) {
        // requant group: QoQ, FP8F128 64 features (the unit), NVFP4 16 (this pair), MXFP 32 (two
        // pairs, both in a half item)
        const float am = ACT == DGM_ACT_QOQ || F128 ? fmaxf(fmaxf(s.amax[0][c], s.amax[1][c]), fmaxf(s.amax[2][c], s.amax[3][c]))
                         : ACT == DGM_ACT_NVFP4 ? s.amax[ip][c]
                                                : fmaxf(s.amax[ip][c], s.amax[ip ^ 1][c]);
        const int row = r0 + s0 + c;
        // lane group kq holds features 16 pr + 4 kq .. +3 of column c
        if (ACT == DGM_ACT_QOQ) {
          // int8 per 64 features (this unit): scale = max(amax / 127, FLT_MIN), round to
          // nearest even, clamp to +-127
          const float sc = fmaxf(am / 127.0f, 1.17549435e-38f);
          uint32_t w = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float v = fminf(fmaxf(rintf(act[i] / sc), -127.f), 127.f);
            w |= ((uint32_t)(int)v & 0xffu) << (8 * i);
          }
          const int src_lo = lane < 16 ? c : c + 32, src_hi = lane < 16 ? c + 16 : c + 48;
          const uint64_t w64 = (uint64_t)__shfl(w, src_lo) | ((uint64_t)__shfl(w, src_hi) << 32);
          if (valid && lane < 32) {
            st_agent64(p.mid + (size_t)row * MB + 16 * pr + (lane < 16 ? 0 : 8), w64);
            if (ip == 0 && lane < 16) st_agent32(p.mid_sf + (size_t)row * (I / 16) + 4 * q, __float_as_uint(sc));
          }
        } else if (ACT == DGM_ACT_NVFP4) {
          // E2M1 per 16 features: sf = E4M3 (round to nearest even) of max(amax, 1e-30) / 6,
          // ties-down E2M1 of act / sf (sm100_b200/test_mega_moe.py:68-80, requant_fp4)
          const uint32_t code = e4m3_encode(fmaxf(am, 1e-30f) / 6.0f);
          const float sc = __builtin_amdgcn_cvt_f32_fp8((int)code, 0);
          uint32_t w = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) w |= e2m1_ties_down(act[i] / sc) << (4 * i);
          const uint64_t w64 = (uint64_t)(w & 0xffffu) | ((uint64_t)(__shfl(w, c + 16) & 0xffffu) << 16) |
                               ((uint64_t)(__shfl(w, c + 32) & 0xffffu) << 32) |
                               ((uint64_t)(__shfl(w, c + 48) & 0xffffu) << 48);
          if (valid && lane < 16) {
            st_agent64(p.mid + (size_t)row * MB + 8 * pr, w64);
            st_agent8(p.mid_sf + (size_t)row * (I / 16) + pr, (uint8_t)code);
          }
        } else if (ACT == DGM_ACT_MXFP4) {
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
            if ((ip & 1) == 0) st_agent8(p.mid_sf + (size_t)row * (I / 32) + (pr >> 1), (uint8_t)code);
          }
        } else {
          // E4M3 with a power-of-two scale per 32 (MXFP8: 2^ceil(log2(max(amax, 1e-30) / 448)))
          // or per 64 (FP8F128: 2^ceil(log2(max(amax / 448, FLT_MIN))), tests/test_four_api_
          // correctness.py:54-62, stored as two equal E8M0 bytes per 32)
          const int code = (int)(F128 ? ceil_log2_f32(fmaxf(am / 448.0f, 1.17549435e-38f))
                                      : ceil_log2_f32(fmaxf(am, 1e-30f) / 448.0f)) + 127;
          const float isc = e8m0_inv((uint32_t)code);
          uint32_t w = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) w |= e4m3_encode(act[i] * isc) << (8 * i);
          // lanes 0-15: features 0-7 (groups 0, 1); lanes 16-31: features 8-15 (groups 2, 3)
          const int src_lo = lane < 16 ? c : c + 32, src_hi = lane < 16 ? c + 16 : c + 48;
          const uint64_t w64 = (uint64_t)__shfl(w, src_lo) | ((uint64_t)__shfl(w, src_hi) << 32);
          if (valid && lane < 32) {
            st_agent64(p.mid + (size_t)row * MB + 16 * pr + (lane < 16 ? 0 : 8), w64);
            if ((ip & 1) == 0 && lane < 16) st_agent8(p.mid_sf + (size_t)row * (I / 32) + (pr >> 1), (uint8_t)code);
          }
        }
      }
      if (st) l1_sig_ticks += wall_clock() - t_e0;
      if (last_slab) {
        pend = a;
        pend_w = hf ? 1 : L1W;
        if (nq != q0) {
#pragma unroll
          for (int g = 0; g < SW1; ++g) sd[g] = sn[g];
        }
        q0 = q1;
        q1 = q2;
        s0 = 0;
      } else {
        s0 += 16;
      }
    }
    if (p.phases & 2) {
      l1_pend = pend;         // (its stores complete while the L2 phase issues its first loads)
      l1_pend_w = pend_w;
    } else {
      wait_mem();             // the last item's stores (and the dummy ring reads)
      __syncthreads();
      if (tid == 0 && pend >= 0) __hip_atomic_fetch_add(&l1_done[pend * CNT_LINE], pend_w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (st && tid == 0) st[2] = wall_clock();

  // ================================================================ L2 phase
  // Item (a, b) = rows 128 RB b .. +128 RB of expert a; wave w owns the RB 16-row blocks
  // at 16 (NW RB b + RB w) .. (TI contiguous tiles over the full K). The wave streams them
  // through a ring of KT2 tile registers; the second half of the ring (and all of it at the
  // end) rolls into the next item's tiles right after the op that consumed a slot. The next
  // item's slab (intermediate rows of another expert) is loaded ahead when that expert's L1
  // arrival is already complete, else staged at the item's start after a bounded wait. Route
  // outputs (bf16) go to `partials`; one item later, when they have completed, each route
  // bumps the arrival counters of its (token, 128-row block)s (no return value).
  // The L2 phase for items of RB 128-row blocks (every wave streams RB 16-row blocks of each):
  // whole units (RB = RB2) or halves (RB = 1, by the rule above), one or the other per launch,
  // each its own code (no branch inside the K loops).
  auto l2_phase = [&](auto rb_c) __attribute__((always_inline)) {
    constexpr int RB = decltype(rb_c)::value, UPE = NBL2 / RB, TI = RB * KT2;
    static_assert(KT2 <= 16, "L2 ring of KT2 tile registers");
    int* claim = cset + CNT_CLAIM + CNT_LINE;
    const uint8_t* w2v = p.w2v;
    const uint32_t* w2s = p.w2s;
    const float* w2r = p.w2r;
    // item v = (active expert a, RB * 128-row slice b): this wave's first 16-row block of it
    auto blk_of = [wv](int v) __attribute__((always_inline)) {
      return (size_t)s.act[v / UPE] * NB2 + (NW * RB) * (v % UPE) + RB * wv;
    };
    auto tile_base = [w2v, lane, blk_of](int v) __attribute__((always_inline)) {
      return w2v + blk_of(v) * KT2 * 1024 + lane * 16;
    };
    // per-item scale registers (the wave's RB contiguous 16-row blocks), loaded one item
    // ahead: MXFP: E8M0 scale dwords; QoQ: meta dwords (4 per K-tile)
    constexpr int MR2 = (4 * TI + 63) / 64;
    constexpr int SW2 = ACT == DGM_ACT_QOQ ? MR2 : ACT == DGM_ACT_NVFP4 ? 1 : RB * KG2;
    auto load_scales = [w2s, lane, blk_of](int v, auto& sw) __attribute__((always_inline)) {
      if constexpr (ACT == DGM_ACT_QOQ) {
        const uint32_t* mb = w2s + blk_of(v) * KT2 * 4;
#pragma unroll
        for (int j = 0; j < MR2; ++j)
          sw[j] = __builtin_nontemporal_load(mb + (64 * j + lane < 4 * TI ? 64 * j + lane : 4 * TI - 1));
      } else if constexpr (ACT == DGM_ACT_NVFP4) {
        sw[0] = 0u;      // (the NVFP4 scales stream with the tiles)
      } else {
        const uint32_t* b = w2s + blk_of(v) * KG2 * 64 + lane;
#pragma unroll
        for (int g = 0; g < RB * KG2; ++g) sw[g] = __builtin_nontemporal_load(b + g * 64);
      }
    };
    // NVFP4: the lane's scale dword of each tile, in a ring beside the tile ring
    const int slane = (((lane >> 5) << 4) | (lane & 15)) * 4;
    auto stile_base = [w2s, slane, blk_of](int v) __attribute__((always_inline)) {
      return reinterpret_cast<const uint8_t*>(w2s) + blk_of(v) * KT2 * 128 + slane;
    };
    const uint8_t* midv = p.mid;
    const uint8_t* mids = p.mid_sf;
    auto load_slab = [midv, mids](SlabRegs<KT2, ACT2, true>& r, int a, int s0) __attribute__((always_inline)) {
      const int rb = s.aoff[a] + s0;
      slab_load<KT2, ACT2, true, true>(r, midv, mids, MB, s.aoff[a + 1] - rb, [rb](int cc) { return rb + cc; },
                                [](int) { return 0.f; });
    };
    // arrivals of item (unit v, slab s0): its routes' outputs for the unit's blocks are complete
    auto arrive = [comb, tid, tkm](int v, int s0) __attribute__((always_inline)) {
      // (the top-k multiplier and the thread index made opaque: what derives from them is
      // computed here, not kept live across the work loop, where it would cost registers or a
      // spill)
      uint32_t tk = tkm;
      int i0 = tid;
      asm volatile("" : "+s"(tk), "+v"(i0));
      const int a = v / UPE, b = v % UPE;
      const int r0 = s.aoff[a] + s0, n = s.aoff[a + 1] - r0;
      // (the route's token from the pool-row table: the division by top-k it replaces sat between
      // the item's two barriers and cost 0.4-1.8 us per layer call; NVFP4 has no table)
      for (int i = i0; i < 16 * RB && i / RB < n; i += FT)
        if (ACT == DGM_ACT_NVFP4 || s.ytok[r0 + i / RB] < 0) {   // (a token's only local route writes y itself)
          const int t = ACT == DGM_ACT_NVFP4 ? div_small(s.routes[r0 + i / RB], tk) : s.ptok[r0 + i / RB];
          __hip_atomic_fetch_add(&comb[(t * NBL2 + RB * b + i % RB) * CNT_LINE], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };
    // units v0 and G + v0 first, then claims (offset by 2 G)
    __syncthreads();
    const int G = gridDim.x;
    // thread 0: the raw counter value of the claim ahead (unit 2 G + value), -1 for none; it is
    // used as returned (any arithmetic on it here would wait for every load issued before it)
    int ahead = -1;
    bool more = 2 * G < U2;   // the claim counter has not run out
    int q0 = v0 < U2 ? v0 : U2;
    int q1 = G + v0 < U2 ? G + v0 : U2;
    int s0 = 0;
    static_assert(KT2 <= RING, "the L2 ring in the shared tile registers");
    uint32_t sd[SW2], sn[SW2];
    SlabRegs<KT2, ACT2, true> pre;
    int ready = -1;           // (thread 0) an active expert whose L1 arrival is known complete
    bool seen = false;        // (stamps) first L1 arrival observed
    int pv = -1, ps0 = 0;     // the previous item, whose arrivals are not sent yet
    int pr_a = 0, pr_n = 0;
    if (p.phases & 1) {
      // probes of the L1 arrivals of the first two units' experts, answered while the L1
      // phase's last stores complete
      if (tid == 0 && q0 < U2) {
        pr_a = __hip_atomic_load(&l1_done[(q0 / UPE) * CNT_LINE], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (q1 < U2) pr_n = __hip_atomic_load(&l1_done[(q1 / UPE) * CNT_LINE], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      // the L1 phase's last unit: its stores have completed (every wave) -> its arrival, before
      // any wait on other workgroups' arrivals
      wait_mem();
      if (tid == 0) s.claimv[1] = q0 < U2 && pr_a >= L1W * QN1 ? 1 : 0;
      __syncthreads();
      if (tid == 0 && l1_pend >= 0) __hip_atomic_fetch_add(&l1_done[l1_pend * CNT_LINE], l1_pend_w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (tid == 0 && q0 < U2 && pr_a >= L1W * QN1) ready = q0 / UPE;
    }
    // (thread 0) the second unit's expert when its probe found it complete (LDS: read once, by
    // the first item's prefetch check)
    if (tid == 0) s.claimv[2] = q1 < U2 && pr_n >= L1W * QN1 ? q1 / UPE : -1;
    if (q0 < U2) {
      if (!handed) {          // (unit q0 = v0: handed over by the L1 phase otherwise)
        const uint8_t* b = tile_base(q0);
#pragma unroll
        for (int k = 0; k < KT2; ++k) wr[k] = ld_stream(b + k * 1024);
        if constexpr (ACT == DGM_ACT_NVFP4) {
          const uint8_t* sb = stile_base(q0);
#pragma unroll
          for (int k = 0; k < KT2; ++k) sr[k] = ld_stream32(sb + k * 128);
        }
      }
      load_scales(q0, sd);
    }
    // the first item's slab, loaded now when its expert's L1 arrival is known complete (stored
    // at the item's start; its loads complete while the tiles and scales above are in flight).
    // (NVFP4 stages it at the item's start: measured no faster this way.)
    bool pre1 = false;
    if (ACT != DGM_ACT_NVFP4 && q0 < U2 && (!(p.phases & 1) || __builtin_amdgcn_readfirstlane(s.claimv[1]) != 0)) {
      load_slab(pre, q0 / UPE, 0);
      pre1 = true;
    }
    while (q0 < U2) {
      const int a = q0 / UPE, b = q0 % UPE;
      const int r0 = s.aoff[a], n = s.aoff[a + 1] - r0;
      const int key = (1 << 30) | (a << 16) | s0;
      if (pre1) {               // (the first item, its slab loaded before the loop)
        pre1 = false;
        slab_store(s, pre);
        staged = key;
        __syncthreads();
      } else if (key != staged) {    // not prefetched: wait for the expert's L1 units, then stage
        const long long w0 = st ? wall_clock() : 0;
        if (a != ready) {
          if (tid == 0 && (p.phases & 1)) spin_until2(&l1_done[a * CNT_LINE], L1W * QN1, p.spin_limit, err, p.host_err);
          ready = a;
        }
        __syncthreads();
        if (st) {
          wait_ticks += wall_clock() - w0;
          if (tid == 0 && !seen) st[3] = wall_clock();
          seen = true;
        }
        if constexpr (ACT == DGM_ACT_QOQ || ACT == DGM_ACT_NVFP4) {
          load_slab(pre, a, s0);            // (pre holds nothing between items)
          slab_store(s, pre);
        } else {
          const int rb = r0 + s0;
          stage_slab<KT2, ACT2, true>(s, p.mid, p.mid_sf, MB, n - s0, [rb](int cc) { return rb + cc; });
        }
        staged = key;
        __syncthreads();
      }
      const bool last_slab = s0 + 16 >= n;
      const int nq = last_slab ? q1 : q0, ns0 = last_slab ? 0 : s0 + 16;
      const bool has_next = nq < U2;
      const int na = has_next ? nq / UPE : -1;
      const int nkey = (1 << 30) | (na << 16) | ns0;
      // prefetch the next item's slab if it differs and its expert's L1 is complete
      bool pf = false;
      if (has_next && nkey != key) {
        if (tid == 0)
          s.claimv[1] = !(p.phases & 1) || na == ready || na == s.claimv[2] ||
                        __hip_atomic_load(&l1_done[na * CNT_LINE], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= L1W * QN1;
        __syncthreads();
        pf = __builtin_amdgcn_readfirstlane(s.claimv[1]) != 0;
        if (pf) {
          ready = na;
          load_slab(pre, na, ns0);
        }
      }
      const uint8_t* cb = tile_base(q0);
      const uint8_t* nb = !has_next ? w2v + lane * 16 : nq == q0 ? cb : tile_base(nq);   // (no next: a dummy read)
      const uint8_t* csb = ACT == DGM_ACT_NVFP4 ? stile_base(q0) : nullptr;
      const uint8_t* nsb = ACT != DGM_ACT_NVFP4 ? nullptr
                           : !has_next ? reinterpret_cast<const uint8_t*>(w2s) + slane : nq == q0 ? csb : stile_base(nq);
      if (has_next && nq != q0) load_scales(nq, sn);
      // QoQ: the row scales s1 of the lane's 4 rows of each block, only used after the K loop
      // (so loaded for this item, here)
      v4u s1r[ACT == DGM_ACT_QOQ ? RB : 1];
      if constexpr (ACT == DGM_ACT_QOQ) {
#pragma unroll
        for (int jb = 0; jb < RB; ++jb)
          s1r[jb] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(w2r + (blk_of(q0) + jb) * 16 + 4 * kq));
      }
      // the unit after q1, claimed during the item that finishes q0 (the value is read in this
      // item's epilogue). NVFP4 claims in the K loop, at tile CT where the refills turn to the
      // next item (its kernel then needs 179 instead of 256 VGPRs and no scratch: 2-5 us faster
      // at M=16-64); the others at the loop's start (A-MXFP8 measured slower, 253 VGPRs).
      auto claim_ahead = [&]() __attribute__((always_inline)) {
        if (tid == 0 && last_slab && q1 < U2 && more) ahead = __hip_atomic_fetch_add(claim, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      };
      constexpr int CT = ACT == DGM_ACT_NVFP4 ? TI - KT2 : -1;
      if constexpr (CT < 0) claim_ahead();
      // ---- K loop over the ring: tile t is K-tile t % KT2 of block t / KT2; B operands are
      // read from LDS two ops ahead
      v4f acc[RB];
#pragma unroll
      for (int j = 0; j < RB; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
      auto bfrag = [lane](int k) __attribute__((always_inline)) {
        return ACT == DGM_ACT_MXFP4 ? as_v8i(s.bst[k][lane][0]) : as_v8i(s.bst[k][lane][0], s.bst[k][lane][Smem::BV - 1]);
      };
      v8i bq0 = bfrag(0), bq1 = bfrag(1 % KT2);
      if constexpr (ACT == DGM_ACT_QOQ) {
        // Per K-tile two int8 ops, one per 64-K chunk (the intermediate's scale changes every
        // 64 features). The down-projection codes are stored chunk-split: low nibbles = chunk 0,
        // high nibbles = chunk 1 XOR 8, so op 0 takes (d & 0x0F0F0F0F) = code and op 1 takes
        // (d & 0xF0F0F0F0) = 16 code - 128 (as int8) with one mask each. With X_h the chunk's
        // value sums and sm_h its scales (per column), one tile later:
        //   f += s2 * (sm_0 M_0 + sm_1 / 16 M_1 + 8 X_1 sm_1 - z (X_0 sm_0 + X_1 sm_1))
        // (the coefficients per column and tile come from LDS, read two ops ahead of use)
        v4i p0 = {0, 0, 0, 0}, p1 = {0, 0, 0, 0};
        uint32_t md_c = qoq_meta<0>(sd, kq), md_n = 0;
        float4 qc_c = s.qc[c][0], qc_n = make_float4(0.f, 0.f, 0.f, 0.f);
        auto promote = [&](auto jc, v4i m0, v4i m1, uint32_t md, float4 q) __attribute__((always_inline)) {
          constexpr int jb = decltype(jc)::value;
          uint32_t zb = md & 0x0F0F0F0Fu, sb = (md >> 4) & 0x0F0F0F0Fu;
          asm("" : "+v"(zb), "+v"(sb));     // (keeps the byte-wise int -> float conversions)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float z = (float)((zb >> (8 * i)) & 0xffu), s2 = (float)((sb >> (8 * i)) & 0xffu);
            float v = fmaf(z, q.w, q.z);
            v = fmaf((float)m1[i], q.y, v);
            v = fmaf((float)m0[i], q.x, v);
            acc[jb][i] = fmaf(s2, v, acc[jb][i]);
          }
        };
        static_for<TI>([&](auto tc) {
          constexpr int t = decltype(tc)::value;
          if constexpr (t == CT) claim_ahead();
          constexpr int k = t % KT2;
          v8i bop = bq0;
          bq0 = bq1;
          if constexpr (t + 2 < TI) bq1 = bfrag((t + 2) % KT2);
          if constexpr (t >= 2) after_values(bop, acc[(t - 2) / KT2]);   // (tile t - 2 promoted)
          const U4 w = wr[k];
          const v4i c0 = {(int)(w.x & 0x0F0F0F0Fu), (int)(w.y & 0x0F0F0F0Fu), (int)(w.z & 0x0F0F0F0Fu),
                          (int)(w.w & 0x0F0F0F0Fu)};
          const v4i c1 = {(int)(w.x & 0xF0F0F0F0u), (int)(w.y & 0xF0F0F0F0u), (int)(w.z & 0xF0F0F0F0u),
                          (int)(w.w & 0xF0F0F0F0u)};
          const v4i a0 = mfma_i8_16x16x64(c0, lo4(bop), v4i{0, 0, 0, 0});
          const v4i a1 = mfma_i8_16x16x64(c1, hi4(bop), v4i{0, 0, 0, 0});
          if constexpr (t + KT2 < TI) wr[k] = ld_stream_after(cb, (t + KT2) * 1024, a1);
          else wr[k] = ld_stream_after(nb, (t + KT2 - TI) * 1024, a1);
          if constexpr (t > 0) promote(std::integral_constant<int, (t - 1) / KT2>{}, p0, p1, md_n, qc_n);
          md_n = md_c;
          qc_n = qc_c;
          if constexpr (t + 1 < TI) {
            md_c = qoq_meta<t + 1>(sd, kq);
            qc_c = s.qc[c][(t + 1) % KT2];
          }
          p0 = a0;
          p1 = a1;
        });
        promote(std::integral_constant<int, (TI - 1) / KT2>{}, p0, p1, md_n, qc_n);
#pragma unroll
        for (int j = 0; j < RB; ++j) {
          acc[j][0] *= __uint_as_float(s1r[j].x);
          acc[j][1] *= __uint_as_float(s1r[j].y);
          acc[j][2] *= __uint_as_float(s1r[j].z);
          acc[j][3] *= __uint_as_float(s1r[j].w);
        }
      } else if constexpr (ACT == DGM_ACT_NVFP4) {
        U4 bn[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bn[j] = s.bst[0][lane][j];
        static_for<TI>([&](auto tc) {
          constexpr int t = decltype(tc)::value;
          if constexpr (t == CT) claim_ahead();
          constexpr int j = t / KT2, k = t % KT2;
          U4 bc[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) bc[i] = bn[i];
          if constexpr (t + 1 < TI) {
#pragma unroll
            for (int i = 0; i < 4; ++i) bn[i] = s.bst[(t + 1) % KT2][lane][i];
          }
          acc[j] = nvfp4_tile(wr[k], sr[k], bc, acc[j]);
          if constexpr (t + KT2 < TI) {
            wr[k] = ld_stream_after(cb, (t + KT2) * 1024, acc[j]);
            sr[k] = ld_stream32_after(csb, (t + KT2) * 128, acc[j]);
          } else {
            wr[k] = ld_stream_after(nb, (t + KT2 - TI) * 1024, acc[j]);
            sr[k] = ld_stream32_after(nsb, (t + KT2 - TI) * 128, acc[j]);
          }
        });
        const float gsc = s.gsl[1][s.act[a]];
#pragma unroll
        for (int j = 0; j < RB; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[j][i] *= gsc;
      } else {
        uint32_t bs0 = s.bsc[0][lane], bs1 = s.bsc[(1 % KT2) >> 2][lane];
        static_for<TI>([&](auto tc) {
          constexpr int t = decltype(tc)::value;
          if constexpr (t == CT) claim_ahead();
          constexpr int j = t / KT2, k = t % KT2;
          const v8i bop = bq0;
          const uint32_t bsw = bs0;
          bq0 = bq1;
          bs0 = bs1;
          if constexpr (t + 2 < TI) {
            bq1 = bfrag((t + 2) % KT2);
            bs1 = s.bsc[((t + 2) % KT2) >> 2][lane];
          }
          acc[j] = mfma_scale_16x16x128_sel<4, FB, k & 3, k & 3>(as_v8i(wr[k]), bop, acc[j],
                                                                 (int)sd[j * KG2 + (k >> 2)], (int)bsw);
          if constexpr (t + KT2 < TI) wr[k] = ld_stream_after(cb, (t + KT2) * 1024, acc[j]);
          else wr[k] = ld_stream_after(nb, (t + KT2 - TI) * 1024, acc[j]);
        });
      }
      // all but this loop's KT2 youngest tile loads (and scale loads) are done: the previous
      // item's stores too
      wait_vm_le<ACT == DGM_ACT_NVFP4 ? 2 * KT2 : KT2>();
      if (s0 + c < n) {
        // each route's output rounded to bf16 (the reference's per-route rule), stored slot-major
        uint16_t* dst = p.partials + (size_t)s.prow[r0 + s0 + c] * H + (NW * RB * b + RB * wv) * 16 + 4 * kq;
#pragma unroll
        for (int j = 0; j < RB; ++j)
          st_agent64(dst + 16 * j, (uint64_t)f32_to_bf16(acc[j][0]) | ((uint64_t)f32_to_bf16(acc[j][1]) << 16) |
                                       ((uint64_t)f32_to_bf16(acc[j][2]) << 32) | ((uint64_t)f32_to_bf16(acc[j][3]) << 48));
        // a token with no other local route: its y rows are this route's output (the combine of
        // one bf16 route output), written here; no arrival, no combine
        const int yt = ACT == DGM_ACT_NVFP4 ? -1 : s.ytok[r0 + s0 + c];
        if (yt >= 0) {
          uint16_t* yd = p.y + (size_t)yt * H + (NW * RB * b + RB * wv) * 16 + 4 * kq;
#pragma unroll
          for (int j = 0; j < RB; ++j)
            *reinterpret_cast<uint64_t*>(yd + 16 * j) =
                (uint64_t)f32_to_bf16(acc[j][0]) | ((uint64_t)f32_to_bf16(acc[j][1]) << 16) |
                ((uint64_t)f32_to_bf16(acc[j][2]) << 32) | ((uint64_t)f32_to_bf16(acc[j][3]) << 48);
        }
      }
      const bool bcast = last_slab && q1 < U2;
      if (tid == 0 && bcast) s.claimv[0] = more ? ahead : -1;
      __syncthreads();                                   // (1) previous outputs complete, slab free
      if (pv >= 0) arrive(pv, ps0);
      pv = q0;
      ps0 = s0;
      int q2 = U2;
      if (bcast) {
        const int raw = __builtin_amdgcn_readfirstlane(s.claimv[0]);
        q2 = raw >= 0 && 2 * G + raw < U2 ? 2 * G + raw : U2;
        if (q2 >= U2) more = false;
      }
      if (pf) {
        slab_store(s, pre);
        staged = nkey;
      }
      __syncthreads();                                   // (2) next slab visible
      if (last_slab) {
        if (nq != q0) {
#pragma unroll
          for (int g = 0; g < SW2; ++g) sd[g] = sn[g];
        }
        q0 = q1;
        q1 = q2;
        s0 = 0;
      } else {
        s0 += 16;
      }
    }
    wait_mem();               // the last item's outputs (and the dummy reads)
    __syncthreads();
    if (pv >= 0) arrive(pv, ps0);
  };
  if (p.phases & 2) {
    if (halves) l2_phase(std::integral_constant<int, 1>{});
    else l2_phase(std::integral_constant<int, RB2>{});
  }
  if (st && tid == 0) st[4] = wall_clock();

  // ================================================================ combine
  // (token t, 128-row block b) pairs, one per wave, two rows per lane, spread over the grid
  // (pair i on wave i / G of workgroup i % G): the wave's lane 0 waits until every local route
  // of t has delivered block b, then the wave sums the routes' bf16 outputs in slot order (fp32)
  // -> bf16 y. No wave waits for another's pair (measured: 1-1.5 us less at M=2-4 than eight
  // consecutive pairs per workgroup behind one barrier). The waits are only on L2 items, which
  // never wait on this phase.
  if (p.phases & 2) {
    constexpr int DIRECT_Y = ACT == DGM_ACT_NVFP4 ? 0 : 1;   // routes per token that need no combine
    constexpr int BR = 16 * NW;
    static_assert(BR == 2 * 64, "a wave's lanes cover a block, two rows each");
    const int P = p.M * NBL2;
    for (int i = (int)blockIdx.x + wv * (int)gridDim.x; i < P; i += (int)gridDim.x * NW) {
      {
        const int need = s.nslot[i / NBL2];
        if (need > DIRECT_Y && lane == 0) spin_until2(&comb[i * CNT_LINE], need, p.spin_limit, err, p.host_err);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);    // (the partial loads below come after the wait)
        const int t = i / NBL2, row = (i % NBL2) * BR + 2 * lane;
        // (y rows of tokens without a local route: zeroed by workgroup 0; with one: written by its
        // L2 unit, except NVFP4's)
        if (s.nslot[t] > DIRECT_Y) {
          // every local route's two values are requested first (one round trip for all of
          // them), then summed in slot order (fp32; a route of another rank adds nothing)
          constexpr int MAXK = 16;                       // (topk <= 16, checked on the host)
          const int tk = p.topk;
          int ex[MAXK];                                  // (all read before any is tested)
#pragma unroll
          for (int sl = 0; sl < MAXK; ++sl) ex[sl] = s.exp_of_route[min(t * tk + sl, FUSED_MAX_ROUTES - 1)];
          uint32_t v[MAXK], use = 0;
#pragma unroll
          for (int sl = 0; sl < MAXK; ++sl) {
            v[sl] = 0u;
            if (sl < tk && ex[sl] >= 0) {
              use |= 1u << sl;
              v[sl] = __hip_atomic_load(
                  reinterpret_cast<const uint32_t*>(p.partials + ((size_t)sl * p.part_rows + t) * H + row),
                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
          }
          float s0 = 0.f, s1 = 0.f;
#pragma unroll
          for (int sl = 0; sl < MAXK; ++sl)
            if ((use >> sl) & 1u) {
              s0 += __uint_as_float(v[sl] << 16);
              s1 += __uint_as_float(v[sl] & 0xffff0000u);
            }
          *reinterpret_cast<uint32_t*>(p.y + (size_t)t * H + row) =
              (uint32_t)f32_to_bf16(s0) | ((uint32_t)f32_to_bf16(s1) << 16);
        }
      }
    }
  }

  // ---------------------------------------------------------------- teardown
  // (test hook: a bounded wait on a counter nothing sets, with a zero spin limit)
  if ((p.debug & 1) && blockIdx.x == 0 && tid == 0) spin_until(p.counters + CNT_NEVER, 1, 0, err, p.host_err);
  if (!FEIN && st && tid == 0) {
    st[6] = l1_load_ticks;
    st[7] = l1_sig_ticks;
  }
  // The workgroup that counted itself last at the start hands the next launch the other
  // counter set: every workgroup of this launch has read the parity (each before counting
  // itself) and none reads it again.
  if (tid == 0 && started == (int)gridDim.x - 1)
    __hip_atomic_store(p.counters + CNT_PARITY, 1 - parity, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (st && tid == 0) st[5] = wall_clock();
}

// per device, per (shape slot, format, form: plain / FEIN / EARLY / TAIL): the resident grid; per
// (shape slot, format): the last launch's grid and form (the grid is what the device keeps
// resident at once, so it depends on the device's CU count)
constexpr int GRID_DEVICES = 64;
struct GridCache { int blocks[3][5][4] = {}; int last[3][5] = {}; int form[3][5] = {}; };
GridCache g_grid[GRID_DEVICES];

GridCache& grid_cache() {
  int dev = 0;
  (void)hipGetDevice(&dev);
  return g_grid[dev >= 0 && dev < GRID_DEVICES ? dev : 0];
}

template <int KT1, int KT2, int ACT, int FORM>
int launch_fused_t(const FusedParams& prm, int slot, hipStream_t stream, bool coop) {
  GridCache& gc = grid_cache();
  int& nb = gc.blocks[slot][ACT][FORM];
  if (nb == 0) {
    int per_cu = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_megamoe<KT1, KT2, ACT, FORM>, FT, 0);
    if (e != hipSuccess || per_cu < 1) per_cu = 1;
    int dev = 0, cus = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    nb = per_cu * (cus > 0 ? cus : 256);
  }
  gc.last[slot][ACT] = nb;
  gc.form[slot][ACT] = FORM;
  if (coop) {
    // (the grid is the device's resident capacity, which a cooperative launch requires)
    FusedParams arg = prm;
    void* args[] = {&arg};
    const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(&k_megamoe<KT1, KT2, ACT, FORM>),
                                                    dim3(nb), dim3(FT), args, 0, stream);
    if (e != hipSuccess) {
      char buf[256];
      snprintf(buf, sizeof(buf), "cooperative launch of the persistent kernel failed: %s", hipGetErrorString(e));
      dgm_set_error(buf);
      return (int)e;
    }
    return 0;
  }
  hipLaunchKernelGGL((k_megamoe<KT1, KT2, ACT, FORM>), dim3(nb), dim3(FT), 0, stream, prm);
  return dgm_last_launch_status();
}

// Early weight streaming (debug bit 3; MXFP4 / MXFP8 activations, the frontend run before the
// launch): where the routes fit one wave and at most 32 of them are expected to be local (all,
// or a share E_local / E of them under expert parallelism: decode batches of up to 4 tokens at
// top-8).
bool use_early(const FusedParams& prm, int act) {
  const long long R = (long long)prm.M * prm.topk;
  return (act == DGM_ACT_MXFP4 || act == DGM_ACT_MXFP8) && !prm.fe_in && (prm.phases & 1) && R <= 64 &&
         R * prm.E_local <= 32LL * prm.E && (prm.debug & 8);
}

// Half units for the last round of L1 units (debug bit 4; A-MXFP at H = 3072, the frontend run
// before the launch): for decode batches of up to 4 tokens at top-8 (<= 32 routes), whose units
// end in a partial round (M=2: 320 units, M=4: 640, on 256 workgroups); the kernel applies them
// when that round is at most half full. An opt-in form: measured slower (that round shares the
// HBM with the other workgroups' L2 weight streams, so halving its units does not end it
// sooner, and every half item pays a whole item's epilogue).
bool use_tail(const FusedParams& prm) {
  return !prm.fe_in && (prm.phases & 1) && (long long)prm.M * prm.topk <= 32 && (prm.debug & 16);
}

template <int KT1, int KT2, int ACT>
int launch_fused_fe(const FusedParams& prm, int slot, hipStream_t stream, bool coop) {
  if constexpr (ACT == DGM_ACT_MXFP4 || ACT == DGM_ACT_MXFP8) {
    if (use_early(prm, ACT)) return launch_fused_t<KT1, KT2, ACT, FORM_EARLY>(prm, slot, stream, coop);
    if constexpr (KT1 == 24) {
      if (use_tail(prm)) return launch_fused_t<KT1, KT2, ACT, FORM_TAIL>(prm, slot, stream, coop);
    }
  }
  return prm.fe_in ? launch_fused_t<KT1, KT2, ACT, FORM_FEIN>(prm, slot, stream, coop)
                   : launch_fused_t<KT1, KT2, ACT, FORM_PLAIN>(prm, slot, stream, coop);
}

}  // namespace

int dgm_fused_grid_blocks(int hidden, int intermediate, int act_format) {
  int slot = hidden == 3072 ? 0 : (hidden == 512 ? 1 : 2);
  if (act_format < DGM_ACT_MXFP4 || act_format > DGM_ACT_FP8F128) return 0;
  return grid_cache().last[slot][act_format];
}

int dgm_fused_form(int hidden, int intermediate, int act_format) {
  int slot = hidden == 3072 ? 0 : (hidden == 512 ? 1 : 2);
  if (act_format < DGM_ACT_MXFP4 || act_format > DGM_ACT_FP8F128) return -1;
  const GridCache& gc = grid_cache();
  return gc.last[slot][act_format] ? gc.form[slot][act_format] : -1;
}

int launch_fused(const FusedParams& prm, int hidden, int intermediate, int act, hipStream_t stream,
                 bool cooperative) {
#define DGM_FUSED_SHAPE(H_, I_, SLOT)                                                          \
  if (hidden == H_ && intermediate == I_) {                                                    \
    constexpr int KA = H_ / 128, KB = I_ / 128;                                               \
    return act == DGM_ACT_MXFP4   ? launch_fused_fe<KA, KB, DGM_ACT_MXFP4>(prm, SLOT, stream, cooperative) \
           : act == DGM_ACT_MXFP8 ? launch_fused_fe<KA, KB, DGM_ACT_MXFP8>(prm, SLOT, stream, cooperative) \
           : act == DGM_ACT_QOQ   ? launch_fused_fe<KA, KB, DGM_ACT_QOQ>(prm, SLOT, stream, cooperative)   \
           : act == DGM_ACT_NVFP4 ? launch_fused_fe<KA, KB, DGM_ACT_NVFP4>(prm, SLOT, stream, cooperative) \
                                  : launch_fused_fe<KA, KB, DGM_ACT_FP8F128>(prm, SLOT, stream, cooperative); \
  }
  DGM_FUSED_SHAPE(3072, 1280, 0)
  DGM_FUSED_SHAPE(512, 256, 1)
  DGM_FUSED_SHAPE(1024, 512, 2)
#undef DGM_FUSED_SHAPE
  dgm_set_error("fused kernel: supported (hidden, intermediate) are (3072, 1280), (512, 256), (1024, 512)");
  return DGM_ERR_INVALID_ARGUMENT;
}
