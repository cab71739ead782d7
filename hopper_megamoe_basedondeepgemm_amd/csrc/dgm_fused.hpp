// Parameters and limits of the persistent MegaMoE kernel (dgm_fused.hip).
#pragma once
#include <stdint.h>
#include <hip/hip_runtime.h>

constexpr int FUSED_MAX_ROUTES = 1024;   // tokens * topk per call
constexpr int FUSED_MAX_LOCAL = 512;     // local experts
constexpr int FUSED_MAX_TOKENS = 256;    // tokens per call
constexpr int FUSED_MAX_NB64 = 64;       // hidden / 64 (hidden <= 4096); combine uses hidden / 128

// int32 counters in the buffer's counter region. Counters that many workgroups update at once
// sit on 64-byte lines of their own (device-scope atomics on one line serialize).
// A header line, then two counter sets: a launch uses set `parity` (header word 0) and clears
// the other set, whose last user (the previous launch on this buffer) has completed; once
// every workgroup has read the parity (each counts itself in CNT_STARTED after reading it), the
// last one to count flips it. So no workgroup clears counters or waits on an atomic at the end
// of a launch, and the state lives in device memory only (graph replays included).
constexpr int CNT_LINE = 16;             // ints per 64-byte line
constexpr int CNT_PARITY = 0;            // header: the counter set the next launch uses
constexpr int CNT_ERROR = 1;             // header: set when a bounded wait expired
constexpr int CNT_NEVER = 2;             // header: never incremented: the target of the debug wait
constexpr int CNT_SET0 = CNT_LINE;       // the first set (the second follows it)
// within a set (every counter at the start of its own line):
constexpr int CNT_STARTED = 0;           // workgroups that have read the parity
constexpr int CNT_CLAIM = CNT_LINE;      // next unclaimed L1 unit; [CNT_CLAIM + CNT_LINE]: L2 unit
constexpr int CNT_L1 = 4 * CNT_LINE;     // L1 units done per active expert slot, one line each
constexpr int CNT_COMB = CNT_L1 + FUSED_MAX_LOCAL * CNT_LINE;   // combine arrivals per (token, 128-row block), one line each
constexpr int CNT_TOTAL = CNT_COMB + FUSED_MAX_TOKENS * (FUSED_MAX_NB64 / 2) * CNT_LINE;
// in-kernel frontend: workgroups past the frontend work, counted on GRID_SLOTS counters (one
// per 64-byte line; workgroup g arrives on slot g % GRID_SLOTS), so the arrivals do not all
// serialize on one address
constexpr int CNT_GRID = CNT_TOTAL;
constexpr int GRID_SLOTS = 32, GRID_STRIDE = 16;
constexpr int CNT_SET = CNT_GRID + 1024;                 // ints per set
constexpr int CNT_ALL = CNT_SET0 + 2 * CNT_SET;

inline __host__ __device__ int a256i(int x) { return (x + 255) & ~255; }

struct FusedParams {
  // (pointers first, then the scalars; the whole block is four 64-byte lines, read at kernel
  // entry: line 0 from w1v, line 1 from x, line 2 from partials, line 3 from router_w)
  const uint8_t* w1v;
  const uint32_t* w1s;
  const uint8_t* w2v;
  const uint32_t* w2s;
  const float* w1r;         // QoQ: per-row weight scales s1 [E_local, N] (null for MXFP4)
  const float* w2r;
  const float* gs1;         // NVFP4: optional per-expert scales of the L1 / L2 outputs (null = 1)
  const float* gs2;
  const uint8_t* x;
  const uint8_t* xsf;
  int64_t* topk_idx;        // read, or written by workgroup 0 when select != 0
  float* topk_w;
  const uint32_t* keys;     // select != 0: top-k keys [M, E] (an unrouted token's row starts with 0)
  float* logits;            // fe_in: fp32 router logits [M, E] written beside the keys
  uint8_t* mid;
  uint8_t* mid_sf;
  uint16_t* partials;       // bf16 route outputs [topk][part_rows][H] (slot-major)
  uint16_t* y;
  uint8_t* pool_out;
  int* recv_stats;
  int* counters;
  int* host_err;            // optional host-visible word set with the error counter (NULL: none)
  long long* stamps;        // optional [stamp_rows][8] wall-clock stamps (see k_megamoe)
  const uint16_t* hidden;   // fe_in: bf16 [M, H] hidden states and bf16 [E, H] router weights
  const uint16_t* router_w;
  int stamp_rows;
  int M, topk, expert_begin, E_local;
  int fe_flags, token_offset, E;   // DGM_FE_* flags of the top-k selection, row 0's global id, experts
  int part_rows;            // rows per slot of `partials` (the buffer's max_tokens)
  int spin_limit;
  float clamp;
  int16_t select;           // select the top-k in the prologue from `keys`
  int16_t fe_in;            // run the frontend (router + cast) in the kernel first: needs select
  int16_t fast_math;
  // Phases run by this launch: bit 0 dispatch + L1 (intermediate rows to `mid`, recv stats),
  // bit 1 L2 + combine. 3 = the whole layer; 1 then 2 = the split API's two launches (the
  // second reads the top-k written by the first and does not wait for L1 arrivals).
  int16_t phases;
  int16_t debug;            // bit 0: one bounded wait that expires (tests of the error reporting);
                            // bit 1 (QoQ): the int32 L1 accumulators to `stamps` [routes][2 I];
                            // bit 2: whole L2 units only; bit 3: early weight streaming;
                            // bit 4: tail half units
};

// cooperative: hipLaunchCooperativeKernel (co-residency guaranteed) instead of a plain launch
int launch_fused(const FusedParams& prm, int hidden, int intermediate, int act, hipStream_t stream,
                 bool cooperative = false);
int dgm_fused_grid_blocks(int hidden, int intermediate, int act_format);
int dgm_fused_form(int hidden, int intermediate, int act_format);
