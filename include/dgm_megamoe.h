/* dgm_megamoe.h - C ABI of the MI355X (gfx950) MegaMoE layer.
 *
 * Plain pointers, sizes and a HIP stream; no torch types. Every call enqueues work on
 * `stream` and returns without host synchronisation. Return value: 0 on success,
 * DGM_ERR_INVALID_ARGUMENT (-1) when a host-side check fails (the message is available
 * from dgm_last_error()), or a positive hipError_t when a launch fails.
 *
 * Each entry cites the reference interface it replaces (path:line in the DeepGEMM
 * MegaMoE fork the interface mirrors).
 */
#ifndef DGM_MEGAMOE_H
#define DGM_MEGAMOE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DGM_ERR_INVALID_ARGUMENT (-1)

/* activation formats (the "act_format" of sm100_b200/test_mega_moe.py:57) */
#define DGM_ACT_MXFP4 0 /* E2M1 + UE8M0 per 32 (W4A4)          */
#define DGM_ACT_MXFP8 1 /* E4M3 + UE8M0 per 32 (W-MXFP4 x A-FP8) */
#define DGM_ACT_NVFP4 3 /* W4A4 NVFP4: E2M1 + E4M3 scale per 16 (activations and weights) */
#define DGM_ACT_QOQ 2   /* QoQ W4A8: int8 activations with one fp32 scale per token, QoQ weights
                           (deep_gemm/quantization_qoq_fused.py:1-11) */
#define DGM_ACT_FP8F128 4 /* E4M3 activations with one fp32 scale per 128 K
                             (per_token_cast_to_fp8(use_ue8m0=False, gran_k=128), deep_gemm/utils/math.py:26-38),
                             MXFP4 weights, FP8 intermediate with a power-of-two scale per 64: the
                             "fp8xmxfp4" split recipe (deep_gemm/mega/__init__.py:70-127, 340-446;
                             tests/test_four_api_correctness.py:54-62, 215) and the fused buffer's
                             recipe (csrc/apis/mega_fused.hpp:78-102). Both launch paths. */

/* frontend flags */
#define DGM_FE_FORCE_BALANCED 1     /* DG_FE_FORCE_BALANCED: tests/test_four_api_correctness.py:125-144 */
#define DGM_FE_ZERO_ROW_UNROUTED 2  /* DG_FE_ZERO_ROW_UNROUTED: deep_gemm/mega/__init__.py:693-696 */
#define DGM_FE_SELECT_IN_MEGA 4     /* DG_FE_SELECT_IN_MEGA: deep_gemm/mega/__init__.py:688-692 -- the frontend
                                       stops after logits + cast; the fused layer selects the top-k */
#define DGM_FE_RAW_WEIGHTS 8        /* router_renormalize=False of deep_gemm/mega/__init__.py:340-360: the routing
                                       weights are the selected logits themselves
                                       (deep_gemm/include/deep_gemm/impls/sm90_mxfp4_mega_moe.cuh:1327-1343) */
#define DGM_FE_NO_CAST 16           /* the router and top-k alone, x / x_sf untouched (the fused router of
                                       deep_gemm/include/deep_gemm/impls/sm90_mxfp4_mega_moe.cuh:1251-1279,
                                       router_input of deep_gemm/mega/__init__.py:340) */

/* Library version and the message of the last failed host-side check (thread-local). */
int dgm_version(void);
const char* dgm_last_error(void);

/* ------------------------------------------------------------------ packers
 * Replaces deep_gemm/quantization_mxfp4_fused.py:29 quantize_to_mxfp4 (rule 0) and
 * deep_gemm/quantization_mxfp4.py:52 quantize_to_mxfp4 (rule 1).
 * w_bf16 [rows, K] -> packed [rows, K/2] (Marlin nibble order), scale_e8m0 [rows, K/32]. */
int dgm_quantize_mxfp4(const void* w_bf16, int64_t rows, int64_t K, int rule,
                       void* packed, void* scale_e8m0, hipStream_t stream);

/* Element types of the weight packers' source (the reference packers take any float tensor and
 * compute on its fp32 value, weight.to(torch.float32): deep_gemm/quantization_mxfp4_fused.py:36,
 * quantization_mxfp4.py:54, quantization_nvfp4.py:62-66, quantization_qoq_fused.py:20). */
#define DGM_SRC_BF16 0
#define DGM_SRC_F16 1
#define DGM_SRC_F32 2

/* The weight packers over a source of src_dtype (DGM_SRC_*); the untyped entry points are
 * these with DGM_SRC_BF16. The source is 16-byte aligned. */
int dgm_quantize_mxfp4_typed(const void* w, int src_dtype, int64_t rows, int64_t K, int rule,
                             void* packed, void* scale_e8m0, hipStream_t stream);
int dgm_quantize_nvfp4_typed(const void* w, int src_dtype, int64_t rows, int64_t K, void* packed,
                             void* scale_ue4m3, hipStream_t stream);
int dgm_quantize_qoq_typed(const void* w, int src_dtype, int64_t rows, int64_t K, void* packed, void* s2,
                           void* z, void* s1_f32, hipStream_t stream);
int dgm_quantize_qoq_int4_typed(const void* w, int src_dtype, int64_t rows, int64_t K, void* packed,
                                void* plane_i32, hipStream_t stream);

/* Replaces sm100_b200/test_mega_moe.py:78 cast_to_fp4_rows (amax_floor 1e-30) and
 * deep_gemm/utils/math.py:85 per_token_cast_to_fp4(use_ue8m0=True, gran_k=32) (amax_floor 1e-4).
 * x_bf16 [rows, K] -> packed [rows, K/2] (low nibble = even K), sf_e8m0 [rows, K/32]. */
int dgm_cast_fp4_rows(const void* x_bf16, int64_t rows, int64_t K, float amax_floor,
                      void* packed, void* sf_e8m0, hipStream_t stream);

/* Replaces deep_gemm/utils/math.py:26 per_token_cast_to_fp8(use_ue8m0=True, gran_k=32).
 * x_bf16 [rows, K] -> q_e4m3 [rows, K], sf_e8m0 [rows, K/32]. */
int dgm_cast_fp8_rows(const void* x_bf16, int64_t rows, int64_t K, void* q_e4m3, void* sf_e8m0,
                      hipStream_t stream);

/* Replaces deep_gemm/quantization_nvfp4.py:62 quantize_to_nvfp4.
 * w_bf16 [rows, K] -> packed [rows, K/2] (Marlin), scale_ue4m3 [rows, K/16]. */
int dgm_quantize_nvfp4(const void* w_bf16, int64_t rows, int64_t K, void* packed,
                       void* scale_ue4m3, hipStream_t stream);

/* Replaces deep_gemm/quantization_qoq_fused.py:18 quantize_to_qoq.
 * w_bf16 [rows, K] -> packed [rows, K/2] (Marlin), s2 u8 [rows, K/128], z u8 [rows, K/128],
 * s1 f32 [rows]. */
int dgm_quantize_qoq(const void* w_bf16, int64_t rows, int64_t K, void* packed, void* s2,
                     void* z, void* s1_f32, hipStream_t stream);

/* Replaces deep_gemm/quantization_qoq_fused.py:78 per_token_cast_to_int8.
 * x_bf16 [rows, K] -> q_i8 [rows, K], sf_f32 [rows]. */
int dgm_cast_int8_rows(const void* x_bf16, int64_t rows, int64_t K, void* q_i8, void* sf_f32,
                       hipStream_t stream);

/* ------------------------------------------------------------------ weight layout
 * Replaces deep_gemm/mega/fused.py:64 transform_mxfp4_weights_for_mega_moe_fused (one
 * matrix per call). packed [E, N, K/2] (src_order 0 = Marlin, 1 = low-nibble-first),
 * scale_e8m0 [E, N, K/32] -> dst_values [E, N/16, K/128, 64, 16] and
 * dst_scales [E, N/16, ceil(K/512), 64, 4] (matrix-core fragment order). l1_interleave
 * pairs gate block j with up block j (16 rows each) as the kernel's SwiGLU needs: 1 for W1
 * rows [gate rows; up rows] (the reference's [E, 2I, H]), 2 for checkpoints that interleave
 * them row by row (row 2i = gate row i, row 2i+1 = up row i); 0 for W2. */
int dgm_transform_fp4_weights(const void* packed, const void* scale_e8m0, int E, int N, int K,
                              int src_order, int l1_interleave, void* dst_values,
                              void* dst_scales, hipStream_t stream);

/* Replaces the weight preparation of the W4A4 NVFP4 path (sm100_b200/mega___init__.py:102-111
 * transform_weights_for_mega_moe, deep_gemm/mega/__init__.py:174 transform_nvfp4_weights_for_mega_moe_sm90),
 * one matrix per call: packed [E, N, K/2] (src_order 0 = Marlin, 1 = low-nibble-first) and E4M3
 * scales [E, N, K/16] -> dst_values [E, N/16, K/128, 64, 16] (f16 matrix-core fragment order)
 * and dst_scales [E, N/16, K/128, 2, 16, 4] (per lane the four 16-block scales of its ops). */
int dgm_transform_nvfp4_weights(const void* packed, const void* scale_e4m3, int E, int N, int K, int src_order,
                                int l1_interleave, void* dst_values, void* dst_scales, hipStream_t stream);

/* ------------------------------------------------------------------ checkpoint formats
 * E2M1 nibble order of packed FP4 codes, any tensor of n_bytes (n_bytes % 4 == 0; 8 codes per
 * 4-byte word): order 0 = Marlin (deep_gemm/quantization_mxfp4.py:66-70 and
 * quantization_nvfp4.py:76-80: byte b = K[b] << 4 | K[b+4]), 1 = low-nibble-first (OCP MX
 * checkpoints, deep_gemm/utils/math.py:100: byte j = K[2j] | K[2j+1] << 4). src == dst converts
 * in place. Replaces the reference's torch nibble shuffles (quantization_mxfp4.py:66-70 one way,
 * quantization_nvfp4.py:176-181 back). */
int dgm_reorder_fp4_nibbles(const void* src, void* dst, int64_t n_bytes, int src_order, int dst_order,
                            hipStream_t stream);

/* Inverse of dgm_transform_fp4_weights: dst values / scales of that call -> packed [E, N, K/2]
 * in dst_order (0 Marlin, 1 low-nibble-first) and scale_e8m0 [E, N, K/32], rows in the order
 * l1_interleave names (as for dgm_transform_fp4_weights). Replaces the fused-layout inversion of
 * deep_gemm/quantization_mxfp4.py:231-262 (dequantize_mxfp4_to_fp32 with fused_input). */
int dgm_untransform_fp4_weights(const void* values, const void* scales, int E, int N, int K, int dst_order,
                                int l1_interleave, void* packed, void* scale_e8m0, hipStream_t stream);

/* Inverse of dgm_transform_nvfp4_weights: -> packed [E, N, K/2] (dst_order) and E4M3 scales
 * [E, N, K/16]. Replaces the layout inversion of deep_gemm/quantization_nvfp4.py:155-181. */
int dgm_untransform_nvfp4_weights(const void* values, const void* scales, int E, int N, int K, int dst_order,
                                  int l1_interleave, void* packed, void* scale_e4m3, hipStream_t stream);

/* Replaces deep_gemm/mega/fused.py:71 transform_qoq_weights_for_mega_moe_fused (one matrix per
 * call). packed [E, N, K/2] (Marlin), s2 / z u8 [E, N, K/128], s1 f32 [E, N] ->
 * dst_values [E, N/16, K/128, 64, 16] (int8 matrix-core fragment order, 4-bit codes; the L1
 * layout (l1_interleave = 1) pairs the nibbles of one 64-K operand, the L2 layout splits them
 * by 64-K chunk with the high one offset by 8),
 * dst_meta [E, N/16, K/128, 16] (byte r = z | s2 << 4 of row r; z and s2 must be < 16), dst_s1 f32 [E, N] (row order of
 * dst_values; l1_interleave pairs gate / up 16-row blocks). */
int dgm_transform_qoq_weights(const void* packed, const void* s2, const void* z, const void* s1, int E, int N,
                              int K, int l1_interleave, void* dst_values, void* dst_meta, void* dst_s1,
                              hipStream_t stream);

/* Replaces deep_gemm/quantization_mxfp4.py:323 quantize_to_qoq_int4 (the split path's QoQ packer):
 * bf16 [rows, K] -> Marlin-packed codes [rows, K/2] and an int32 plane [rows, K/128] holding
 * s2 | z << 8 | bf16(s1) << 16 per (row, K128 group). The codes, s2, z and s1 equal
 * dgm_quantize_qoq's. */
int dgm_quantize_qoq_int4(const void* w_bf16, int64_t rows, int64_t K, void* packed, void* plane_i32,
                          hipStream_t stream);

/* Replaces deep_gemm/mega/__init__.py:308 transform_qoq_int4_weights_for_mega_moe_sm90 (one matrix
 * per call): dgm_transform_qoq_weights with s2, z and s1 read from the int4 packer's plane
 * (z and s2 must be < 16). */
int dgm_transform_qoq_int4_weights(const void* packed, const void* plane_i32, int E, int N, int K, int l1_interleave,
                                   void* dst_values, void* dst_meta, void* dst_s1, hipStream_t stream);

/* ------------------------------------------------------------------ fused buffer
 * Replaces csrc/apis/mega_fused.hpp:31-76 get_symm_buffer_size_for_fused_mega_moe:
 * byte offsets of every view inside one device buffer (single GPU, no symmetric memory). */
typedef struct DgmBufferLayout {
  size_t total_bytes;
  size_t x, x_sf, topk_idx, topk_weights;       /* frontend outputs / fused-layer inputs  */
  size_t logits;                                /* fp32 router logits [max_tokens, E]      */
  size_t fe_keys;                               /* u32 top-k keys [max_tokens, E] (fable_frontend_keys) */
  size_t pool;                                  /* dispatch table (see DgmPoolTable)       */
  size_t mid, mid_sf;                           /* L1 -> L2 activations (pool-row order)   */
  size_t partials;                              /* bf16 [topk, max_tokens, H] route outputs (combine_partials) */
  size_t counters;                              /* int32 scratch counters                  */
  int32_t x_row_bytes, mid_row_bytes, max_routes, max_tokens;
  /* the shape the buffer was laid out for: every launch on it is refused (DGM_ERR_INVALID_ARGUMENT,
     before anything is enqueued) unless num_tokens <= max_tokens, topk <= topk, num_experts <=
     num_experts, num_local_experts <= num_local_experts, hidden (and intermediate) equal, and the
     call's activation format needs at most x_row_bytes / x_sf_row_bytes / mid_row_bytes /
     mid_sf_row_bytes per row */
  int32_t topk, num_experts, num_local_experts, hidden, intermediate, act_format;
  int32_t x_sf_row_bytes, mid_sf_row_bytes;
} DgmBufferLayout;

int dgm_fused_buffer_layout(int max_tokens, int num_experts, int num_local_experts, int topk,
                            int hidden, int intermediate, int act_format, DgmBufferLayout* out);

/* ------------------------------------------------------------------ frontend
 * Replaces csrc/fable_frontend.h:49-53 launch_router_quant_topk_frontend (and the Python
 * deep_gemm/mega/__init__.py:671 fable_router_quant_topk_frontend): bf16 router GEMV with
 * fp32 accumulation in a fixed order, bf16 logits, top-k (value desc, index asc), fp32
 * softmax of the k logits, activation cast, into the buffer views x / x_sf / topk_idx /
 * topk_weights (and the fp32 logits). The top-k keys (orderable bf16 logit << 16 | 0xFFFF - e,
 * the reference's compact key array, deep_gemm/mega/__init__.py:737) go to the fe_keys view;
 * with DGM_FE_ZERO_ROW_UNROUTED an all-zero hidden row gets zero keys (unrouted).
 * token_offset = global id of row 0 (forced-balanced rule). With DGM_FE_SELECT_IN_MEGA the
 * top-k is left to the fused layer (DgmMoeArgs.select_in_mega), which selects from the keys;
 * topk_idx / topk_weights are written by that call instead. router_weight_bf16 NULL: the
 * activation cast alone (the hidden_input path of deep_gemm/mega/__init__.py:340
 * mxfp4_mega_moe, sm90_mxfp4_mega_moe.cuh:1208-1243), no routing flags. */
int dgm_router_topk_launch(const void* hidden_bf16, const void* router_weight_bf16,
                           int num_tokens, int hidden, int num_experts, int topk, int act_format,
                           int flags, int token_offset, void* buffer,
                           const DgmBufferLayout* layout, hipStream_t stream);

/* dgm_router_topk_launch with the reference's frontend phase stamps (stamps=1 of
 * deep_gemm/mega/__init__.py:671, read back by fable_frontend_stamps, :743-756): stamps is
 * int64 [stamp_rows, 8]; frontend workgroup b (< stamp_rows; rows are the router workgroups,
 * then the cast workgroups) writes [0] entry, [3] its logits and keys stored (router rows),
 * [5] its cast stored (cast rows), [6] its hardware position (HW_ID | XCC_ID << 32), [7] exit,
 * on the 100 MHz wall clock; unused slots 0. NULL / 0 rows = no stamps. */
int dgm_router_topk_launch_stamped(const void* hidden_bf16, const void* router_weight_bf16,
                                   int num_tokens, int hidden, int num_experts, int topk, int act_format,
                                   int flags, int token_offset, void* buffer, const DgmBufferLayout* layout,
                                   int64_t* stamps, int stamp_rows, hipStream_t stream);

/* Workgroups of the frontend launch for a shape (router = 0: the cast alone), i.e. the rows
 * dgm_router_topk_launch_stamped can stamp. Replaces deep_gemm/mega/__init__.py:653
 * fable_frontend_router_ctas for sizing the stamps (that one counts router workgroups only). */
int dgm_frontend_workgroups(int num_tokens, int hidden, int num_experts, int act_format, int flags, int router);

/* Replaces the router_logits input of deep_gemm/mega/__init__.py:340 mxfp4_mega_moe (the SM90
 * kernel's kRouterLogitsInput path, deep_gemm/include/deep_gemm/impls/sm90_mxfp4_mega_moe.cuh:1295-1343):
 * bf16 logits [num_tokens, num_experts] -> the top-k keys (fe_keys view) and, unless
 * DGM_FE_SELECT_IN_MEGA, topk_idx / topk_weights: the k largest logits (ties: the lower expert),
 * weights = softmax over them, or the logits themselves with DGM_FE_RAW_WEIGHTS.
 * DGM_FE_FORCE_BALANCED as for dgm_router_topk_launch. */
int dgm_router_logits_topk_launch(const void* logits_bf16, int num_tokens, int num_experts, int topk, int flags,
                                  int token_offset, void* buffer, const DgmBufferLayout* layout, hipStream_t stream);

/* ------------------------------------------------------------------ fused layer
 * Replaces csrc/apis/mega_fused.hpp:78-102 run_fused / _C.mxfp4_mega_moe_fused and
 * deep_gemm/mega/fused.py:97 mxfp4_mega_moe_fused for one GPU's share of the layer:
 * dispatch of the buffer's topk_idx into per-expert pools (token asc, slot asc), L1
 * grouped GEMM (gate/up) + SwiGLU + requant, L2 grouped GEMM, top-k weighted combine. */
typedef struct DgmMoeArgs {
  int32_t num_tokens, hidden, intermediate, num_experts, expert_begin, num_local_experts, topk;
  int32_t act_format;
  float activation_clamp;
  int32_t fast_math;      /* 1: hardware exp2 / reciprocal in SiLU (reference default) */
  int32_t select_in_mega; /* 1: select the top-k from a key array (fe_keys, else the buffer's keys
                             after a DGM_FE_SELECT_IN_MEGA frontend call) and write topk_idx / weights */
  int32_t fe_flags;       /* with select_in_mega: the frontend's DGM_FE_* flags */
  int32_t token_offset;   /* with select_in_mega: global id of row 0 */
  const void* w1_values;  /* [E_local, 2I/16, H/128, 64, 16] */
  const void* w1_scales;  /* MXFP: [E_local, 2I/16, ceil(H/512), 64, 4]; QoQ: meta [E_local, 2I/16, H/128, 16];
                             NVFP4: [E_local, 2I/16, H/128, 2, 16, 4] */
  const void* w2_values;  /* [E_local, H/16, I/128, 64, 16] */
  const void* w2_scales;  /* MXFP: [E_local, H/16, ceil(I/512), 64, 4]; QoQ: meta [E_local, H/16, I/128, 16];
                             NVFP4: [E_local, H/16, I/128, 2, 16, 4] */
  int32_t* recv_stats;    /* [E_local] cumulative_local_expert_recv_stats, may be NULL */
  void* y;                /* bf16 [num_tokens, hidden] */
  void* buffer;
  const DgmBufferLayout* layout;
  int64_t* phase_stamps;  /* optional [phase_stamp_rows, 8] wall-clock stamps (phase_stamps of
                             deep_gemm/mega/fused.py:97); NULL = off. Workgroups beyond
                             phase_stamp_rows record nothing. */
  int32_t phase_stamp_rows;
  const float* w1_row_scales; /* QoQ: s1 [E_local, 2I] (dgm_transform_qoq_weights order); else unused */
  const float* w2_row_scales; /* QoQ: s1 [E_local, H]; else unused */
  const float* l1_global_scales; /* NVFP4: optional fp32 [E_local] per-expert scale of the L1 output
                                    (deep_gemm/mega/__init__.py:277 nvfp4_mega_moe); NULL = 1 */
  const float* l2_global_scales; /* NVFP4: the same for the L2 output */
  /* In-kernel frontend (deep_gemm/mega/__init__.py:451 mxfp4_mega_moe_from_bf16 as one launch):
   * with fe_in_mega = 1 the kernel first computes the router logits, zero-row flags and the
   * activation cast into the buffer (the work of dgm_router_topk_launch) of hidden_states, then selects
   * the top-k itself (select_in_mega is implied; num_tokens <= 64). fe_flags / token_offset as
   * for dgm_router_topk_launch. */
  int32_t fe_in_mega;
  const void* hidden_states; /* bf16 [num_tokens, hidden] */
  const void* router_weight; /* bf16 [num_experts, hidden] */
  /* With select_in_mega: the u32 key array [num_tokens, num_experts] to select from (the fe_keys
   * argument of deep_gemm/mega/fused.py:97; a token whose first key is 0 is unrouted); NULL = the
   * buffer's fe_keys view. */
  const void* fe_keys;
  /* Optional host-visible int32 word (pinned host memory, device-accessible): set to 1 when a
   * bounded wait of the persistent kernel expires, beside the buffer's error counter, so the
   * host can check a launch's outcome later without synchronising. NULL = none. */
  int32_t* host_error;
  /* Test hook, 0 in normal use. Bit 0: the persistent kernel additionally runs one bounded wait
   * on a counter nothing sets, with a zero spin limit, so the wait expires and the error
   * reporting (error counter, host_error) can be tested without a real failure. Bit 1 (QoQ, the
   * persistent kernel): phase_stamps receives the exact int32 L1 accumulators
   * (sum over K128 groups of s2 * sum (code - z) * x8, per route in pool order and W1 row, gate
   * rows then up rows: int32 [routes][2 I]) instead of stamps, for bit-exact tests. Bit 2: the
   * persistent kernel runs whole L2 units even where it would run half units (units filling at
   * most half the grid), so tests cover both forms at small shapes. Bit 3: the persistent kernel
   * runs its early-weight-streaming form where that form applies (at most 32 local routes
   * expected, MXFP4 / MXFP8 activations, the frontend run before the launch): the first L1
   * unit's weight tiles are requested before the pool table is built. Measured slower than the
   * default form at every size it applies to; kept so tests and benchmarks can compare them.
   * Bit 4: the persistent kernel runs its tail-half-unit form where that form applies (up to 32
   * routes, MXFP4 / MXFP8 activations, hidden 3072: the last round of L1 units, when at most half
   * full, runs as half units of 32 features, each 16-row block's K split over two waves).
   * Measured slower than the default form; kept so tests and benchmarks can compare them. */
  int32_t debug_flags;
  /* DGM_LAUNCH_* flags, 0 = the default plain launch. The persistent kernel's workgroups wait on
   * each other (bounded), so they must all be resident at once: the plain launch sizes the grid
   * to what the device keeps resident, which holds when no other work occupies the compute
   * units. DGM_LAUNCH_COOPERATIVE launches it cooperatively (hipLaunchCooperativeKernel), which
   * guarantees co-residency for callers that share the GPU with other streams or processes, at
   * a cost of ~14-19 us per call on MI355X. No counterpart in the reference (a plain launch). */
  int32_t launch_flags;
} DgmMoeArgs;

#define DGM_LAUNCH_COOPERATIVE 1

int dgm_megamoe_fused_launch(const DgmMoeArgs* args, hipStream_t stream);

/* No counterpart in the reference: dgm_megamoe_fused_launch for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * The same layer, but the persistent kernel's workspace (dispatch table, L1 -> L2 rows, route
 * outputs, counters) is a file-scope device array of ~4.9 MB held by each GPU the library runs on,
 * not the buffer's views: the buffer supplies only the inputs (x / x_sf, or the keys / topk views)
 * and args->y the output; the buffer's pool, l2_acts and combine_partials views are not written.
 * Limits: num_tokens * topk <= 512, num_tokens <= 256, hidden <= 3072, intermediate <= 1280
 * (beyond them: DGM_ERR_INVALID_ARGUMENT, nothing launched). No hipMalloc / hipFree is called;
 * the first call on a device clears the array's counters with a fill kernel on `stream`, and
 * every launch clears the counter set that the next launch uses. All calls on one GPU share its array: calls that overlap
 * (unordered streams) race. Expired waits are reported only through args->host_error. */
int dgm_megamoe_fused_launch_noalloc(const DgmMoeArgs* args, hipStream_t stream);

/* Replaces csrc/apis/mega.hpp:550 _C.mxfp4_mega_moe_split / deep_gemm/mega/__init__.py:579
 * mxfp4_mega_moe_split and :584 qoq_mega_moe_split: the same layer as separate launches instead
 * of one persistent kernel, identical numerics. MXFP4 / MXFP8: dispatch, L1, L2, combine
 * kernels; QoQ / NVFP4: the persistent kernel twice, dispatch + L1 then L2 + combine (the
 * fused kernel's limits on tokens, routes and local experts apply). fe_in_mega is rejected. */
int dgm_megamoe_split_launch(const DgmMoeArgs* args, hipStream_t stream);

/* Device address of pinned host memory (hipHostGetDevicePointer), e.g. for
 * DgmMoeArgs.host_error. No counterpart in the reference (its error path is a device trap). */
int dgm_host_device_pointer(const void* host, void** device);

/* Diagnostics (no counterpart in the reference). dgm_device_cu_count: compute units of the
 * current device. dgm_fused_workgroups: workgroups of the persistent kernel for a shape (0 before
 * its first launch). dgm_fused_last_form: the form its last launch for a shape ran, 0 plain,
 * 1 with the in-kernel frontend, 2 with early weight streaming, 3 with tail half units (-1
 * before its first launch).
 * The lane-layout probes of the tests live in a library of their own (include/dgm_probe.h). */
int dgm_device_cu_count(void);
int dgm_fused_workgroups(int hidden, int intermediate, int act_format);
/* sizeof(DgmMoeArgs) and sizeof(DgmBufferLayout) as this library was built, so a binding can
 * check its own struct layouts against the library's (no counterpart in the reference). */
int dgm_abi_struct_sizes(size_t* moe_args, size_t* buffer_layout);
int dgm_fused_last_form(int hidden, int intermediate, int act_format);

#ifdef __cplusplus
}
#endif
#endif /* DGM_MEGAMOE_H */
