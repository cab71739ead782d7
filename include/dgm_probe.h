/* dgm_probe.h - test-only probes of the MI355X MegaMoE build (libdgm_probe.so).
 *
 * Not part of the layer's library and with no counterpart in the reference: single gfx950
 * instructions on caller-provided lane data, so the tests can pin the lane layouts and
 * conversions the kernels assume. Device pointers; 0 on success, -1 on a bad argument, a
 * positive hipError_t when the launch fails.
 */
#ifndef DGM_PROBE_H
#define DGM_PROBE_H

#include <hip/hip_runtime.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One V_MFMA_SCALE_F32_16X16X128_F8F6F4 on 64 lane fragments (a, b: 64 x 32 bytes; sa, sb: 64
 * int32 scale words; out: 64 x 4 fp32). fmt 4 = E2M1, 0 = E4M3; pairs (4,4), (4,0), (0,0). */
int dgm_probe_mfma_scale(const void* a, const void* b, const void* sa, const void* sb, void* out,
                         int fmt_a, int fmt_b, hipStream_t stream);
/* Same with E2M1 x E2M1 operands and the scale taken from byte `sel` (0..3) of sa / sb. */
int dgm_probe_mfma_scale_sel(const void* a, const void* b, const void* sa, const void* sb, void* out,
                             int sel, hipStream_t stream);
/* One int8 op (V_MFMA_I32_16X16X64_I8): a, b 64 x 16 bytes, out 64 x 4 int32. */
int dgm_probe_mfma_i8(const void* a, const void* b, void* out, hipStream_t stream);
/* Same for V_MFMA_F32_16X16X32_F16 (a, b: 64 x 8 halves; out: 64 x 4 fp32), and the NVFP4 path's
 * conversions: for i < n, out_h[4i+j] = V_CVT_SCALEF32_PK_F16_FP4(byte j of src[i], scale[i])
 * (two f16), out_f[4i+j] = V_CVT_F32_FP8(byte j of src[i]) (E4M3). */
int dgm_probe_mfma_f16(const void* a, const void* b, void* out, hipStream_t stream);
int dgm_probe_cvt_fp4(const void* src, const void* scale, void* out_h, void* out_f, int n, hipStream_t stream);
/* GLOBAL_LOAD_LDS_DWORDX4 with a wave-uniform LDS base: four waves each load 1 KB of src (4 KB)
 * into LDS and read back the 16 bytes at base + 16 * lane (out: 256 x 16 bytes). */
int dgm_probe_global_load_lds(const void* src, void* out, hipStream_t stream);

/* Platform probes (the figures the fused kernel's design is measured against).
 * dgm_probe_stream_read: HBM read bandwidth of the fused kernel's streaming pattern without its
 * arithmetic: `blocks` workgroups of 8 waves; each wave reads runs of 24 consecutive 1 KB tiles
 * (the first bytes / 24 KB whole runs of src, 16-byte aligned, each read once) through a ring of
 * `depth` (4, 12 or 24) non-temporal loads. sink: one writable device word.
 * dgm_probe_empty_launch: a kernel of `blocks` x `threads` that returns at entry (the launch
 * floor). */
int dgm_probe_stream_read(const void* src, int64_t bytes, int depth, int blocks, void* sink, hipStream_t stream);
int dgm_probe_empty_launch(int blocks, int threads, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* DGM_PROBE_H */
