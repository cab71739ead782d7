// Diagnostic: one block-scaled matrix-core op on caller-provided lane fragments, so the
// tests can check the lane layout the kernels assume (A row l%16 / B column l%16, K chunk
// 32*(l/16), scale byte of that 32-block; D[4*(l/16)+i][l%16] in result register i).
#include "dgm_common.hpp"
#include "dgm_abi_internal.hpp"

using namespace dgm;

template <int FA, int FB>
__global__ void k_probe(const v8i* a, const v8i* b, const int* sa, const int* sb, float* out) {
  int l = threadIdx.x;
  v4f c = {0.f, 0.f, 0.f, 0.f};
  c = mfma_scale_16x16x128<FA, FB>(a[l], b[l], c, sa[l], sb[l]);
  for (int i = 0; i < 4; ++i) out[l * 4 + i] = c[i];
}

template <int SEL>
__global__ void k_probe_sel(const v8i* a, const v8i* b, const int* sa, const int* sb, float* out) {
  int l = threadIdx.x;
  v4f c = {0.f, 0.f, 0.f, 0.f};
  c = mfma_scale_16x16x128_sel<4, 4, SEL, SEL>(a[l], b[l], c, sa[l], sb[l]);
  for (int i = 0; i < 4; ++i) out[l * 4 + i] = c[i];
}

// Byte select of the scale words (E2M1 x E2M1): the scale used is byte `sel` of sa / sb.
extern "C" int dgm_probe_mfma_scale_sel(const void* a, const void* b, const void* sa, const void* sb,
                                        void* out, int sel, hipStream_t stream) {
  DGM_CHECK_ARG(a && b && sa && sb && out && sel >= 0 && sel < 4, "bad argument");
  const v8i* A = (const v8i*)a;
  const v8i* B = (const v8i*)b;
  switch (sel) {
    case 0: hipLaunchKernelGGL((k_probe_sel<0>), dim3(1), dim3(64), 0, stream, A, B, (const int*)sa, (const int*)sb, (float*)out); break;
    case 1: hipLaunchKernelGGL((k_probe_sel<1>), dim3(1), dim3(64), 0, stream, A, B, (const int*)sa, (const int*)sb, (float*)out); break;
    case 2: hipLaunchKernelGGL((k_probe_sel<2>), dim3(1), dim3(64), 0, stream, A, B, (const int*)sa, (const int*)sb, (float*)out); break;
    default: hipLaunchKernelGGL((k_probe_sel<3>), dim3(1), dim3(64), 0, stream, A, B, (const int*)sa, (const int*)sb, (float*)out); break;
  }
  return dgm_last_launch_status();
}

extern "C" int dgm_probe_mfma_scale(const void* a, const void* b, const void* sa, const void* sb,
                                    void* out, int fmt_a, int fmt_b, hipStream_t stream) {
  DGM_CHECK_ARG(a && b && sa && sb && out, "null pointer");
  const v8i* A = (const v8i*)a;
  const v8i* B = (const v8i*)b;
  if (fmt_a == 4 && fmt_b == 4)
    hipLaunchKernelGGL((k_probe<4, 4>), dim3(1), dim3(64), 0, stream, A, B, (const int*)sa, (const int*)sb, (float*)out);
  else if (fmt_a == 4 && fmt_b == 0)
    hipLaunchKernelGGL((k_probe<4, 0>), dim3(1), dim3(64), 0, stream, A, B, (const int*)sa, (const int*)sb, (float*)out);
  else if (fmt_a == 0 && fmt_b == 0)
    hipLaunchKernelGGL((k_probe<0, 0>), dim3(1), dim3(64), 0, stream, A, B, (const int*)sa, (const int*)sb, (float*)out);
  else
    DGM_CHECK_ARG(false, "fmt pairs (4,4), (4,0), (0,0)");
  return dgm_last_launch_status();
}

// One int8 matrix-core op (V_MFMA_I32_16X16X64_I8) on caller-provided lane fragments
// (a, b: 64 x 16 bytes; out: 64 x 4 int32), to pin the lane layout of the W4A8 path.
__global__ void k_probe_i8(const v4i* a, const v4i* b, v4i* out) {
  const int l = threadIdx.x;
  v4i c = {0, 0, 0, 0};
  c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[l], b[l], c, 0, 0, 0);
  out[l] = c;
}

extern "C" int dgm_probe_mfma_i8(const void* a, const void* b, void* out, hipStream_t stream) {
  DGM_CHECK_ARG(a && b && out, "null pointer");
  hipLaunchKernelGGL(k_probe_i8, dim3(1), dim3(64), 0, stream, (const v4i*)a, (const v4i*)b, (v4i*)out);
  return dgm_last_launch_status();
}

// One f16 matrix-core op (V_MFMA_F32_16X16X32_F16) on caller-provided lane fragments (a, b:
// 64 x 8 halves; out: 64 x 4 fp32), to pin the lane layout of the NVFP4 path.
__global__ void k_probe_f16(const v8h* a, const v8h* b, v4f* out) {
  const int l = threadIdx.x;
  v4f c = {0.f, 0.f, 0.f, 0.f};
  out[l] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[l], b[l], c, 0, 0, 0);
}

extern "C" int dgm_probe_mfma_f16(const void* a, const void* b, void* out, hipStream_t stream) {
  DGM_CHECK_ARG(a && b && out, "null pointer");
  hipLaunchKernelGGL(k_probe_f16, dim3(1), dim3(64), 0, stream, (const v8h*)a, (const v8h*)b, (v4f*)out);
  return dgm_last_launch_status();
}

// The conversions of the NVFP4 path: for each i < n, out_h[4 i + j] = the two f16 of
// V_CVT_SCALEF32_PK_F16_FP4 on byte j of src[i] with the fp32 scale[i]; out_f[4 i + j] =
// V_CVT_F32_FP8 of byte j of src[i] (E4M3).
__global__ void k_probe_cvt(const uint32_t* src, const float* scale, uint32_t* out_h, float* out_f, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t v = src[i];
  const float sc = scale[i];
  out_h[4 * i + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 0));
  out_h[4 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 1));
  out_h[4 * i + 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 2));
  out_h[4 * i + 3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 3));
  out_f[4 * i + 0] = __builtin_amdgcn_cvt_f32_fp8((int)v, 0);
  out_f[4 * i + 1] = __builtin_amdgcn_cvt_f32_fp8((int)v, 1);
  out_f[4 * i + 2] = __builtin_amdgcn_cvt_f32_fp8((int)v, 2);
  out_f[4 * i + 3] = __builtin_amdgcn_cvt_f32_fp8((int)v, 3);
}

extern "C" int dgm_probe_cvt_fp4(const void* src, const void* scale, void* out_h, void* out_f, int n,
                                 hipStream_t stream) {
  DGM_CHECK_ARG(src && scale && out_h && out_f && n >= 0, "null pointer or n < 0");
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_probe_cvt, dim3((n + 255) / 256), dim3(256), 0, stream, (const uint32_t*)src,
                     (const float*)scale, (uint32_t*)out_h, (float*)out_f, n);
  return dgm_last_launch_status();
}
