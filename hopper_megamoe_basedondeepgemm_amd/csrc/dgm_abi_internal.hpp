// Host-side helpers shared by the C-ABI translation units: argument checks that record a
// message (the reference's DG_HOST_ASSERT shape: "Assertion failed: <file>:<line>: <cond>")
// and the workspace layout of one fused MegaMoE buffer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/dgm_megamoe.h"

void dgm_set_error(const char* msg);

#define DGM_STR2(x) #x
#define DGM_STR(x) DGM_STR2(x)
#define DGM_CHECK_ARG(cond, what)                                                          \
  do {                                                                                     \
    if (!(cond)) {                                                                         \
      dgm_set_error("Assertion failed: " __FILE__ ":" DGM_STR(__LINE__) ": " #cond " (" what ")"); \
      return DGM_ERR_INVALID_ARGUMENT;                                                     \
    }                                                                                      \
  } while (0)

static inline int dgm_last_launch_status() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char buf[256];
    snprintf(buf, sizeof(buf), "HIP launch failed: %s", hipGetErrorString(e));
    dgm_set_error(buf);
    return (int)e;
  }
  return 0;
}

static constexpr inline size_t dgm_align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Bytes of the dispatch table of E_local experts and max_routes routes (meta line, counts,
// active list, offsets, route ids; each 256-byte aligned).
static constexpr inline size_t dgm_pool_bytes(int E_local, int max_routes) {
  return 256 + dgm_align256((size_t)E_local * 4) * 2 + dgm_align256((size_t)(E_local + 1) * 4) +
         dgm_align256((size_t)max_routes * 4);
}

// Device memory the persistent kernel uses beyond its inputs and outputs: the dispatch table,
// the L1 -> L2 rows and scales, the bf16 route outputs ([topk][part_rows][H]) and the int32
// counters (which start at zero and are returned to zero by every launch).
struct DgmWorkspace {
  uint8_t* pool;
  uint8_t* mid;
  uint8_t* mid_sf;
  uint16_t* partials;
  int part_rows;
  int* counters;
};

// Row bytes of the activation codes / scales and of the intermediate codes / scales that a call in
// act_format needs (hidden H, intermediate I): MXFP4 / NVFP4 codes are half a byte, the others a
// byte; x scales E8M0 per 32 (NVFP4 E4M3 per 16; QoQ and FP8F128 fp32 per 128, the same H / 32
// bytes); intermediate scales E8M0 per 32 (QoQ fp32 per 64, NVFP4 E4M3 per 16, FP8F128 sized as
// QoQ's).
struct DgmRowBytes { size_t x, x_sf, mid, mid_sf; };
static inline DgmRowBytes dgm_row_bytes(int act_format, int hidden, int intermediate) {
  const bool fp4 = act_format == DGM_ACT_MXFP4 || act_format == DGM_ACT_NVFP4;
  DgmRowBytes r;
  r.x = fp4 ? hidden / 2 : hidden;
  r.x_sf = act_format == DGM_ACT_NVFP4 ? hidden / 16 : hidden / 32;
  r.mid = fp4 ? intermediate / 2 : intermediate;
  r.mid_sf = act_format == DGM_ACT_QOQ || act_format == DGM_ACT_NVFP4 || act_format == DGM_ACT_FP8F128
                 ? intermediate / 16 : intermediate / 32;
  return r;
}
// A call's shape against the shape its buffer was laid out for (intermediate < 0: a frontend
// call, which writes no intermediate rows; num_local_experts < 0: not checked). 0, or
// DGM_ERR_INVALID_ARGUMENT with the message set.
int dgm_check_layout_call(const DgmBufferLayout* L, int num_tokens, int topk, int num_experts, int num_local_experts,
                          int hidden, int intermediate, int act_format);
// Host-side checks of a fused-layer call (0, or DGM_ERR_INVALID_ARGUMENT with the message set).
int dgm_check_fused_args(const DgmMoeArgs* A);
// One launch of the persistent kernel over the workspace w, running `phases` of the layer
// (1: dispatch + L1, 2: L2 + combine, 3: both); the top-k selection launch first when the
// call selects from keys above the in-kernel selection's token count.
int dgm_fused_launch_ws(const DgmMoeArgs* A, int phases, const DgmWorkspace& w, hipStream_t stream);
