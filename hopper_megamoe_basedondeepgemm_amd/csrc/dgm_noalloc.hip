// The fused MegaMoE layer with no device allocation on the call path or in its workspace: the
// persistent kernel's workspace (dispatch table, L1 -> L2 rows and scales, bf16 route outputs,
// int32 counters) lives in one file-scope device array, `scratch`, of a fixed maximum size,
// instead of the caller's buffer. For callers that cannot allocate (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc). Every call on a device shares that
// device's array: calls that overlap on one GPU race (they must be ordered, e.g. on one stream).
#include <mutex>

#include "dgm_abi_internal.hpp"
#include "dgm_fused.hpp"

namespace {

// Limits of the array: routes (tokens * topk), hidden and intermediate sizes (the largest shape
// the persistent kernel is built for: H 3072, I 1280).
constexpr int NA_MAX_ROUTES = 512;
constexpr int NA_MAX_HIDDEN = 3072;
constexpr int NA_MAX_INTER = 1280;
// Regions (each 256-byte aligned): counters, dispatch table, intermediate rows (at most one byte
// per feature) and their scales (at most I / 16 bytes per row), route outputs (bf16).
constexpr size_t NA_OFF_CNT = 0;
constexpr size_t NA_OFF_POOL = NA_OFF_CNT + dgm_align256((size_t)CNT_ALL * 4);
constexpr size_t NA_OFF_MID = NA_OFF_POOL + dgm_align256(dgm_pool_bytes(FUSED_MAX_LOCAL, NA_MAX_ROUTES));
constexpr size_t NA_OFF_MID_SF = NA_OFF_MID + dgm_align256((size_t)NA_MAX_ROUTES * NA_MAX_INTER);
constexpr size_t NA_OFF_PART = NA_OFF_MID_SF + dgm_align256((size_t)NA_MAX_ROUTES * (NA_MAX_INTER / 16));
constexpr size_t NA_BYTES = NA_OFF_PART + dgm_align256((size_t)NA_MAX_ROUTES * NA_MAX_HIDDEN * 2);
static_assert(NA_BYTES < 5u * 1024 * 1024, "a modest array");

constexpr int NA_MAX_DEVICES = 64;

}  // namespace

// The workspace array. In host code its name is a host-side stand-in, not a device address:
// only the per-device address from hipGetSymbolAddress below is ever passed to a kernel.
static __device__ __align__(256) uint8_t scratch[NA_BYTES];

namespace {

std::mutex g_na_mu;
uint8_t* g_na_ptr[NA_MAX_DEVICES];        // device address of `scratch` per device (null: not set up)

__global__ void k_na_clear(uint32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// Once per device, with that device current: the array's device address, and its counters
// cleared by a fill kernel on `stream` (every launch then clears the counter set that the next
// launch uses).
int na_setup(int dev, hipStream_t stream, uint8_t** out) {
  std::lock_guard<std::mutex> lk(g_na_mu);
  if (!g_na_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      dgm_set_error("no-alloc layer: hipGetSymbolAddress of the workspace array failed");
      return e != hipSuccess ? (int)e : DGM_ERR_INVALID_ARGUMENT;
    }
    constexpr int n = (int)(dgm_align256((size_t)CNT_ALL * 4) / 4);
    hipLaunchKernelGGL(k_na_clear, dim3(64), dim3(256), 0, stream, (uint32_t*)((uint8_t*)ptr + NA_OFF_CNT), n);
    const int st = dgm_last_launch_status();
    if (st) return st;
    g_na_ptr[dev] = (uint8_t*)ptr;
  }
  *out = g_na_ptr[dev];
  return 0;
}

}  // namespace

extern "C" int dgm_megamoe_fused_launch_noalloc(const DgmMoeArgs* A, hipStream_t stream) {
  const int chk = dgm_check_fused_args(A);
  if (chk) return chk;
  DGM_CHECK_ARG((int64_t)A->num_tokens * A->topk <= NA_MAX_ROUTES,
                "no-alloc layer: num_tokens * topk must be <= 512 (the workspace array's size)");
  DGM_CHECK_ARG(A->num_tokens <= FUSED_MAX_TOKENS && A->num_local_experts <= FUSED_MAX_LOCAL,
                "no-alloc layer: num_tokens <= 256 and num_local_experts <= 512");
  DGM_CHECK_ARG(A->hidden <= NA_MAX_HIDDEN && A->intermediate <= NA_MAX_INTER,
                "no-alloc layer: hidden <= 3072 and intermediate <= 1280 (the workspace array's size)");
  if (A->num_tokens == 0) return 0;
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    dgm_set_error("no-alloc layer: hipGetDevice failed");
    return (int)e;
  }
  DGM_CHECK_ARG(dev >= 0 && dev < NA_MAX_DEVICES, "no-alloc layer: device index < 64");
  uint8_t* base = nullptr;
  const int st = na_setup(dev, stream, &base);
  if (st) return st;
  DgmWorkspace w;
  w.pool = base + NA_OFF_POOL;
  w.mid = base + NA_OFF_MID;
  w.mid_sf = base + NA_OFF_MID_SF;
  w.partials = (uint16_t*)(base + NA_OFF_PART);
  w.part_rows = A->num_tokens;
  w.counters = (int*)(base + NA_OFF_CNT);
  return dgm_fused_launch_ws(A, 3, w, stream);
}
