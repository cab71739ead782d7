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

static inline size_t dgm_align256(size_t x) { return (x + 255) & ~(size_t)255; }
