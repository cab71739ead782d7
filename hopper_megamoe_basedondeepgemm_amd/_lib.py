"""ctypes binding of libdgm_megamoe.so (the C ABI declared in include/dgm_megamoe.h).

The library is the product path: there is no CPU fallback. If the shared library is not
built, or no GPU is present, calls raise instead of computing anything elsewhere.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdgm_megamoe.so")
PROBE_LIB_PATH = os.path.join(_HERE, "libdgm_probe.so")     # the tests' lane-layout probes

ACT_FORMATS = {"mxfp4": 0, "mxfp8": 1, "fp8": 1, "qoq": 2, "nvfp4": 3, "fp8f128": 4}
FE_FORCE_BALANCED = 1
FE_ZERO_ROW_UNROUTED = 2
FE_SELECT_IN_MEGA = 4
FE_RAW_WEIGHTS = 8
FE_NO_CAST = 16

EXPORTS = [
    "dgm_version", "dgm_last_error", "dgm_quantize_mxfp4", "dgm_cast_fp4_rows", "dgm_cast_fp8_rows",
    "dgm_quantize_nvfp4", "dgm_quantize_qoq", "dgm_cast_int8_rows", "dgm_transform_fp4_weights",
    "dgm_fused_buffer_layout", "dgm_router_topk_launch", "dgm_megamoe_fused_launch",
    "dgm_megamoe_split_launch",
    "dgm_device_cu_count", "dgm_fused_workgroups", "dgm_fused_last_form", "dgm_abi_struct_sizes",
    "dgm_transform_qoq_weights", "dgm_transform_nvfp4_weights", "dgm_quantize_qoq_int4",
    "dgm_transform_qoq_int4_weights", "dgm_host_device_pointer", "dgm_megamoe_fused_launch_noalloc",
    "dgm_reorder_fp4_nibbles", "dgm_untransform_fp4_weights", "dgm_untransform_nvfp4_weights",
    "dgm_router_logits_topk_launch", "dgm_router_topk_launch_stamped", "dgm_frontend_workgroups",
    "dgm_quantize_mxfp4_typed", "dgm_quantize_nvfp4_typed", "dgm_quantize_qoq_typed", "dgm_quantize_qoq_int4_typed",
]
# source element types of the weight packers (DGM_SRC_*)
SRC_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def src_dtype(t):
    """The packers' code for t's element type (bf16, fp16 or fp32; anything else raises)."""
    if t.dtype not in SRC_DTYPES:
        raise TypeError(f"weights are packed from bf16, fp16 or fp32, got {t.dtype}")
    return SRC_DTYPES[t.dtype]


class BufferLayout(ctypes.Structure):
    _fields_ = [("total_bytes", ctypes.c_size_t), ("x", ctypes.c_size_t), ("x_sf", ctypes.c_size_t),
                ("topk_idx", ctypes.c_size_t), ("topk_weights", ctypes.c_size_t),
                ("logits", ctypes.c_size_t), ("fe_keys", ctypes.c_size_t), ("pool", ctypes.c_size_t),
                ("mid", ctypes.c_size_t),
                ("mid_sf", ctypes.c_size_t), ("partials", ctypes.c_size_t), ("counters", ctypes.c_size_t),
                ("x_row_bytes", ctypes.c_int32), ("mid_row_bytes", ctypes.c_int32),
                ("max_routes", ctypes.c_int32), ("max_tokens", ctypes.c_int32),
                ("topk", ctypes.c_int32), ("num_experts", ctypes.c_int32), ("num_local_experts", ctypes.c_int32),
                ("hidden", ctypes.c_int32), ("intermediate", ctypes.c_int32), ("act_format", ctypes.c_int32),
                ("x_sf_row_bytes", ctypes.c_int32), ("mid_sf_row_bytes", ctypes.c_int32)]


LAUNCH_COOPERATIVE = 1      # DGM_LAUNCH_COOPERATIVE


class MoeArgs(ctypes.Structure):
    _fields_ = [("num_tokens", ctypes.c_int32), ("hidden", ctypes.c_int32), ("intermediate", ctypes.c_int32),
                ("num_experts", ctypes.c_int32), ("expert_begin", ctypes.c_int32),
                ("num_local_experts", ctypes.c_int32), ("topk", ctypes.c_int32),
                ("act_format", ctypes.c_int32), ("activation_clamp", ctypes.c_float),
                ("fast_math", ctypes.c_int32), ("select_in_mega", ctypes.c_int32), ("fe_flags", ctypes.c_int32),
                ("token_offset", ctypes.c_int32),
                ("w1_values", ctypes.c_void_p), ("w1_scales", ctypes.c_void_p),
                ("w2_values", ctypes.c_void_p), ("w2_scales", ctypes.c_void_p),
                ("recv_stats", ctypes.c_void_p), ("y", ctypes.c_void_p), ("buffer", ctypes.c_void_p),
                ("layout", ctypes.POINTER(BufferLayout)), ("phase_stamps", ctypes.c_void_p),
                ("phase_stamp_rows", ctypes.c_int32), ("w1_row_scales", ctypes.c_void_p),
                ("w2_row_scales", ctypes.c_void_p), ("l1_global_scales", ctypes.c_void_p),
                ("l2_global_scales", ctypes.c_void_p), ("fe_in_mega", ctypes.c_int32),
                ("hidden_states", ctypes.c_void_p), ("router_weight", ctypes.c_void_p),
                ("fe_keys", ctypes.c_void_p), ("host_error", ctypes.c_void_p), ("debug_flags", ctypes.c_int32),
                ("launch_flags", ctypes.c_int32)]


_lib = None


def load():
    """Load the shared library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run `python -m hopper_megamoe_basedondeepgemm_amd.build`")
    lib = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    sig = {
        "dgm_version": ([], i32),
        "dgm_last_error": ([], ctypes.c_char_p),
        "dgm_quantize_mxfp4": ([vp, i64, i64, i32, vp, vp, vp], i32),
        "dgm_quantize_mxfp4_typed": ([vp, i32, i64, i64, i32, vp, vp, vp], i32),
        "dgm_quantize_nvfp4_typed": ([vp, i32, i64, i64, vp, vp, vp], i32),
        "dgm_quantize_qoq_typed": ([vp, i32, i64, i64, vp, vp, vp, vp, vp], i32),
        "dgm_quantize_qoq_int4_typed": ([vp, i32, i64, i64, vp, vp, vp], i32),
        "dgm_cast_fp4_rows": ([vp, i64, i64, f32, vp, vp, vp], i32),
        "dgm_cast_fp8_rows": ([vp, i64, i64, vp, vp, vp], i32),
        "dgm_quantize_nvfp4": ([vp, i64, i64, vp, vp, vp], i32),
        "dgm_quantize_qoq": ([vp, i64, i64, vp, vp, vp, vp, vp], i32),
        "dgm_quantize_qoq_int4": ([vp, i64, i64, vp, vp, vp], i32),
        "dgm_transform_qoq_int4_weights": ([vp, vp, i32, i32, i32, i32, vp, vp, vp, vp], i32),
        "dgm_cast_int8_rows": ([vp, i64, i64, vp, vp, vp], i32),
        "dgm_transform_fp4_weights": ([vp, vp, i32, i32, i32, i32, i32, vp, vp, vp], i32),
        "dgm_fused_buffer_layout": ([i32, i32, i32, i32, i32, i32, i32, ctypes.POINTER(BufferLayout)], i32),
        "dgm_router_topk_launch": ([vp, vp, i32, i32, i32, i32, i32, i32, i32, vp,
                                    ctypes.POINTER(BufferLayout), vp], i32),
        "dgm_router_topk_launch_stamped": ([vp, vp, i32, i32, i32, i32, i32, i32, i32, vp,
                                            ctypes.POINTER(BufferLayout), vp, i32, vp], i32),
        "dgm_frontend_workgroups": ([i32, i32, i32, i32, i32, i32], i32),
        "dgm_megamoe_fused_launch": ([ctypes.POINTER(MoeArgs), vp], i32),
        "dgm_megamoe_split_launch": ([ctypes.POINTER(MoeArgs), vp], i32),
        "dgm_megamoe_fused_launch_noalloc": ([ctypes.POINTER(MoeArgs), vp], i32),
        "dgm_device_cu_count": ([], i32),
        "dgm_fused_workgroups": ([i32, i32, i32], i32),
        "dgm_fused_last_form": ([i32, i32, i32], i32),
        "dgm_abi_struct_sizes": ([ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)], i32),
        "dgm_transform_qoq_weights": ([vp, vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp], i32),
        "dgm_transform_nvfp4_weights": ([vp, vp, i32, i32, i32, i32, i32, vp, vp, vp], i32),
        "dgm_host_device_pointer": ([vp, ctypes.POINTER(vp)], i32),
        "dgm_reorder_fp4_nibbles": ([vp, vp, i64, i32, i32, vp], i32),
        "dgm_router_logits_topk_launch": ([vp, i32, i32, i32, i32, i32, vp, ctypes.POINTER(BufferLayout), vp], i32),
        "dgm_untransform_fp4_weights": ([vp, vp, i32, i32, i32, i32, i32, vp, vp, vp], i32),
        "dgm_untransform_nvfp4_weights": ([vp, vp, i32, i32, i32, i32, i32, vp, vp, vp], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


PROBE_EXPORTS = ["dgm_probe_mfma_scale", "dgm_probe_mfma_scale_sel", "dgm_probe_mfma_i8", "dgm_probe_mfma_f16",
                 "dgm_probe_cvt_fp4", "dgm_probe_global_load_lds", "dgm_probe_stream_read", "dgm_probe_empty_launch"]
_probe = None


def load_probe():
    """The tests' probe library (include/dgm_probe.h; raises if it has not been built)."""
    global _probe
    if _probe is not None:
        return _probe
    if not os.path.exists(PROBE_LIB_PATH):
        raise RuntimeError(f"{PROBE_LIB_PATH} is not built; run `python -m hopper_megamoe_basedondeepgemm_amd.build`")
    lib = ctypes.CDLL(PROBE_LIB_PATH)
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    sig = {
        "dgm_probe_mfma_scale": ([vp, vp, vp, vp, vp, i32, i32, vp], i32),
        "dgm_probe_mfma_scale_sel": ([vp, vp, vp, vp, vp, i32, vp], i32),
        "dgm_probe_mfma_i8": ([vp, vp, vp, vp], i32),
        "dgm_probe_mfma_f16": ([vp, vp, vp, vp], i32),
        "dgm_probe_cvt_fp4": ([vp, vp, vp, vp, i32, vp], i32),
        "dgm_probe_global_load_lds": ([vp, vp, vp], i32),
        "dgm_probe_stream_read": ([vp, ctypes.c_int64, i32, i32, vp, vp], i32),
        "dgm_probe_empty_launch": ([i32, i32, vp], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _probe = lib
    return lib


def check(status):
    if status != 0:
        msg = load().dgm_last_error().decode(errors="replace")
        raise RuntimeError(f"dgm error {status}: {msg}")


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("MI355X path: tensors must live on the GPU (no CPU fallback)")


def host_device_pointer(t):
    """Device address of a pinned host tensor (for words the kernels write and the host reads)."""
    assert t.is_pinned()
    out = ctypes.c_void_p()
    check(load().dgm_host_device_pointer(ctypes.c_void_p(t.data_ptr()), ctypes.byref(out)))
    return out.value


def layout(max_tokens, num_experts, num_local_experts, topk, hidden, intermediate, act_format):
    out = BufferLayout()
    check(load().dgm_fused_buffer_layout(max_tokens, num_experts, num_local_experts, topk, hidden,
                                         intermediate, act_format, ctypes.byref(out)))
    return out
