"""NVFP4 weight packer, on the GPU.

Mirrors deep_gemm/quantization_nvfp4.py:62 ``quantize_to_nvfp4``: per 16-K group the
smallest UE4M3 >= amax/6 (the reference's ceil with its -1e-6 mantissa fudge), E2M1
midpoint nibbles of w / scale, Marlin byte order (HIP kernel dgm_quantize_nvfp4).
"""
import torch

from . import _lib


def quantize_to_nvfp4(weight: torch.Tensor, group_size: int = 16):
    """bf16 / fp16 / fp32 ``(..., K)`` -> ``(packed uint8 (..., K/2) Marlin order, E4M3 scales uint8
    (..., K/16))``."""
    assert group_size == 16
    code = _lib.src_dtype(weight)
    _lib.require_gpu(weight)
    w = weight.contiguous()
    *outer, K = w.shape
    rows = w.numel() // K
    packed = torch.empty((*outer, K // 2), dtype=torch.uint8, device=w.device)
    scale = torch.empty((*outer, K // 16), dtype=torch.uint8, device=w.device)
    _lib.check(_lib.load().dgm_quantize_nvfp4_typed(_lib.ptr(w), code, rows, K, _lib.ptr(packed), _lib.ptr(scale),
                                                    _lib.stream()))
    return packed, scale
