"""MXFP4 weight packer of the fused MegaMoE path, on the GPU.

Mirrors deep_gemm/quantization_mxfp4_fused.py:29 ``quantize_to_mxfp4``: per 32-K group
exp = ceil(log2(max(amax, 1e-38) / 6)) (-127 for an all-zero group), E2M1 nibbles of
w / 2^exp by the midpoint rule (ties to the smaller magnitude, sign bit for every negative),
Marlin byte order. Runs as a HIP kernel (dgm_quantize_mxfp4, rule 0).
"""
import torch

from . import _lib

MXFP4_GROUP_SIZE = 32


def _pack(weight, rule):
    assert weight.is_floating_point()
    code = _lib.src_dtype(weight)        # bf16 / fp16 / fp32, read as their fp32 values
    _lib.require_gpu(weight)
    w = weight.contiguous()
    *outer, K = w.shape
    assert K % MXFP4_GROUP_SIZE == 0
    rows = w.numel() // K
    packed = torch.empty((*outer, K // 2), dtype=torch.uint8, device=w.device)
    scale = torch.empty((*outer, K // 32), dtype=torch.uint8, device=w.device)
    _lib.check(_lib.load().dgm_quantize_mxfp4_typed(_lib.ptr(w), code, rows, K, rule, _lib.ptr(packed),
                                                    _lib.ptr(scale), _lib.stream()))
    return packed, scale


def quantize_to_mxfp4(weight: torch.Tensor, group_size: int = MXFP4_GROUP_SIZE):
    """bf16 / fp16 / fp32 ``(..., K)`` -> ``(packed uint8 (..., K/2) Marlin order, scale_e8m0 uint8
    (..., K/32))``."""
    assert group_size == MXFP4_GROUP_SIZE
    return _pack(weight, 0)


def e8m0_to_fp32(scale_e8m0: torch.Tensor) -> torch.Tensor:
    return torch.exp2(scale_e8m0.to(torch.int32).float() - 127.0)
