"""MXFP4 weight packer of the split MegaMoE path, on the GPU.

Mirrors deep_gemm/quantization_mxfp4.py:52 ``quantize_to_mxfp4``: amax >= 1e-30, scale code
clamp(ceil(log2(clamp(amax/6, 2^-126, 2^127))) + 127, 1, 254), E2M1 midpoint nibbles,
Marlin byte order (HIP kernel dgm_quantize_mxfp4, rule 1).
"""
import torch

from .quantization_mxfp4_fused import _pack, MXFP4_GROUP_SIZE


def quantize_to_mxfp4(weight: torch.Tensor, group_size: int = MXFP4_GROUP_SIZE):
    assert group_size == MXFP4_GROUP_SIZE
    return _pack(weight, 1)
