"""Weight packers of the split MegaMoE path, on the GPU.

Mirrors deep_gemm/quantization_mxfp4.py:52 ``quantize_to_mxfp4``: amax >= 1e-30, scale code
clamp(ceil(log2(clamp(amax/6, 2^-126, 2^127))) + 127, 1, 254), E2M1 midpoint nibbles,
Marlin byte order (HIP kernel dgm_quantize_mxfp4, rule 1); and :323 ``quantize_to_qoq_int4``
(the QoQ chain of quantize_to_qoq with an int32 coefficient plane, HIP kernel
dgm_quantize_qoq_int4).
"""
import torch

from . import _lib
from .quantization_mxfp4_fused import _pack, MXFP4_GROUP_SIZE


def quantize_to_mxfp4(weight: torch.Tensor, group_size: int = MXFP4_GROUP_SIZE):
    assert group_size == MXFP4_GROUP_SIZE
    return _pack(weight, 1)


def quantize_to_qoq_int4(weight: torch.Tensor, group_size: int = 128):
    """Returns ``(packed uint8 [E, N, K/2] (Marlin), plane int32 [E, N, K/128])`` with plane =
    s2 | z << 8 | bf16(s1) << 16 per (row, K128 group)."""
    assert group_size == 128
    assert weight.dim() == 3
    code = _lib.src_dtype(weight)
    _lib.require_gpu(weight)
    w = weight.contiguous()
    E, N, K = w.shape
    assert K % 128 == 0
    packed = torch.empty((E, N, K // 2), dtype=torch.uint8, device=w.device)
    plane = torch.empty((E, N, K // 128), dtype=torch.int32, device=w.device)
    _lib.check(_lib.load().dgm_quantize_qoq_int4_typed(_lib.ptr(w), code, E * N, K, _lib.ptr(packed), _lib.ptr(plane),
                                                       _lib.stream()))
    return packed, plane
