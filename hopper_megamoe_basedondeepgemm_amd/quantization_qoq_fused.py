"""QoQ W4A8 packer and per-token int8 cast, on the GPU.

Mirrors deep_gemm/quantization_qoq_fused.py:18 ``quantize_to_qoq`` (s1 = bf16(amax/120),
w8 = clamp(rne(w/s1), +-112), per K128 s2 = clamp(ceil((mx-mn)/15), 1, 15),
z = clamp(rne(-mn/s2), 0, 15), code = clamp(rne(w8/s2 + z), 0, 15), Marlin order) and
:78 ``per_token_cast_to_int8`` (sf = amax/127, q = clamp(rne(x/sf), +-127)).
"""
import torch

from . import _lib

QOQ_GROUP_SIZE = 128


def quantize_to_qoq(weight: torch.Tensor, group_size: int = QOQ_GROUP_SIZE):
    """bf16 / fp16 / fp32 ``(..., K)`` -> ``(packed (..., K/2) Marlin, s2 (..., K/128), z (..., K/128),
    s1 fp32 (...))``."""
    assert group_size == QOQ_GROUP_SIZE
    code = _lib.src_dtype(weight)
    _lib.require_gpu(weight)
    w = weight.contiguous()
    *outer, K = w.shape
    rows = w.numel() // K
    dev = w.device
    packed = torch.empty((*outer, K // 2), dtype=torch.uint8, device=dev)
    s2 = torch.empty((*outer, K // 128), dtype=torch.uint8, device=dev)
    z = torch.empty((*outer, K // 128), dtype=torch.uint8, device=dev)
    s1 = torch.empty(tuple(outer), dtype=torch.float32, device=dev)
    _lib.check(_lib.load().dgm_quantize_qoq_typed(_lib.ptr(w), code, rows, K, _lib.ptr(packed), _lib.ptr(s2),
                                                  _lib.ptr(z), _lib.ptr(s1), _lib.stream()))
    return packed, s2, z, s1


def per_token_cast_to_int8(x: torch.Tensor, gran_k: int = 128):
    """Returns ``(int8 [M, K], sf fp32 [M, K/gran_k])`` (one scale per token, repeated)."""
    _lib.require_gpu(x)
    assert x.dtype == torch.bfloat16 and x.dim() == 2
    x = x.contiguous()
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    sf = torch.empty((M,), dtype=torch.float32, device=x.device)
    _lib.check(_lib.load().dgm_cast_int8_rows(_lib.ptr(x), M, K, _lib.ptr(q), _lib.ptr(sf), _lib.stream()))
    return q, sf[:, None].expand(M, K // gran_k).contiguous()
