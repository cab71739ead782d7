"""Activation casts (GPU) and small helpers mirroring deep_gemm/utils/math.py."""
import torch

from . import _lib


def ceil_div(x: int, y: int) -> int:
    return (x + y - 1) // y


def align(x: int, y: int) -> int:
    return ceil_div(x, y) * y


def per_token_cast_to_fp4(x: torch.Tensor, use_ue8m0: bool = True, gran_k: int = 32,
                          use_packed_ue8m0: bool = False, amax_floor: float = 1e-4):
    """deep_gemm/utils/math.py:85 ``per_token_cast_to_fp4(use_ue8m0=True, gran_k=32)``:
    packed E2M1 [M, K/2] (low nibble = even K) and UE8M0 scales. Returns the scales as
    fp32 powers of two ([M, K/32]), or as raw E8M0 bytes viewed as int32 when
    ``use_packed_ue8m0``. ``amax_floor=1e-30`` gives the W4A4 test cast
    (sm100_b200/test_mega_moe.py:78)."""
    if not use_ue8m0 or gran_k != 32:
        raise NotImplementedError("MI355X path implements the UE8M0 / 32 MX cast")
    _lib.require_gpu(x)
    assert x.dtype == torch.bfloat16 and x.dim() == 2
    x = x.contiguous()
    M, K = x.shape
    packed = torch.empty((M, K // 2), dtype=torch.uint8, device=x.device)
    sf = torch.empty((M, K // 32), dtype=torch.uint8, device=x.device)
    _lib.check(_lib.load().dgm_cast_fp4_rows(_lib.ptr(x), M, K, float(amax_floor), _lib.ptr(packed),
                                             _lib.ptr(sf), _lib.stream()))
    if use_packed_ue8m0:
        return packed, sf.view(torch.int32)
    return packed, (sf.to(torch.int32) << 23).view(torch.float32)


def per_token_cast_to_fp8(x: torch.Tensor, use_ue8m0: bool = True, gran_k: int = 32,
                          use_packed_ue8m0: bool = False):
    """deep_gemm/utils/math.py:26 ``per_token_cast_to_fp8(use_ue8m0=True, gran_k=32)``:
    E4M3 [M, K] and UE8M0 scales (fp32 powers of two, or packed bytes as int32)."""
    if not use_ue8m0 or gran_k != 32:
        raise NotImplementedError("MI355X path implements the UE8M0 / 32 MX cast")
    _lib.require_gpu(x)
    assert x.dtype == torch.bfloat16 and x.dim() == 2
    x = x.contiguous()
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.uint8, device=x.device)
    sf = torch.empty((M, K // 32), dtype=torch.uint8, device=x.device)
    _lib.check(_lib.load().dgm_cast_fp8_rows(_lib.ptr(x), M, K, _lib.ptr(q), _lib.ptr(sf), _lib.stream()))
    q = q.view(torch.float8_e4m3fn)
    if use_packed_ue8m0:
        return q, sf.view(torch.int32)
    return q, (sf.to(torch.int32) << 23).view(torch.float32)
