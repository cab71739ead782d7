"""Checkpoint ingestion for the FP4 weight formats, both ways, on the GPU.

Three layouts of the same E2M1 codes:

* ``"ocp"`` (alias ``"low_first"``): OCP MX / NVFP4 checkpoints, two codes per byte, the
  element with the lower K index in the low nibble (deep_gemm/utils/math.py:99-100).
* ``"marlin"``: the reference's packer order, every 8 K codes -> 4 bytes with byte b =
  K[b] << 4 | K[b+4] (deep_gemm/quantization_mxfp4.py:66-70, quantization_nvfp4.py:76-80).
* the fused kernel's tile layout (``transform_mxfp4_weights_for_mega_moe_fused`` /
  ``transform_nvfp4_weights_for_mega_moe_fused``), which the ``untransform_*`` calls invert.

W1 of a checkpoint may hold gate and up rows as two halves (``gate_up="concat"``, the
reference's [E, 2I, H]) or interleaved row by row (``gate_up="interleaved"``: row 2i = gate
row i, row 2i+1 = up row i). Block-shaped checkpoint tensors ``[E, N, K/32, 16]`` (MXFP4) are
accepted wherever ``[E, N, K/2]`` is. Every conversion is a HIP kernel of the native library.
"""
import torch

from . import _lib
from .mega import transform_mxfp4_weights_for_mega_moe_fused, transform_nvfp4_weights_for_mega_moe_fused

ORDERS = {"marlin": 0, "ocp": 1, "low_first": 1}
GATE_UP = {"concat": 1, "interleaved": 2}


def _order(name):
    if name not in ORDERS:
        raise ValueError(f"nibble order {name!r}: one of {sorted(ORDERS)}")
    return ORDERS[name]


def _as_packed3(packed):
    """[E, N, K/2] view of packed codes given as [E, N, K/2] or blocks [E, N, G, B]."""
    if packed.dim() == 4:
        E, N, G, B = packed.shape
        return packed.reshape(E, N, G * B)
    assert packed.dim() == 3, f"packed codes must be [E, N, K/2] or [E, N, K/32, 16], got {tuple(packed.shape)}"
    return packed


def reorder_fp4_nibbles(packed, src_order, dst_order, out=None):
    """The same E2M1 codes in another nibble order (``"ocp"`` / ``"low_first"`` <-> ``"marlin"``),
    any shape with a last dimension of whole 4-byte words; ``out=packed`` converts in place.
    (A Marlin word holds 8 codes of one row, so a row that ends mid-word would mix two rows.)"""
    assert packed.dtype == torch.uint8 and packed.is_contiguous(), "contiguous uint8 codes"
    assert packed.dim() >= 1 and packed.shape[-1] % 4 == 0, \
        f"the last dimension ({tuple(packed.shape)}) must be whole 4-byte words (8 codes)"
    _lib.require_gpu(packed)
    if out is None:
        out = torch.empty_like(packed)
    assert out.dtype == torch.uint8 and out.is_contiguous() and out.shape == packed.shape
    _lib.check(_lib.load().dgm_reorder_fp4_nibbles(_lib.ptr(packed), _lib.ptr(out), packed.numel(),
                                                   _order(src_order), _order(dst_order), _lib.stream()))
    return out


def ocp_to_marlin(packed, out=None):
    return reorder_fp4_nibbles(packed, "ocp", "marlin", out)


def marlin_to_ocp(packed, out=None):
    return reorder_fp4_nibbles(packed, "marlin", "ocp", out)


def _untransform_one(fn, values, scales, sc_per_row, l1_mode, dst_order):
    _lib.require_gpu(values, scales)
    assert values.dtype == torch.uint8 and values.dim() == 5 and values.shape[-2:] == (64, 16)
    E, NB, KT = values.shape[:3]
    N, K = NB * 16, KT * 128
    packed = torch.empty((E, N, K // 2), dtype=torch.uint8, device=values.device)
    sc = torch.empty((E, N, K // sc_per_row), dtype=torch.uint8, device=values.device)
    _lib.check(fn(_lib.ptr(values.contiguous()), _lib.ptr(scales.contiguous()), E, N, K, _order(dst_order), l1_mode,
                  _lib.ptr(packed), _lib.ptr(sc), _lib.stream()))
    return packed, sc


def untransform_mxfp4_weights_for_mega_moe_fused(w1, w2, dst_order="marlin", gate_up="concat"):
    """Inverse of ``transform_mxfp4_weights_for_mega_moe_fused``: the fused weights
    ``((w1_values, w1_scales, _), (w2_values, w2_scales, _))`` -> ``((packed [E, 2I, H/2],
    scale_e8m0 [E, 2I, H/32]), (packed [E, H, I/2], scale [E, H, I/32]))`` in ``dst_order``,
    W1 rows as ``gate_up`` names. Bit-exact round trip (the padding scale bytes of a last
    partial 4-tile group are not carried)."""
    fn = _lib.load().dgm_untransform_fp4_weights
    return (_untransform_one(fn, w1[0], w1[1], 32, GATE_UP[gate_up], dst_order),
            _untransform_one(fn, w2[0], w2[1], 32, 0, dst_order))


def untransform_nvfp4_weights_for_mega_moe_fused(w1, w2, dst_order="marlin", gate_up="concat"):
    """Inverse of ``transform_nvfp4_weights_for_mega_moe_fused``: ``((w1_values, w1_scales),
    (w2_values, w2_scales))`` -> ``((packed, E4M3 scales [E, 2I, H/16]), (packed, scales
    [E, H, I/16]))`` in ``dst_order``."""
    fn = _lib.load().dgm_untransform_nvfp4_weights
    return (_untransform_one(fn, w1[0], w1[1], 16, GATE_UP[gate_up], dst_order),
            _untransform_one(fn, w2[0], w2[1], 16, 0, dst_order))


def _transform_fp4(packed, scale, l1_mode, src_order, nvfp4):
    packed = _as_packed3(packed)
    _lib.require_gpu(packed, scale)
    assert packed.dtype == torch.uint8 and scale.dtype == torch.uint8
    E, N, Kh = packed.shape
    K = 2 * Kh
    per = 16 if nvfp4 else 32
    if N % 32 or K % 128 or N == 0 or K == 0:
        raise ValueError(f"rows N={N} must be a multiple of 32 and K={K} of 128")
    assert tuple(scale.shape) == (E, N, K // per), (tuple(scale.shape), (E, N, K // per))
    if nvfp4:
        vals = torch.empty((E, N // 16, K // 128, 64, 16), dtype=torch.uint8, device=packed.device)
        sc = torch.empty((E, N // 16, K // 128, 2, 16, 4), dtype=torch.uint8, device=packed.device)
        _lib.check(_lib.load().dgm_transform_nvfp4_weights(
            _lib.ptr(packed.contiguous()), _lib.ptr(scale.contiguous()), E, N, K, _order(src_order), l1_mode,
            _lib.ptr(vals), _lib.ptr(sc), _lib.stream()))
        return vals, sc
    KT = K // 128
    vals = torch.empty((E, N // 16, KT, 64, 16), dtype=torch.uint8, device=packed.device)
    sc = torch.empty((E, N // 16, (KT + 3) // 4, 64, 4), dtype=torch.uint8, device=packed.device)
    _lib.check(_lib.load().dgm_transform_fp4_weights(
        _lib.ptr(packed.contiguous()), _lib.ptr(scale.contiguous()), E, N, K, _order(src_order), l1_mode,
        _lib.ptr(vals), _lib.ptr(sc), _lib.stream()))
    return vals, sc, None


def mxfp4_checkpoint_to_mega_moe(gate_up, down, order="ocp", gate_up_rows="concat"):
    """MXFP4 checkpoint tensors -> the fused kernel's weights (as
    ``transform_mxfp4_weights_for_mega_moe_fused`` returns them). ``gate_up = (codes, scales)``
    with codes [E, 2I, H/2] or blocks [E, 2I, H/32, 16] and E8M0 scales [E, 2I, H/32];
    ``down`` likewise for [E, H, I]. ``order``: nibble order of the codes; ``gate_up_rows``:
    ``"concat"`` (gate rows, then up rows) or ``"interleaved"`` (row 2i gate, 2i+1 up)."""
    return (_transform_fp4(gate_up[0], gate_up[1], GATE_UP[gate_up_rows], order, False),
            _transform_fp4(down[0], down[1], 0, order, False))


def nvfp4_checkpoint_to_mega_moe(gate_up, down, order="ocp", gate_up_rows="concat"):
    """NVFP4 checkpoint tensors (codes [E, N, K/2], E4M3 scales [E, N, K/16]) -> the fused
    kernel's NVFP4 weights (as ``transform_nvfp4_weights_for_mega_moe_fused`` returns them)."""
    return (_transform_fp4(gate_up[0], gate_up[1], GATE_UP[gate_up_rows], order, True),
            _transform_fp4(down[0], down[1], 0, order, True))


def mega_moe_to_mxfp4_checkpoint(w1, w2, order="ocp", gate_up_rows="concat"):
    """The fused MXFP4 weights back to checkpoint tensors (inverse of
    ``mxfp4_checkpoint_to_mega_moe``; codes as [E, N, K/2])."""
    return untransform_mxfp4_weights_for_mega_moe_fused(w1, w2, dst_order=order, gate_up=gate_up_rows)


def mega_moe_to_nvfp4_checkpoint(w1, w2, order="ocp", gate_up_rows="concat"):
    return untransform_nvfp4_weights_for_mega_moe_fused(w1, w2, dst_order=order, gate_up=gate_up_rows)


__all__ = ["reorder_fp4_nibbles", "ocp_to_marlin", "marlin_to_ocp",
           "untransform_mxfp4_weights_for_mega_moe_fused", "untransform_nvfp4_weights_for_mega_moe_fused",
           "mxfp4_checkpoint_to_mega_moe", "nvfp4_checkpoint_to_mega_moe",
           "mega_moe_to_mxfp4_checkpoint", "mega_moe_to_nvfp4_checkpoint"]
