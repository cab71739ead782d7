"""MegaMoE Python API on MI355X: buffers, weight transforms, frontend and the fused layer.

Mirrors the reference entry points (deep_gemm/mega/fused.py, deep_gemm/mega/__init__.py)
with the same names and argument meaning. ``group=None`` means one GPU. Work runs in the
HIP library (libdgm_megamoe.so) on the current torch stream; nothing here computes.
"""
import ctypes
import os
import types
from typing import Optional, Tuple

import torch

from . import _lib


# ----------------------------------------------------------------------------- buffer
class FusedSymmBuffer:
    """Single-process counterpart of deep_gemm/mega/fused.py:79 ``FusedSymmBuffer``.

    One device allocation holds every view the layer uses. On one GPU no symmetric memory
    or rendezvous is needed; ``ep_size`` / ``ep_rank`` select which expert-parallel share
    the layer computes (local experts ``[ep_rank * E / ep_size, (ep_rank + 1) * E / ep_size)``),
    so one GPU can run exactly one rank's share of an EP layer.

    Views: x, x_sf, topk_idx, topk_weights (frontend outputs / layer inputs), l1_acts and
    l1_acts_sf (aliases of x / x_sf: routed rows are read in place), l2_acts / l2_acts_sf
    (L1 -> L2 activations in pool order), combine_partials (bf16 [topk, tokens, H]: each local
    route's output rounded to bf16, as the reference's view; slots without a local route are not
    written), logits (fp32 router logits), fe_keys (int32 [tokens, E] top-k keys of the
    frontend, see ``fable_frontend_keys``) and pool (dispatch table, int32).
    act_format "mxfp4" / "mxfp8": uint8 codes with E8M0 scale bytes per 32; "nvfp4": E2M1 codes
    (low nibble first) with E4M3 scale bytes per 16; "qoq": int8 codes, x_sf fp32 [tokens, H/128]
    (one scale per token, repeated), l2_acts_sf fp32 [routes, I/64]; "fp8f128" (the split
    recipe of ``SymmBuffer``): E4M3 codes with fp32 scales per 128 (x_sf [tokens, H/128]), an
    E4M3 intermediate with E8M0 bytes per 32."""

    def __init__(self, group, num_experts, max_tokens, topk, hidden, intermediate,
                 act_format="mxfp4", ep_size=None, ep_rank=None, device=None, buffer=None):
        if group is not None:
            ep_size = group.size() if ep_size is None else ep_size
            ep_rank = group.rank() if ep_rank is None else ep_rank
        ep_size = 1 if ep_size is None else int(ep_size)
        ep_rank = 0 if ep_rank is None else int(ep_rank)
        assert num_experts % ep_size == 0 and 0 <= ep_rank < ep_size
        self.group = group
        self.num_experts = num_experts
        self.num_max_tokens_per_rank = max_tokens
        self.num_topk = topk
        self.hidden = hidden
        self.intermediate_hidden = intermediate
        self.act_format = act_format
        self.act_code = _lib.ACT_FORMATS[act_format]
        self.ep_size, self.ep_rank = ep_size, ep_rank
        self.num_local_experts = num_experts // ep_size
        self.expert_begin = ep_rank * self.num_local_experts
        self.layout = _lib.layout(max_tokens, num_experts, self.num_local_experts, topk, hidden,
                                  intermediate, self.act_code)
        if buffer is None:
            dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
            self.buffer = torch.zeros(self.layout.total_bytes, dtype=torch.uint8, device=dev)
        else:     # a caller-owned (zeroed) allocation of at least layout.total_bytes
            _lib.require_gpu(buffer)
            assert buffer.is_contiguous() and buffer.nbytes >= self.layout.total_bytes, \
                (buffer.nbytes, self.layout.total_bytes)
            self.buffer = buffer.view(torch.uint8).view(-1)
        L, b = self.layout, self.buffer
        R = max_tokens * topk

        def view(off, n, dtype, shape):
            return b[off:off + n * torch.tensor([], dtype=dtype).element_size()].view(dtype).view(*shape)

        xb = L.x_row_bytes
        qoq = act_format == "qoq"
        f128 = act_format == "fp8f128"
        sfv = 16 if act_format == "nvfp4" else 32
        if qoq:   # int8 codes, fp32 scale per token repeated over the H / 128 slots
            self.x = view(L.x, max_tokens * xb, torch.int8, (max_tokens, xb))
            self.x_sf = view(L.x_sf, max_tokens * (hidden // 128), torch.float32, (max_tokens, hidden // 128))
        elif f128:  # E4M3 codes, fp32 scale per 128
            self.x = view(L.x, max_tokens * xb, torch.float8_e4m3fn, (max_tokens, xb))
            self.x_sf = view(L.x_sf, max_tokens * (hidden // 128), torch.float32, (max_tokens, hidden // 128))
        else:     # codes, E8M0 scale bytes per 32 (NVFP4: E4M3 per 16)
            self.x = view(L.x, max_tokens * xb, torch.uint8, (max_tokens, xb))
            self.x_sf = view(L.x_sf, max_tokens * (hidden // sfv), torch.uint8, (max_tokens, hidden // sfv))
        self.topk_idx = view(L.topk_idx, R, torch.int64, (max_tokens, topk))
        self.topk_weights = view(L.topk_weights, R, torch.float32, (max_tokens, topk))
        self.logits = view(L.logits, max_tokens * num_experts, torch.float32, (max_tokens, num_experts))
        self.fe_keys = view(L.fe_keys, max_tokens * num_experts, torch.int32, (max_tokens, num_experts))
        mb = L.mid_row_bytes
        if qoq:   # int8 codes, fp32 scale per 64 features
            self.l2_acts = view(L.mid, R * mb, torch.int8, (R, mb))
            self.l2_acts_sf = view(L.mid_sf, R * (intermediate // 64), torch.float32, (R, intermediate // 64))
        elif f128:  # E4M3 codes, E8M0 bytes per 32 (each per-64 power-of-two scale twice)
            self.l2_acts = view(L.mid, R * mb, torch.float8_e4m3fn, (R, mb))
            self.l2_acts_sf = view(L.mid_sf, R * (intermediate // 32), torch.uint8, (R, intermediate // 32))
        else:
            self.l2_acts = view(L.mid, R * mb, torch.uint8, (R, mb))
            self.l2_acts_sf = view(L.mid_sf, R * (intermediate // sfv), torch.uint8, (R, intermediate // sfv))
        self.combine_partials = view(L.partials, R * hidden, torch.bfloat16, (topk, max_tokens, hidden))
        self.l1_acts, self.l1_acts_sf = self.x, self.x_sf
        self.handle = types.SimpleNamespace(buffer_ptrs=[b.data_ptr()])
        # host-visible error word (pinned host memory the kernel writes when a bounded wait
        # expires): checked at the start of the next call on this buffer without synchronising
        self._host_err = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self._host_err_dev = _lib.host_device_pointer(self._host_err)

    def pool_table(self):
        """(counts [E_local], active experts, offsets [n_active+1], routes [total]) as CPU
        tensors, read back from the device dispatch table."""
        E = self.num_local_experts
        a256 = lambda v: (v + 255) // 256 * 256
        base = self.layout.pool
        raw = self.buffer[base:base + 256 + 2 * a256(E * 4) + a256((E + 1) * 4) +
                          a256(self.num_max_tokens_per_rank * self.num_topk * 4)].cpu()
        meta = raw[:256].view(torch.int32)
        n_active, total = int(meta[0]), int(meta[1])
        o = 256
        counts = raw[o:o + 4 * E].view(torch.int32).clone(); o += a256(E * 4)
        active = raw[o:o + 4 * n_active].view(torch.int32).clone(); o += a256(E * 4)
        offsets = raw[o:o + 4 * (n_active + 1)].view(torch.int32).clone(); o += a256((E + 1) * 4)
        routes = raw[o:o + 4 * total].view(torch.int32).clone()
        return counts, active, offsets, routes

    def kernel_error(self):
        """Error flag of the persistent kernel (1 when a bounded wait expired; it stays set until
        ``clear_error``). Synchronises."""
        return int(self.buffer[self.layout.counters + 4:self.layout.counters + 8].view(torch.int32).item())

    def host_error(self):
        """The host-visible copy of the error flag, as far as the launches on this buffer have
        completed (no synchronisation)."""
        return int(self._host_err[0])

    def clear_error(self):
        """Clears the error flag and its host-visible copy (synchronises)."""
        torch.cuda.synchronize()
        self.buffer[self.layout.counters + 4:self.layout.counters + 8].zero_()
        self._host_err.zero_()
        torch.cuda.synchronize()

    def destroy(self):
        self.buffer = None
        self.handle = None
        self.group = None


def get_fused_symm_buffer_for_mega_moe(group, num_experts, max_tokens, topk, hidden, intermediate,
                                       act_format="mxfp4", ep_size=None, ep_rank=None):
    """deep_gemm/mega/fused.py:88 (``group=None`` -> one GPU)."""
    return FusedSymmBuffer(group, num_experts, max_tokens, topk, hidden, intermediate, act_format,
                           ep_size=ep_size, ep_rank=ep_rank)


# ----------------------------------------------------------------------------- weight transform
def _transform_one(packed, scale, l1_interleave, src_order):
    _lib.require_gpu(packed, scale)
    assert packed.dtype == torch.uint8 and scale.dtype == torch.uint8 and packed.dim() == 3
    E, N, Kh = packed.shape
    K = Kh * 2
    assert scale.shape == (E, N, K // 32)
    KT, NB = K // 128, N // 16
    KG = (KT + 3) // 4
    vals = torch.empty((E, NB, KT, 64, 16), dtype=torch.uint8, device=packed.device)
    scl = torch.empty((E, NB, KG, 64, 4), dtype=torch.uint8, device=packed.device)
    _lib.check(_lib.load().dgm_transform_fp4_weights(
        _lib.ptr(packed.contiguous()), _lib.ptr(scale.contiguous()), E, N, K, src_order,
        int(l1_interleave), _lib.ptr(vals), _lib.ptr(scl), _lib.stream()))
    return vals, scl, None


def transform_mxfp4_weights_for_mega_moe_fused(l1, l2, src_order="marlin"):
    """deep_gemm/mega/fused.py:64. Inputs: ``(packed [E, 2I, H/2], scale_e8m0 [E, 2I, H/32])``
    and ``(packed [E, H, I/2], scale [E, H, I/32])`` from ``quantize_to_mxfp4`` (Marlin order;
    ``src_order="low_first"`` accepts OCP low-nibble-first packing). Returns
    ``((w1_values, w1_scales, None), (w2_values, w2_scales, None))`` in matrix-core fragment
    order; the third item (the reference's per-row 2^e_ref) is None because the E8M0 scales
    are applied exactly by the matrix cores. Invariant kept from the reference:
    dequant(transform(q)) == interleave(dequant(q))."""
    so = {"marlin": 0, "low_first": 1}[src_order]
    return _transform_one(l1[0], l1[1], True, so), _transform_one(l2[0], l2[1], False, so)


def _transform_qoq_one(q, l1_interleave):
    packed, s2, z, s1 = q
    _lib.require_gpu(packed, s2, z, s1)
    assert packed.dtype == torch.uint8 and s2.dtype == torch.uint8 and z.dtype == torch.uint8
    assert s1.dtype == torch.float32 and packed.dim() == 3
    E, N, Kh = packed.shape
    K = Kh * 2
    assert s2.shape == (E, N, K // 128) and z.shape == (E, N, K // 128) and s1.shape == (E, N)
    assert N % 16 == 0 and K % 128 == 0, (N, K)
    # the fused layout keeps z and s2 as one nibble each (quantize_to_qoq: z 0..15, s2 1..15)
    if int(torch.maximum(s2.max(), z.max()).item()) > 15:
        raise ValueError("QoQ meta out of range: z and s2 must be < 16")
    KT, NB = K // 128, N // 16
    vals = torch.empty((E, NB, KT, 64, 16), dtype=torch.uint8, device=packed.device)
    meta = torch.empty((E, NB, KT, 16), dtype=torch.uint8, device=packed.device)
    rs = torch.empty((E, N), dtype=torch.float32, device=packed.device)
    _lib.check(_lib.load().dgm_transform_qoq_weights(
        _lib.ptr(packed.contiguous()), _lib.ptr(s2.contiguous()), _lib.ptr(z.contiguous()),
        _lib.ptr(s1.contiguous()), E, N, K, int(l1_interleave), _lib.ptr(vals), _lib.ptr(meta), _lib.ptr(rs),
        _lib.stream()))
    return vals, meta, rs


def transform_qoq_weights_for_mega_moe_fused(l1, l2):
    """deep_gemm/mega/fused.py:71. Inputs: ``quantize_to_qoq`` tuples ``(packed [E, N, K/2],
    s2 [E, N, K/128], z [E, N, K/128], s1 [E, N])`` for W1 [E, 2I, H] and W2 [E, H, I].
    Returns ``((w1_values, w1_meta, w1_s1), (w2_values, w2_meta, w2_s1))``: 4-bit codes in
    int8 matrix-core fragment order, per (row, K128) zero points and group scales, per-row
    scales. Invariant: dequant(transform(q)) == interleave(dequant(q))."""
    return _transform_qoq_one(l1, True), _transform_qoq_one(l2, False)


def _transform_nvfp4_one(packed, scale, l1_interleave, src_order):
    _lib.require_gpu(packed, scale)
    assert packed.dtype == torch.uint8 and scale.dtype == torch.uint8 and packed.dim() == 3
    E, N, Kh = packed.shape
    K = Kh * 2
    assert tuple(scale.shape) == (E, N, K // 16), (scale.shape, packed.shape)
    assert N % 32 == 0 and K % 128 == 0, (N, K)
    vals = torch.empty((E, N // 16, K // 128, 64, 16), dtype=torch.uint8, device=packed.device)
    sc = torch.empty((E, N // 16, K // 128, 2, 16, 4), dtype=torch.uint8, device=packed.device)
    order = {"marlin": 0, "low_first": 1}[src_order]
    _lib.check(_lib.load().dgm_transform_nvfp4_weights(_lib.ptr(packed.contiguous()), _lib.ptr(scale.contiguous()),
                                                       E, N, K, order, int(l1_interleave), _lib.ptr(vals),
                                                       _lib.ptr(sc), _lib.stream()))
    return vals, sc


def transform_nvfp4_weights_for_mega_moe_fused(l1, l2, src_order="marlin"):
    """NVFP4 W4A4 weights (``(packed [E, N, K/2], E4M3 scales [E, N, K/16])`` per matrix, from
    ``quantize_to_nvfp4`` (Marlin order) or the W4A4 row cast (``src_order="low_first"``,
    sm100_b200/test_mega_moe.py:68-93)) -> the fused kernel's layout for the f16 matrix core
    (the role of sm100_b200/mega___init__.py:102 ``transform_weights_for_mega_moe`` and
    deep_gemm/mega/__init__.py:174 ``transform_nvfp4_weights_for_mega_moe_sm90``). L1 gate/up
    blocks are interleaved. Returns ``((w1_values, w1_scales), (w2_values, w2_scales))``."""
    return _transform_nvfp4_one(*l1, True, src_order), _transform_nvfp4_one(*l2, False, src_order)


def _transform_qoq_int4_one(q, l1_interleave):
    packed, plane = q
    _lib.require_gpu(packed, plane)
    assert packed.dtype == torch.uint8 and plane.dtype == torch.int32 and packed.dim() == 3
    E, N, Kh = packed.shape
    K = Kh * 2
    assert tuple(plane.shape) == (E, N, K // 128) and N % 16 == 0 and K % 128 == 0, (plane.shape, packed.shape)
    # the fused layout keeps z and s2 as one nibble each (quantize_to_qoq_int4: z <= 15, s2 <= 15)
    pl = plane.contiguous()
    if int(torch.maximum(pl & 0xFF, (pl >> 8) & 0xFF).max().item()) > 15:
        raise ValueError("QoQ plane out of range: z and s2 must be < 16")
    vals = torch.empty((E, N // 16, K // 128, 64, 16), dtype=torch.uint8, device=packed.device)
    meta = torch.empty((E, N // 16, K // 128, 16), dtype=torch.uint8, device=packed.device)
    rs = torch.empty((E, N), dtype=torch.float32, device=packed.device)
    _lib.check(_lib.load().dgm_transform_qoq_int4_weights(
        _lib.ptr(packed.contiguous()), _lib.ptr(pl), E, N, K, int(l1_interleave), _lib.ptr(vals), _lib.ptr(meta),
        _lib.ptr(rs), _lib.stream()))
    return vals, meta, rs


def transform_qoq_int4_weights_for_mega_moe_sm90(l1_weights, l2_weights, block_n: int = 128):
    """deep_gemm/mega/__init__.py:308: ``quantize_to_qoq_int4`` pairs ``(packed [E, N, K/2],
    plane int32 [E, N, K/128])`` -> the same layout as ``transform_qoq_weights_for_mega_moe_fused``
    (values, meta, s1) per matrix. ``block_n`` picks an SM90 tile there and has no effect here."""
    assert block_n in (128, 256)
    return _transform_qoq_int4_one(l1_weights, True), _transform_qoq_int4_one(l2_weights, False)


def transform_weights_for_mega_moe(l1, l2):
    """sm100_b200/mega___init__.py:102 for its W4A4 layer: low-nibble-first packed weights
    (per_token_cast_to_fp4 style) with one scale byte per 32 K (UE8M0: MXFP4 layout) or per 16 K
    (E4M3: NVFP4 layout); the scale count per row picks the format."""
    packed, sf = l1
    per_row = sf.shape[-1] * sf.element_size()
    k = 2 * packed.shape[-1]
    if per_row == k // 16:
        return transform_nvfp4_weights_for_mega_moe_fused(l1, l2, src_order="low_first")
    assert per_row == k // 32, f"scales per row {per_row} fit neither K/32 nor K/16 (K={k})"
    return transform_mxfp4_weights_for_mega_moe_fused(l1, l2, src_order="low_first")


# ----------------------------------------------------------------------------- frontend
SELECT_IN_MEGA_MAX_TOKENS = 64    # every workgroup of the fused kernel reads all tokens' logits
FE_ROUTER_TILE_MIN_TOKENS = 64    # the frontend's router rows of 8 tokens (csrc FE_TILE_MIN_TOKENS)
# csrc/fable_frontend.h kFEPath* (deep_gemm/mega/__init__.py:593): the launch-shape families of the
# reference's frontend. Here one router kernel serves every shape; fable_frontend_path names the
# family whose options apply (FE_PATH_CC: select_in_mega and zero-row unrouting available).
FE_PATH_WMMA, FE_PATH_SWAPAB, FE_PATH_CC = 0, 1, 2


def fable_frontend_path(m: int, h: int = 3072, e: int = 384, topk: int = 8) -> int:
    """deep_gemm/mega/__init__.py:600: the option family of the frontend for (m, h, e, topk):
    FE_PATH_CC up to SELECT_IN_MEGA_MAX_TOKENS tokens (the key array, select_in_mega and zero-row
    unrouting apply), FE_PATH_WMMA beyond."""
    assert m >= 0 and h % 512 == 0 and 0 < topk <= min(e, 16)
    return FE_PATH_CC if m <= SELECT_IN_MEGA_MAX_TOKENS else FE_PATH_WMMA


def fable_frontend_router_ctas(m: int, e: int, h: int = 3072, topk: int = 8) -> int:
    """deep_gemm/mega/__init__.py:653: router workgroups of the frontend launch for (m, h, e,
    topk): four experts per workgroup (one wave each) over 4 tokens, or over 8 tokens from
    FE_ROUTER_TILE_MIN_TOKENS on (the 8 hidden rows staged in LDS and shared by the waves)."""
    return ((e + 3) // 4) * ((m + 7) // 8 if m >= FE_ROUTER_TILE_MIN_TOKENS else (m + 3) // 4)


def fable_frontend_workspace_bytes(e: int, max_tokens: int = 64) -> int:
    """deep_gemm/mega/__init__.py:597: bytes of the frontend's scratch (fp32 logits and the u32
    key array of up to ``max_tokens`` tokens; both live in the layer buffer here)."""
    return 2 * 4 * e * max_tokens


def fable_frontend_workspace(sym_buffer, e: int, device=None) -> torch.Tensor:
    """deep_gemm/mega/__init__.py:658: the frontend's workspace of ``sym_buffer``: the buffer's
    logits and key-array region (uint8; zeroed with the buffer, no separate allocation)."""
    b = sym_buffer
    assert e == b.num_experts
    L = b.layout
    return b.buffer[L.logits:L.fe_keys + 4 * e * b.num_max_tokens_per_rank]


def fable_router_weight_fragment_layout(router_weight: torch.Tensor) -> torch.Tensor:
    """deep_gemm/mega/__init__.py:617: the reference's swapab A-fragment order of [E, K] bf16
    router weights ([E/16][K/32][half][g][t][8], same shape). Accepted by the frontend with
    ``wlayout="pre"``, which undoes it: this frontend reads row-major weights."""
    e, k = router_weight.shape
    assert router_weight.dtype == torch.bfloat16 and e % 16 == 0 and k % 32 == 0
    v = router_weight.contiguous().view(e // 16, 2, 8, k // 32, 4, 8)
    return v.permute(0, 3, 1, 2, 4, 5).contiguous().view(e, k)


def _router_weight_row_major(router_weight, wlayout):
    """Row-major router weights from a frontend ``wlayout`` ('row' / 'fragment': as given; 'pre':
    the fragment order of fable_router_weight_fragment_layout, undone)."""
    if wlayout is None:
        wlayout = os.environ.get("DG_FE_ROUTER_WLAYOUT", "fragment")
    if isinstance(wlayout, str):
        wlayout = {"row": 0, "fragment": 1, "pre": 2, "0": 0, "1": 1, "2": 2}[wlayout.strip().lower()]
    if int(wlayout) != 2:
        return router_weight
    e, k = router_weight.shape
    v = router_weight.contiguous().view(e // 16, k // 32, 2, 8, 4, 8)
    return v.permute(0, 2, 3, 1, 4, 5).contiguous().view(e, k)

def fable_router_quant_topk_frontend(hidden: torch.Tensor, router_weight: torch.Tensor, sym_buffer,
                                     quant: Optional[str] = None, stamps=None, l2_persist=None,
                                     wlayout=None, select_in_mega=None, zero_row_unrouted=None,
                                     force_balanced=None, token_offset: int = 0):
    """deep_gemm/mega/__init__.py:671: router GEMV (bf16 in, fp32 accumulate, bf16 logits) ->
    top-k (value desc, index asc) -> fp32 softmax of the k logits -> activation cast into
    ``sym_buffer.x / x_sf / topk_idx / topk_weights``. ``quant`` defaults to the buffer's
    activation format. ``force_balanced`` (env DG_FE_FORCE_BALANCED) replaces the routing by
    the forced-balanced rule after the router ran; ``zero_row_unrouted`` (env
    DG_FE_ZERO_ROW_UNROUTED, default 1) leaves all-zero rows unrouted. ``select_in_mega`` (env
    DG_FE_SELECT_IN_MEGA, default 0; tokens <= 64): stop after the logits and the cast; the
    next fused call on this buffer selects the top-k (in its prologue up to 8 tokens, else in a
    selection launch just before it) and writes ``topk_idx / topk_weights``, which are not valid
    before that call. ``stamps`` (env DG_FE_STAMPS, default 0): every frontend workgroup records
    phase stamps, read back with ``fable_frontend_stamps`` (the stamp rows are allocated on the
    first stamped call and kept with the buffer). ``l2_persist`` is an H20 tuning knob with no
    effect here; ``wlayout="pre"`` takes router weights in the fragment order of
    ``fable_router_weight_fragment_layout`` ("row" / "fragment": row-major weights, as given)."""
    b = sym_buffer
    _lib.require_gpu(hidden, router_weight)
    router_weight = _router_weight_row_major(router_weight, wlayout)
    assert hidden.dtype == torch.bfloat16 and router_weight.dtype == torch.bfloat16
    m, h = hidden.shape
    e = router_weight.size(0)
    assert h == b.hidden and e == b.num_experts and router_weight.size(1) == h
    assert m <= b.num_max_tokens_per_rank
    if quant is not None and quant != b.act_format:
        raise ValueError(f"buffer was sized for {b.act_format!r}, got quant={quant!r}")
    if force_balanced is None:
        force_balanced = os.environ.get("DG_FE_FORCE_BALANCED", "0") == "1"
    if zero_row_unrouted is None:
        zero_row_unrouted = os.environ.get("DG_FE_ZERO_ROW_UNROUTED", "1") == "1"
    if select_in_mega is None:
        select_in_mega = os.environ.get("DG_FE_SELECT_IN_MEGA", "0") == "1"
    select_in_mega = bool(select_in_mega) and m <= SELECT_IN_MEGA_MAX_TOKENS
    flags = (_lib.FE_FORCE_BALANCED if force_balanced else 0) | \
            (_lib.FE_ZERO_ROW_UNROUTED if zero_row_unrouted else 0)
    b._fe_select = (flags, int(token_offset)) if select_in_mega else None
    if select_in_mega:
        flags |= _lib.FE_SELECT_IN_MEGA
    if stamps is None:
        stamps = int(os.environ.get("DG_FE_STAMPS", "0"))
    st_ptr, st_rows = None, 0
    if stamps:
        st_rows = _lib.load().dgm_frontend_workgroups(m, h, e, b.act_code, flags, 1)
        have = getattr(b, "_fe_stamps", None)
        if have is None or have.size(0) < st_rows:
            b._fe_stamps = torch.zeros((max(st_rows, 1), 8), dtype=torch.int64, device=b.buffer.device)
        b._fe_stamps.zero_()
        st_ptr = b._fe_stamps
    b._fe_stamp_rows = st_rows
    hidden = hidden.contiguous()
    router_weight = router_weight.contiguous()
    _lib.check(_lib.load().dgm_router_topk_launch_stamped(
        _lib.ptr(hidden), _lib.ptr(router_weight), m, h, e, b.num_topk, b.act_code, flags,
        int(token_offset), _lib.ptr(b.buffer), ctypes.byref(b.layout), _lib.ptr(st_ptr), st_rows, _lib.stream()))


def fable_frontend_stamps(sym_buffer, e: int = None) -> torch.Tensor:
    """deep_gemm/mega/__init__.py:743: int64 [workgroups, 8] phase stamps of the last frontend call
    made with ``stamps=1`` on this buffer, in ns (the GPU's 100 MHz wall clock x 10; unused slots
    0). Rows: the router workgroups ([0] entry, [3] logits and keys stored, [6] hardware position
    HW_ID | XCC_ID << 32, [7] exit), then the cast workgroups ([0] entry, [5] cast stored, [6],
    [7]). The top-k selection runs in a launch of its own (or in the fused layer's prologue) and
    is not stamped here; the fused layer has its own ``phase_stamps``."""
    b = sym_buffer
    assert e is None or e == b.num_experts
    rows = getattr(b, "_fe_stamp_rows", 0)
    if not rows:
        raise RuntimeError("no stamped frontend call on this buffer: pass stamps=1 (or DG_FE_STAMPS=1)")
    out = b._fe_stamps[:rows].clone()
    pos = out[:, 6].clone()
    out.mul_(10)
    out[:, 6] = pos
    return out


def get_nvfp4_mega_moe_sm90_block_n(intermediate_hidden: int) -> int:
    """deep_gemm/mega/__init__.py:226: the SM90 NVFP4 N tile (128), kept for callers that pass it
    on; the MI355X layout (``transform_nvfp4_weights_for_mega_moe_fused``) has one tile shape."""
    assert intermediate_hidden > 0 and intermediate_hidden % 128 == 0
    return 128


def get_nvfp4_mega_moe_sm90_weight_layout(hidden: int, intermediate_hidden: int) -> str:
    """deep_gemm/mega/__init__.py:232: the packed-value layout the SM90 NVFP4 path caches for a
    model shape ("prmt_groups" when hidden > 2 * intermediate_hidden, else "marlin"). Kept for
    callers that record it; ``transform_nvfp4_weights_for_mega_moe_fused`` takes Marlin or
    low-nibble-first codes and writes one MI355X layout for every shape."""
    assert hidden > 0 and hidden % 128 == 0
    assert intermediate_hidden > 0 and intermediate_hidden % 128 == 0
    return "prmt_groups" if hidden > 2 * intermediate_hidden else "marlin"


def fable_frontend_keys(sym_buffer) -> torch.Tensor:
    """deep_gemm/mega/__init__.py:737: flat int32 view of the frontend's compact key array (token
    t, expert x at [t * E + x]) in this buffer, the array the fused layer selects from under
    ``select_in_mega``. Key = orderable(bf16 logit) << 16 | (0xFFFF - x); all keys of an
    unrouted (all-zero) row are 0."""
    return sym_buffer.fe_keys.view(-1)


# ----------------------------------------------------------------------------- fused layer
_ENTRY_FOR = {"qoq": "qoq_mega_moe_fused", "nvfp4": "fp4_fp4_mega_moe / nvfp4_mega_moe"}


def _check_host_error(b):
    if b.host_error():
        raise RuntimeError("MegaMoE: a bounded wait of an earlier launch on this buffer expired, so that launch's "
                           "output is wrong (workgroups not co-resident, or counters left inconsistent); "
                           "buffer.clear_error() resets the flag")


def _fused(y, l1, l2, b, stats, activation_clamp, num_tokens=None, split=False, phase_stamps=None,
           fast_math=True, fmt=None, global_scales=(None, None), fe=None, fe_keys=None, act=None):
    _check_host_error(b)
    args = _moe_args(y, l1, l2, b, stats, activation_clamp, num_tokens, phase_stamps, fast_math, fmt,
                     global_scales, fe, fe_keys, act)
    fn = _lib.load().dgm_megamoe_split_launch if split else _lib.load().dgm_megamoe_fused_launch
    _lib.check(fn(ctypes.byref(args), _lib.stream()))
    if os.environ.get("DG_CHECK_ERRORS", "0") == "1":     # debug: wait for the launch and check it
        torch.cuda.synchronize()
        if b.kernel_error():
            raise RuntimeError("MegaMoE: a bounded wait of this launch expired; its output is wrong")


def cooperative_launch(b):
    """Whether layer calls on buffer b launch the persistent kernel cooperatively: the buffer's
    ``cooperative`` attribute when set, else env ``DG_MEGA_COOPERATIVE=1``. The kernel's
    workgroups wait on each other, so they must all be resident at once; the default plain launch
    sizes its grid to the device's resident capacity, which holds when nothing else occupies the
    compute units. A cooperative launch guarantees it for callers that share the GPU with other
    streams or processes, at ~14-19 us per call (same results bit for bit). No counterpart in the
    reference."""
    c = getattr(b, "cooperative", None)
    return bool(c) if c is not None else os.environ.get("DG_MEGA_COOPERATIVE", "0") == "1"


def _moe_args(y, l1, l2, b, stats, activation_clamp, num_tokens=None, phase_stamps=None, fast_math=True,
              fmt=None, global_scales=(None, None), fe=None, fe_keys=None, act=None):
    """The C-ABI argument block (DgmMoeArgs) of one layer call on buffer b, after the checks."""
    act = act or b.act_format
    fmt = fmt or "mxfp4"         # (the MXFP entries pass no format)
    kind = lambda f: f if f in ("qoq", "nvfp4") else "mxfp"
    if kind(fmt) != kind(act):
        raise ValueError(f"buffer was sized for {act!r}: use "
                         f"{_ENTRY_FOR.get(act, 'mxfp4_mega_moe_fused / _split')}")
    qoq = act == "qoq"
    nv = act == "nvfp4"
    if nv:
        (w1, sf1), (w2, sf2) = l1, l2
        rs1 = rs2 = None
    else:     # (values, scales[, row scales]): MXFP4 weights carry no third item that is used
        w1, sf1, rs1 = l1[0], l1[1], (l1[2] if len(l1) > 2 else None)
        w2, sf2, rs2 = l2[0], l2[1], (l2[2] if len(l2) > 2 else None)
    _lib.require_gpu(y, w1, sf1, w2, sf2, stats)
    assert y.dtype == torch.bfloat16 and y.is_contiguous() and y.size(1) == b.hidden
    m = y.size(0) if num_tokens is None else num_tokens
    assert m <= b.num_max_tokens_per_rank
    E_l, H, I = b.num_local_experts, b.hidden, b.intermediate_hidden
    kg = lambda k: (k // 128 + 3) // 4
    assert tuple(w1.shape) == (E_l, 2 * I // 16, H // 128, 64, 16) and w1.dtype == torch.uint8, w1.shape
    assert tuple(w2.shape) == (E_l, H // 16, I // 128, 64, 16) and w2.dtype == torch.uint8, w2.shape
    if nv:    # E4M3 scales [E, N/16, K/128, 2, 16, 4]
        assert tuple(sf1.shape) == (E_l, 2 * I // 16, H // 128, 2, 16, 4) and sf1.dtype == torch.uint8, sf1.shape
        assert tuple(sf2.shape) == (E_l, H // 16, I // 128, 2, 16, 4) and sf2.dtype == torch.uint8, sf2.shape
        for g in global_scales:
            if g is not None:
                _lib.require_gpu(g)
                assert g.dtype == torch.float32 and g.numel() == E_l and g.is_contiguous()
    elif qoq:   # meta [E, N/16, K/128, 16] (z | s2 << 4 per row), row scales s1 [E, N]
        _lib.require_gpu(rs1, rs2)
        assert tuple(sf1.shape) == (E_l, 2 * I // 16, H // 128, 16) and sf1.dtype == torch.uint8, sf1.shape
        assert tuple(sf2.shape) == (E_l, H // 16, I // 128, 16) and sf2.dtype == torch.uint8, sf2.shape
        assert tuple(rs1.shape) == (E_l, 2 * I) and rs1.dtype == torch.float32 and rs1.is_contiguous(), rs1.shape
        assert tuple(rs2.shape) == (E_l, H) and rs2.dtype == torch.float32 and rs2.is_contiguous(), rs2.shape
    else:
        assert tuple(sf1.shape) == (E_l, 2 * I // 16, kg(H), 64, 4) and sf1.dtype == torch.uint8, sf1.shape
        assert tuple(sf2.shape) == (E_l, H // 16, kg(I), 64, 4) and sf2.dtype == torch.uint8, sf2.shape
    assert all(t.is_contiguous() for t in (w1, sf1, w2, sf2))
    if stats is not None:
        assert stats.dtype == torch.int32 and stats.numel() == E_l
    sel = getattr(b, "_fe_select", None)
    if fe is not None:        # in-kernel frontend: (hidden, router_weight, flags, token_offset)
        hidden, router_weight, fe_flags, fe_off = fe
        sel = (fe_flags, fe_off)
        b._fe_select = None
        fe_keys = None
    elif fe_keys is not None:
        # the caller's key array (the reference's compact keys: token t, expert x at t * E + x)
        _lib.require_gpu(fe_keys)
        assert fe_keys.dtype in (torch.int32, torch.uint32) and fe_keys.is_contiguous(), fe_keys.dtype
        assert fe_keys.numel() >= m * b.num_experts, (fe_keys.numel(), m, b.num_experts)
        sel = (sel[0] & _lib.FE_FORCE_BALANCED if sel else 0, sel[1] if sel else 0)
    args = _lib.MoeArgs(num_tokens=m, hidden=b.hidden, intermediate=b.intermediate_hidden,
                        num_experts=b.num_experts, expert_begin=b.expert_begin, num_local_experts=E_l,
                        topk=b.num_topk, act_format=_lib.ACT_FORMATS[act],
                        activation_clamp=float(activation_clamp if activation_clamp is not None else 3.0e38),
                        fast_math=int(bool(fast_math)), select_in_mega=int(sel is not None),
                        fe_flags=sel[0] if sel else 0, token_offset=sel[1] if sel else 0,
                        w1_values=w1.data_ptr(), w1_scales=sf1.data_ptr(), w2_values=w2.data_ptr(),
                        w2_scales=sf2.data_ptr(), recv_stats=stats.data_ptr() if stats is not None else None,
                        y=y.data_ptr(), buffer=b.buffer.data_ptr(), layout=ctypes.pointer(b.layout),
                        phase_stamps=phase_stamps.data_ptr() if phase_stamps is not None else None,
                        phase_stamp_rows=phase_stamps.numel() // 8 if phase_stamps is not None else 0,
                        w1_row_scales=rs1.data_ptr() if qoq else None,
                        w2_row_scales=rs2.data_ptr() if qoq else None,
                        l1_global_scales=global_scales[0].data_ptr() if global_scales[0] is not None else None,
                        l2_global_scales=global_scales[1].data_ptr() if global_scales[1] is not None else None,
                        fe_in_mega=int(fe is not None),
                        hidden_states=fe[0].data_ptr() if fe is not None else None,
                        router_weight=fe[1].data_ptr() if fe is not None else None,
                        fe_keys=fe_keys.data_ptr() if fe_keys is not None else None,
                        host_error=b._host_err_dev, debug_flags=getattr(b, "_debug_flags", 0),
                        launch_flags=_lib.LAUNCH_COOPERATIVE if cooperative_launch(b) else 0)
    if phase_stamps is not None:
        assert phase_stamps.dtype == torch.int64 and phase_stamps.is_cuda and phase_stamps.is_contiguous()
    return args


def mxfp4_mega_moe_fused(y, l1, l2, b, cumulative_local_expert_recv_stats=None, activation_clamp=10.0,
                         fast_math=True, phase_stamps=None, fe_keys=None):
    """deep_gemm/mega/fused.py:97: the layer over the routing and activations already in the
    buffer (written by ``fable_router_quant_topk_frontend`` or by the caller): dispatch,
    L1 + SwiGLU + requant, L2, top-k combine into ``y`` (bf16 [tokens, H]), as one launch of the
    persistent kernel. On an "fp8f128" buffer (the reference's fused buffer: E4M3 activations with
    fp32 scales per 128) it runs that recipe: each K-tile's product promoted by its scale, fp32
    gate / up, a power-of-two E4M3 intermediate per 64 features.
    ``phase_stamps`` (optional int64 CUDA tensor [rows, 8]; workgroups >= rows skip): per-workgroup
    100 MHz wall-clock stamps (see ``fused_workgroups``). ``fast_math`` (default True, as in the
    reference): hardware exp2 / reciprocal in SiLU's sigmoid; False = IEEE expf and division.
    ``fe_keys``: an int32 key array [tokens, E] (``fable_frontend_keys``; the frontend's compact
    keys, orderable bf16 logit << 16 | 0xFFFF - expert, a zero first key = unrouted token) the
    top-k is selected from in the kernel's prologue; by default the buffer's own keys when the
    frontend ran with ``select_in_mega``, else the buffer's ``topk_idx`` / ``topk_weights``.
    A bounded wait that expired in an earlier launch on this buffer raises here (the host-visible
    error word; ``DG_CHECK_ERRORS=1`` checks every launch at once, synchronising)."""
    _fused(y, l1, l2, b, cumulative_local_expert_recv_stats, activation_clamp, phase_stamps=phase_stamps,
           fast_math=fast_math, fe_keys=fe_keys)


def qoq_mega_moe_fused(y, l1, l2, b, cumulative_local_expert_recv_stats=None, activation_clamp=10.0,
                       fast_math=True, phase_stamps=None, fe_keys=None):
    """deep_gemm/mega/fused.py:102: the QoQ W4A8 layer (``get_fused_symm_buffer_for_mega_moe(...,
    act_format="qoq")``, weights from ``transform_qoq_weights_for_mega_moe_fused``): int8
    activations with one scale per token, 4-bit weight codes with per-(row, K128) zero point and
    integer scale and per-row fp32 scale, exact int32 group sums; fp32 gate / up, SiLU * up *
    routing weight, int8 requant per 64 features, L2 (each route rounded to bf16), fp32 combine ->
    bf16 ``y``. ``fe_keys`` as for ``mxfp4_mega_moe_fused``. Limits per call (QoQ and NVFP4 run
    only on the persistent kernel): tokens x topk <= 1024, tokens <= 256, local experts <= 512;
    beyond them the call raises RuntimeError (no launch)."""
    _fused(y, l1, l2, b, cumulative_local_expert_recv_stats, activation_clamp, phase_stamps=phase_stamps,
           fast_math=fast_math, fmt="qoq", fe_keys=fe_keys)


def fp4_fp4_mega_moe(y, l1_weights, l2_weights, sym_buffer, cumulative_local_expert_recv_stats=None,
                     recipe=None, activation="swiglu", activation_clamp=None, fast_math=True):
    """sm100_b200/mega___init__.py:244 W4A4 entry: packed E2M1 activations and weights. On an
    ``act_format="nvfp4"`` buffer (E4M3 scale per 16; weights from
    ``transform_nvfp4_weights_for_mega_moe_fused``) it runs the NVFP4 layer; on an "mxfp4"
    buffer the MXFP4 layer (weights from ``transform_mxfp4_weights_for_mega_moe_fused``).
    ``activation_clamp=None`` = no clamp. NVFP4 limits per call: tokens x topk <= 1024, tokens
    <= 256, local experts <= 512 (RuntimeError beyond them; MXFP4 has none)."""
    b = sym_buffer
    assert b.act_format in ("mxfp4", "nvfp4"), "buffer must be created with act_format mxfp4/nvfp4"
    vec = 16 if b.act_format == "nvfp4" else 32
    assert recipe is None or tuple(recipe)[2] == vec, recipe
    assert activation == "swiglu", activation
    _fused(y, l1_weights, l2_weights, b, cumulative_local_expert_recv_stats, activation_clamp,
           fast_math=fast_math, fmt=b.act_format)


def nvfp4_mega_moe(y, l1_weights, l2_weights, sym_buffer, cumulative_local_expert_recv_stats=None,
                   l1_global_scales=None, l2_global_scales=None, recipe=(128, 128, 128), activation="swiglu",
                   activation_clamp=None, fast_math=True, kernel_family="auto", family_threshold=256):
    """deep_gemm/mega/__init__.py:277 NVFP4 entry with per-expert fp32 global scales
    (``l1_global_scales`` / ``l2_global_scales`` [E_local], multiplied into the L1 / L2
    outputs), here on an ``act_format="nvfp4"`` buffer (W4A4). ``recipe``, ``kernel_family`` and
    ``family_threshold`` select SM90 kernel families there; here "split" runs the same kernel as
    two launches. Both families run on the persistent kernel, so a call holds at most 1024 routes
    (tokens x topk), 256 tokens and 512 local experts; beyond them it raises
    RuntimeError before any launch."""
    assert sym_buffer.act_format == "nvfp4", "buffer must be created with act_format='nvfp4'"
    assert activation == "swiglu", activation
    if kernel_family not in ("auto", "split", "fused"):
        raise ValueError("kernel_family must be one of 'auto', 'fused', or 'split'")
    if family_threshold <= 0:
        raise ValueError("family_threshold must be positive")
    # 'split' (or 'auto' above family_threshold tokens): two launches, dispatch + L1 then L2 +
    # combine, with the fused launch's results bit for bit
    split = kernel_family == "split" or (kernel_family == "auto" and y.size(0) > family_threshold)
    _fused(y, l1_weights, l2_weights, sym_buffer, cumulative_local_expert_recv_stats, activation_clamp,
           split=split, fast_math=fast_math, fmt="nvfp4", global_scales=(l1_global_scales, l2_global_scales))


def _weights_kind(l1):
    """Activation format a layer's weights imply: QoQ (values, meta [.., 16], s1), NVFP4
    (values, E4M3 scales [.., 2, 16, 4]) or MXFP4 (values, E8M0 scales [.., 64, 4][, None])."""
    sf = l1[1]
    if len(l1) == 3 and l1[2] is not None and sf.dim() == 4 and sf.size(-1) == 16:
        return "qoq"
    if sf.dim() == 6:
        return "nvfp4"
    return "mxfp"


def _cast_into(b, hidden_input, act):
    """The activation cast of ``hidden_input`` (bf16 [tokens, H]) into the buffer's x / x_sf."""
    _lib.require_gpu(hidden_input)
    assert hidden_input.dtype == torch.bfloat16 and hidden_input.size(1) == b.hidden
    assert hidden_input.size(0) <= b.num_max_tokens_per_rank
    h = hidden_input.contiguous()
    _lib.check(_lib.load().dgm_router_topk_launch(
        _lib.ptr(h), None, h.size(0), b.hidden, b.num_experts, b.num_topk, _lib.ACT_FORMATS[act], 0, 0,
        _lib.ptr(b.buffer), ctypes.byref(b.layout), _lib.stream()))


def _split_entry(fmts, y, l1_weights, l2_weights, sym_buffer, cumulative_local_expert_recv_stats=None,
                 l1_global_scales=None, l2_global_scales=None, recipe=None, activation="swiglu",
                 activation_clamp=None, fast_math=True, attn_tp_size=1, attn_tp_group=None,
                 broadcast_output=False, router_input=None, router_weight=None, router_logits=None,
                 router_renormalize=True, tp_combine_output=None, hidden_input=None, act=None):
    """The split API's argument list (deep_gemm/mega/__init__.py:340-433 mxfp4_mega_moe).
    ``hidden_input`` (bf16 [tokens, H]): cast into x / x_sf first. ``router_input`` /
    ``router_weight``: the router and top-k run on those (x / x_sf are left as they are; an
    all-zero router_input row is unrouted unless DG_FE_ZERO_ROW_UNROUTED=0);
    ``router_logits`` (bf16 [tokens, E]): the top-k of those logits. ``router_renormalize``:
    weights = softmax over the top-k, else the selected values themselves. Otherwise the routing
    in the buffer (topk_idx / topk_weights) is used. One GPU: attn_tp_size must be 1."""
    b = sym_buffer
    act = act or b.act_format
    if act not in fmts:
        raise ValueError(f"buffer was sized for {act!r}; this entry point takes {fmts}")
    assert activation == "swiglu", activation
    assert (router_input is None) == (router_weight is None)
    assert router_logits is None or router_input is None
    if recipe is not None:
        assert len(tuple(recipe)) == 3, recipe
    if attn_tp_size != 1 or tp_combine_output is not None or broadcast_output:
        raise NotImplementedError("attention-TP layouts need more than one GPU")
    if act != "nvfp4" and (l1_global_scales is not None or l2_global_scales is not None):
        raise ValueError("per-expert global scales are an NVFP4 option")
    m = y.size(0)
    if hidden_input is not None:
        assert tuple(hidden_input.shape) == tuple(y.shape), (hidden_input.shape, y.shape)
        _cast_into(b, hidden_input, act)
    flags = 0 if router_renormalize else _lib.FE_RAW_WEIGHTS
    if router_input is not None:
        _lib.require_gpu(router_input, router_weight)
        assert router_input.dtype == torch.bfloat16 and router_weight.dtype == torch.bfloat16
        assert tuple(router_input.shape) == (m, b.hidden)
        assert tuple(router_weight.shape) == (b.num_experts, b.hidden)
        if not router_renormalize:
            raise NotImplementedError("router_input with router_renormalize=False: pass the weights' "
                                      "logits as router_logits instead")
        ri, rw = router_input.contiguous(), router_weight.contiguous()
        # (an all-zero router_input row is left unrouted, as the frontend does by default:
        # env DG_FE_ZERO_ROW_UNROUTED)
        zr = _lib.FE_ZERO_ROW_UNROUTED if os.environ.get("DG_FE_ZERO_ROW_UNROUTED", "1") == "1" else 0
        _lib.check(_lib.load().dgm_router_topk_launch(
            _lib.ptr(ri), _lib.ptr(rw), m, b.hidden, b.num_experts, b.num_topk, _lib.ACT_FORMATS[act],
            _lib.FE_NO_CAST | zr, 0, _lib.ptr(b.buffer), ctypes.byref(b.layout), _lib.stream()))
        b._fe_select = None
    elif router_logits is not None:
        _lib.require_gpu(router_logits)
        assert router_logits.dtype == torch.bfloat16 and tuple(router_logits.shape) == (m, b.num_experts)
        rl = router_logits.contiguous()
        _lib.check(_lib.load().dgm_router_logits_topk_launch(
            _lib.ptr(rl), m, b.num_experts, b.num_topk, flags, 0, _lib.ptr(b.buffer), ctypes.byref(b.layout),
            _lib.stream()))
        b._fe_select = None
    _fused(y, l1_weights, l2_weights, b, cumulative_local_expert_recv_stats, activation_clamp, split=True,
           fast_math=fast_math, fmt=act, global_scales=(l1_global_scales, l2_global_scales), act=act)


def qoq_mega_moe_split(y, l1_weights, l2_weights, sym_buffer, *args, **kwargs):
    """deep_gemm/mega/__init__.py:584: the QoQ W4A8 layer as two launches of the persistent
    kernel (dispatch + L1 into the buffer's intermediate rows, then L2 + combine), on an
    ``act_format="qoq"`` buffer; weights from ``transform_qoq_weights_for_mega_moe_fused`` or
    ``transform_qoq_int4_weights_for_mega_moe_sm90``. Same results as ``qoq_mega_moe_fused``
    bit for bit. Arguments as ``mxfp4_mega_moe`` (activation_clamp default None = no clamp).
    Limits per call, as for the fused launch: tokens x topk <= 1024, tokens <= 256, local
    experts <= 512 (RuntimeError beyond them, before any launch)."""
    _split_entry(("qoq",), y, l1_weights, l2_weights, sym_buffer, *args, **kwargs)


def fused_workgroups(b):
    """Workgroups of the persistent kernel for this buffer's shape (after its first launch)."""
    return _lib.load().dgm_fused_workgroups(b.hidden, b.intermediate_hidden, b.act_code)


FUSED_FORMS = {0: "plain", 1: "in-kernel frontend", 2: "early weight streaming", 3: "tail half units"}


def fused_last_form(b):
    """The form the persistent kernel's last launch for this buffer's shape and format ran (a
    key of ``FUSED_FORMS``; -1 before the first). Two opt-in forms, both measured slower than the
    default: early weight streaming for small routed sets (MXFP4 / MXFP8 activations, at most 32
    local routes expected), turned on by the buffer's ``_debug_flags`` bit 3, and tail half units
    for up to 32 routes (A-MXFP4 / A-MXFP8 at H = 3072: the last round of L1 units, when at most
    half full, runs as half units), bit 4."""
    return _lib.load().dgm_fused_last_form(b.hidden, b.intermediate_hidden, b.act_code)


def mxfp4_mega_moe_split(y, l1_weights, l2_weights, sym_buffer, *args, **kwargs):
    """deep_gemm/mega/__init__.py:579 split API: the same layer as separate launches (dispatch,
    L1 + SwiGLU + requant, L2, combine) with the fused path's numerics, on an "mxfp4" / "mxfp8"
    fused buffer. Arguments as ``mxfp4_mega_moe`` (:340; activation_clamp default None = no
    clamp)."""
    _split_entry(("mxfp4", "mxfp8", "fp8"), y, l1_weights, l2_weights, sym_buffer, *args, **kwargs)


class SymmBuffer(FusedSymmBuffer):
    """deep_gemm/mega/__init__.py:20 ``SymmBuffer``, the split path's buffer, on one GPU.

    ``mma_type="fp8xmxfp4"`` (the SM90 split recipe): ``x`` E4M3 [tokens, H] with ``x_sf`` fp32
    [tokens, H/128] (``per_token_cast_to_fp8(x, use_ue8m0=False, gran_k=128)``; the QoQ layer
    reads int8 bytes with the per-token scale repeated, ``per_token_cast_to_int8``),
    ``topk_idx`` int64 / ``topk_weights`` fp32 [tokens, topk]; ``l1_acts`` / ``l1_acts_sf`` alias
    x / x_sf (routed rows are read in place); ``l2_acts`` E4M3 [routes, I] with ``l2_acts_sf``
    E8M0 bytes [routes, I/32]. ``mma_type="fp8xfp4"``: x E4M3 with the UE8M0 scales of each
    32 elements packed four to an int32 (``x_sf`` int32 [tokens, H/128]). ``num_ring_tokens`` sizes
    the reference's ring pool; here every route has its own row."""

    _MMA = {"fp8xmxfp4": "fp8f128", "fp8xfp4": "mxfp8"}

    def __init__(self, group, num_experts, num_max_tokens_per_rank, num_topk, hidden, intermediate_hidden,
                 num_ring_tokens=None, mma_type="fp8xfp4", activation="swiglu"):
        assert activation == "swiglu", f"Only `swiglu` activation is supported, got `{activation}`"
        if mma_type not in self._MMA:
            raise ValueError(f"mma_type {mma_type!r}: one of {sorted(self._MMA)}")
        super().__init__(group, num_experts, num_max_tokens_per_rank, num_topk, hidden, intermediate_hidden,
                         act_format=self._MMA[mma_type])
        self.mma_type = mma_type
        self.num_ring_tokens = num_ring_tokens if num_ring_tokens is not None else num_max_tokens_per_rank * num_topk
        if mma_type == "fp8xfp4":      # UE8M0 bytes per 32, four to an int32
            self.x = self.x.view(torch.float8_e4m3fn)
            self.x_sf = self.x_sf.view(torch.int32)
            self.l1_acts, self.l1_acts_sf = self.x, self.x_sf

    def destroy(self):
        super().destroy()
        self.x = self.x_sf = None


def get_symm_buffer_for_mega_moe(group, num_experts, num_max_tokens_per_rank, num_topk, hidden,
                                 intermediate_hidden, use_fp8_dispatch=None, mma_type="fp8xfp4",
                                 activation="swiglu"):
    """deep_gemm/mega/__init__.py:70: the split path's buffer (``group=None``: one GPU)."""
    if use_fp8_dispatch is not None:
        assert use_fp8_dispatch == (mma_type.split("x")[0] == "fp8")
    return SymmBuffer(group, num_experts, num_max_tokens_per_rank, num_topk, hidden, intermediate_hidden,
                      num_max_tokens_per_rank * num_topk, mma_type=mma_type, activation=activation)


def get_mxfp4_mega_moe_sm90_block_n(hidden, intermediate_hidden, expected_m_per_rank=None):
    """deep_gemm/mega/__init__.py:244: the SM90 N tile; accepted for the interface, one layout
    serves every tile choice here."""
    assert hidden % 128 == 0 and intermediate_hidden % 128 == 0
    if expected_m_per_rank is None:
        return 128
    crossover = 192 if intermediate_hidden <= 2048 else 384
    return 256 if expected_m_per_rank >= crossover else 128


def transform_mxfp4_weights_for_mega_moe_sm90(l1_weights, l2_weights, block_n=None, block_k=128, group_size=32,
                                              expected_m_per_rank=None):
    """deep_gemm/mega/__init__.py:257: MXFP4 weights ``(packed [E, N, K/2] (Marlin, as
    deep_gemm/quantization_mxfp4.py quantize_to_mxfp4 writes them), E8M0 scales [E, N, K/32])``
    -> ``((w1_values, w1_scales), (w2_values, w2_scales))`` in the matrix-core fragment layout
    (gate / up blocks of W1 interleaved), for ``mxfp4_mega_moe``. ``block_n`` picks an SM90
    tile there and has no effect here."""
    assert block_n in (None, 128, 256) and block_k == 128 and group_size == 32
    (v1, s1, _), (v2, s2, _) = transform_mxfp4_weights_for_mega_moe_fused(l1_weights, l2_weights)
    return (v1, s1), (v2, s2)


def mxfp4_mega_moe(y, l1_weights, l2_weights, sym_buffer, cumulative_local_expert_recv_stats=None,
                   l1_global_scales=None, l2_global_scales=None, recipe=None, activation="swiglu",
                   activation_clamp=None, fast_math=True, attn_tp_size=1, attn_tp_group=None,
                   broadcast_output=False, router_input=None, router_weight=None, router_logits=None,
                   router_renormalize=True, tp_combine_output=None, hidden_input=None, _cpp_op=None):
    """deep_gemm/mega/__init__.py:340: the split MegaMoE layer on a ``SymmBuffer``.

    MXFP4 weights (``transform_mxfp4_weights_for_mega_moe_sm90``) on an ``mma_type="fp8xmxfp4"``
    buffer: E4M3 activations with fp32 scales per 128 (each K-tile's products times its scale),
    fp32 gate / up, clamp, SiLU * up * routing weight, E4M3 intermediate with one power-of-two
    scale per 64 features, L2, each route rounded to bf16, fp32 slot-order combine
    (tests/test_four_api_correctness.py:421-446). On an ``"fp8xfp4"`` buffer: the MXFP8 layer
    (UE8M0 scales per 32). QoQ weights (``transform_qoq_int4_weights_for_mega_moe_sm90``, the
    ``int4_mega_moe`` alias) run the QoQ W4A8 layer on the same buffer (int8 bytes in x, the
    token's scale in x_sf). ``activation_clamp=None``: no clamp. Routing inputs as in the
    reference: the buffer's topk_idx / topk_weights, or ``router_input`` + ``router_weight``, or
    ``router_logits`` (bf16); ``hidden_input`` (bf16) is cast into x / x_sf first."""
    b = sym_buffer
    kind = _weights_kind(l1_weights)
    if kind == "qoq":
        if b.act_format not in ("fp8f128", "qoq"):
            raise ValueError("QoQ weights need an mma_type='fp8xmxfp4' SymmBuffer (or a 'qoq' fused buffer)")
        act = "qoq"
    elif kind == "nvfp4":
        act = "nvfp4"
    else:
        act = b.act_format
    _split_entry(("fp8f128", "mxfp8", "mxfp4", "qoq", "nvfp4"), y, l1_weights, l2_weights, b,
                 cumulative_local_expert_recv_stats, l1_global_scales, l2_global_scales, recipe, activation,
                 activation_clamp, fast_math, attn_tp_size, attn_tp_group, broadcast_output, router_input,
                 router_weight, router_logits, router_renormalize, tp_combine_output, hidden_input, act=act)


# deep_gemm/mega/__init__.py:448: one entry for both weight families (the weights pick the layer)
int4_mega_moe = mxfp4_mega_moe


def mxfp4_mega_moe_from_bf16(y, hidden_states, router_weight, l1, l2, b,
                             cumulative_local_expert_recv_stats=None, activation_clamp=10.0,
                             force_balanced=None, token_offset=0, phase_stamps=None, one_launch=None, **_):
    """deep_gemm/mega/__init__.py:451: frontend + fused layer from bf16 hidden states: the
    frontend launch, then the fused launch (the top-k selected in its prologue up to 8 tokens,
    by a selection launch between the two up to 64, by the frontend beyond).
    ``one_launch`` (env DG_ONE_LAUNCH=1; up to 64 tokens): a single launch instead, in which the
    fused kernel computes the router logits, zero-row flags and activation cast itself (spread
    over all workgroups) and meets at a grid-wide arrival counter before its prologue; same
    results bit for bit, 1.5-4.3 us slower than the two launches on MI355X (the grid-wide arrival
    and the key reload after it cost more than the second launch does)."""
    # (a qoq buffer runs the QoQ layer: the reference's DG_W4A8_INT=1 route; an nvfp4 buffer the
    # W4A4 NVFP4 layer)
    m = hidden_states.size(0)
    if one_launch is None:
        one_launch = os.environ.get("DG_ONE_LAUNCH", "0") == "1"
    if one_launch and m <= SELECT_IN_MEGA_MAX_TOKENS and b.hidden % 512 == 0:
        # one launch: the fused kernel runs the frontend (router, zero-row flags, cast) itself
        _lib.require_gpu(hidden_states, router_weight)
        assert hidden_states.dtype == torch.bfloat16 and router_weight.dtype == torch.bfloat16
        assert hidden_states.size(1) == b.hidden and tuple(router_weight.shape) == (b.num_experts, b.hidden)
        if force_balanced is None:
            force_balanced = os.environ.get("DG_FE_FORCE_BALANCED", "0") == "1"
        zero_row = os.environ.get("DG_FE_ZERO_ROW_UNROUTED", "1") == "1"
        flags = (_lib.FE_FORCE_BALANCED if force_balanced else 0) | (_lib.FE_ZERO_ROW_UNROUTED if zero_row else 0)
        assert y.size(0) == m
        _fused(y, l1, l2, b, cumulative_local_expert_recv_stats, activation_clamp, fmt=b.act_format,
               fe=(hidden_states.contiguous(), router_weight.contiguous(), flags, int(token_offset)),
               phase_stamps=phase_stamps)
        return y
    fable_router_quant_topk_frontend(hidden_states, router_weight, b, force_balanced=force_balanced,
                                     token_offset=token_offset, select_in_mega=True)
    _fused(y, l1, l2, b, cumulative_local_expert_recv_stats, activation_clamp, fmt=b.act_format,
           phase_stamps=phase_stamps)
    return y
