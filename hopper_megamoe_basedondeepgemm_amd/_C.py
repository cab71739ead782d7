"""The reference's ``deep_gemm._C`` MegaMoE functions, with the same names and positional
argument order (csrc/python_api.cpp:18-30 registration; csrc/apis/mega_fused.hpp:31-105 and
csrc/apis/mega.hpp:375-560, 741-800 definitions), over the HIP library's C ABI.

Buffers: ``get_symm_buffer_size_for_fused_mega_moe`` / ``get_symm_buffer_size_for_mega_moe``
return ``(nbytes, slice_fn)``; the caller allocates ``nbytes`` (zeroed) and calls ``slice_fn``
on it, as the reference's Python classes do. Both lay out the reference's fused-buffer bytes:
x [tokens, H] bytes (E4M3, or int8 for QoQ) with fp32 scales per 128 (``x_sf`` [tokens, H/128]),
topk_idx / topk_weights, the intermediate rows and the bf16 route outputs. ``slice_fn`` records
the layout under the buffer's address; the layer calls find it there (a buffer must be sliced
before its first call). ``sym_buffer_ptrs`` / ``rank_idx`` name one GPU's share: one pointer,
rank 0.

``mxfp4_mega_moe_fused`` runs the layer on E4M3 activations with fp32 scales per 128 (the
input format tests/test_four_api_correctness.py:215 writes into this buffer), MXFP4 weights from
``transform_mxfp4_weights_for_mega_moe_fused``, as one launch of the persistent kernel;
``qoq_mega_moe_fused`` the QoQ W4A8 layer.
"""
import weakref

import torch

from . import _lib
from . import mega


# (data_ptr, rank, activation format) -> (shape, FusedSymmBuffer over the caller's tensor). An
# entry lives as long as the caller's tensor object does (a finalizer on it removes the entry and
# with it the wrapper's view of the storage), and slicing the same memory for another shape
# replaces it.
_BUFFERS = {}


def _release(key, b):
    if key in _BUFFERS and _BUFFERS[key][1] is b:
        del _BUFFERS[key]


def _wrap(buffer, num_ranks, num_experts, max_tokens, topk, hidden, intermediate, rank=0, act="fp8f128"):
    key = (buffer.data_ptr(), int(rank), act)
    shape = (int(num_ranks), int(num_experts), int(max_tokens), int(topk), int(hidden), int(intermediate))
    hit = _BUFFERS.get(key)
    if hit is None or hit[0] != shape or hit[1].buffer.nbytes > buffer.nbytes:
        b = mega.FusedSymmBuffer(None, num_experts, max_tokens, topk, hidden, intermediate, act_format=act,
                                 ep_size=num_ranks, ep_rank=rank, buffer=buffer)
        _BUFFERS[key] = (shape, b)
        weakref.finalize(buffer, _release, key, b)
        return b
    return hit[1]


def _views(b, with_partials):
    q = b.x.view(torch.float8_e4m3fn) if b.x.dtype != torch.float8_e4m3fn else b.x
    out = (q, b.x_sf, b.topk_idx, b.topk_weights, q, b.x_sf, b.l2_acts, b.l2_acts_sf)
    return out + (b.combine_partials,) if with_partials else out


def _lookup(buffer, rank, act="fp8f128"):
    hit = _BUFFERS.get((buffer.data_ptr(), int(rank), act))
    if hit is not None:
        return hit[1]
    for (ptr, r, a), (_, b) in list(_BUFFERS.items()):
        if ptr == buffer.data_ptr() and r == int(rank):     # the same memory in the other format
            return _wrap(buffer, b.ep_size, b.num_experts, b.num_max_tokens_per_rank, b.num_topk,
                         b.hidden, b.intermediate_hidden, rank, act)
    raise RuntimeError("MegaMoE buffer not sliced: call the slice function of "
                       "get_symm_buffer_size_for_(fused_)mega_moe on it first")


# ----------------------------------------------------------------------------- fused API
def get_symm_buffer_size_for_fused_mega_moe(num_ranks, num_experts, max_tokens, topk, hidden, intermediate):
    """csrc/apis/mega_fused.hpp:31: (nbytes, slice_fn); slice_fn(buffer) -> (x, x_sf, topk_idx,
    topk_weights, l1_acts, l1_acts_sf, l2_acts, l2_acts_sf, combine_partials)."""
    assert num_experts % num_ranks == 0
    L = _lib.layout(max_tokens, num_experts, num_experts // num_ranks, topk, hidden, intermediate,
                    _lib.ACT_FORMATS["fp8f128"])

    def slice_fn(buffer):
        return _views(_wrap(buffer, num_ranks, num_experts, max_tokens, topk, hidden, intermediate), True)
    return int(L.total_bytes), slice_fn


def _run_fused(act, y, l1, l2, stats, s1, s2, buffer, ptrs, rank, max_tokens, num_experts, topk, clamp,
               fast_math, phase_stamps, fe_keys):
    b = _lookup(buffer, rank, act)
    assert b.num_max_tokens_per_rank == max_tokens and b.num_experts == num_experts and b.num_topk == topk
    assert len(ptrs) == b.ep_size, (len(ptrs), b.ep_size)
    w1 = (l1[0], l1[1], s1)
    w2 = (l2[0], l2[1], s2)
    # one launch of the persistent kernel (beyond its limits, 1024 routes, 256 tokens, 512 local
    # experts, the E4M3 layer runs as the split path's kernels, with the same results)
    mega._fused(y, w1, w2, b, stats, clamp, phase_stamps=phase_stamps, fast_math=fast_math, fmt=act,
                fe_keys=fe_keys, act=act)


def mxfp4_mega_moe_fused(y, l1, l2, stats, s1, s2, buffer, ptrs, rank, max_tokens, num_experts, topk, clamp,
                         fast_math, phase_stamps=None, fe_keys=None):
    """csrc/apis/mega_fused.hpp:101: ``(y, (w1, sf1), (w2, sf2), stats?, rs1, rs2, buffer, ptrs,
    rank, max_tokens, E, topk, clamp?, fast_math, phase_stamps?, fe_keys?)``; rs1 / rs2 are the
    third items of ``transform_mxfp4_weights_for_mega_moe_fused`` (unused by MXFP4)."""
    _run_fused("fp8f128", y, l1, l2, stats, s1, s2, buffer, ptrs, rank, max_tokens, num_experts, topk, clamp,
               fast_math, phase_stamps, fe_keys)


def qoq_mega_moe_fused(y, l1, l2, stats, s1, s2, buffer, ptrs, rank, max_tokens, num_experts, topk, clamp,
                       fast_math, phase_stamps=None, fe_keys=None):
    """csrc/apis/mega_fused.hpp:103: the QoQ W4A8 layer; l1 / l2 = (values, meta) and s1 / s2 the
    per-row scales of ``transform_qoq_weights_for_mega_moe_fused``."""
    _run_fused("qoq", y, l1, l2, stats, s1, s2, buffer, ptrs, rank, max_tokens, num_experts, topk, clamp,
               fast_math, phase_stamps, fe_keys)


# ----------------------------------------------------------------------------- split API
def get_token_alignment_for_mega_moe():
    """csrc/apis/mega.hpp:26: token-count alignment of the split buffer (none needed here)."""
    return 1


def get_ring_limit_for_mega_moe(num_max_tokens_per_rank, num_experts_per_rank, num_topk, num_ranks):
    """csrc/apis/mega.hpp:30: (min, max) pool rows; every route has its own row here."""
    n = num_max_tokens_per_rank * num_topk * num_ranks
    return n, n


def get_legacy_pool_tokens_for_mega_moe(num_max_tokens_per_rank, num_experts_per_rank, num_topk, num_ranks):
    """csrc/apis/mega.hpp:46."""
    return num_max_tokens_per_rank * num_topk * num_ranks


def get_symm_buffer_size_for_mega_moe(num_ranks, num_experts, num_max_tokens_per_rank, num_topk, hidden,
                                      intermediate_hidden, mma_type, activation, num_ring_tokens):
    """csrc/apis/mega.hpp:50: (nbytes, slice_fn); slice_fn(buffer) -> (x, x_sf, topk_idx,
    topk_weights, l1_acts, l1_acts_sf, l2_acts, l2_acts_sf)."""
    assert activation == "swiglu"
    if mma_type != "fp8xmxfp4":
        raise ValueError(f"mma_type {mma_type!r}: this layout serves 'fp8xmxfp4'")
    n, _ = get_symm_buffer_size_for_fused_mega_moe(num_ranks, num_experts, num_max_tokens_per_rank, num_topk,
                                                   hidden, intermediate_hidden)

    def slice_fn(buffer):
        b = _wrap(buffer, num_ranks, num_experts, num_max_tokens_per_rank, num_topk, hidden, intermediate_hidden)
        return _views(b, False)
    return n, slice_fn


def mxfp4_mega_moe(y, l1_weights, l2_weights, cumulative_local_expert_recv_stats, l1_global_scales,
                   l2_global_scales, router_input, router_weight, router_logits, router_renormalize,
                   tp_combine_output, hidden_input, sym_buffer, sym_buffer_ptrs, rank_idx, num_max_tokens_per_rank,
                   num_experts, num_topk, attn_tp_size, recipe, activation, activation_clamp, fast_math,
                   num_ring_tokens):
    """csrc/apis/mega.hpp:378: the split layer; MXFP4 weights (values, scales) or QoQ weights
    (values, meta, s1) pick the layer, as ``deep_gemm.mxfp4_mega_moe`` does."""
    kind = mega._weights_kind(l1_weights)
    b = _lookup(sym_buffer, rank_idx, "fp8f128")
    assert b.num_max_tokens_per_rank == num_max_tokens_per_rank and b.num_experts == num_experts
    assert b.num_topk == num_topk and len(sym_buffer_ptrs) == b.ep_size
    act = "qoq" if kind == "qoq" else "fp8f128"
    mega._split_entry(("fp8f128", "qoq"), y, l1_weights, l2_weights, b, cumulative_local_expert_recv_stats,
                      l1_global_scales, l2_global_scales, recipe, activation, activation_clamp, fast_math,
                      attn_tp_size, None, False, router_input, router_weight, router_logits, router_renormalize,
                      tp_combine_output, hidden_input, act=act)


int4_mega_moe = mxfp4_mega_moe


# ----------------------------------------------------------------------------- frontend
def fable_frontend_router_ctas(m, h, e, topk):
    """csrc/apis/mega.hpp:774."""
    return mega.fable_frontend_router_ctas(m, e, h, topk)


def fable_frontend_path(m, h, e, topk):
    """csrc/apis/mega.hpp:778."""
    return mega.fable_frontend_path(m, h, e, topk)


def fable_router_quant_topk_frontend(hidden, router_weight, x, x_sf, topk_idx, topk_weights, workspace, mode, stamps,
                                     l2_persist, wlayout, select_in_mega, zero_row_unrouted):
    """csrc/apis/mega.hpp:744: router + top-k + activation cast into the views of a sliced buffer
    (``x`` must be that buffer's x view); mode 0 = E4M3 with fp32 scales per 128, 1 = QoQ int8.
    With select_in_mega the keys stay in the buffer (its ``fe_keys`` view) for the layer call;
    with ``stamps`` the frontend workgroups' phase stamps (``fable_frontend_stamps``) are also
    copied where the reference's wrapper reads them (``workspace`` byte 256 + 1024 E, at most 256
    rows); ``l2_persist`` is not used here."""
    assert mode in (0, 1)
    act = "qoq" if mode == 1 else "fp8f128"
    cands = [b for (p, r, a), (_, b) in _BUFFERS.items() if p == x.data_ptr() and a == act] or \
            [b for (p, r, a), (_, b) in _BUFFERS.items() if p == x.data_ptr()]
    if not cands:
        raise RuntimeError("x must be the x view of a sliced MegaMoE buffer")
    b = cands[0] if cands[0].act_format == act else _lookup(cands[0].buffer, cands[0].ep_rank, act)
    assert topk_idx.data_ptr() == b.topk_idx.data_ptr() and topk_weights.data_ptr() == b.topk_weights.data_ptr()
    mega.fable_router_quant_topk_frontend(hidden, router_weight, b, wlayout=int(wlayout),
                                          select_in_mega=bool(select_in_mega),
                                          zero_row_unrouted=bool(zero_row_unrouted), stamps=int(bool(stamps)))
    if stamps and workspace is not None:
        e = router_weight.size(0)
        off = 256 + 4 * 64 * e * 4          # deep_gemm/mega/__init__.py:754
        st = mega.fable_frontend_stamps(b)[:_FRONTEND_STAMP_ROWS]
        if workspace.nbytes >= off + _FRONTEND_STAMP_ROWS * 64:
            region = workspace.view(torch.uint8)[off:off + _FRONTEND_STAMP_ROWS * 64].view(torch.int64).view(-1, 8)
            region.zero_()
            region[:st.size(0)].copy_(st)
    if select_in_mega:
        # the key array also where the reference's wrapper reads it (deep_gemm/mega/__init__.py:594,
        # workspace + 256 + 64 KB; fable_frontend_keys) and hands it back as fe_keys
        m, e = hidden.size(0), router_weight.size(0)
        off = _FRONTEND_CC_KEYS_OFF
        if workspace is not None and workspace.nbytes >= off + 4 * m * e:
            workspace.view(torch.uint8)[off:off + 4 * m * e].view(torch.int32).copy_(b.fe_keys[:m].reshape(-1))


_FRONTEND_CC_KEYS_OFF = 256 + 64 * 1024
_FRONTEND_STAMP_ROWS = 256          # deep_gemm/mega/__init__.py:590 (_FRONTEND_STAMPS_BYTES = 256 x 8 x 8)
