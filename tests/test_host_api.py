"""Host-side API checks (CPU, no GPU): the buffer layouts the split recipe shares between its
two layers, the frontend's option family and workgroup count, the reference-order router weight
permutation and its inverse, and the ``_C`` module's names."""
import numpy as np
import pytest
import torch

from hopper_megamoe_basedondeepgemm_amd import _lib, mega


def _fields(L):
    return {f: getattr(L, f) for f, _ in _lib.BufferLayout._fields_}


@pytest.mark.parametrize("shape", [(8, 384, 384, 8, 3072, 1280), (16, 48, 48, 8, 512, 256), (5, 32, 16, 8, 1024, 512)])
def test_fp8f128_and_qoq_share_one_layout(shape):
    """One split buffer serves the fp8 x MXFP4 layer and the QoQ layer (int4_mega_moe): the two
    formats' layouts are identical field by field."""
    a = _lib.layout(*shape, _lib.ACT_FORMATS["fp8f128"])
    b = _lib.layout(*shape, _lib.ACT_FORMATS["qoq"])
    fa, fb = _fields(a), _fields(b)
    assert fa.pop("act_format") != fb.pop("act_format")
    assert fa == fb
    T, E, El, k, H, I = shape
    assert a.x_sf - a.x >= T * H and a.x_row_bytes == H and a.mid_row_bytes == I


def test_frontend_path_and_router_workgroups():
    assert mega.fable_frontend_path(8) == mega.FE_PATH_CC
    assert mega.fable_frontend_path(64) == mega.FE_PATH_CC
    assert mega.fable_frontend_path(65) == mega.FE_PATH_WMMA
    assert mega.fable_frontend_router_ctas(8, 384) == 96 * 2
    assert mega.fable_frontend_router_ctas(1, 48) == 12
    assert mega.fable_frontend_router_ctas(63, 384) == 96 * 16
    assert mega.fable_frontend_router_ctas(64, 384) == 96 * 8
    assert mega.fable_frontend_router_ctas(100, 48) == 12 * 13


def test_router_weight_fragment_layout_inverse():
    """wlayout='pre' takes the reference's fragment order (deep_gemm/mega/__init__.py:617-628):
    lane (g, t) of half h in block (G, b) holds W[16 G + 8 h + g][32 b + 8 t .. +7]."""
    E, K = 32, 64
    w = torch.arange(E * K, dtype=torch.float32).reshape(E, K).to(torch.bfloat16)
    f = mega.fable_router_weight_fragment_layout(w)
    flat = f.reshape(-1).float().numpy()
    G, b, h, g, t = 1, 1, 1, 3, 2          # element 0 of that lane
    pos = ((((G * (K // 32) + b) * 2 + h) * 8 + g) * 4 + t) * 8
    assert flat[pos] == float(w[16 * G + 8 * h + g, 32 * b + 8 * t])
    assert torch.equal(mega._router_weight_row_major(f, "pre"), w)
    assert mega._router_weight_row_major(w, "row") is w


def test_c_module_names():
    from hopper_megamoe_basedondeepgemm_amd import _C
    for name in ("get_symm_buffer_size_for_fused_mega_moe", "mxfp4_mega_moe_fused", "qoq_mega_moe_fused",
                 "get_symm_buffer_size_for_mega_moe", "mxfp4_mega_moe", "int4_mega_moe",
                 "fable_router_quant_topk_frontend", "fable_frontend_router_ctas", "fable_frontend_path",
                 "get_token_alignment_for_mega_moe", "get_ring_limit_for_mega_moe",
                 "get_legacy_pool_tokens_for_mega_moe"):
        assert callable(getattr(_C, name)), name
    n, slice_fn = _C.get_symm_buffer_size_for_fused_mega_moe(1, 48, 8, 8, 3072, 1280)
    assert n == _lib.layout(8, 48, 48, 8, 3072, 1280, _lib.ACT_FORMATS["fp8f128"]).total_bytes
    assert _C.get_ring_limit_for_mega_moe(8, 48, 8, 1) == (64, 64)
    with pytest.raises(ValueError):
        _C.get_symm_buffer_size_for_mega_moe(1, 48, 8, 8, 3072, 1280, "bf16xbf16", "swiglu", 64)


def test_bench_reads_its_committed_profiles():
    """bench.py's roofline.traffic and mfma_util come from the committed rocprofv3 summaries
    under profiles/: both parse to the values those files state (HBM bytes per headline launch
    within 2 % of the 401.1 MB of active-expert weights; matrix cores a few percent busy)."""
    import importlib.util
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    t = bench.profiled_traffic_bytes()
    assert t is not None and abs(t / 401.1e6 - 1) < 0.02, t
    u = bench.profiled_mfma_util()
    assert u is not None and 0 < u < 0.2, u
    assert bench.profiled_mfma_util("k_megamoe<24,10,3,0>", ("M=64", "NVFP4")) > u   # (VALU co-bound, busier)


def test_reorder_fp4_nibbles_refuses_rows_of_partial_words():
    """A Marlin word holds 8 codes of one row: a last dimension that is not whole 4-byte words
    would let a word straddle two rows, so the checkpoint helper refuses it before any launch."""
    from hopper_megamoe_basedondeepgemm_amd import checkpoint
    with pytest.raises(AssertionError, match="4-byte words"):
        checkpoint.reorder_fp4_nibbles(torch.zeros((3, 6), dtype=torch.uint8), "ocp", "marlin")


def test_route_to_token_multiply_is_exact_within_the_host_limits():
    """The fused kernel maps a route to its token as (route * ceil(2^20 / topk)) >> 20 instead of
    an integer division (dgm_fused.hip, div_small). Exact for every route below the per-call
    route limit and every top-k the host accepts (topk <= 16, checked before any launch): the
    product overshoots route / topk by less than 2^-10 < 1 / topk. Checked here for all pairs,
    with the limits read from the sources so that raising one re-runs the check at the new
    bound."""
    import os
    import re
    root = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                        "hopper_megamoe_basedondeepgemm_amd", "csrc")
    hpp = open(os.path.join(root, "dgm_fused.hpp")).read()
    max_routes = int(re.search(r"FUSED_MAX_ROUTES\s*=\s*(\d+)", hpp).group(1))
    src = open(os.path.join(root, "dgm_megamoe.hip")).read()
    assert "topk <= 16" in src
    r = np.arange(max_routes, dtype=np.uint64)
    for d in range(1, 17):
        m = (0x100000 + d - 1) // d
        assert np.array_equal((r * np.uint64(m)) >> np.uint64(20), r // np.uint64(d)), d
        assert int(r[-1]) * m < 2 ** 32          # (the kernel multiplies in 32 bits)
