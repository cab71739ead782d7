"""CPU checks of the C-ABI library: it loads, exports every symbol include/*.h declares, and
its host-side argument checks reject bad shapes with a message (no GPU work is launched)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols(header):
    txt = open(os.path.join(ROOT, "include", header)).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(dgm_\w+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    """libdgm_megamoe.so exports what include/dgm_megamoe.h declares, libdgm_probe.so (the tests'
    probes) what include/dgm_probe.h declares, and every header is one of the two."""
    from hopper_megamoe_basedondeepgemm_amd import _lib
    assert sorted(os.path.basename(h) for h in glob.glob(os.path.join(ROOT, "include", "*.h"))) == \
        ["dgm_megamoe.h", "dgm_probe.h"]
    for header, lib, exports in (("dgm_megamoe.h", _lib.load(), _lib.EXPORTS),
                                 ("dgm_probe.h", _lib.load_probe(), _lib.PROBE_EXPORTS)):
        names = declared_symbols(header)
        assert len(names) >= 5
        for n in names:
            assert hasattr(lib, n), n
        assert set(names) == set(exports)
    assert not any(n.startswith("dgm_probe") for n in declared_symbols("dgm_megamoe.h"))


def test_struct_layouts_match_the_library():
    """The ctypes mirrors of DgmMoeArgs and DgmBufferLayout have the sizes the library was built
    with (a field added on one side only would shift every later field)."""
    from hopper_megamoe_basedondeepgemm_amd import _lib
    a, b = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert _lib.load().dgm_abi_struct_sizes(ctypes.byref(a), ctypes.byref(b)) == 0
    assert a.value == ctypes.sizeof(_lib.MoeArgs) and b.value == ctypes.sizeof(_lib.BufferLayout)
    assert _lib.MoeArgs.launch_flags.offset + 4 <= a.value


def test_host_checks_and_layout():
    from hopper_megamoe_basedondeepgemm_amd import _lib
    lib = _lib.load()
    st = lib.dgm_quantize_mxfp4(ctypes.c_void_p(16), 4, 33, 0, ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert st == -1 and b"multiple of 32" in lib.dgm_last_error()
    with pytest.raises(RuntimeError, match="topk"):
        _lib.layout(16, 384, 48, 17, 3072, 1280, 0)
    L = _lib.layout(16, 384, 48, 8, 3072, 1280, 1)
    offs = [L.x, L.x_sf, L.topk_idx, L.topk_weights, L.logits, L.fe_keys, L.pool, L.mid, L.mid_sf, L.partials,
            L.counters, L.total_bytes]
    assert offs == sorted(offs) and all(o % 256 == 0 for o in offs)
    assert L.x_row_bytes == 3072 and L.mid_row_bytes == 1280 and L.max_routes == 128 and L.max_tokens == 16
    assert L.fe_keys - L.logits >= 16 * 384 * 4
    assert L.partials + 128 * 3072 * 2 <= L.counters        # bf16 [topk, max_tokens, H]


def test_empty_batch_and_null_rows():
    """No tokens: the frontend entry points return 0 before any GPU work, with no row pointers
    (an empty tensor has none); with tokens, a missing row pointer is an error."""
    from hopper_megamoe_basedondeepgemm_amd import _lib
    lib = _lib.load()
    L = _lib.layout(16, 384, 384, 8, 3072, 1280, 1)
    buf = ctypes.c_void_p(256)              # (never dereferenced on these paths)
    st = lib.dgm_router_topk_launch(None, None, 0, 3072, 384, 8, 1, 0, 0, buf, ctypes.byref(L), None)
    assert st == 0
    st = lib.dgm_router_logits_topk_launch(None, 0, 384, 8, 0, 0, buf, ctypes.byref(L), None)
    assert st == 0
    st = lib.dgm_router_topk_launch(None, None, 4, 3072, 384, 8, 1, 0, 0, buf, ctypes.byref(L), None)
    assert st == -1 and b"null pointer" in lib.dgm_last_error()


def test_product_path_has_no_cpu_fallback():
    import torch
    import hopper_megamoe_basedondeepgemm_amd as dgm
    w = torch.zeros((2, 64), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        dgm.quantization_mxfp4_fused.quantize_to_mxfp4(w)


def test_launches_refuse_calls_beyond_the_buffers_shape():
    """Every launch checks the call's shape against the one its buffer was laid out for, before
    anything is enqueued: route outputs are [topk][max_tokens][H] and x rows [max_tokens, H or
    H/2], so a larger topk (even with fewer tokens, same routes), more tokens (with a smaller
    topk), another hidden / intermediate size, more experts, or an activation format with wider
    rows would write past the views."""
    from hopper_megamoe_basedondeepgemm_amd import _lib
    lib = _lib.load()
    L = _lib.layout(16, 384, 48, 8, 3072, 1280, _lib.ACT_FORMATS["mxfp4"])
    assert (L.topk, L.num_experts, L.num_local_experts, L.hidden, L.intermediate) == (8, 384, 48, 3072, 1280)
    assert L.x_row_bytes == 1536 and L.x_sf_row_bytes == 96 and L.mid_row_bytes == 640 and L.mid_sf_row_bytes == 40
    buf, p = ctypes.c_void_p(256), ctypes.c_void_p(4096)     # (never dereferenced: refused first)

    def fe(tokens, hidden, experts, topk, act):
        st = lib.dgm_router_topk_launch(p, p, tokens, hidden, experts, topk, act, 0, 0, buf, ctypes.byref(L), None)
        return st, lib.dgm_last_error()

    st, msg = fe(8, 3072, 384, 16, 0)          # 8 x 16 = 128 routes fit, but slot 8.. would overrun
    assert st == -1 and b"topk exceeds" in msg
    st, msg = fe(32, 3072, 384, 4, 0)          # 32 x 4 = 128 routes, but 32 > 16 token rows
    assert st == -1 and b"max_tokens" in msg
    st, msg = fe(8, 4096, 384, 8, 0)
    assert st == -1 and b"hidden differs" in msg
    st, msg = fe(8, 3072, 512, 8, 0)
    assert st == -1 and b"num_experts exceeds" in msg
    st, msg = fe(8, 3072, 384, 8, _lib.ACT_FORMATS["mxfp8"])    # E4M3 rows are twice as wide
    assert st == -1 and b"wider x" in msg
    st = lib.dgm_router_logits_topk_launch(p, 8, 384, 16, 0, 0, buf, ctypes.byref(L), None)
    assert st == -1 and b"topk exceeds" in lib.dgm_last_error()

    def moe(**kw):
        a = _lib.MoeArgs(num_tokens=8, hidden=3072, intermediate=1280, num_experts=384, expert_begin=0,
                         num_local_experts=48, topk=8, act_format=0, activation_clamp=10.0, fast_math=1,
                         w1_values=4096, w1_scales=4096, w2_values=4096, w2_scales=4096, y=4096, buffer=256,
                         layout=ctypes.pointer(L))
        for k, v in kw.items():
            setattr(a, k, v)
        return a

    for fn in (lib.dgm_megamoe_fused_launch, lib.dgm_megamoe_split_launch, lib.dgm_megamoe_fused_launch_noalloc):
        for kw, what in (({"topk": 16, "num_tokens": 8}, b"topk exceeds"),
                         ({"topk": 4, "num_tokens": 32}, b"max_tokens"),
                         ({"intermediate": 2048}, b"intermediate differs"),
                         ({"num_local_experts": 96, "num_experts": 384}, b"num_local_experts exceeds"),
                         ({"act_format": _lib.ACT_FORMATS["mxfp8"]}, b"wider x")):
            st = fn(ctypes.byref(moe(**kw)), None)
            assert st == -1 and what in lib.dgm_last_error(), (fn, kw, lib.dgm_last_error())
