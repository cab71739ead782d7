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
