"""Pins of the oracle's checkpoint-format functions (oracle/packers.py, "checkpoint formats"):
the two nibble orders against hand-worked bytes and the reference's own packed codes, the tile
layouts against the decoders the matrix-core probes pin (tests/gpu_common.py), and the round
trips through every row mode."""
import os

import numpy as np
import pytest

from oracle import numerics as nu
from oracle import packers as pk
from tests.gpu_common import decode_native, decode_native_nvfp4, interleave16


def test_nibble_orders_known_answer():
    # codes K0..K7 = 1..8: OCP byte j = K[2j] | K[2j+1] << 4; Marlin byte b = K[b] << 4 | K[b+4]
    # (deep_gemm/quantization_mxfp4.py:66-70: "byte b: low = K[b+4], high = K[b]")
    n = np.arange(1, 9, dtype=np.uint8)[None]
    ocp = pk.pack_low_first(n)
    marlin = pk.pack_marlin(n)
    np.testing.assert_array_equal(ocp[0], [0x21, 0x43, 0x65, 0x87])
    np.testing.assert_array_equal(marlin[0], [0x15, 0x26, 0x37, 0x48])
    np.testing.assert_array_equal(pk.marlin_to_low_first(marlin), ocp)
    np.testing.assert_array_equal(pk.low_first_to_marlin(ocp), marlin)


def test_ocp_order_against_reference_codes(golden_dir):
    """The reference's own low-nibble-first codes (per_token_cast_to_fp4,
    deep_gemm/utils/math.py:99-100, golden fp4_act) decode, low nibble = even K, to within one
    E2M1 step of x: a swapped nibble order would not."""
    g = dict(np.load(os.path.join(golden_dir, "fp4_act.npz")))
    x, packed, sf = g["x"], g["packed"], g["sf"]
    v = nu.e2m1_decode(pk.unpack_low_first(packed)) * np.repeat(sf, 32, axis=1)
    assert np.all(np.abs(v - x) <= np.repeat(sf, 32, axis=1) * 1.0 + 1e-6)
    swapped = nu.e2m1_decode(pk.unpack_marlin(packed)) * np.repeat(sf, 32, axis=1)
    assert np.abs(swapped - x).max() > 1.0
    # Marlin codes of the same elements convert back and forth losslessly
    m = pk.low_first_to_marlin(packed)
    np.testing.assert_array_equal(pk.unpack_marlin(m), pk.unpack_low_first(packed))
    np.testing.assert_array_equal(pk.marlin_to_low_first(m), packed)


def _mxfp4_case(seed, E=2, N=64, K=640):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((E, N, K)) * 0.05).astype(np.float32)
    return pk.quantize_to_mxfp4_split(w)


@pytest.mark.parametrize("l1_mode", [0, 1, 2])
def test_fp4_tile_layout_decodes_to_reference_rows(l1_mode):
    """decode(tile(q)) == the reference dequant in native row order (interleave16 for W1):
    the tile layout the matrix-core probes pin, for each W1 row mode."""
    packed, scale = _mxfp4_case(3)
    deq = pk.dequantize_mxfp4_marlin(packed, scale)
    if l1_mode == 2:
        # a checkpoint whose W1 interleaves gate / up rows: row 2i = gate i, 2i+1 = up i
        I = packed.shape[1] // 2
        order = np.stack([np.arange(I), I + np.arange(I)], 1).reshape(-1)
        packed, scale = packed[:, order], scale[:, order]
    vals, sc = pk.fp4_to_tile(packed, scale, "marlin", l1_mode)
    want = deq if l1_mode == 0 else interleave16(deq)
    np.testing.assert_array_equal(decode_native(vals, sc), want)
    # K = 640: 5 K-tiles, the last scale group's padding bytes are 2^0
    assert (sc[:, :, -1, :, 1:] == 127).all()


@pytest.mark.parametrize("order", ["marlin", "ocp"])
@pytest.mark.parametrize("l1_mode", [0, 1, 2])
def test_fp4_tile_round_trips(order, l1_mode):
    packed, scale = _mxfp4_case(4)
    src = packed if order == "marlin" else pk.marlin_to_low_first(packed)
    vals, sc = pk.fp4_to_tile(src, scale, order, l1_mode)
    back, bsc = pk.fp4_from_tile(vals, sc, order, l1_mode)
    np.testing.assert_array_equal(back, src)
    np.testing.assert_array_equal(bsc, scale)
    # and tile -> checkpoint -> tile on arbitrary tile bytes (padding scale bytes fixed at 2^0)
    rng = np.random.default_rng(5)
    tv = rng.integers(0, 256, vals.shape, dtype=np.uint8)
    ts = rng.integers(0, 256, sc.shape, dtype=np.uint8)
    ts[:, :, -1, :, 1:] = 127
    p2, s2 = pk.fp4_from_tile(tv, ts, order, l1_mode)
    v3, s3 = pk.fp4_to_tile(p2, s2, order, l1_mode)
    np.testing.assert_array_equal(v3, tv)
    np.testing.assert_array_equal(s3, ts)


def _nvfp4_case(seed, E=2, N=64, K=256):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((E, N, K)) * 0.05).astype(np.float32)
    return pk.quantize_to_nvfp4(w)


@pytest.mark.parametrize("l1_mode", [0, 1, 2])
def test_nvfp4_tile_layout_decodes_to_reference_rows(l1_mode):
    packed, scale = _nvfp4_case(6)
    deq = pk.dequantize_nvfp4(packed, scale)
    if l1_mode == 2:
        I = packed.shape[1] // 2
        order = np.stack([np.arange(I), I + np.arange(I)], 1).reshape(-1)
        packed, scale = packed[:, order], scale[:, order]
    vals, sc = pk.nvfp4_to_tile(packed, scale, "marlin", l1_mode)
    want = deq if l1_mode == 0 else interleave16(deq)
    np.testing.assert_array_equal(decode_native_nvfp4(vals, sc), want)


@pytest.mark.parametrize("order", ["marlin", "ocp"])
@pytest.mark.parametrize("l1_mode", [0, 1, 2])
def test_nvfp4_tile_round_trips(order, l1_mode):
    packed, scale = _nvfp4_case(7)
    src = packed if order == "marlin" else pk.marlin_to_low_first(packed)
    vals, sc = pk.nvfp4_to_tile(src, scale, order, l1_mode)
    back, bsc = pk.nvfp4_from_tile(vals, sc, order, l1_mode)
    np.testing.assert_array_equal(back, src)
    np.testing.assert_array_equal(bsc, scale)
    rng = np.random.default_rng(8)
    tv = rng.integers(0, 256, vals.shape, dtype=np.uint8)
    ts = rng.integers(0, 256, sc.shape, dtype=np.uint8)
    v3, s3 = pk.nvfp4_to_tile(*pk.nvfp4_from_tile(tv, ts, order, l1_mode), order, l1_mode)
    np.testing.assert_array_equal(v3, tv)
    np.testing.assert_array_equal(s3, ts)


def test_native_rows_are_permutations():
    for mode in (0, 1, 2):
        r = pk.native_src_rows(128, mode)
        assert sorted(r.tolist()) == list(range(128))
    # mode 1 and mode 2 put the same (gate, up) features side by side
    r1, r2 = pk.native_src_rows(64, 1), pk.native_src_rows(64, 2)
    gate1 = r1[(np.arange(64) // 16) % 2 == 0]
    gate2 = r2[(np.arange(64) // 16) % 2 == 0]
    np.testing.assert_array_equal(gate1, np.arange(32))
    np.testing.assert_array_equal(gate2, 2 * np.arange(32))
