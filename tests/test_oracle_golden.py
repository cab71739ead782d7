"""The oracle against the golden vectors written by tests/golden/make_golden.py from the
reference's own packer functions (bit-exact)."""
import os

import numpy as np
import pytest

from oracle import numerics as nu
from oracle import packers as pk


def load(golden_dir, name):
    return dict(np.load(os.path.join(golden_dir, name + ".npz")))


def test_mxfp4_fused_packer(golden_dir):
    g = load(golden_dir, "mxfp4_fused")
    p, s = pk.quantize_to_mxfp4_fused(g["w"])
    np.testing.assert_array_equal(p, g["packed"])
    np.testing.assert_array_equal(s, g["scale"])


def test_mxfp4_split_packer(golden_dir):
    g = load(golden_dir, "mxfp4_split")
    p, s = pk.quantize_to_mxfp4_split(g["w"])
    np.testing.assert_array_equal(p, g["packed"])
    np.testing.assert_array_equal(s, g["scale"])


def test_nvfp4_packer(golden_dir):
    g = load(golden_dir, "nvfp4")
    p, s = pk.quantize_to_nvfp4(g["w"])
    np.testing.assert_array_equal(s, g["scale"])
    np.testing.assert_array_equal(p, g["packed"])


def test_ue4m3_ceil(golden_dir):
    g = load(golden_dir, "ue4m3_ceil")
    np.testing.assert_array_equal(nu.fp32_to_ue4m3_ceil(g["x"]), g["code"])


def test_qoq_packer(golden_dir):
    g = load(golden_dir, "qoq")
    p, s2, z, s1 = pk.quantize_to_qoq(g["w"])
    np.testing.assert_array_equal(s1, g["s1"])
    np.testing.assert_array_equal(s2, g["s2"])
    np.testing.assert_array_equal(z, g["z"])
    np.testing.assert_array_equal(p, g["packed"])


def test_qoq_int4_packer(golden_dir):
    """The split path's packer (int32 coefficient plane) and its dequantisation; its codes, s2,
    z and s1 equal quantize_to_qoq's on the same weights (s2 never exceeds 15: |w8| <= 112)."""
    g = load(golden_dir, "qoq_int4")
    p, plane = pk.quantize_to_qoq_int4(g["w"])
    np.testing.assert_array_equal(p, g["packed"])
    np.testing.assert_array_equal(plane, g["plane"])
    np.testing.assert_array_equal(pk.dequantize_qoq_int4(g["packed"], g["plane"]), g["deq"])
    f = load(golden_dir, "qoq")
    fp, s2, z, s1 = pk.qoq_int4_to_fused(g["packed"], g["plane"])
    np.testing.assert_array_equal(fp, f["packed"])
    np.testing.assert_array_equal(s2, f["s2"])
    np.testing.assert_array_equal(z, f["z"])
    np.testing.assert_array_equal(s1.view(np.uint32), f["s1"].view(np.uint32))


def test_int8_act(golden_dir):
    g = load(golden_dir, "int8_act")
    q, sf = pk.per_token_cast_to_int8(g["x"])
    np.testing.assert_array_equal(q, g["q"])
    np.testing.assert_array_equal(sf, g["sf"][:, 0])


def test_fp4_act(golden_dir):
    g = load(golden_dir, "fp4_act")
    p, sf = pk.per_token_cast_to_fp4(g["x"])
    np.testing.assert_array_equal(p, g["packed"])
    np.testing.assert_array_equal(sf, g["sf"])


def test_fp8_act(golden_dir):
    g = load(golden_dir, "fp8_act_ue8m0")
    q, sf = pk.per_token_cast_to_fp8_ue8m0(g["x"])
    np.testing.assert_array_equal(sf, g["sf"])
    np.testing.assert_array_equal(q, g["q"])
    g = load(golden_dir, "fp8_act_f32")
    q, sf = pk.per_token_cast_to_fp8_f32sf(g["x"])
    np.testing.assert_array_equal(sf, g["sf"])
    np.testing.assert_array_equal(q, g["q"])


def test_e2m1_and_ue8m0(golden_dir):
    g = load(golden_dir, "e2m1")
    np.testing.assert_array_equal(nu.e2m1_code_ties_down(g["x"]), g["code"])
    g = load(golden_dir, "ue8m0")
    np.testing.assert_array_equal(nu.ceil_to_ue8m0(g["x"]), g["y"])
