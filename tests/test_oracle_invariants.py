"""Checks that pin the oracle beyond the golden vectors: library diff tests (torch casts),
brute force over small domains, closed forms, and layer invariants. Each check is chosen so
a plausible transcription slip (a dropped term, wrong tie rule, swapped operand) fails."""
import numpy as np
import pytest
import torch

from oracle import numerics as nu
from oracle import packers as pk
from oracle import moe


def test_bf16_exhaustive_vs_torch():
    bits = np.arange(1 << 16, dtype=np.uint32)
    f = (bits << 16).view(np.float32)
    ok = ~np.isnan(f)
    np.testing.assert_array_equal(nu.f32_to_bf16_bits(f[ok]), bits[ok].astype(np.uint16))
    rng = np.random.default_rng(0)
    x = rng.standard_normal(1 << 20).astype(np.float32) * np.float32(3.0)
    # include exact ties (low 16 bits == 0x8000)
    t = (rng.integers(0, 1 << 15, 4096, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, t[~np.isnan(t)]])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(nu.f32_to_bf16_bits(x), ref)


def test_e4m3_vs_torch():
    codes = np.arange(256, dtype=np.uint8)
    vals = nu.e4m3_decode(codes)
    tv = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(np.isnan(vals), np.isnan(tv))
    ok = ~np.isnan(tv)
    np.testing.assert_array_equal(vals[ok], tv[ok])
    rng = np.random.default_rng(1)
    x = np.concatenate([
        (rng.standard_normal(1 << 20) * 50).astype(np.float32),
        (rng.standard_normal(1 << 16) * 2.0 ** -8).astype(np.float32),
        # midpoints between adjacent codes (ties)
        ((tv[1:0x7E] + tv[2:0x7F]) / 2).astype(np.float32),
        -((tv[1:0x7E] + tv[2:0x7F]) / 2).astype(np.float32),
        np.array([0.0, -0.0, 448.0, 464.0, 470.0, 479.0, -464.0], np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(nu.e4m3_encode(x), ref)


def _nearest_fp4_code(v, ties_up_magnitude=False):
    """Textbook nearest search over the 8 magnitudes; ties to the smaller magnitude."""
    mag = np.abs(v)[:, None]
    d = np.abs(mag - nu.FP4_VALUES[None, :])
    return np.argmin(d, axis=1).astype(np.uint8)      # argmin picks the first (smaller) on ties


def test_e2m1_rules_bruteforce():
    bits = np.arange(1 << 16, dtype=np.uint32)
    x = (bits << 16).view(np.float32)
    x = x[np.isfinite(x) & (np.abs(x) <= 6.0)]
    mag = _nearest_fp4_code(x)
    c1 = nu.e2m1_code_ties_down(x)
    np.testing.assert_array_equal(c1 & 7, mag)
    np.testing.assert_array_equal(c1 >> 3, ((x < 0) & (mag != 0)).astype(np.uint8))
    c2 = nu.e2m1_nibble_bucketize(x)
    np.testing.assert_array_equal(c2 & 7, mag)
    np.testing.assert_array_equal(c2 >> 3, (x < 0).astype(np.uint8))
    # reference KAT: nibble -> value, -0 nibble decodes to -0.0
    vals = nu.e2m1_decode(np.arange(16))
    assert list(vals[:8]) == [0, .5, 1, 1.5, 2, 3, 4, 6]
    assert np.signbit(vals[8]) and vals[8] == 0


def test_ceil_to_ue8m0_closed_form():
    rng = np.random.default_rng(2)
    x = np.abs(rng.standard_normal(100000).astype(np.float32)) * np.float32(2.0) ** \
        rng.integers(-60, 60, 100000).astype(np.float32)
    y = nu.ceil_to_ue8m0(x)
    # smallest power of two >= x
    assert (y >= x).all()
    assert ((y / 2) < x).all()
    assert (nu.ceil_to_ue8m0(np.float32(0.0)) == np.float32(2.0 ** -126))


def test_ceil_log2_vs_torch():
    xs = []
    for e in range(-40, 40):
        p = np.float32(2.0 ** e)
        v = p
        for _ in range(64):
            v = np.nextafter(v, np.float32(np.inf), dtype=np.float32)
            xs.append(v)
        xs.append(p)
        xs.append(np.nextafter(p, np.float32(0), dtype=np.float32))
    x = np.array(xs, dtype=np.float32)
    ref = torch.ceil(torch.log2(torch.from_numpy(x))).numpy()
    np.testing.assert_array_equal(nu.ceil_log2_f32(x), ref)


def test_marlin_roundtrip_and_order():
    rng = np.random.default_rng(3)
    nib = rng.integers(0, 16, (3, 64), dtype=np.uint8)
    p = pk.pack_marlin(nib)
    np.testing.assert_array_equal(pk.unpack_marlin(p), nib)
    # byte b of each 4-byte chunk: high nibble K[b], low nibble K[b+4]
    assert p[0, 0] == (nib[0, 0] << 4 | nib[0, 4])
    assert p[0, 3] == (nib[0, 3] << 4 | nib[0, 7])
    q = pk.pack_low_first(nib)
    assert q[0, 0] == (nib[0, 0] | nib[0, 1] << 4)
    np.testing.assert_array_equal(pk.unpack_low_first(q), nib)


def test_mxfp4_dequant_bound():
    rng = np.random.default_rng(4)
    w = nu.round_bf16(rng.standard_normal((4, 8, 256)).astype(np.float32) * np.float32(0.02))
    p, s = pk.quantize_to_mxfp4_fused(w)
    d = pk.dequantize_mxfp4_marlin(p, s)
    scale = nu.e8m0_to_f32(s)
    # nearest-E2M1 rounding: error <= half the largest step (1.0) times the group scale
    err = np.abs(d - w).reshape(4, 8, 8, 32).max(-1)
    assert (err <= scale * 1.0 + 1e-12).all()


def test_router_order_within_one_ulp_of_torch():
    rng = np.random.default_rng(5)
    x = nu.round_bf16(rng.standard_normal((8, 3072)).astype(np.float32))
    w = nu.round_bf16(rng.standard_normal((48, 3072)).astype(np.float32) * np.float32(0.02))
    a = nu.f32_to_bf16_bits(moe.router_logits_f32(x, w)).astype(np.int32)
    tl = (torch.from_numpy(x) @ torch.from_numpy(w).T).to(torch.bfloat16).view(torch.int16).numpy()
    b = tl.astype(np.int32) & 0xFFFF
    sa = np.where(a & 0x8000, -(a & 0x7FFF), a)
    sb = np.where(b & 0x8000, -(b & 0x7FFF), b)
    assert np.abs(sa - sb).max() <= 1
    # fp64 exact sum within fp32 rounding of the deterministic order
    ex = (x.astype(np.float64) @ w.astype(np.float64).T)
    assert np.abs(moe.router_logits_f32(x, w) - ex).max() < 1e-4


def test_topk_tie_rule_and_softmax():
    # equal logits: slots follow ascending expert index; softmax exactly 1/k
    lg = np.zeros((1, 16), np.float32)
    lg[0, [3, 9, 1, 12]] = 1.0
    idx, w, _ = moe.topk_softmax(lg, 4)
    assert idx.tolist() == [[1, 3, 9, 12]]
    assert (w == np.float32(0.25)).all()
    # -0 and +0 tie -> index order
    lg = np.array([[-0.0, 0.0, -1.0]], np.float32)
    idx, _, _ = moe.topk_softmax(lg, 2)
    assert idx.tolist() == [[0, 1]]
    # brute force against a stable argsort on values for random bf16 logits
    rng = np.random.default_rng(6)
    lg = nu.round_bf16(rng.standard_normal((32, 48)).astype(np.float32))
    lg[:, 5] = lg[:, 6]
    idx, w, lb = moe.topk_softmax(lg, 8)
    ref = np.argsort(-lb.astype(np.float64), axis=1, kind="stable")[:, :8]
    np.testing.assert_array_equal(idx, ref)
    tw = torch.softmax(torch.from_numpy(np.take_along_axis(lb, ref, 1)), dim=-1).numpy()
    np.testing.assert_allclose(w, tw, rtol=2e-6, atol=0)


def test_balanced_routing_properties():
    idx, w = moe.balanced_routing(16, 384, 8)
    assert (w == np.float32(0.125)).all()
    # slot s lands in group s; 16 tokens -> 128 distinct experts, one route each
    assert ((idx // 48) == np.arange(8)[None, :]).all()
    assert len(np.unique(idx)) == 128
    counts, active, off, routes = moe.dispatch(idx, 0, 48)
    assert counts.sum() == 16 and len(active) == 16


def test_dispatch_order_and_counts():
    rng = np.random.default_rng(7)
    idx = np.stack([rng.permutation(20)[:4] for _ in range(9)])
    idx[2, 1] = -1
    counts, active, off, routes = moe.dispatch(idx, 4, 12)
    ref = np.bincount(idx[(idx >= 4) & (idx < 16)] - 4, minlength=12)
    np.testing.assert_array_equal(counts, ref)
    for a, e in enumerate(active):
        r = routes[off[a]:off[a + 1]]
        assert (np.diff(r) > 0).all()
        assert all(idx[x // 4, x % 4] == e + 4 for x in r)


def _small_layer(act_format, seed=8, M=4, H=512, I=256, E=16, topk=4):
    rng = np.random.default_rng(seed)
    x = nu.round_bf16(rng.standard_normal((M, H)).astype(np.float32))
    rw = nu.round_bf16(rng.standard_normal((E, H)).astype(np.float32) * np.float32(0.05))
    w1 = nu.round_bf16(rng.standard_normal((E, 2 * I, H)).astype(np.float32) * np.float32(0.05))
    w2 = nu.round_bf16(rng.standard_normal((E, H, I)).astype(np.float32) * np.float32(0.05))
    W1 = pk.dequantize_mxfp4_marlin(*pk.quantize_to_mxfp4_fused(w1))
    W2 = pk.dequantize_mxfp4_marlin(*pk.quantize_to_mxfp4_fused(w2))
    return x, rw, W1, W2


@pytest.mark.parametrize("fmt", ["mxfp4", "mxfp8"])
def test_layer_invariants(fmt):
    x, rw, W1, W2 = _small_layer(fmt)
    x[1] = 0.0
    r = moe.layer_forward(x, rw, W1, W2, 0, fmt, topk=4)
    assert (r["y"][1] == 0).all()                      # zero row -> exactly zero output
    # the layer is the sum of its routes
    y2 = np.zeros_like(r["y"])
    for rid, v in r["routes"].items():
        y2[rid // 4] += v
    np.testing.assert_allclose(r["y"], y2, rtol=0, atol=1e-6)
    # expert-parallel split: the layer = sum of the shares of disjoint local ranges
    a = moe.moe_forward(r["x_dq"], r["topk_idx"], r["topk_w"], W1[:8], W2[:8], 0, fmt)[0]
    b = moe.moe_forward(r["x_dq"], r["topk_idx"], r["topk_w"], W1[8:], W2[8:], 8, fmt)[0]
    np.testing.assert_allclose(a + b, r["y"], rtol=1e-5, atol=1e-5)


def test_layer_against_float64_bruteforce():
    """Route by route in float64 with the same quantisation decisions; catches a
    transposed weight, a swapped gate/up half or a missing routing weight."""
    x, rw, W1, W2 = _small_layer("mxfp4", seed=9)
    r = moe.layer_forward(x, rw, W1, W2, 0, "mxfp4", topk=4)
    I = W1.shape[1] // 2
    for rid, v in r["routes"].items():
        t, s = divmod(rid, 4)
        e = r["topk_idx"][t, s]
        h = W1[e].astype(np.float64) @ r["x_dq"][t].astype(np.float64)
        g = np.minimum(nu.round_bf16(h[:I].astype(np.float32)), 10.0).astype(np.float64)
        u = np.clip(nu.round_bf16(h[I:].astype(np.float32)), -10.0, 10.0).astype(np.float64)
        a = g / (1 + np.exp(-g)) * u * r["topk_w"][t, s]
        mid = moe.requant_mid(a.astype(np.float32)[None], "mxfp4")[0].astype(np.float64)
        o = W2[e].astype(np.float64) @ mid
        rel = np.linalg.norm(o - v) / np.linalg.norm(o)
        assert rel < 2e-2, rel     # requant boundary flips only
