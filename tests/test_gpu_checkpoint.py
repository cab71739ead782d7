"""GPU parity of checkpoint ingestion (bit-exact): the nibble-order kernel, the inverse tile
transforms and the W1 row modes against the oracle (oracle/packers.py, checkpoint formats), and
checkpoint -> fused weights -> checkpoint round trips."""
import numpy as np
import pytest
import torch

from oracle import packers as pk
from tests.gpu_common import need_gpu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_bytes", [4, 64, 4 * 1001, 1 << 20])
def test_reorder_fp4_nibbles(n_bytes):
    need_gpu()
    from hopper_megamoe_basedondeepgemm_amd import checkpoint as ck
    print(f"reorder n_bytes={n_bytes}", flush=True)
    rng = np.random.default_rng(n_bytes)
    src = rng.integers(0, 256, n_bytes, dtype=np.uint8)
    t = torch.from_numpy(src).cuda()
    np.testing.assert_array_equal(ck.marlin_to_ocp(t).cpu().numpy(), pk.marlin_to_low_first(src[None])[0])
    np.testing.assert_array_equal(ck.ocp_to_marlin(t).cpu().numpy(), pk.low_first_to_marlin(src[None])[0])
    # in place, there and back
    ck.ocp_to_marlin(t, out=t)
    ck.marlin_to_ocp(t, out=t)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(t.cpu().numpy(), src)


def test_reorder_rejects_partial_words():
    """Rows of partial words: refused by the Python helper (a word would straddle two rows) and,
    for a byte count that is not whole words, by the C ABI itself."""
    need_gpu()
    from hopper_megamoe_basedondeepgemm_amd import checkpoint as ck, _lib
    t = torch.zeros(6, dtype=torch.uint8, device="cuda")
    with pytest.raises(AssertionError, match="4-byte words"):
        ck.ocp_to_marlin(t)
    with pytest.raises(AssertionError, match="4-byte words"):
        ck.ocp_to_marlin(torch.zeros((2, 6), dtype=torch.uint8, device="cuda"))
    with pytest.raises(RuntimeError, match="n_bytes % 4"):
        _lib.check(_lib.load().dgm_reorder_fp4_nibbles(_lib.ptr(t), _lib.ptr(t), 6, 1, 0, _lib.stream()))


def _weights(seed, E, I, H, nvfp4):
    rng = np.random.default_rng(seed)
    w1 = (rng.standard_normal((E, 2 * I, H)) * 0.05).astype(np.float32)
    w2 = (rng.standard_normal((E, H, I)) * 0.05).astype(np.float32)
    q = pk.quantize_to_nvfp4 if nvfp4 else pk.quantize_to_mxfp4_split
    return q(w1), q(w2)


def _cuda(*a):
    return tuple(torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in a)


@pytest.mark.parametrize("fmt", ["mxfp4", "nvfp4"])
@pytest.mark.parametrize("order", ["marlin", "ocp"])
@pytest.mark.parametrize("gate_up", ["concat", "interleaved"])
def test_checkpoint_transform_and_inverse(fmt, order, gate_up):
    """checkpoint -> fused layout == the oracle's tile layout; fused -> checkpoint == the input;
    an OCP / interleaved checkpoint gives the same fused bytes as the reference's Marlin /
    concatenated packing of the same weights."""
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import checkpoint as ck
    print(f"checkpoint fmt={fmt} order={order} gate_up={gate_up}", flush=True)
    nv = fmt == "nvfp4"
    E, I, H = 2, 128, 640 if not nv else 256         # MXFP4 H = 640: a partial last scale group
    (p1, s1), (p2, s2) = _weights(11, E, I, H, nv)
    mode = {"concat": 1, "interleaved": 2}[gate_up]
    c1 = p1 if order == "marlin" else pk.marlin_to_low_first(p1)
    c2 = p2 if order == "marlin" else pk.marlin_to_low_first(p2)
    d1, e1 = c1, s1
    if gate_up == "interleaved":
        rows = np.stack([np.arange(I), I + np.arange(I)], 1).reshape(-1)
        d1, e1 = c1[:, rows], s1[:, rows]
    to_tile = pk.nvfp4_to_tile if nv else pk.fp4_to_tile
    conv = ck.nvfp4_checkpoint_to_mega_moe if nv else ck.mxfp4_checkpoint_to_mega_moe
    back = ck.mega_moe_to_nvfp4_checkpoint if nv else ck.mega_moe_to_mxfp4_checkpoint
    w1, w2 = conv(_cuda(d1, e1), _cuda(c2, s2), order=order, gate_up_rows=gate_up)
    torch.cuda.synchronize()
    for got, (pp, ss, m) in ((w1, (d1, e1, mode)), (w2, (c2, s2, 0))):
        want_v, want_s = to_tile(pp, ss, order, m)
        np.testing.assert_array_equal(got[0].cpu().numpy(), want_v)
        np.testing.assert_array_equal(got[1].cpu().numpy(), want_s)
    (b1, bs1), (b2, bs2) = back(w1, w2, order=order, gate_up_rows=gate_up)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(b1.cpu().numpy(), d1)
    np.testing.assert_array_equal(bs1.cpu().numpy(), e1)
    np.testing.assert_array_equal(b2.cpu().numpy(), c2)
    np.testing.assert_array_equal(bs2.cpu().numpy(), s2)
    # the reference's own form of the same weights lands on the same fused bytes
    ref = (dgm.transform_nvfp4_weights_for_mega_moe_fused if nv else dgm.transform_mxfp4_weights_for_mega_moe_fused)(
        _cuda(p1, s1), _cuda(p2, s2))
    torch.cuda.synchronize()
    for a, b in zip(ref, (w1, w2)):
        np.testing.assert_array_equal(a[0].cpu().numpy(), b[0].cpu().numpy())
        np.testing.assert_array_equal(a[1].cpu().numpy(), b[1].cpu().numpy())


def test_checkpoint_rejects_short_k():
    need_gpu()
    from hopper_megamoe_basedondeepgemm_amd import checkpoint as ck
    (p1, s1), (p2, s2) = _weights(13, 1, 64, 256, False)      # W2 K = I = 64 < one K-tile
    with pytest.raises(ValueError, match="of 128"):
        ck.mxfp4_checkpoint_to_mega_moe(_cuda(p1, s1), _cuda(p2, s2), order="marlin")


def test_checkpoint_blocks_shape():
    """[E, N, K/32, 16] blocks (the usual MXFP4 checkpoint tensor shape) are accepted."""
    need_gpu()
    from hopper_megamoe_basedondeepgemm_amd import checkpoint as ck
    (p1, s1), (p2, s2) = _weights(12, 1, 128, 256, False)
    o1, o2 = pk.marlin_to_low_first(p1), pk.marlin_to_low_first(p2)
    a = ck.mxfp4_checkpoint_to_mega_moe(_cuda(o1, s1), _cuda(o2, s2))
    b = ck.mxfp4_checkpoint_to_mega_moe(_cuda(o1.reshape(1, 256, 8, 16), s1), _cuda(o2.reshape(1, 256, 4, 16), s2))
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x[0].cpu().numpy(), y[0].cpu().numpy())
        np.testing.assert_array_equal(x[1].cpu().numpy(), y[1].cpu().numpy())
