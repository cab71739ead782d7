"""Shared helpers for the GPU parity tests: seeded inputs, native-layout decoding, metrics."""
import numpy as np
import pytest
import torch

from oracle import numerics as nu
from oracle import packers as pk


def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import hopper_megamoe_basedondeepgemm_amd as dgm  # noqa: F401  (loads the HIP library)
    from hopper_megamoe_basedondeepgemm_amd import _lib
    _lib.load()


def bf16_cpu(a):
    """numpy f32 -> torch bf16 CPU tensor (values must already be bf16-representable)."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)


def randn_bf16(rng, shape, scale=1.0):
    return nu.round_bf16(rng.standard_normal(shape).astype(np.float32) * np.float32(scale))


def decode_native(vals, scales):
    """Native fragment-order weights -> f32 [E, N, K] in native row order.
    vals [E, NB, KT, 64, 16] u8, scales [E, NB, KG, 64, 4] u8."""
    vals = np.asarray(vals)
    scales = np.asarray(scales)
    E, NB, KT, L, B = vals.shape
    lo = vals & 0xF
    hi = vals >> 4
    nib = np.stack([lo, hi], axis=-1).reshape(E, NB, KT, 64, 32)          # k-within-lane 0..31
    v = nu.e2m1_decode(nib)
    sc = np.zeros((E, NB, KT, 64), dtype=np.uint8)
    for kt in range(KT):
        sc[:, :, kt, :] = scales[:, :, kt // 4, :, kt % 4]
    v = v * nu.e8m0_to_f32(sc)[..., None]
    # lane l -> row l % 16, k = 128 kt + 32 (l // 16) + j
    v = v.reshape(E, NB, KT, 4, 16, 32).transpose(0, 1, 4, 2, 3, 5)      # E NB r KT kq j
    return v.reshape(E, NB * 16, KT * 128).astype(np.float32)


def interleave16(w):
    """Native L1 row order: block pair p = (gate rows 16p.., up rows I + 16p..)."""
    E, N, K = w.shape
    I = N // 2
    g = w[:, :I].reshape(E, I // 16, 16, K)
    u = w[:, I:].reshape(E, I // 16, 16, K)
    return np.stack([g, u], axis=2).reshape(E, N, K)


def layer_metrics(y, ref):
    from oracle.moe import metrics
    return metrics(y, ref)
