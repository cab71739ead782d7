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


def decode_native_qoq(vals, meta, s1, l1=True):
    """QoQ native layout -> f32 [E, N, K] in native row order: (code - z) * s2 * s1.
    vals [E, NB, KT, 64, 16], meta [E, NB, KT, 16] (byte r = z | s2 << 4), s1 [E, N].
    l1: the paired-nibble L1 layout, else the chunk-split L2 layout (high nibble ^ 8)."""
    vals = np.asarray(vals).astype(np.int64)
    meta = np.asarray(meta).astype(np.int64)
    E, NB, KT, L, B = vals.shape
    d = vals.reshape(E, NB, KT, 64, 4, 4)                    # dword q of the lane, byte b
    lo, hi = d & 0xF, d >> 4
    code = np.zeros((E, NB, KT, 64, 2, 16), np.int64)
    if l1:
        # op h: dword 2h byte b -> K j = b (lo), 4 + b (hi); dword 2h+1 -> 8 + b, 12 + b
        for h in range(2):
            code[..., h, 0:4] = lo[..., 2 * h, :]
            code[..., h, 4:8] = hi[..., 2 * h, :]
            code[..., h, 8:12] = lo[..., 2 * h + 1, :]
            code[..., h, 12:16] = hi[..., 2 * h + 1, :]
    else:
        # dword q byte b: lo -> op 0 K j = 4q + b, hi ^ 8 -> op 1 K j = 4q + b
        code[..., 0, :] = lo.reshape(E, NB, KT, 64, 16)
        code[..., 1, :] = (hi ^ 8).reshape(E, NB, KT, 64, 16)
    # lane l: row l % 16, op h, K = 64 h + 16 (l // 16) + j
    c = code.reshape(E, NB, KT, 4, 16, 2, 16).transpose(0, 1, 4, 2, 5, 3, 6)  # E NB r KT h g j
    c = c.reshape(E, NB, 16, KT, 128)
    z = (meta & 15).transpose(0, 1, 3, 2)                       # E NB r KT
    s2 = (meta >> 4).transpose(0, 1, 3, 2)
    w = (c - z[..., None]) * s2[..., None]
    w = w.reshape(E, NB * 16, KT * 128).astype(np.float32)
    return (w * np.asarray(s1, dtype=np.float32)[..., None]).astype(np.float32)


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


def decode_native_nvfp4(vals, scales):
    """NVFP4 native layout -> f32 [E, N, K] in native row order: E2M1(code) * E4M3(scale).
    vals [E, NB, KT, 64, 16] (lane l = row l%16, dword j = K 32 j + 8 (l/16) .. +8, low nibble
    first), scales [E, NB, KT, 2, 16, 4] (dword (p, r) byte j = block 2 j + p of row r)."""
    vals = np.asarray(vals)
    scales = np.asarray(scales)
    E, NB, KT, L, B = vals.shape
    lo, hi = vals & 0xF, vals >> 4
    nib = np.stack([lo, hi], axis=-1).reshape(E, NB, KT, 4, 16, 4, 8)     # g, r, j, k
    v = nu.e2m1_decode(nib)
    # scale of (g, r, j): scales[..., g // 2, r, j]
    sc = np.zeros((E, NB, KT, 4, 16, 4), np.float32)
    for g in range(4):
        sc[:, :, :, g] = nu.e4m3_decode(scales[:, :, :, g // 2])
    v = v * sc[..., None]
    # K within the tile = 32 j + 8 g + k; rows r
    v = v.transpose(0, 1, 4, 2, 5, 3, 6)                                  # E NB r KT j g k
    return v.reshape(E, NB * 16, KT * 128).astype(np.float32)


def oracle_routes_parallel(x_dq, idx, w, experts, deq1, deq2, expert_begin, E_local, I, act_format, workers=16,
                           **kw):
    """moe.moe_forward per active local expert on a thread pool (numpy releases the GIL in the
    dequantisation and the products), the route outputs merged and combined in slot order by
    moe.combine_routes. experts: local expert id -> (W1 args, W2 args) for deq1 / deq2 (the
    packed bytes of that expert). Returns (y [M, H] f32, routes dict)."""
    import os
    from concurrent.futures import ThreadPoolExecutor
    from oracle import moe
    M, topk = idx.shape
    H = x_dq.shape[1]

    class _One:
        def __init__(self, e, fn, args, shape):
            self.e, self.fn, self.args, self.shape = e, fn, args, shape

        def __getitem__(self, i):
            assert i == self.e
            return self.fn(*self.args)

    def one(e):
        a1, a2 = experts[e]
        sub = np.where(idx == expert_begin + e, idx, -1)
        W1 = _One(e, deq1, a1, (E_local, 2 * I, H))
        W2 = _One(e, deq2, a2, (E_local, H, I))
        _, r = moe.moe_forward(x_dq, sub, w, W1, W2, expert_begin, act_format, **kw)
        return r

    routes = {}
    with ThreadPoolExecutor(max_workers=min(workers, os.cpu_count() or 1)) as ex:
        for r in ex.map(one, sorted(experts)):
            routes.update(r)
    return moe.combine_routes(routes, M, topk, H), routes


def active_local_experts(idx, expert_begin, E_local):
    loc = np.asarray(idx) - expert_begin
    return sorted({int(v) for v in loc.ravel() if 0 <= v < E_local and v + expert_begin >= 0})
