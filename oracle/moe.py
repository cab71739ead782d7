"""CPU restatement of the exact-quantised MegaMoE layer (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
this module; the product path never calls it.

Stages, each citing the reference rule it restates:
  router      tests/test_four_api_correctness.py:371-374 (fp32 GEMM -> bf16 -> stable sort
              desc -> fp32 softmax of the 8 selected logits); key order of the frontend
              deep_gemm/include/deep_gemm/impls/fable_cc_select.cuh:6-9 (value desc, index asc).
  balanced    tests/test_four_api_correctness.py:125-144 (slot s -> s*G + (g + 7 s) % G, 1/topk).
  dispatch    build-defined canonical order (token asc, slot asc) per local expert; counts
              equal bincount(topk_idx) (the reference's own order is atomic-ticket order).
  act quant   sm100_b200/test_mega_moe.py:68-93 (MXFP4 rows), deep_gemm/utils/math.py:26-38
              (MXFP8 E4M3 + UE8M0/32).
  experts     sm100_b200/test_mega_moe.py:411-486: fp32 x_dq @ W1^T, gate/up rounded to
              bf16, clamp (gate <= c, up in [-c, c]), silu(gate)*up*w, per-32 requant
              (MXFP4: ceil_to_ue8m0(amax/6) + ties-down E2M1; MXFP8: 2^ceil(log2(amax/448))
              + E4M3), fp32 @ W2^T; each route's output rounded to bf16 and the routes summed
              in fp32 in slot order (tests/test_four_api_correctness.py:443-444, the rule of
              the H20 fused kernel's L2 epilogue, sm90_fp4_mega_moe_h20_fused_body.inl:1991-1994).
  qoq         deep_gemm/quantization_qoq_fused.py:78-91 (per-token int8 cast);
              tests/test_four_api_correctness.py:421-446 (dequantised weights, fp32 gate/up
              without bf16 rounding, per-64 int8 requant, per-route bf16, fp32 sum).
  nvfp4       sm100_b200/test_mega_moe.py:68-93 (W4A4 row cast: E4M3 RNE of amax/6 per 16,
              ties-down E2M1), :431-438 (per-16 requant), optional per-expert global scales
              of deep_gemm/mega/__init__.py:277 on the L1 / L2 outputs.

Router accumulation order. The reference's logits are an fp32 GEMM whose summation order is
unspecified (torch / cuBLAS / the frontend's K-split). This build fixes one order and uses
it on both sides, so logits and therefore top-k are bit-exact: for each (token, expert),
lane l in 0..63 sums k = 512 j + 8 l + i (j ascending, then i ascending) with fp32
adds of exact bf16 x bf16 products, then the 64 lane sums are combined by the xor
butterfly (offsets 32, 16, 8, 4, 2, 1). ``router_logits_torch_order`` gives the plain
fp32 GEMM for the <= 1-bf16-ulp comparison.
"""
import numpy as np

from .numerics import (as_f32, round_bf16, f32_to_bf16_bits, bf16_bits_to_f32,
                       ceil_to_ue8m0, ceil_log2_f32, e2m1_code_ties_down, e2m1_decode,
                       e4m3_encode, e4m3_decode)
from . import packers

LANES = 64
VEC = 8


# ----------------------------------------------------------------------------- router
def router_logits_f32(x_bf16_f32, w_bf16_f32):
    """Deterministic-order fp32 logits [M, E] (see module docstring)."""
    x = as_f32(x_bf16_f32)
    w = as_f32(w_bf16_f32)
    M, K = x.shape
    E = w.shape[0]
    assert K % (LANES * VEC) == 0
    J = K // (LANES * VEC)
    xr = x.reshape(M, J, LANES, VEC)
    wr = w.reshape(E, J, LANES, VEC)
    acc = np.zeros((M, E, LANES), dtype=np.float32)
    for j in range(J):
        for i in range(VEC):
            acc = acc + xr[:, None, j, :, i] * wr[None, :, j, :, i]
    lane = np.arange(LANES)
    for off in (32, 16, 8, 4, 2, 1):
        acc = acc + acc[:, :, lane ^ off]
    return acc[:, :, 0].astype(np.float32)


def router_logits_torch_order(x_bf16_f32, w_bf16_f32):
    """Plain fp32 GEMM (BLAS order), the reference's ``x.float() @ W.float().T``."""
    return (as_f32(x_bf16_f32) @ as_f32(w_bf16_f32).T).astype(np.float32)


def topk_keys(logits_bf16_bits, E):
    """Frontend key (deep_gemm/include/deep_gemm/impls/fable_frontend_device.cuh:252-257):
    orderable(bf16) << 16 | (0xFFFF - e), with -0 mapped to +0 first."""
    b = np.asarray(logits_bf16_bits, dtype=np.uint32)
    b = np.where(b == 0x8000, 0, b)
    o = np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000)
    e = np.arange(E, dtype=np.uint32)
    return ((o << 16) | (0xFFFF - e)).astype(np.uint32)


def topk_softmax(logits_f32, topk):
    """bf16-rounded logits -> top-k by (value desc, index asc) -> fp32 softmax over the k
    selected values: w_k = exp(v_k - v_0) / sum_{j<k} (sequential sum, v_0 the max).
    Returns (idx int64 [M, k], weights f32 [M, k], bf16 logits as f32 [M, E])."""
    M, E = logits_f32.shape
    bits = f32_to_bf16_bits(logits_f32)
    lb = bf16_bits_to_f32(bits)
    keys = topk_keys(bits, E)
    order = np.argsort(-keys.astype(np.int64), axis=1, kind="stable")[:, :topk]
    vals = np.take_along_axis(lb, order, axis=1)
    ex = np.exp((vals - vals[:, :1]).astype(np.float32)).astype(np.float32)
    s = np.zeros(M, dtype=np.float32)
    for k in range(topk):
        s = (s + ex[:, k]).astype(np.float32)
    w = (ex / s[:, None]).astype(np.float32)
    return order.astype(np.int64), w, lb


def balanced_routing(M, E, topk, token_offset=0, num_ranks=None):
    """Forced-balanced routing (tests/test_four_api_correctness.py:125-144, the same rule as
    tests/profile_four_api_h20.py:139-160): global token g, slot s -> expert
    s*G + (g + 7 s) % G with G = E / num_ranks (the EP rank's expert count, T4:138), so slot s
    lands on EP rank s; weight 1/topk exactly. The rule gives every rank exactly one route per
    token only when topk == num_ranks (the reference runs 8 ranks at top-8); num_ranks defaults
    to topk, the case the device kernels implement (their G is E / topk)."""
    if num_ranks is None:
        num_ranks = topk
    assert E % num_ranks == 0 and topk <= num_ranks, (E, topk, num_ranks)
    G = E // num_ranks
    g = np.arange(M, dtype=np.int64)[:, None] + token_offset
    s = np.arange(topk, dtype=np.int64)[None, :]
    idx = s * G + (g + 7 * s) % G
    return idx, np.full((M, topk), 1.0 / topk, dtype=np.float32)


def dispatch(topk_idx, expert_begin, num_local):
    """Canonical pools: for each local expert (ascending) the routes (t, s) with
    topk_idx[t, s] == expert, ordered by (t asc, s asc). Returns (counts [num_local],
    active experts (local ids, ascending), offsets [n_active+1], routes int64 t*topk+s)."""
    M, topk = topk_idx.shape
    loc = topk_idx - expert_begin
    valid = (topk_idx >= 0) & (loc >= 0) & (loc < num_local)
    counts = np.bincount(loc[valid], minlength=num_local).astype(np.int64)
    active = np.nonzero(counts)[0]
    routes = []
    offsets = [0]
    for e in active:
        t, s = np.nonzero((loc == e) & valid)
        rid = t * topk + s
        routes.extend(sorted(rid.tolist()))
        offsets.append(len(routes))
    return counts, active, np.array(offsets, dtype=np.int64), np.array(routes, dtype=np.int64)


# ----------------------------------------------------------------------------- activation formats
def quant_act(x_f32, act_format):
    """Input activation cast. 'mxfp4': cast_to_fp4_rows (UE8M0/32, ties-down E2M1);
    'mxfp8': per_token_cast_to_fp8(use_ue8m0, gran 32). Returns (codes, sf_byte, dequant)."""
    if act_format == "mxfp4":
        p, sf, sfb = packers.cast_to_fp4_rows(x_f32, 32)
        return p, sfb, packers.dequant_fp4_rows(p, sf, 32)
    if act_format == "mxfp8":
        q, sf = packers.per_token_cast_to_fp8_ue8m0(x_f32, 32)
        sfb = ((sf.view(np.uint32) >> 23) & 0xFF).astype(np.uint8)
        return q, sfb, packers.dequant_fp8_rows(q, sf, 32)
    if act_format == "fp8f128":
        # the SM90 split recipe's activations: per_token_cast_to_fp8(use_ue8m0=False, gran_k=128)
        # (deep_gemm/utils/math.py:26-38; tests/test_four_api_correctness.py:215, x_reference :226-230)
        q, sf = packers.per_token_cast_to_fp8_f32sf(x_f32, 128)
        return q, sf, packers.dequant_fp8_rows(q, sf, 128)
    if act_format == "nvfp4":
        # W4A4 NVFP4 row cast (sm100_b200/test_mega_moe.py:68-93, act_format 'nvfp4')
        p, sf, sfb = packers.cast_to_nvfp4_rows(x_f32)
        return p, sfb, packers.dequant_fp4_rows(p, sf, 16)
    if act_format == "qoq":
        # per_token_cast_to_int8 (deep_gemm/quantization_qoq_fused.py:78-91); x_reference of
        # tests/test_four_api_correctness.py:243-246: int8 * the token's scale
        q, sf = packers.per_token_cast_to_int8(x_f32)
        return q, sf, (q.astype(np.float32) * sf[:, None]).astype(np.float32)
    raise ValueError(act_format)


def requant_mid(a, act_format):
    """Intermediate requant of the kernel (sm100_b200/test_mega_moe.py:425-437), per 32."""
    a = as_f32(a)
    g = a.reshape(*a.shape[:-1], -1, 32)
    amax = np.maximum(np.abs(g).max(axis=-1, keepdims=True), np.float32(1e-30))
    if act_format == "mxfp4":
        sf = ceil_to_ue8m0(amax / np.float32(6.0))
        codes = e2m1_code_ties_down(g / sf)
        return (e2m1_decode(codes) * sf).reshape(a.shape).astype(np.float32)
    if act_format == "mxfp8":
        sf = np.exp2(ceil_log2_f32(amax / np.float32(448.0))).astype(np.float32)
        return (e4m3_decode(e4m3_encode(g / sf)) * sf).reshape(a.shape).astype(np.float32)
    if act_format == "qoq":
        return requant_mid_qoq(a)[2]
    if act_format == "nvfp4":
        return requant_mid_nvfp4(a)
    if act_format == "fp8f128":
        return requant_mid_fp8_64(a)[2]
    raise ValueError(act_format)


def requant_mid_fp8_64(a):
    """FP8 intermediate requant of tests/test_four_api_correctness.py:54-62 (non-QoQ branch), the
    rule of the fp8 x MXFP4 split recipe: per 64 features, scale = 2^ceil(log2(max(amax / 448,
    tiny))), E4M3 (round to nearest even) of a / scale. Returns (E4M3 codes, E8M0 bytes of the
    scales [.., n/64], dequantised)."""
    a = as_f32(a)
    g = a.reshape(*a.shape[:-1], -1, 64)
    amax = np.abs(g).max(axis=-1, keepdims=True)
    sa = np.maximum(amax / np.float32(448.0), FLT_TINY).astype(np.float32)
    e = ceil_log2_f32(sa)
    sc = np.exp2(e).astype(np.float32)
    codes = e4m3_encode(g / sc)
    return (codes.reshape(a.shape), (e[..., 0] + 127).astype(np.uint8),
            (e4m3_decode(codes) * sc).reshape(a.shape).astype(np.float32))


def requant_mid_nvfp4(a):
    """W4A4 NVFP4 intermediate requant (sm100_b200/test_mega_moe.py:431-438 ``requant_fp4`` with
    the NVFP4 rule of :68-72): per 16, sf = E4M3(max(amax, 1e-30) / 6) (round to nearest even),
    ties-down E2M1 of a / sf; returns the dequantised values."""
    a = as_f32(a)
    g = a.reshape(*a.shape[:-1], -1, 16)
    amax = np.maximum(np.abs(g).max(axis=-1, keepdims=True), np.float32(1e-30))
    sf = e4m3_decode(e4m3_encode(amax / np.float32(6.0)))
    with np.errstate(divide="ignore", invalid="ignore"):
        codes = e2m1_code_ties_down(g / sf)
    return (e2m1_decode(codes) * sf).reshape(a.shape).astype(np.float32)


FLT_TINY = np.float32(np.finfo(np.float32).tiny)


def requant_mid_qoq(a):
    """QoQ intermediate requant (tests/test_four_api_correctness.py:54-60, qoq branch): per 64
    features, scale = max(amax / 127, tiny), q = clamp(rne(a / scale), +-127).
    Returns (int8 codes, scales [.., n/64], dequantised)."""
    a = as_f32(a)
    g = a.reshape(*a.shape[:-1], -1, 64)
    amax = np.abs(g).max(axis=-1, keepdims=True)
    sc = np.maximum(amax / np.float32(127.0), FLT_TINY).astype(np.float32)
    q = np.clip(np.rint(g / sc), -127, 127).astype(np.float32)
    return (q.astype(np.int8).reshape(a.shape), sc[..., 0],
            (q * sc).reshape(a.shape).astype(np.float32))


def silu(x):
    """x * sigmoid(x) with sigmoid = 1 / (1 + exp(-x)), the reference's
    ``gate * torch.sigmoid(gate)`` (sm100_b200/test_mega_moe.py:459)."""
    x = as_f32(x)
    return (x * (np.float32(1.0) / (np.float32(1.0) + np.exp(-x)))).astype(np.float32)


class LazyDequant:
    """Per-expert dequantisation on access (``W[e]`` -> f32 [N, K]) so the layer oracle can
    run at full layer shapes while touching only the routed experts."""

    def __init__(self, packed, scale, fn=None):
        self.packed, self.scale = packed, scale
        self.fn = fn or packers.dequantize_mxfp4_marlin
        E, N, Kh = packed.shape
        self.shape = (E, N, Kh * 2)

    def __getitem__(self, e):
        if isinstance(e, slice):
            return LazyDequant(self.packed[e], self.scale[e], self.fn)
        return self.fn(self.packed[e], self.scale[e])


# ----------------------------------------------------------------------------- layer
def moe_forward(x_dq, topk_idx, topk_w, W1, W2, expert_begin, act_format, clamp=10.0,
                bf16_gate_up=True, route_bf16=True, gs1=None, gs2=None):
    """Expert part of the layer on dequantised inputs.

    x_dq [M, H] f32 (dequantised activations), topk_idx [M, k], topk_w [M, k],
    W1 [E_local, 2I, H] f32 (gate rows 0..I-1, up rows I..2I-1), W2 [E_local, H, I] f32.
    route_bf16: each route's output rounded to bf16 (tests/test_four_api_correctness.py:443);
    y[t] = fp32 sum of the token's local routes in slot order (:444).
    Returns (y_f32 [M, H], per-route outputs dict rid -> f32 [H])."""
    M, H = x_dq.shape
    E_local, twoI, _ = W1.shape
    I = twoI // 2
    topk = topk_idx.shape[1]
    c = np.float32(clamp)
    routes = {}
    for e in range(E_local):
        t_ids, s_ids = np.nonzero(topk_idx == expert_begin + e)
        if t_ids.size == 0:
            continue
        w1e, w2e = W1[e], W2[e]
        h = (x_dq[t_ids] @ w1e.T).astype(np.float32)
        if gs1 is not None:    # per-expert output scale (deep_gemm/mega/__init__.py:277 global scales)
            h = (h * np.float32(gs1[e])).astype(np.float32)
        gate, up = h[:, :I], h[:, I:]
        if bf16_gate_up:
            gate, up = round_bf16(gate), round_bf16(up)
        gate = np.minimum(gate, c)
        up = np.clip(up, -c, c)
        act = ((silu(gate) * up).astype(np.float32) * topk_w[t_ids, s_ids][:, None]).astype(np.float32)
        act = requant_mid(act, act_format)
        out = (act @ w2e.T).astype(np.float32)
        if gs2 is not None:
            out = (out * np.float32(gs2[e])).astype(np.float32)
        if route_bf16:
            out = round_bf16(out)
        for n, (t, s) in enumerate(zip(t_ids, s_ids)):
            routes[int(t) * topk + int(s)] = out[n]
    return combine_routes(routes, M, topk, H), routes


def combine_routes(routes, M, topk, H):
    """y[t] = fp32 sum of the token's route outputs in slot order (tests/test_four_api_correctness.py:444,
    ``routes.sum(dim=1)`` over slots); tokens without a route give 0."""
    y = np.zeros((M, H), dtype=np.float32)
    for t in range(M):
        for s in range(topk):
            r = routes.get(t * topk + s)
            if r is not None:
                y[t] = (y[t] + r).astype(np.float32)
    return y


def moe_forward_qoq(x_dq, topk_idx, topk_w, W1, W2, expert_begin, clamp=10.0):
    """QoQ W4A8 layer of tests/test_four_api_correctness.py:421-446 on dequantised weights
    (dequantize_qoq) and activations: fp32 gate/up (no bf16 rounding), clamp, SiLU * up * w,
    per-64 int8 requant, fp32 down projection rounded to bf16 per route, fp32 sum."""
    return moe_forward(x_dq, topk_idx, topk_w, W1, W2, expert_begin, "qoq", clamp, bf16_gate_up=False,
                       route_bf16=True)


def qoq_group_acc(codes, z, x8):
    """The W4A8 kernel's int32 accumulator of one K128 group (exact): sum_k (code - z) * x8.
    codes [N, 128] (0..15), z [N], x8 [T, 128] int8 -> int64 [N, T]."""
    return (codes.astype(np.int64) - z.astype(np.int64)[:, None]) @ x8.astype(np.int64).T


def layer_forward(hidden_bf16_f32, router_w_bf16_f32, W1, W2, expert_begin, act_format,
                  topk=8, clamp=10.0, force_balanced=False, token_offset=0):
    """Router + top-k + activation cast + experts. Returns a dict with every intermediate."""
    E = router_w_bf16_f32.shape[0]
    logits = router_logits_f32(hidden_bf16_f32, router_w_bf16_f32)
    idx, w, lb = topk_softmax(logits, topk)
    if force_balanced:
        idx, w = balanced_routing(hidden_bf16_f32.shape[0], E, topk, token_offset)
    codes, sfb, x_dq = quant_act(hidden_bf16_f32, act_format)
    y, routes = moe_forward(x_dq, idx, w, W1, W2, expert_begin, act_format, clamp)
    return dict(logits=logits, logits_bf16=lb, topk_idx=idx, topk_w=w, x_codes=codes,
                x_sf=sfb, x_dq=x_dq, y=y, routes=routes)


def metrics(y, ref):
    """cos per row (min), rel-RMSE, max abs (tests/test_four_api_correctness.py:69-97;
    sm100_b200/test_mega_moe.py:488)."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    num = (y * r).sum(-1)
    den = np.sqrt((y * y).sum(-1) * (r * r).sum(-1))
    cos = np.where(den > 0, num / np.where(den > 0, den, 1), 1.0)
    rel = np.sqrt(((y - r) ** 2).sum()) / max(np.sqrt((r * r).sum()), 1e-12)
    return dict(cos_min=float(cos.min()) if cos.size else 1.0, rel_rmse=float(rel),
                max_abs=float(np.abs(y - r).max()) if y.size else 0.0)
