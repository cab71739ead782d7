"""Seeded random layer shapes through the persistent kernel: expert counts, EP shares and ranks,
top-k from 1 to 16, token counts from 1 to 64, both A-MXFP formats, real or forced-balanced
routing, all-zero rows, the top-k selected in the frontend or in the kernel's prologue. Each case
is checked as the fixed-shape tests are: frontend keys, top-k and activation codes and the pool
table bit-exact against the oracle, recv stats, y within the north star's tolerance; and the
split launches give the fused kernel's y bit for bit."""
import numpy as np
import pytest
import torch

from tests.gpu_common import need_gpu
from tests.test_gpu_layer import make_weights, run_layer, check_frontend, check_pool, check_y

pytestmark = pytest.mark.gpu


def _cases(n=40, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        H, I = [(512, 256), (1024, 512)][int(rng.integers(2))]
        ep = [1, 2, 4][int(rng.integers(3))]
        e_local = int(rng.integers(2, 41))
        E = e_local * ep
        topk = int(rng.integers(1, min(16, E) + 1))
        M = int(rng.integers(1, 65))
        while M * topk > 512:
            M //= 2
        fmt = ["mxfp4", "mxfp8"][i % 2]
        balanced = E % topk == 0 and rng.random() < 0.5
        zero_rows = () if balanced or M < 3 else tuple(sorted(set(int(v) for v in rng.integers(0, M, int(rng.integers(0, 3))))))
        select = bool(rng.integers(2))
        rank = int(rng.integers(ep))
        out.append((i, M, E, e_local, rank * e_local, H, I, topk, fmt, balanced, zero_rows, select))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"case{c[0]}")
def test_random_shape(case):
    need_gpu()
    import hopper_megamoe_basedondeepgemm_amd as dgm
    i, M, E, e_local, begin, H, I, topk, fmt, balanced, zero_rows, select = case
    print(f"random shape {i}: M={M} E={E} local={e_local}@{begin} H={H} I={I} topk={topk} {fmt} "
          f"balanced={balanced} zero_rows={zero_rows} select_in_mega={select}", flush=True)
    weights = make_weights(e_local, H, I, 9000 + i)
    r = run_layer(M, E, e_local, begin, H, I, topk, fmt, seed=9100 + i, force_balanced=balanced,
                  zero_rows=zero_rows, weights=weights, select_in_mega=select)
    check_frontend(r, fmt, M, force_balanced=balanced, zero_rows=zero_rows)
    check_pool(r, e_local, begin)
    check_y(r, zero_rows=zero_rows)
    (t1, t2), _, _ = weights
    y2 = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    dgm.mxfp4_mega_moe_split(y2, t1, t2, r["buf"], activation_clamp=10.0)
    torch.cuda.synchronize()
    assert r["buf"].kernel_error() == 0
    np.testing.assert_array_equal(y2.float().cpu().numpy(), r["y"])
