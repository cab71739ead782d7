"""Write the golden vectors under tests/golden/ from the reference's own Python packers.

Run in the build container only (the reference tree is not present on GPU boxes):
    python tests/golden/make_golden.py /root/reference [fixture names to rewrite]

What it does: loads the reference's torch-only packer files by path (no package __init__,
no extension module), feeds them seeded inputs built here (bf16-representable values plus
edge patterns: rounding ties, values a hair above powers of two, all-zero groups, tiny
negatives), and stores inputs and outputs as .npz fixtures. Nothing of the reference's
source is copied; the fixtures are data. The functions covered are the ones no closed
form pins completely (the log2-based scale rules, the NVFP4 ceil with its -1e-6 fudge,
the QoQ integer chain), per the oracle's header.
"""
import importlib.util
import os
import sys
import types

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def load_ref(ref_root):
    pkg = types.ModuleType("dgref")
    pkg.__path__ = [os.path.join(ref_root, "deep_gemm")]
    sys.modules["dgref"] = pkg
    mods = {}
    for name in ("quantization_nvfp4", "quantization_mxfp4", "quantization_mxfp4_fused",
                 "quantization_qoq_fused"):
        mods[name] = importlib.import_module("dgref." + name)
    spec = importlib.util.spec_from_file_location(
        "dgref_math", os.path.join(ref_root, "deep_gemm", "utils", "math.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    mods["math"] = m
    return mods


def bf16_round(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def weight_inputs(rng, E, N, K, scale):
    w = rng.standard_normal((E, N, K)).astype(np.float32) * scale
    w = bf16_round(w)
    # edge rows: exact E2M1 midpoints x power-of-two scales, an all-zero group,
    # tiny negatives, amax a hair above / below powers of two
    edges = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0], dtype=np.float32)
    row = np.tile(np.concatenate([edges, -edges]), K // 16)[:K] * np.float32(0.125)
    w[0, 0] = row
    w[0, 1, :32] = 0.0
    w[0, 1, 32:64] = -1e-3
    w[0, 1, 40] = 0.75
    for i in range(min(8, N - 2)):
        v = np.float32(6.0 * 2.0 ** (i - 4))
        hair = np.nextafter(v, np.float32(np.inf), dtype=np.float32)
        w[0, 2 + i, 0:32] = np.linspace(-1, 1, 32, dtype=np.float32) * v
        w[0, 2 + i, 0] = hair                      # amax/6 a hair above a power of two
        w[0, 2 + i, 32:64] = np.linspace(-1, 1, 32, dtype=np.float32) * v
    return w


def main(ref_root, only=()):
    mods = load_ref(ref_root)
    rng = np.random.default_rng(20261201)
    out = {}

    # ---------------- MXFP4 weight packers (fused and split)
    w = weight_inputs(rng, 2, 32, 256, 0.02)
    tw = torch.from_numpy(w)
    p, s = mods["quantization_mxfp4_fused"].quantize_to_mxfp4(tw)
    out["mxfp4_fused"] = dict(w=w, packed=p.numpy(), scale=s.numpy())
    p, s = mods["quantization_mxfp4"].quantize_to_mxfp4(tw)
    out["mxfp4_split"] = dict(w=w, packed=p.numpy(), scale=s.numpy())

    # ---------------- NVFP4 packer + UE4M3 ceil over a dense sweep
    p, s = mods["quantization_nvfp4"].quantize_to_nvfp4(tw)
    out["nvfp4"] = dict(w=w, packed=p.numpy(), scale=s.numpy())
    sweep = np.concatenate([
        np.geomspace(2.0 ** -12, 600.0, 20000).astype(np.float32),
        np.array([2.0 ** e * (1 + m / 8.0) for e in range(-9, 9) for m in range(8)], np.float32),
        np.array([np.nextafter(np.float32(2.0 ** e * (1 + m / 8.0)), np.float32(np.inf))
                  for e in range(-9, 9) for m in range(8)], np.float32),
        np.array([np.nextafter(np.float32(2.0 ** e * (1 + m / 8.0)), np.float32(0))
                  for e in range(-9, 9) for m in range(8)], np.float32),
    ])
    code = mods["quantization_nvfp4"].fp32_to_ue4m3_ceil(torch.from_numpy(sweep))
    out["ue4m3_ceil"] = dict(x=sweep, code=code.numpy())

    # ---------------- QoQ W4A8 packer + per-token int8
    wq = weight_inputs(rng, 2, 16, 256, 0.05)
    pq, s2, z, s1 = mods["quantization_qoq_fused"].quantize_to_qoq(torch.from_numpy(wq).to(torch.bfloat16))
    out["qoq"] = dict(w=wq, packed=pq.numpy(), s2=s2.numpy(), z=z.numpy(), s1=s1.numpy())
    # the split path's QoQ int4 packer (int32 coefficient plane) on the same weights, and its
    # reference dequantisation
    pi4, plane = mods["quantization_mxfp4"].quantize_to_qoq_int4(torch.from_numpy(wq).to(torch.bfloat16))
    deq = mods["quantization_mxfp4"].dequantize_qoq_int4(pi4, plane)
    out["qoq_int4"] = dict(w=wq, packed=pi4.numpy(), plane=plane.numpy(), deq=deq.numpy())
    xa = bf16_round(rng.standard_normal((4, 512)).astype(np.float32))
    qb, sf = mods["quantization_qoq_fused"].per_token_cast_to_int8(torch.from_numpy(xa).to(torch.bfloat16))
    out["int8_act"] = dict(x=xa, q=qb.view(torch.int8).numpy(), sf=sf.numpy())

    # ---------------- activation casts (utils.math)
    xa = bf16_round(rng.standard_normal((6, 3072)).astype(np.float32))
    xa[0, :32] = 0.0
    xa[1, :32] = np.tile(np.array([0.25, 0.75, 1.75, 3.5, -0.25, -0.75, -1.75, -3.5], np.float32), 4) / 8
    xa[1, 5] = 6.0 / 8
    txa = torch.from_numpy(xa).to(torch.bfloat16)
    m = mods["math"]
    p4, sf4 = m.per_token_cast_to_fp4(txa, use_ue8m0=True, gran_k=32)
    out["fp4_act"] = dict(x=xa, packed=p4.view(torch.uint8).numpy(), sf=sf4.numpy())
    q8, sf8 = m.per_token_cast_to_fp8(txa, use_ue8m0=True, gran_k=32)
    out["fp8_act_ue8m0"] = dict(x=xa, q=q8.view(torch.uint8).numpy(), sf=sf8.numpy())
    q8b, sf8b = m.per_token_cast_to_fp8(txa, use_ue8m0=False, gran_k=128)
    out["fp8_act_f32"] = dict(x=xa, q=q8b.view(torch.uint8).numpy(), sf=sf8b.numpy())
    e2 = np.linspace(-7, 7, 4097).astype(np.float32)
    out["e2m1"] = dict(x=e2, code=m._quantize_to_fp4_e2m1(torch.from_numpy(e2)).view(torch.uint8).numpy())
    ue = np.concatenate([np.geomspace(1e-30, 1e30, 5000).astype(np.float32),
                         np.array([2.0 ** e for e in range(-30, 30)], np.float32)])
    out["ue8m0"] = dict(x=ue, y=m.ceil_to_ue8m0(torch.from_numpy(ue)).numpy())

    for name, d in out.items():
        if only and name not in only:
            continue
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **d)
        print(name, {k: v.shape for k, v in d.items()})


if __name__ == "__main__":
    # optional further arguments: the fixture names to (re)write, e.g. qoq_int4
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference", set(sys.argv[2:]))
