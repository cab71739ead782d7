"""Benchmark of the MI355X MegaMoE layer (one GPU).

Headline workload = benchmark config 2: the full E384 / H3072 / I1280 / top-8 layer resident on
one GPU (W-MXFP4 x A-MXFP8), forced-balanced routing, M=8 tokens per step (one step = one
layer forward from bf16 hidden states: the frontend launch (router + activation cast), then the
fused kernel: top-8 in its prologue, dispatch, L1, L2, combine). Also sweeps M = 2, 4, 8, 16 for
three activation formats (A-MXFP8, A-MXFP4, and the reference fused buffer's E4M3 with fp32
scales per 128) and the QoQ W4A8 layer (int8 activations, QoQ 4-bit weights), config 0 (48
experts, M=2, softmax routing) and config 1 (one EP rank's 48 experts of the 384-way router,
M=8), the NVFP4 W4A4 layer at M = 16, 64, 128 with seeded unbalanced routing (config 4), and
one seeded unbalanced-routing A-MXFP8 run at M=16. Before every timed step >= 1 GiB is written and
then 1 GiB of other data is read, so neither the 256 MB MALL nor the L2s hold weights (and
no dirty lines are left to drain inside the timed region); per step, HIP events on the
layer's stream bracket the layer (and, for two launches, the frontend and the fused kernel).

Prints ONE JSON line (the driver contract). Data are synthetic (seeded randn weights of the
layer's shape, packed on the GPU with the MXFP4 packer).
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

E, H, I, TOPK = 384, 3072, 1280, 8
MXFP4_EXPERT_BYTES = 6266880          # W1 + W2 values + E8M0 scales of one expert
# QoQ W4A8: 4-bit codes (5,898,240 B) + one meta byte (z | s2 << 4) per row and K128 group
# (2I * H/128 + H * I/128 = 92,160 B) + fp32 row scales s1 ((2I + H) * 4 = 22,528 B)
QOQ_EXPERT_BYTES = 6012928
# NVFP4 W4A4: E2M1 values (5,898,240 B) + one E4M3 scale per 16 (737,280 B)
NVFP4_EXPERT_BYTES = 6635520
HBM_PEAK_GBS = 8000.0


def profiled_traffic_bytes():
    """HBM bytes per launch of the fused kernel at the headline workload, from the committed
    rocprofv3 counter summary (FETCH_SIZE + WRITE_SIZE, scaled by a plain device copy), or None."""
    path = os.path.join(HERE, "profiles", "k_megamoe_E384_M8_mxfp8_hbm_traffic.txt")
    try:
        for ln in open(path):
            if ln.strip().startswith("traffic (fetch + write) ="):
                return int(float(ln.split("=")[1].split()[0]) * 1e6)
    except OSError:
        pass
    return None


def profiled_mfma_util(kernel="k_megamoe<24,10,1,0>", workload=("M=8", "A-MXFP8")):
    """Matrix-core busy fraction of the fused kernel at the headline workload, from the committed
    rocprofv3 counter summary (SQ_VALU_MFMA_BUSY_CYCLES over all SIMD cycles), or None."""
    path = os.path.join(HERE, "profiles", "k_megamoe_E384_mfma_valu_counters.txt")
    try:
        for ln in open(path):
            f = ln.split()
            if len(f) >= 8 and f[0] == kernel and tuple(f[1:3]) == workload:
                return float(f[7])
    except (OSError, ValueError):
        pass
    return None


def phase_stamps_report(torch, dgm, weights, router_w, reps=9):
    """Per-workgroup phase stamps of the fused kernel (its phase_stamps output: 100 MHz wall
    clock at entry, dispatch table ready, L1 units done, first L1 arrival observed by the L2
    phase, L2 units done, exit; plus the L1 K-loop and epilogue ticks): for each workload the
    launch with the median event time of `reps`, each after a cache eviction, printed as
    min / p10 / median / p90 / max over the workgroups in us from the earliest entry. The
    one-launch layer (frontend in the kernel; M=2 and M=8) adds its frontend stamps: router and
    cast work done, grid-wide arrival passed (its event time covers the whole layer)."""
    flush = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    flush_rd = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    share = tuple(tuple(t[:E // 8] if t is not None else None for t in w) for w in weights)
    names = ("entry", "dispatch ready", "L1 done", "first L1 seen", "L2 done", "exit")
    bufs = {}
    # (M=2 and config 1 in the kernel's forms, on one buffer: the default, and the opt-in early
    # weight streaming (debug flag bit 3) and, at M=2, tail half units (bit 4))
    # (one = the one-launch layer: the frontend runs in the fused kernel)
    for M, ep, act, flags, one in ((2, 1, "mxfp8", 0, False), (2, 1, "mxfp8", 8, False), (2, 1, "mxfp8", 16, False),
                                   (2, 1, "mxfp8", 0, True), (8, 1, "mxfp8", 0, False), (8, 1, "mxfp8", 0, True),
                                   (16, 1, "mxfp8", 0, False), (8, 8, "mxfp4", 0, False), (8, 8, "mxfp4", 8, False)):
        w = share if ep > 1 else weights
        buf = bufs.get((M, ep, act))
        if buf is None:
            buf = bufs[(M, ep, act)] = dgm.get_fused_symm_buffer_for_mega_moe(None, E, M, TOPK, H, I, act_format=act,
                                                                              ep_size=ep, ep_rank=0)
        buf._debug_flags = flags
        g = torch.Generator(device="cuda")
        g.manual_seed(4000 + M)
        x = torch.randn((M, H), generator=g, device="cuda").to(torch.bfloat16)
        y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
        st = torch.zeros((1024, 8), dtype=torch.int64, device="cuda")
        runs = []
        for _ in range(reps):
            flush.fill_(1)
            flush_rd.sum()
            if not one:
                dgm.fable_router_quant_topk_frontend(x, router_w, buf, force_balanced=True, select_in_mega=True)
            st.zero_()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            if one:
                dgm.mxfp4_mega_moe_from_bf16(y, x, router_w, w[0], w[1], buf, force_balanced=True, one_launch=True,
                                             phase_stamps=st)
            else:
                dgm.mxfp4_mega_moe_fused(y, w[0], w[1], buf, phase_stamps=st)
            e1.record()
            torch.cuda.synchronize()
            runs.append((e0.elapsed_time(e1) * 1e3, st.clone()))
        runs.sort(key=lambda r: r[0])
        ev, st = runs[len(runs) // 2]
        G = dgm.mega.fused_workgroups(buf)
        a = st[:G].cpu().numpy().astype(np.float64)
        t0 = a[:, 0].min()
        n_active = int((buf.pool_table()[0] > 0).sum())
        form = dgm.mega.FUSED_FORMS.get(dgm.mega.fused_last_form(buf), "?")
        print(f"M={M} ep_share={ep} A-{act.upper()} ({form} form{', one launch' if one else ''}) active experts "
              f"{n_active}, {G} workgroups, kernel "
              f"{ev:.1f} us by events; us from the earliest entry (min / p10 / median / p90 / max):")
        rows = list(enumerate(names))
        if one:
            rows = rows[:1] + [(6, "router+cast"), (7, "grid arrival")] + rows[1:]
        for c, nm in rows:
            v = a[:, c]
            v = (v[v > 0] - t0) / 100.0 if c == 3 else (v - t0) / 100.0    # (0: never waited)
            if len(v):
                q = np.percentile(v, [0, 10, 50, 90, 100])
                print(f"  {nm:15s}" + "".join(f" {x:7.2f}" for x in q))
        k = a[:, 6][a[:, 6] > 0] / 100.0
        e = a[:, 7][a[:, 6] > 0] / 100.0
        if len(k) and not one:
            print(f"  per workgroup with L1 work: L1 K loops {np.median(k):.2f} us (median), "
                  f"L1 epilogues {np.median(e):.2f} us (median)")
        sys.stdout.flush()


def probes_report(torch, reps=15):
    """The platform figures the fused kernel is measured against (the probe library,
    include/dgm_probe.h), each launch after a 1 GiB write + 1 GiB read eviction, HIP events on the
    launch stream, median of `reps`:
      * HBM read probe: the fused kernel's streaming pattern (runs of 24 consecutive 1 KB tiles per
        wave, a ring of non-temporal loads, 256 workgroups of 8 waves) without its arithmetic, at
        the weight bytes of config 1 (50 MB) and of the headline (401 MB), ring depths 4 / 12 / 24;
      * the launch floor: an empty kernel of 256 x 512 and 1 x 64 threads;
      * the per-workgroup rate of the same pattern on 32 to 256 workgroups, ring depths 4 / 12 / 24."""
    from hopper_megamoe_basedondeepgemm_amd import _lib
    lib = _lib.load_probe()
    flush = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    flush_rd = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    src = torch.ones(64 * MXFP4_EXPERT_BYTES // 4 + 4096, dtype=torch.int32, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()

    def timed(fn):
        ts = []
        for _ in range(reps):
            flush.fill_(1)
            flush_rd.sum()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3)
        return float(np.median(ts)), float(np.min(ts))

    print("HBM read probe (256 workgroups x 8 waves, runs of 24 x 1 KB tiles, non-temporal loads), "
          "median / min of %d after a 1 GiB eviction:" % reps)
    for experts in (8, 64):
        nbytes = experts * MXFP4_EXPERT_BYTES // (24 * 1024) * (24 * 1024)
        for depth in (4, 12, 24):
            med, mn = timed(lambda: _lib.check(lib.dgm_probe_stream_read(_lib.ptr(src), nbytes, depth, 256,
                                                                          _lib.ptr(sink), _lib.stream())))
            print(f"  {nbytes / 1e6:7.1f} MB  ring {depth:2d}: {med:7.2f} us ({mn:7.2f} min) = "
                  f"{nbytes / (med * 1e-6) / 1e12:5.2f} TB/s")
    print("empty kernel (returns at entry), median / min of %d after a 1 GiB eviction:" % reps)
    floor = None
    for blocks, threads in ((256, 512), (1, 64)):
        med, mn = timed(lambda: _lib.check(lib.dgm_probe_empty_launch(blocks, threads, _lib.stream())))
        floor = med if floor is None else floor
        print(f"  {blocks:4d} x {threads:3d} threads: {med:6.2f} us ({mn:6.2f} min) by events")
    # the same pattern on fewer workgroups (the small shapes and the tail of every shape, where
    # the HBM is not saturated): each wave streams 4 runs (768 KB per workgroup); per-workgroup
    # rate over the event time minus the empty kernel's
    print("HBM read probe on fewer workgroups (4 runs of 24 x 1 KB per wave, 768 KB per workgroup), "
          "median of %d; GB/s per workgroup over (time - empty kernel):" % reps)
    for blocks in (32, 64, 128, 160, 256):
        nbytes = blocks * 8 * 4 * 24 * 1024
        row = []
        for depth in (4, 12, 24):
            med, _ = timed(lambda: _lib.check(lib.dgm_probe_stream_read(_lib.ptr(src), nbytes, depth, blocks,
                                                                         _lib.ptr(sink), _lib.stream())))
            row.append(f"ring {depth:2d} {med:6.2f} us {nbytes / blocks / ((med - floor) * 1e-6) / 1e9:5.1f}")
        print(f"  {blocks:3d} workgroups ({nbytes / 1e6:6.1f} MB): " + " | ".join(row))
    sys.stdout.flush()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_weights(torch, seed, n_experts, chunk=32):
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_mxfp4_fused as qf
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    p1 = torch.empty((n_experts, 2 * I, H // 2), dtype=torch.uint8, device="cuda")
    s1 = torch.empty((n_experts, 2 * I, H // 32), dtype=torch.uint8, device="cuda")
    p2 = torch.empty((n_experts, H, I // 2), dtype=torch.uint8, device="cuda")
    s2 = torch.empty((n_experts, H, I // 32), dtype=torch.uint8, device="cuda")
    for e0 in range(0, n_experts, chunk):
        e1 = min(n_experts, e0 + chunk)
        w = (torch.randn((e1 - e0, 2 * I, H), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        p1[e0:e1], s1[e0:e1] = qf.quantize_to_mxfp4(w)
        w = (torch.randn((e1 - e0, H, I), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        p2[e0:e1], s2[e0:e1] = qf.quantize_to_mxfp4(w)
        del w
    t = dgm.transform_mxfp4_weights_for_mega_moe_fused((p1, s1), (p2, s2))
    torch.cuda.synchronize()
    return t, (p1, s1, p2, s2)


def build_qoq_weights(torch, seed, n_experts, chunk=32):
    """The same layer's weights in the QoQ W4A8 format (quantize_to_qoq on the GPU, then the
    fused layout)."""
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_qoq_fused as qq
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    dev = "cuda"

    def alloc(N, K):
        return (torch.empty((n_experts, N, K // 2), dtype=torch.uint8, device=dev),
                torch.empty((n_experts, N, K // 128), dtype=torch.uint8, device=dev),
                torch.empty((n_experts, N, K // 128), dtype=torch.uint8, device=dev),
                torch.empty((n_experts, N), dtype=torch.float32, device=dev))
    q1, q2 = alloc(2 * I, H), alloc(H, I)
    for e0 in range(0, n_experts, chunk):
        e1 = min(n_experts, e0 + chunk)
        for q, (N, K) in ((q1, (2 * I, H)), (q2, (H, I))):
            w = (torch.randn((e1 - e0, N, K), generator=g, device=dev) * 0.02).to(torch.bfloat16)
            for dst, src in zip(q, qq.quantize_to_qoq(w)):
                dst[e0:e1] = src
            del w
    t = dgm.transform_qoq_weights_for_mega_moe_fused(q1, q2)
    del q1, q2
    torch.cuda.synchronize()
    return t


def build_nvfp4_weights(torch, seed, n_experts, chunk=32):
    """The layer's weights in the NVFP4 W4A4 format (quantize_to_nvfp4 on the GPU, then the
    fused layout)."""
    import hopper_megamoe_basedondeepgemm_amd as dgm
    from hopper_megamoe_basedondeepgemm_amd import quantization_nvfp4 as qn
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    q = []
    for N, K in ((2 * I, H), (H, I)):
        p = torch.empty((n_experts, N, K // 2), dtype=torch.uint8, device="cuda")
        sc = torch.empty((n_experts, N, K // 16), dtype=torch.uint8, device="cuda")
        for e0 in range(0, n_experts, chunk):
            e1 = min(n_experts, e0 + chunk)
            w = (torch.randn((e1 - e0, N, K), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
            p[e0:e1], sc[e0:e1] = qn.quantize_to_nvfp4(w)
            del w
        q.append((p, sc))
    t = dgm.transform_nvfp4_weights_for_mega_moe_fused(q[0], q[1])
    del q
    torch.cuda.synchronize()
    return t


def time_layer(torch, dgm, M, weights, router_w, act, steps, warmup, seed, force_balanced=True, ep_size=1,
               n_experts=E):
    """Times `steps` layer forwards, each between two HIP events on the layer's stream (the
    layer time), then `steps` more with a third event between the frontend and the fused MoE
    kernel for the split between them (an event between two launches delays the second one,
    so the split runs are not used for the layer time)."""
    (t1, t2) = weights
    fused = {"qoq": dgm.qoq_mega_moe_fused, "nvfp4": dgm.fp4_fp4_mega_moe}.get(act, dgm.mxfp4_mega_moe_fused)
    expert_bytes = {"qoq": QOQ_EXPERT_BYTES, "nvfp4": NVFP4_EXPERT_BYTES}.get(act, MXFP4_EXPERT_BYTES)
    # (ep_size > 1: one EP rank's share, experts 0 .. E / ep_size - 1, on this GPU)
    buf = dgm.get_fused_symm_buffer_for_mega_moe(None, n_experts, M, TOPK, H, I, act_format=act, ep_size=ep_size,
                                                 ep_rank=0)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((M, H), generator=g, device="cuda").to(torch.bfloat16)
    y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    flush = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    flush_rd = torch.ones(1 << 28, dtype=torch.float32, device="cuda")

    def evict():
        # >= 1 GiB written, then 1 GiB of other data read: neither the 256 MB MALL nor the
        # L2s hold weights, and no dirty lines of the write are left to be written back
        # inside the timed region
        flush.fill_(1)
        flush_rd.sum()
    stream = torch.cuda.current_stream()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]

    one = False          # (the one-launch layer, DG_ONE_LAUNCH, measures about the same)

    def layer(e=None):
        if e: e[0].record(stream)
        if one:
            dgm.mxfp4_mega_moe_from_bf16(y, x, router_w, t1, t2, buf, force_balanced=force_balanced)
            if e: e[1].record(stream)
        else:
            dgm.fable_router_quant_topk_frontend(x, router_w, buf, force_balanced=force_balanced, select_in_mega=True)
            if e: e[1].record(stream)
            fused(y, t1, t2, buf)
        if e: e[2].record(stream)

    def layer2(e):            # start and end events only
        e[0].record(stream)
        layer()
        e[2].record(stream)

    for _ in range(warmup):
        evict()
        layer()
    torch.cuda.synchronize()
    ev2 = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        evict()
        layer2(ev2[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    us = np.array([e[0].elapsed_time(e[2]) * 1e3 for e in ev2])
    for i in range(steps):
        evict()
        layer(ev[i])
    torch.cuda.synchronize()
    if one:   # (one kernel: the MoE kernel time is the layer time)
        us_fe = np.zeros_like(us)
        us_moe = np.array([e[0].elapsed_time(e[2]) * 1e3 for e in ev])
    else:
        us_fe = np.array([e[0].elapsed_time(e[1]) * 1e3 for e in ev])
        us_moe = np.array([e[1].elapsed_time(e[2]) * 1e3 for e in ev])
    counts = buf.pool_table()[0]
    n_active = int((counts > 0).sum())
    ok = bool(torch.isfinite(y.float()).all()) and buf.kernel_error() == 0
    return dict(us_median=float(np.median(us)), us_min=float(us.min()), fe_us=float(np.median(us_fe)),
                moe_us=float(np.median(us_moe)), moe_us_min=float(us_moe.min()), n_active=n_active,
                weight_bytes=n_active * expert_bytes, finite=ok, wall_s=wall, y=y, x=x, buf=buf)


def copy_calibration(torch, mib, reps=3):
    """A plain device copy of `mib` MiB (read mib, write mib), for scaling HBM counters."""
    a = torch.ones(mib << 18, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()


def host_cpu():
    """(model name, physical cores) of the host, from lscpu."""
    import subprocess
    model, cores, sockets = "unknown", None, 1
    try:
        for ln in subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout.splitlines():
            k, _, v = ln.partition(":")
            k, v = k.strip(), v.strip()
            if k == "Model name":
                model = v
            elif k == "Core(s) per socket":
                cores = int(v)
            elif k == "Socket(s)":
                sockets = int(v)
    except Exception:
        pass
    return model, (cores * sockets if cores else os.cpu_count())


def _dequant_active(packed, experts, workers=16):
    """{expert: (W1, W2) f32} for the given experts, dequantised on a thread pool (the oracle's
    packers; numpy releases the GIL)."""
    import torch
    from concurrent.futures import ThreadPoolExecutor
    from oracle import packers as pk
    sel = torch.tensor(experts, dtype=torch.long, device=packed[0].device)
    p1, s1, p2, s2 = [t.index_select(0, sel).cpu().numpy() for t in packed]
    with ThreadPoolExecutor(max_workers=min(workers, os.cpu_count() or 1)) as ex:
        ws = list(ex.map(lambda i: (pk.dequantize_mxfp4_marlin(p1[i], s1[i]), pk.dequantize_mxfp4_marlin(p2[i], s2[i])),
                         range(len(experts))))
    return dict(zip(experts, ws))


def cpu_baseline_and_parity(packed, headline, router_w, M, act, reps=400):
    """The oracle (oracle/moe.py, numpy fp32) on the headline step's own inputs (its bf16 hidden
    states, router weights and packed weights, forced-balanced routing): the step's parity (top-k
    and activation codes bit-exact, y against the oracle's y: min per-row cos, rel-RMSE), and the
    oracle layer timed on the host (router + top-8 + cast, then every expert route with the active
    experts' weights dequantised beforehand, as the reference's CPU path does; median of `reps`).
    Returns (cpu_baseline dict, parity dict)."""
    from oracle import moe
    x = headline["x"].float().cpu().numpy()
    rw = router_w.float().cpu().numpy()
    buf = headline["buf"]
    logits = moe.router_logits_f32(x, rw)
    idx, w = moe.balanced_routing(M, E, TOPK)
    codes, sfb, x_dq = moe.quant_act(x, act)
    experts = sorted({int(v) for v in idx.ravel()})
    pre = _dequant_active(packed, experts)
    W1, W2 = _Sel(pre, 0, (E, 2 * I, H)), _Sel(pre, 1, (E, H, I))
    ref, _ = moe.moe_forward(x_dq, idx, w, W1, W2, 0, act)
    y = headline["y"].float().cpu().numpy()
    m = moe.metrics(y, ref)
    parity = dict(cos_min=round(m["cos_min"], 7), rel_rmse=round(m["rel_rmse"], 6),
                  topk_bit_exact=bool((buf.topk_idx[:M].cpu().numpy() == idx).all()),
                  codes_bit_exact=bool((buf.x[:M].cpu().numpy() == codes).all() and (buf.x_sf[:M].cpu().numpy() == sfb).all()),
                  gate="cos >= 0.9999 and rel-RMSE <= 0.005",
                  oracle="oracle/moe.py on this step's inputs (A-%s, M=%d, %d active experts)" % (act.upper(), M, len(experts)))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        lg = moe.router_logits_f32(x, rw)
        moe.topk_softmax(lg, TOPK)
        moe.quant_act(x, act)
        moe.moe_forward(x_dq, idx, w, W1, W2, 0, act)
        times.append(time.perf_counter() - t0)
    threads = _blas_threads()
    model, phys = host_cpu()
    cpu = dict(value=round(float(np.median(times)) * 1e6, 1), unit="us/layer", cores=threads, kind="port",
               cpu_model=model, physical_cores=phys,
               sample=f"oracle (numpy fp32) on the headline step's inputs: the whole M={M} layer (router + top-8 + "
                      f"cast, then all {TOPK * M} expert routes with the {len(experts)} active experts' weights "
                      f"dequantised beforehand), median of {reps}; A-{act.upper()}; cores = BLAS threads")
    return cpu, parity


def _blas_threads():
    try:
        from threadpoolctl import threadpool_info
        return max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:
        return 1


def cpu_config_baselines(packed, c0, c1, router_w, reps=60):
    """The oracle timed on the host at BASELINE's configs 0 and 1, on the inputs of the GPU runs of
    the same configs (their bf16 hidden states; the same packed weights, experts 0-47):
      c0: E=48 (router weight = rows 0-47 of the 384-way one), M=2, softmax top-8, A-MXFP4;
      c1: one EP rank's share of the 384-way layer, M=8 forced-balanced, A-MXFP4 (the 384-way
          router for this rank's tokens, then its 8 local routes).
    Per forward: router GEMV + top-8 + activation cast + the local routes (the routed experts'
    weights dequantised beforehand); median of `reps`. Returns {name: dict}."""
    from oracle import moe
    out = {}
    rw = router_w.float().cpu().numpy()
    for name, r, rwn, balanced in (("c0_E48_M2_mxfp4", c0, rw[:48], False), ("c1_ep_share_M8_mxfp4", c1, rw, True)):
        if r is None:
            continue
        x = r["x"].float().cpu().numpy()
        M = x.shape[0]
        logits = moe.router_logits_f32(x, rwn)
        idx, w, _ = moe.topk_softmax(logits, TOPK)
        if balanced:
            idx, w = moe.balanced_routing(M, rwn.shape[0], TOPK)
        experts = sorted({int(v) for v in idx.ravel() if 0 <= v < 48})
        pre = _dequant_active(packed, experts)
        W1, W2 = _Sel(pre, 0, (48, 2 * I, H)), _Sel(pre, 1, (48, H, I))
        codes, sfb, x_dq = moe.quant_act(x, "mxfp4")
        ref, _ = moe.moe_forward(x_dq, idx, w, W1, W2, 0, "mxfp4")
        m = moe.metrics(r["y"].float().cpu().numpy(), ref)
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            lg = moe.router_logits_f32(x, rwn)
            moe.topk_softmax(lg, TOPK)
            moe.quant_act(x, "mxfp4")
            moe.moe_forward(x_dq, idx, w, W1, W2, 0, "mxfp4")
            times.append(time.perf_counter() - t0)
        n_routes = int(((idx >= 0) & (idx < 48)).sum())
        out[name] = dict(value=round(float(np.median(times)) * 1e6, 1), unit="us/layer", cores=_blas_threads(),
                         kind="port", gpu_us=round(r["us_median"], 2),
                         gpu_parity=dict(cos_min=round(m["cos_min"], 7), rel_rmse=round(m["rel_rmse"], 6)),
                         sample=f"oracle (numpy fp32): {M} tokens, {n_routes} local routes on {len(experts)} experts, "
                                f"median of {reps}")
    return out


class _Sel:
    """W[e] of pre-dequantised experts (the oracle touches only routed experts)."""

    def __init__(self, pre, i, shape):
        self.pre, self.i, self.shape = pre, i, shape

    def __getitem__(self, e):
        return self.pre[e][self.i]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--m", type=int, default=8, help="M of the headline line")
    ap.add_argument("--act", default="mxfp8", choices=["mxfp8", "mxfp4"], help="activation format of the headline line")
    ap.add_argument("--sweep", default="2,4,8,16",
                    help="M values of the sweep (A-MXFP8, A-MXFP4 and the fused buffer's A-FP8 with fp32 scales per 128)")
    ap.add_argument("--sweep-steps", type=int, default=10)
    ap.add_argument("--no-qoq", action="store_true", help="skip the QoQ W4A8 sweep")
    ap.add_argument("--nvfp4-sweep", default="16,64,128",
                    help="M values of the NVFP4 W4A4 sweep (seeded unbalanced routing); empty = skip")
    ap.add_argument("--no-unbalanced", action="store_true")
    ap.add_argument("--no-c1", action="store_true", help="skip the config 1 line (one EP rank's 48 experts)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--phase-stamps", action="store_true",
                    help="print the fused kernel's per-workgroup phase stamps (M=2/8/16, config 1) and exit")
    ap.add_argument("--probes", action="store_true",
                    help="print the platform probes (HBM read bandwidth of the streaming pattern, empty-kernel "
                         "launch floor) and exit")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="also run a plain device copy of this many MiB (HBM counter scaling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the MegaMoE layer here has no multi-GPU "
                                   "path, so --gpus must be 1"}))
        sys.exit(2)
    import torch
    import hopper_megamoe_basedondeepgemm_amd as dgm
    torch.cuda.set_device(0)
    if args.probes:
        probes_report(torch)
        return
    log("building E384 weights ...")
    weights, packed = build_weights(torch, 1234, E)
    g = torch.Generator(device="cuda")
    g.manual_seed(99)
    if args.phase_stamps:
        router_w0 = (torch.randn((E, H), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        phase_stamps_report(torch, dgm, weights, router_w0)
        return
    router_w = (torch.randn((E, H), generator=g, device="cuda") * 0.02).to(torch.bfloat16)

    def entry(r):
        gbs = r["weight_bytes"] / (r["moe_us"] * 1e-6) / 1e9
        return dict(us=round(r["us_median"], 2), us_min=round(r["us_min"], 2), frontend_us=round(r["fe_us"], 2),
                    moe_us=round(r["moe_us"], 2), active_experts=r["n_active"], weight_MB=round(r["weight_bytes"] / 1e6, 1),
                    moe_weight_GBps=round(gbs, 1), moe_hbm_frac=round(gbs / HBM_PEAK_GBS, 4), ok=r["finite"])

    main_r = time_layer(torch, dgm, args.m, weights, router_w, args.act, args.steps, args.warmup, 500 + args.m)
    log(f"headline M={args.m} {args.act}: {entry(main_r)}")
    sweep = {}
    for act in ("mxfp8", "mxfp4", "fp8f128"):
        sweep[act] = {}
        for M in [int(v) for v in args.sweep.split(",") if v]:
            r = time_layer(torch, dgm, M, weights, router_w, act, args.sweep_steps, args.warmup, 500 + M)
            sweep[act][M] = entry(r)
            log(f"M={M} {act}: {sweep[act][M]}")
    c0_r = c1_r = None
    if not args.no_c1:
        share = tuple(tuple(t[:E // 8] if t is not None else None for t in w) for w in weights)
        # benchmark config 0 on the GPU: 48 experts (all local), a 48-way router (rows 0-47 of the
        # 384-way one), M=2, softmax top-8 routing, W-MXFP4 x A-MXFP4
        c0_r = time_layer(torch, dgm, 2, share, router_w[:E // 8].contiguous(), "mxfp4", args.sweep_steps,
                          args.warmup, 202, force_balanced=False, n_experts=E // 8)
        sweep["c0_E48_M2_mxfp4"] = entry(c0_r)
        log(f"config 0 (E48, M=2, mxfp4, softmax routing): {sweep['c0_E48_M2_mxfp4']}")
        # benchmark config 1: one EP rank's share (local experts 0-47 of the 384-way router),
        # W-MXFP4 x A-MXFP4, M=8 forced-balanced: 8 rows on 8 local experts
        c1_r = time_layer(torch, dgm, 8, share, router_w, "mxfp4", args.sweep_steps, args.warmup, 508, ep_size=8)
        sweep["c1_ep_share_M8_mxfp4"] = entry(c1_r)
        log(f"config 1 (E48 share, M=8, mxfp4): {sweep['c1_ep_share_M8_mxfp4']}")
        del share
    if not args.no_qoq and [v for v in args.sweep.split(",") if v]:
        log("building E384 QoQ weights ...")
        qw = build_qoq_weights(torch, 4321, E)
        sweep["qoq"] = {}
        for M in [int(v) for v in args.sweep.split(",") if v]:
            r = time_layer(torch, dgm, M, qw, router_w, "qoq", args.sweep_steps, args.warmup, 500 + M)
            sweep["qoq"][M] = entry(r)
            log(f"M={M} qoq: {sweep['qoq'][M]}")
        del qw
    nv_ms = [int(v) for v in args.nvfp4_sweep.split(",") if v]
    if nv_ms:
        log("building E384 NVFP4 weights ...")
        nw = build_nvfp4_weights(torch, 5678, E)
        sweep["nvfp4_unbalanced"] = {}
        for M in nv_ms:
            r = time_layer(torch, dgm, M, nw, router_w, "nvfp4", args.sweep_steps, args.warmup, 900 + M,
                           force_balanced=False)
            sweep["nvfp4_unbalanced"][M] = entry(r)
            log(f"M={M} nvfp4 unbalanced: {sweep['nvfp4_unbalanced'][M]}")
        del nw
    if not args.no_unbalanced:
        r = time_layer(torch, dgm, 16, weights, router_w, "mxfp8", args.sweep_steps, args.warmup, 777,
                       force_balanced=False)
        sweep["mxfp8_unbalanced_M16"] = entry(r)
        log(f"unbalanced M=16 mxfp8: {sweep['mxfp8_unbalanced_M16']}")
    if args.copy_calib_mib:
        copy_calibration(torch, args.copy_calib_mib)
    cpu, parity = None, None
    if not args.no_cpu_baseline:
        try:
            t0 = time.perf_counter()
            cpu, parity = cpu_baseline_and_parity(packed, main_r, router_w, args.m, args.act)
            cpu["sample"] += f"; {time.perf_counter() - t0:.1f} s of host time incl. the dequantisation"
            cpu["configs"] = cpu_config_baselines(packed, c0_r, c1_r, router_w)
            log(f"cpu baseline: {cpu}")
            log(f"headline parity: {parity}")
        except Exception as ex:  # reported, never fatal
            cpu = dict(value=None, unit="us/layer", cores=None, kind="port", sample=f"failed: {ex}")
    us = main_r["us_median"]
    moe_us = main_r["moe_us"]
    achieved = main_r["weight_bytes"] / (moe_us * 1e-6) / 1e9
    line = {
        "metric": "us per MoE layer at M=2/4/8/16 (E384 H3072 I1280 top-8); weight HBM GB/s",
        "value": round(us, 2), "unit": "us/layer", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(us / 1e3, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "mxfp4xmxfp8" if args.act == "mxfp8" else "mxfp4xmxfp4",
        "data": "synthetic: seeded randn bf16 weights packed to MXFP4 on the GPU, forced-balanced routing",
        "config": {"workload": f"E384 layer on one GPU (benchmark config 2), W-MXFP4 x A-{args.act.upper()}, "
                               f"M={args.m}, forced-balanced; value = frontend + fused MoE kernel",
                   "M": args.m, "experts": E, "hidden": H, "intermediate": I, "topk": TOPK,
                   "active_experts": main_r["n_active"], "frontend_us": round(main_r["fe_us"], 2),
                   "moe_kernel_us": round(moe_us, 2), "sweep": sweep, "mall_flush_bytes": 1 << 30},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic_bytes() if (args.m == 8 and args.act == "mxfp8") else None,
                     "kernel": "k_megamoe (fused persistent MoE kernel); achieved = active-expert MXFP4 weight "
                               "bytes (6,266,880 B per expert) / median kernel time (HIP events)"},
        "mfma_util": {"value": profiled_mfma_util() if (args.m == 8 and args.act == "mxfp8") else None,
                      "what": "SQ_VALU_MFMA_BUSY_CYCLES / all SIMD cycles of k_megamoe at this workload "
                              "(rocprofv3 counters, profiles/k_megamoe_E384_mfma_valu_counters.txt): the "
                              "layer is HBM-bound, the matrix cores mostly idle"},
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
