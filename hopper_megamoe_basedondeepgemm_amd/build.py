"""Build the HIP shared libraries in-tree for gfx950 (hipcc, ahead of time): libdgm_megamoe.so
(the layer) and libdgm_probe.so (the tests' lane-layout probes).

Each source is compiled to an object file in its own hipcc process (in parallel), then the
objects are linked into their shared library."""
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libdgm_megamoe.so")
PROBE_LIB = os.path.join(HERE, "libdgm_probe.so")
SOURCES = ["dgm_megamoe.hip", "dgm_fused.hip", "dgm_packers.hip", "dgm_noalloc.hip"]
PROBE_SOURCES = ["dgm_probe.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # packed-fp32 VALU forms are kept out of every kernel (see the module docs)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # no wave-level rewriting of atomics: the fused kernel's work-claim atomics return values
    # that are consumed a whole work item later, and the rewrite (reduce + broadcast) would
    # consume them at once, i.e. wait for every weight tile still in flight
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-I" + os.path.join(os.path.dirname(HERE), "include"),
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l and l.strip())
    return r.returncode, errs


def build(verbose=False):
    srcs = SOURCES + PROBE_SOURCES
    with tempfile.TemporaryDirectory(prefix="dgm_build_") as td:
        objs = {src: os.path.join(td, os.path.splitext(src)[0] + ".o") for src in srcs}
        cmds = [[HIPCC] + FLAGS + ["-c", os.path.join(CSRC, src), "-o", objs[src]] for src in srcs]
        if verbose:
            for c in cmds:
                print(" ".join(c), flush=True)
        with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
            results = list(ex.map(_run, cmds))
        for (rc, errs), src in zip(results, srcs):
            if rc != 0:
                raise RuntimeError(f"hipcc failed on {src} ({rc}):\n{errs}")
            if verbose and errs:
                print(errs)
        for lib, group in ((LIB, SOURCES), (PROBE_LIB, PROBE_SOURCES)):
            tmp = lib + ".tmp"
            rc, errs = _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + [objs[g] for g in group] + ["-o", tmp])
            if rc != 0:
                raise RuntimeError(f"link of {os.path.basename(lib)} failed ({rc}):\n{errs}")
            os.replace(tmp, lib)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
