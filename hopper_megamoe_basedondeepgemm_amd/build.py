"""Build the HIP shared library libdgm_megamoe.so in-tree for gfx950 (hipcc, ahead of time).

Each source is compiled to an object file in its own hipcc process (in parallel), then the
objects are linked into the shared library."""
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libdgm_megamoe.so")
SOURCES = ["dgm_megamoe.hip", "dgm_fused.hip", "dgm_packers.hip", "dgm_probe.hip", "dgm_noalloc.hip"]
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
    tmp = LIB + ".tmp"
    with tempfile.TemporaryDirectory(prefix="dgm_build_") as td:
        objs = [os.path.join(td, os.path.splitext(s)[0] + ".o") for s in SOURCES]
        cmds = [[HIPCC] + FLAGS + ["-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(SOURCES, objs)]
        if verbose:
            for c in cmds:
                print(" ".join(c), flush=True)
        with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
            results = list(ex.map(_run, cmds))
        for (rc, errs), src in zip(results, SOURCES):
            if rc != 0:
                raise RuntimeError(f"hipcc failed on {src} ({rc}):\n{errs}")
            if verbose and errs:
                print(errs)
        rc, errs = _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + objs + ["-o", tmp])
        if rc != 0:
            raise RuntimeError(f"link failed ({rc}):\n{errs}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
