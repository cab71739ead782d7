"""Build the HIP shared library libdgm_megamoe.so in-tree for gfx950 (hipcc, ahead of time)."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libdgm_megamoe.so")
SOURCES = ["dgm_megamoe.hip", "dgm_fused.hip", "dgm_packers.hip", "dgm_probe.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # packed-fp32 VALU forms are kept out of every kernel (see the module docs)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # no wave-level rewriting of atomics: the fused kernel's work-claim atomics return values
    # that are consumed a whole work item later, and the rewrite (reduce + broadcast) would
    # consume them at once, i.e. wait for every weight tile still in flight
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-I" + os.path.join(os.path.dirname(HERE), "include"),
]


def build(verbose=False):
    tmp = LIB + ".tmp"
    cmd = [HIPCC] + FLAGS + [os.path.join(CSRC, s) for s in SOURCES] + ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{errs}")
    if verbose and errs:
        print(errs)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
