"""Build the HIP libraries of the package in-tree with hipcc for gfx950.

Each library is one ``hipcc -shared`` over its sources in ``csrc/``; the output
``.so`` sits next to this file and is what ``_lib.py`` loads.
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ARCH = os.environ.get("MSD_OFFLOAD_ARCH", "gfx950")

# Packed FP32 VALU ops are disabled for all device code (compiler flag, device pass only).
HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-Wno-unused-command-line-argument"]

LIBS = {
    "libmsdecode.so": ["csrc/msdecode.hip", "csrc/sample.hip", "csrc/prefill.hip", "csrc/batched.hip",
                       "csrc/xent.hip"],
}


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose=False):
    cc = hipcc()
    for lib, srcs in LIBS.items():
        out = os.path.join(HERE, lib)
        tmp = out + ".tmp"
        cmd = [cc, *HIPCC_FLAGS, "-o", tmp, *[os.path.join(HERE, s) for s in srcs]]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError(f"hipcc failed for {lib}")
        os.replace(tmp, out)
    return [os.path.join(HERE, lib) for lib in LIBS]


if __name__ == "__main__":
    for p in build(verbose=True):
        print("built", p)
