"""Builds libfst_hip.so (gfx950) in-tree with hipcc.

Usage: python -m fastar_amd.build   (or fastar_amd.build.build_lib()).
The library lands in fastar_amd/lib/ so it travels with the source tree.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libfst_hip.so")

SOURCES = ["fst_moe.hip", "fst_gemv.hip", "fst_accept.hip", "fst_hc.hip", "fst_dense.hip", "fst_synth_dev.hip", "fst_api.cpp", "fst_bank.cpp", "fst_layout.cpp", "fst_synth.cpp"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-result",
    "-Wno-unused-value",
    # packed fp32 VALU ops are disabled for correctness on these boxes
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# per-source flags.  fst_moe.hip: no wave-aggregated expansion of atomics.
# Its global atomics run on one lane (its LDS atomics have per-lane addresses,
# which the expansion does not combine), and the expansion reads the returned
# value at once, so the fused launch's work claim (whose value is used one
# super-block later) would wait there for every load in flight, the weight
# prefetch included.
EXTRA_FLAGS = {
    "fst_moe.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def _hipcc():
    for c in ("/opt/rocm/bin/hipcc", "hipcc"):
        if os.path.sep not in c or os.path.exists(c):
            return c
    return "hipcc"


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), out))
    return out


def build_lib(verbose=False):
    os.makedirs(LIBDIR, exist_ok=True)
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = []
    for src in SOURCES:
        obj = os.path.join(objdir, src.replace(".", "_") + ".o")
        cmd = [_hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
        out = _run(cmd)
        if verbose and out.strip():
            print(out)
        objs.append(obj)
    tmp = LIB + ".tmp"
    _run([_hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


def build_oracle():
    script = os.path.join(ROOT, "oracle", "build.sh")
    _run(["bash", script])
    return os.path.join(ROOT, "oracle", "_build", "libfst_oracle.so")


if __name__ == "__main__":
    print(build_lib(verbose="-v" in sys.argv))
    print(build_oracle())
