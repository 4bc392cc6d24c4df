"""Build the in-tree HIP library ``libadafactor8bit_amd.so`` for gfx950.

    python adafactor-8bit_amd/build.py            # compile (always rebuilds)

The library is plain C ABI (include/adafactor8bit_amd.h); no torch headers are
needed, so the build is a few hipcc invocations with explicit flags:
  -ffp-contract=off                        no silent FMA contraction: the kernels
                                           place every fma the reference's CPU
                                           arithmetic performs explicitly
  -fhip-fp32-correctly-rounded-divide-sqrt IEEE '/' and sqrtf where used
  -fno-gpu-flush-denormals-to-zero         keep subnormals (clamp(min=1e-38))
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed fp32 VALU ops
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "adafactor8bit", "libadafactor8bit_amd.so")
SOURCES = ["a8_abi.cpp", "a8_update1d.hip", "a8_update1d_k.hip", "a8_full1d.hip", "a8_factored.hip", "a8_apollo.hip",
           "a8_decode.hip", "a8_sgd.hip", "a8_prims.hip", "a8_apollo_x.hip", "a8_step.hip"]
LIBS = ["-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib"]
ARCH = os.environ.get("A8_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
         "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]


def sources():
    return [os.path.join(CSRC, s) for s in SOURCES]


def build(verbose: bool = True) -> str:
    objs = []
    bdir = os.path.join(HERE, "_build")
    os.makedirs(bdir, exist_ok=True)
    procs = []
    for src in sources():
        obj = os.path.join(bdir, os.path.basename(src) + ".o")
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        cmd = [HIPCC] + FLAGS + lang + ["-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((subprocess.Popen(cmd), src))
        objs.append(obj)
    for p, src in procs:
        if p.wait() != 0:
            raise RuntimeError(f"hipcc failed on {src}")
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", tmp] + objs + LIBS
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.check_call(cmd)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
    print("built", OUT)
