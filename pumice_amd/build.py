"""Build recipe of the gfx950 sampler library (pumice_amd/libpumice_sampler.so:
the sampler and the LM head).

hipcc cross-compiles for gfx950 without a GPU.  Flags:
  -ffp-contract=off                        no fused multiply-add except where the
                                           source writes fmaf, so the GPU rounds
                                           exactly like the CPU restatement
  -fhip-fp32-correctly-rounded-divide-sqrt IEEE division for the penalty t/rep
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                           no v_pk_*_f32 instructions
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libpumice_sampler.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_SOURCES = ["pss_sampler.hip", "plh_lmhead.hip", "plh_pack.hip"]
C_SOURCES = ["pss_generate.c"]
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]
C_FLAGS = ["-O2", "-fPIC", "-std=c11", "-ffp-contract=off", "-Wall", "-Wextra"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        l for l in (res.stdout + res.stderr).splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in l
    )
    if res.returncode != 0:
        raise RuntimeError("build failed:\n" + " ".join(cmd) + "\n" + out)
    if verbose and out.strip():
        print(out, flush=True)


def build(verbose=False):
    """Compile every source into pumice_amd/libpumice_sampler.so (always rebuilds)."""
    objs = []
    try:
        for src in C_SOURCES:
            obj = os.path.join(CSRC, src[:-2] + ".o")
            _run(["gcc", *C_FLAGS, "-I" + INCLUDE, "-I" + CSRC, "-c", os.path.join(CSRC, src),
                  "-o", obj], verbose)
            objs.append(obj)
        for src in HIP_SOURCES:
            obj = os.path.join(CSRC, src[:-4] + ".o")
            _run([HIPCC, *HIP_FLAGS, "-I" + INCLUDE, "-I" + CSRC, "-c", os.path.join(CSRC, src),
                  "-o", obj], verbose)
            objs.append(obj)
        tmp = LIB + ".tmp"
        _run([HIPCC, "--offload-arch=gfx950", "--hip-link", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
        os.replace(tmp, LIB)
    finally:
        for o in objs:
            if os.path.exists(o):
                os.remove(o)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
