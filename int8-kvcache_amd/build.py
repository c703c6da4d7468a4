"""Build the in-tree HIP library libkvq_int8.so for gfx950 (hipcc, no JIT cache).

Run as a script (python int8-kvcache_amd/build.py) or through __graft_entry__.build(). The library
lands next to this file's kvq/ package so that it travels with the source tree.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc", "kvq_int8.hip")
OUT = os.path.join(HERE, "kvq", "libkvq_int8.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",                               # every fma in the kernels is written out
    "-fhip-fp32-correctly-rounded-divide-sqrt",        # x / s is IEEE division (bit-exact codes)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",             # MFMA results in VGPRs (no v_accvgpr_read copies)
]


def build(verbose=False):
    tmp = OUT + ".tmp"
    cmd = [HIPCC, *FLAGS, SRC, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
