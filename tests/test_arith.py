"""Host-side proofs for arithmetic shortcuts inside the HIP kernels, checked over every input they can
see (IEEE fp32 behaves the same on the host and on gfx950 for these operations: round-to-nearest-even
multiply and fused multiply-add, no denormals in the ranges involved)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _run_c(tmp_path, name):
    exe = str(tmp_path / name)
    src = os.path.join(HERE, "arith", name + ".c")
    subprocess.run(["gcc", "-O2", "-march=native", "-fopenmp", "-ffp-contract=off", src, "-o", exe, "-lm"], check=True)
    res = subprocess.run([exe], capture_output=True, text=True)
    return res.returncode, res.stdout.strip()


def test_div127_is_ieee_division_on_all_tile_maxima(tmp_path):
    """attn_kernel's ps = max(div127(pm), 1e-30): the two-FMA quotient equals fl(pm / 127) for all
    2^30 floats pm in [2^-126, 1] (smaller pm give ps = 1e-30 either way, as pm / 127 < 1e-30)."""
    rc, out = _run_c(tmp_path, "div127_check")
    assert rc == 0 and out.endswith("mismatched 0"), out
