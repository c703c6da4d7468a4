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


def test_quant_cache_rounding_shortcut_matches_ieee_codes(tmp_path):
    """quant_cache's codes: t = fma(x, r, 1.5 * 2^23), e = fma(x, r, -(t - 1.5 * 2^23)) with r within
    1 ulp of 1/s give clamp(rint(fl(x / s)), +-127) whenever |e| < 0.5 - 2^-14 (the kernel's exact
    pass covers the rest): every finite bf16 and 2^20 random fp32 x, 2000 scales (a quarter of them
    putting some x exactly on a tie), r at RN(1/s) and one ulp either side."""
    rc, out = _run_c(tmp_path, "quant_round_check")
    assert rc == 0 and out.endswith("mismatched 0"), out
