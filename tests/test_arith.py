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


def test_division_free_codes_match_ieee_codes(tmp_path):
    """The cache write's and the q quantization's codes (code_magic): q = clamp(fl(x * y), +-254) with
    y = fl(1 / s), f = fma(fma(-q, s, x), y, q), t = clamp(fl(f + 1.5 * 2^23), +-127) give
    clamp(rint(fl(x / s)), +-127) bit for bit: every bf16 but NaN (infinities included), 2^20 random
    fp32 x and fp32 x on and within 4 ulps of half-integer quotients, 2400 scales (a third of them
    bf16 absolute maxima / 127, a third putting a chosen x exactly on a tie)."""
    rc, out = _run_c(tmp_path, "quant_exact_check")
    assert rc == 0 and out.endswith("mismatched 0"), out
