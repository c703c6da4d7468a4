import json
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "int8-kvcache_amd"), REPO, os.path.join(REPO, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")


def record(test, **metrics):
    """Append metrics to $OUT/test_metrics.jsonl (as the reference's tests/conftest.py:15-20 does),
    so runs leave numbers, not just PASS."""
    out = os.environ.get("OUT")
    if out:
        os.makedirs(out, exist_ok=True)
        with open(os.path.join(out, "test_metrics.jsonl"), "a") as f:
            f.write(json.dumps({"test": test, **metrics}) + "\n")


def q_code_flips(c):
    """[T, Hq] bool for a golden case: rows whose q codes differ between the kernel's fp32 q arithmetic
    (q' = fl32(q * s_k), fp32 scale and quotient) and int8_ref's fp64 one (kvq/int8_ref.py:108-115 with
    kvq/quant.py:46-51): bf16 q puts quotients on exact rounding ties, which the two break differently."""
    import torch
    from oracle import kvq_oracle as O

    q, ks = c["q"], c["static"]["k_scale"]
    ksr = ks.repeat_interleave(q.shape[1] // ks.shape[0], 0)  # [Hq, D | 1]
    per_channel = ks.shape[-1] > 1
    codes = []
    for dt in (torch.float32, torch.float64):
        x = q.to(dt) * ksr.to(dt) if per_channel else q.to(dt)
        codes.append(O.quantize(x, O.scale_from_absmax(x.abs().amax(-1, keepdim=True))))
    return (codes[0] != codes[1]).any(-1)


def nan_like(t):
    """An output buffer that starts as NaN, so a row a kernel fails to write cannot pass a check."""
    import torch
    return torch.full_like(t, float("nan"))


def nan_segm(T, H, S, D, device="cuda"):
    """Split-KV partial buffers (segm_out [T, H, S, D], segm_max / segm_sum [T, H, S]) filled with NaN:
    a piece that is merged but never written shows up in the output."""
    import torch
    nan = float("nan")
    return (torch.full((T, H, S, D), nan, device=device), torch.full((T, H, S), nan, device=device),
            torch.full((T, H, S), nan, device=device))


@pytest.fixture(scope="session")
def golden():
    from safetensors.torch import load_file

    d = os.path.join(REPO, "tests", "golden")
    with open(os.path.join(d, "golden.json")) as f:
        meta = json.load(f)
    return load_file(os.path.join(d, "golden.safetensors")), meta
