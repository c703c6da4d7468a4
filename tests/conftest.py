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
