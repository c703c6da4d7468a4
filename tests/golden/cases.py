"""Definitions of the seeded parity cases shared by the golden-vector script and the tests.

Inputs are regenerated from numpy PCG64 seeds (kvq/synth.py), so the fixtures hold only outputs and
checksums. Shapes follow the reference's test cases (tests/conftest.py:69-88) and BASELINE config c0.
"""
import importlib.util
import os

import torch

_SYNTH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "..", "int8-kvcache_amd", "kvq", "synth.py")
_spec = importlib.util.spec_from_file_location("kvq_synth_golden", _SYNTH)
synth = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(synth)

SHORT = ([2, 4, 8, 3, 1, 5, 7, 1, 6], [40, 700, 1029, 8, 2047, 96, 3000, 15, 512])
MIXED = ([1, 1, 7, 33, 128, 1, 300, 9, 4], [600, 31, 7, 500, 128, 1500, 900, 2000, 64])
EDGE = ([1, 1, 1, 8, 3, 2, 1], [1, 33, 16, 8, 49, 2, 32])


def _cache_static(case, per_channel=True):
    hkv, d = case["k"].shape[2], case["k"].shape[3]
    return synth.scales_from(case["k"].reshape(-1, hkv, d), case["v"].reshape(-1, hkv, d), per_channel, True)


def build(name):
    """Returns dict(q, k, v, cu, seq_lens, block_table, static, per_channel, scale) on the CPU."""
    if name in ("c0_pc", "c0_ph"):
        c = synth.c0_case(per_channel=name == "c0_pc")
        c["per_channel"] = name == "c0_pc"
    elif name == "c0_pc_nomu":
        # config c0 as BASELINE.json states it: static per-channel scales, k_mu = 0 (no smooth-K)
        c = synth.c0_case(per_channel=True, smooth=False)
        c["per_channel"] = True
    elif name in ("short_28_4", "short_14_2_d64", "short_32_8_ph"):
        hq, hkv, d = {"short_28_4": (28, 4, 128), "short_14_2_d64": (14, 2, 64), "short_32_8_ph": (32, 8, 128)}[name]
        c = synth.paged_case(hq, hkv, *SHORT, head_dim=d, seed=21, dist="randn", scale=3.0)
        c["per_channel"] = name != "short_32_8_ph"
        c["static"] = _cache_static(c, c["per_channel"])
    elif name == "edge":
        c = synth.paged_case(28, 4, *EDGE, seed=23, params=synth.channel_params(4, 128))
        c["per_channel"] = True
        c["static"] = synth.calibration_scales(4, 128, synth.channel_params(4, 128))
    elif name == "mixed":
        c = synth.paged_case(28, 4, *MIXED, seed=25, dist="randn", scale=3.0)
        c["per_channel"] = True
        c["static"] = _cache_static(c)
    else:
        raise KeyError(name)
    c["scale"] = c["q"].shape[-1] ** -0.5
    return c


NAMES = ["c0_pc", "c0_pc_nomu", "c0_ph", "short_28_4", "short_14_2_d64", "short_32_8_ph", "edge", "mixed"]
WITH_BF16_REF = ["c0_pc", "c0_pc_nomu", "c0_ph", "short_28_4", "mixed"]
# cases also stored with q scales per 32 channels (int8_ref Cfg(q_gran="group32"), per-channel K)
WITH_QGROUP32 = ["c0_pc", "short_28_4", "short_14_2_d64", "mixed"]


def stored_rows(name, cu):
    """Query rows whose outputs the fixture keeps: all of them, except in "mixed", where each long
    request keeps its first 2 and last 8 rows (the last rows see the whole context)."""
    rows = []
    cu = [int(x) for x in cu.tolist()]
    for r in range(len(cu) - 1):
        a, b = cu[r], cu[r + 1]
        if name != "mixed" or b - a <= 10:
            rows += list(range(a, b))
        else:
            rows += [a, a + 1] + list(range(b - 8, b))
    return torch.tensor(rows, dtype=torch.long)


def quant_special():
    """Inputs that exercise the code formula's corner cases: exact ties, saturation, tiny values."""
    g = synth.rng(31)
    ties = torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5, 127.4999, 127.5, -127.5, 128.0, -128.0,
                         200.0, -1e6, 0.0, -0.0, 1e-30, -1e-30, 63.5, 64.5], dtype=torch.float32)
    rnd = torch.from_numpy(g.standard_normal(4096).astype("float32")) * 60.0
    x = torch.cat([ties, rnd])
    s_ties = torch.ones_like(ties)
    s_rnd = torch.from_numpy(g.uniform(0.01, 2.0, 4096).astype("float32"))
    return x, torch.cat([s_ties, s_rnd])
