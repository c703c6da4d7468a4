"""The attention's tuning variables (KVQ_PREFETCH, KVQ_LDS_RING, KVQ_LDS_PREFETCH, KVQ_V32_KSPLIT,
KVQ_V32_RING, KVQ_XCD_ORDER, KVQ_SEG_COST, KVQ_KSPLIT): each value the library accepts changes only how
the work is scheduled -- ring depths, key splits, the stream-K partition, the workgroup order -- so every
setting must give the oracle's result (implementation B, kvq/int8_ref.py) at the strict bar. The variables
are read at every call. Three batches reach the three instantiations they steer: decode rows (the register
ring of attn_kernel), 3-token queries (21 rows per kv head: the shared LDS ring of attn_kernel) and 8-token
verification rows (56 rows: verify_kernel); each with the split buffers (pieces cut and merged) and
without (one pass)."""
import os

import pytest
import torch
from conftest import nan_like, nan_segm

from kvq import cuda_kernels as ck
from kvq import synth
from test_gpu_kernels import check_attention, dev, int8_cache, oracle_attention

pytestmark = pytest.mark.gpu

LENS = [4100, 33, 1, 517, 2048, 90, 1200, 16, 3000, 700]
_CASES = {}


def _case(q_len, d):
    """A batch of 10 requests of q_len query tokens (28 / 4 heads, or 14 / 2 at d64), its INT8 cache and
    the oracle's output (computed once per batch)."""
    key = (q_len, d)
    if key not in _CASES:
        hq, hkv = (28, 4) if d == 128 else (14, 2)
        params = synth.channel_params(hkv, d)
        c = synth.paged_case(hq, hkv, [q_len] * len(LENS), [max(L, q_len) for L in LENS], head_dim=d,
                             seed=700 + 10 * q_len + d, params=params)
        c["static"] = synth.calibration_scales(hkv, d, params)
        c["scale"] = d ** -0.5
        kq, vq = int8_cache(c)
        _CASES[key] = (c, kq, vq, oracle_attention(c, kq, vq))
    return _CASES[key]


KNOBS = ([("KVQ_PREFETCH", v) for v in ("2", "3", "4", "6", "8")]
         + [("KVQ_LDS_RING", "0")]
         + [("KVQ_LDS_PREFETCH", v) for v in ("3", "4", "6")]
         + [("KVQ_V32_KSPLIT", v) for v in ("1", "2")]
         + [("KVQ_V32_RING", v) for v in ("2", "3", "4")]
         + [("KVQ_XCD_ORDER", "0")]
         + [("KVQ_SEG_COST", v) for v in ("0", "1", "64")]
         + [("KVQ_KSPLIT", v) for v in ("2", "4")])


@pytest.mark.parametrize("q_len", [1, 3, 8])
@pytest.mark.parametrize("knob,value", KNOBS)
def test_tuning_variables_keep_the_result(knob, value, q_len, monkeypatch):
    c, kq, vq, ref = _case(q_len, 128)
    d = dev(c)
    T = d["q"].shape[0]
    monkeypatch.setenv(knob, value)
    for segm in (False, True):
        out = ck.decode_attention(d["q"], dev(kq), dev(vq), nan_like(d["q"]), d["cu"], d["seq_lens"], d["block_table"],
                                  c["scale"], d["static"], segm=nan_segm(T, 28, 16, 128) if segm else None,
                                  max_query_len=q_len)
        assert torch.isfinite(out.float()).all(), (knob, value, q_len, segm)
        check_attention(ref, out, "tuning_knob", knob=knob, value=value, q_len=q_len, segm=segm)


@pytest.mark.parametrize("value", ["2", "3", "4"])
@pytest.mark.parametrize("q_len", [1, 3])
def test_register_ring_depths_d64(value, q_len, monkeypatch):
    """head_dim 64 is instantiated for ring depths 2, 3 and 4."""
    c, kq, vq, ref = _case(q_len, 64)
    d = dev(c)
    T = d["q"].shape[0]
    monkeypatch.setenv("KVQ_PREFETCH", value)
    for segm in (False, True):
        out = ck.decode_attention(d["q"], dev(kq), dev(vq), nan_like(d["q"]), d["cu"], d["seq_lens"], d["block_table"],
                                  c["scale"], d["static"], segm=nan_segm(T, 14, 16, 64) if segm else None,
                                  max_query_len=q_len)
        check_attention(ref, out, "tuning_knob_d64", value=value, q_len=q_len, segm=segm)
