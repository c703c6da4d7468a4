"""KVQ_DEBUG_DUMP (kvq.debug_dump): the long path's prefill call saved for an offline replay, as the
reference's dump of its FlashAttention call (kvq/cuda_kernels.py:123-127) and scripts/replay_fa_call.py.

On the CPU: a dump of a mixed batch's call loads without unpickling code, its host-side bounds report is
clean, and replaying it through the oracle -- fp32 attention over the temporary cache its block table
describes, filled by the oracle's page dequantization -- reproduces implementation A on the original INT8
cache for every row the work list covers. Corrupted dumps (a table entry past the temporary cache, a key
count past the copied pages, a work entry past a request's rows, pages of another request) are reported.
On the GPU: the dump written by a real paged_attention call, replayed on the HIP prefill kernel, against
the oracle on the replay's tensors.
"""
import os

import pytest
import torch
from conftest import record

from oracle import kvq_oracle as O
from kvq import cuda_kernels as ck
from kvq import debug_dump
from kvq import synth

ROWS = 128   # (token, q head) rows per work-list entry of the prefill kernel


def _batch(hq=28, hkv=4, d=128):
    q_lens, seq_lens = [1, 40, 3, 200, 1, 77], [100, 90, 300, 900, 17, 1500]
    c = synth.paged_case(hq, hkv, q_lens, seq_lens, head_dim=d, seed=91, dist="randn", scale=3.0)
    c["static"] = synth.scales_from(c["k"].reshape(-1, hkv, d), c["v"].reshape(-1, hkv, d))
    c["scale"] = d ** -0.5
    kq = O.quantize(c["k"].float() - c["static"]["k_mu"], c["static"]["k_scale"])
    vq = O.quantize(c["v"], c["static"]["v_scale"])
    return c, kq, vq


def oracle_replay(d, q, kt, vt):
    """The dumped call under the oracle: fp32 attention (paged_attention_ref) over the temporary cache for
    the requests the work list names; [T, Hq, D] with NaN on the other rows."""
    cu, sl, bt = d["cu_seqlens_q"], d["seq_lens"], d["block_table"]
    out = torch.full(q.shape, float("nan"))
    for r in sorted(set(d["tile_req"].tolist())):
        t0, t1 = int(cu[r]), int(cu[r + 1])
        cu_r = torch.tensor([0, t1 - t0], dtype=torch.int32)
        out[t0:t1] = O.paged_attention_ref(q[t0:t1].cpu().float(), kt.cpu(), vt.cpu(), cu_r, sl[r:r + 1], bt[r:r + 1],
                                           d["softmax_scale"]).float()
    return out


def _dump(tmp_path, c, kq, vq):
    plan = ck.plan_long(c["cu"], c["seq_lens"], 16)
    hq, hkv = c["q"].shape[1], c["k"].shape[2]
    tile_req, tile_row = plan.tiles(hq // hkv, "cpu", rows=ROWS)
    kt, vt = O.dequant_pages_ref(kq, vq, c["block_table"], torch.from_numpy(plan.src_req), torch.from_numpy(plan.src_j),
                                 c["static"])
    out = torch.empty_like(c["q"])
    path = str(tmp_path / "long_call.pt")
    debug_dump.dump_long_call(path, c["q"], out, c["cu"], c["seq_lens"], plan, kt, tile_req, tile_row,
                              int((c["cu"][1:] - c["cu"][:-1]).max()), ROWS, c["scale"])
    return path, plan, kt, vt


def test_dump_replays_through_the_oracle(tmp_path):
    c, kq, vq = _batch()
    path, plan, kt, vt = _dump(tmp_path, c, kq, vq)
    d = debug_dump.load(path)
    assert debug_dump.check(d) == []
    assert d["q_shape"] == tuple(c["q"].shape) and d["kt_shape"] == tuple(kt.shape)
    assert d["max_seqlen_k"] == 1500 and d["block_size"] == 16
    rep = oracle_replay(d, c["q"], kt, vt)
    ref = O.paged_static_attention(O.CFG32_Q32, c["static"], True, ck.SHORT_Q)(
        c["q"].float(), kq, vq, c["cu"], c["seq_lens"], c["block_table"], c["scale"])
    rows = torch.cat([torch.arange(int(c["cu"][r]), int(c["cu"][r + 1])) for r in plan.long_req.tolist()])
    e = O.compare(ref[rows], rep[rows])
    record("debug_dump_oracle_replay", **e)
    assert e["rel_l2"] < 1e-5, e
    covered = torch.zeros(c["q"].shape[0], dtype=torch.bool)
    covered[rows] = True
    assert torch.isnan(rep[~covered]).all() and not torch.isnan(rep[covered]).any()


@pytest.mark.parametrize("fault", ["page_past_cache", "keys_past_pages", "rows_past_request", "foreign_page"])
def test_check_reports_corrupted_dumps(tmp_path, fault):
    c, kq, vq = _batch()
    path, plan, kt, vt = _dump(tmp_path, c, kq, vq)
    d = debug_dump.load(path)
    r = int(plan.long_req[0])
    if fault == "page_past_cache":
        d["block_table"][r, 0] = kt.shape[0]
    elif fault == "keys_past_pages":
        d["seq_lens"][r] = 16 * d["block_table"].shape[1] + 1
    elif fault == "rows_past_request":
        i = int((d["tile_req"] == r).nonzero()[0])
        d["tile_row"][i] = 10 ** 6
    else:
        other = int(plan.long_req[1])
        d["block_table"][r, 0] = d["block_table"][other, 0]
    errs = debug_dump.check(d)
    assert errs and all(f"req {r}" in e for e in errs), errs


@pytest.mark.gpu
def test_dump_of_a_real_call_replays_on_the_gpu(tmp_path, monkeypatch):
    """KVQ_DEBUG_DUMP set around a mixed-batch paged_attention call: the dump is written, its bounds report
    is clean, and the replay on the HIP prefill kernel (random tensors, the dumped metadata) matches the
    oracle on those tensors for every covered row (the reference's long-row bar, rel_l2 < 1e-2, and
    max-abs 2e-2); the replay leaves the other rows untouched."""
    c, kq, vq = _batch()
    path = str(tmp_path / "real_call.pt")
    monkeypatch.setenv("KVQ_DEBUG_DUMP", path)
    plan = ck.plan_long(c["cu"], c["seq_lens"], 16)
    dc = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in c.items()}
    st = {k: v.cuda() for k, v in c["static"].items()}
    ck.paged_attention(dc["q"], kq.cuda(), vq.cuda(), torch.empty_like(dc["q"]), dc["cu"], dc["seq_lens"],
                       dc["block_table"], 200, c["scale"], st, plan)
    torch.cuda.synchronize()
    assert os.path.exists(path)
    d = debug_dump.load(path)
    assert debug_dump.check(d) == []
    q, kt, vt, out = debug_dump.replay(d, seed=3)
    torch.cuda.synchronize()
    ref = oracle_replay(d, q, kt, vt)
    cov = ~torch.isnan(ref[:, 0, 0])
    e = O.compare(ref[cov], out.cpu()[cov])
    record("debug_dump_gpu_replay", **e)
    assert e["rel_l2"] < 1e-2 and e["max_abs"] <= 2e-2, e
    assert torch.isnan(out.cpu()[~cov].float()).all()
