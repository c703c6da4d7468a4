"""The two KVQ_SHORT_Q settings the reference runs besides its default of 8 (kvq/cuda_kernels.py:19-21):

* SHORT_Q = 1 (scripts/ext_specdec.sh:30,41): speculative verification rows (2..8 query tokens) go down the
  long path -- dequant_pages + the bf16 prefill consumer -- while vLLM's host lengths are optimistic upper
  bounds (async speculative decoding assumes every draft was accepted). The reference's long path once
  took those bounds as the key counts and lost accuracy (docs/WALKTHROUGH.md:375-378); here the host
  lengths only size the temporary cache, attention reads the exact lengths on the device.
* SHORT_Q = 1000000 (scripts/stage10_accuracy.sh:14, docs/WALKTHROUGH.md:267): every row, prefill
  included, runs on the INT8 kernel (the teacher-forced NLL of the decode numerics). The kernel takes any
  query length (the reference sizes its m-tiles from max_query_len, kvq/cuda/int8_kv.cu:618-619),
  also beyond 65,535 tokens of one request.

SHORT_Q is read once at import, as in the reference; the tests set the module attribute.
"""
import pytest
import torch
from conftest import nan_like, nan_segm, record

from oracle import kvq_oracle as O
from kvq import cuda_kernels as ck
from kvq import synth
from test_gpu_kernels import check_attention, dev, int8_cache, oracle_attention, short_rows

pytestmark = pytest.mark.gpu


@pytest.fixture
def short_q(monkeypatch):
    def set_to(v):
        monkeypatch.setattr(ck, "SHORT_Q", v)
    return set_to


def test_short_q_1_verification_rows_use_device_lengths(short_q):
    """SHORT_Q=1: requests of 2..8 query tokens take dequant + prefill; the plan is built from host lengths
    16 keys longer than the true ones (pages of rejected drafts, present in the cache and the block table).
    Those rows match implementation A over the true lengths (rel_l2 < 1e-2, the reference's long-row bar,
    tests/test_cuda_kernels.py:119), and on every row where attending to the extra keys would change the
    output by more than 0.1 the kernel is within 2e-2 of the true-length answer. Decode rows (1 token) stay
    on the INT8 kernel (strict bar against B)."""
    short_q(1)
    q_lens = [5, 1, 8, 3, 1, 8, 2, 1, 6]
    true = [700, 300, 2049, 96, 17, 1200, 40, 5000, 333]
    upper = [n + 16 for n in true]
    c = synth.paged_case(28, 4, q_lens, upper, seed=81, dist="randn", scale=3.0)
    c["static"] = synth.scales_from(c["k"].reshape(-1, 4, 128), c["v"].reshape(-1, 4, 128))
    c["scale"] = 128 ** -0.5
    kq, vq = int8_cache(c)
    cfg = O.CFG32_Q32
    run = O.paged_static_attention(cfg, c["static"], True, 1)
    args = (c["q"].float(), kq, vq, c["cu"])
    ref_true = run(*args, torch.tensor(true, dtype=torch.int32), c["block_table"], c["scale"])
    ref_upper = run(*args, c["seq_lens"], c["block_table"], c["scale"])
    plan = ck.plan_long(c["cu"], c["seq_lens"], 16)          # host upper bounds
    assert plan is not None and plan.has_short
    assert plan.max_seqlen_k == max(u for u, n in zip(upper, q_lens) if n > 1)
    dc = dev(c)
    out = ck.paged_attention(dc["q"], dev(kq), dev(vq), nan_like(dc["q"]), dc["cu"],
                             torch.tensor(true, dtype=torch.int32, device="cuda"), dc["block_table"], max(q_lens),
                             c["scale"], dc["static"], plan).cpu()
    long = ~short_rows(c["cu"], 1)
    e = O.compare(ref_true[long], out[long])
    record("short_q_1_long_rows", **e)
    assert e["rel_l2"] < 1e-2, e
    moved = (ref_upper - ref_true).abs().amax(-1)[long] > 0.1     # [rows, heads] the extra keys would change
    assert moved.any(), "the extra keys change no row: the check would not tell the two lengths apart"
    dev_true = (out[long] - ref_true[long]).abs().amax(-1)
    record("short_q_1_moved_rows", rows=int(moved.sum()), max_abs=float(dev_true[moved].max()))
    assert float(dev_true[moved].max()) <= 2e-2
    check_attention(ref_true[~long], out[~long], "short_q_1_decode_rows")


def _sampled_rows_oracle(c, kq, vq, req, tokens):
    """Rows `tokens` of request `req` under implementation B, each as a one-token request whose key count
    is the row's causal limit (L - q_len + 1 + t): B's numerics of a row depend only on the keys it sees,
    its q scale and P tiles aligned at key 0, all of which this keeps."""
    cu = c["cu"]
    t0, ql, L = int(cu[req]), int(cu[req + 1] - cu[req]), int(c["seq_lens"][req])
    q = c["q"][[t0 + t for t in tokens]]
    lens = torch.tensor([L - ql + 1 + t for t in tokens], dtype=torch.int32)
    bt = c["block_table"][req:req + 1].expand(len(tokens), -1).contiguous()
    cu1 = torch.arange(len(tokens) + 1, dtype=torch.int32)
    return O.paged_static_attention(O.CFG32_Q32, c["static"], True, 8)(q.float(), kq, vq, cu1, lens, bt, c["scale"])


@pytest.mark.parametrize("splits", [0, 8])
def test_short_q_large_runs_prefill_on_the_int8_kernel(short_q, splits):
    """SHORT_Q=1000000: a 3,000-token prefill request (q_len = L), a verification request and a decode row in
    one paged_attention call -- no long path, everything on the INT8 kernel (the 32-row kernel, 21,000 rows
    per kv head), without split buffers and with them (prefill rows cut and merged: the merge grid's z
    blocks stride over the request's 3,000 tokens). 24 sampled rows of the prefill request and every row
    of the others against B."""
    short_q(1_000_000)
    q_lens, seq_lens = [3000, 7, 1], [3000, 2100, 900]
    c = synth.paged_case(28, 4, q_lens, seq_lens, seed=83, params=synth.channel_params(4, 128))
    c["static"] = synth.calibration_scales(4, 128, synth.channel_params(4, 128))
    c["scale"] = 128 ** -0.5
    kq, vq = int8_cache(c)
    assert ck.plan_long(c["cu"], c["seq_lens"], 16) is None
    dc = dev(c)
    T = c["q"].shape[0]
    segm = nan_segm(T, 28, splits, 128) if splits else None
    out = ck.paged_attention(dc["q"], dev(kq), dev(vq), nan_like(dc["q"]), dc["cu"], dc["seq_lens"],
                             dc["block_table"], max(q_lens), c["scale"], dc["static"], None, segm).cpu()
    assert torch.isfinite(out.float()).all()
    r = synth.rng(84)
    tokens = sorted({0, 1, 31, 32, 33, 1023, 2047, 2999} | set(int(x) for x in r.integers(0, 3000, 16)))
    ref = _sampled_rows_oracle(c, kq, vq, 0, tokens)
    check_attention(ref, out[tokens], "short_q_large_prefill_rows", splits=splits)
    sub = dict(c, q=c["q"][3000:], cu=c["cu"][1:] - 3000, seq_lens=c["seq_lens"][1:], block_table=c["block_table"][1:])
    check_attention(oracle_attention(sub, kq, vq), out[3000:], "short_q_large_other_rows", splits=splits)


@pytest.mark.parametrize("splits", [0, 4])
def test_short_q_large_beyond_65535_query_tokens(short_q, splits):
    """A request of 70,000 query tokens (2 q / 2 kv heads, head_dim 64) on the INT8 kernel: beyond the
    65,535 a grid dimension holds, which the kernel's query tokens never map to; sampled rows against B."""
    short_q(1_000_000)
    n = 70_000
    c = synth.paged_case(2, 2, [n], [n], head_dim=64, seed=85, params=synth.channel_params(2, 64))
    c["static"] = synth.calibration_scales(2, 64, synth.channel_params(2, 64))
    c["scale"] = 64 ** -0.5
    kq, vq = int8_cache(c)
    dc = dev(c)
    segm = nan_segm(n, 2, splits, 64) if splits else None
    out = ck.decode_attention(dc["q"], dev(kq), dev(vq), nan_like(dc["q"]), dc["cu"], dc["seq_lens"],
                              dc["block_table"], c["scale"], dc["static"], segm=segm, max_query_len=n).cpu()
    assert torch.isfinite(out.float()).all()
    r = synth.rng(86)
    tokens = sorted({0, 65534, 65535, 65536, n - 1} | set(int(x) for x in r.integers(0, n, 11)))
    check_attention(_sampled_rows_oracle(c, kq, vq, 0, tokens), out[tokens], "short_q_large_70k", splits=splits)
