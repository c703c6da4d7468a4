"""The vLLM backend on the GPU, the way a vLLM worker drives it (reference kvq/vllm_int8/backend.py:
149-184): the step's K/V are written into vLLM's interleaved int8 cache by do_kv_cache_update (codes
bit-exact against the oracle), and forward() answers a mixed batch -- decode rows, speculative
verification rows, long prefill rows -- through the metadata builder's plan and split buffers, within
the attention bars against the oracle -- with the builder's split buffers (few requests, skewed lengths,
more short tokens than the buffers' rows) and without them (many requests of even length: one pass).
vLLM itself is replaced by tests/vllm_stub."""
import os
import sys
from types import SimpleNamespace

import numpy as np
import pytest
import torch
from conftest import nan_like, record

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "vllm_stub"))

from vllm.v1.attention.backends.triton_attn import CommonAttentionMetadata  # noqa: E402

from oracle import kvq_oracle as O  # noqa: E402
from kvq import scales, synth  # noqa: E402
from kvq.vllm_int8 import backend  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"
HQ, HKV, D, BS = 28, 4, 128, 16


BATCHES = {
    # decode, verification and long prefill rows, short ones after the long (tokens past the buffers'
    # 64 rows: run whole)
    "mixed": ([1, 4, 1, 40, 1, 8, 130, 1], [700, 64, 1, 40, 2049, 300, 500, 33], True),
    # few short requests
    "short_split": ([1, 4, 1, 8, 1, 3, 1, 1], [700, 64, 1, 2300, 2049, 300, 5000, 33], True),
    # skewed decode batch with more short tokens than the buffers' 64 rows
    "many_decode": ([1] * 90 + [5, 20, 3], [int(x) for x in synth.rng(5).integers(1, 4000, 90)] + [9000, 700, 300],
                    True),
    # requests whose pairs give every CU a whole number of them (x 4 kv heads = 2 per CU), even lengths:
    # one pass
    "many_even": ([1] * 128, [1500] * 128, False),
}


@pytest.mark.parametrize("batch", list(BATCHES))
@pytest.mark.parametrize("cfg", ["B_channel_smooth", "B_head"])
def test_backend_step_matches_oracle(tmp_path, monkeypatch, cfg, batch):
    per_channel = cfg.startswith("B_channel")
    smooth = cfg.endswith("smooth")
    q_lens, seq_lens, with_buffers = BATCHES[batch]
    B = len(q_lens)
    rng = synth.rng(77)
    c = synth.paged_case(HQ, HKV, q_lens, seq_lens, seed=31, params=synth.channel_params(HKV, D))
    k_all, v_all = c["k"].reshape(-1, HKV, D), c["v"].reshape(-1, HKV, D)
    st = synth.scales_from(k_all, v_all, per_channel, smooth)
    if not smooth:
        del st["k_mu"]                   # a scale file without smooth-K has no mean
    name = "model.layers.0.self_attn.attn"
    scales.save(str(tmp_path / "s.safetensors"), {name: st})
    monkeypatch.setenv("KVQ_SCALES", str(tmp_path / "s.safetensors"))
    monkeypatch.setenv("KVQ_CFG", cfg)

    impl = backend.Int8StaticImpl(HQ, D, D ** -0.5, HKV, kv_cache_dtype="int8_static")
    vcfg = SimpleNamespace(compilation_config=SimpleNamespace(static_forward_context={name: SimpleNamespace(impl=impl)}),
                           speculative_config=None,
                           model_config=SimpleNamespace(num_heads=HQ, num_kv_heads=HKV, head_size=D),
                           scheduler_config=SimpleNamespace(max_num_seqs=64))
    monkeypatch.setenv("KVQ_SPLIT_MB", "256")
    builder = backend.Int8StaticBuilder(SimpleNamespace(block_size=BS), [name], vcfg, DEV)

    # write every request's K/V through the backend, in two steps (history, then the step's tokens)
    nb = int(c["block_table"].max()) + 8
    kv_cache = torch.zeros(nb, HKV, BS, 2 * D, dtype=torch.int8, device=DEV)
    bt = c["block_table"]
    slots = torch.cat([bt[r, torch.arange(L) // BS].long() * BS + torch.arange(L) % BS for r, L in enumerate(seq_lens)])
    k_rows = torch.cat([c["k"][bt[r, torch.arange(L) // BS].long(), torch.arange(L) % BS] for r, L in enumerate(seq_lens)])
    v_rows = torch.cat([c["v"][bt[r, torch.arange(L) // BS].long(), torch.arange(L) % BS] for r, L in enumerate(seq_lens)])
    cut = int(rng.integers(1, k_rows.shape[0]))
    for lo, hi in ((0, cut), (cut, k_rows.shape[0])):
        # five padded rows with slot -1 at the end, as under graph capture
        key = torch.cat([k_rows[lo:hi], torch.ones(5, HKV, D, dtype=k_rows.dtype)]).to(DEV)
        val = torch.cat([v_rows[lo:hi], torch.ones(5, HKV, D, dtype=v_rows.dtype)]).to(DEV)
        sl = torch.cat([slots[lo:hi], torch.full((5,), -1, dtype=torch.long)]).to(DEV)
        impl.do_kv_cache_update(None, key, val, kv_cache, sl)
    kc, vc = impl._caches(kv_cache)
    sd = dict(st, k_mu=st.get("k_mu", torch.zeros(HKV, D)))
    kq = O.quantize(c["k"].float() - sd["k_mu"], sd["k_scale"])
    vq = O.quantize(c["v"].float(), sd["v_scale"])
    blk, off = slots // BS, slots % BS                    # exactly the written slots
    assert torch.equal(kc.cpu()[blk, off], kq[blk, off]) and torch.equal(vc.cpu()[blk, off], vq[blk, off])

    cu = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32)
    common = CommonAttentionMetadata(query_start_loc=cu.to(DEV), query_start_loc_cpu=cu,
                                     seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=DEV), num_reqs=B,
                                     num_actual_tokens=int(cu[-1]), max_query_len=max(q_lens), max_seq_len=max(seq_lens),
                                     block_table_tensor=bt.to(DEV), slot_mapping=slots.to(DEV),
                                     seq_lens_cpu_upper_bound=torch.tensor(seq_lens, dtype=torch.int32))
    md = builder.build(0, common)
    has_long = max(q_lens) > 8
    assert (md.kvq_long is not None) == has_long and (not has_long or md.kvq_long.has_short)
    T = int(cu[-1])
    assert (md.kvq_segm is not None) == with_buffers
    assert builder.kvq_segm[1].shape[0] == 64
    q = c["q"].to(DEV)
    out = nan_like(torch.empty(T + 3, HQ, D, dtype=torch.bfloat16, device=DEV))   # vLLM pads the output
    impl.forward(None, q, None, None, kv_cache, md, out)
    cfg_o = O.CFG32_Q32 if per_channel else O.CFG32_HEAD_Q32
    ref = O.paged_static_attention(cfg_o, sd, True, 8)(c["q"].float(), kc.cpu(), vc.cpu(), cu,
                                                        torch.tensor(seq_lens, dtype=torch.int32), bt, D ** -0.5)
    short = torch.repeat_interleave(torch.tensor(q_lens) <= 8, torch.tensor(q_lens))
    got = out[:T].cpu()
    err_s = O.compare(ref[short], got[short])
    err_l = O.compare(ref[~short], got[~short]) if has_long else None
    record("vllm_backend_step", cfg=cfg, batch=batch, short=err_s, long=err_l if has_long else None)
    assert err_s["max_abs"] <= 2e-2 and err_s["mean_abs"] <= 2e-3 and err_s["rel_l2"] < 5e-3, err_s
    if has_long:
        assert err_l["rel_l2"] < 1e-2, err_l      # long rows: bf16 attention on dequantized pages
