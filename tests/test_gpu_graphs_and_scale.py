"""HIP-graph capture (the reference's tests/test_cudagraph.py) and parity at the benchmark sizes
(configs c2, c3, c4 of BASELINE.json), through size-independent checks: sampled requests against the
CPU oracle, split-count invariance, and the bit-exact cache codes of the GPU fill."""
import math
import os

import pytest
import torch
from conftest import nan_like, nan_segm, record

from oracle import kvq_oracle as O
from kvq import cuda_kernels as ck
from kvq import synth

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = 128 ** -0.5
SEQ_LENS = [100, 2000, 37, 512, 1500, 64, 999, 3000]


def _case(q_len, seed=0):
    c = synth.paged_case(28, 4, [q_len] * 8, SEQ_LENS, seed=seed, dist="randn", scale=3.0)
    st = synth.scales_from(c["k"].reshape(-1, 4, 128), c["v"].reshape(-1, 4, 128))
    kq = O.quantize(c["k"].float() - st["k_mu"], st["k_scale"])
    vq = O.quantize(c["v"], st["v_scale"])
    d = {k: v.to(DEV) for k, v in c.items()}
    return d, kq.to(DEV), vq.to(DEV), {k: v.to(DEV) for k, v in st.items()}


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


@pytest.mark.parametrize("q_len", [1, 4, 5])
@pytest.mark.parametrize("split", ["auto", "segm16"])
def test_replay_matches_eager_with_new_inputs(q_len, split):
    """tests/test_cudagraph.py:37-53: a captured call replayed with new q and one more key per request
    is bit-identical to the eager call; replayed several times with eager work in between."""
    d, kq, vq, st = _case(q_len)
    T = d["q"].shape[0]
    segm = None
    if split == "segm16":
        segm = nan_segm(T, 28, 16, 128)
    out = nan_like(d["q"])

    def attn(o):
        return ck.decode_attention(d["q"], kq, vq, o, d["cu"], d["seq_lens"], d["block_table"], SCALE, st,
                                   segm=segm, max_query_len=q_len)

    g = _capture(lambda: attn(out))
    for rep in range(3):
        q2 = synth.paged_case(28, 4, [q_len] * 8, SEQ_LENS, seed=7 + rep, dist="randn", scale=3.0)["q"]
        d["q"].copy_(q2.to(DEV))
        d["seq_lens"].add_(1)
        g.replay()
        torch.cuda.synchronize()
        ref = attn(nan_like(d["q"]))
        torch.cuda.synchronize()
        err = O.compare(ref.cpu(), out.cpu())
        record("graph_replay", q_len=q_len, split=split, rep=rep, **err)
        assert err["max_abs"] == 0.0


def test_scales_must_be_updated_in_place():
    """tests/test_cudagraph.py:56-84: rebinding a scale tensor does not reach the graph, an in-place
    update does."""
    d, kq, vq, st = _case(1)
    out = nan_like(d["q"])
    attn = lambda o, s: ck.decode_attention(d["q"], kq, vq, o, d["cu"], d["seq_lens"], d["block_table"], SCALE, s)
    g = _capture(lambda: attn(out, st))
    g.replay()
    torch.cuda.synchronize()
    before = out.clone()
    rebound = dict(st, v_scale=st["v_scale"] * 2)
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, before)
    expected = attn(nan_like(d["q"]), rebound)
    assert not torch.allclose(out, expected)
    st["v_scale"].mul_(2)                     # same storage the graph captured
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, expected)


def test_quant_cache_capture_skips_padded_slots():
    """tests/test_cudagraph.py:87-101: under a full graph the slot mapping is padded with -1."""
    T, H, D, nb, bs = 64, 4, 128, 32, 16
    key = torch.randn(T, H, D, device=DEV).to(torch.bfloat16)
    val = torch.randn(T, H, D, device=DEV).to(torch.bfloat16)
    slots = torch.full((T,), -1, dtype=torch.long, device=DEV)
    kc = torch.zeros(nb, bs, H, D, dtype=torch.int8, device=DEV)
    vc = torch.zeros_like(kc)
    st = {k: v.to(DEV) for k, v in synth.scales_from(key.cpu(), val.cpu()).items()}
    g = _capture(lambda: ck.quant_reshape_and_cache(key, val, kc, vc, slots, st))
    for rep in range(2):
        kc.zero_()
        vc.zero_()
        slots.fill_(-1)
        slots[:10 + rep] = torch.arange(10 + rep, device=DEV) * 3
        g.replay()
        torch.cuda.synchronize()
        assert int((kc != 0).flatten(2).any(-1).sum()) == 10 + rep


# ------------------------------------------------------------------ benchmark-size parity
def _request_oracle(kc, vc, bt, r, L, q_rows, st, per_channel=True, q_len=1):
    """Oracle output of one request of a big batch: copy its pages to the host, renumber them."""
    pages = -(-L // kc.shape[1])
    ids = bt[r, :pages].long()
    kq, vq = kc[ids].cpu(), vc[ids].cpu()
    cfg = O.CFG32_Q32 if per_channel else O.CFG32_HEAD_Q32
    f = O.paged_static_attention(cfg, {k: v.cpu() for k, v in st.items()}, True, 8)
    return f(q_rows.cpu().float(), kq, vq, torch.tensor([0, q_len], dtype=torch.int32),
             torch.tensor([L], dtype=torch.int32), torch.arange(pages, dtype=torch.int32)[None], SCALE)


def _interleaved(nb, hkv, bs, d):
    kv = torch.empty(nb, hkv, bs, 2 * d, dtype=torch.int8, device=DEV)
    kc, vc = kv.transpose(1, 2).split(d, dim=-1)
    return kv, kc, vc


def test_c2_full_size_sampled_parity():
    """c2: 128 requests x 32768 keys in vLLM's interleaved cache, filled through the quantize-and-cache
    kernel. Checks: the fill's codes for a sample of blocks are bit-exact; 16 requests spread over the
    batch (so over the stream-K workers' ranges: every 9th request from the 4th, and the first and last)
    match the oracle with split buffers (a captured graph's call: segments cut once, a second kernel
    merges); the output without them (bench.py's one pass, nothing cut) agrees."""
    B, L, hq, hkv, d, bs = 128, 32768, 28, 4, 128, 16
    pages = L // bs
    nb = B * pages + 64
    params = synth.channel_params(hkv, d)
    st = {k: v.to(DEV) for k, v in synth.calibration_scales(hkv, d, params).items()}
    kv, kc, vc = _interleaved(nb, hkv, bs, d)
    synth.fill_cache_gpu(kc, vc, st, params, seed=3, write=ck.quant_reshape_and_cache)
    # regenerate the first chunk's bf16 K/V and check the codes of 64 blocks of it bit for bit
    g = torch.Generator(device=DEV).manual_seed(3)
    gain, mean = torch.from_numpy(params[0]).to(DEV), torch.from_numpy(params[1]).to(DEV)
    k0 = (torch.randn(1 << 20, hkv, d, generator=g, device=DEV) * gain + mean).to(torch.bfloat16)[:64 * bs].cpu()
    stc = {k: v.cpu() for k, v in st.items()}
    assert torch.equal(kc[:64].cpu().reshape(-1, hkv, d), O.quantize(k0.float() - stc["k_mu"], stc["k_scale"]))
    bt = synth.random_block_table(B, [pages] * B, nb, 4, DEV)
    q = torch.randn(B, hq, d, generator=g, device=DEV).to(torch.bfloat16)
    cu = torch.arange(B + 1, dtype=torch.int32, device=DEV)
    sl = torch.full((B,), L, dtype=torch.int32, device=DEV)
    out = ck.decode_attention(q, kc, vc, nan_like(q), cu, sl, bt, SCALE, st,
                              segm=nan_segm(B, hq, ck.choose_splits(bt.shape[1] * bs), d))
    for r in sorted({0, 127} | set(range(3, 128, 9))):
        ref = _request_oracle(kc, vc, bt, r, L, q[r:r + 1], st)
        err = O.compare(ref, out[r:r + 1].cpu())
        record("c2_sampled", request=r, **err)
        assert err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3, (r, err)
    one = ck.decode_attention(q, kc, vc, nan_like(q), cu, sl, bt, SCALE, st)
    e = O.compare(one.cpu(), out.cpu())
    record("c2_split_invariance", **e)
    assert e["rel_l2"] < 1e-3 and e["max_abs"] <= 1e-2


@pytest.mark.parametrize("split", [True, False])
def test_c3_verification_full_parity(split):
    """c3: 64 requests x 8 causal query tokens, L log-uniform in [512, 8192]: every request against
    the oracle, with split buffers (bench.py's call) and without (one pass)."""
    lens = synth.c3_lens()
    c = synth.paged_case(28, 4, [8] * 64, lens, seed=13, params=synth.channel_params(4, 128), pool=1)
    c["static"] = synth.calibration_scales(4, 128, synth.channel_params(4, 128))
    st = c["static"]
    kq = O.quantize(c["k"].float() - st["k_mu"], st["k_scale"])
    vq = O.quantize(c["v"], st["v_scale"])
    ref = O.paged_static_attention(O.CFG32_Q32, st, True, 8)(c["q"].float(), kq, vq, c["cu"], c["seq_lens"],
                                                               c["block_table"], SCALE)
    d = {k: v.to(DEV) for k, v in c.items() if isinstance(v, torch.Tensor)}
    segm = nan_segm(d["q"].shape[0], 28, ck.choose_splits(d["block_table"].shape[1] * 16), 128) if split else None
    out = ck.decode_attention(d["q"], kq.to(DEV), vq.to(DEV), nan_like(d["q"]), d["cu"], d["seq_lens"],
                              d["block_table"], SCALE, {k: v.to(DEV) for k, v in st.items()}, segm=segm,
                              max_query_len=8)
    err = O.compare(ref, out.cpu())
    record("c3_full", split=split, **err)
    assert err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3 and err["rel_l2"] < 5e-3, err


@pytest.mark.parametrize("split", [True, False])
def test_c4_decode_rows_sampled_parity(split):
    """c4 decode part: Llama-3 heads (32 / 8), 96 requests with L log-uniform in [1, 32768] (incl. 1,
    17 and 32768): 12 requests against the oracle, with split buffers and without."""
    lens = synth.c4_lens()
    hq, hkv, d, bs = 32, 8, 128, 16
    pages = [-(-L // bs) for L in lens]
    nb = sum(pages) + 64
    params = synth.channel_params(hkv, d)
    st = {k: v.to(DEV) for k, v in synth.calibration_scales(hkv, d, params).items()}
    kv, kc, vc = _interleaved(nb, hkv, bs, d)
    synth.fill_cache_gpu(kc, vc, st, params, seed=50, write=ck.quant_reshape_and_cache)
    bt = synth.random_block_table(96, pages, nb, 51, DEV)
    g = torch.Generator(device=DEV).manual_seed(7)
    q = torch.randn(96, hq, d, generator=g, device=DEV).to(torch.bfloat16)
    cu = torch.arange(97, dtype=torch.int32, device=DEV)
    segm = nan_segm(96, hq, ck.choose_splits(bt.shape[1] * bs), d) if split else None
    out = ck.decode_attention(q, kc, vc, nan_like(q), cu, torch.tensor(lens, dtype=torch.int32, device=DEV),
                              bt, SCALE, st, segm=segm)
    order = sorted(range(96), key=lambda r: lens[r])
    for r in [0, 1, 2] + order[::10]:
        ref = _request_oracle(kc, vc, bt, r, lens[r], q[r:r + 1], st)
        err = O.compare(ref, out[r:r + 1].cpu())
        record("c4_sampled", request=r, L=lens[r], split=split, **err)
        assert err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3, (r, lens[r], err)


def test_c4_full_batch_in_one_paged_attention_call():
    """c4 as one step: 96 decode rows (L log-uniform in [1, 32768]) and 4 prefill requests of 16384 tokens
    in a single paged_attention call (plan_long for the long requests, no split buffers: 65,632 tokens,
    the one-pass INT8 path), Llama-3 heads 32 / 8. Sampled decode rows against the oracle, sampled
    prefill rows against fp32 attention over the dequantized pages."""
    dec = synth.c4_lens()
    hq, hkv, d, bs = 32, 8, 128, 16
    Q = 16384
    lens = dec + [Q] * 4
    q_lens = [1] * len(dec) + [Q] * 4
    pages = [-(-L // bs) for L in lens]
    nb = sum(pages) + 64
    params = synth.channel_params(hkv, d)
    st = {k: v.to(DEV) for k, v in synth.calibration_scales(hkv, d, params).items()}
    kv, kc, vc = _interleaved(nb, hkv, bs, d)
    synth.fill_cache_gpu(kc, vc, st, params, seed=70, write=ck.quant_reshape_and_cache)
    bt = synth.random_block_table(len(lens), pages, nb, 71, DEV)
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(q_lens), 0).tolist()), dtype=torch.int32)
    sl = torch.tensor(lens, dtype=torch.int32)
    g = torch.Generator(device=DEV).manual_seed(72)
    T = int(cu[-1])
    q = torch.randn(T, hq, d, generator=g, device=DEV).to(torch.bfloat16)
    plan = ck.plan_long(cu, sl, bs)
    assert plan is not None and plan.has_short and plan.src_req.shape[0] == 4 * (Q // bs)
    out = ck.paged_attention(q, kc, vc, nan_like(q), cu.to(DEV), sl.to(DEV), bt, Q, SCALE, st, plan)
    torch.cuda.synchronize()
    order = sorted(range(len(dec)), key=lambda r: dec[r])
    for r in [order[0], order[1], order[47], order[-2], order[-1]] + order[5::20]:
        ref = _request_oracle(kc, vc, bt, r, lens[r], q[int(cu[r]):int(cu[r]) + 1], st)
        err = O.compare(ref, out[int(cu[r]):int(cu[r]) + 1].cpu())
        record("c4_one_call_decode", request=r, L=lens[r], **err)
        assert err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3, (r, lens[r], err)
    rng = synth.rng(73)
    for r in range(len(dec), len(lens)):
        ids = bt[r, :pages[r]].long()
        k = (kc[ids].float() * st["k_scale"]).to(torch.bfloat16).float().reshape(Q, hkv, d)   # dequant_pages
        v = (vc[ids].float() * st["v_scale"]).to(torch.bfloat16).float().reshape(Q, hkv, d)
        kT = k.repeat_interleave(hq // hkv, dim=1).permute(1, 2, 0).contiguous()
        vv = v.repeat_interleave(hq // hkv, dim=1).permute(1, 0, 2).contiguous()
        for t in sorted({0, Q - 1} | set(int(x) for x in rng.integers(0, Q, 6))):
            qi = q[int(cu[r]) + t].float()[:, None, :].contiguous()
            sc = torch.matmul(qi, kT) / math.sqrt(d)
            sc[:, :, t + 1:] = float("-inf")
            o = torch.matmul(torch.softmax(sc, dim=-1), vv).squeeze(1)
            err = O.compare(o.cpu(), out[int(cu[r]) + t].float().cpu())
            record("c4_one_call_prefill", request=r, row=t, **err)
            assert err["max_abs"] <= 2e-2 and err["rel_l2"] < 1e-2, (r, t, err)
