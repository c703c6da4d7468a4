"""The bf16 paged prefill attention (kvq_paged_prefill_attention), the consumer of the long-query path
(the reference hands dequant_pages' output to vLLM's FlashAttention, kvq/cuda_kernels.py:106-131).
A floating-point kernel: checked against a plain fp32 torch attention over the same bf16 pages
(bottom-right causal), at the reference's long-row bar (rel_l2 < 1e-2, tests/test_cuda_kernels.py:119)
and tighter max / mean error bars; rows outside the work list must stay untouched."""
import math

import numpy as np
import pytest
import torch
from conftest import nan_like, record

from oracle import kvq_oracle as O
from kvq import cuda_kernels as ck
from kvq import synth

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _temp_cache(q_lens, seq_lens, hkv, d, bs, seed):
    """A bf16 temporary cache laid out as plan_long lays it out (pages of long requests consecutive)."""
    cu = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32)
    plan = ck.plan_long(cu, torch.tensor(seq_lens), bs)
    g = torch.Generator().manual_seed(seed)
    P = plan.src_req.shape[0]
    kt = (torch.randn(P, bs, hkv, d, generator=g) * 1.5).to(torch.bfloat16)
    vt = torch.randn(P, bs, hkv, d, generator=g).to(torch.bfloat16)
    return cu, plan, kt, vt


def _reference(q, kt, vt, cu, seq_lens, plan, scale, rows=None):
    """fp32 attention of the long requests' rows over their pages (consecutive in the temporary cache)."""
    bs, hkv, d = kt.shape[1:]
    hq = q.shape[1]
    G = hq // hkv
    first = {}
    for p, r in enumerate(plan.src_req.tolist()):
        first.setdefault(r, p)
    out = {}
    for r in plan.long_req.tolist():
        Q, L = int(cu[r + 1] - cu[r]), int(seq_lens[r])
        npg = -(-L // bs)
        k = kt[first[r]:first[r] + npg].reshape(npg * bs, hkv, d)[:L].float()
        v = vt[first[r]:first[r] + npg].reshape(npg * bs, hkv, d)[:L].float()
        ts = range(Q) if rows is None else rows[r]
        for t in ts:
            qi = q[int(cu[r]) + t].float()                                     # [Hq, D]
            kk = k[:L - Q + 1 + t].repeat_interleave(G, dim=1)               # [keys, Hq, D]
            vv = v[:L - Q + 1 + t].repeat_interleave(G, dim=1)
            s = torch.einsum("hd,khd->hk", qi, kk) * scale
            p = torch.softmax(s, dim=-1)
            out[(r, t)] = torch.einsum("hk,khd->hd", p, vv)
    return out


@pytest.mark.parametrize("shape", [(28, 4, 128), (32, 8, 128), (14, 2, 64), (12, 2, 128)])
def test_prefill_matches_fp32_reference(shape):
    hq, hkv, d = shape
    q_lens = [100, 1, 37, 64, 9, 300, 3]
    seq_lens = [100, 50, 517, 64, 2000, 1000, 700]      # q_len == L, > SHORT_Q and partial pages
    cu, plan, kt, vt = _temp_cache(q_lens, seq_lens, hkv, d, 16, seed=hq)
    T = int(cu[-1])
    q = (torch.randn(T, hq, d, generator=torch.Generator().manual_seed(1)) * 2).to(torch.bfloat16)
    scale = d ** -0.5
    out = nan_like(q.to(DEV))
    tile_req, tile_row = plan.tiles(hq // hkv, DEV)
    src_req, src_j, bt = plan.gpu(DEV)
    ck.ext().paged_prefill_attention(q.to(DEV), kt.to(DEV), vt.to(DEV), out, cu.to(DEV),
                                     torch.tensor(seq_lens, dtype=torch.int32, device=DEV), bt, tile_req, tile_row, scale)
    out = out.cpu()
    ref = _reference(q, kt, vt, cu, seq_lens, plan, scale)
    got = torch.stack([out[int(cu[r]) + t] for (r, t) in ref]).float()
    exp = torch.stack(list(ref.values()))
    err = O.compare(exp, got)
    record("prefill_vs_fp32", shape=list(shape), **err)
    assert err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3 and err["rel_l2"] < 1e-2, err
    # rows of short requests (q_len <= SHORT_Q) are not in the work list: untouched
    for r, Q in enumerate(q_lens):
        if Q <= ck.SHORT_Q:
            assert torch.isnan(out[int(cu[r]):int(cu[r + 1])].float()).all(), r


def test_c4_prefill_full_size_sampled():
    """c4's prefill part: 4 requests x 16384 tokens (q_len = L), Llama-3 heads 32 / 8, read from the INT8
    cache through dequant_pages + the prefill kernel (long_attention); 48 rows per request (first,
    last, random) against fp32 attention over the dequantized pages."""
    hq, hkv, d, bs = 32, 8, 128, 16
    Q = L = 16384
    B = 4
    pages = L // bs
    nb = B * pages + 32
    params = synth.channel_params(hkv, d)
    st = {k: v.to(DEV) for k, v in synth.calibration_scales(hkv, d, params).items()}
    kv = torch.empty(nb, hkv, bs, 2 * d, dtype=torch.int8, device=DEV)
    kc, vc = kv.transpose(1, 2).split(d, dim=-1)
    synth.fill_cache_gpu(kc, vc, st, params, seed=61, write=ck.quant_reshape_and_cache)
    bt = synth.random_block_table(B, [pages] * B, nb, 62, DEV)
    g = torch.Generator(device=DEV).manual_seed(63)
    q = torch.randn(B * Q, hq, d, generator=g, device=DEV).to(torch.bfloat16)
    cu = torch.arange(B + 1, dtype=torch.int32) * Q
    sl = torch.full((B,), L, dtype=torch.int32)
    plan = ck.plan_long(cu, sl, bs)
    out = nan_like(q)
    ck.long_attention(q, kc, vc, out, cu.to(DEV), sl.to(DEV), bt, Q, plan, d ** -0.5, st)
    torch.cuda.synchronize()
    rng = synth.rng(64)
    worst = {"max_abs": 0.0, "mean_abs": 0.0, "rel_l2": 0.0}
    for r in range(B):
        ids = bt[r, :pages].long()
        k = (kc[ids].float() * st["k_scale"]).to(torch.bfloat16).float().reshape(L, hkv, d)   # dequant_pages
        v = (vc[ids].float() * st["v_scale"]).to(torch.bfloat16).float().reshape(L, hkv, d)
        kT = k.repeat_interleave(hq // hkv, dim=1).permute(1, 2, 0).contiguous()          # [Hq, D, L]
        vv = v.repeat_interleave(hq // hkv, dim=1).permute(1, 0, 2).contiguous()          # [Hq, L, D]
        rows = sorted({0, 1, 15, 16, Q - 1, Q - 2} | set(int(x) for x in rng.integers(0, Q, 42)))
        for t in rows:
            qi = q[r * Q + t].float()[:, None, :].contiguous()                            # [Hq, 1, D]
            s = torch.matmul(qi, kT) / math.sqrt(d)                                       # [Hq, 1, L]
            s[:, :, t + 1:] = float("-inf")                                               # causal
            o = torch.matmul(torch.softmax(s, dim=-1), vv).squeeze(1)                     # [Hq, D]
            e = O.compare(o.cpu(), out[r * Q + t].cpu())
            for key in worst:
                worst[key] = max(worst[key], e[key])
    record("c4_prefill_sampled", **worst)
    assert worst["max_abs"] <= 2e-2 and worst["rel_l2"] < 1e-2, worst


def test_prefill_score_jump_takes_the_rescaling_pass():
    """A key far past the first tile whose scores exceed every earlier one by much more than 2^64
    (log2 units): the fast pass flags its workgroups and they are recomputed with rescaling; the
    result still matches fp32 attention (where the outlier key dominates every row that sees it)."""
    hq, hkv, d = 28, 4, 128
    q_lens, seq_lens = [200, 40], [1000, 300]
    cu, plan, kt, vt = _temp_cache(q_lens, seq_lens, hkv, d, 16, seed=3)
    T = int(cu[-1])
    q = (torch.randn(T, hq, d, generator=torch.Generator().manual_seed(4)) + 0.5).to(torch.bfloat16)
    first = {}
    for p, r in enumerate(plan.src_req.tolist()):
        first.setdefault(r, p)
    for r, key in ((0, 850), (1, 130)):                   # outliers past tile 0, visible to later rows
        kt[first[r] + key // 16, key % 16] = 60.0
    scale = d ** -0.5
    out = nan_like(q.to(DEV))
    tile_req, tile_row = plan.tiles(hq // hkv, DEV)
    _, _, bt = plan.gpu(DEV)
    ck.ext().paged_prefill_attention(q.to(DEV), kt.to(DEV), vt.to(DEV), out, cu.to(DEV),
                                     torch.tensor(seq_lens, dtype=torch.int32, device=DEV), bt, tile_req, tile_row, scale)
    out = out.cpu()
    ref = _reference(q, kt, vt, cu, seq_lens, plan, scale)
    got = torch.stack([out[int(cu[r]) + t] for (r, t) in ref]).float()
    err = O.compare(torch.stack(list(ref.values())), got)
    record("prefill_score_jump", **err)
    assert torch.isfinite(got).all() and err["max_abs"] <= 2e-2 and err["rel_l2"] < 1e-2, err


@pytest.mark.parametrize("layout", ["permuted", "bs32", "bs64_permuted", "padded_pages", "one_page_moved"])
def test_prefill_page_layouts(layout):
    """The kernel reads a request's pages without the block table when they are one run of consecutive
    ids in a cache of whole pages (the layout plan_long + dequant_pages produce), and through the
    table otherwise: pages in shuffled order, one page of a run moved elsewhere, pages with a stride
    beyond block_size slots, and larger blocks (one or two pages per 32-key tile). Every layout holds
    the same logical keys, so each must match the fp32 attention over them."""
    hq, hkv, d = 12, 2, 128
    bs = {"bs32": 32, "bs64_permuted": 64}.get(layout, 16)
    q_lens = [100, 3, 300, 40]
    seq_lens = [100, 700, 1000, 2000]
    cu, plan, kt, vt = _temp_cache(q_lens, seq_lens, hkv, d, bs, seed=7)
    P = kt.shape[0]
    T = int(cu[-1])
    q = (torch.randn(T, hq, d, generator=torch.Generator().manual_seed(8)) * 2).to(torch.bfloat16)
    scale = d ** -0.5
    ref = _reference(q, kt, vt, cu, seq_lens, plan, scale)       # over the logical pages
    _, _, bt = plan.gpu(DEV)
    bt = bt.cpu().long()
    ktp, vtp = kt, vt
    if layout in ("permuted", "bs64_permuted", "one_page_moved"):
        perm = torch.randperm(P + 3, generator=torch.Generator().manual_seed(9))[:P]   # logical -> physical
        if layout == "one_page_moved":
            perm = torch.arange(P)
            perm[P // 2] = P + 2                                  # one page of a run lives elsewhere
        ktp = torch.zeros(P + 3, bs, hkv, d, dtype=kt.dtype)
        vtp = torch.zeros_like(ktp)
        ktp[perm], vtp[perm] = kt, vt
        bt = torch.where(bt >= 0, perm[bt.clamp(min=0)], bt)
    elif layout == "padded_pages":                                # page stride of bs + 1 slots
        ktp = torch.zeros(P, bs + 1, hkv, d, dtype=kt.dtype)
        vtp = torch.zeros_like(ktp)
        ktp[:, :bs], vtp[:, :bs] = kt, vt
    kd, vd = ktp.to(DEV), vtp.to(DEV)
    if layout == "padded_pages":
        kd, vd = kd[:, :bs], vd[:, :bs]
    out = nan_like(q.to(DEV))
    tile_req, tile_row = plan.tiles(hq // hkv, DEV)
    ck.ext().paged_prefill_attention(q.to(DEV), kd, vd, out, cu.to(DEV),
                                     torch.tensor(seq_lens, dtype=torch.int32, device=DEV),
                                     bt.to(torch.int32).to(DEV), tile_req, tile_row, scale)
    out = out.cpu()
    got = torch.stack([out[int(cu[r]) + t] for (r, t) in ref]).float()
    err = O.compare(torch.stack(list(ref.values())), got)
    record("prefill_page_layouts", layout=layout, **err)
    assert torch.isfinite(got).all() and err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3 and err["rel_l2"] < 1e-2, err
