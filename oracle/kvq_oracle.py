"""CPU oracle for the static INT8 KV-cache path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only
as the checker or as the timed CPU baseline. The product path (int8-kvcache_amd/kvq) never imports it:
when the HIP library is missing the product raises instead of falling back here.

This is a from-scratch restatement, in PyTorch on the CPU, of the reference's numerics:

  quantize / dequantize / scale_from_absmax     kvq/quant.py:46-55
  gather_pages / run_paged                      kvq/ref_attn.py:20-59
  attend_bf16 / paged_attention_ref / compare   kvq/ref_attn.py:62-102
  implementation A and B (attend_int8)          kvq/int8_ref.py:56-143
  paged_static_attention                        kvq/int8_ref.py:162-197
  plan_long                                     kvq/cuda_kernels.py:80-103

How each function is pinned (tests/test_oracle.py):
  quantize, quant codes of q, dequantize: closed forms + an independent C restatement
      (oracle/quant_ref.c, IEEE fp32 division and rintf) + golden vectors from the reference.
  run_paged / paged_attention_ref: brute-force per-row loop on tiny inputs + golden vectors.
  attend_int8 (B, CFG32): algebra-exact mode equals fp64 attention on dequantized K/V; one-key
      context gives v_i8 * s_v; identical keys give the mean of V; brute force per row with explicit
      per-tile P quantization; golden vectors from the reference.
  plan_long: the reference's known-answer test (tests/test_cuda_kernels.py:88-97).
"""
from dataclasses import dataclass

import numpy as np
import torch

QMAX = 127.0


# ----------------------------------------------------------------------------------------------
# Quantization formulas (kvq/quant.py:46-55)
# ----------------------------------------------------------------------------------------------
def scale_from_absmax(amax):
    """Dequantization step from an |x| max: amax / 127, floored at 1e-8 (fp32)."""
    return torch.clamp(amax / QMAX, min=1e-8)


def quantize(x, scale):
    """Symmetric int8 codes: fp32 division, round half to even, saturate at +-127 (never -128)."""
    y = torch.round(x.float() / scale)
    return torch.clamp(y, -QMAX, QMAX).to(torch.int8)


def dequantize(q, scale, dtype=torch.float32):
    """fp32 product of code and scale, then one rounding to `dtype`."""
    return (q.float() * scale).to(dtype)


# ----------------------------------------------------------------------------------------------
# Paging skeleton (kvq/ref_attn.py:20-59)
# ----------------------------------------------------------------------------------------------
def gather_pages(cache, block_table, max_len):
    """cache [nb, bs, H, D], block_table [B, W] -> [B, max_len, H, D] (rows past a request's length
    are whatever the pages hold)."""
    bs = cache.shape[1]
    n_pages = -(-max_len // bs)
    pages = cache[block_table[:, :n_pages].long()]          # [B, n_pages, bs, H, D]
    return pages.reshape(pages.shape[0], n_pages * bs, *pages.shape[3:])[:, :max_len]


def run_paged(attend, q, k_cache, v_cache, cu_seqlens_q, seq_lens, block_table, causal=True, max_rows=512,
              attend_multi=None):
    """Dispatch a paged batch to dense `attend(qb, k, v, mask, valid)` calls.

    Requests with one query token are batched together (padded to the longest context, `valid`
    masks the padding); longer requests run one at a time in chunks of at most `max_rows` query
    rows, with the bottom-right causal mask (query row i of a request with n query tokens and
    context L sees keys 0 .. L - n + i). Requests with zero query tokens produce nothing.
    """
    multi = attend_multi if attend_multi is not None else attend
    out = torch.empty(q.shape[0], q.shape[1], v_cache.shape[-1], dtype=q.dtype)
    cu = [int(x) for x in cu_seqlens_q.tolist()]
    lens = [int(x) for x in seq_lens.tolist()]
    nreq = len(cu) - 1
    single = [r for r in range(nreq) if cu[r + 1] - cu[r] == 1]
    if single:
        idx = torch.tensor(single, dtype=torch.long)
        kmax = max(lens[r] for r in single)
        valid = torch.arange(kmax)[None, :] < torch.tensor([lens[r] for r in single])[:, None]
        rows = torch.tensor([cu[r] for r in single], dtype=torch.long)
        res = attend(q[rows][:, None], gather_pages(k_cache, block_table[idx], kmax),
                     gather_pages(v_cache, block_table[idx], kmax), valid[:, None, :], valid)
        out[rows] = res[:, 0].to(q.dtype)
    for r in range(nreq):
        n = cu[r + 1] - cu[r]
        if n <= 1:
            continue
        L = lens[r]
        k = gather_pages(k_cache, block_table[r:r + 1], L)
        v = gather_pages(v_cache, block_table[r:r + 1], L)
        keys = torch.arange(L)
        valid = torch.ones(1, L, dtype=torch.bool)
        for s in range(0, n, max_rows):
            e = min(n, s + max_rows)
            if causal:
                qpos = (L - n) + torch.arange(s, e)
                mask = keys[None, :] <= qpos[:, None]
            else:
                mask = valid.expand(e - s, L)
            res = multi(q[cu[r] + s:cu[r] + e][None], k, v, mask[None], valid)
            out[cu[r] + s:cu[r] + e] = res[0].to(q.dtype)
    return out


def _grouped(qb, hkv):
    """[b, R, Hq, D] -> [b, R, Hkv, G, D]: q head h reads kv head h // G."""
    b, r, hq, d = qb.shape
    return qb.reshape(b, r, hkv, hq // hkv, d)


def attend_bf16(qb, k, v, mask, softmax_scale):
    """Textbook attention in fp32 (kvq/ref_attn.py:62-90): softmax over keys with masked keys at -inf."""
    hkv = k.shape[2]
    s = torch.einsum("brhgd,bkhd->bhgrk", _grouped(qb, hkv).float(), k.float()) * softmax_scale
    s = s.masked_fill(~mask[:, None, None], float("-inf"))
    p = torch.softmax(s, dim=-1)
    o = torch.einsum("bhgrk,bkhd->brhgd", p, v.float())
    return o.flatten(2, 3)


def paged_attention_ref(q, k_cache, v_cache, cu_seqlens_q, seq_lens, block_table, softmax_scale, causal=True):
    """The bf16 golden: fp32 attention over the original paged K/V (kvq/ref_attn.py:88-90)."""
    return run_paged(lambda qb, k, v, mask, valid: attend_bf16(qb, k, v, mask, softmax_scale),
                     q, k_cache, v_cache, cu_seqlens_q, seq_lens, block_table, causal)


def compare(ref, out):
    """Error summary {max_abs, mean_abs, rel_l2, cos} (kvq/ref_attn.py:93-102)."""
    a, b = ref.float(), out.float()
    d = (a - b).abs()
    return {
        "max_abs": d.max().item() if d.numel() else 0.0,
        "mean_abs": d.mean().item() if d.numel() else 0.0,
        "rel_l2": ((a - b).norm() / a.norm().clamp(min=1e-12)).item(),
        "cos": torch.nn.functional.cosine_similarity(a.flatten(), b.flatten(), dim=0).item(),
    }


# ----------------------------------------------------------------------------------------------
# Implementations A and B (kvq/int8_ref.py)
# ----------------------------------------------------------------------------------------------
@dataclass(frozen=True)
class Cfg:
    """Numerics of the INT8 path (kvq/int8_ref.py:33-42). The HIP kernels implement
    impl=B, q_gran=token_head, p_quant=tile, p_norm=quant with p_tile=32."""
    impl: str = "B"
    k_gran: str = "per_channel"
    v_gran: str = "per_channel"
    smooth_k: bool = False
    q_gran: str = "token_head"      # none | token_head | group<n>
    p_quant: str = "tile"           # none | tile
    p_tile: int = 64
    p_norm: str = "quant"           # quant | exact
    # Not a field of the reference's Cfg: "fp64" is int8_ref's q quantization (q' and its scale in
    # float64, kvq/int8_ref.py:83-91); "fp32" is the kernel contract stated by the reference's
    # tests/test_cuda_kernels.py:52-54 (fp32 product, fp32 scale, fp32 division). They differ only
    # where q' / s_q lands on a rounding tie, which bf16 q values make common when the K scale is per
    # head (q is then quantized as is).
    q_arith: str = "fp64"


CFG32 = Cfg(smooth_k=True, p_tile=32)
CFG32_HEAD = Cfg(smooth_k=True, p_tile=32, k_gran="per_head", v_gran="per_head")
CFG32_Q32 = Cfg(smooth_k=True, p_tile=32, q_arith="fp32")
CFG32_HEAD_Q32 = Cfg(smooth_k=True, p_tile=32, k_gran="per_head", v_gran="per_head", q_arith="fp32")
CFG32_G32 = Cfg(smooth_k=True, p_tile=32, q_gran="group32")
CFG32_G32_Q32 = Cfg(smooth_k=True, p_tile=32, q_gran="group32", q_arith="fp32")


def attend_dequant(qb, kq, ks, vq, vs, mask, softmax_scale):
    """Implementation A on int8 K/V: dequantize to bf16, then the fp32 golden attention
    (kvq/int8_ref.py:72-75)."""
    return attend_bf16(qb, dequantize(kq, ks, torch.bfloat16), dequantize(vq, vs, torch.bfloat16), mask,
                       softmax_scale)


def quant_p_tiles(e, p_tile):
    """Quantize e = exp(s - rowmax) in tiles of p_tile keys along the last dim, aligned at key 0:
    tile scale = max(tile) / 127 floored at 1e-30, code = round(e / scale); returns code * scale
    (kvq/int8_ref.py:94-105)."""
    K = e.shape[-1]
    pad = (-K) % p_tile
    t = torch.nn.functional.pad(e, (0, pad)).reshape(*e.shape[:-1], (K + pad) // p_tile, p_tile)
    s = torch.clamp(t.amax(-1, keepdim=True) / QMAX, min=1e-30)
    t = torch.round(t / s) * s
    return t.reshape(*e.shape[:-1], K + pad)[..., :K]


def quant_q_rows(qg, ks, arith="fp64"):
    """One q scale per (token, q head) row of qg [b, R, Hkv, G, D]: returns (codes as float64, scales).
    fp64: q' = q * s_k in float64, s = max(amax / 127, 1e-8) in float64, codes = round(f32(q') / s)
    (kvq/int8_ref.py:83-91 with kvq/quant.py:46-51). fp32: the same steps in float32."""
    per_channel = ks.shape[-1] > 1
    if arith == "fp32":
        x = qg.float() * ks.float()[:, :, :, None, :] if per_channel else qg.float()
    else:
        x = qg.double() * ks.double()[:, :, :, None, :] if per_channel else qg.double()
    sq = scale_from_absmax(x.abs().amax(-1, keepdim=True))
    return quantize(x, sq).double(), sq


def attend_int8(qb, kq, ks, vq, vs, mask, softmax_scale, cfg):
    """Implementation B (kvq/int8_ref.py:108-143): INT8 arithmetic with integer dot products
    evaluated exactly in float64.

    qb [b, R, Hq, D] float, kq/vq [b, K, Hkv, D] int8, ks/vs 4-D scales [b|1, 1, Hkv, D] (per
    channel) or [b|1, 1, Hkv, 1] (per head), mask [b, R, K].
      per-channel K: q' = q * s_k[h, :] (fp64), quantized per (token, q head) (or per group);
      per-head K: q quantized as is, s_k multiplies the scores;
      scores -> fp32, masked softmax numerator e = exp(s - rowmax), P quantized per tile,
      o = (P_hat . v_i8) / sum(P_hat) * s_v.
    """
    assert cfg.v_gran != "per_token_head"
    hkv = kq.shape[2]
    qg = _grouped(qb, hkv).double()                               # [b, R, Hkv, G, D]
    ks_d = ks.double()
    if ks.shape[-1] > 1:
        qf = qg * ks_d[:, :, :, None, :]                          # fold s_k[h, d] into q
        post = 1.0
    else:
        qf = qg
        post = ks_d.permute(0, 2, 3, 1).unsqueeze(2)              # [b|1, Hkv, 1, 1, 1] on the scores
    kd = kq.double()
    if cfg.q_gran.startswith("group"):
        n = int(cfg.q_gran[5:])
        if cfg.q_arith == "fp32":   # the kernel's contract: q' = fl32(q * s_k), fp32 scale and division
            qf = (qg.float() * ks.float()[:, :, :, None, :]) if ks.shape[-1] > 1 else qg.float()
        qs = qf.reshape(*qf.shape[:-1], qf.shape[-1] // n, n)     # [b, R, Hkv, G, C, n]
        sq = scale_from_absmax(qs.abs().amax(-1, keepdim=True))
        qi = quantize(qs, sq).double()
        part = torch.einsum("brhgcn,bkhcn->bhgrkc", qi, kd.reshape(*kd.shape[:-1], kd.shape[-1] // n, n))
        scores = (part * sq.double()[..., 0].permute(0, 2, 3, 1, 4)[:, :, :, :, None, :]).sum(-1)
    else:
        if cfg.q_gran == "none":
            qi, sq = qf, torch.ones_like(qf[..., :1])
        else:
            qi, sq = quant_q_rows(qg, ks, cfg.q_arith)
        scores = torch.einsum("brhgd,bkhd->bhgrk", qi, kd) * sq.double().permute(0, 2, 3, 1, 4)
    scores = (scores * post * softmax_scale).float()
    scores = scores.masked_fill(~mask[:, None, None], float("-inf"))
    e = torch.exp(scores - scores.amax(-1, keepdim=True))
    e_hat = quant_p_tiles(e, cfg.p_tile) if cfg.p_quant == "tile" else e
    denom = (e_hat if cfg.p_norm == "quant" else e).sum(-1, keepdim=True)
    o = torch.einsum("bhgrk,bkhd->brhgd", e_hat.double(), vq.double())
    o = o / denom.double().permute(0, 3, 1, 2, 4)
    o = o * vs.double()[:, :, :, None, :]
    return o.flatten(2, 3).float()


def paged_static_attention(cfg, static, cache_is_int8=True, short_q=1):
    """Static-scale attention as the backend runs it (kvq/int8_ref.py:162-197): requests with at
    most `short_q` query tokens use B, longer ones dequantize (A)."""
    ks, vs = static["k_scale"][None, None], static["v_scale"][None, None]
    mu = static.get("k_mu")
    state = {}

    def prep(k, v):
        if cache_is_int8:
            return k, v
        kf = k.float() - (mu[None, None] if mu is not None else 0)
        return quantize(kf, ks), quantize(v, vs)

    def decode(qb, k, v, mask, valid):
        kq, vq = prep(k, v)
        return attend_int8(qb, kq, ks, vq, vs, mask, state["scale"], cfg)

    def prefill(qb, k, v, mask, valid):
        if qb.shape[1] <= short_q:
            return decode(qb, k, v, mask, valid)
        kq, vq = prep(k, v)
        return attend_dequant(qb, kq, ks, vq, vs, mask, state["scale"])

    def fn(q, k_cache, v_cache, cu_seqlens_q, seq_lens, block_table, softmax_scale, causal=True):
        state["scale"] = softmax_scale
        return run_paged(decode, q, k_cache, v_cache, cu_seqlens_q, seq_lens, block_table, causal,
                         attend_multi=prefill)

    return fn


def quant_q_ref(q, k_scale, group=None):
    """fp32 q quantization as tests/test_cuda_kernels.py:52-54 states it: q' = f32(q) * s_k[h // G, :]
    (per-channel K scale; a per-head scale is not folded), one scale per `group` channels,
    s = max(amax / 127, 1e-8), code = rint(q' / s) saturated. Returns (codes [T,Hq,D], scales [T,Hq,D/group])."""
    T, hq, d = q.shape
    group = group or d
    hkv = k_scale.shape[0]
    x = q.float().reshape(T, hkv, hq // hkv, d)
    if k_scale.shape[-1] > 1:
        x = x * k_scale.float()[None, :, None, :]
    x = x.reshape(T, hq, d // group, group)
    s = scale_from_absmax(x.abs().amax(-1, keepdim=True))
    return quantize(x, s).reshape(T, hq, d), s[..., 0]


def quant_cache_ref(key, value, k_cache, v_cache, slot_mapping, static):
    """Quantize + scatter (kvq/vllm_int8/backend.py:155-164 torch path; kernel contract
    kvq/cuda/int8_kv.cu:55-84): the first n = len(slot_mapping) rows, slot < 0 skipped. In place."""
    n = slot_mapping.shape[0]
    slots = slot_mapping.long()
    ok = slots >= 0
    kq = quantize(key[:n].float() - static["k_mu"], static["k_scale"])
    vq = quantize(value[:n].float(), static["v_scale"])
    bs = k_cache.shape[1]
    k_cache[slots[ok] // bs, slots[ok] % bs] = kq[ok]
    v_cache[slots[ok] // bs, slots[ok] % bs] = vq[ok]


def dequant_pages_ref(k_cache, v_cache, block_table, src_req, src_j, static, dtype=torch.bfloat16):
    """Pages of the int8 cache as a contiguous bf16 cache [P, bs, H, D]
    (kvq/cuda/int8_kv.cu:505-542, formula kvq/quant.py:54-55; K keeps k - mu)."""
    pages = block_table.long()[src_req.long(), src_j.long()]
    ks, vs = static["k_scale"], static["v_scale"]
    return dequantize(k_cache[pages], ks, dtype), dequantize(v_cache[pages], vs, dtype)


# ----------------------------------------------------------------------------------------------
# Host plan of the long-query path (kvq/cuda_kernels.py:61-103)
# ----------------------------------------------------------------------------------------------
def plan_long_ref(query_start_loc, seq_lens, block_size, short_q=8):
    """Returns None when no request has more than short_q query tokens, else a dict with
    src_req, src_j (temporary page -> request and page index), block_table (temporary cache,
    at least ceil(256 / bs) columns wider than the longest long request), max_seqlen_k, has_short."""
    qsl = np.asarray(query_start_loc, dtype=np.int64)
    nreq = len(qsl) - 1
    qlen = qsl[1:] - qsl[:-1]
    is_long = qlen > short_q
    if not is_long.any():
        return None
    seq = np.asarray(seq_lens, dtype=np.int64)[:nreq]
    npages = np.where(is_long, (seq + block_size - 1) // block_size, 0)
    src_req, src_j = [], []
    for r in range(nreq):
        for j in range(int(npages[r])):
            src_req.append(r)
            src_j.append(j)
    width = int(npages.max()) + (256 + block_size - 1) // block_size
    bt = np.zeros((nreq, width), dtype=np.int32)
    for p, (r, j) in enumerate(zip(src_req, src_j)):
        bt[r, j] = p
    return {"src_req": np.array(src_req, dtype=np.int32), "src_j": np.array(src_j, dtype=np.int32),
            "block_table": bt, "max_seqlen_k": int(seq[is_long].max()),
            "has_short": bool((qlen[~is_long] > 0).any())}
