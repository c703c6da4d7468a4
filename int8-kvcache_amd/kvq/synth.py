"""Seeded synthetic workloads of the benchmark configurations (BASELINE configs c0..c4).

Host-side generators draw with numpy PCG64, so the CPU container and the GPU box produce identical
inputs for the same seed. The multi-GB caches of the large configurations are filled on the GPU
instead (torch generator + this package's quantize-and-cache kernel).

Distribution "c0" (the model-like one): K = N(0,1) * gain[h,d] + mean[h,d] with gain ~ LogNormal(0,1)
and mean ~ N(0, 0.5) (0.5 is the standard deviation), V = N(0,1), q = N(0,1); bf16.
Distribution "randn": q, K = N(0,1) * scale, V = N(0,1) (the reference tests' random_paged_case,
tests/conftest.py:45-65).
"""
import math

import numpy as np
import torch

QMAX = 127.0


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def channel_params(hkv, d, seed=11):
    """Per-(kv head, channel) gain and mean of the c0 K distribution."""
    r = rng(seed)
    gain = np.exp(r.standard_normal((hkv, d))).astype(np.float32)
    mean = (0.5 * r.standard_normal((hkv, d))).astype(np.float32)
    return gain, mean


def draw_kv(r, n, hkv, d, params=None, scale=1.0):
    """float32 K, V [n, hkv, d]; params = channel_params(...) for the c0 distribution, None for randn."""
    k = r.standard_normal((n, hkv, d), dtype=np.float32)
    if params is not None:
        k = k * params[0][None] + params[1][None]
    else:
        k = k * np.float32(scale)
    v = r.standard_normal((n, hkv, d), dtype=np.float32)
    return k, v


def bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)


def scales_from(k, v, per_channel=True, smooth=True):
    """Static scales from sample rows k, v [n, H, D] (float): k_mu = mean (or 0), scale = max|x| / 127
    floored at 1e-8, per channel or per head (the reference's calibration rule, kvq/scales.py:13-34,
    tests/conftest.py:96-107)."""
    k, v = k.float(), v.float()
    mu = k.mean(0) if smooth else torch.zeros_like(k[0])
    ka, va = (k - mu).abs().amax(0), v.abs().amax(0)
    if not per_channel:
        ka, va = ka.amax(-1, keepdim=True), va.amax(-1, keepdim=True)
    return {"k_scale": torch.clamp(ka / QMAX, min=1e-8).contiguous(),
            "v_scale": torch.clamp(va / QMAX, min=1e-8).contiguous(),
            "k_mu": mu.contiguous()}


def calibration_scales(hkv, d, params, per_channel=True, smooth=True, seed=0, n=4096):
    """c0 scales: from a separate seeded 4096-token sample of the same distribution."""
    k, v = draw_kv(rng(seed), n, hkv, d, params)
    return scales_from(bf16(k), bf16(v), per_channel, smooth)


def paged_case(hq, hkv, q_lens, seq_lens, head_dim=128, block_size=16, seed=1, dist="c0", scale=1.0, pool=2,
               params=None):
    """A paged batch on the CPU: q bf16 [T, hq, D], k/v bf16 [nb, bs, hkv, D], cu int32 [B+1],
    seq_lens int32 [B], block_table int32 [B, max_pages] (a random permutation of a pool `pool` times
    larger than needed, plus 8 spare blocks)."""
    r = rng(seed)
    q_lens, seq_lens = list(q_lens), list(seq_lens)
    pages = [-(-s // block_size) for s in seq_lens]
    nb = pool * sum(pages) + 8
    perm = r.permutation(nb).astype(np.int32)
    bt = np.zeros((len(seq_lens), max(max(pages), 1)), dtype=np.int32)
    off = 0
    for i, p in enumerate(pages):
        bt[i, :p] = perm[off:off + p]
        off += p
    cu = np.zeros(len(q_lens) + 1, dtype=np.int32)
    cu[1:] = np.cumsum(q_lens)
    q = r.standard_normal((int(cu[-1]), hq, head_dim), dtype=np.float32)
    if dist == "randn":
        q = q * np.float32(scale)
        k, v = draw_kv(r, nb * block_size, hkv, head_dim, None, scale)
    else:
        if params is None:
            params = channel_params(hkv, head_dim)
        k, v = draw_kv(r, nb * block_size, hkv, head_dim, params)
    shape = (nb, block_size, hkv, head_dim)
    return {"q": bf16(q), "k": bf16(k).reshape(shape), "v": bf16(v).reshape(shape),
            "cu": torch.from_numpy(cu), "seq_lens": torch.tensor(seq_lens, dtype=torch.int32),
            "block_table": torch.from_numpy(bt)}


def log_uniform_lengths(r, n, lo, hi):
    """n integers floor(exp(U(ln lo, ln hi))), clipped to [lo, hi]."""
    x = np.floor(np.exp(r.uniform(math.log(lo), math.log(hi), n))).astype(np.int64)
    return np.clip(x, lo, hi).tolist()


# ------------------------------------------------------------------------------------------------
# The benchmark configurations
# ------------------------------------------------------------------------------------------------
C0_LENS = [17, 300, 1024, 2049]


def c0_case(seed=1, per_channel=True, smooth=True):
    """c0: 4 decode requests x {17, 300, 1024, 2049}, 28/4/128, bs 16, c0 distribution."""
    params = channel_params(4, 128)
    case = paged_case(28, 4, [1] * 4, C0_LENS, 128, 16, seed=seed, params=params)
    case["static"] = calibration_scales(4, 128, params, per_channel, smooth)
    return case


def c1_inputs(seed=5, T=16384, hkv=4, d=128, num_blocks=4096, block_size=16, pad_frac=0.02):
    """c1: T new tokens (c0 distribution) + a collision-free slot mapping into num_blocks x bs slots
    with ~pad_frac of the entries = -1."""
    params = channel_params(hkv, d)
    r = rng(seed)
    k, v = draw_kv(r, T, hkv, d, params)
    slots = r.permutation(num_blocks * block_size)[:T].astype(np.int64)
    slots[r.random(T) < pad_frac] = -1
    return {"key": bf16(k), "value": bf16(v), "slots": torch.from_numpy(slots),
            "static": calibration_scales(hkv, d, params), "num_blocks": num_blocks, "block_size": block_size}


def c3_lens(seed=7, n=64):
    return log_uniform_lengths(rng(seed), n, 512, 8192)


def c4_lens(seed=9, n_decode=96):
    """c4 decode lengths: ceil(exp(U(0, ln 32768))), forced to include 1 and a few non-multiples of 16."""
    r = rng(seed)
    x = np.ceil(np.exp(r.uniform(0.0, math.log(32768), n_decode))).astype(np.int64)
    x = np.clip(x, 1, 32768)
    x[0], x[1], x[2] = 1, 17, 32768
    return x.tolist()


# ------------------------------------------------------------------------------------------------
# GPU-side construction of large paged caches
# ------------------------------------------------------------------------------------------------
def random_block_table(num_reqs, pages_per_req, num_blocks, seed, device):
    """[num_reqs, max_pages] int32: distinct physical blocks drawn from a permutation of num_blocks."""
    g = torch.Generator(device=device).manual_seed(seed)
    total = int(sum(pages_per_req))
    perm = torch.randperm(num_blocks, generator=g, device=device)[:total].to(torch.int32)
    bt = torch.zeros(num_reqs, max(pages_per_req), dtype=torch.int32, device=device)
    off = 0
    for i, p in enumerate(pages_per_req):
        bt[i, :p] = perm[off:off + p]
        off += p
    return bt


def fill_cache_gpu(k_cache, v_cache, static, params, seed=3, chunk_tokens=1 << 20, write=None):
    """Fill every slot of int8 caches [nb, bs, H, D] with c0-distribution K/V quantized by `write`
    (kvq.cuda_kernels.quant_reshape_and_cache): drawn on the GPU in chunks, never on the host."""
    nb, bs, hkv, d = k_cache.shape
    dev = k_cache.device
    g = torch.Generator(device=dev).manual_seed(seed)
    gain = torch.from_numpy(params[0]).to(dev)
    mean = torch.from_numpy(params[1]).to(dev)
    total = nb * bs
    for s in range(0, total, chunk_tokens):
        n = min(chunk_tokens, total - s)
        k = (torch.randn(n, hkv, d, generator=g, device=dev) * gain + mean).to(torch.bfloat16)
        v = torch.randn(n, hkv, d, generator=g, device=dev).to(torch.bfloat16)
        slots = torch.arange(s, s + n, dtype=torch.int64, device=dev)
        write(k, v, k_cache, v_cache, slots, static)
