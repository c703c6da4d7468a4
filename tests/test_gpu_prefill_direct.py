"""KVQ_PREFILL_DIRECT: the long requests' attention read straight from the INT8 pages
(kvq_int8_prefill_attention) instead of dequant_pages followed by the bf16 prefill kernel.

=1: each 32-key tile is converted in LDS with dequant_pages' arithmetic, (bf16)(code x scale), and then
runs the bf16 kernel's MFMA sequence, so the bar is bit-identity with the two-kernel path on the same
inputs (rows outside the work list stay NaN in both). The two-kernel path itself is checked against the
oracle and fp32 attention in test_gpu_kernels.py and test_gpu_prefill.py.
=fold: the scales folded into q and the output (tests at the end of this file)."""
import pytest
import torch
from conftest import nan_like, record

import cases
from kvq import cuda_kernels as ck
from kvq import synth
from test_gpu_kernels import dev, int8_cache

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _both_paths(q, kc, vc, cu, sl, bt, plan, max_q, scale, st, monkeypatch):
    """long_attention's output through the two-kernel path and through the direct one."""
    outs = []
    for direct in ("0", "1"):
        monkeypatch.setenv("KVQ_PREFILL_DIRECT", direct)
        out = nan_like(q)
        ck.long_attention(q, kc, vc, out, cu, sl, bt, max_q, plan, scale, st)
        outs.append(out)
    torch.cuda.synchronize()
    return outs


def _check_identical(two, direct, cu, what, **kw):
    long_rows = torch.repeat_interleave((cu[1:] - cu[:-1]).cpu() > ck.SHORT_Q, (cu[1:] - cu[:-1]).cpu().long())
    assert torch.isfinite(two[long_rows.to(two.device)].float()).all(), (what, kw)
    same = torch.equal(two.view(torch.int16), direct.view(torch.int16))
    diff = (two.float() - direct.float()).abs().nan_to_num(0.0).max().item()
    record("prefill_direct_bits", what=what, identical=same, max_abs_diff=diff, **kw)
    assert same, (what, kw, diff)


@pytest.mark.parametrize("shape", [(28, 4, 128), (12, 2, 128), (14, 2, 64), (32, 8, 128)])
@pytest.mark.parametrize("case", ["mixed", "prefill"])
@pytest.mark.parametrize("per_channel", [True, False])
def test_direct_prefill_bit_identical(shape, case, per_channel, monkeypatch):
    """Pages in random order (the block table is read per tile), per-channel and per-head scales,
    both head dims, short requests left alone."""
    hq, hkv, d = shape
    q_lens, seq_lens = cases.MIXED if case == "mixed" else ([256, 97, 40], [256, 1200, 3001])
    c = synth.paged_case(hq, hkv, q_lens, seq_lens, head_dim=d, seed=21, dist="randn", scale=3.0)
    c["static"] = synth.scales_from(c["k"].reshape(-1, hkv, d), c["v"].reshape(-1, hkv, d), per_channel)
    kq, vq = int8_cache(c)
    plan = ck.plan_long(c["cu"], c["seq_lens"], 16)
    dc = dev(c)
    two, direct = _both_paths(dc["q"], dev(kq), dev(vq), dc["cu"], dc["seq_lens"], dc["block_table"], plan,
                              max(q_lens), d ** -0.5, dc["static"], monkeypatch)
    _check_identical(two, direct, dc["cu"], "random_pages", shape=list(shape), case=case, per_channel=per_channel)


@pytest.mark.parametrize("layout", ["vllm_interleaved", "consecutive_pages", "bs32", "bs64", "host_upper_bound"])
def test_direct_prefill_layouts(layout, monkeypatch):
    """vLLM's interleaved [nb, H, bs, 2D] cache views (page stride beyond block_size slots); a cache
    whose requests own consecutive page ids (the kernel reads them without the block table); larger
    blocks (one or two pages per tile); host lengths that over-state the keys (the device lengths
    rule)."""
    hq, hkv, d = 28, 4, 128
    bs = {"bs32": 32, "bs64": 64}.get(layout, 16)
    q_lens, seq_lens = [300, 1, 64, 17], [1000, 40, 2100, 17]
    c = synth.paged_case(hq, hkv, q_lens, seq_lens, head_dim=d, block_size=bs, seed=22, dist="randn", scale=3.0)
    c["static"] = synth.scales_from(c["k"].reshape(-1, hkv, d), c["v"].reshape(-1, hkv, d), True)
    kq, vq = int8_cache(c)
    bt = c["block_table"]
    if layout == "consecutive_pages":            # request r's logical page j -> physical first[r] + j
        npg = [-(-L // bs) for L in seq_lens]
        first = torch.cumsum(torch.tensor([0] + npg[:-1]), 0)
        perm = torch.zeros(kq.shape[0], dtype=torch.long)
        new_bt = torch.zeros_like(bt)
        kq2, vq2 = torch.zeros_like(kq), torch.zeros_like(vq)
        for r, n in enumerate(npg):
            for j in range(n):
                kq2[first[r] + j] = kq[bt[r, j]]
                vq2[first[r] + j] = vq[bt[r, j]]
                new_bt[r, j] = int(first[r]) + j
        kq, vq, bt = kq2, vq2, new_bt
    kc_d, vc_d = dev(kq), dev(vq)
    if layout == "vllm_interleaved":
        kv = torch.cat([kq, vq], -1).transpose(1, 2).contiguous()       # [nb, H, bs, 2D]
        kc_d, vc_d = dev(kv).transpose(1, 2).split(d, dim=-1)
    host_sl = c["seq_lens"] + (5 if layout == "host_upper_bound" else 0)
    if layout == "host_upper_bound":
        bt = torch.cat([bt, bt[:, :1].expand(-1, 2)], 1)
    plan = ck.plan_long(c["cu"], host_sl, bs)
    dc = dev(c)
    two, direct = _both_paths(dc["q"], kc_d, vc_d, dc["cu"], dc["seq_lens"], dev(bt), plan, max(q_lens), d ** -0.5,
                              dc["static"], monkeypatch)
    _check_identical(two, direct, dc["cu"], "layout", layout=layout)


def test_direct_prefill_score_jump(monkeypatch):
    """One key past the first tile whose scores exceed the first tile's by far more than 2^60 (log2
    units): the fast pass hands the workgroup to the rescaling pass, which converts its tiles again."""
    hq, hkv, d, bs = 28, 4, 128, 16
    q_lens, seq_lens = [200, 40], [1000, 300]
    g = torch.Generator().manual_seed(23)
    nb = 200
    kq = torch.randint(-20, 21, (nb, bs, hkv, d), generator=g, dtype=torch.int8)
    vq = torch.randint(-127, 128, (nb, bs, hkv, d), generator=g, dtype=torch.int8)
    bt = torch.randperm(nb, generator=g)[:2 * 63].to(torch.int32).reshape(2, 63)
    for r, key in ((0, 850), (1, 130)):
        kq[bt[r, key // bs], key % bs] = 127
    st = {"k_scale": torch.full((hkv, d), 0.1), "v_scale": torch.rand(hkv, d, generator=g) * 0.02 + 1e-3}
    cu = torch.tensor([0, 200, 240], dtype=torch.int32)
    sl = torch.tensor(seq_lens, dtype=torch.int32)
    q = (torch.randn(240, hq, d, generator=g) + 0.5).to(torch.bfloat16)
    plan = ck.plan_long(cu, sl, bs)
    two, direct = _both_paths(dev(q), dev(kq), dev(vq), dev(cu), dev(sl), dev(bt), plan, 200, d ** -0.5, dev(st),
                              monkeypatch)
    _check_identical(two, direct, dev(cu), "score_jump")


def test_direct_prefill_c4_full_size(monkeypatch):
    """c4's prefill part at full size: 4 requests x 16384 tokens (q_len = L), heads 32 / 8, vLLM's
    interleaved INT8 cache filled by the cache-write kernel, pages in random order."""
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
    two, direct = _both_paths(q, kc, vc, cu.to(DEV), sl.to(DEV), bt, plan, Q, d ** -0.5, st, monkeypatch)
    _check_identical(two, direct, cu.to(DEV), "c4_full_size")


def test_direct_prefill_allocates_no_temporary_cache(monkeypatch):
    """The direct path's peak memory over a long batch stays below the temporary cache's size."""
    hq, hkv, d, bs = 32, 8, 128, 16
    Q = L = 4096
    nb = L // bs + 8
    kq = torch.randint(-127, 128, (nb, bs, hkv, d), dtype=torch.int8, device=DEV)
    vq = torch.randint(-127, 128, (nb, bs, hkv, d), dtype=torch.int8, device=DEV)
    st = {"k_scale": torch.full((hkv, 1), 0.01, device=DEV), "v_scale": torch.full((hkv, 1), 0.01, device=DEV)}
    bt = torch.arange(L // bs, dtype=torch.int32, device=DEV).reshape(1, -1)
    q = torch.randn(Q, hq, d, device=DEV).to(torch.bfloat16)
    cu = torch.tensor([0, Q], dtype=torch.int32)
    sl = torch.tensor([L], dtype=torch.int32)
    plan = ck.plan_long(cu, sl, bs)
    out = nan_like(q)
    temp_bytes = 2 * plan.src_req.shape[0] * bs * hkv * d * 2
    for mode in ("1", "fold"):
        monkeypatch.setenv("KVQ_PREFILL_DIRECT", mode)
        ck.long_attention(q, kq, vq, out, cu.to(DEV), sl.to(DEV), bt, Q, plan, d ** -0.5, st)   # warm (work list)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        ck.long_attention(q, kq, vq, out, cu.to(DEV), sl.to(DEV), bt, Q, plan, d ** -0.5, st)
        torch.cuda.synchronize()
        extra = torch.cuda.max_memory_allocated() - base
        record("prefill_direct_memory", mode=mode, extra_bytes=int(extra), temp_cache_bytes=int(temp_bytes))
        assert extra < temp_bytes // 16, (mode, extra, temp_bytes)


# ------------------------------------------------------------------ KVQ_PREFILL_DIRECT=fold
# The codes are converted exactly and the scales move: k_scale into q (one bf16 rounding of q x k_scale
# per q element, in place of one of code x k_scale per K element) and v_scale onto the fp32 output (no
# rounding of code x v_scale at all). Not bit-identical to the two-kernel path, so it is held to the
# oracle's long-row bar and to fp32 attention over the fp32-dequantized pages -- where it must be no
# less accurate than the two-kernel path.

@pytest.mark.parametrize("shape", [(28, 4, 128), (14, 2, 64), (32, 8, 128)])
@pytest.mark.parametrize("per_channel", [True, False])
def test_fold_mixed_batch_matches_oracle(shape, per_channel, monkeypatch):
    """Long rows of a mixed batch against implementation A of the oracle at the reference's long-row bar
    (rel_l2 < 1e-2, tests/test_cuda_kernels.py:119, as test_mixed_batch_matches_oracle holds the
    two-kernel path to); short rows untouched by the long path."""
    from oracle import kvq_oracle as O
    from test_gpu_kernels import oracle_attention, short_rows
    hq, hkv, d = shape
    q_lens, seq_lens = cases.MIXED
    c = synth.paged_case(hq, hkv, q_lens, seq_lens, head_dim=d, seed=24, dist="randn", scale=3.0)
    c["static"] = synth.scales_from(c["k"].reshape(-1, hkv, d), c["v"].reshape(-1, hkv, d), per_channel)
    c["scale"] = d ** -0.5
    kq, vq = int8_cache(c)
    ref = oracle_attention(c, kq, vq, per_channel)
    plan = ck.plan_long(c["cu"], c["seq_lens"], 16)
    dc = dev(c)
    monkeypatch.setenv("KVQ_PREFILL_DIRECT", "fold")
    out = nan_like(dc["q"])
    ck.long_attention(dc["q"], dev(kq), dev(vq), out, dc["cu"], dc["seq_lens"], dc["block_table"], max(q_lens),
                      plan, c["scale"], dc["static"])
    out = out.cpu()
    short = short_rows(c["cu"])
    assert torch.isnan(out[short].float()).all()
    err = O.compare(ref[~short], out[~short])
    record("prefill_fold_vs_oracle", shape=list(shape), per_channel=per_channel, **err)
    assert err["rel_l2"] < 1e-2, err


def _fp32_truth_errors(q, kc, vc, st, bt, outs, Q, B, hq, hkv, d, bs, rows_per_req, seed):
    """Worst max-abs, mean-abs and pooled rel_l2 of each output against fp32 attention over K / V =
    code x scale in fp32 (no bf16 rounding), on sampled rows of each request (q_len = L = Q)."""
    import math
    pages = Q // bs
    rng = synth.rng(seed)
    acc = {k: [0.0, 0.0, 0.0, 0.0, 0] for k in outs}      # max_abs, sum_abs, err^2, ref^2, n
    for r in range(B):
        ids = bt[r, :pages].long()
        k = (kc[ids].float() * st["k_scale"]).reshape(Q, hkv, d)
        v = (vc[ids].float() * st["v_scale"]).reshape(Q, hkv, d)
        kT = k.repeat_interleave(hq // hkv, dim=1).permute(1, 2, 0).contiguous()
        vv = v.repeat_interleave(hq // hkv, dim=1).permute(1, 0, 2).contiguous()
        rows = sorted({0, 1, 15, 16, Q - 1, Q - 2} | set(int(x) for x in rng.integers(0, Q, rows_per_req)))
        for t in rows:
            qi = q[r * Q + t].float()[:, None, :].contiguous()
            s = torch.matmul(qi, kT) / math.sqrt(d)
            s[:, :, t + 1:] = float("-inf")
            o = torch.matmul(torch.softmax(s, dim=-1), vv).squeeze(1)
            for name, out in outs.items():
                e = out[r * Q + t].float() - o
                a = acc[name]
                a[0] = max(a[0], e.abs().max().item())
                a[1] += e.abs().sum().item()
                a[2] += e.pow(2).sum().item()
                a[3] += o.pow(2).sum().item()
                a[4] += e.numel()
    return {k: {"max_abs": a[0], "mean_abs": a[1] / a[4], "rel_l2": (a[2] / a[3]) ** 0.5} for k, a in acc.items()}


def test_fold_c4_full_size_against_fp32(monkeypatch):
    """c4's prefill part at full size (4 x 16384 tokens, heads 32 / 8): the folded path within the
    long-row bar of fp32 attention over the exact dequantized values, and no less accurate there than
    dequant_pages + the bf16 kernel."""
    hq, hkv, d, bs = 32, 8, 128, 16
    Q = L = 16384
    B = 4
    pages = L // bs
    nb = B * pages + 32
    params = synth.channel_params(hkv, d)
    st = {k: v.to(DEV) for k, v in synth.calibration_scales(hkv, d, params).items()}
    kv = torch.empty(nb, hkv, bs, 2 * d, dtype=torch.int8, device=DEV)
    kc, vc = kv.transpose(1, 2).split(d, dim=-1)
    synth.fill_cache_gpu(kc, vc, st, params, seed=71, write=ck.quant_reshape_and_cache)
    bt = synth.random_block_table(B, [pages] * B, nb, 72, DEV)
    g = torch.Generator(device=DEV).manual_seed(73)
    q = torch.randn(B * Q, hq, d, generator=g, device=DEV).to(torch.bfloat16)
    cu = torch.arange(B + 1, dtype=torch.int32) * Q
    sl = torch.full((B,), L, dtype=torch.int32)
    plan = ck.plan_long(cu, sl, bs)
    outs = {}
    for mode in ("0", "fold"):
        monkeypatch.setenv("KVQ_PREFILL_DIRECT", mode)
        out = nan_like(q)
        ck.long_attention(q, kc, vc, out, cu.to(DEV), sl.to(DEV), bt, Q, plan, d ** -0.5, st)
        outs[mode] = out
    torch.cuda.synchronize()
    err = _fp32_truth_errors(q, kc, vc, st, bt, outs, Q, B, hq, hkv, d, bs, 26, seed=74)
    record("prefill_fold_c4_vs_fp32", fold=err["fold"], two_kernel=err["0"])
    assert err["fold"]["rel_l2"] < 1e-2 and err["fold"]["max_abs"] <= 4e-2, err
    assert err["fold"]["mean_abs"] <= err["0"]["mean_abs"] and err["fold"]["rel_l2"] <= err["0"]["rel_l2"], err


def test_fold_score_jump(monkeypatch):
    """The rescaling pass with folded scales: outlier keys past the first tile (as
    test_direct_prefill_score_jump), against fp32 attention over the exact dequantized values."""
    import math
    hq, hkv, d, bs = 28, 4, 128, 16
    g = torch.Generator().manual_seed(23)
    nb = 200
    kq = torch.randint(-20, 21, (nb, bs, hkv, d), generator=g, dtype=torch.int8)
    vq = torch.randint(-127, 128, (nb, bs, hkv, d), generator=g, dtype=torch.int8)
    bt = torch.randperm(nb, generator=g)[:2 * 63].to(torch.int32).reshape(2, 63)
    for r, key in ((0, 850), (1, 130)):
        kq[bt[r, key // bs], key % bs] = 127
    st = {"k_scale": torch.full((hkv, d), 0.1), "v_scale": torch.rand(hkv, d, generator=g) * 0.02 + 1e-3}
    q_lens, seq_lens = [200, 40], [1000, 300]
    cu = torch.tensor([0, 200, 240], dtype=torch.int32)
    sl = torch.tensor(seq_lens, dtype=torch.int32)
    q = (torch.randn(240, hq, d, generator=g) + 0.5).to(torch.bfloat16)
    plan = ck.plan_long(cu, sl, bs)
    monkeypatch.setenv("KVQ_PREFILL_DIRECT", "fold")
    out = nan_like(dev(q))
    ck.long_attention(dev(q), dev(kq), dev(vq), out, dev(cu), dev(sl), dev(bt), 200, plan, d ** -0.5, dev(st))
    out = out.cpu().float()
    worst = 0.0
    for r in range(2):
        Qr, L = q_lens[r], seq_lens[r]
        npg = -(-L // bs)
        k = (kq[bt[r, :npg].long()].float() * st["k_scale"]).reshape(-1, hkv, d)[:L]
        v = (vq[bt[r, :npg].long()].float() * st["v_scale"]).reshape(-1, hkv, d)[:L]
        for t in range(Qr):
            qi = q[int(cu[r]) + t].float()
            kk = k[:L - Qr + 1 + t].repeat_interleave(hq // hkv, dim=1).permute(1, 2, 0)
            vv = v[:L - Qr + 1 + t].repeat_interleave(hq // hkv, dim=1).permute(1, 0, 2)
            p = torch.softmax(torch.matmul(qi[:, None, :], kk) / math.sqrt(d), dim=-1)
            o = torch.matmul(p, vv).squeeze(1)
            worst = max(worst, (out[int(cu[r]) + t] - o).abs().max().item())
    record("prefill_fold_score_jump", max_abs=worst)
    assert torch.isfinite(out[:240]).all() and worst <= 2e-2, worst
