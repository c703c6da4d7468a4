"""Parity of the HIP kernels (through the C ABI) with the CPU oracle and the reference's golden vectors.

Bars: cache codes, q codes and dequantized pages bit-exact; attention within max-abs 2e-2, mean-abs
2e-3 and rel_l2 5e-3 of implementation B (Cfg(p_tile=32), kvq/int8_ref.py) in bf16; long rows of a
mixed batch within rel_l2 1e-2 of implementation A (tests/test_cuda_kernels.py:119 of the reference).
"""
import os

import numpy as np
import pytest
import torch
from conftest import nan_like, nan_segm, q_code_flips, record

import cases
from oracle import c_oracle
from oracle import kvq_oracle as O
from kvq import cuda_kernels as ck
from kvq import synth

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATOL_MAX, ATOL_MEAN, REL_L2 = 2e-2, 2e-3, 5e-3


def dev(x):
    if isinstance(x, dict):
        return {k: dev(v) for k, v in x.items()}
    return x.to(DEV) if isinstance(x, torch.Tensor) else x


def int8_cache(c):
    st = c["static"]
    return O.quantize(c["k"].float() - st["k_mu"], st["k_scale"]), O.quantize(c["v"], st["v_scale"])


def oracle_attention(c, kq, vq, per_channel=True, short_q=8, q_arith="fp32"):
    """Implementation B (p_tile 32) for the short requests, A for the long ones, evaluated with fp32
    output (q passed as float32 -- the same values as the bf16 q). q_arith "fp32" is the kernel's q
    contract; "fp64" is int8_ref's own q rounding (the golden fixtures)."""
    cfg = {(True, "fp32"): O.CFG32_Q32, (False, "fp32"): O.CFG32_HEAD_Q32,
           (True, "fp64"): O.CFG32, (False, "fp64"): O.CFG32_HEAD}[(per_channel, q_arith)]
    return O.paged_static_attention(cfg, c["static"], True, short_q)(c["q"].float(), kq, vq, c["cu"], c["seq_lens"],
                                                                     c["block_table"], c["scale"])


def check_attention(ref, out, what, ref_fp64=None, **kw):
    """Strict bar (BASELINE): max-abs <= 2e-2, mean-abs <= 2e-3 of the bf16 kernel output against B in
    fp32 with the kernel's q contract; plus the reference's own bar (rel_l2 < 5e-3,
    tests/test_cuda_kernels.py:75) against int8_ref's fp64 q rounding when given."""
    err = O.compare(ref, out.cpu())
    record(what, **kw, **err)
    assert err["max_abs"] <= ATOL_MAX and err["mean_abs"] <= ATOL_MEAN and err["rel_l2"] < REL_L2, (what, kw, err)
    if ref_fp64 is not None:
        e64 = O.compare(ref_fp64, out.cpu())
        record(what + "_vs_fp64_q", **kw, **e64)
        assert e64["rel_l2"] < REL_L2, (what, kw, e64)
    return err


def short_rows(cu, limit=ck.SHORT_Q):
    q_lens = (cu[1:] - cu[:-1]).long()
    return torch.repeat_interleave(q_lens <= limit, q_lens)


# ------------------------------------------------------------------ quant + cache write
@pytest.fixture(params=["rows", "lanes"])
def qc_kernel(request, monkeypatch):
    """The fused cache write's two kernels (KVQ_QC_KERNEL): the wavefront-row kernel (the default where
    a token's channels are whole wavefronts; other shapes take the lane kernel) and the lane kernel."""
    monkeypatch.setenv("KVQ_QC_KERNEL", request.param)
    return request.param


@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("per_channel", [True, False])
def test_quant_cache_matches_oracle(per_channel, D, qc_kernel):
    """tests/test_cuda_kernels.py:26-43 of the reference: vLLM's [nb, H, bs, 2D] layout, 8 padded key
    rows, every 17th slot -1, keys x5; codes bit-exact."""
    r = synth.rng(0)
    T, H, nb, bs = 200, 4, 64, 16
    key = synth.bf16(r.standard_normal((T + 8, H, D)) * 5)
    value = synth.bf16(r.standard_normal((T + 8, H, D)))
    slots = torch.from_numpy(r.permutation(nb * bs)[:T].astype(np.int64))
    slots[::17] = -1
    st = synth.scales_from(key[:T], value[:T], per_channel)
    kv = torch.zeros(nb, H, bs, 2 * D, dtype=torch.int8)
    kc, vc = kv.transpose(1, 2).split(D, dim=-1)
    O.quant_cache_ref(key, value, kc, vc, slots, st)
    kv_d = torch.zeros(nb, H, bs, 2 * D, dtype=torch.int8, device=DEV)
    kc_d, vc_d = kv_d.transpose(1, 2).split(D, dim=-1)
    ck.quant_reshape_and_cache(dev(key), dev(value), kc_d, vc_d, dev(slots), dev(st))
    assert torch.equal(kv_d.cpu(), kv)


@pytest.mark.parametrize("H,D", [(8, 128), (12, 128), (32, 128), (16, 64), (2, 128), (1, 64)])
@pytest.mark.parametrize("layout", ["interleaved", "separate"])
def test_quant_cache_head_counts_and_packed_qkv(H, D, layout, qc_kernel):
    """Head counts whose channels fill 1, 2, 3 or 8 wavefronts per token (the wavefront-row kernel)
    and fewer than one (the lane kernel); K/V are strided views of a packed qkv activation
    [T, Hq + 2H, D], the cache vLLM's interleaved [nb, H, bs, 2D] or two separate [nb, bs, H, D]
    caches. 7 padded rows at the end, every 13th slot -1; codes bit-exact. Slot 0 is never a target:
    a padded row's store (which the wavefront-row kernel issues and the hardware drops) would land
    there if it were not dropped."""
    r = synth.rng(H * 1000 + D)
    T, nb, bs, Hq = 300, 48, 16, 2 * H
    qkv = synth.bf16(r.standard_normal((T + 7, Hq + 2 * H, D)) * 3)
    key, value = qkv[:, Hq:Hq + H], qkv[:, Hq + H:]
    slots = torch.from_numpy(1 + r.permutation(nb * bs - 1)[:T].astype(np.int64))
    slots[::13] = -1
    st = synth.scales_from(key[:T], value[:T], per_channel=(H % 2 == 0))
    if layout == "interleaved":
        kv = torch.zeros(nb, H, bs, 2 * D, dtype=torch.int8)
        kc, vc = kv.transpose(1, 2).split(D, dim=-1)
        kv_d = torch.zeros_like(kv, device=DEV)
        kc_d, vc_d = kv_d.transpose(1, 2).split(D, dim=-1)
    else:
        kc, vc = torch.zeros(nb, bs, H, D, dtype=torch.int8), torch.zeros(nb, bs, H, D, dtype=torch.int8)
        kc_d, vc_d = torch.zeros_like(kc, device=DEV), torch.zeros_like(vc, device=DEV)
    O.quant_cache_ref(key, value, kc, vc, slots, st)
    qkv_d = qkv.to(DEV)
    ck.quant_reshape_and_cache(qkv_d[:, Hq:Hq + H], qkv_d[:, Hq + H:], kc_d, vc_d, dev(slots), dev(st))
    assert torch.equal(kc_d.cpu(), kc) and torch.equal(vc_d.cpu(), vc)


def test_quant_cache_c1_full_size_bit_exact(qc_kernel):
    """BASELINE config c1: 16384 tokens x 4 x 128, ~2% padded slots, 4096 x 16 interleaved cache."""
    c = synth.c1_inputs()
    nb, bs = c["num_blocks"], c["block_size"]
    kv = torch.zeros(nb, 4, bs, 256, dtype=torch.int8)
    kc, vc = kv.transpose(1, 2).split(128, dim=-1)
    O.quant_cache_ref(c["key"], c["value"], kc, vc, c["slots"], c["static"])
    kv_d = torch.zeros_like(kv, device=DEV)
    kc_d, vc_d = kv_d.transpose(1, 2).split(128, dim=-1)
    ck.quant_reshape_and_cache(dev(c["key"]), dev(c["value"]), kc_d, vc_d, dev(c["slots"]), dev(c["static"]))
    assert torch.equal(kv_d.cpu(), kv)
    # the C restatement agrees on the valid rows as well
    ok = c["slots"] >= 0
    rows = c_oracle.quant_rows(c["key"][ok], c["static"]["k_mu"], c["static"]["k_scale"])
    s = c["slots"][ok]
    assert torch.equal(kc[s // bs, s % bs], rows)


def test_quant_cache_rounding_boundaries(qc_kernel):
    """Quotients on and within a few ulp of half-integers (where a rounding of x * (1/s) that is not
    corrected to fl(x / s) would go wrong), and saturation: bit-exact against the IEEE C restatement."""
    r = synth.rng(2)
    n, H, D = 512, 4, 128
    k = torch.from_numpy(r.integers(-140, 140, (n, H, D)).astype(np.float32) + 0.5) * 0.25   # exact ties
    x = synth.bf16(k.numpy())
    s_pc = torch.full((H, D), 0.25)
    near = synth.bf16(r.standard_normal((n, H, D)) * 10)
    kk = torch.from_numpy(np.round(near.float().numpy() / 0.0731) + 0.5).float()
    s_near = (near.float() / kk).abs().clamp(min=1e-3)[0].contiguous()   # per-channel scales making rows near ties
    for key, ks in ((x, s_pc), (near, s_near)):
        st = {"k_scale": ks, "v_scale": ks.clone(), "k_mu": torch.zeros(H, D)}
        kc = torch.zeros(n // 16, 16, H, D, dtype=torch.int8, device=DEV)
        vc = torch.zeros_like(kc)
        slots = torch.arange(n, dtype=torch.int64)
        ck.quant_reshape_and_cache(dev(key), dev(key), kc, vc, dev(slots), dev(st))
        ref = c_oracle.quant_rows(key, None, ks)
        assert torch.equal(kc.cpu().reshape(n, H, D), ref)
        assert torch.equal(vc.cpu().reshape(n, H, D), ref)



def test_quant_cache_saturates_infinite_and_overflowing_quotients(qc_kernel):
    """K/V rows holding +-inf, the largest bf16 values and ordinary values, with scales small enough that
    x / s overflows to +-inf for some of them: every such code saturates to +-127, as IEEE division
    then rint and the clamp give (the kernel clamps its first quotient estimate so that no NaN can
    appear in the correction). Bit-exact against the C restatement and the torch oracle."""
    r = synth.rng(5)
    n, H, D = 64, 4, 128
    x = r.standard_normal((n, H, D)).astype(np.float32) * 4
    special = np.array([np.inf, -np.inf, 3.38e38, -3.38e38, 1e30, -1e30, 0.0, -0.0], dtype=np.float32)
    idx = r.integers(0, n * H * D, 4096)
    x.reshape(-1)[idx] = special[r.integers(0, len(special), idx.size)]
    key = synth.bf16(x)
    for s in (torch.full((H, D), 0.05), torch.full((H, D), 1e-30), torch.from_numpy(r.uniform(1e-3, 2.0, (H, D)).astype(np.float32))):
        st = {"k_scale": s.contiguous(), "v_scale": s.contiguous(), "k_mu": torch.zeros(H, D)}
        kc = torch.zeros(n // 16, 16, H, D, dtype=torch.int8, device=DEV)
        vc = torch.zeros_like(kc)
        slots = torch.arange(n, dtype=torch.int64)
        ck.quant_reshape_and_cache(dev(key), dev(key), kc, vc, dev(slots), dev(st))
        ref = c_oracle.quant_rows(key, None, s)
        assert torch.equal(ref, O.quantize(key.float(), s)), "the two oracles agree"
        assert torch.equal(kc.cpu().reshape(n, H, D), ref)
        assert torch.equal(vc.cpu().reshape(n, H, D), ref)


# ------------------------------------------------------------------ q quantization
@pytest.mark.parametrize("group", [128, 32])
@pytest.mark.parametrize("per_channel", [True, False])
def test_quant_q_matches_oracle(group, per_channel):
    """tests/test_cuda_kernels.py:46-55: 37 x 28 x 128, codes bit-exact, scales equal."""
    r = synth.rng(1)
    q = synth.bf16(r.standard_normal((37, 28, 128)))
    ks = torch.from_numpy((r.random((4, 128 if per_channel else 1)) + 0.01).astype(np.float32))
    qi, qs = ck.quant_q(dev(q), dev(ks), group)
    ci, cs = c_oracle.quant_q(q, ks, group)
    assert torch.equal(qi.cpu(), ci) and torch.equal(qs.cpu(), cs)


# ------------------------------------------------------------------ attention: golden vectors
@pytest.mark.parametrize("name", cases.NAMES)
def test_attention_matches_reference_golden(golden, name):
    """Kernel output vs the reference's own implementation B output (fixture), plus the bf16-golden
    drift (compare() against paged_attention_ref on the original bf16 K/V) where the fixture has it."""
    g, _ = golden
    c = cases.build(name)
    kq, vq = int8_cache(c)
    d = dev(c)
    out = nan_like(d["q"])
    if name == "mixed":
        plan = ck.plan_long(c["cu"], c["seq_lens"], 16)
        ck.paged_attention(d["q"], dev(kq), dev(vq), out, d["cu"], d["seq_lens"], d["block_table"],
                           int((c["cu"][1:] - c["cu"][:-1]).max()), c["scale"], d["static"], plan)
    else:
        ck.decode_attention(d["q"], dev(kq), dev(vq), out, d["cu"], d["seq_lens"], d["block_table"], c["scale"],
                            d["static"], max_query_len=int((c["cu"][1:] - c["cu"][:-1]).max()))
    rows = cases.stored_rows(name, c["cu"])
    o = out.cpu()[rows]
    short = short_rows(c["cu"])[rows]
    ref = g[f"{name}|int8_b"]                      # the reference's B (fp64 q rounding), bf16
    e = O.compare(ref[short], o[short])
    # rows whose q codes the fp32 q contract and int8_ref's fp64 q rounding break differently
    # (test_oracle_fp32_q_matches_golden_off_flipped_rows: the oracle's fp32 variant deviates there alike)
    flips = q_code_flips(c)[rows][short]
    dev_row = (o[short].float() - ref[short].float()).abs().amax(-1)
    e_flip = float(dev_row[flips].max()) if flips.any() else 0.0
    record("golden_int8_b", case=name, flipped_rows=int(flips.sum()), max_abs_flipped=e_flip, **e)
    # against the reference's own fp64-q output: its rel_l2 bar and the strict mean bar over every short
    # row, the strict max bar on every row whose q codes agree
    assert e["rel_l2"] < REL_L2 and e["mean_abs"] <= ATOL_MEAN, e
    assert float(dev_row[~flips].max()) <= ATOL_MAX, (float(dev_row[~flips].max()), e)
    strict = oracle_attention(c, kq, vq, c["per_channel"])[rows]
    check_attention(strict[short], o[short], "golden_case_vs_fp32q_oracle", case=name)
    if (~short).any():
        assert O.compare(ref[~short], o[~short])["rel_l2"] < 1e-2
    if f"{name}|bf16_ref" in g:
        # reported, not a parity bar: the distance of the INT8 path from bf16 attention on the original
        # K/V (large for the c0 distribution, whose high-gain channels sharpen the softmax); it must be
        # the reference B's own drift up to the kernel-vs-B difference
        drift = O.compare(g[f"{name}|bf16_ref"], o)
        record("bf16_golden_drift", case=name, **drift)
        ref_drift = O.compare(g[f"{name}|bf16_ref"], ref)
        assert abs(drift["rel_l2"] - ref_drift["rel_l2"]) < 0.01, (drift, ref_drift)


@pytest.mark.parametrize("name", cases.WITH_QGROUP32)
@pytest.mark.parametrize("split", [False, True])
def test_attention_qgroup32_matches_reference_golden(golden, name, split):
    """q scales per 32 channels (q_group=32: the B_*_qgroup32 configurations, kvq/int8_ref.py:120-129)
    against the reference's own output (fixture, rel_l2 bar of the reference's tests) and the oracle's
    fp32-q group path (strict bar); head_dim 64 and 128, decode to 8-token rows, with and without split
    buffers, and a mixed batch whose long rows take the dequantize + prefill path."""
    g, _ = golden
    c = cases.build(name)
    kq, vq = int8_cache(c)
    d = dev(c)
    out = nan_like(d["q"])
    T, hq, D = d["q"].shape
    maxq = int((c["cu"][1:] - c["cu"][:-1]).max())
    segm = nan_segm(T, hq, 16, D) if split else None
    if name == "mixed":
        plan = ck.plan_long(c["cu"], c["seq_lens"], 16)
        ck.paged_attention(d["q"], dev(kq), dev(vq), out, d["cu"], d["seq_lens"], d["block_table"], maxq, c["scale"],
                           d["static"], plan, segm, q_group=32)
    else:
        ck.decode_attention(d["q"], dev(kq), dev(vq), out, d["cu"], d["seq_lens"], d["block_table"], c["scale"],
                            d["static"], segm=segm, max_query_len=maxq, q_group=32)
    rows = cases.stored_rows(name, c["cu"])
    o = out.cpu()[rows]
    short = short_rows(c["cu"])[rows]
    ref = g[f"{name}|int8_b_qgroup32"]
    e = O.compare(ref[short], o[short])
    record("golden_int8_b_qgroup32", case=name, split=split, **e)
    assert e["rel_l2"] < REL_L2, e
    strict = O.paged_static_attention(O.CFG32_G32_Q32, c["static"], True, 8)(
        c["q"].float(), kq, vq, c["cu"], c["seq_lens"], c["block_table"], c["scale"])[rows]
    check_attention(strict[short], o[short], "qgroup32_vs_fp32q_oracle", case=name, split=split)
    if (~short).any():
        assert O.compare(ref[~short], o[~short])["rel_l2"] < 1e-2


# ------------------------------------------------------------------ attention: reference test matrix
SHAPES = [(28, 4, 128), (12, 2, 128), (32, 8, 128), (16, 1, 128), (14, 2, 64), (16, 4, 64)]
CASES = {"decode": ([1] * 12, [17, 300, 1, 1024, 2047, 64, 129, 900, 3000, 5, 333, 1500]),
         "short": cases.SHORT}


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("case", ["decode", "short"])
@pytest.mark.parametrize("variant", ["single", "segments", "per_head"])
def test_short_queries_match_oracle(shape, case, variant):
    """tests/test_cuda_kernels.py:58-75: decode and <= 8-token causal queries, head_dim 128 / 64,
    single pass / 16 split segments / per-head scales."""
    hq, hkv, d = shape
    q_lens, seq_lens = CASES[case]
    c = synth.paged_case(hq, hkv, q_lens, seq_lens, head_dim=d, seed=hq + d, dist="randn", scale=3.0)
    per_channel = variant != "per_head"
    c["static"] = synth.scales_from(c["k"].reshape(-1, hkv, d), c["v"].reshape(-1, hkv, d), per_channel)
    c["scale"] = d ** -0.5
    kq, vq = int8_cache(c)
    ref = oracle_attention(c, kq, vq, per_channel)
    ref64 = oracle_attention(c, kq, vq, per_channel, q_arith="fp64")
    dc = dev(c)
    T = c["q"].shape[0]
    segm = None
    if variant == "segments":
        segm = nan_segm(T, hq, 16, d)
    out = ck.decode_attention(dc["q"], dev(kq), dev(vq), nan_like(dc["q"]), dc["cu"], dc["seq_lens"],
                              dc["block_table"], c["scale"], dc["static"], segm=segm, max_query_len=max(q_lens))
    check_attention(ref, out, "short_queries", ref_fp64=ref64, heads=list(shape), case=case, variant=variant)


def test_kernel_leaves_long_requests_alone():
    c = synth.paged_case(28, 4, *cases.MIXED, seed=3, dist="randn", scale=3.0)
    c["static"] = synth.scales_from(c["k"].reshape(-1, 4, 128), c["v"].reshape(-1, 4, 128))
    kq, vq = int8_cache(c)
    d = dev(c)
    out = torch.full_like(d["q"], 7.0)
    ck.decode_attention(d["q"], dev(kq), dev(vq), out, d["cu"], d["seq_lens"], d["block_table"], 128 ** -0.5,
                        d["static"], max_query_len=300)
    short = short_rows(c["cu"])
    o = out.cpu()
    assert (o[~short] == 7.0).all() and not (o[short] == 7.0).any()


@pytest.mark.parametrize("S", [2, 3, 16, 64])
def test_split_counts_agree(S):
    """Any split of the context gives the single-pass result up to fp32 reassociation; empty splits
    (more splits than 32-key tiles) are handled."""
    c = synth.paged_case(28, 4, [1, 1, 1, 4], [5000, 40, 1, 2100], seed=S, params=synth.channel_params(4, 128))
    c["static"] = synth.calibration_scales(4, 128, synth.channel_params(4, 128))
    c["scale"] = 128 ** -0.5
    kq, vq = int8_cache(c)
    d = dev(c)
    args = (d["q"], dev(kq), dev(vq))
    rest = (d["cu"], d["seq_lens"], d["block_table"], 128 ** -0.5, d["static"])
    T = d["q"].shape[0]
    one = ck.decode_attention(*args, nan_like(d["q"]), *rest, max_query_len=4).cpu()
    segm = nan_segm(T, 28, S, 128)
    many = ck.decode_attention(*args, nan_like(d["q"]), *rest, segm=segm, max_query_len=4).cpu()
    err = O.compare(one, many)
    record("split_vs_single", S=S, **err)
    assert err["rel_l2"] < 1e-3 and err["max_abs"] <= 1e-2
    check_attention(oracle_attention(c, kq, vq), many, "split_vs_oracle", S=S)


def test_no_split_buffers_means_one_pass_and_no_allocation():
    """Without split buffers decode_attention / paged_attention (no long requests) cut nothing and take no
    memory from torch's allocator (the reference runs S = 1 then, kvq/cuda/int8_kv.cu:612-613); the
    output matches the oracle, long skewed requests included."""
    c = synth.paged_case(28, 4, [1, 8, 1, 3, 1], [9000, 700, 1, 2100, 33], seed=21, params=synth.channel_params(4, 128))
    c["static"] = synth.calibration_scales(4, 128, synth.channel_params(4, 128))
    c["scale"] = 128 ** -0.5
    kq, vq = int8_cache(c)
    d = dev(c)
    kq_d, vq_d = dev(kq), dev(vq)
    outs = [nan_like(d["q"]), nan_like(d["q"])]
    ck.ext()
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    ck.decode_attention(d["q"], kq_d, vq_d, outs[0], d["cu"], d["seq_lens"], d["block_table"], c["scale"],
                        d["static"], max_query_len=8)
    ck.paged_attention(d["q"], kq_d, vq_d, outs[1], d["cu"], d["seq_lens"], d["block_table"], 8, c["scale"],
                       d["static"])
    torch.cuda.synchronize()
    assert torch.cuda.max_memory_allocated() == before and torch.cuda.memory_allocated() == before
    ref = oracle_attention(c, kq, vq)
    for i, o in enumerate(outs):
        check_attention(ref, o, "one_pass_no_alloc", call=i)
    assert torch.equal(outs[0], outs[1])


SPLIT_ROW_BATCHES = {
    # verification rows (56 per kv head: the 32-row kernel) around a long request
    "verify": ([1, 4, 40, 8, 1, 3, 1, 1], [6000, 3000, 500, 9000, 2100, 7000, 33, 12000], 8),
    # decode rows (the 16-row kernel with key splits) around a long request
    "decode": ([1, 1, 1, 40, 1, 1, 1, 1, 1, 1], [6000, 3000, 9000, 500, 2100, 7000, 33, 12000, 1, 4000], 1),
}


@pytest.mark.parametrize("batch", list(SPLIT_ROW_BATCHES))
@pytest.mark.parametrize("rows", [0, 1, 5, 13, 22])
def test_split_buffers_with_fewer_rows_than_tokens(batch, rows):
    """Split buffers of R < T token rows (kvq_int8_decode_attention_ex): requests whose tokens all lie
    below R may be cut, the others run whole; every short row matches the oracle, long requests are left
    alone, and nothing is written past the buffers' R rows."""
    q_lens, seq_lens, maxq = SPLIT_ROW_BATCHES[batch]
    c = synth.paged_case(28, 4, q_lens, seq_lens, seed=41, params=synth.channel_params(4, 128))
    c["static"] = synth.calibration_scales(4, 128, synth.channel_params(4, 128))
    c["scale"] = 128 ** -0.5
    kq, vq = int8_cache(c)
    d = dev(c)
    T = d["q"].shape[0]
    assert rows < T
    full = nan_segm(rows + 2, 28, 8, 128)
    segm = tuple(t[:rows] for t in full)
    out = torch.full_like(d["q"], 7.0)
    ck.decode_attention(d["q"], dev(kq), dev(vq), out, d["cu"], d["seq_lens"], d["block_table"], c["scale"],
                        d["static"], segm=segm, max_query_len=maxq)
    torch.cuda.synchronize()
    for t in full:
        assert torch.isnan(t[rows:]).all()
    short = short_rows(c["cu"])
    o = out.cpu()
    assert (o[~short] == 7.0).all()
    ref = oracle_attention(c, kq, vq)
    check_attention(ref[short], o[short], "split_rows_below_tokens", batch=batch, rows=rows)


@pytest.mark.parametrize("reported", [1, 3])
def test_split_merge_covers_underreported_max_query_len(reported):
    """A caller that reports a smaller max_query_len than the batch holds still gets every row of every
    cut request merged (the merge grid walks all query tokens of a request)."""
    c = synth.paged_case(28, 4, [8, 5, 8, 1], [6000, 4100, 300, 5000], seed=31, params=synth.channel_params(4, 128))
    c["static"] = synth.calibration_scales(4, 128, synth.channel_params(4, 128))
    c["scale"] = 128 ** -0.5
    kq, vq = int8_cache(c)
    d = dev(c)
    T = d["q"].shape[0]
    out = ck.decode_attention(d["q"], dev(kq), dev(vq), nan_like(d["q"]), d["cu"], d["seq_lens"], d["block_table"],
                              c["scale"], d["static"], segm=nan_segm(T, 28, 32, 128), max_query_len=reported)
    assert torch.isfinite(out.float()).all()
    check_attention(oracle_attention(c, kq, vq), out, "underreported_max_query_len", reported=reported)


# ------------------------------------------------------------------ mixed batches (long path)
@pytest.mark.parametrize("shape", [(28, 4, 128), (12, 2, 128), (14, 2, 64)])
@pytest.mark.parametrize("case", ["mixed", "prefill", "serving"])
@pytest.mark.parametrize("per_channel", [True, False])
def test_mixed_batch_matches_oracle(shape, case, per_channel):
    """tests/test_cuda_kernels.py:100-119: long requests via dequant_pages + bf16 attention, short
    ones via the INT8 kernel."""
    hq, hkv, d = shape
    if case == "mixed":
        q_lens, seq_lens = cases.MIXED
    elif case == "prefill":
        q_lens, seq_lens = [256, 97], [256, 1200]
    else:
        r = synth.rng(11)
        ql = [int(x) for x in r.integers(39, 74, 68)] + [1] * 188
        sl = [n + int(r.integers(0, 20)) for n in ql[:68]] + [int(x) for x in r.integers(100, 400, 188)]
        perm = r.permutation(256)
        q_lens, seq_lens = [ql[i] for i in perm], [sl[i] for i in perm]
    c = synth.paged_case(hq, hkv, q_lens, seq_lens, head_dim=d, seed=5, dist="randn", scale=3.0)
    c["static"] = synth.scales_from(c["k"].reshape(-1, hkv, d), c["v"].reshape(-1, hkv, d), per_channel)
    c["scale"] = d ** -0.5
    kq, vq = int8_cache(c)
    ref = oracle_attention(c, kq, vq, per_channel)
    ref64 = oracle_attention(c, kq, vq, per_channel, q_arith="fp64")
    plan = ck.plan_long(c["cu"], c["seq_lens"], 16)
    assert plan is not None and plan.has_short == (case != "prefill")
    dc = dev(c)
    out = ck.paged_attention(dc["q"], dev(kq), dev(vq), nan_like(dc["q"]), dc["cu"], dc["seq_lens"],
                             dc["block_table"], max(q_lens), c["scale"], dc["static"], plan).cpu()
    short = short_rows(c["cu"])
    res = {"long": O.compare(ref[~short], out[~short])["rel_l2"]}
    if short.any():
        res["short"] = O.compare(ref[short], out[short])["rel_l2"]
        check_attention(ref[short], out[short], "mixed_short", ref_fp64=ref64[short], heads=list(shape), case=case)
    record("mixed_batch", heads=list(shape), case=case, per_channel=per_channel, **res)
    assert res["long"] < 1e-2


def test_long_path_uses_gpu_lengths():
    """Host lengths may be upper bounds: the plan copies extra pages, attention uses the GPU lengths."""
    c = synth.paged_case(28, 4, *cases.MIXED, seed=6, dist="randn", scale=3.0)
    c["static"] = synth.scales_from(c["k"].reshape(-1, 4, 128), c["v"].reshape(-1, 4, 128))
    c["scale"] = 128 ** -0.5
    kq, vq = int8_cache(c)
    ref = oracle_attention(c, kq, vq)
    bt = torch.cat([c["block_table"], c["block_table"][:, :1].expand(-1, 2)], 1)
    plan = ck.plan_long(c["cu"], c["seq_lens"] + 5, 16)
    dc = dev(c)
    out = ck.paged_attention(dc["q"], dev(kq), dev(vq), nan_like(dc["q"]), dc["cu"], dc["seq_lens"],
                             dev(bt), 300, c["scale"], dc["static"], plan).cpu()
    assert O.compare(ref, out)["rel_l2"] < 1e-2


@pytest.mark.parametrize("per_channel", [True, False])
@pytest.mark.parametrize("D", [128, 64])
def test_dequant_pages_bit_exact(per_channel, D):
    c = synth.paged_case(16, 4, [20, 1, 40], [300, 50, 700], head_dim=D, seed=9, dist="randn", scale=3.0)
    c["static"] = synth.scales_from(c["k"].reshape(-1, 4, D), c["v"].reshape(-1, 4, D), per_channel)
    kq, vq = int8_cache(c)
    plan = ck.plan_long(c["cu"], c["seq_lens"], 16)
    src_req, src_j = torch.from_numpy(plan.src_req), torch.from_numpy(plan.src_j)
    ko_ref, vo_ref = O.dequant_pages_ref(kq, vq, c["block_table"], src_req, src_j, c["static"])
    P = src_req.shape[0]
    ko = torch.full((P, 16, 4, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    vo = nan_like(ko)
    ck.ext().dequant_pages(dev(kq), dev(vq), ko, vo, dev(c["block_table"]), dev(src_req), dev(src_j),
                           dev(c["static"]["k_scale"]), dev(c["static"]["v_scale"]))
    assert torch.equal(ko.cpu().view(torch.int16), ko_ref.view(torch.int16))
    assert torch.equal(vo.cpu().view(torch.int16), vo_ref.view(torch.int16))


def test_dequant_pages_vllm_layout():
    """Interleaved [nb, H, bs, 2D] cache views, as the backend hands them over."""
    c = synth.paged_case(28, 4, [33], [400], seed=10, dist="randn", scale=3.0)
    c["static"] = synth.scales_from(c["k"].reshape(-1, 4, 128), c["v"].reshape(-1, 4, 128))
    kq, vq = int8_cache(c)
    kv = torch.cat([kq, vq], -1).transpose(1, 2).contiguous()           # [nb, H, bs, 2D]
    kc_d, vc_d = dev(kv).transpose(1, 2).split(128, dim=-1)
    plan = ck.plan_long(c["cu"], c["seq_lens"], 16)
    src_req, src_j = torch.from_numpy(plan.src_req), torch.from_numpy(plan.src_j)
    ko_ref, vo_ref = O.dequant_pages_ref(kq, vq, c["block_table"], src_req, src_j, c["static"])
    ko = torch.full((src_req.shape[0], 16, 4, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    vo = nan_like(ko)
    ck.ext().dequant_pages(kc_d, vc_d, ko, vo, dev(c["block_table"]), dev(src_req), dev(src_j),
                           dev(c["static"]["k_scale"]), dev(c["static"]["v_scale"]))
    assert torch.equal(ko.cpu().view(torch.int16), ko_ref.view(torch.int16))
    assert torch.equal(vo.cpu().view(torch.int16), vo_ref.view(torch.int16))


def _random_pages(nb, bs, H, D, P, seed, per_channel):
    """Random int8 caches [nb, bs, H, D], a one-row block table of P distinct random blocks, the
    page list (request 0, pages 0..P-1) and scales."""
    g = torch.Generator().manual_seed(seed)
    kq = torch.randint(-127, 128, (nb, bs, H, D), generator=g, dtype=torch.int8)
    vq = torch.randint(-127, 128, (nb, bs, H, D), generator=g, dtype=torch.int8)
    bt = torch.randperm(nb, generator=g)[:P].to(torch.int32).reshape(1, P)
    src_req, src_j = torch.zeros(P, dtype=torch.int32), torch.arange(P, dtype=torch.int32)
    shape = (H, D) if per_channel else (H, 1)
    st = {"k_scale": torch.rand(shape, generator=g) * 0.05 + 1e-3, "v_scale": torch.rand(shape, generator=g) * 0.05 + 1e-3,
          "k_mu": torch.zeros(H, D)}
    return kq, vq, bt, src_req, src_j, st


def _check_dequant(kq, vq, bt, src_req, src_j, st):
    ko_ref, vo_ref = O.dequant_pages_ref(kq, vq, bt, src_req, src_j, st)
    P, (_, bs, H, D) = src_req.shape[0], kq.shape
    ko = torch.full((P, bs, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    vo = nan_like(ko)
    ck.ext().dequant_pages(dev(kq), dev(vq), ko, vo, dev(bt), dev(src_req), dev(src_j), dev(st["k_scale"]),
                           dev(st["v_scale"]))
    assert torch.equal(ko.cpu().view(torch.int16), ko_ref.view(torch.int16))
    assert torch.equal(vo.cpu().view(torch.int16), vo_ref.view(torch.int16))


@pytest.mark.parametrize("D,bs", [(128, 8), (128, 16), (128, 32), (64, 16), (64, 32), (64, 64), (128, 4), (64, 8)])
def test_dequant_pages_block_sizes(D, bs):
    """Block sizes from 4 to 64 rows at both head dims (one or several 4-row passes of the kernel per
    page, a partial last pass at bs 8 / D 64); per-head scales at bs 16; bit-exact."""
    _check_dequant(*_random_pages(400, bs, 4, D, 300, seed=bs * 7 + D, per_channel=(bs != 16)))


def test_attention_on_vllm_interleaved_layout():
    c = synth.c0_case()
    kq, vq = int8_cache(c)
    kv = torch.cat([kq, vq], -1).transpose(1, 2).contiguous()
    kc_d, vc_d = dev(kv).transpose(1, 2).split(128, dim=-1)
    d = dev(c)
    out = ck.decode_attention(d["q"], kc_d, vc_d, nan_like(d["q"]), d["cu"], d["seq_lens"],
                              d["block_table"], 128 ** -0.5, d["static"])
    check_attention(oracle_attention(c | {"scale": 128 ** -0.5}, kq, vq), out, "vllm_layout")


# ------------------------------------------------------------------ stream-K coverage
def _serving_batch(hq=12, hkv=2, d=128):
    """256 requests: 188 decode rows (L 100..399) and 68 long requests the INT8 kernel skips."""
    r = synth.rng(11)
    ql = [int(x) for x in r.integers(39, 74, 68)] + [1] * 188
    sl = [n + int(r.integers(0, 20)) for n in ql[:68]] + [int(x) for x in r.integers(100, 400, 188)]
    perm = r.permutation(256)
    return synth.paged_case(hq, hkv, [ql[i] for i in perm], [sl[i] for i in perm], head_dim=d, seed=5,
                            dist="randn", scale=3.0)


@pytest.fixture(scope="module")
def serving():
    c = _serving_batch()
    c["static"] = synth.scales_from(c["k"].reshape(-1, 2, 128), c["v"].reshape(-1, 2, 128), True)
    c["scale"] = 128 ** -0.5
    kq, vq = int8_cache(c)
    ref = oracle_attention(c, kq, vq)
    return c, dev(kq), dev(vq), ref, short_rows(c["cu"])


@pytest.mark.parametrize("target_waves", [0, 3, 1001, 2045])
@pytest.mark.parametrize("splits", [1, 4, 64])
def test_every_worker_count_covers_the_batch(serving, target_waves, splits):
    """Every unit of the batch is computed whatever the number of persistent workgroups (here 682, 1,
    333 and 681 workgroups of 3 wavefronts: none a multiple of the 8 XCDs) and split cap; outputs and
    partial buffers start as NaN, so a skipped worker would show."""
    c, kq, vq, ref, short = serving
    d = dev(c)
    T = d["q"].shape[0]
    os.environ["KVQ_TARGET_WAVES"] = str(target_waves)
    try:
        if splits == 1:
            out = ck.decode_attention(d["q"], kq, vq, nan_like(d["q"]), d["cu"], d["seq_lens"], d["block_table"],
                                      c["scale"], d["static"], max_query_len=73)
        else:
            out = ck.decode_attention(d["q"], kq, vq, nan_like(d["q"]), d["cu"], d["seq_lens"], d["block_table"],
                                      c["scale"], d["static"], segm=nan_segm(T, 12, splits, 128), max_query_len=73)
    finally:
        del os.environ["KVQ_TARGET_WAVES"]
    out = out.cpu()[short]
    assert torch.isfinite(out.float()).all(), (target_waves, splits)
    check_attention(ref[short], out, "worker_coverage", target_waves=target_waves, splits=splits)


@pytest.mark.parametrize("kind", ["decode", "verify"])
@pytest.mark.parametrize("fast_max", [None, "1"])
def test_plan_beyond_cached_requests_and_64bit_scans(fast_max, kind):
    """A batch of 300 requests (more than the plan keeps in registers: the locate scan reloads requests
    256..299) gives the same result with the plan's 32-bit DPP scans and with its 64-bit shuffle scans
    (KVQ_PLAN_FAST_MAX=1 forces them) -- the same partition, bit for bit -- and matches the oracle; decode
    rows run the 16-row kernel, verification rows the 32-row one."""
    r = synth.rng(23)
    q_lens = [1] * 280 + ([1] * 20 if kind == "decode" else [int(x) for x in r.integers(2, 9, 20)])
    seq_lens = [int(x) for x in r.integers(1, 1500, 300)]
    c = synth.paged_case(28, 4, q_lens, seq_lens, seed=29, params=synth.channel_params(4, 128))
    c["static"] = synth.calibration_scales(4, 128, synth.channel_params(4, 128))
    c["scale"] = 128 ** -0.5
    kq, vq = int8_cache(c)
    d = dev(c)
    T = d["q"].shape[0]
    outs = []
    for env in (None, fast_max):
        if env is not None:
            os.environ["KVQ_PLAN_FAST_MAX"] = env
        try:
            outs.append(ck.decode_attention(d["q"], dev(kq), dev(vq), nan_like(d["q"]), d["cu"], d["seq_lens"],
                                            d["block_table"], c["scale"], d["static"], segm=nan_segm(T, 28, 16, 128),
                                            max_query_len=max(q_lens)).cpu())
        finally:
            os.environ.pop("KVQ_PLAN_FAST_MAX", None)
    assert torch.equal(outs[0], outs[1])
    check_attention(oracle_attention(c, kq, vq), outs[1], "plan_300_requests", fast_max=fast_max, kind=kind)


# ------------------------------------------------------------------ concurrent streams
def test_two_streams_merge_independently():
    """Two streams run split attention on different batches at the same time (each with its own split
    buffers); both results match their single-stream runs exactly: a launch keeps no state between or
    across calls."""
    cs = []
    for seed in (1, 2):
        c = synth.paged_case(28, 4, [1] * 24 + [3] * 8, [int(x) for x in synth.rng(seed).integers(200, 3000, 32)],
                             seed=seed, params=synth.channel_params(4, 128))
        c["static"] = synth.calibration_scales(4, 128, synth.channel_params(4, 128))
        kq, vq = int8_cache(c)
        cs.append((dev(c), dev(kq), dev(vq)))

    def run(i, out):
        d, kq, vq = cs[i]
        T = d["q"].shape[0]
        return ck.decode_attention(d["q"], kq, vq, out, d["cu"], d["seq_lens"], d["block_table"], 128 ** -0.5, d["static"],
                                   segm=nan_segm(T, 28, 16, 128), max_query_len=3)

    ref = [run(i, nan_like(cs[i][0]["q"])).clone() for i in range(2)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [nan_like(cs[i][0]["q"]) for i in range(2)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for rep in range(20):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                run(i, outs[i])
    for s in streams:
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(outs[i], ref[i]), i


# ------------------------------------------------------------------ key splits inside a workgroup
@pytest.mark.parametrize("q_len", [1, 2, 3, 5])
@pytest.mark.parametrize("segm", [False, True])
def test_key_split_workgroups_agree(q_len, segm):
    """Rows of one (request, kv head) split over 4 / 2 / 1 wavefronts of a workgroup (by query length:
    7, 14, 21, 35 rows) and merged through LDS give the unsplit result (KVQ_KSPLIT=1) up to fp32
    reassociation, and both match the oracle."""
    lens = [4100, 33, 1, 517, 2048, 90, 1200, 16]
    c = synth.paged_case(28, 4, [q_len] * 8, [max(L, q_len) for L in lens], seed=40 + q_len,
                         params=synth.channel_params(4, 128))
    c["static"] = synth.calibration_scales(4, 128, synth.channel_params(4, 128))
    c["scale"] = 128 ** -0.5
    kq, vq = int8_cache(c)
    d = dev(c)
    T = d["q"].shape[0]

    def run():
        return ck.decode_attention(d["q"], dev(kq), dev(vq), nan_like(d["q"]), d["cu"], d["seq_lens"], d["block_table"],
                                   c["scale"], d["static"], segm=nan_segm(T, 28, 16, 128) if segm else None,
                                   max_query_len=q_len).cpu()
    split = run()
    os.environ["KVQ_KSPLIT"] = "1"
    try:
        plain = run()
    finally:
        del os.environ["KVQ_KSPLIT"]
    e = O.compare(plain, split)
    record("ksplit_vs_plain", q_len=q_len, segm=segm, **e)
    assert torch.isfinite(split.float()).all() and e["rel_l2"] < 1e-3 and e["max_abs"] <= 1e-2, e
    check_attention(oracle_attention(c, kq, vq), split, "ksplit_vs_oracle", q_len=q_len)


# ------------------------------------------------------------------ block sizes beyond 16
@pytest.mark.parametrize("bs", [32, 64])
@pytest.mark.parametrize("H,D", [(4, 128), (2, 64), (3, 128)])
def test_quant_cache_block_sizes(bs, H, D, qc_kernel):
    """Cache blocks of 32 and 64 slots (vLLM's other block sizes), interleaved layout; both kernels
    (H x D a multiple of 512 or not); codes bit-exact."""
    r = synth.rng(bs * 100 + H * 10 + D)
    T, nb = 500, 24
    key = synth.bf16(r.standard_normal((T, H, D)) * 4)
    value = synth.bf16(r.standard_normal((T, H, D)))
    slots = torch.from_numpy(r.permutation(nb * bs)[:T].astype(np.int64))
    slots[::11] = -1
    st = synth.scales_from(key, value, per_channel=True)
    kv = torch.zeros(nb, H, bs, 2 * D, dtype=torch.int8)
    kc, vc = kv.transpose(1, 2).split(D, dim=-1)
    O.quant_cache_ref(key, value, kc, vc, slots, st)
    kv_d = torch.zeros_like(kv, device=DEV)
    kc_d, vc_d = kv_d.transpose(1, 2).split(D, dim=-1)
    ck.quant_reshape_and_cache(dev(key), dev(value), kc_d, vc_d, dev(slots), dev(st))
    assert torch.equal(kv_d.cpu(), kv)


@pytest.mark.parametrize("bs", [32, 64])
@pytest.mark.parametrize("shape", [(28, 4, 128), (14, 2, 64), (32, 8, 128)])
@pytest.mark.parametrize("case", ["decode", "short"])
def test_attention_block_sizes(bs, shape, case):
    """Decode rows (the register-ring kernel) and up-to-8-token causal queries (the LDS-ring kernel
    when a (request, kv head) has more than 32 rows) over caches of 32- and 64-slot blocks, with and
    without split buffers: against the oracle at the attention bar."""
    hq, hkv, d = shape
    q_lens, seq_lens = CASES[case]
    c = synth.paged_case(hq, hkv, q_lens, seq_lens, head_dim=d, block_size=bs, seed=bs + hq + d, dist="randn",
                         scale=3.0)
    c["static"] = synth.scales_from(c["k"].reshape(-1, hkv, d), c["v"].reshape(-1, hkv, d), True)
    c["scale"] = d ** -0.5
    kq, vq = int8_cache(c)
    ref = oracle_attention(c, kq, vq, True)
    ref64 = oracle_attention(c, kq, vq, True, q_arith="fp64")
    dc = dev(c)
    T = c["q"].shape[0]
    for segm in (None, nan_segm(T, hq, 8, d)):
        out = ck.decode_attention(dc["q"], dev(kq), dev(vq), nan_like(dc["q"]), dc["cu"], dc["seq_lens"],
                                  dc["block_table"], c["scale"], dc["static"], segm=segm,
                                  max_query_len=max(q_lens))
        check_attention(ref, out, "block_sizes", ref_fp64=ref64, heads=list(shape), case=case, bs=bs)


def test_attention_events_hook_times_one_call():
    """kvq_set_attention_events (no counterpart in the reference; bench.py's timing hook): the next
    decode_attention call records the pair around its attention kernel on its stream and forgets it,
    so a later call records nothing into the same events; the output is unaffected."""
    import ctypes
    from kvq import _native
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventQuery.argtypes = [ctypes.c_void_p]
    ev = [ctypes.c_void_p(), ctypes.c_void_p()]
    for e in ev:
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
    try:
        c = synth.paged_case(28, 4, [1] * 6, [300, 1000, 4000, 17, 2047, 64], seed=5, dist="randn", scale=3.0)
        c["static"] = synth.scales_from(c["k"].reshape(-1, 4, 128), c["v"].reshape(-1, 4, 128), True)
        kq, vq = int8_cache(c)
        dc = dev(c)
        lib = _native.load()
        assert lib.kvq_set_attention_events(ev[0], ev[1]) == 0
        out1 = ck.decode_attention(dc["q"], dev(kq), dev(vq), nan_like(dc["q"]), dc["cu"], dc["seq_lens"],
                                   dc["block_table"], 128 ** -0.5, dc["static"])
        torch.cuda.synchronize()
        ms = ctypes.c_float()
        assert hip.hipEventElapsedTime(ctypes.byref(ms), ev[0], ev[1]) == 0 and ms.value > 0
        first = ms.value
        out2 = ck.decode_attention(dc["q"], dev(kq), dev(vq), nan_like(dc["q"]), dc["cu"], dc["seq_lens"],
                                   dc["block_table"], 128 ** -0.5, dc["static"])
        torch.cuda.synchronize()
        assert hip.hipEventElapsedTime(ctypes.byref(ms), ev[0], ev[1]) == 0 and ms.value == first  # not re-recorded
        assert torch.equal(out1, out2)
    finally:
        for e in ev:
            hip.hipEventDestroy(e)


@pytest.mark.parametrize("nbytes,wg", [(1 << 20, 64), ((1 << 20) + 48, 7), (16, 1), (5 * 4096 + 16, 2048)])
def test_stream_read_probe_reads_every_word_once(nbytes, wg):
    """kvq_stream_read (bench.py's read-ceiling probe, no counterpart in the reference): the XOR of the
    lanes' outputs is the XOR of every 32-bit word of the buffer, whatever the grid."""
    from kvq import _native
    g = torch.Generator().manual_seed(nbytes + wg)
    host = torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), generator=g, dtype=torch.int32)
    buf = host.to(DEV)
    out = torch.full((wg * 256,), 0x5A5A5A5A, dtype=torch.int32, device=DEV)
    _native.call("kvq_stream_read", buf.data_ptr(), nbytes, out.data_ptr(), wg, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(host.numpy().view(np.uint32))


@pytest.mark.parametrize("rd,wr,wg", [(2 << 20, 1 << 20, 64), (1 << 20, 2 << 20, 7), (4096 * 3, 4096 * 3, 5),
                                      (32, 16, 1), ((1 << 20) + 32, (1 << 19) + 16, 1000)])
def test_stream_rw_probe_writes_exactly_its_bytes(rd, wr, wg):
    """kvq_stream_rw (bench.py's read + write floor, no counterpart in the reference): every 16-byte chunk of
    the destination is written and nothing past it, whatever the grid and ratio; other ratios are refused."""
    from kvq import _native
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (rd // 4,), dtype=torch.int32, device=DEV)
    dst = torch.full((wr // 4 + 64,), 0x5A5A5A5A, dtype=torch.int32, device=DEV)
    _native.call("kvq_stream_rw", src.data_ptr(), rd, dst.data_ptr(), wr, wg, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    chunks = dst[:wr // 4].view(-1, 4).cpu()
    assert not (chunks == 0x5A5A5A5A).all(dim=1).any()
    assert (dst[wr // 4:] == 0x5A5A5A5A).all()
    with pytest.raises(_native.NativeError, match="ratio|2 : 1"):
        _native.call("kvq_stream_rw", src.data_ptr(), 48, dst.data_ptr(), 16, 1, torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("H,D", [(4, 128), (2, 64), (3, 128)])
def test_stream_scatter_probe_writes_the_cache_writes_bytes(H, D):
    """kvq_stream_scatter (bench.py's cache-write floor, no counterpart in the reference): exactly the cache
    rows the fused write fills (valid slots of the interleaved layout), each byte the bf16's high byte."""
    from kvq import _native
    r = synth.rng(H * 1000 + D)
    T, nb, bs = 301, 40, 16
    key = torch.from_numpy(r.integers(-2 ** 15, 2 ** 15, (T, H, D)).astype(np.int16)).to(DEV)
    value = torch.from_numpy(r.integers(-2 ** 15, 2 ** 15, (T, H, D)).astype(np.int16)).to(DEV)
    slots = torch.from_numpy(r.permutation(nb * bs)[:T].astype(np.int64))
    slots[::7] = -1
    kv = torch.zeros(nb, H, bs, 2 * D, dtype=torch.int8, device=DEV)
    kc, vc = kv.transpose(1, 2).split(D, dim=-1)
    _native.call("kvq_stream_scatter", key.data_ptr(), key.stride(0), key.stride(1), value.data_ptr(), value.stride(0),
                 value.stride(1), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2),
                 slots.to(DEV).data_ptr(), T, H, D, nb, bs, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    want = torch.zeros(nb, bs, H, 2 * D, dtype=torch.int8)
    ok = slots >= 0
    hi = lambda x: (x.cpu()[ok].view(torch.uint8).reshape(-1, H, D, 2)[..., 1]).view(torch.int8)
    want[slots[ok] // bs, slots[ok] % bs] = torch.cat([hi(key), hi(value)], -1)
    assert torch.equal(kv.transpose(1, 2).cpu(), want)


@pytest.mark.parametrize("wg_per_cu", ["1", "2"])
def test_quant_cache_ring_path_bit_exact(monkeypatch, wg_per_cu):
    """The wavefront-row kernel's token ring (more tokens per wavefront than it keeps in flight at
    once), forced by a small grid (KVQ_QC_WG_PER_CU): c1's full input, codes bit-exact."""
    monkeypatch.setenv("KVQ_QC_WG_PER_CU", wg_per_cu)
    c = synth.c1_inputs()
    nb, bs = c["num_blocks"], c["block_size"]
    n = c["slots"].shape[0] - 5                          # not a multiple of the wavefront count
    kv = torch.zeros(nb, 4, bs, 256, dtype=torch.int8)
    kc, vc = kv.transpose(1, 2).split(128, dim=-1)
    O.quant_cache_ref(c["key"], c["value"], kc, vc, c["slots"][:n], c["static"])
    kv_d = torch.zeros_like(kv, device=DEV)
    kc_d, vc_d = kv_d.transpose(1, 2).split(128, dim=-1)
    ck.quant_reshape_and_cache(dev(c["key"]), dev(c["value"]), kc_d, vc_d, dev(c["slots"][:n]), dev(c["static"]))
    assert torch.equal(kv_d.cpu(), kv)


# ------------------------------------------------------------------ 32-row verification wavefronts
@pytest.mark.parametrize("shape", [(28, 4, 128, [8, 5, 8, 6]), (32, 4, 128, [5, 8, 3, 8]), (28, 4, 64, [8, 8, 5, 7]),
                                   (64, 4, 128, [8, 3, 6, 1]), (14, 1, 128, [4, 8, 3, 8])])
@pytest.mark.parametrize("split", [False, True])
def test_rows32_kernel_matches_the_16_row_kernel(shape, split):
    """Batches with more than 32 (token, q head) rows per kv head run 32-row wavefronts on the 32x32 int8
    MFMA (verify_kernel): the same per-element arithmetic as the 16-row tiles (KVQ_ROWS32=0), so the
    outputs agree to bf16 rounding, and both match the oracle; G x q_len of 35..512 rows, head_dim 64
    and 128, with and without split buffers."""
    hq, hkv, d, q_lens = shape
    lens = [3000, 700, 64 * 32 + 5, 17]
    c = synth.paged_case(hq, hkv, q_lens, [max(L, q) for L, q in zip(lens, q_lens)], head_dim=d, seed=hq + d,
                         params=synth.channel_params(hkv, d))
    c["static"] = synth.calibration_scales(hkv, d, synth.channel_params(hkv, d))
    c["scale"] = d ** -0.5
    kq, vq = int8_cache(c)
    dd = dev(c)
    T = dd["q"].shape[0]

    def run():
        return ck.decode_attention(dd["q"], dev(kq), dev(vq), nan_like(dd["q"]), dd["cu"], dd["seq_lens"],
                                   dd["block_table"], c["scale"], dd["static"],
                                   segm=nan_segm(T, hq, 16, d) if split else None, max_query_len=max(q_lens)).cpu()
    new = run()
    os.environ["KVQ_ROWS32"] = "0"
    try:
        old = run()
    finally:
        del os.environ["KVQ_ROWS32"]
    assert torch.isfinite(new.float()).all()
    e = O.compare(old, new)
    record("rows32_vs_rows16", shape=str(shape), split=split, **e)
    assert e["max_abs"] <= 1e-2 and e["rel_l2"] < 1e-3, e
    check_attention(oracle_attention(c, kq, vq), new, "rows32_vs_oracle", shape=str(shape), split=split)
