#!/usr/bin/env python3
"""Benchmark of the static INT8 KV-cache hot path on one MI355X.

Headline (BASELINE.json metric, config c2): INT8 paged decode attention, 128 requests x 32768 keys,
28 q / 4 kv heads, head_dim 128, block 16, in vLLM's interleaved [nb, H, bs, 2D] int8 cache (filled
with c0-distribution codes by this package's quantize-and-cache kernel), shuffled block tables over
263,168 blocks. A step is one kvq.cuda_kernels.decode_attention call made as the vLLM backend makes it
for this batch when it runs eagerly or under piecewise graphs: its per-step split rule
(cuda_kernels.split_pays) sees 128 requests x 4 kv heads of equal length, two whole (request, kv head)
pairs per CU, and passes no split buffers -- one pass, nothing cut, nothing allocated -- with every input
resident in HBM. Under vLLM's full-graph decode (the backend declares UNIFORM_BATCH) a captured graph
always carries the backend's split buffers, since its replays see other lengths; that call (attention
kernel + split merge) is timed beside it as c2_other_call.

Prints ONE JSON line. `value` is algorithmic bytes / step time (GB/s); `roofline` times the attention
kernel alone with HIP events recorded around it on its own stream; `cpu_baseline` times the CPU oracle
(the reference's implementation B + run_paged restated) on a bounded sample of the same requests and
checks the GPU output of those requests against it. `extra` carries configs c1 (fused quantize +
cache write), c3 (8-token verification) and c4 (Llama-3 mixed batch: decode rows + page dequant).

  python bench.py [--steps K] [--warmup W] [--no-cpu] [--no-extra]
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "int8-kvcache_amd"))

import numpy as np  # noqa: E402
import torch  # noqa: E402

from kvq import _native, synth  # noqa: E402
from kvq import cuda_kernels as ck  # noqa: E402

with open(os.path.join(REPO, "BASELINE.json")) as _f:
    METRIC = json.load(_f)["metric"]
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_GBS = 8000.0          # MI355X HBM3E
PEAK_INT8_OPS = 5.0e15     # dense int8 MFMA
DEV = "cuda"


# ------------------------------------------------------------------------------------------------ HIP events
class HipEvents:
    """Raw hipEvent_t pairs, for timing only: created without the system-scope fence at record
    (hipEventDisableSystemFence), whose cache writeback and invalidation cost ~2.5 us per recorded
    event on these boxes. The library records pairs around its next attention kernel
    (kvq_set_attention_events); record() puts one on a given stream."""

    DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self, n):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.pairs = []
        for _ in range(n):
            a, b = ctypes.c_void_p(), ctypes.c_void_p()
            assert self.hip.hipEventCreateWithFlags(ctypes.byref(a), self.DISABLE_SYSTEM_FENCE) == 0
            assert self.hip.hipEventCreateWithFlags(ctypes.byref(b), self.DISABLE_SYSTEM_FENCE) == 0
            self.pairs.append((a, b))

    def record(self, i, which, stream):
        assert self.hip.hipEventRecord(self.pairs[i][which], ctypes.c_void_p(stream)) == 0

    def elapsed_ms(self, i):
        ms = ctypes.c_float()
        a, b = self.pairs[i]
        assert self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value

    def close(self):
        for a, b in self.pairs:
            self.hip.hipEventDestroy(a)
            self.hip.hipEventDestroy(b)


def interleaved_cache(nb, hkv, bs, d):
    """vLLM's int8 layout [nb, H, bs, 2D] and its K / V views [nb, bs, H, D] (backend.py:145-147)."""
    kv = torch.empty(nb, hkv, bs, 2 * d, dtype=torch.int8, device=DEV)
    kc, vc = kv.transpose(1, 2).split(d, dim=-1)
    return kv, kc, vc


# ------------------------------------------------------------------------------------------------ c2 headline
def build_c2(B=128, L=32768, hq=28, hkv=4, d=128, bs=16):
    pages = L // bs
    nb = B * pages + 1024
    params = synth.channel_params(hkv, d)
    st = {k: v.to(DEV) for k, v in synth.calibration_scales(hkv, d, params).items()}
    kv, kc, vc = interleaved_cache(nb, hkv, bs, d)
    synth.fill_cache_gpu(kc, vc, st, params, seed=3, write=ck.quant_reshape_and_cache)
    bt = synth.random_block_table(B, [pages] * B, nb, 4, DEV)
    g = torch.Generator(device=DEV).manual_seed(5)
    q = torch.randn(B, hq, d, generator=g, device=DEV).to(torch.bfloat16)
    cu = torch.arange(B + 1, dtype=torch.int32, device=DEV)
    sl = torch.full((B,), L, dtype=torch.int32, device=DEV)
    alg = (B * L * hkv * d * 2 + 2 * B * hq * d * 2 + B * pages * 4 + (2 * B + 1) * 4 + 2 * hkv * d * 4)
    return {"q": q, "kc": kc, "vc": vc, "kv": kv, "cu": cu, "sl": sl, "bt": bt, "st": st, "B": B, "L": L,
            "hq": hq, "hkv": hkv, "d": d, "bs": bs, "alg_bytes": alg, "kv_bytes": B * L * hkv * d * 2}


def backend_passes_split_buffers(q_lens, seq_lens, num_kv_heads):
    """Whether the vLLM backend hands the kernel its split buffers for this batch, outside graph capture
    (kvq.vllm_int8.backend Int8StaticBuilder._split_for -> cuda_kernels.split_pays): not for short-query
    requests of even length whose (request, kv head) pairs give every CU a whole number of them."""
    return ck.split_pays(np.asarray(q_lens), np.asarray(seq_lens), num_kv_heads, ck.one_pass_fill(DEV))


def time_c2(w, steps, warmup, split=True):
    """Step time and attention-kernel time of c2. split: the call carries split buffers allocated once
    beforehand, as the vLLM backend's (SPLIT_PIECES pieces per row); otherwise the one-pass call without
    them (nothing cut, nothing allocated).

    The timed region (host clock between two device synchronizations) holds exactly the steps' calls,
    bracketed by one pair of HIP events on the launch stream: their interval / steps is the average
    launch duration of the call's kernels (the one-pass call is one kernel; gaps between launches
    included). Per-kernel durations -- the library's event pair around each attention kernel -- come
    from as many calls again right after, outside the timed region (a recorded event costs ~2.5 us of
    the step even without the system fence)."""
    out = torch.empty_like(w["q"])
    scale = w["d"] ** -0.5
    splits = ck.SPLIT_PIECES if split else 1
    segm = ck.split_buffers(w["B"], w["hq"], w["d"], splits, DEV) if split else None

    def step():
        ck.decode_attention(w["q"], w["kc"], w["vc"], out, w["cu"], w["sl"], w["bt"], scale, w["st"], segm=segm)

    for _ in range(warmup):
        step()
    region = HipEvents(1)
    stream = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    region.record(0, 0, stream)
    for i in range(steps):
        step()
    region.record(0, 1, stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    region_ms = region.elapsed_ms(0) / steps
    region.close()
    ev = HipEvents(steps)
    lib = _native.load()
    for i in range(steps):
        a, b = ev.pairs[i]
        lib.kvq_set_attention_events(a, b)
        step()
    torch.cuda.synchronize()
    kern_ms = [ev.elapsed_ms(i) for i in range(steps)]
    ev.close()
    return out, (t1 - t0) * 1e3 / steps, region_ms, statistics.mean(kern_ms), statistics.median(kern_ms), splits


def read_ceiling(buf, reps=10):
    """GB/s a plain streaming read of `buf` sustains on this device (the library's kvq_stream_read):
    what HBM delivers to a read-only stream, the ceiling beside the attention kernel's rate."""
    nbytes = buf.numel() * buf.element_size() // 16 * 16
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    stream = torch.cuda.current_stream().cuda_stream
    best = (0.0, 0)
    for per_cu in (4, 8):   # the better of two grid sizes
        wg = cus * per_cu
        out = torch.empty(wg * 256, dtype=torch.int32, device=DEV)
        for _ in range(2):
            _native.call("kvq_stream_read", buf.data_ptr(), nbytes, out.data_ptr(), wg, stream)
        ev = HipEvents(reps)
        for i in range(reps):
            ev.record(i, 0, stream)
            _native.call("kvq_stream_read", buf.data_ptr(), nbytes, out.data_ptr(), wg, stream)
            ev.record(i, 1, stream)
        torch.cuda.synchronize()
        ts = [ev.elapsed_ms(i) for i in range(reps)]
        ev.close()
        best = max(best, (nbytes / (statistics.median(ts) * 1e-3) / 1e9, per_cu))
    return best


def mfma_ceiling(reps=5):
    """TFLOP/s of back-to-back dense bf16 MFMAs (the library's kvq_mfma_probe: 16x16x32, the prefill
    kernel's instruction) on random bf16 operands, 8 workgroups of 4 wavefronts per CU, ~7 ms per launch,
    timed as the prefill kernel is (graph replays of 3 calls): the rate the box delivers under its power
    limit over such a burst, the ceiling beside the prefill kernel's rate."""
    g = torch.Generator(device=DEV).manual_seed(11)
    data = torch.randn(8192, generator=g, device=DEV).to(torch.bfloat16)
    wg = torch.cuda.get_device_properties(0).multi_processor_count * 8
    out = torch.empty(wg * 256, dtype=torch.float32, device=DEV)
    iters = 12288
    stream = torch.cuda.current_stream
    ms = _median_event_ms(lambda i: _native.call("kvq_mfma_probe", data.data_ptr(), iters, out.data_ptr(), wg,
                                                 stream().cuda_stream), reps, 1, calls=3)
    return wg * 4 * iters * 8 * 16384 / ms / 1e9, wg


# ------------------------------------------------------------------------------------------------ CPU baseline
def cpu_baseline(w, out, budget_s=12.0, max_reqs=128):
    """The CPU oracle (port of int8_ref B + run_paged) on whole c2 requests until ~budget_s of CPU work;
    also the parity of the GPU output on those requests."""
    sys.path.insert(0, REPO)
    from oracle import kvq_oracle as O

    # every core this process may run on (its affinity mask, which a container's CPU share sets)
    threads = len(os.sched_getaffinity(0)) or 1
    torch.set_num_threads(threads)
    st = {k: v.cpu() for k, v in w["st"].items()}
    f = O.paged_static_attention(O.CFG32_Q32, st, True, 8)
    pages = w["L"] // w["bs"]
    t_total, n, errs, kv_bytes = 0.0, 0, [], 0
    one = torch.tensor([0, 1], dtype=torch.int32)
    while n < max_reqs and t_total < budget_s:
        r = (n * 37) % w["B"]
        ids = w["bt"][r, :pages].long()
        kq, vq = w["kc"][ids].cpu(), w["vc"][ids].cpu()
        q = w["q"][r:r + 1].cpu()
        bt = torch.arange(pages, dtype=torch.int32)[None]
        sl = torch.tensor([w["L"]], dtype=torch.int32)
        t0 = time.perf_counter()
        ref = f(q.float(), kq, vq, one, sl, bt, w["d"] ** -0.5)
        t_total += time.perf_counter() - t0
        kv_bytes += w["L"] * w["hkv"] * w["d"] * 2
        e = O.compare(ref, out[r:r + 1].cpu())
        errs.append(e)
        n += 1
    # one request on one thread
    r = 0
    ids = w["bt"][r, :pages].long()
    kq, vq, q = w["kc"][ids].cpu(), w["vc"][ids].cpu(), w["q"][r:r + 1].cpu()
    bt = torch.arange(pages, dtype=torch.int32)[None]
    sl = torch.tensor([w["L"]], dtype=torch.int32)
    torch.set_num_threads(1)
    t0 = time.perf_counter()
    f(q.float(), kq, vq, one, sl, bt, w["d"] ** -0.5)
    t1_us = (time.perf_counter() - t0) * 1e6
    torch.set_num_threads(threads)
    parity = {"requests_checked": n, "max_abs": max(e["max_abs"] for e in errs),
              "mean_abs": statistics.mean(e["mean_abs"] for e in errs),
              "rel_l2_max": max(e["rel_l2"] for e in errs), "bar": "max_abs<=2e-2, mean_abs<=2e-3"}
    parity["ok"] = parity["max_abs"] <= 2e-2 and parity["mean_abs"] <= 2e-3
    parity["c0_bf16_drift"] = c0_drift(O)
    res = {"value": round(kv_bytes / t_total / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
           "sample": f"{n} whole c2 requests (32768 keys, 28/4/128) through the oracle's implementation B "
                     f"(float64) + run_paged on the host, {t_total:.1f} s; KV bytes / s",
           "us_per_request": round(t_total / n * 1e6, 1), "os_cpu_count": os.cpu_count(),
           "one_thread": {"us_per_request": round(t1_us, 1),
                          "GBps": round(w["L"] * w["hkv"] * w["d"] * 2 / (t1_us * 1e-6) / 1e9, 4)},
           "small_configs": cpu_small_configs(O, threads)}
    torch.set_num_threads(threads)
    return res, parity


def c0_drift(O):
    """The bf16-golden drift (kvq/ref_attn.py:93-102's compare against paged_attention_ref, fp32
    attention over the original bf16 K/V) of the GPU kernel on c0, next to implementation B's own drift
    and the kernel's distance from B. The int8 cache holds K - mu: that shifts every score of a row by
    the same q . mu, so the softmax, and the comparison, are unchanged."""
    c0 = synth.c0_case()
    st = c0["static"]
    kq = O.quantize(c0["k"].float() - st["k_mu"], st["k_scale"])
    vq = O.quantize(c0["v"].float(), st["v_scale"])
    scale = 128 ** -0.5
    args = (c0["cu"], c0["seq_lens"], c0["block_table"], scale)
    b = O.paged_static_attention(O.CFG32_Q32, st, True, 8)(c0["q"].float(), kq, vq, *args)
    gold = O.paged_attention_ref(c0["q"], c0["k"], c0["v"], *args)
    out = torch.empty(c0["q"].shape, dtype=torch.bfloat16, device=DEV)
    ck.decode_attention(c0["q"].to(DEV), kq.to(DEV), vq.to(DEV), out, c0["cu"].to(DEV), c0["seq_lens"].to(DEV),
                        c0["block_table"].to(DEV), scale, {k: v.to(DEV) for k, v in st.items()})
    o = out.cpu()
    rnd = lambda e: {k: round(float(v), 6) for k, v in e.items()}
    return {"kernel_vs_B": rnd(O.compare(b, o)), "kernel_vs_bf16_golden": rnd(O.compare(gold, o)),
            "B_vs_bf16_golden": rnd(O.compare(gold, b))}


def cpu_small_configs(O, threads, reps=5):
    """The oracle on the configurations the host finishes in moments: c0 (4 decode requests x {17, 300,
    1024, 2049}, the whole attention) and c1's quantize + scatter (16384 tokens into the paged cache);
    median wall ms of `reps` runs after one warm-up, with `threads` threads and with one."""
    c0 = synth.c0_case()
    st = c0["static"]
    kq = O.quantize(c0["k"].float() - st["k_mu"], st["k_scale"])
    vq = O.quantize(c0["v"].float(), st["v_scale"])
    f = O.paged_static_attention(O.CFG32_Q32, st, True, 8)
    c1 = synth.c1_inputs()
    kc = torch.zeros(c1["num_blocks"], c1["block_size"], 4, 128, dtype=torch.int8)
    vc = torch.zeros_like(kc)

    def run_c0():
        f(c0["q"].float(), kq, vq, c0["cu"], c0["seq_lens"], c0["block_table"], 128 ** -0.5)

    def run_c1():
        O.quant_cache_ref(c1["key"], c1["value"], kc, vc, c1["slots"], c1["static"])

    out = {}
    for name, fn in (("c0_attention", run_c0), ("c1_quant_cache", run_c1)):
        for nt in (threads, 1):
            torch.set_num_threads(nt)
            fn()
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                fn()
                ts.append((time.perf_counter() - t0) * 1e3)
            out[f"{name}_ms_{nt}t"] = round(statistics.median(ts), 3)
    return out


# ------------------------------------------------------------------------------------------------ extras
def _median_event_ms(fn, reps, rotate, calls=20):
    """Device time per call: `calls` calls (cycling over `rotate` buffer sets) are captured in one HIP
    graph, the graph is replayed `reps` times between fence-free HIP events on the current stream, and
    the median replay time / calls is returned -- the host's per-call launch overhead is not in it."""
    for i in range(rotate):
        fn(i)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(rotate):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(calls):
            fn(i % rotate)
    g.replay()
    torch.cuda.synchronize()
    # untimed replays for ~100 ms first: a GPU that has idled while the host built the workload, or that
    # meets freshly written buffers, runs its first tens of ms of work a few percent slower (c4's decode
    # rows: 123-124 against 119 us per call over the first ~50 ms)
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    for _ in range(max(2, min(4000, int(100e-3 / max(time.perf_counter() - t0, 1e-6))))):
        g.replay()
    torch.cuda.synchronize()
    ev = HipEvents(reps)
    stream = torch.cuda.current_stream().cuda_stream
    for i in range(reps):
        ev.record(i, 0, stream)
        g.replay()
        ev.record(i, 1, stream)
    torch.cuda.synchronize()
    ms = statistics.median(ev.elapsed_ms(i) for i in range(reps)) / calls
    ev.close()
    return ms


def rw_floor(read_bytes, write_bytes, reps=20):
    """Device time of a plain in-order stream that reads `read_bytes` and writes `write_bytes` (the
    library's kvq_stream_rw probe), under the same graph-replay protocol as the kernels it bounds, with
    enough distinct buffer sets to exceed the 256 MB last-level cache; the best of 4, 8 and 16
    workgroups per CU. Returns (us, workgroups per CU)."""
    sets = max(1, -(-300 * 2 ** 20 // (read_bytes + write_bytes)))
    bufs = [(torch.empty(read_bytes // 4, dtype=torch.int32, device=DEV).random_(),
             torch.empty(write_bytes // 4, dtype=torch.int32, device=DEV)) for _ in range(sets)]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    best = None
    for per_cu in (4, 8, 16):
        def fn(i, wg=cus * per_cu):
            src, dst = bufs[i]
            _native.call("kvq_stream_rw", src.data_ptr(), read_bytes, dst.data_ptr(), write_bytes, wg,
                         torch.cuda.current_stream().cuda_stream)
        ms = _median_event_ms(fn, reps, sets)
        if best is None or ms < best[0]:
            best = (ms, per_cu)
    del bufs
    return best[0] * 1e3, best[1]


def _c1_at(T, num_blocks, nsets, reps):
    """Kernel and scatter-floor time of the fused quantize + cache write for T tokens (c0 distribution,
    ~2% padding) into num_blocks x 16 interleaved caches, nsets distinct input / cache sets rotated."""
    sets = []
    for s in range(nsets):
        c = synth.c1_inputs(seed=5 + s, T=T, num_blocks=num_blocks)
        kv, kc, vc = interleaved_cache(c["num_blocks"], 4, c["block_size"], 128)
        sets.append((c["key"].to(DEV), c["value"].to(DEV), kc, vc, c["slots"].to(DEV),
                     {k: v.to(DEV) for k, v in c["static"].items()}))
    t_valid = int((sets[0][4] >= 0).sum())

    def fn(i):
        k, v, kc, vc, sl, st = sets[i]
        ck.quant_reshape_and_cache(k, v, kc, vc, sl, st)

    ms = _median_event_ms(fn, reps, len(sets))

    # the floor: the same bytes read and scattered by slot into the same caches, without the arithmetic
    def scatter(i):
        k, v, kc, vc, sl, st = sets[i]
        _native.call("kvq_stream_scatter", k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0),
                     v.stride(1), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), sl.data_ptr(),
                     sl.shape[0], kc.shape[2], kc.shape[3], kc.shape[0], kc.shape[1],
                     torch.cuda.current_stream().cuda_stream)

    ms_sc = _median_event_ms(scatter, reps, len(sets))
    set_bytes = sum(t.numel() * t.element_size() for t in sets[0][:4])
    del sets
    return ms, ms_sc, t_valid, set_bytes


def bench_c1(reps=20):
    """Fused quantize + cache write, 16384 tokens x 4 x 128, ~2% padding, 4096 x 16 interleaved cache.
    4 distinct input/cache sets (~400 MB) are rotated to defeat the 256 MB last-level cache. The same at
    4x the tokens (65,536 into 16,384 x 16 slots, 2 sets, ~390 MB) shows what the kernel sustains once a
    launch's ramp-up and tail are a smaller share of it."""
    T = 16384
    ms, ms_sc, t_valid, _ = _c1_at(T, 4096, 4, reps)
    alg = t_valid * 3072 + T * 8 + 6144
    # and a plain in-order stream of those bytes (no scatter)
    f_us, f_wg = rw_floor(t_valid * 2048, t_valid * 1024)
    sc_alg = t_valid * 3072
    T4 = 4 * T
    ms4, ms4_sc, t4_valid, set4 = _c1_at(T4, 16384, 2, reps)
    alg4 = t4_valid * 3072 + T4 * 8 + 6144
    return {"us": round(ms * 1e3, 2), "GBps": round(alg / ms / 1e6, 1), "frac": round(alg / ms / 1e6 / PEAK_GBS, 4),
            "alg_bytes": alg, "tokens": T, "valid": t_valid,
            "ceiling": {"us": round(ms_sc * 1e3, 2), "GBps": round(sc_alg / ms_sc / 1e6, 1),
                        "frac_of_peak": round(sc_alg / ms_sc / 1e6 / PEAK_GBS, 4),
                        "kernel_vs_ceiling": round(ms / ms_sc, 3),
                        "how": "kvq_stream_scatter: c1's K/V rows read and one byte per element written through "
                               "slot_mapping into the same interleaved caches (the write's traffic and scatter, no "
                               "arithmetic), same graph replay and rotation"},
            "ceiling_linear": {"us": round(f_us, 2), "GBps": round(sc_alg / f_us / 1e3, 1),
                               "kernel_vs_ceiling": round(ms * 1e3 / f_us, 3),
                               "how": "kvq_stream_rw: %d B read + %d B written in order (no scatter), %d workgroups "
                                      "per CU" % (t_valid * 2048, t_valid * 1024, f_wg)},
            "x4_tokens": {"tokens": T4, "valid": t4_valid, "us": round(ms4 * 1e3, 2),
                          "GBps": round(alg4 / ms4 / 1e6, 1), "frac": round(alg4 / ms4 / 1e6 / PEAK_GBS, 4),
                          "ceiling_us": round(ms4_sc * 1e3, 2),
                          "ceiling_frac_of_peak": round(t4_valid * 3072 / ms4_sc / 1e6 / PEAK_GBS, 4),
                          "kernel_vs_ceiling": round(ms4 / ms4_sc, 3), "rotated_bytes": 2 * set4,
                          "how": "the same kernel and scatter floor at 4x c1's tokens, 16,384 x 16 slots, 2 rotated "
                                 "input / cache sets"}}


def bench_c3(reps=20, one_pass=True):
    """64 requests x 8 query tokens (causal), L log-uniform in [512, 8192], 28/4/128: two cache copies
    (~360 MB) rotated."""
    lens = synth.c3_lens()
    hq, hkv, d, bs = 28, 4, 128, 16
    pages = [-(-L // bs) for L in lens]
    nb = sum(pages) + 64
    params = synth.channel_params(hkv, d)
    st = {k: v.to(DEV) for k, v in synth.calibration_scales(hkv, d, params).items()}
    sets = []
    for s in range(2):
        kv, kc, vc = interleaved_cache(nb, hkv, bs, d)
        synth.fill_cache_gpu(kc, vc, st, params, seed=30 + s, write=ck.quant_reshape_and_cache)
        sets.append((kc, vc, synth.random_block_table(64, pages, nb, 40 + s, DEV)))
    g = torch.Generator(device=DEV).manual_seed(6)
    q = torch.randn(64 * 8, hq, d, generator=g, device=DEV).to(torch.bfloat16)
    cu = torch.arange(65, dtype=torch.int32, device=DEV) * 8
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    segm = ck.split_buffers(q.shape[0], hq, d, ck.SPLIT_PIECES, DEV)
    assert backend_passes_split_buffers([8] * 64, lens, hkv)   # the backend's call for this batch

    def fn(i, segm=segm):
        kc, vc, bt = sets[i]
        ck.decode_attention(q, kc, vc, out, cu, sl, bt, d ** -0.5, st, segm=segm, max_query_len=8)

    ms = _median_event_ms(fn, reps, len(sets))
    ms1 = _median_event_ms(lambda i: fn(i, None), reps, len(sets)) if one_pass else float("nan")
    kvb = sum(lens) * hkv * d * 2
    alg = kvb + 2 * q.numel() * 2 + sum(pages) * 4 + 129 * 4 + 2 * hkv * d * 4
    ops = sum(lens) * hkv * 28672
    return {"us": round(ms * 1e3, 2), "GBps": round(alg / ms / 1e6, 1), "frac": round(alg / ms / 1e6 / PEAK_GBS, 4),
            "alg_bytes": alg, "useful_int8_ops": ops, "mfma_util": round(ops / (ms * 1e-3) / PEAK_INT8_OPS, 5),
            "one_pass_us": round(ms1 * 1e3, 2)}


def bench_c4(reps=10, one_pass=True):
    """Llama-3 heads (32 / 8, d128): 96 decode rows (L log-uniform in [1, 32768]) through the INT8
    kernel, and the 4 x 16384-token prefill requests' pages dequantized to bf16 (dequant_pages)."""
    lens = synth.c4_lens()
    hq, hkv, d, bs = 32, 8, 128, 16
    pre = [16384] * 4
    dec_pages = [-(-L // bs) for L in lens]
    pre_pages = [L // bs for L in pre]
    nb = sum(dec_pages) + sum(pre_pages) + 64
    params = synth.channel_params(hkv, d)
    st = {k: v.to(DEV) for k, v in synth.calibration_scales(hkv, d, params).items()}
    kv, kc, vc = interleaved_cache(nb, hkv, bs, d)
    synth.fill_cache_gpu(kc, vc, st, params, seed=50, write=ck.quant_reshape_and_cache)
    bt = synth.random_block_table(100, dec_pages + pre_pages, nb, 51, DEV)
    g = torch.Generator(device=DEV).manual_seed(7)
    q = torch.randn(96, hq, d, generator=g, device=DEV).to(torch.bfloat16)
    cu = torch.arange(97, dtype=torch.int32, device=DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    segm = ck.split_buffers(96, hq, d, ck.SPLIT_PIECES, DEV)
    assert backend_passes_split_buffers([1] * 96, lens, hkv)   # the backend's call for this batch
    ms_dec = _median_event_ms(lambda i: ck.decode_attention(q, kc, vc, out, cu, sl, bt[:96], d ** -0.5, st, segm=segm),
                              reps, 1)
    ms_dec1 = _median_event_ms(lambda i: ck.decode_attention(q, kc, vc, out, cu, sl, bt[:96], d ** -0.5, st), reps,
                               1) if one_pass else float("nan")
    cu_all = torch.tensor([0] + [int(x) for x in torch.cumsum(torch.tensor([1] * 96 + pre), 0)], dtype=torch.int32)
    plan = ck.plan_long(cu_all, torch.tensor(lens + pre), bs)
    src_req, src_j, _ = plan.gpu(DEV)
    P = src_req.shape[0]
    ko = torch.empty(P, bs, hkv, d, dtype=torch.bfloat16, device=DEV)
    vo = torch.empty_like(ko)
    ms_dq = _median_event_ms(lambda i: ck.ext().dequant_pages(kc, vc, ko, vo, bt, src_req, src_j, st["k_scale"],
                                                              st["v_scale"]), reps, 1)
    # the prefill consumer over the temporary bf16 cache: 4 x 16384 query tokens, causal
    qp = torch.randn(sum(pre), hq, d, generator=g, device=DEV).to(torch.bfloat16)
    cu_p = torch.tensor([0] + [int(x) for x in torch.cumsum(torch.tensor(pre), 0)], dtype=torch.int32)
    plan_p = ck.plan_long(cu_p, torch.tensor(pre), bs)
    _, _, bt_p = plan_p.gpu(DEV)
    tr, tw = plan_p.tiles(hq // hkv, DEV)
    kt_p = torch.empty(plan_p.src_req.shape[0], bs, hkv, d, dtype=torch.bfloat16, device=DEV)
    vt_p = torch.empty_like(kt_p)
    ck.ext().dequant_pages(kc, vc, kt_p, vt_p, bt[96:], *plan_p.gpu(DEV)[:2], st["k_scale"], st["v_scale"])
    op = torch.empty_like(qp)
    cu_pd, sl_pd = cu_p.to(DEV), torch.tensor(pre, dtype=torch.int32, device=DEV)
    ms_pf = _median_event_ms(lambda i: ck.ext().paged_prefill_attention(qp, kt_p, vt_p, op, cu_pd, sl_pd, bt_p, tr, tw,
                                                                        d ** -0.5), max(3, reps // 2), 1, calls=3)
    pf_flop = sum(L * (L + 1) // 2 for L in pre) * hq * d * 4
    del kt_p, vt_p
    # the same attention reading the INT8 pages itself (KVQ_PREFILL_DIRECT=1, bit-identical; =fold, scales
    # folded into q and the output): one kernel in place of dequant_pages + the one above
    ms_pf8, ms_pf8f = (_median_event_ms(lambda i: ck.ext().int8_prefill_attention(
        qp, kc, vc, op, cu_pd, sl_pd, bt[96:], tr, tw, d ** -0.5, st["k_scale"], st["v_scale"], fold),
        max(3, reps // 2), 1, calls=3) for fold in (False, True))
    dq_read = P * bs * hkv * d * 2
    f_us, f_wg = rw_floor(dq_read, 2 * dq_read, reps=reps)
    dec_alg = sum(lens) * hkv * d * 2 + 2 * q.numel() * 2 + sum(dec_pages) * 4
    dq_alg = P * bs * hkv * d * 2 * (1 + 2) + P * 12
    mfma_tf, mfma_wg = mfma_ceiling(max(3, reps // 2))
    return {"decode_us": round(ms_dec * 1e3, 2), "decode_GBps": round(dec_alg / ms_dec / 1e6, 1),
            "decode_frac": round(dec_alg / ms_dec / 1e6 / PEAK_GBS, 4), "decode_one_pass_us": round(ms_dec1 * 1e3, 2),
            "dequant_us": round(ms_dq * 1e3, 2), "dequant_GBps": round(dq_alg / ms_dq / 1e6, 1),
            "dequant_frac": round(dq_alg / ms_dq / 1e6 / PEAK_GBS, 4), "dequant_pages": P,
            "dequant_ceiling": {"us": round(f_us, 2), "GBps": round(3 * dq_read / f_us / 1e3, 1),
                                "frac_of_peak": round(3 * dq_read / f_us / 1e3 / PEAK_GBS, 4),
                                "kernel_vs_ceiling": round(ms_dq * 1e3 / f_us, 3),
                                "how": "kvq_stream_rw: %d B read + %d B written in order (the pages' codes and their "
                                       "bf16 values, no page gather, no arithmetic), %d workgroups per CU"
                                       % (dq_read, 2 * dq_read, f_wg)},
            "prefill_ms": round(ms_pf, 3), "prefill_TFLOPs": round(pf_flop / ms_pf / 1e9, 1),
            "prefill_frac_bf16": round(pf_flop / ms_pf / 1e9 / PEAK_BF16_TFLOPS, 4), "prefill_flop": pf_flop,
            "prefill_direct_ms": round(ms_pf8, 3), "prefill_fold_ms": round(ms_pf8f, 3),
            "prefill_two_kernel_ms": round(ms_dq + ms_pf, 3),
            "mfma_ceiling": {"TFLOPs": round(mfma_tf, 1), "frac_of_peak": round(mfma_tf / PEAK_BF16_TFLOPS, 4),
                             "prefill_vs_ceiling": round(pf_flop / ms_pf / 1e9 / mfma_tf, 4),
                             "how": "kvq_mfma_probe: back-to-back 16x16x32 bf16 MFMAs on random bf16 operands, "
                                    "8 chains per wavefront, %d workgroups of 4 wavefronts" % mfma_wg}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy 5 times (HBM counter calibration)")
    ap.add_argument("--extras", default="",
                    help="only run these extra workloads (comma list of c1, c3, c4) and print their JSON; for "
                         "profiling one kernel's workload")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path has no multi-GPU mode (every kernel shards per request / "
              "kv head with no exchange, so each GPU would run this same workload on its share). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=DEV)
        src.fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": 1 << 30, "copies": 5}))
        return
    ck.ext()
    if args.extras:
        runs = {"c1": ("c1_quant_cache", bench_c1), "c3": ("c3_verify_8tok", bench_c3), "c4": ("c4_llama3_mixed", bench_c4)}
        names = [x.strip() for x in args.extras.split(",") if x.strip()]
        bad = [x for x in names if x not in runs]
        if bad:
            ap.error("unknown extras %s (choose from c1, c3, c4)" % bad)
        # profiling runs: only the calls with split buffers (the one-pass variants launch the same kernel)
        kw = lambda x: {} if x == "c1" else {"one_pass": False}
        print(json.dumps({"extra": {runs[x][0]: runs[x][1](**kw(x)) for x in names}}), flush=True)
        return
    print("# building c2 workload", file=sys.stderr, flush=True)
    w = build_c2()
    torch.cuda.synchronize()
    print("# timing c2", file=sys.stderr, flush=True)
    # the call as the vLLM backend makes it for this batch outside graph capture: 128 requests x 4 kv heads
    # of even length give every CU two pairs, so no split buffers (one pass); the call with split buffers (what a
    # captured graph replays) is reported beside it
    split = backend_passes_split_buffers([1] * w["B"], [w["L"]] * w["B"], w["hkv"])
    # the other call is timed first, after 30 untimed calls (~20 ms): a GPU that has idled while the host
    # built the workload runs the first ~20 ms of calls ~3% slower (measured: 668 vs 645 us per kernel,
    # both variants, whichever runs first), so both timings start from a busy GPU
    _, ms1, _, k1_mean, _, s1 = time_c2(w, max(5, args.steps // 2), 30, split=not split)
    out, ms_step, launch_ms, kern_ms_mean, kern_ms_med, splits = time_c2(w, args.steps, args.warmup, split=split)
    alg = w["alg_bytes"]
    res = {
        "metric": METRIC,
        "value": round(alg / (ms_step * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "us_per_call": round(ms_step * 1e3, 1),
        "kv_GBps": round(w["kv_bytes"] / (ms_step * 1e-3) / 1e9, 1),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 (int32 MFMA accumulate, fp32 softmax, bf16 out)",
        "data": "synthetic (c0 distribution, seeded)",
        "config": {"workload": "c2: INT8 paged decode attention, 128 requests x 32768 keys, 28 q / 4 kv heads, "
                               "d128, block 16, vLLM interleaved int8 cache, shuffled block tables",
                   "split_buffers": split, "max_splits": splits,
                   "call": "kvq.cuda_kernels.decode_attention as the vLLM backend calls it for this batch eagerly "
                           "or under piecewise graphs (requests of even length, two (request, kv head) pairs per CU: "
                           "no split buffers, one pass, nothing allocated); a full-graph replay carries the split "
                           "buffers: c2_other_call" if not split else
                           "kvq.cuda_kernels.decode_attention with split buffers, as the vLLM backend calls it",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(alg / (launch_ms * 1e-3) / 1e9, 1), "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(alg / (launch_ms * 1e-3) / 1e9 / PEAK_GBS, 4), "traffic": None,
                     "kernel": "attn_kernel<128, 2, false> (one pass)",
                     "launch_us_timed_region": round(launch_ms * 1e3, 1),
                     "how": "algorithmic bytes / (HIP event interval around the timed region's launches / steps)",
                     "kernel_us_mean": round(kern_ms_mean * 1e3, 1), "kernel_us_median": round(kern_ms_med * 1e3, 1),
                     "kernel_events": "the library's event pair around each attention kernel, as many calls again "
                                      "right after the timed region",
                     "alg_bytes_per_launch": alg},
    }
    res["c2_other_call"] = {
        "what": ("with split buffers allocated once beforehand (%d pieces per row at most, the vLLM backend's "
                 "buffers, which a captured graph always gets): segments cut across workgroups where the plan "
                 "calls for it, fp32 partials merged by split_reduce_kernel" % s1) if not split else
                "without split buffers: one pass, each (request, kv head) whole in one workgroup",
        "us_per_call": round(ms1 * 1e3, 1), "kernel_us_mean": round(k1_mean * 1e3, 1),
        "GBps": round(alg / (ms1 * 1e-3) / 1e9, 1), "frac": round(alg / (ms1 * 1e-3) / 1e9 / PEAK_GBS, 4)}
    ceil_gbs, ceil_wg = read_ceiling(w["kv"])
    res["roofline"]["read_ceiling"] = {
        "GBps": round(ceil_gbs, 1), "frac_of_peak": round(ceil_gbs / PEAK_GBS, 4),
        "kernel_frac_of_ceiling": round(res["roofline"]["achieved"] / ceil_gbs, 4),
        "how": "kvq_stream_read over the c2 cache's %d bytes (contiguous share per workgroup, 8 loads in flight per lane, "
               "%d workgroups of 256 lanes per CU, the better of 4 and 8), HIP events, median of 10" % (w["kv"].numel(), ceil_wg)}
    prof = os.path.join(REPO, "profiles", "attn_kernel_c2_traffic.json")
    if os.path.exists(prof):   # HBM bytes per launch from the committed rocprofv3 --pmc runs of this workload
        with open(prof) as f:
            t = json.load(f)
        res["roofline"]["traffic"] = t["traffic_bytes"]
        res["roofline"]["traffic_source"] = "profiles/attn_kernel_c2_decode_128x32k.md (FETCH_SIZE x %.3f + WRITE_SIZE x %.3f)" % (
            t["fetch_factor"], t["write_factor"])
    if not args.no_cpu:
        print("# cpu baseline", file=sys.stderr, flush=True)
        res["cpu_baseline"], res["parity"] = cpu_baseline(w, out)
    del w
    torch.cuda.empty_cache()
    if not args.no_extra:
        print("# extras", file=sys.stderr, flush=True)
        res["extra"] = {"c1_quant_cache": bench_c1(), "c3_verify_8tok": bench_c3(), "c4_llama3_mixed": bench_c4()}
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
