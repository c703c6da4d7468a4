"""kvq_int8_decode_attention_noalloc (split partials in the library's own device array, no allocation)
against kvq_int8_decode_attention with caller-owned split buffers, both called through the C ABI: two
calls in a row on the same array, the second with a smaller batch, each bit-identical to the existing
entry point's output and within the attention bar of the oracle; sizes beyond the array are rejected
before anything is launched."""
import ctypes

import pytest
import torch
from conftest import nan_like, nan_segm, record

from oracle import kvq_oracle as O
from kvq import _native, synth

pytestmark = pytest.mark.gpu
DEV = "cuda"
HQ, HKV, D, S = 28, 4, 128, 16


def _case(q_lens, seq_lens, seed):
    c = synth.paged_case(HQ, HKV, q_lens, seq_lens, seed=seed, params=synth.channel_params(HKV, D))
    c["static"] = synth.calibration_scales(HKV, D, synth.channel_params(HKV, D))
    st = c["static"]
    kq = O.quantize(c["k"].float() - st["k_mu"], st["k_scale"])
    vq = O.quantize(c["v"], st["v_scale"])
    ref = O.paged_static_attention(O.CFG32_Q32, st, True, 8)(c["q"].float(), kq, vq, c["cu"], c["seq_lens"],
                                                               c["block_table"], D ** -0.5)
    d = {k: v.to(DEV) for k, v in c.items() if isinstance(v, torch.Tensor)}
    d["static"] = {k: v.to(DEV) for k, v in st.items()}
    d["kc"], d["vc"] = kq.to(DEV), vq.to(DEV)
    return d, ref


def _common(d, out):
    """Arguments shared by both entry points, in header order, up to the head counts / scales."""
    q, kc, vc, st = d["q"], d["kc"], d["vc"], d["static"]
    return dict(
        q=(q.data_ptr(), q.stride(0), q.stride(1)),
        cache=(kc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), vc.data_ptr(), vc.stride(0), vc.stride(1),
               vc.stride(2), kc.shape[0], kc.shape[1], HKV, D),
        rest=(out.data_ptr(), out.stride(0), out.stride(1), d["cu"].data_ptr(), d["seq_lens"].data_ptr(),
              d["block_table"].data_ptr(), d["block_table"].stride(0), d["cu"].shape[0] - 1, HQ,
              st["k_scale"].data_ptr(), st["k_scale"].shape[1], st["v_scale"].data_ptr(), st["v_scale"].shape[1],
              D ** -0.5))


def _with_buffers(d, splits):
    out = nan_like(d["q"])
    so, sm, ss = nan_segm(d["q"].shape[0], HQ, splits, D)
    a = _common(d, out)
    _native.call("kvq_int8_decode_attention", *a["q"], *a["cache"], *a["rest"], so.data_ptr(), sm.data_ptr(),
                 ss.data_ptr(), sm.stride(0), sm.stride(1), splits, 0, 8, 8, torch.cuda.current_stream().cuda_stream)
    return out


def _noalloc(d, splits, out=None):
    out = nan_like(d["q"]) if out is None else out
    a = _common(d, out)
    _native.call("kvq_int8_decode_attention_noalloc", *a["q"], d["q"].shape[0], *a["cache"], *a["rest"], splits, 0,
                 8, 8, torch.cuda.current_stream().cuda_stream)
    return out


def test_noalloc_matches_the_buffered_entry_point_twice_in_a_row():
    big = _case([1, 8, 4, 1, 8, 2], [9000, 3000, 700, 16, 5200, 33], seed=61)
    small = _case([8, 1, 3], [2100, 600, 97], seed=62)
    for name, (d, ref) in (("big", big), ("small", small)):
        want = _with_buffers(d, S)
        got = nan_like(d["q"])
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        _noalloc(d, S, got)
        torch.cuda.synchronize()
        assert torch.cuda.max_memory_allocated() == before == torch.cuda.memory_allocated()
        assert torch.isfinite(got.float()).all(), name
        assert torch.equal(got, want), name
        err = O.compare(ref, got.cpu())
        record("noalloc_vs_oracle", case=name, **err)
        assert err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3 and err["rel_l2"] < 5e-3, (name, err)


def test_noalloc_single_pass_needs_no_scratch():
    d, ref = _case([1, 1, 6], [4000, 10, 900], seed=63)
    got = _noalloc(d, 1)
    assert torch.equal(got, _with_buffers(d, 1))
    err = O.compare(ref, got.cpu())
    assert err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3, err


def test_noalloc_rejects_partials_beyond_the_scratch():
    lib = _native.load()
    cap = lib.kvq_noalloc_scratch_bytes()
    assert cap == 64 << 20
    d, _ = _case([1, 1], [100, 200], seed=64)
    out = nan_like(d["q"])
    a = _common(d, out)
    tokens = cap // (HQ * 64 * (D + 2) * 4) + 1   # 64 splits of this many rows overflow the array
    rc = lib.kvq_int8_decode_attention_noalloc(*a["q"], tokens, *a["cache"], *a["rest"], 64, 0, 8, 8,
                                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 1 and b"scratch" in lib.kvq_last_error()
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()   # nothing was launched
