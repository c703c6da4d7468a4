"""The C-ABI boundary and the host-side logic of kvq.cuda_kernels, without a GPU: the library loads and
exports what include/kvq_int8.h declares, arguments the reference rejects are rejected before any
launch, the KVQ_DEBUG input check, the split heuristic, and the scale file format."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from kvq import _native, scales
from kvq import cuda_kernels as ck

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    with open(os.path.join(REPO, "include", "kvq_int8.h")) as f:
        return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(kvq_\w+)\s*\(", f.read(), re.M)))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    names = _declared()
    assert set(names) == set(_native.SIGNATURES), "ctypes signatures out of sync with the header"
    for n in names:
        assert hasattr(lib, n), n
    assert lib.kvq_abi_version() == _native.ABI_VERSION


def _raw(name):
    return getattr(_native.load(), name)


def test_abi_rejects_bad_arguments_before_launch():
    lib = _native.load()
    nul = None
    # head_dim 96
    rc = lib.kvq_quant_cache(nul, 0, 0, nul, 0, 0, nul, 0, 0, 0, nul, 0, 0, 0, nul, 4, 4, 96, 16, 16, nul, 96, nul, 96,
                             nul, nul)
    assert rc == 1 and b"head_dim must be 64 or 128" in lib.kvq_last_error()
    # zero tokens: nothing to do, success without touching the GPU
    rc = lib.kvq_quant_cache(nul, 0, 0, nul, 0, 0, nul, 0, 0, 0, nul, 0, 0, 0, nul, 0, 4, 128, 16, 16, nul, 128, nul,
                             128, nul, nul)
    assert rc == 0 and lib.kvq_last_error() == b""
    # block size 24
    args = [nul, 0, 0, nul, 0, 0, 0, nul, 0, 0, 0, 64, 24, 4, 128, nul, 0, 0, nul, nul, nul, 0, 1, 28, nul, 128, nul,
            128, 0.1, nul, nul, nul, 0, 0, 1, 0, 1, 8, nul]
    assert lib.kvq_int8_decode_attention(*args) == 1 and b"power of two" in lib.kvq_last_error()
    args[12] = 16
    args[34] = 65                      # num_splits
    assert lib.kvq_int8_decode_attention(*args) == 1 and b"at most 64" in lib.kvq_last_error()
    args[34] = 1
    args[23] = 30                      # 30 q heads over 4 kv heads
    assert lib.kvq_int8_decode_attention(*args) == 1 and b"head counts" in lib.kvq_last_error()
    rc = lib.kvq_quant_q(nul, 0, 0, 5, 28, 64, nul, 4, 64, 64, nul, nul, nul)
    assert rc == 1 and b"head_dim 128" in lib.kvq_last_error()
    rc = lib.kvq_dequant_pages(nul, 0, 0, 0, nul, 0, 0, 0, 10, 16, 4, 128, nul, nul, nul, 0, nul, nul, 3, nul, 7,
                               nul, 128, nul)
    assert rc == 1 and b"scale columns" in lib.kvq_last_error()
    # INT8 prefill: scale columns 7; then an int8 slot stride of 8 bytes (the DMA moves 16-byte chunks)
    p8 = [nul, 0, 0, nul, 0, 128, 0, nul, 0, 128, 0, 64, 16, 4, 128, nul, 0, 0, nul, nul, nul, 0, 28, nul, nul, 1,
          128, 0.1, nul, 7, nul, 128, 0, nul]
    assert lib.kvq_int8_prefill_attention(*p8) == 1 and b"scale columns" in lib.kvq_last_error()
    p8[29], p8[5] = 1, 8
    assert lib.kvq_int8_prefill_attention(*p8) == 1 and b"16-byte aligned" in lib.kvq_last_error()
    p8[5] = 128
    p8[14] = 96
    assert lib.kvq_int8_prefill_attention(*p8) == 1 and b"head_dim must be 64 or 128" in lib.kvq_last_error()
    p8[14], p8[32] = 128, 2
    assert lib.kvq_int8_prefill_attention(*p8) == 1 and b"fold_scales must be 0 or 1" in lib.kvq_last_error()


def test_noalloc_rejects_oversized_calls_before_any_device_call():
    """kvq_int8_decode_attention_noalloc checks its sizes before it looks up its device array: head counts
    beyond the merge grid's, and partials beyond the array, compared by division -- sizes whose product
    would overflow 64 bits (2^31 - 1 tokens x 262,140 q heads x 64 splits x 130 floats) are rejected, not
    wrapped into a small number."""
    lib = _native.load()
    nul = None

    def call(T, hq, S, d=128):
        return lib.kvq_int8_decode_attention_noalloc(nul, 0, 0, T, nul, 0, 0, 0, nul, 0, 0, 0, 64, 16, 4, d, nul, 0, 0,
                                                     nul, nul, nul, 0, 1, hq, nul, d, nul, d, 0.1, S, 0, 1, 8, nul)
    assert call(8, 65535 * 4 + 1, 1) == 1 and b"bad sizes" in lib.kvq_last_error()
    assert call(2 ** 31 - 1, 65535 * 4, 64) == 1 and b"scratch holds" in lib.kvq_last_error()
    assert call(2 ** 31 - 1, 28, 2) == 1 and b"scratch holds" in lib.kvq_last_error()
    per_token = 28 * 16 * 130 * 4
    assert call(lib.kvq_noalloc_scratch_bytes() // per_token + 1, 28, 16) == 1
    assert b"scratch holds" in lib.kvq_last_error()


def test_native_call_raises_with_message():
    with pytest.raises(_native.NativeError, match="head_dim must be 64 or 128"):
        _native.call("kvq_dequant_pages", None, 0, 0, 0, None, 0, 0, 0, 10, 16, 4, 96, None, None, None, 0, None,
                     None, 3, None, 96, None, 96, None)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    # no fallback: without the built library, the ops API raises instead of computing anything
    monkeypatch.setattr(_native, "_LIB", None)
    monkeypatch.setattr(_native, "LIB_PATH", str(tmp_path / "libkvq_int8.so"))
    monkeypatch.setattr(ck, "_EXT", None)
    with pytest.raises(_native.NativeError, match="is not built"):
        ck.ext()
    with pytest.raises(_native.NativeError, match="is not built"):
        _native.call("kvq_abi_version")


def test_wrong_abi_version_fails_loudly(monkeypatch):
    monkeypatch.setattr(_native, "_LIB", None)
    monkeypatch.setattr(_native, "ABI_VERSION", _native.ABI_VERSION + 1000)
    with pytest.raises(_native.NativeError, match="rebuild it"):
        _native.load()


# ------------------------------------------------------------ Python API: the reference's TORCH_CHECKs
def test_python_api_shape_checks():
    q = torch.zeros(3, 28, 64, dtype=torch.bfloat16)
    kc = torch.zeros(8, 24, 4, 64, dtype=torch.int8)
    st = {"k_scale": torch.ones(4, 64), "v_scale": torch.ones(4, 64), "k_mu": torch.zeros(4, 64)}
    cu = torch.tensor([0, 1, 2, 3], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="block_size must be a power of two >= 16"):
        ck.decode_attention(q, kc, kc, q.clone(), cu, cu[1:], cu[None], 0.1, st, segm=(None, None, None))
    with pytest.raises(RuntimeError, match="standalone q quantization: head_dim 128"):
        ck.quant_q(q, st["k_scale"])
    key = torch.zeros(5, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="contiguous last dim"):
        ck.quant_reshape_and_cache(key, key, kc, kc, torch.zeros(5, dtype=torch.long), st)
    kc16 = torch.zeros(8, 16, 4, 64, dtype=torch.int8)
    sm = torch.zeros(3, 28, 65)
    with pytest.raises(RuntimeError, match="at most 64 split-KV segments"):
        ck.decode_attention(q, kc16, kc16, q.clone(), cu, cu[1:], cu[None], 0.1, st,
                            segm=(torch.zeros(3, 28, 65, 64), sm, sm))
    with pytest.raises(RuntimeError, match="on the GPU"):   # CPU tensors never reach the library
        ck.decode_attention(q, kc16, kc16, q.clone(), cu, cu[1:], torch.zeros(3, 4, dtype=torch.int32), 0.1, st,
                            segm=(torch.zeros(3, 28, 2, 64), torch.zeros(3, 28, 2), torch.zeros(3, 28, 2)))


def test_prefill_direct_switch_is_checked(monkeypatch):
    """KVQ_PREFILL_DIRECT takes 0, 1 or fold; anything else is an error before any launch."""
    monkeypatch.setenv("KVQ_PREFILL_DIRECT", "yes")
    q = torch.zeros(40, 28, 128, dtype=torch.bfloat16)
    kc = torch.zeros(8, 16, 4, 128, dtype=torch.int8)
    st = {"k_scale": torch.ones(4, 128), "v_scale": torch.ones(4, 128), "k_mu": torch.zeros(4, 128)}
    cu, sl = torch.tensor([0, 40], dtype=torch.int32), torch.tensor([40], dtype=torch.int32)
    plan = ck.plan_long(cu, sl, 16)
    with pytest.raises(RuntimeError, match="KVQ_PREFILL_DIRECT must be 0, 1 or fold"):
        ck.long_attention(q, kc, kc, q.clone(), cu, sl, torch.arange(3, dtype=torch.int32)[None], 40, plan, 0.1, st)


def test_empty_batches_return_early():
    q = torch.zeros(0, 28, 128, dtype=torch.bfloat16)
    kc = torch.zeros(8, 16, 4, 128, dtype=torch.int8)
    st = {"k_scale": torch.ones(4, 128), "v_scale": torch.ones(4, 128), "k_mu": torch.zeros(4, 128)}
    ck.decode_attention(q, kc, kc, q, torch.zeros(1, dtype=torch.int32), torch.zeros(0, dtype=torch.int32),
                        torch.zeros(0, 1, dtype=torch.int32), 0.1, st, segm=(None, None, None))
    ck.quant_reshape_and_cache(q[:, :4], q[:, :4], kc, kc, torch.zeros(0, dtype=torch.long), st)
    qi, qs = ck.quant_q(q, st["k_scale"])
    assert qi.shape == (0, 28, 128) and qs.shape == (0, 28, 1)


# ------------------------------------------------------------ KVQ_DEBUG host check (cuda_kernels.py:134-169)
def _batch():
    q = torch.zeros(6, 28, 128, dtype=torch.bfloat16)
    kc = torch.zeros(10, 16, 4, 128, dtype=torch.int8)
    cu = torch.tensor([0, 1, 3, 6], dtype=torch.int32)
    sl = torch.tensor([20, 2, 40], dtype=torch.int32)
    bt = torch.tensor([[1, 2, 0], [3, 0, 0], [4, 5, 6]], dtype=torch.int32)
    return q, kc, cu, sl, bt


def test_check_inputs_accepts_a_valid_batch():
    ck.check_inputs(*_batch(), None)


@pytest.mark.parametrize("mutate,msg", [
    (lambda b: b[4].__setitem__((2, 1), 10), "outside \\[0, 10\\)"),
    (lambda b: b[3].__setitem__(1, 1), "seq_len 1 < q_len 2"),
    (lambda b: b[3].__setitem__(2, 49), "4 pages > block_table width 3"),
    (lambda b: b[2].__setitem__(3, 7), "cu_seqlens_q\\[-1\\] 7 > 6 query rows"),
])
def test_check_inputs_reports(mutate, msg):
    b = list(_batch())
    mutate(b)
    with pytest.raises(RuntimeError, match=msg):
        ck.check_inputs(*b, None)


def test_check_inputs_plan_coverage():
    q = torch.zeros(30, 28, 128, dtype=torch.bfloat16)
    kc = torch.zeros(40, 16, 4, 128, dtype=torch.int8)
    cu = torch.tensor([0, 1, 30], dtype=torch.int32)
    sl = torch.tensor([5, 60], dtype=torch.int32)
    bt = torch.tensor([[1, 0, 0, 0], [2, 3, 4, 5]], dtype=torch.int32)
    plan = ck.plan_long(cu, sl - 20, 16)          # too few pages copied for 60 keys
    with pytest.raises(RuntimeError, match="fewer copied pages than keys"):
        ck.check_inputs(q, kc, cu, sl, bt, plan)
    ck.check_inputs(q, kc, cu, sl, bt, ck.plan_long(cu, sl, 16))


# ------------------------------------------------------------ split heuristic
def test_choose_splits():
    """Cap on splits per request: contexts cut into >= 128-key ranges, at most 64."""
    assert ck.choose_splits(32768) == 64
    assert ck.choose_splits(512) == 4
    assert ck.choose_splits(100) == 1 and ck.choose_splits(0) == 1
    os.environ["KVQ_SPLITS"] = "3"
    try:
        assert ck.choose_splits(32768) == 3
    finally:
        del os.environ["KVQ_SPLITS"]


# ------------------------------------------------------------ scale format (kvq/scales.py)
def test_scales_roundtrip_and_format(tmp_path):
    r = np.random.Generator(np.random.PCG64(0))
    d = {f"model.layers.{i}.self_attn.attn": {"k_scale": torch.from_numpy(r.random((4, 128), dtype=np.float32)),
                                               "v_scale": torch.from_numpy(r.random((4, 1), dtype=np.float32)),
                                               "k_mu": torch.zeros(4, 128)} for i in range(2)}
    p = str(tmp_path / "s.safetensors")
    scales.save(p, d)
    from safetensors.torch import load_file
    raw = load_file(p)
    assert "model.layers.1.self_attn.attn|k_scale" in raw and raw["model.layers.0.self_attn.attn|v_scale"].shape == (4, 1)
    back = scales.load(p)
    for n in d:
        for k in d[n]:
            assert torch.equal(back[n][k], d[n][k])
    sl = scales.for_layer(back, "model.layers.0.self_attn.attn", 1, 2, "cpu")
    assert torch.equal(sl["k_scale"], d["model.layers.0.self_attn.attn"]["k_scale"][2:4])


def test_scales_shard_replicates_when_fewer_heads_than_ranks():
    t = torch.arange(2)[:, None].float()
    assert [scales.shard(t, r, 4).item() for r in range(4)] == [0, 0, 1, 1]
    assert scales.shard(torch.arange(8)[:, None], 3, 4).flatten().tolist() == [6, 7]


def test_from_stats_max_and_smooth():
    st = {"tokens": torch.tensor(4.0), "k_sum": torch.full((2, 3), 4.0), "k_max": torch.full((2, 3), 3.0),
          "k_min": torch.full((2, 3), -1.0), "k_absmax": torch.full((2, 3), 3.0), "v_absmax": torch.full((2, 3), 2.54)}
    out = scales.from_stats(st, smooth_k=True)
    assert torch.allclose(out["k_mu"], torch.ones(2, 3))
    assert torch.allclose(out["k_scale"], torch.full((2, 3), 2.0 / 127))   # max(3 - 1, 1 - (-1)) / 127
    assert torch.allclose(out["v_scale"], torch.full((2, 3), 0.02))
    assert scales.from_stats(st, granularity="per_head")["k_scale"].shape == (2, 1)
