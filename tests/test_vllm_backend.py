"""The vLLM drop-in (kvq.vllm_int8.backend, kvq.vllm_plugin, kvq.capture) against the reference's
behaviour (kvq/vllm_int8/backend.py:48-184, kvq/vllm_plugin.py:9-25, kvq/capture.py:25-118), on the
CPU with the vLLM interface stand-in of tests/vllm_stub: registration, configuration checks, scale
hand-out per layer and TP rank, the long-query plan in the metadata builder, graph-support levels,
cache views, and the calibration statistics feeding kvq.scales."""
import os
import sys
from types import SimpleNamespace

import numpy as np
import pytest
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "vllm_stub"))

import vllm.distributed as vdist  # noqa: E402  (the stand-in)
from vllm.v1.attention.backend import AttentionCGSupport  # noqa: E402
from vllm.v1.attention.backends import registry  # noqa: E402
from vllm.v1.attention.backends.triton_attn import CommonAttentionMetadata, TritonAttentionImpl  # noqa: E402

from kvq import capture, cuda_kernels as ck, scales, vllm_plugin  # noqa: E402
from kvq.vllm_int8 import backend  # noqa: E402

HQ, HKV, D, BS = 28, 4, 128, 16


@pytest.fixture(autouse=True)
def _env(monkeypatch):
    for v in ("KVQ_CFG", "KVQ_KERNEL", "KVQ_SCALES", "KVQ_DRAFT_SCALES", "KVQ_CAPTURE", "KVQ_ATTN", "KVQ_MLA"):
        monkeypatch.delenv(v, raising=False)
    vdist.TP_RANK, vdist.TP_SIZE = 0, 1
    backend.SCALE_FILES.clear()
    yield
    vdist.TP_RANK, vdist.TP_SIZE = 0, 1


def _impl(num_kv_heads=HKV, cfg=None, monkeypatch=None):
    if cfg:
        monkeypatch.setenv("KVQ_CFG", cfg)
    return backend.Int8StaticImpl(HQ, D, D ** -0.5, num_kv_heads, kv_cache_dtype="int8_static")


def _layer_scales(hkv=HKV, smooth=True, per_head=False, seed=0):
    g = torch.Generator().manual_seed(seed)
    cols = 1 if per_head else D
    d = {"k_scale": torch.rand(hkv, cols, generator=g) + 0.01, "v_scale": torch.rand(hkv, cols, generator=g) + 0.01}
    if smooth:
        d["k_mu"] = torch.randn(hkv, D, generator=g)
    return d


# ------------------------------------------------------------------ plugin
def test_plugin_registers_custom_backend_by_class_path():
    registry.REGISTRY.clear()
    vllm_plugin.register()
    path = registry.REGISTRY[registry.AttentionBackendEnum.CUSTOM]
    assert path == "kvq.vllm_int8.backend.Int8StaticBackend"
    mod, cls = path.rsplit(".", 1)
    backend_cls = getattr(__import__(mod, fromlist=[cls]), cls)
    assert backend_cls.get_name() == "CUSTOM" and backend_cls.supported_kv_cache_dtypes == ["int8_static"]
    assert backend_cls.get_impl_cls() is backend.Int8StaticImpl
    assert backend_cls.get_builder_cls() is backend.Int8StaticBuilder
    spec = object()
    assert backend_cls.customize_spec(spec) is spec


def test_plugin_warns_while_int8_static_is_unregistered(tmp_path, monkeypatch, caplog):
    """register() names the fix when the installed vLLM would reject kv_cache_dtype="int8_static", and is
    quiet once kvq.vllm_dtype has registered it (a vLLM-shaped tree stands in for the installed vLLM)."""
    import logging

    from kvq import vllm_dtype
    from test_vllm_dtype import make_tree

    pkg = make_tree(tmp_path)
    monkeypatch.setattr(vllm_dtype, "find_vllm", lambda: pkg)
    with caplog.at_level(logging.WARNING):
        vllm_plugin.register()
    assert "python -m kvq.vllm_dtype" in caplog.text and "config/cache.py" in caplog.text
    caplog.clear()
    vllm_dtype.install(pkg)
    with caplog.at_level(logging.WARNING):
        vllm_plugin.register()
    assert "int8_static" not in caplog.text


def test_plugin_refuses_study_paths_it_does_not_ship(monkeypatch):
    monkeypatch.setenv("KVQ_ATTN", "B_channel")
    with pytest.raises(RuntimeError, match="KVQ_ATTN"):
        vllm_plugin.register()


def test_plugin_installs_capture(monkeypatch):
    calls = []
    monkeypatch.setenv("KVQ_CAPTURE", "1")
    monkeypatch.setattr(capture, "install", lambda: calls.append(1))
    vllm_plugin.register()
    assert calls == [1]


# ------------------------------------------------------------------ impl
@pytest.mark.parametrize("cfg", ["B_channel_smooth", "B_channel", "B_head_smooth", "B_head", "B_channel_qgroup32",
                                 "B_channel_smooth_qgroup32"])
def test_impl_accepts_the_kernel_configs(cfg, monkeypatch):
    impl = _impl(cfg=cfg, monkeypatch=monkeypatch)
    assert impl.cfg_name == cfg and impl.kv_cache_dtype == "int8_static"
    assert impl.fused_output_quant_supported(None) is False
    assert impl.q_group == (32 if cfg.endswith("qgroup32") else None)


@pytest.mark.parametrize("cfg", ["A_channel", "B_channel_pnone", "B_channel_qtensor", "B_channel_smooth_qnone"])
def test_impl_rejects_configs_the_kernels_do_not_compute(cfg, monkeypatch):
    with pytest.raises(AssertionError, match="implement B"):
        _impl(cfg=cfg, monkeypatch=monkeypatch)


def test_impl_rejects_other_cache_dtypes_and_the_torch_path(monkeypatch):
    with pytest.raises(AssertionError):
        backend.Int8StaticImpl(HQ, D, 0.1, HKV, kv_cache_dtype="auto")
    monkeypatch.setenv("KVQ_KERNEL", "torch")
    with pytest.raises(NotImplementedError, match="KVQ_KERNEL=torch"):
        _impl()


def test_set_static_checks_and_fills_zero_mean(monkeypatch):
    impl = _impl(cfg="B_channel", monkeypatch=monkeypatch)
    st = _layer_scales(smooth=False)
    impl.set_static({k: v.double() for k, v in st.items()})
    assert impl.static["k_scale"].dtype == torch.float32 and impl.static["k_scale"].is_contiguous()
    assert torch.equal(impl.static["k_mu"], torch.zeros(HKV, D))
    with pytest.raises(AssertionError, match="smooth-K"):
        impl.set_static(_layer_scales(smooth=True))
    with pytest.raises(AssertionError):
        impl.set_static(_layer_scales(hkv=2, smooth=False))
    with pytest.raises(AssertionError, match="per_channel"):
        impl.set_static(_layer_scales(smooth=False, per_head=True))
    head = _impl(cfg="B_head_smooth", monkeypatch=monkeypatch)
    head.set_static(_layer_scales(smooth=True, per_head=True))
    assert head.static["k_scale"].shape == (HKV, 1)


def test_cache_views_split_the_interleaved_layout(monkeypatch):
    impl = _impl(monkeypatch=monkeypatch)
    kv = torch.arange(3 * HKV * BS * 2 * D, dtype=torch.int32).reshape(3, HKV, BS, 2 * D)
    kc, vc = impl._caches(kv)
    assert kc.shape == vc.shape == (3, BS, HKV, D) and kc.stride(3) == 1
    assert kc[2, 5, 1, 7] == kv[2, 1, 5, 7] and vc[2, 5, 1, 7] == kv[2, 1, 5, D + 7]


def test_forward_profiling_run_zeroes_output(monkeypatch):
    impl = _impl(monkeypatch=monkeypatch)
    out = torch.ones(4, HQ, D)
    assert impl.forward(None, None, None, None, None, None, out) is out and not out.any()


# ------------------------------------------------------------------ builder
def _vllm_config(layers, spec_tokens=None, max_num_seqs=32):
    ctx = {name: SimpleNamespace(impl=impl) for name, impl in layers.items()}
    spec = None if spec_tokens is None else SimpleNamespace(num_speculative_tokens=spec_tokens)
    return SimpleNamespace(compilation_config=SimpleNamespace(static_forward_context=ctx), speculative_config=spec,
                           model_config=SimpleNamespace(num_heads=HQ, num_kv_heads=HKV, head_size=D),
                           scheduler_config=SimpleNamespace(max_num_seqs=max_num_seqs))


def _write_scales(path, names, hkv=HKV, smooth=True):
    scales.save(str(path), {n: _layer_scales(hkv=hkv, smooth=smooth, seed=i) for i, n in enumerate(names)})


@pytest.mark.parametrize("tp", [(0, 1), (1, 2), (3, 8)])
def test_builder_hands_each_layer_its_tp_slice(tmp_path, monkeypatch, tp):
    names = [f"model.layers.{i}.self_attn.attn" for i in range(3)]
    _write_scales(tmp_path / "s.safetensors", names)
    monkeypatch.setenv("KVQ_SCALES", str(tmp_path / "s.safetensors"))
    vdist.TP_RANK, vdist.TP_SIZE = tp
    heads = max(1, HKV // tp[1])
    layers = {n: _impl(num_kv_heads=heads, monkeypatch=monkeypatch) for n in names}
    backend.Int8StaticBuilder(SimpleNamespace(block_size=BS), names, _vllm_config(layers), "cpu")
    full = scales.load(str(tmp_path / "s.safetensors"))
    for n in names:
        for k in ("k_scale", "v_scale", "k_mu"):
            assert torch.equal(layers[n].static[k], scales.shard(full[n][k], *tp))


def test_builder_reads_draft_model_scales(tmp_path, monkeypatch):
    _write_scales(tmp_path / "main.safetensors", ["model.layers.0.self_attn.attn"])
    _write_scales(tmp_path / "draft.safetensors", ["model.layers.0.self_attn.attn"], hkv=HKV)
    monkeypatch.setenv("KVQ_SCALES", str(tmp_path / "main.safetensors"))
    monkeypatch.setenv("KVQ_DRAFT_SCALES", str(tmp_path / "draft.safetensors"))
    name = "draft_model.model.layers.0.self_attn.attn"
    layers = {name: _impl(monkeypatch=monkeypatch)}
    backend.Int8StaticBuilder(SimpleNamespace(block_size=BS), [name], _vllm_config(layers), "cpu")
    draft = scales.load(str(tmp_path / "draft.safetensors"))["model.layers.0.self_attn.attn"]
    assert torch.equal(layers[name].static["v_scale"], draft["v_scale"])


def test_builder_requires_scales(monkeypatch):
    with pytest.raises(RuntimeError, match="KVQ_SCALES"):
        backend.Int8StaticBuilder(SimpleNamespace(block_size=BS), [], _vllm_config({}), "cpu")


def _common(q_lens, seq_lens, upper=None):
    cu = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32)
    return CommonAttentionMetadata(query_start_loc=cu, query_start_loc_cpu=cu, seq_lens=torch.tensor(seq_lens, dtype=torch.int32),
                                   num_reqs=len(q_lens), num_actual_tokens=int(sum(q_lens)), max_query_len=max(q_lens),
                                   max_seq_len=max(seq_lens), block_table_tensor=torch.zeros(len(q_lens), 64, dtype=torch.int32),
                                   slot_mapping=torch.zeros(int(sum(q_lens)), dtype=torch.int64),
                                   seq_lens_cpu_upper_bound=upper)


def test_builder_plans_the_long_queries_once_per_step(tmp_path, monkeypatch):
    _write_scales(tmp_path / "s.safetensors", ["l0"])
    monkeypatch.setenv("KVQ_SCALES", str(tmp_path / "s.safetensors"))
    b = backend.Int8StaticBuilder(SimpleNamespace(block_size=BS), ["l0"], _vllm_config({"l0": _impl(monkeypatch=monkeypatch)}), "cpu")
    md = b.build(0, _common([1, 1, 4], [100, 7, 300]))
    assert md.kvq_long is None and md.max_query_len == 4
    c = _common([1, 40, 3, 200], [100, 90, 300, 900], upper=torch.tensor([100, 95, 300, 910], dtype=torch.int32))
    md = b.build(0, c)
    ref = ck.plan_long(c.query_start_loc_cpu, c.seq_lens_cpu_upper_bound, BS)
    assert md.kvq_long is not None and md.kvq_long.has_short
    for f in ("src_req", "src_j", "block_table"):
        assert np.array_equal(getattr(md.kvq_long, f), getattr(ref, f))
    assert md.kvq_long.max_seqlen_k == 910


def _split_builder(tmp_path, monkeypatch, spec_tokens=None, max_num_seqs=32):
    _write_scales(tmp_path / "s.safetensors", ["l0"])
    monkeypatch.setenv("KVQ_SCALES", str(tmp_path / "s.safetensors"))
    return backend.Int8StaticBuilder(SimpleNamespace(block_size=BS), ["l0"],
                                     _vllm_config({"l0": _impl(monkeypatch=monkeypatch)}, spec_tokens, max_num_seqs),
                                     "cpu")


@pytest.mark.parametrize("spec,max_seqs,mb,rows", [(None, 32, None, 32), (3, 32, None, 128), (9, 32, None, 256),
                                                   (None, 4096, None, 256 * 2 ** 20 // (HQ * 16 * (D + 2) * 4)),
                                                   (None, 32, "0", 0)])
def test_builder_split_buffers_cover_a_full_batchs_short_tokens(tmp_path, monkeypatch, spec, max_seqs, mb, rows):
    """The builder's own split buffers: max_num_seqs x (1 + speculative tokens, at most SHORT_Q) token rows
    of HQ x 16 pieces, within KVQ_SPLIT_MB (default 256 MiB); none at KVQ_SPLIT_MB=0."""
    if mb is not None:
        monkeypatch.setenv("KVQ_SPLIT_MB", mb)
    b = _split_builder(tmp_path, monkeypatch, spec, max_seqs)
    if rows == 0:
        assert b.kvq_segm is None
        return
    so, sm, ss = b.kvq_segm
    assert tuple(so.shape) == (rows, HQ, backend.SPLIT_PIECES, D) and tuple(sm.shape) == tuple(ss.shape) == (rows, HQ, 16)
    assert so.dtype == sm.dtype == ss.dtype == torch.float32


def test_builder_passes_split_buffers_unless_one_pass_serves(tmp_path, monkeypatch):
    """Per step: split buffers for batches with too few (request, kv head) pairs to give every CU one,
    with pairs that spread over the CUs unevenly (1.5, 2.5 per CU), for skewed lengths and when host
    lengths are unknown; none for requests of even length that give every CU a whole number of pairs,
    or when no request has a short query. A graph being captured always gets them."""
    b = _split_builder(tmp_path, monkeypatch, max_num_seqs=1024)
    assert b.kvq_fill == 256 and backend.Int8StaticBuilder.reorder_batch_threshold == ck.SHORT_Q
    n = b.kvq_fill // HKV                                     # requests whose pairs give every CU one
    even = torch.full((n,), 4096, dtype=torch.int32)
    assert b.build(0, _common([1] * (n - 1), [4096] * (n - 1), upper=even[:n - 1])).kvq_segm is b.kvq_segm
    assert b.build(0, _common([1] * n, [4096] * n, upper=even)).kvq_segm is None
    for per_cu, split in ((1.5, True), (2, False), (2.5, True), (3, False), (4, False)):
        m = int(per_cu * n)
        assert (b.build(0, _common([1] * m, [4096] * m, upper=torch.full((m,), 4096, dtype=torch.int32))).kvq_segm
                is b.kvq_segm) == split, per_cu
    nearly = even.clone()
    nearly[0] = 4300                                          # max / mean just under 1.05: still even
    assert b.build(0, _common([1] * n, nearly.tolist(), upper=nearly)).kvq_segm is None
    skew = even.clone()
    skew[0] = 32768
    assert b.build(0, _common([1] * n, skew.tolist(), upper=skew)).kvq_segm is b.kvq_segm
    assert b.build(0, _common([1] * n, [4096] * n)).kvq_segm is b.kvq_segm            # no host lengths
    # long-query requests do not count: the short ones alone are too few
    mixed = _common([1] * (n - 1) + [100], [4096] * n, upper=torch.full((n,), 4096, dtype=torch.int32))
    assert b.build(0, mixed).kvq_segm is b.kvq_segm
    assert b.build(0, _common([100, 40], [900, 500], upper=torch.tensor([900, 500]))).kvq_segm is None
    assert b.build_for_cudagraph_capture(_common([1] * n, [4096] * n, upper=even)).kvq_segm is b.kvq_segm


def test_host_lengths_never_sync_the_device():
    """The split rule's host lengths: vLLM's upper bounds, else a stored seq_lens_cpu; a seq_lens_cpu that
    the metadata computes on access (a device-to-host copy in recent vLLM) is not touched -- the lengths
    then count as unknown and the split buffers go in."""
    upper, stored = torch.tensor([5, 6]), torch.tensor([7, 8])
    assert backend._host_seq_lens(SimpleNamespace(seq_lens_cpu_upper_bound=upper, seq_lens_cpu=stored)) is upper
    assert backend._host_seq_lens(SimpleNamespace(seq_lens_cpu=stored)) is stored
    touched = []

    class Computed:
        seq_lens_cpu_upper_bound = None

        @property
        def seq_lens_cpu(self):
            touched.append(1)
            return stored
    assert backend._host_seq_lens(Computed()) is None and not touched


@pytest.mark.parametrize("spec,level", [(None, "UNIFORM_BATCH"), (7, "UNIFORM_BATCH"), (8, "UNIFORM_SINGLE_TOKEN_DECODE")])
def test_graph_support_follows_the_verification_length(spec, level):
    cfg = _vllm_config({}, spec_tokens=spec)
    assert backend.Int8StaticBuilder.get_cudagraph_support(cfg, None) is getattr(AttentionCGSupport, level)


# ------------------------------------------------------------------ calibration capture
def test_capture_statistics_feed_from_stats(monkeypatch):
    capture.reset()

    class Impl(TritonAttentionImpl):
        pass

    capture.install(Impl)
    impl = Impl(HQ, D, 0.1, HKV, kv_cache_dtype="auto")
    g = torch.Generator().manual_seed(3)
    cache = torch.zeros(64, HKV, BS, 2 * D, dtype=torch.bfloat16)
    layer = SimpleNamespace(layer_name="model.layers.5.self_attn.attn")
    ks, vs = [], []
    for step, n in enumerate([37, 1, 300]):
        key = (torch.randn(n + 3, HKV, D, generator=g) * 2 + 0.5).to(torch.bfloat16)
        val = torch.randn(n + 3, HKV, D, generator=g).to(torch.bfloat16)
        slots = torch.randperm(64 * BS, generator=g)[:n]
        slots[::5] = -1                                       # padded entries are not recorded
        impl.do_kv_cache_update(layer, key, val, cache, slots)
        ks.append(key[:n][slots >= 0].float())
        vs.append(val[:n][slots >= 0].float())
    k, v = torch.cat(ks), torch.cat(vs)
    st = capture.collect()["stats"][layer.layer_name]
    assert st["tokens"] == k.shape[0]
    assert torch.equal(st["k_absmax"], k.abs().amax(0)) and torch.equal(st["v_absmax"], v.abs().amax(0))
    assert torch.equal(st["k_max"], k.amax(0)) and torch.equal(st["k_min"], k.amin(0))
    assert torch.allclose(st["k_sum"], k.double().sum(0), rtol=0, atol=1e-9)
    out = scales.from_stats(st, smooth_k=True)
    mu = k.mean(0)
    assert torch.allclose(out["k_mu"], mu, atol=1e-6)
    assert torch.allclose(out["k_scale"], torch.maximum(k.amax(0) - mu, mu - k.amin(0)) / 127, rtol=1e-5)
    assert capture.layer_index(layer.layer_name) == 5
    smp = capture.collect()["samples"][layer.layer_name]
    assert smp["k"].shape[0] == k.shape[0] and smp["k"].dtype == torch.float16   # under the sample budget
    capture.reset()


def test_merge_tp_rebuilds_the_model_wide_heads():
    """Each rank recorded its own kv heads; merging puts them back in head order (stats rows, sample
    columns) and keeps one replica when heads are replicated over ranks."""
    def rank(r, heads):
        h = torch.tensor(heads, dtype=torch.float32)[:, None].expand(-1, 3)
        return {"tp_rank": r, "stats": {"l": {"tokens": 5, "k_absmax": h.clone(), "v_absmax": h + 100}},
                "samples": {"l": {"k": h[None].expand(2, -1, -1).clone(), "v": h[None].expand(2, -1, -1) + 100}}}
    st, smp = scales.merge_tp([rank(1, [2, 3]), rank(0, [0, 1])], 4)                 # 4 heads over 2 ranks
    assert st["l"]["k_absmax"][:, 0].tolist() == [0, 1, 2, 3] and st["l"]["tokens"] == 5
    assert smp["l"]["v"][0, :, 0].tolist() == [100, 101, 102, 103]
    st, smp = scales.merge_tp([rank(r, [r * 2 // 4]) for r in (3, 2, 1, 0)], 2)     # 2 heads over 4 ranks
    assert st["l"]["k_absmax"][:, 0].tolist() == [0, 1] and smp["l"]["k"].shape == (2, 2, 3)
    st, _ = scales.merge_tp([rank(0, [0, 1, 2, 3])], 4)
    assert st["l"]["k_absmax"].shape == (4, 3)


def test_from_stats_quantile_of_the_samples():
    """q<frac> scales: the round(frac * tokens)-th smallest |x| per channel over the samples (here |x| runs
    1..200 in every channel, so q0.9 picks 180 and q1.0 the maximum), K centred on its mean first."""
    vals = torch.arange(1, 201, dtype=torch.float32)
    sign = torch.where(torch.arange(200) % 2 == 0, 1.0, -1.0)
    x = (vals * sign)[:, None, None].expand(200, 2, 3).clone()
    st = {"tokens": torch.tensor(200.0), "k_sum": torch.full((2, 3), 200.0 * 7), "k_max": x.amax(0) + 7,
          "k_min": x.amin(0) + 7, "k_absmax": (x + 7).abs().amax(0), "v_absmax": x.abs().amax(0)}
    out = scales.from_stats(st, {"k": x + 7, "v": x}, method="q0.9", smooth_k=True)
    assert torch.allclose(out["k_mu"], torch.full((2, 3), 7.0))
    assert torch.equal(out["k_scale"], torch.full((2, 3), 180.0) / 127) and torch.equal(out["v_scale"], out["k_scale"])
    full = scales.from_stats(st, {"k": x + 7, "v": x}, method="q1.0", granularity="per_head")
    assert torch.equal(full["v_scale"], torch.full((2, 1), 200.0) / 127) and "k_mu" not in full
    with pytest.raises(ValueError):
        scales.from_stats(st, method="p99")
    with pytest.raises(ValueError):
        scales.from_stats(st, granularity="per_token")


def test_scale_file_keys_and_layer_names_with_separators(tmp_path):
    """'<layer>|<field>' keys; layer names with dots round-trip, unknown fields are refused."""
    d = {"draft_model.model.layers.3.self_attn.attn": {"k_scale": torch.ones(2, 1), "v_scale": torch.ones(2, 1)}}
    p = str(tmp_path / "a.safetensors")
    scales.save(p, d)
    back = scales.load(p)
    assert list(back) == list(d) and torch.equal(back[next(iter(d))]["k_scale"], torch.ones(2, 1))
    with pytest.raises(ValueError):
        scales.save(p, {"l": {"k_scales": torch.ones(1, 1)}})
