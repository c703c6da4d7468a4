"""Calibration capture: record what vLLM writes into the KV cache, per attention layer, so that static
scales can be computed (reference kvq/capture.py:1-118; scales.from_stats turns the result into a
scale set, scales.merge_tp joins tensor-parallel ranks, scales.save writes the file).

Installed by the plugin when KVQ_CAPTURE=1. It wraps the bf16 attention backend's do_kv_cache_update
and keeps, per layer:
  * running per-(kv head, channel) statistics of K and V: |x| max, signed max / min, and the sum in
    float64 (for the smooth-K mean) -- the keys scales.from_stats reads;
  * a sample of K/V rows (fp16, host memory) for quantile scales: every token until
    KVQ_CAPTURE_MAX_TOKENS / 2, then a random eighth of each batch, up to KVQ_CAPTURE_MAX_TOKENS.
Read back per worker with collect() (e.g. through LLM.collective_rpc).

The backend that is wrapped is KVQ_CAPTURE_BACKEND ("module:Class") or, by default, vLLM's
Triton attention implementation, which serves bf16 caches on ROCm.
"""
import importlib
import os

import torch

STATE = {"stats": {}, "samples": {}}
MAX_SAMPLE_TOKENS = int(os.environ.get("KVQ_CAPTURE_MAX_TOKENS", "16384"))
DEFAULT_BACKEND = "vllm.v1.attention.backends.triton_attn:TritonAttentionImpl"


def layer_index(name):
    return int(name.split("layers.")[1].split(".")[0])


def record(name, key, value):
    """Fold one batch of valid K/V rows ([tokens, kv_heads, D]) into layer `name`'s statistics. One
    min/max pass per side: max |x| over tokens equals max(max x, -min x) exactly."""
    if key.shape[0] == 0:
        return  # a step whose slots are all padding
    st = STATE["stats"].setdefault(name, {"tokens": 0})
    for side, x in (("k", key), ("v", value)):
        lo, hi = torch.aminmax(x.float(), dim=0)
        total = x.double().sum(0)
        if f"{side}_max" in st:
            torch.maximum(st[f"{side}_max"], hi, out=st[f"{side}_max"])
            torch.minimum(st[f"{side}_min"], lo, out=st[f"{side}_min"])
            st[f"{side}_sum"] += total
        else:
            st[f"{side}_max"], st[f"{side}_min"], st[f"{side}_sum"] = hi, lo, total
        st[f"{side}_absmax"] = torch.maximum(st[f"{side}_max"], -st[f"{side}_min"])
    st["tokens"] += key.shape[0]
    _sample(name, key, value)


def _sample(name, key, value):
    """Keep rows for quantile scales: all of them up to half the budget, then an eighth of each batch."""
    smp = STATE["samples"].setdefault(name, {"k": [], "v": [], "n": 0})
    if smp["n"] >= MAX_SAMPLE_TOKENS:
        return
    if smp["n"] > MAX_SAMPLE_TOKENS // 2:
        keep = torch.randperm(key.shape[0], device=key.device)[: max(1, key.shape[0] // 8)]
        key, value = key[keep], value[keep]
    smp["k"].append(key.to(torch.float16).cpu())
    smp["v"].append(value.to(torch.float16).cpu())
    smp["n"] += key.shape[0]


def _impl_class():
    spec = os.environ.get("KVQ_CAPTURE_BACKEND", DEFAULT_BACKEND)
    module, cls = spec.split(":")
    return getattr(importlib.import_module(module), cls)


def install(impl_cls=None):
    """Wrap impl_cls.do_kv_cache_update (default: KVQ_CAPTURE_BACKEND) to record every write."""
    impl_cls = impl_cls or _impl_class()
    orig_update = impl_cls.do_kv_cache_update

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        n = slot_mapping.shape[0]
        valid = slot_mapping >= 0
        record(layer.layer_name, key[:n][valid], value[:n][valid])
        return orig_update(self, layer, key, value, kv_cache, slot_mapping)

    impl_cls.do_kv_cache_update = do_kv_cache_update
    return impl_cls


def collect(worker=None):
    """This worker's statistics and samples on the host, tagged with its TP rank and size (the input
    of scales.merge_tp)."""
    try:
        from vllm.distributed import get_tensor_model_parallel_rank, get_tensor_model_parallel_world_size
        rank, size = get_tensor_model_parallel_rank(), get_tensor_model_parallel_world_size()
    except (ImportError, AssertionError):
        rank, size = 0, 1
    out = {"stats": {}, "samples": {}, "tp_rank": rank, "tp_size": size}
    for name, st in STATE["stats"].items():
        out["stats"][name] = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in st.items()}
    for name, smp in STATE["samples"].items():
        out["samples"][name] = {"k": torch.cat(smp["k"]), "v": torch.cat(smp["v"])}
    return out


def reset():
    STATE["stats"].clear()
    STATE["samples"].clear()
