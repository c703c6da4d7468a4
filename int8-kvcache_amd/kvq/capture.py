"""Calibration capture: what vLLM writes into the KV cache, per attention layer, so that static scales can
be computed (the reference's kvq/capture.py:1-118; scales.from_stats turns the result into a scale set,
scales.merge_tp joins tensor-parallel ranks, scales.save writes the file).

Installed by the plugin when KVQ_CAPTURE=1: it wraps a bf16 attention backend's do_kv_cache_update and
folds every batch of valid (slot >= 0) K/V rows into a per-layer record of
  * running per-(kv head, channel) statistics of K and V: signed max and min, |x| max (= max(max, -min)),
    and the sum in float64 (for the smooth-K mean) -- the fields scales.from_stats reads;
  * a host-side fp16 sample of rows for quantile scales, bounded by KVQ_CAPTURE_MAX_TOKENS: every row
    while the sample holds at most half the budget, then a random eighth (at least one row) of each
    batch, until the budget is reached.
collect() hands the records of one worker back (e.g. through LLM.collective_rpc).

The wrapped backend is KVQ_CAPTURE_BACKEND ("module:Class") or, by default, vLLM's Triton attention
implementation, which serves bf16 caches on ROCm.
"""
import importlib
import os

import torch

MAX_SAMPLE_TOKENS = int(os.environ.get("KVQ_CAPTURE_MAX_TOKENS", "16384"))
DEFAULT_BACKEND = "vllm.v1.attention.backends.triton_attn:TritonAttentionImpl"


class LayerRecord:
    """Statistics and row sample of one attention layer."""

    def __init__(self):
        self.tokens = 0
        self.hi, self.lo, self.total = {}, {}, {}      # side -> [heads, D] running max / min / float64 sum
        self.sample = {"k": [], "v": []}
        self.sampled = 0

    def add(self, key, value, budget):
        for side, x in (("k", key), ("v", value)):
            lo, hi = torch.aminmax(x.float(), dim=0)
            total = x.double().sum(dim=0)
            if side in self.hi:
                self.hi[side] = torch.maximum(self.hi[side], hi)
                self.lo[side] = torch.minimum(self.lo[side], lo)
                self.total[side] = self.total[side] + total
            else:
                self.hi[side], self.lo[side], self.total[side] = hi, lo, total
        self.tokens += key.shape[0]
        self._keep_rows(key, value, budget)

    def _keep_rows(self, key, value, budget):
        if self.sampled >= budget:
            return
        if self.sampled > budget // 2:       # past half the budget: an eighth of the batch, at random
            pick = torch.randperm(key.shape[0], device=key.device)[:max(1, key.shape[0] // 8)]
            key, value = key.index_select(0, pick), value.index_select(0, pick)
        self.sample["k"].append(key.to(torch.float16).cpu())
        self.sample["v"].append(value.to(torch.float16).cpu())
        self.sampled += key.shape[0]

    def stats(self):
        """The fields scales.from_stats reads, on the host."""
        out = {"tokens": self.tokens}
        for side in self.hi:
            hi, lo = self.hi[side].cpu(), self.lo[side].cpu()
            out.update({f"{side}_max": hi, f"{side}_min": lo, f"{side}_absmax": torch.maximum(hi, -lo),
                        f"{side}_sum": self.total[side].cpu()})
        return out

    def samples(self):
        return {side: torch.cat(rows) for side, rows in self.sample.items()}


RECORDS = {}   # layer name -> LayerRecord (this process)


def layer_index(name):
    """Decoder layer number in a vLLM layer name ("model.layers.<i>.self_attn.attn")."""
    return int(name.split("layers.")[1].split(".")[0])


def record(name, key, value):
    """Fold one batch of valid K/V rows ([tokens, kv heads, D]) into layer `name`'s record."""
    if key.shape[0]:
        RECORDS.setdefault(name, LayerRecord()).add(key, value, MAX_SAMPLE_TOKENS)


def _impl_class():
    module, cls = os.environ.get("KVQ_CAPTURE_BACKEND", DEFAULT_BACKEND).split(":")
    return getattr(importlib.import_module(module), cls)


def install(impl_cls=None):
    """Wrap impl_cls.do_kv_cache_update (default: KVQ_CAPTURE_BACKEND) so every cache write is recorded
    before it happens."""
    impl_cls = impl_cls or _impl_class()
    write = impl_cls.do_kv_cache_update

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        rows = slot_mapping.shape[0]
        real = slot_mapping >= 0
        record(layer.layer_name, key[:rows][real], value[:rows][real])
        return write(self, layer, key, value, kv_cache, slot_mapping)

    impl_cls.do_kv_cache_update = do_kv_cache_update
    return impl_cls


def _tp_position():
    try:
        from vllm.distributed import get_tensor_model_parallel_rank, get_tensor_model_parallel_world_size
        return get_tensor_model_parallel_rank(), get_tensor_model_parallel_world_size()
    except (ImportError, AssertionError):
        return 0, 1


def collect(worker=None):
    """This worker's records on the host, tagged with its TP rank and size (the input of
    scales.merge_tp): {"stats": {layer: {...}}, "samples": {layer: {"k", "v"}}, "tp_rank", "tp_size"}."""
    rank, size = _tp_position()
    return {"stats": {name: r.stats() for name, r in RECORDS.items()},
            "samples": {name: r.samples() for name, r in RECORDS.items()},
            "tp_rank": rank, "tp_size": size}


def reset():
    RECORDS.clear()
