"""Static INT8 KV-cache attention backend for vLLM (registered as AttentionBackendEnum.CUSTOM), running
the MI355X kernels of kvq.cuda_kernels -- drop-in for the reference's kvq/vllm_int8/backend.py:1-184.

Run vLLM with kv_cache_dtype="int8_static" and attention_config={"backend": "CUSTOM"} (the plugin
kvq.vllm_plugin registers the class), and
  KVQ_SCALES        calibrated static scales (safetensors, kvq.scales format)
  KVQ_DRAFT_SCALES  scales of a speculative-decoding draft model (layers prefixed "draft_model.")
  KVQ_CFG           numerics name; the kernels implement B_channel_smooth (default), B_channel,
                    B_head_smooth and B_head (implementation B, per-(token, head) q, per-tile P)
  KVQ_KERNEL        "cuda" (default; the name is kept for compatibility -- it selects these HIP kernels)

What the backend changes relative to vLLM's Triton backend, whose metadata it reuses:
  * the cache is int8 (vLLM's int8_static cache dtype), K and V of a (block, kv head) interleaved per
    token as in every vLLM paged cache: [num_blocks, H, block_size, 2 D];
  * do_kv_cache_update quantizes the step's new K/V with the static scales while writing them
    (quant_reshape_and_cache), for prefill and decode alike;
  * requests with more than cuda_kernels.SHORT_Q query tokens read their pages dequantized to bf16
    (dequant_pages + a bf16 prefill attention); the page table of that temporary cache is computed
    once per step for all layers, in the metadata builder (plan_long);
  * requests with at most SHORT_Q query tokens (decode, speculative verification) run the INT8 MFMA
    kernel: q quantized on the fly, K/V scales static.
Full graphs are offered only for uniform batches the INT8 kernel covers alone
(get_cudagraph_support); the long-query path sizes buffers from host-side lengths.
"""
import os
from typing import ClassVar

import torch
from vllm.logger import init_logger
from vllm.v1.attention.backend import AttentionCGSupport
from vllm.v1.attention.backends.triton_attn import (
    TritonAttentionBackend,
    TritonAttentionImpl,
    TritonAttentionMetadataBuilder,
)

from kvq import cuda_kernels, scales

logger = init_logger("vllm.kvq")  # a child of vLLM's logger, so vLLM's handler prints it
_SCALES_CACHE = {}

# KVQ_CFG names (the reference's kvq/int8_ref.py:201-223 table) that these kernels implement, with the
# scale layout each implies: (K/V granularity, smooth-K). Every other name of that table is an
# ablation or an implementation-A configuration the kernels do not compute.
KERNEL_CONFIGS = {
    "B_channel_smooth": ("per_channel", True),
    "B_channel": ("per_channel", False),
    "B_head_smooth": ("per_head", True),
    "B_head": ("per_head", False),
}


def _kernel():
    return os.environ.get("KVQ_KERNEL", "cuda")


def _load_scales(path):
    if path not in _SCALES_CACHE:
        _SCALES_CACHE[path] = scales.load(path)
    return _SCALES_CACHE[path]


class Int8StaticBackend(TritonAttentionBackend):
    supported_kv_cache_dtypes: ClassVar[list] = ["int8_static"]

    @staticmethod
    def get_name() -> str:
        return "CUSTOM"

    @staticmethod
    def get_impl_cls():
        return Int8StaticImpl

    @staticmethod
    def get_builder_cls():
        return Int8StaticBuilder

    @classmethod
    def customize_spec(cls, spec):
        return spec  # the scales are per layer in the backend, not stored in the KV pages


class Int8StaticBuilder(TritonAttentionMetadataBuilder):
    """Triton-backend metadata (lengths, block table, split-KV buffers) plus, when a batch holds
    long-query requests, the page table of their temporary bf16 cache (cuda_kernels.plan_long), built
    once per step for all layers. The builder is created after the model is loaded and before graph
    capture, so it hands each layer its static scales here: persistent GPU tensors a captured graph
    keeps pointing at (reference backend.py:68-115)."""

    # a draft-decode step that reuses an older metadata object would also reuse its long-query plan
    supports_draft_decode_metadata_update = False

    @classmethod
    def get_cudagraph_support(cls, vllm_config, kv_cache_spec):
        # Full graphs only for uniform batches the INT8 kernel covers alone; mixed batches run
        # piecewise (attention eager), because the long-query path reads host-side lengths.
        spec = vllm_config.speculative_config
        q_len = 1 + (spec.num_speculative_tokens if spec is not None else 0)
        if q_len <= cuda_kernels.SHORT_Q:
            return AttentionCGSupport.UNIFORM_BATCH
        return AttentionCGSupport.UNIFORM_SINGLE_TOKEN_DECODE

    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        super().__init__(kv_cache_spec, layer_names, vllm_config, device)
        from vllm.distributed import get_tensor_model_parallel_rank, get_tensor_model_parallel_world_size

        path = os.environ.get("KVQ_SCALES")
        if not path:
            raise RuntimeError("kv_cache_dtype int8_static needs calibrated scales: set KVQ_SCALES")
        all_scales = _load_scales(path)
        ctx = vllm_config.compilation_config.static_forward_context
        rank, size = get_tensor_model_parallel_rank(), get_tensor_model_parallel_world_size()
        for name in layer_names:
            src, key = all_scales, name
            if name not in all_scales and os.environ.get("KVQ_DRAFT_SCALES"):
                # a speculative-decoding draft model (prefix "draft_model.") has its own calibration
                src, key = _load_scales(os.environ["KVQ_DRAFT_SCALES"]), name[name.index("model.layers"):]
            if key not in src:
                raise RuntimeError(f"no static scales for layer {name!r} in {path}")
            ctx[name].impl.set_static(scales.for_layer(src, key, rank, size, device))
        logger.info("kvq: static INT8 scales for %d layers from %s (tp %d/%d, cfg %s, MI355X kernels)",
                    len(layer_names), path, rank, size, os.environ.get("KVQ_CFG", "B_channel_smooth"))

    def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
        md = super().build(common_prefix_len, common_attn_metadata, fast_build)
        md.kvq_long = None
        c = common_attn_metadata
        if c.max_query_len > cuda_kernels.SHORT_Q:
            # host lengths may be upper bounds: the plan only reads the long-query rows, where they are exact
            seq_cpu = c.seq_lens_cpu_upper_bound if getattr(c, "seq_lens_cpu_upper_bound", None) is not None \
                else c.seq_lens.cpu()
            md.kvq_long = cuda_kernels.plan_long(c.query_start_loc_cpu, seq_cpu, self.block_size)
        return md


class Int8StaticImpl(TritonAttentionImpl):
    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        assert self.kv_cache_dtype == "int8_static", self.kv_cache_dtype
        self.cfg_name = os.environ.get("KVQ_CFG", "B_channel_smooth")
        kernel = _kernel()
        if kernel == "torch":
            raise NotImplementedError("KVQ_KERNEL=torch (the reference's pure-PyTorch research path) is not part "
                                      "of this package; use the default KVQ_KERNEL=cuda (MI355X HIP kernels)")
        assert kernel in ("cuda", "hip"), kernel
        assert self.cfg_name in KERNEL_CONFIGS, (
            f"the INT8 kernels implement B with per-(token, head) q and per-tile P "
            f"({', '.join(KERNEL_CONFIGS)}), not {self.cfg_name}")
        self.granularity, self.smooth_k = KERNEL_CONFIGS[self.cfg_name]
        self.static = None
        cuda_kernels.ext()  # load the library now, at model build time, long before graph capture

    def fused_output_quant_supported(self, quant_key):
        return False  # the kernels write bf16 output only

    def set_static(self, static):
        """This layer's scales (this TP rank's kv heads); kept as contiguous fp32 GPU tensors for the
        lifetime of the engine. Update them in place, never rebind, once graphs are captured."""
        assert static["k_scale"].shape[0] == self.num_kv_heads, (static["k_scale"].shape, self.num_kv_heads)
        assert ("k_mu" in static) == self.smooth_k, "smooth-K config and scales file disagree"
        want = self.head_size if self.granularity == "per_channel" else 1
        assert static["k_scale"].shape[-1] == want and static["v_scale"].shape[-1] == want, (
            f"{self.cfg_name} expects {self.granularity} scales", static["k_scale"].shape)
        static = {k: v.float().contiguous() for k, v in static.items()}
        if "k_mu" not in static:
            static["k_mu"] = torch.zeros_like(static["k_scale"].expand(-1, self.head_size)).contiguous()
        self.static = static

    def _caches(self, kv_cache):
        # [num_blocks, H, block, 2 D] -> two [num_blocks, block, H, D] strided views (K | V halves)
        return kv_cache.transpose(1, 2).split(self.head_size, dim=-1)

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        key_cache, value_cache = self._caches(kv_cache)
        cuda_kernels.quant_reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, self.static)

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output, output_scale=None,
                output_block_scale=None):
        if attn_metadata is None:
            return output.fill_(0)  # memory-profiling run
        md = attn_metadata
        n = md.num_actual_tokens
        num_reqs = md.query_start_loc.shape[0] - 1
        key_cache, value_cache = self._caches(kv_cache)
        segm = None
        if num_reqs <= md.seq_threshold_3D and n <= md.softmax_segm_max.shape[0]:
            segm = (md.softmax_segm_output, md.softmax_segm_max, md.softmax_segm_expsum)
        cuda_kernels.paged_attention(query[:n], key_cache, value_cache, output[:n], md.query_start_loc, md.seq_lens,
                                     md.block_table, md.max_query_len, self.scale, self.static,
                                     getattr(md, "kvq_long", None), segm)
        return output
