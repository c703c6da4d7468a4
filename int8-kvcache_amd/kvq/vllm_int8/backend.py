"""Static INT8 KV-cache attention backend for vLLM (AttentionBackendEnum.CUSTOM) on the MI355X kernels of
kvq.cuda_kernels. A drop-in for the reference's kvq/vllm_int8/backend.py:1-184: the same classes, the
vLLM hooks they override, environment variables and graph-support levels (vLLM's extension interface),
with its own plumbing.

Run vLLM with kv_cache_dtype="int8_static" and attention_config={"backend": "CUSTOM"} (the plugin
kvq.vllm_plugin registers the class), and
  KVQ_SCALES        calibrated static scales (safetensors, kvq.scales format)
  KVQ_DRAFT_SCALES  scales of a speculative-decoding draft model (layers prefixed "draft_model.")
  KVQ_CFG           numerics name; the kernels implement B_channel_smooth (default), B_channel,
                    B_head_smooth, B_head (implementation B, per-(token, head) q, per-tile P) and
                    B_channel_smooth_qgroup32, B_channel_qgroup32 (q scales per 32 channels)
  KVQ_KERNEL        "cuda" (default; the name is kept for compatibility -- it selects these HIP kernels)

  KVQ_SPLIT_MB      device memory of the backend's split buffers (default 256; 0: none, every request
                    whole in one workgroup)

Per step and layer the backend
  * writes the step's new K/V into the int8 cache quantized with the static scales
    (do_kv_cache_update -> quant_reshape_and_cache); vLLM's cache is [num_blocks, H, block_size, 2 D],
    K and V of a (block, kv head) interleaved per token;
  * runs attention (forward -> paged_attention): requests with more than cuda_kernels.SHORT_Q query
    tokens through dequant_pages + the bf16 prefill kernel (their page plan is made once per step in the
    metadata builder), the others through the INT8 MFMA kernel, with q quantized on the fly.
The INT8 kernel balances a batch by cutting its longest (request, kv head) pairs across workgroups; the
cut pieces go to split buffers that the builder allocates once, sized for the short-query tokens of a
full batch (vLLM's own split buffers hold only 128 // kv-heads requests' rows, and the reference passes
them only to batches that small). Short-query requests are ordered first (reorder_batch_threshold), so
their tokens are the buffers' rows. Each step the builder passes them unless the batch is one that a
single pass serves as well: requests whose (request, kv head) pairs fill every CU with a whole number
of pairs each (one workgroup per CU streams them in turn) and lengths within 5% of even.
Full graphs are offered only for uniform batches the INT8 kernel covers alone (the long-query path sizes
buffers from host-side lengths).
"""
import inspect
import os
from typing import ClassVar

import numpy as np
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

DEFAULT_CFG = "B_channel_smooth"
# KVQ_CFG names of the reference's numerics table (kvq/int8_ref.py:201-223) these kernels compute, with
# what each implies: (K/V scale granularity, smooth-K, q scale group: None = per (token, q head)). The
# table's other names are ablations or implementation-A configurations.
KERNEL_CONFIGS = {
    "B_channel_smooth": ("per_channel", True, None),
    "B_channel": ("per_channel", False, None),
    "B_head_smooth": ("per_head", True, None),
    "B_head": ("per_head", False, None),
    # q scales per 32 channels (q_gran "group32", kvq/int8_ref.py:120-129)
    "B_channel_smooth_qgroup32": ("per_channel", True, 32),
    "B_channel_qgroup32": ("per_channel", False, 32),
}
SPLIT_PIECES = cuda_kernels.SPLIT_PIECES   # pieces per (request, kv head) the split buffers hold
DRAFT_PREFIX_END = "model.layers"   # a draft layer "draft_model.model.layers.<i>..." is "model.layers.<i>..."
                                    # in the draft's own calibration file


class _ScaleFiles:
    """Scale files read once per process (every layer's builder shares them)."""

    def __init__(self):
        self.files = {}

    def get(self, path):
        if path not in self.files:
            self.files[path] = scales.load(path)
        return self.files[path]

    def clear(self):
        self.files.clear()


SCALE_FILES = _ScaleFiles()


def _check_kernel_choice():
    kernel = os.environ.get("KVQ_KERNEL", "cuda")
    if kernel == "torch":
        raise NotImplementedError("KVQ_KERNEL=torch (the reference's pure-PyTorch research path) is not part "
                                  "of this package; use the default KVQ_KERNEL=cuda (MI355X HIP kernels)")
    assert kernel in ("cuda", "hip"), f"unknown KVQ_KERNEL {kernel!r}"


def _layer_scale_set(layer, main_path):
    """(scale set, key) holding `layer`'s scales: the main file, or for a draft-model layer that the
    main file lacks, KVQ_DRAFT_SCALES under the layer's name inside the draft model."""
    main = SCALE_FILES.get(main_path)
    if layer in main:
        return main, layer
    draft_path = os.environ.get("KVQ_DRAFT_SCALES")
    at = layer.find(DRAFT_PREFIX_END)
    if draft_path and at >= 0:
        draft = SCALE_FILES.get(draft_path)
        if layer[at:] in draft:
            return draft, layer[at:]
    raise RuntimeError(f"no static scales for layer {layer!r} in {main_path}"
                       + (f" or {draft_path}" if draft_path else ""))


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
    """Triton-backend metadata (lengths, block table) plus the split buffers this step's INT8 call gets
    (kvq_segm, see _split_for) and, when a step holds long-query requests, their temporary bf16 page plan (cuda_kernels.plan_long, built once per step for
    all layers). vLLM creates the builder after loading the model and before capturing graphs, so it is
    where every layer receives its static scales: persistent GPU tensors captured graphs keep pointing
    at (reference backend.py:68-115)."""

    # a draft-decode step that reuses an older metadata object would also reuse its long-query plan
    supports_draft_decode_metadata_update = False
    # requests with at most SHORT_Q query tokens first: their tokens are then rows [0, n) of the batch,
    # the rows the split buffers hold
    reorder_batch_threshold = cuda_kernels.SHORT_Q

    @classmethod
    def get_cudagraph_support(cls, vllm_config, kv_cache_spec):
        """Whole-graph capture for uniform batches whose query length (1 + speculative tokens) the INT8
        kernel serves alone; otherwise single-token decode batches only. Mixed batches run piecewise."""
        spec = vllm_config.speculative_config
        verify_len = 1 if spec is None else 1 + spec.num_speculative_tokens
        return (AttentionCGSupport.UNIFORM_BATCH if verify_len <= cuda_kernels.SHORT_Q
                else AttentionCGSupport.UNIFORM_SINGLE_TOKEN_DECODE)

    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        super().__init__(kv_cache_spec, layer_names, vllm_config, device)
        from vllm.distributed import get_tensor_model_parallel_rank, get_tensor_model_parallel_world_size

        path = os.environ.get("KVQ_SCALES")
        if not path:
            raise RuntimeError("kv_cache_dtype int8_static needs calibrated scales: set KVQ_SCALES")
        tp = (get_tensor_model_parallel_rank(), get_tensor_model_parallel_world_size())
        layers = vllm_config.compilation_config.static_forward_context
        for layer in layer_names:
            src, key = _layer_scale_set(layer, path)
            layers[layer].impl.set_static(scales.for_layer(src, key, *tp, device))
        impl = layers[layer_names[0]].impl if layer_names else None
        self.kvq_hkv = impl.num_kv_heads if impl else 1
        self.kvq_segm = self._split_buffers_for(vllm_config, impl.num_heads, impl.head_size, device) if impl else None
        self.kvq_fill = cuda_kernels.one_pass_fill(device)
        logger.info("kvq: static INT8 scales for %d layers from %s (tp %d/%d, cfg %s, MI355X kernels, split "
                    "buffers for %d tokens)", len(layer_names), path, tp[0], tp[1],
                    os.environ.get("KVQ_CFG", DEFAULT_CFG), 0 if self.kvq_segm is None else self.kvq_segm[1].shape[0])

    @staticmethod
    def _split_buffers_for(vllm_config, num_heads, head_size, device):
        """Split buffers [rows, Hq, SPLIT_PIECES(, D)] for the short-query tokens of a full batch
        (max_num_seqs requests of 1 + speculative tokens each), within KVQ_SPLIT_MB; None if none fit.
        Allocated once, before graph capture; every layer's call reuses them (calls are stream-ordered)."""
        spec = vllm_config.speculative_config
        per_req = min(cuda_kernels.SHORT_Q, 1 if spec is None else 1 + spec.num_speculative_tokens)
        per_row = num_heads * SPLIT_PIECES * (head_size + 2) * 4
        budget = int(float(os.environ.get("KVQ_SPLIT_MB", "256")) * 2 ** 20)
        rows = min(vllm_config.scheduler_config.max_num_seqs * per_req, budget // per_row)
        if rows <= 0:
            return None
        return cuda_kernels.split_buffers(rows, num_heads, head_size, SPLIT_PIECES, device)

    def _split_for(self, c, capturing=False):
        """The split buffers for this step, or None where one pass serves as well (cuda_kernels.split_pays:
        short-query requests whose pairs fill the CUs evenly, host-side lengths even). A graph being captured always
        gets them: its replays see other lengths, and the kernel cuts only what the lengths it reads on
        the device call for."""
        if self.kvq_segm is None:
            return None
        if capturing:
            return self.kvq_segm
        lens = _host_seq_lens(c)
        pays = cuda_kernels.split_pays(np.diff(c.query_start_loc_cpu.numpy()), None if lens is None else lens.numpy(),
                                       self.kvq_hkv, self.kvq_fill)
        return self.kvq_segm if pays else None

    def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
        md = super().build(common_prefix_len, common_attn_metadata, fast_build)
        c = common_attn_metadata
        md.kvq_long = None
        if c.max_query_len > cuda_kernels.SHORT_Q:
            # host-side lengths: upper bounds are fine, the plan only copies pages of the long requests
            upper = getattr(c, "seq_lens_cpu_upper_bound", None)
            md.kvq_long = cuda_kernels.plan_long(c.query_start_loc_cpu, c.seq_lens.cpu() if upper is None else upper,
                                                 self.block_size)
        md.kvq_segm = self._split_for(c)
        return md

    def build_for_cudagraph_capture(self, common_attn_metadata):
        md = super().build_for_cudagraph_capture(common_attn_metadata)
        md.kvq_segm = self._split_for(common_attn_metadata, capturing=True)
        return md


def _host_seq_lens(c):
    """Host-side key counts of a batch without a device sync: vLLM's upper bounds when it has them, else
    seq_lens_cpu if it is stored data (recent vLLM computes seq_lens_cpu on access from the device tensor,
    a device-to-host copy per step); None (unknown) otherwise."""
    lens = getattr(c, "seq_lens_cpu_upper_bound", None)
    if lens is not None:
        return lens
    if isinstance(inspect.getattr_static(c, "seq_lens_cpu", None), property):
        return None
    return getattr(c, "seq_lens_cpu", None)


class Int8StaticImpl(TritonAttentionImpl):
    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        assert self.kv_cache_dtype == "int8_static", self.kv_cache_dtype
        _check_kernel_choice()
        self.cfg_name = os.environ.get("KVQ_CFG", DEFAULT_CFG)
        assert self.cfg_name in KERNEL_CONFIGS, (
            f"the INT8 kernels implement B with per-(token, head) or per-32-channel q and per-tile P "
            f"({', '.join(KERNEL_CONFIGS)}), not {self.cfg_name}")
        self.granularity, self.smooth_k, self.q_group = KERNEL_CONFIGS[self.cfg_name]
        self.static = None
        cuda_kernels.ext()  # load the library now, at model build time, long before graph capture

    def fused_output_quant_supported(self, quant_key):
        return False  # the kernels write bf16 output only

    def set_static(self, static):
        """This layer's scales (this TP rank's kv heads), kept as contiguous float32 GPU tensors for the
        engine's lifetime; once graphs are captured, update them in place, never rebind. A config without
        smooth-K gets an all-zero mean."""
        cols = self.head_size if self.granularity == "per_channel" else 1
        assert static["k_scale"].shape[0] == self.num_kv_heads, (static["k_scale"].shape, self.num_kv_heads)
        assert ("k_mu" in static) == self.smooth_k, "smooth-K config and scales file disagree"
        assert static["k_scale"].shape[-1] == cols and static["v_scale"].shape[-1] == cols, (
            f"{self.cfg_name} expects {self.granularity} scales", static["k_scale"].shape)
        prepared = {field: t.float().contiguous() for field, t in static.items()}
        prepared.setdefault("k_mu", torch.zeros(self.num_kv_heads, self.head_size, dtype=torch.float32,
                                                device=prepared["k_scale"].device))
        self.static = prepared

    def _caches(self, kv_cache):
        """vLLM's [num_blocks, H, block_size, 2 D] int8 cache as the kernels' K and V views
        [num_blocks, block_size, H, D] (strided, no copy)."""
        by_slot = kv_cache.permute(0, 2, 1, 3)
        return by_slot[..., :self.head_size], by_slot[..., self.head_size:]

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        k_cache, v_cache = self._caches(kv_cache)
        cuda_kernels.quant_reshape_and_cache(key, value, k_cache, v_cache, slot_mapping, self.static)

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output, output_scale=None,
                output_block_scale=None):
        if attn_metadata is None:
            return output.fill_(0)  # memory-profiling run
        md = attn_metadata
        n = md.num_actual_tokens
        k_cache, v_cache = self._caches(kv_cache)
        cuda_kernels.paged_attention(query[:n], k_cache, v_cache, output[:n], md.query_start_loc, md.seq_lens,
                                     md.block_table, md.max_query_len, self.scale, self.static,
                                     getattr(md, "kvq_long", None), getattr(md, "kvq_segm", None),
                                     q_group=self.q_group)
        return output
