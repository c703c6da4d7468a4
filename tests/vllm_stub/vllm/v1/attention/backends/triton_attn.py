"""The Triton attention backend's classes as the kvq backend uses them: constructor arguments,
attributes, and the metadata fields read in forward (query_start_loc, seq_lens, block_table,
max_query_len, num_actual_tokens, seq_threshold_3D and the split-KV buffers softmax_segm_*), and the
builder's hooks the kvq builder overrides (build, build_for_cudagraph_capture)."""
from dataclasses import dataclass

import torch

from vllm.v1.attention.backend import AttentionCGSupport

NUM_SEGMENTS = 16
MIN_LAUNCH_GRID_SIZE_2D = 128   # the Triton backend uses its split-KV (3D) kernel below this many programs


class TritonAttentionBackend:
    supported_kv_cache_dtypes = ["auto", "bfloat16"]

    @staticmethod
    def get_name():
        return "TRITON_ATTN"

    @staticmethod
    def get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size, cache_dtype_str="auto"):
        return (num_blocks, num_kv_heads, block_size, 2 * head_size)


@dataclass
class TritonAttentionMetadata:
    num_actual_tokens: int
    max_query_len: int
    query_start_loc: torch.Tensor
    max_seq_len: int
    seq_lens: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    seq_threshold_3D: int
    softmax_segm_output: torch.Tensor
    softmax_segm_max: torch.Tensor
    softmax_segm_expsum: torch.Tensor


@dataclass
class CommonAttentionMetadata:
    query_start_loc: torch.Tensor
    query_start_loc_cpu: torch.Tensor
    seq_lens: torch.Tensor
    num_reqs: int
    num_actual_tokens: int
    max_query_len: int
    max_seq_len: int
    block_table_tensor: torch.Tensor
    slot_mapping: torch.Tensor
    seq_lens_cpu_upper_bound: torch.Tensor = None


class TritonAttentionMetadataBuilder:
    _cudagraph_support = AttentionCGSupport.ALWAYS

    @classmethod
    def get_cudagraph_support(cls, vllm_config, kv_cache_spec):
        return cls._cudagraph_support

    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        self.kv_cache_spec = kv_cache_spec
        self.layer_names = layer_names
        self.vllm_config = vllm_config
        self.device = device
        self.block_size = kv_cache_spec.block_size
        mc = vllm_config.model_config
        # as vLLM's Triton builder: batches of up to MIN_LAUNCH_GRID_SIZE_2D // kv heads requests get the
        # split-KV buffers, which hold that many query rows; larger batches get none
        self.seq_threshold_3D = MIN_LAUNCH_GRID_SIZE_2D // mc.num_kv_heads
        rows = self.seq_threshold_3D
        self.softmax_segm_output = torch.empty(rows, mc.num_heads, NUM_SEGMENTS, mc.head_size, dtype=torch.float32,
                                               device=device)
        self.softmax_segm_max = torch.empty(rows, mc.num_heads, NUM_SEGMENTS, dtype=torch.float32, device=device)
        self.softmax_segm_expsum = torch.empty_like(self.softmax_segm_max)

    def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
        c = common_attn_metadata
        return TritonAttentionMetadata(
            num_actual_tokens=c.num_actual_tokens, max_query_len=c.max_query_len, query_start_loc=c.query_start_loc,
            max_seq_len=c.max_seq_len, seq_lens=c.seq_lens, block_table=c.block_table_tensor,
            slot_mapping=c.slot_mapping, seq_threshold_3D=self.seq_threshold_3D,
            softmax_segm_output=self.softmax_segm_output, softmax_segm_max=self.softmax_segm_max,
            softmax_segm_expsum=self.softmax_segm_expsum)

    def build_for_cudagraph_capture(self, common_attn_metadata):
        """vLLM's AttentionMetadataBuilder default: the metadata a graph is captured with."""
        return self.build(0, common_attn_metadata)


class TritonAttentionImpl:
    def __init__(self, num_heads, head_size, scale, num_kv_heads, alibi_slopes=None, sliding_window=None,
                 kv_cache_dtype="auto", logits_soft_cap=None, attn_type="decoder", kv_sharing_target_layer_name=None,
                 sinks=None):
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads
        self.kv_cache_dtype = kv_cache_dtype

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        """bf16 cache write (the stand-in for vLLM's reshape_and_cache)."""
        n = slot_mapping.shape[0]
        slots = slot_mapping.long()
        ok = slots >= 0
        bs = kv_cache.shape[2]
        kc, vc = kv_cache.transpose(1, 2).split(self.head_size, dim=-1)
        blk, off = slots[ok] // bs, slots[ok] % bs
        kc[blk, off] = key[:n][ok].to(kv_cache.dtype)
        vc[blk, off] = value[:n][ok].to(kv_cache.dtype)
