"""Operator API of the static INT8 KV cache on MI355X -- drop-in for the reference's kvq/cuda_kernels.py.

Same names, arguments, defaults, environment variables and error behaviour as the reference module
(kvq/cuda_kernels.py:1-183); the kernels behind it are the gfx950 HIP kernels of libkvq_int8.so,
reached through its C ABI (include/kvq_int8.h) with ctypes. The library is built in-tree ahead of
time (int8-kvcache_amd/build.py); ext() loads it and raises if it is missing -- there is no fallback.

Attention on the INT8 cache is split by query length (reference kvq/cuda_kernels.py:1-11):
  * requests with at most SHORT_Q query tokens run the INT8 MFMA kernel (implementation B);
  * longer ones have their pages dequantized into a bf16 paged cache (dequant_pages, HIP) that a
    bf16 prefill attention reads (implementation A). The page table of that temporary cache comes
    from plan_long(), once per step for all layers.
In a mixed batch the long requests run first, then the INT8 kernel writes the short requests' rows.

Everything is enqueued on the current torch stream; no call synchronises the host except the
KVQ_DEBUG=1 input check, so fixed-shape calls can be captured in a HIP graph.
"""
import os
from dataclasses import dataclass

import numpy as np
import torch

from . import _native

# q_len at or below this: INT8 kernel; above: dequantize + bf16 attention (cuda_kernels.py:18-21).
SHORT_Q = int(os.environ.get("KVQ_SHORT_Q", 8))

MAX_SPLITS = 64

_EXT = None


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _check_cuda(name, *ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        _check(t.is_cuda, f"{name}: every tensor must be on the GPU (got {t.device})")
        if dev is None:
            dev = t.device
        _check(t.device == dev, f"{name}: tensors on different devices ({dev} vs {t.device})")


def _scale_cols(s, name, heads, d):
    _check(s.dtype == torch.float32 and s.is_contiguous() and s.dim() == 2,
           f"{name}: scales must be contiguous float32 [num_kv_heads, D] or [num_kv_heads, 1], got "
           f"{tuple(s.shape)} {s.dtype}")
    _check(s.shape[0] == heads and s.shape[1] in (1, d),
           f"{name}: scale shape {tuple(s.shape)} does not match {heads} kv heads x head_dim {d}")
    return s.shape[1]


class _Ext:
    """The native ops under the reference's pybind names (kvq/cuda/int8_kv.cu:674-679), taking
    torch tensors; each checks what the reference TORCH_CHECKs, then calls the C ABI."""

    def __init__(self):
        _native.load()

    # kvq/cuda/int8_kv.cu:554-575
    def quant_cache(self, key, value, kc, vc, slots, ks, vs, kmu):
        n, H = slots.shape[0], key.shape[1]
        _check(key.shape[2] == kc.shape[3] and key.stride(2) == 1 and kc.stride(3) == 1, "contiguous last dim")
        _check(value.shape[2] == vc.shape[3] and value.stride(2) == 1 and vc.stride(3) == 1, "contiguous last dim")
        if n == 0:
            return
        _check_cuda("quant_cache", key, value, kc, vc, slots, ks, vs, kmu)
        _check(key.dtype == torch.bfloat16 and value.dtype == torch.bfloat16, "quant_cache: key/value must be bf16")
        _check(kc.dtype == torch.int8 and vc.dtype == torch.int8, "quant_cache: caches must be int8")
        _check(slots.dtype == torch.int64 and slots.dim() == 1 and slots.stride(0) == 1,
               "quant_cache: slot_mapping must be a contiguous int64 vector")
        _check(key.shape[0] >= n and value.shape[0] >= n, "quant_cache: fewer key rows than slots")
        _check(kc.shape == vc.shape and kc.shape[2] == H, "quant_cache: cache shapes disagree with key")
        d = key.shape[2]
        kcols = _scale_cols(ks, "quant_cache k_scale", H, d)
        vcols = _scale_cols(vs, "quant_cache v_scale", H, d)
        _check(kmu.dtype == torch.float32 and kmu.is_contiguous() and tuple(kmu.shape) == (H, d),
               "quant_cache: k_mu must be contiguous float32 [num_kv_heads, D]")
        _native.call("kvq_quant_cache", key.data_ptr(), key.stride(0), key.stride(1), value.data_ptr(),
                     value.stride(0), value.stride(1), kc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2),
                     vc.data_ptr(), vc.stride(0), vc.stride(1), vc.stride(2), slots.data_ptr(), n, H, d,
                     kc.shape[0], kc.shape[1], ks.data_ptr(), kcols, vs.data_ptr(), vcols, kmu.data_ptr(),
                     _stream(key))

    # kvq/cuda/int8_kv.cu:577-598
    def quant_q(self, q, ks, group):
        T, Hq = q.shape[0], q.shape[1]
        _check(q.shape[2] == 128 and group in (128, 32), "standalone q quantization: head_dim 128")
        q_i8 = torch.empty(T, Hq, 128, dtype=torch.int8, device=q.device)
        q_s = torch.empty(T, Hq, 128 // group, dtype=torch.float32, device=q.device)
        if T == 0:
            return [q_i8, q_s]
        _check_cuda("quant_q", q, ks)
        _check(q.dtype == torch.bfloat16 and q.stride(2) == 1, "quant_q: q must be bf16 with a contiguous last dim")
        hkv = ks.shape[0]
        _check(hkv > 0 and Hq % hkv == 0, f"quant_q: {Hq} q heads not a multiple of {hkv} kv heads")
        kcols = _scale_cols(ks, "quant_q k_scale", hkv, 128)
        _native.call("kvq_quant_q", q.data_ptr(), q.stride(0), q.stride(1), T, Hq, 128, ks.data_ptr(), hkv, kcols,
                     group, q_i8.data_ptr(), q_s.data_ptr(), _stream(q))
        return [q_i8, q_s]

    # kvq/cuda/int8_kv.cu:600-648
    def int8_decode_attention(self, q, kc, vc, out, cu_q, seq_lens, block_table, ks, vs, softmax_scale, segm_out,
                              segm_max, segm_sum, max_query_len, qmax, q_group=None):
        num_seqs, Hq, Hkv = cu_q.shape[0] - 1, q.shape[1], kc.shape[2]
        _check(q.shape[2] == kc.shape[3] and kc.stride(3) == 1 and q.stride(2) == 1, "unsupported shape/layout")
        bs = kc.shape[1]
        _check(bs >= 16 and (bs & (bs - 1)) == 0, "block_size must be a power of two >= 16")
        if num_seqs == 0:
            return
        split = segm_max is not None
        S = segm_max.shape[2] if split else 1
        _check(S <= MAX_SPLITS, f"at most {MAX_SPLITS} split-KV segments")
        _check_cuda("int8_decode_attention", q, kc, vc, out, cu_q, seq_lens, block_table, ks, vs, segm_out,
                    segm_max, segm_sum)
        _check(q.dtype == torch.bfloat16 and out.dtype == torch.bfloat16, "int8_decode_attention: q/out must be bf16")
        _check(kc.dtype == torch.int8 and vc.dtype == torch.int8 and vc.shape == kc.shape and vc.stride(3) == 1,
               "int8_decode_attention: caches must be int8 [num_blocks, block_size, kv_heads, D] views")
        _check(out.shape[1:] == q.shape[1:] and out.stride(2) == 1 and out.shape[0] >= q.shape[0],
               "int8_decode_attention: out must match q")
        for t, nm in ((cu_q, "cu_seqlens_q"), (seq_lens, "seq_lens"), (block_table, "block_table")):
            _check(t.dtype == torch.int32, f"int8_decode_attention: {nm} must be int32")
        _check(cu_q.is_contiguous() and seq_lens.is_contiguous() and block_table.stride(-1) == 1,
               "int8_decode_attention: index tensors must be contiguous")
        _check(seq_lens.shape[0] >= num_seqs and block_table.shape[0] >= num_seqs,
               "int8_decode_attention: seq_lens / block_table have fewer rows than requests")
        _check(Hq % Hkv == 0, f"int8_decode_attention: {Hq} q heads not a multiple of {Hkv} kv heads")
        d = q.shape[2]
        kcols = _scale_cols(ks, "int8_decode_attention k_scale", Hkv, d)
        vcols = _scale_cols(vs, "int8_decode_attention v_scale", Hkv, d)
        seg_st = seg_sh = 0
        if split:
            _check(segm_out is not None and segm_sum is not None, "int8_decode_attention: split buffers missing")
            for t in (segm_out, segm_max, segm_sum):
                _check(t.dtype == torch.float32 and t.shape[0] == segm_max.shape[0] and t.shape[1] == Hq and
                       t.shape[2] == S, "int8_decode_attention: split buffers must be float32 [rows, Hq, S(, D)]")
            _check(segm_max.stride(2) == 1 and segm_sum.stride() == segm_max.stride(),
                   "int8_decode_attention: segm_max / segm_sum layouts differ")
            seg_st, seg_sh = segm_max.stride(0), segm_max.stride(1)
            _check(segm_out.shape[3] == d and segm_out.stride(3) == 1 and segm_out.stride(2) == d and
                   segm_out.stride(1) == seg_sh * d and segm_out.stride(0) == seg_st * d,
                   "int8_decode_attention: segm_out must be laid out as segm_max x head_dim")
        _check(q_group in (None, d, 32), f"int8_decode_attention: q scales per row or per 32 channels, not {q_group}")
        grouped = q_group == 32
        args = [q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2),
                vc.data_ptr(), vc.stride(0), vc.stride(1), vc.stride(2), kc.shape[0], bs, Hkv, d, out.data_ptr(),
                out.stride(0), out.stride(1), cu_q.data_ptr(), seq_lens.data_ptr(), block_table.data_ptr(),
                block_table.stride(0), num_seqs, Hq, ks.data_ptr(), kcols, vs.data_ptr(), vcols, float(softmax_scale),
                segm_out.data_ptr() if split else None, segm_max.data_ptr() if split else None,
                segm_sum.data_ptr() if split else None, seg_st, seg_sh, S, _target_waves(), int(max_query_len),
                int(qmax)]
        rows = segm_max.shape[0] if split else 0
        if grouped or rows < q.shape[0]:
            # tokens past the buffers' rows are never cut (kvq_int8_decode_attention_ex)
            args.insert(-3, rows)
            _native.call("kvq_int8_decode_attention_ex", *args, 32 if grouped else d, _stream(q))
        else:
            _native.call("kvq_int8_decode_attention", *args, _stream(q))

    # kvq/cuda/int8_kv.cu:650-672
    def dequant_pages(self, kc, vc, ko, vo, block_table, src_req, src_j, ks, vs):
        n, bs, H = src_req.shape[0], kc.shape[1], kc.shape[2]
        _check(kc.stride(3) == 1 and ko.is_contiguous() and vo.is_contiguous() and src_j.shape[0] == n, "layout")
        if n == 0:
            return
        _check_cuda("dequant_pages", kc, vc, ko, vo, block_table, src_req, src_j, ks, vs)
        d = kc.shape[3]
        _check(kc.dtype == torch.int8 and vc.dtype == torch.int8 and vc.shape == kc.shape and vc.stride(3) == 1,
               "dequant_pages: caches must be int8")
        _check(ko.dtype == torch.bfloat16 and vo.dtype == torch.bfloat16 and tuple(ko.shape) == (n, bs, H, d) and
               tuple(vo.shape) == (n, bs, H, d), "dequant_pages: outputs must be bf16 [P, block_size, H, D]")
        for t, nm in ((block_table, "block_table"), (src_req, "src_req"), (src_j, "src_j")):
            _check(t.dtype == torch.int32, f"dequant_pages: {nm} must be int32")
        _check(src_req.is_contiguous() and src_j.is_contiguous() and block_table.stride(-1) == 1,
               "dequant_pages: index tensors must be contiguous")
        kcols = _scale_cols(ks, "dequant_pages k_scale", H, d)
        vcols = _scale_cols(vs, "dequant_pages v_scale", H, d)
        _native.call("kvq_dequant_pages", kc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), vc.data_ptr(),
                     vc.stride(0), vc.stride(1), vc.stride(2), kc.shape[0], bs, H, d, ko.data_ptr(), vo.data_ptr(),
                     block_table.data_ptr(), block_table.stride(0), src_req.data_ptr(), src_j.data_ptr(), n,
                     ks.data_ptr(), kcols, vs.data_ptr(), vcols, _stream(kc))

    # consumer of the temporary cache: in place of flash_attn_varlen_func (kvq/cuda_kernels.py:128-130)
    def paged_prefill_attention(self, q, kt, vt, out, cu_q, seq_lens, block_table, tile_req, tile_row, softmax_scale):
        n = tile_req.shape[0]
        if n == 0:
            return
        _check_cuda("paged_prefill_attention", q, kt, vt, out, cu_q, seq_lens, block_table, tile_req, tile_row)
        _check(q.dtype == torch.bfloat16 and kt.dtype == torch.bfloat16 and vt.dtype == torch.bfloat16 and
               out.dtype == torch.bfloat16, "paged_prefill_attention: q, caches and out must be bf16")
        _check(kt.dim() == 4 and vt.shape == kt.shape and kt.stride(3) == 1 and vt.stride(3) == 1 and q.stride(2) == 1
               and out.stride(2) == 1 and out.shape[1:] == q.shape[1:] and q.shape[2] == kt.shape[3],
               "paged_prefill_attention: unsupported shape/layout")
        for t, nm in ((cu_q, "cu_seqlens_q"), (seq_lens, "seq_lens"), (block_table, "block_table"),
                      (tile_req, "tile_req"), (tile_row, "tile_row")):
            _check(t.dtype == torch.int32, f"paged_prefill_attention: {nm} must be int32")
        _check(block_table.stride(-1) == 1 and tile_row.shape[0] == n, "paged_prefill_attention: index layout")
        P, bs, Hkv, d = kt.shape
        _native.call("kvq_paged_prefill_attention", q.data_ptr(), q.stride(0), q.stride(1), kt.data_ptr(), kt.stride(0),
                     kt.stride(1), kt.stride(2), vt.data_ptr(), vt.stride(0), vt.stride(1), vt.stride(2), P, bs, Hkv, d,
                     out.data_ptr(), out.stride(0), out.stride(1), cu_q.data_ptr(), seq_lens.data_ptr(),
                     block_table.data_ptr(), block_table.stride(0), q.shape[1], tile_req.data_ptr(),
                     tile_row.data_ptr(), n, self.prefill_rows, float(softmax_scale), _stream(q))

    # the same attention read straight from the INT8 pages, in place of dequant_pages + the call above
    # (no counterpart in the reference, which always dequantizes first: kvq/cuda_kernels.py:106-131).
    # fold=False: bit-identical to that pair; True: scales folded into q and the output (faster)
    def int8_prefill_attention(self, q, kc, vc, out, cu_q, seq_lens, block_table, tile_req, tile_row, softmax_scale,
                               ks, vs, fold=False):
        n = tile_req.shape[0]
        if n == 0:
            return
        _check_cuda("int8_prefill_attention", q, kc, vc, out, cu_q, seq_lens, block_table, tile_req, tile_row, ks, vs)
        _check(q.dtype == torch.bfloat16 and out.dtype == torch.bfloat16 and kc.dtype == torch.int8 and
               vc.dtype == torch.int8, "int8_prefill_attention: q and out must be bf16, the caches int8")
        _check(kc.dim() == 4 and vc.shape == kc.shape and kc.stride(3) == 1 and vc.stride(3) == 1 and q.stride(2) == 1
               and out.stride(2) == 1 and out.shape[1:] == q.shape[1:] and q.shape[2] == kc.shape[3],
               "int8_prefill_attention: unsupported shape/layout")
        for t, nm in ((cu_q, "cu_seqlens_q"), (seq_lens, "seq_lens"), (block_table, "block_table"),
                      (tile_req, "tile_req"), (tile_row, "tile_row")):
            _check(t.dtype == torch.int32, f"int8_prefill_attention: {nm} must be int32")
        _check(block_table.stride(-1) == 1 and tile_row.shape[0] == n, "int8_prefill_attention: index layout")
        nb, bs, Hkv, d = kc.shape
        kcols = _scale_cols(ks, "int8_prefill_attention k_scale", Hkv, d)
        vcols = _scale_cols(vs, "int8_prefill_attention v_scale", Hkv, d)
        _native.call("kvq_int8_prefill_attention", q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), kc.stride(0),
                     kc.stride(1), kc.stride(2), vc.data_ptr(), vc.stride(0), vc.stride(1), vc.stride(2), nb, bs, Hkv,
                     d, out.data_ptr(), out.stride(0), out.stride(1), cu_q.data_ptr(), seq_lens.data_ptr(),
                     block_table.data_ptr(), block_table.stride(0), q.shape[1], tile_req.data_ptr(),
                     tile_row.data_ptr(), n, self.prefill_rows, float(softmax_scale), ks.data_ptr(), kcols,
                     vs.data_ptr(), vcols, int(bool(fold)), _stream(q))

    @property
    def prefill_rows(self):
        """(token, q head) rows per work-list entry of the prefill kernel."""
        return int(_native.load().kvq_prefill_rows_per_tile())


def ext():
    """The native library (loaded once). Raises if libkvq_int8.so is missing -- callable eagerly at
    backend init, before any graph capture (reference kvq/cuda_kernels.py:26-39)."""
    global _EXT
    if _EXT is None:
        _EXT = _Ext()
    return _EXT


def quant_reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, static):
    """Quantize the step's new K/V with the static scales and write them through slot_mapping
    (reference kvq/cuda_kernels.py:42-44)."""
    ext().quant_cache(key, value, key_cache, value_cache, slot_mapping, static["k_scale"], static["v_scale"],
                      static["k_mu"])


def quant_q(q, k_scale, group=None):
    """(q_i8 [T, Hq, 128], q_scale [T, Hq, 128 / group]) (reference kvq/cuda_kernels.py:47-48)."""
    return tuple(ext().quant_q(q, k_scale, group or q.shape[-1]))


MIN_SPLIT_KEYS = 128   # the kernels never cut a split shorter than 4 tiles of 32 keys


def choose_splits(max_context):
    """Split buffers' piece count for a caller that sizes them from shapes alone (bench.py, tests): enough
    for the longest possible context (block-table width x block size) to be cut into ranges of 128 keys,
    at most 64. KVQ_SPLITS overrides it (1 = never split). A pure function of host-side shapes, so a
    captured graph and the eager call agree."""
    env = os.environ.get("KVQ_SPLITS")
    if env:
        return max(1, min(MAX_SPLITS, int(env)))
    return int(max(1, min(MAX_SPLITS, -(-max(max_context, 1) // MIN_SPLIT_KEYS))))


def split_buffers(num_tokens, num_q_heads, head_dim, splits, device):
    """(segm_out [T, Hq, S, D], segm_max [T, Hq, S], segm_sum [T, Hq, S]) float32: the split buffers
    decode_attention / paged_attention take as `segm` (what vLLM's Triton metadata holds as
    softmax_segm_output / _max / _expsum)."""
    return (torch.empty(num_tokens, num_q_heads, splits, head_dim, dtype=torch.float32, device=device),
            torch.empty(num_tokens, num_q_heads, splits, dtype=torch.float32, device=device),
            torch.empty(num_tokens, num_q_heads, splits, dtype=torch.float32, device=device))


SPLIT_PIECES = 16        # pieces per (request, kv head) of the vLLM backend's split buffers (as vLLM's own)
EVEN_LENGTHS = 1.05      # a batch whose longest short request is within this factor of the mean is even
ROUND_SLACK = 1.1        # one pass: the busiest CU's whole pairs at most this far above an even share


def one_pass_fill(device):
    """The CUs: a call without split buffers runs one workgroup per CU, each streaming whole (request,
    kv head) pairs in turn."""
    dev = torch.device(device)
    return torch.cuda.get_device_properties(dev).multi_processor_count if dev.type == "cuda" else 256


def split_pays(query_lens, seq_lens, num_kv_heads, fill):
    """Whether split buffers pay for a batch, from host-side lengths (numpy; seq_lens None = unknown): with
    them the kernel cuts the longest (request, kv head) pairs across workgroups and merges the pieces in
    a second launch; without, each pair runs whole in one of `fill` workgroups (one per CU). One pass
    serves as well only when the short-query requests (1..SHORT_Q tokens) give at least `fill` pairs,
    whole pairs spread over the CUs within ROUND_SLACK of evenly (1, 2, 3, 4 pairs per CU, not 1.5 or
    2.5: there the busiest CUs stream a pair more than the rest), and their lengths are within
    EVEN_LENGTHS of even. False when no request has a short query."""
    q = np.asarray(query_lens)
    short = (q >= 1) & (q <= SHORT_Q)
    n = int(short.sum())
    if n == 0:
        return False
    pairs = n * num_kv_heads
    if seq_lens is None or pairs < fill:
        return True
    if -(-pairs // fill) * fill > ROUND_SLACK * pairs:
        return True
    ls = np.asarray(seq_lens)[:len(q)][short].astype(np.int64)
    return int(ls.max()) * n > EVEN_LENGTHS * int(ls.sum())


def _target_waves():
    """Wavefronts the kernel spreads a batch over (KVQ_TARGET_WAVES; 0 = as many as the kernel keeps resident)."""
    return int(os.environ.get("KVQ_TARGET_WAVES", "0"))


def decode_attention(q, k_cache, v_cache, out, cu_seqlens_q, seq_lens, block_table, softmax_scale, static,
                     segm=None, max_query_len=1, q_group=None):
    """INT8 attention for the requests with at most SHORT_Q query tokens (others are skipped).
    max_query_len bounds the short queries' length (reference kvq/cuda_kernels.py:51-58).

    segm = (segm_out [R, Hq, S, D], segm_max [R, Hq, S], segm_sum [R, Hq, S]) allows up to S pieces per
    (request, kv head) (the reference always uses S); the kernel gives each as many of them as its share
    of the batch's work calls for. The reference needs R >= T (its buffers are indexed by token); here a
    request with a token at or past row R is simply never cut, so buffers sized for the short requests
    of a batch that puts them first serve it too. Without segm nothing is cut and nothing is allocated:
    one pass, each (request, kv head) whole in one workgroup (the reference's S = 1,
    kvq/cuda/int8_kv.cu:612-613).

    q_group: None (one q scale per (token, q head), the reference kernel's numerics) or 32 (one per 32
    channels: the B_*_qgroup32 configurations of kvq/int8_ref.py:120-129, an addition to the reference's
    operator API)."""
    so, sm, ss = segm if segm is not None else (None, None, None)
    ext().int8_decode_attention(q, k_cache, v_cache, out, cu_seqlens_q, seq_lens, block_table, static["k_scale"],
                                static["v_scale"], softmax_scale, so, sm, ss, max_query_len, SHORT_Q, q_group)
    return out


@dataclass
class LongPlan:
    """Temporary bf16 paged cache for the long-query requests of one step (reference
    kvq/cuda_kernels.py:61-77). Built on the host; the GPU copies are made on first use."""
    src_req: np.ndarray         # [P] request of temporary page p
    src_j: np.ndarray           # [P] page index of temporary page p inside that request
    block_table: np.ndarray     # [num_reqs, max_pages] into the temporary cache (rows of short requests unused)
    max_seqlen_k: int           # from the host-side upper bound
    has_short: bool             # any request left for the INT8 kernel
    block_size: int             # page size of both caches
    long_req: np.ndarray = None  # [R] the long requests, their query lengths and host key-count bounds
    long_qlen: np.ndarray = None
    long_seq: np.ndarray = None
    _gpu: tuple = None
    _tiles: dict = None

    def gpu(self, device):
        if self._gpu is None:
            self._gpu = tuple(torch.from_numpy(a).to(device) for a in (self.src_req, self.src_j, self.block_table))
        return self._gpu

    def tiles(self, group, device, rows=None):
        """Work list of the prefill kernel for `group` q heads per kv head: (request, first row) of
        every `rows` (token, q head) rows of the long requests, the ones with the most keys to read
        first (they finish last). Built on the host, copied once per plan and group."""
        if rows is None:
            rows = ext().prefill_rows
        if self._tiles is None:
            self._tiles = {}
        if (group, rows) not in self._tiles:
            req, row, cost = [], [], []
            for r, qn, sl in zip(self.long_req.tolist(), self.long_qlen.tolist(), self.long_seq.tolist()):
                for r0 in range(0, qn * group, rows):
                    t_last = min(qn - 1, (r0 + rows - 1) // group)
                    req.append(r)
                    row.append(r0)
                    cost.append(sl - qn + 1 + t_last)
            order = np.argsort(-np.asarray(cost, dtype=np.int64), kind="stable")
            self._tiles[(group, rows)] = tuple(torch.from_numpy(np.asarray(x, dtype=np.int32)[order]).to(device)
                                               for x in (req, row))
        return self._tiles[(group, rows)]


def plan_long(query_start_loc_cpu, seq_lens_cpu, block_size):
    """Page table of the temporary cache, or None when no request has more than SHORT_Q query
    tokens (reference kvq/cuda_kernels.py:80-103). Host lengths may be upper bounds: they only
    decide how many pages are copied."""
    qsl = np.asarray(query_start_loc_cpu, dtype=np.int64)
    nreq = qsl.shape[0] - 1
    q_lens = qsl[1:] - qsl[:-1]
    is_long = q_lens > SHORT_Q
    if not is_long.any():
        return None
    seq = np.asarray(seq_lens_cpu, dtype=np.int64)[:nreq]
    npages = np.where(is_long, (seq + block_size - 1) // block_size, 0)
    first = np.concatenate([[0], np.cumsum(npages)[:-1]])
    total = int(npages.sum())
    src_req = np.repeat(np.arange(nreq, dtype=np.int64), npages).astype(np.int32)
    src_j = (np.arange(total, dtype=np.int64) - np.repeat(first, npages)).astype(np.int32)
    # a bf16 prefill kernel that walks KV in tiles of up to 256 keys may look up pages past the last
    # key: the table is one such tile wider than the longest request, extra entries -> temporary page 0
    width = int(npages.max()) + (256 + block_size - 1) // block_size
    bt = np.zeros((nreq, width), dtype=np.int32)
    bt[src_req, src_j] = np.arange(total, dtype=np.int32)
    return LongPlan(src_req=src_req, src_j=src_j, block_table=bt, max_seqlen_k=int(seq[is_long].max()),
                    has_short=bool((q_lens[~is_long] > 0).any()), block_size=block_size,
                    long_req=np.nonzero(is_long)[0].astype(np.int32), long_qlen=q_lens[is_long].astype(np.int64),
                    long_seq=seq[is_long].astype(np.int64))


def long_attention(q, k_cache, v_cache, out, cu_seqlens_q, seq_lens, block_table, max_query_len, plan, softmax_scale,
                   static):
    """Dequantize the long requests' pages into a temporary bf16 paged cache (dequant_pages), then bf16
    paged prefill attention over it (reference kvq/cuda_kernels.py:106-131, which calls vLLM's
    FlashAttention with block_table = plan.block_table). Only the long requests' rows are written;
    short requests are left to decode_attention. The key counts are read on the device (seq_lens), the
    plan's host lengths only size the temporary cache and order the work. KVQ_DEBUG_DUMP=path saves the
    prefill call's metadata there first (kvq.debug_dump; the reference's dump, kvq/cuda_kernels.py:123-127).
    KVQ_PREFILL_DIRECT (read at every call): 1 = one kernel reads the INT8 pages itself instead
    (int8_prefill_attention) -- no temporary cache, bit-identical output; fold = the same with the scales
    folded into q and the output (faster, not bit-identical); 0 (default) = the two kernels."""
    bs, h, d = k_cache.shape[1:]
    _check(bs == plan.block_size, f"block size {bs} != plan block size {plan.block_size}")
    tile_req, tile_row = plan.tiles(q.shape[1] // h, q.device)
    kt_shape = (plan.src_req.shape[0], bs, h, d)
    if os.environ.get("KVQ_DEBUG_DUMP"):  # the prefill call's metadata, for an offline replay (kvq.debug_dump)
        from . import debug_dump
        debug_dump.dump_long_call(os.environ["KVQ_DEBUG_DUMP"], q, out, cu_seqlens_q, seq_lens, plan, kt_shape,
                                  tile_req, tile_row, max_query_len, ext().prefill_rows, softmax_scale)
    direct = os.environ.get("KVQ_PREFILL_DIRECT", "0")
    if direct in ("1", "fold"):
        # the INT8 pages read directly: no temporary cache ("1": same output bits; "fold": scales folded)
        ext().int8_prefill_attention(q, k_cache, v_cache, out, cu_seqlens_q, seq_lens, block_table, tile_req,
                                     tile_row, softmax_scale, static["k_scale"], static["v_scale"], direct == "fold")
        return out
    _check(direct == "0", f"KVQ_PREFILL_DIRECT must be 0, 1 or fold, got {direct!r}")
    src_req, src_j, bt_tmp = plan.gpu(q.device)
    kt = torch.empty(kt_shape, dtype=q.dtype, device=q.device)
    vt = torch.empty_like(kt)
    ext().dequant_pages(k_cache, v_cache, kt, vt, block_table, src_req, src_j, static["k_scale"], static["v_scale"])
    ext().paged_prefill_attention(q, kt, vt, out, cu_seqlens_q, seq_lens, bt_tmp, tile_req, tile_row, softmax_scale)
    return out


def check_inputs(q, k_cache, cu_seqlens_q, seq_lens, block_table, plan):
    """KVQ_DEBUG=1: host-side bounds checks of one batch before the kernels run (syncs the GPU;
    skipped while a graph is being captured). Same checks and messages as the reference
    (kvq/cuda_kernels.py:134-169)."""
    if q.is_cuda and torch.cuda.is_current_stream_capturing():
        return
    cu, sl, bt = cu_seqlens_q.cpu().long(), seq_lens.cpu().long(), block_table.cpu().long()
    nb, bs = k_cache.shape[:2]
    n = cu.numel() - 1
    q_lens = cu[1:] - cu[:-1]
    errs = []
    if int(cu[-1]) > q.shape[0]:
        errs.append(f"cu_seqlens_q[-1] {int(cu[-1])} > {q.shape[0]} query rows")
    if sl.numel() < n or bt.shape[0] < n:
        errs.append(f"seq_lens {sl.numel()} / block_table {tuple(bt.shape)} rows < {n} requests")
    else:
        for r in torch.nonzero(q_lens > 0).flatten().tolist():
            L, ql = int(sl[r]), int(q_lens[r])
            pages = -(-L // bs)
            if L < ql:
                errs.append(f"req {r}: seq_len {L} < q_len {ql}")
            if pages > bt.shape[1]:
                errs.append(f"req {r}: {pages} pages > block_table width {bt.shape[1]}")
            elif pages and (int(bt[r, :pages].min()) < 0 or int(bt[r, :pages].max()) >= nb):
                errs.append(f"req {r} (q_len {ql}, seq_len {L}): page ids {bt[r, :pages].tolist()[:8]}... "
                            f"outside [0, {nb})")
    if plan is not None and sl.numel() >= n and bt.shape[0] >= n:
        src_req, src_j = torch.from_numpy(plan.src_req).long(), torch.from_numpy(plan.src_j).long()
        if src_j.numel() and int(src_j.max()) >= bt.shape[1]:
            errs.append("pages to dequantize outside the block table")
        else:
            sp = bt[src_req, src_j]
            if sp.numel() and (int(sp.min()) < 0 or int(sp.max()) >= nb):
                errs.append(f"pages to dequantize outside [0, {nb})")
        copied = torch.bincount(src_req, minlength=n)[:n]
        short_cover = torch.nonzero((q_lens > SHORT_Q) & (copied * bs < sl[:n])).flatten().tolist()
        if short_cover:
            r = short_cover[0]
            errs.append(f"{len(short_cover)} long requests with fewer copied pages than keys, e.g. req {r}: "
                        f"{int(copied[r])} pages for {int(sl[r])} keys")
    if errs:
        raise RuntimeError("kvq input check: " + "; ".join(errs[:8]))


def paged_attention(q, k_cache, v_cache, out, cu_seqlens_q, seq_lens, block_table, max_query_len, softmax_scale,
                    static, plan=None, segm=None, q_group=None):
    """Both paths for one batch, as the backend runs them (plan from plan_long, None if all short)
    (reference kvq/cuda_kernels.py:172-183). q_group as decode_attention's (the INT8 rows only)."""
    if os.environ.get("KVQ_DEBUG") == "1":
        check_inputs(q, k_cache, cu_seqlens_q, seq_lens, block_table, plan)
    if plan is not None:
        long_attention(q, k_cache, v_cache, out, cu_seqlens_q, seq_lens, block_table, max_query_len, plan,
                       softmax_scale, static)
    if plan is None or plan.has_short:
        decode_attention(q, k_cache, v_cache, out, cu_seqlens_q, seq_lens, block_table, softmax_scale, static,
                         segm, max_query_len, q_group)
    return out
