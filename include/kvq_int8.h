/* C ABI of the MI355X (gfx950) static INT8 KV-cache kernels.
 *
 * Every entry point takes plain device pointers, element strides (int64) and a hipStream_t passed
 * as void*. Nothing here allocates device memory or synchronises the host: each call validates its
 * arguments, enqueues its kernels on `stream` and returns 0, or returns a nonzero KVQ_ERR_* code
 * without launching anything; kvq_last_error() then describes the failure (thread-local string).
 *
 * Layout conventions (all strides in elements of the pointed-to type):
 *   key/value      bf16  [T, H, D]       strides (st, sh, 1)
 *   k/v cache      int8  [nb, bs, H, D]  strides (sb, sn, sh, 1) -- vLLM's interleaved
 *                                         [nb, H, bs, 2D] view or separate caches alike
 *   q / out        bf16  [T, Hq, D]      strides (st, sh, 1)
 *   slot_mapping   int64 [n], -1 = padding (skipped)
 *   cu_seqlens_q   int32 [B + 1], seq_lens int32 [B], block_table int32 [B, W] (row stride)
 *   k/v scales     fp32  [Hkv, D] (per channel) or [Hkv, 1] (per head), contiguous; k_mu fp32 [Hkv, D]
 * head_dim D is 64 or 128; block_size a power of two >= 16. Base pointers of bf16 / int8 rows must be
 * 16-byte aligned and their row strides multiples of 16 bytes (vLLM's views satisfy this).
 * Page ids read from a block table outside [0, num_blocks) are replaced by page 0 inside the kernels,
 * so a malformed table yields garbage rows rather than a memory fault (the reference leaves this
 * undefined; its KVQ_DEBUG host check, mirrored in kvq/cuda_kernels.py, reports such tables).
 */
#ifndef KVQ_INT8_H
#define KVQ_INT8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  KVQ_OK = 0,
  KVQ_ERR_ARG = 1,     /* shape / layout / value rejected before launch */
  KVQ_ERR_LAUNCH = 2,  /* the HIP runtime reported an error for the launch */
};

/* Fused quantize + reshape_and_cache.
 * Replaces the pybind op quant_cache (reference kvq/cuda/int8_kv.cu:554-575, kernel :55-84), bound
 * as kvq/cuda_kernels.py:42-44 quant_reshape_and_cache.
 *   kc[slot / bs, slot % bs, h, d] = sat127(rint(fl((f32(key[t,h,d]) - k_mu[h,d]) / k_scale)))
 *   vc[...]                        = sat127(rint(fl(f32(value[t,h,d]) / v_scale)))
 * for t < n_tokens whose slot is in [0, num_blocks * block_size); other slots are skipped.
 * k_scale_cols / v_scale_cols: D (per channel) or 1 (per head). head_dim 64 or 128; rows, strides
 * and the per-channel tables / k_mu 16-byte aligned. Any head count when num_heads * head_dim is a
 * multiple of 512 and the key / value extents and a cache row's head span are below 2 GiB (the
 * wavefront-per-token kernel); otherwise num_heads * head_dim <= 2048. Stream-ordered, allocates
 * nothing. */
int kvq_quant_cache(const void* key, int64_t key_st, int64_t key_sh, const void* value, int64_t val_st,
                    int64_t val_sh, int8_t* k_cache, int64_t kc_sb, int64_t kc_sn, int64_t kc_sh, int8_t* v_cache,
                    int64_t vc_sb, int64_t vc_sn, int64_t vc_sh, const int64_t* slot_mapping, int64_t n_tokens,
                    int64_t num_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size,
                    const float* k_scale, int64_t k_scale_cols, const float* v_scale, int64_t v_scale_cols,
                    const float* k_mu, void* stream);

/* Standalone q quantization (k scale folded in).
 * Replaces the pybind op quant_q (reference kvq/cuda/int8_kv.cu:577-598, kernel :89-111), bound as
 * kvq/cuda_kernels.py:47-48. x = f32(q[t,h,:]) * k_scale[h / G, :] when k_scale_cols == D (a per-head
 * K scale is not folded); one scale s = max(amax_group / 127, 1e-8) per `group` channels (128 or 32,
 * D = 128); q_i8 = sat127(rint(fl(x / s))). Outputs: q_i8 contiguous [T, Hq, 128], q_scale contiguous
 * [T, Hq, 128 / group]. */
int kvq_quant_q(const void* q, int64_t q_st, int64_t q_sh, int64_t num_tokens, int64_t num_q_heads,
                int64_t head_dim, const float* k_scale, int64_t num_kv_heads, int64_t k_scale_cols,
                int64_t group, int8_t* q_i8, float* q_scale, void* stream);

/* INT8 paged attention for requests with 1 <= q_len <= qmax (decode, spec-decode verification),
 * implementation B of the reference (kvq/int8_ref.py:108-143 with p_tile = 32).
 * Replaces the pybind op int8_decode_attention (reference kvq/cuda/int8_kv.cu:600-648, kernels
 * :168-463 and :472-503), bound as kvq/cuda_kernels.py:51-58 decode_attention.
 * Requests with q_len == 0 or q_len > qmax are skipped (their out rows untouched).
 * Work is split stream-K: the batch is one line of units -- request by request, kv head by kv head,
 * group of up to four 16-row tiles of (token, q head) rows, then 32-key tile -- and each of about
 * target_waves / w workgroups of w <= 4 wavefronts (target_waves 0 = as many wavefronts as the chosen
 * kernel keeps resident on the device) takes an equal contiguous range of it; the wavefronts of a workgroup split a range by row
 * tile and, for short queries, by interleaved key tiles merged in LDS. A (request, kv head, row
 * group) that one workgroup covers whole writes out directly; one that is cut writes fp32 pieces to
 * segm_out [T, Hq, S, D] and segm_max / segm_sum [T, Hq, S] (element (t, h, s) at
 * t * seg_st + h * seg_sh + s, segm_out at that index * D + d), which a second kernel merges.
 * num_splits (<= 64) is S, the most pieces the buffers hold: no segment is cut into more.
 * num_splits == 1 (the reference's single pass without split buffers, int8_kv.cu:612-613): nothing
 * is cut and segm_* may be NULL -- each (request, kv head, row group) runs whole in the workgroup
 * whose range it starts in, its keys split over the workgroup's wavefronts and merged in LDS; one
 * kernel, no second launch. The split buffers are scratch of the call: their contents are internal
 * (segm_sum carries the piece count in its sign), as the reference's. */
int kvq_int8_decode_attention(const void* q, int64_t q_st, int64_t q_sh, const int8_t* k_cache, int64_t k_sb,
                              int64_t k_sn, int64_t k_sh, const int8_t* v_cache, int64_t v_sb, int64_t v_sn,
                              int64_t v_sh, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
                              int64_t head_dim, void* out,
                              int64_t o_st, int64_t o_sh, const int32_t* cu_seqlens_q, const int32_t* seq_lens,
                              const int32_t* block_table, int64_t bt_stride, int64_t num_seqs, int64_t num_q_heads,
                              const float* k_scale, int64_t k_scale_cols, const float* v_scale,
                              int64_t v_scale_cols, double softmax_scale, float* segm_out, float* segm_max,
                              float* segm_sum, int64_t seg_st, int64_t seg_sh, int64_t num_splits,
                              int64_t target_waves, int64_t max_query_len, int64_t qmax, void* stream);

/* kvq_int8_decode_attention with two additions to the reference's operator, bound by
 * kvq/cuda_kernels.py decode_attention / paged_attention (q_group=, and split buffers of fewer rows):
 *  - q_group: head_dim is kvq_int8_decode_attention's one q scale per (token, q head); 32 quantizes q
 *    with one scale per 32 channels and sums the groups' scaled integer dots in fp32 -- the reference's
 *    numerics configurations B_channel_qgroup32 / B_channel_smooth_qgroup32 (q_gran "group32",
 *    kvq/int8_ref.py:120-129), which its CUDA kernel does not implement (kvq/vllm_int8/backend.py:125-128
 *    rejects them).
 *  - segm_rows: the split buffers' token rows. The reference indexes them by token and so needs a row
 *    for every token of q (int8_kv.cu:612-620); here a request whose tokens do not all lie in
 *    [0, segm_rows) is never cut (it runs whole, written directly), so a caller may pass buffers sized
 *    for its short requests only -- e.g. for a batch that puts them first -- and still have the longest
 *    of those cut across workgroups. segm_rows >= T is kvq_int8_decode_attention.
 * Other arguments and results as kvq_int8_decode_attention. */
int kvq_int8_decode_attention_ex(const void* q, int64_t q_st, int64_t q_sh, const int8_t* k_cache, int64_t k_sb,
                                 int64_t k_sn, int64_t k_sh, const int8_t* v_cache, int64_t v_sb, int64_t v_sn,
                                 int64_t v_sh, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
                                 int64_t head_dim, void* out, int64_t o_st, int64_t o_sh, const int32_t* cu_seqlens_q,
                                 const int32_t* seq_lens, const int32_t* block_table, int64_t bt_stride,
                                 int64_t num_seqs, int64_t num_q_heads, const float* k_scale, int64_t k_scale_cols,
                                 const float* v_scale, int64_t v_scale_cols, double softmax_scale, float* segm_out,
                                 float* segm_max, float* segm_sum, int64_t seg_st, int64_t seg_sh, int64_t num_splits,
                                 int64_t segm_rows, int64_t target_waves, int64_t max_query_len, int64_t qmax,
                                 int64_t q_group, void* stream);

/* kvq_int8_decode_attention without split buffers from the caller and without any allocation: no
 * counterpart in the reference. For callers that cannot allocate device memory around the call (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments and
 * results as kvq_int8_decode_attention with num_splits pieces, except that the split partials live in
 * a device array of the library (kvq_noalloc_scratch_bytes() bytes, 64 MiB, per GPU, held until the
 * process ends) instead of segm_out / segm_max / segm_sum; num_tokens (rows of q / out) sizes them.
 * Rejected (KVQ_ERR_ARG) when num_tokens * num_q_heads * num_splits * (head_dim + 2) * 4 bytes exceed
 * that array; num_splits == 1 uses none of it. Calls on one GPU share the array: calls that overlap
 * on one GPU (concurrent streams or threads) race and must be serialised by the caller. */
int kvq_int8_decode_attention_noalloc(const void* q, int64_t q_st, int64_t q_sh, int64_t num_tokens,
                                      const int8_t* k_cache, int64_t k_sb, int64_t k_sn, int64_t k_sh,
                                      const int8_t* v_cache, int64_t v_sb, int64_t v_sn, int64_t v_sh,
                                      int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
                                      void* out, int64_t o_st, int64_t o_sh, const int32_t* cu_seqlens_q,
                                      const int32_t* seq_lens, const int32_t* block_table, int64_t bt_stride,
                                      int64_t num_seqs, int64_t num_q_heads, const float* k_scale,
                                      int64_t k_scale_cols, const float* v_scale, int64_t v_scale_cols,
                                      double softmax_scale, int64_t num_splits, int64_t target_waves,
                                      int64_t max_query_len, int64_t qmax, void* stream);

/* Size in bytes of the device array kvq_int8_decode_attention_noalloc keeps its split partials in. */
int kvq_noalloc_scratch_bytes(void);

/* Dequantize pages of the INT8 cache into a contiguous bf16 cache [P, bs, H, D] (long-query path).
 * Replaces the pybind op dequant_pages (reference kvq/cuda/int8_kv.cu:650-672, kernel :505-542),
 * called from kvq/cuda_kernels.py:120-122. Output page p is page src_j[p] of request src_req[p]:
 * physical page block_table[src_req[p] * bt_stride + src_j[p]]. ko = bf16_rne(f32(k_i8) * k_scale)
 * (K keeps k - mu), vo likewise. */
int kvq_dequant_pages(const int8_t* k_cache, int64_t k_sb, int64_t k_sn, int64_t k_sh, const int8_t* v_cache,
                      int64_t v_sb, int64_t v_sn, int64_t v_sh, int64_t num_blocks, int64_t block_size, int64_t num_heads,
                      int64_t head_dim, void* k_out, void* v_out, const int32_t* block_table, int64_t bt_stride,
                      const int32_t* src_req, const int32_t* src_j, int64_t num_pages, const float* k_scale,
                      int64_t k_scale_cols, const float* v_scale, int64_t v_scale_cols, void* stream);

/* bf16 paged prefill attention over the temporary cache that kvq_dequant_pages fills: the consumer
 * the reference delegates to vLLM's FlashAttention (kvq/cuda_kernels.py:128-130,
 * flash_attn_varlen_func(q, kt, vt, out, cu_seqlens_q, seqused_k, ..., causal=True,
 * block_table=plan.block_table)); no pybind counterpart. For the rows listed by the work list
 * (tile_req[i], tile_row[i]): rows_per_tile (= kvq_prefill_rows_per_tile()) rows (token, q head) =
 * (r / G, r % G) of request tile_req[i] from row tile_row[i] on, every kv head;
 * o = softmax(q k^T * softmax_scale) v over keys
 * j <= seq_lens[req] - q_len + t (bottom-right causal), fp32 softmax and accumulation, P rounded to
 * bf16 for the PV product. Caches: bf16 [num_blocks, block_size, H, D] views, element strides; key j
 * of request r is slot j % block_size of page block_table[r * bt_stride + j / block_size].
 * Rows not in the work list are not written. */
int kvq_paged_prefill_attention(const void* q, int64_t q_st, int64_t q_sh, const void* k_cache, int64_t k_sb,
                                int64_t k_sn, int64_t k_sh, const void* v_cache, int64_t v_sb, int64_t v_sn,
                                int64_t v_sh, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
                                int64_t head_dim, void* out, int64_t o_st, int64_t o_sh,
                                const int32_t* cu_seqlens_q, const int32_t* seq_lens, const int32_t* block_table,
                                int64_t bt_stride, int64_t num_q_heads, const int32_t* tile_req,
                                const int32_t* tile_row, int64_t num_tiles, int64_t rows_per_tile,
                                double softmax_scale, void* stream);

/* The same attention read straight from the INT8 pages, in place of kvq_dequant_pages followed by
 * kvq_paged_prefill_attention -- no temporary bf16 cache. No counterpart in the reference, which always
 * dequantizes first (kvq/cuda_kernels.py:106-131). Caches: int8 [num_blocks, block_size, H, D] views
 * with byte strides (multiples of 16) and block_table the requests' own pages, as
 * kvq_int8_decode_attention takes them; k_scale / v_scale as kvq_dequant_pages takes them
 * (k_scale_cols 1 or head_dim). Work list and rows as kvq_paged_prefill_attention. fold_scales 0: K and
 * V converted as kvq_dequant_pages converts them, output bit-identical to that pair's; 1: the codes
 * converted exactly, k_scale folded into q (bf16(q x k_scale)) and v_scale applied to the fp32 output
 * (faster; not bit-identical). */
int kvq_int8_prefill_attention(const void* q, int64_t q_st, int64_t q_sh, const int8_t* k_cache, int64_t k_sb,
                               int64_t k_sn, int64_t k_sh, const int8_t* v_cache, int64_t v_sb, int64_t v_sn,
                               int64_t v_sh, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
                               int64_t head_dim, void* out, int64_t o_st, int64_t o_sh,
                               const int32_t* cu_seqlens_q, const int32_t* seq_lens, const int32_t* block_table,
                               int64_t bt_stride, int64_t num_q_heads, const int32_t* tile_req,
                               const int32_t* tile_row, int64_t num_tiles, int64_t rows_per_tile,
                               double softmax_scale, const float* k_scale, int64_t k_scale_cols,
                               const float* v_scale, int64_t v_scale_cols, int64_t fold_scales, void* stream);

/* Rows per work-list entry of kvq_paged_prefill_attention. No counterpart in the reference. */
int kvq_prefill_rows_per_tile(void);

/* Instrumentation, no counterpart in the reference: when set (non-NULL hipEvent_t handles), the next
 * kvq_int8_decode_attention call on this thread records `start` on its stream right before the
 * attention kernel and `stop` right after it (before the split merge), then forgets the pair. Lets a
 * benchmark time the attention kernel alone with events. Returns 0. */
int kvq_set_attention_events(void* start, void* stop);

/* Instrumentation, no counterpart in the reference: reads `bytes` bytes at `data` (16-byte aligned, a
 * multiple of 16) once with `workgroups` workgroups of 256 lanes (each streaming a contiguous share,
 * non-temporal loads) and writes each lane's XOR of the 32-bit words it read to out[workgroups * 256]. Timing it gives the
 * streaming-read rate HBM sustains on the device, the ceiling bench.py reports beside the attention
 * kernel. Stream-ordered, allocates nothing. */
int kvq_stream_read(const void* data, int64_t bytes, uint32_t* out, int64_t workgroups, void* stream);

/* Dense-bf16 MFMA probe, no counterpart in the reference: `workgroups` x 4 wavefronts each run 8
 * independent chains of 16x16x32 bf16 MFMAs for `iters` rounds (a multiple of 4) on operands from `data`
 * (16 KB of bf16, 16-byte aligned), storing one float per thread in `out` (workgroups x 256). FLOP per
 * launch: workgroups x 4 x iters x 8 x 16,384. bench.py times it for the bf16 rate the box sustains
 * under its power limit, the ceiling beside the prefill kernel's. */
int kvq_mfma_probe(const void* data, int64_t iters, float* out, int64_t workgroups, void* stream);

/* Instrumentation, no counterpart in the reference: reads `read_bytes` at `src` and writes `write_bytes`
 * at `dst` once, in order, with `workgroups` workgroups of 256 lanes (each a contiguous share of both,
 * the two streams interleaved in the fixed ratio of their sizes; non-temporal loads and stores; the
 * written values depend on what was read). The sizes are multiples of 16 bytes in the ratio 2 : 1,
 * 1 : 1 or 1 : 2 (KVQ_ERR_ARG otherwise). Timing it at a kernel's byte mix -- 2 : 1 for
 * kvq_quant_cache, 1 : 2 for kvq_dequant_pages -- gives the cost of a plain stream of those bytes on
 * the device: the floor bench.py reports beside those kernels. Stream-ordered, allocates nothing. */
int kvq_stream_rw(const void* src, int64_t read_bytes, void* dst, int64_t write_bytes, int64_t workgroups,
                  void* stream);

/* Instrumentation, no counterpart in the reference: the memory traffic of kvq_quant_cache without its
 * arithmetic. Reads the key and value rows [T, H, D] bf16 (heads contiguous) of the tokens whose slot is
 * in [0, num_blocks * block_size) and writes one byte per element (the bf16's high byte) to both caches'
 * rows (slot / block_size, slot % block_size, head) -- caches of strides c_sb, c_sn, c_sh bytes (the K
 * and V views of one layout share them). Timed beside kvq_quant_cache it gives the floor of a stream of
 * those bytes scattered by slot. Stream-ordered, allocates nothing. */
int kvq_stream_scatter(const void* key, int64_t key_st, int64_t key_sh, const void* value, int64_t val_st,
                       int64_t val_sh, int8_t* k_cache, int8_t* v_cache, int64_t c_sb, int64_t c_sn, int64_t c_sh,
                       const int64_t* slot_mapping, int64_t n_tokens, int64_t num_heads, int64_t head_dim,
                       int64_t num_blocks, int64_t block_size, void* stream);

/* Text of the last error on this thread ("" if none). */
const char* kvq_last_error(void);

/* ABI version of this library (bumped on any signature change or new entry point). */
int kvq_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* KVQ_INT8_H */
