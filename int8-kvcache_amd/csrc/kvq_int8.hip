// Static INT8 KV-cache kernels for MI355X (gfx950, CDNA4), behind the C ABI of include/kvq_int8.h.
//
//   quant_cache_kernel     fused quantize + reshape_and_cache of one step's new K/V
//   quant_q_kernel         standalone q quantization (per-channel K scale folded in)
//   attn_kernel            INT8 paged attention for short queries (implementation B, p_tile 32) on
//                          int8 MFMA; optional split of the context + split_reduce_kernel
//   dequant_pages_kernel   int8 pages -> contiguous bf16 pages for the long-query (prefill) path
//
// Numerics follow the reference's implementation B (kvq/int8_ref.py:108-143, CUDA contract
// kvq/cuda/int8_kv.cu:11-15):
//   q' = q * s_k[kvh, :]; q_i8 = rint(q' / s_q), one s_q per (token, q head)
//   s  = (q_i8 . k_i8) * s_q * softmax_scale * log2(e)                 (int32 accumulation)
//   P  = exp2(s - m) quantized per (row, 32-key tile aligned at key 0): p_i8 = rint(P / (max P / 127))
//   o  = sum_tiles (p_i8 . v_i8) * ps_tile / sum_tiles(sum p_i8 * ps_tile) * s_v[d]
//
// MFMA mapping of the attention (one wavefront = one (request, kv head, split, row group)):
//   QK  S^T[key][row]  = K[key][:] . Q^T[:][row]   v_mfma_i32_16x16x64_i8, A = K (16 keys), B = q rows
//   PV  O^T[chan][row] = V^T[chan][key] . P^T[key][row]   v_mfma_i32_16x16x32_i8 (K = one 32-key tile)
// The QK accumulator leaves lane (row n = lane % 16, group g = lane / 16) holding keys 16b + 4g + i
// (b = 0, 1; i = 0..3) of the tile: exactly the 8 key slots that lane supplies to the PV B operand,
// so P never moves between lanes. V^T rows are re-assembled in registers (8x8 byte transpose with
// v_perm_b32) from 8-byte row loads. With channel tile t and row m of V^T standing for channel
// (D/16) * m + t, every lane ends with D/4 consecutive output channels of its row.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <type_traits>

#include "../../include/kvq_int8.h"

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int WAVE = 64;
constexpr int TILE = 32;          // keys per attention tile = P quantization tile
constexpr int MAX_SPLITS = 64;    // split_reduce_kernel keeps one split per lane
constexpr int MAX_ROW_TILES = 4;  // row tiles (wavefronts) per attention workgroup
constexpr int MIN_SPLIT_TILES = 4;  // shortest split: 4 tiles = 128 keys
constexpr int DEFAULT_WAVES_PER_CU = 8;
constexpr int DEFAULT_KSPLIT = 2;     // key splits per row tile: skewed batches (c4) run 9% faster
                                      // than with 4 (2-wavefront workgroups, twice as many); c2 the same
constexpr int DEFAULT_LDS_PREFETCH = 3;   // shared LDS ring slots (3, 4 and 6 time the same on c3)
constexpr int DEFAULT_SEG_COST = 8;   // a segment's fixed cost, in tile units: skewed batches (c4's
                                      // lengths; 10 x 32k + 86 x 1 keys) time best at 6-16
constexpr int DEFAULT_SEG_COST_LDS_RING = 12;  // the same for the LDS-ring kernel (4 row tiles filling
                                               // one ring): verification batches time best at 12
// register ring of the decode kernel: tiles in flight per wavefront (PF - 1 ahead of the one computed).
// Under full load HBM latency grows with the bytes in flight (~5 us at 2 tiles ahead per wavefront), and
// every piece of a segment pays it twice at its start (page ids, then K/V): one tile ahead streams as
// fast and starts pieces sooner (same-box A/B: c4 decode rows 128.2 -> 124.9 us, c2 645 -> 643 us).
constexpr int DEFAULT_PREFETCH = 2;
constexpr int DEFAULT_V32_RING = 2;     // verify_kernel's ring slots (3 with one key split)
constexpr int DEFAULT_V32_KSPLIT = 2;   // verify_kernel's key splits per workgroup
constexpr int DEFAULT_SEG_COST_V32_KS2 = 14;  // fixed cost of a segment in verify_kernel with 2 key splits
constexpr int NUM_XCDS = 8;

// ------------------------------------------------------------------------------------------------
// Scalar helpers
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even (NaN -> canonical quiet NaN).
__device__ __forceinline__ uint32_t bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) { return bf16_rne(a) | (bf16_rne(b) << 16); }

__device__ __forceinline__ float sat127(float n) { return __builtin_fminf(__builtin_fmaxf(n, -127.f), 127.f); }

// Four integral floats in [-127, 127] -> four int8 bytes (little endian).
__device__ __forceinline__ uint32_t pack_i8x4(float a, float b, float c, float d) {
  const uint32_t u = (uint32_t)(int)a & 0xffu, v = (uint32_t)(int)b & 0xffu;
  const uint32_t w = (uint32_t)(int)c & 0xffu, x = (uint32_t)(int)d & 0xffu;
  return u | (v << 8) | (w << 16) | (x << 24);
}

// Code of x / s: rint of the correctly rounded fp32 quotient, saturated to [-127, 127]
// (kvq/quant.py:50-51), by IEEE division.
__device__ __forceinline__ float code_exact(float x, float s) { return sat127(__builtin_rintf(x / s)); }

// x / 127, correctly rounded, for every float x in [2^-126, 1] (the range of a P tile maximum):
// q = fl(x * fl(1/127)), the remainder x - 127 q is exact in one FMA, and one more FMA corrects q.
// Checked against IEEE division for all 2^30 floats of that range on the host (tests/test_arith.py).
// Below 2^-126 the caller clamps the result to 1e-30 anyway.
__device__ __forceinline__ float div127(float x) {
  constexpr float R = 1.f / 127.f;
  const float q = x * R;
  return __builtin_fmaf(__builtin_fmaf(-q, 127.f, x), R, q);
}

// Reductions over the lanes l, l ^ 16, l ^ 32, l ^ 48 -- the four lane groups of one row (or one
// column) of the 16x16 MFMA layouts -- with the gfx950 lane-swap instructions: each swap leaves the
// pair {v[l], v[l ^ 32]} (then {v[l], v[l ^ 16]}) in the two results of every lane, no LDS round trip.
__device__ __forceinline__ int group4_max(int v) {
  const auto a = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
  v = max((int)a[0], (int)a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
  return max((int)b[0], (int)b[1]);
}
__device__ __forceinline__ float group4_fmax(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __builtin_fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __builtin_fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float group4_sum(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o; o >>= 1) x = __builtin_fmaxf(x, __shfl_xor(x, o, WAVE));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o; o >>= 1) x += __shfl_xor(x, o, WAVE);
  return x;
}

// ------------------------------------------------------------------------------------------------
// Fused quantize + reshape_and_cache (reference kvq/cuda/int8_kv.cu:55-84).
// Each lane owns 8 channels of one head for the whole launch (their scales' reciprocals and K means in
// registers), so a token's K and V rows are read as contiguous runs (1 KB each for H = 4, D = 128) and
// each (token, head) writes its 128-byte K and V code rows with 16 consecutive lanes -- the 256-byte
// K|V run of a slot in vLLM's interleaved layout. Two kernels: quant_cache_rows_kernel when a token's
// H * D channels fill whole wavefronts (wave-uniform addressing, below), quant_cache_kernel otherwise
// (lanes of a wavefront may hold different tokens). Both walk their tokens with a ring of loads in
// flight.
//
// Codes: code_magic per channel -- the correctly rounded quotient fl(x / s) from the lane's y = fl(1 / s)
// and the scale itself in three operations, rounded to an integer by adding M = 1.5 * 2^23 (ties to
// even), which leaves the code in t's low mantissa bits, so the code byte is read straight out of
// clamp(t, M +- 127). No branch: ties (x / s exactly k + 0.5 -- common with bf16 inputs, e.g. x at
// half a channel's absolute maximum) cost nothing extra.
// ------------------------------------------------------------------------------------------------
constexpr int QC_CPL = 8;     // channels per lane
#ifndef QC_PF
#define QC_PF 5               // quant_cache_kernel: ring of token loads per lane (QC_PF - 1 ahead)
#endif
constexpr int QC_BLOCK = 256;
#ifndef QC_WAVES
#define QC_WAVES 4            // quant_cache_kernel: at least this many waves per SIMD (<= 128 VGPRs)
#endif
constexpr float QC_MAGIC = 12582912.0f;  // 1.5 * 2^23
#ifndef QC_NT_LOAD
#define QC_NT_LOAD 1          // K/V rows are read once: streaming loads
#endif
#ifndef QC_NT_STORE
#define QC_NT_STORE 1         // codes are written once: streaming stores
#endif
template <typename T>
__device__ __forceinline__ T qc_load(const T* p) {
  if constexpr (QC_NT_LOAD) return __builtin_nontemporal_load(p);
  else return *p;
}
template <typename T>
__device__ __forceinline__ void qc_store(T v, T* p) {
  if constexpr (QC_NT_STORE) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// The same code as code_exact, plus QC_MAGIC, without a division: y = fl(1 / s) (IEEE division, once
// per channel), so q = fl(x * y) is within an ulp of x / s, the remainder x - q s is exact in one FMA
// and q + (x - q s) y, rounded once, is fl(x / s) (Markstein's theorem: a correctly rounded quotient
// from a correctly rounded reciprocal); adding QC_MAGIC (1.5 * 2^23, even) then rounds that to an
// integer, ties to even, as rint does. q is first clamped to +-254: a quotient beyond it, infinite
// included, then still comes out beyond +-127 (instead of a NaN remainder) and saturates. Checked
// against code_exact on the host for every finite and infinite bf16 x and fp32 x on and next to the
// ties, over thousands of scales (tests/test_arith.py).
__device__ __forceinline__ float code_magic(float x, float s, float y) {
  const float q = __builtin_fminf(__builtin_fmaxf(x * y, -254.f), 254.f);
  const float qf = __builtin_fmaf(__builtin_fmaf(-q, s, x), y, q);
  return __builtin_fminf(__builtin_fmaxf(qf + QC_MAGIC, QC_MAGIC - 127.f), QC_MAGIC + 127.f);
}

// code bytes (little endian) of 4 values t = fl(c + QC_MAGIC)
__device__ __forceinline__ uint32_t pack_magic4(float t0, float t1, float t2, float t3) {
  const uint32_t lo = __builtin_amdgcn_perm(__float_as_uint(t1), __float_as_uint(t0), 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(__float_as_uint(t3), __float_as_uint(t2), 0x04000c0cu);
  return lo | hi;
}

// the lane's 8 scales: 8 consecutive entries of a per-channel table (16-byte aligned), or the head's
// one scale broadcast (pc is uniform: a scalar branch)
__device__ __forceinline__ void load_scales8(const float* __restrict__ p, int pc, float (&o)[QC_CPL]) {
  if (pc) {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  } else {
    const float v = *p;
#pragma unroll
    for (int e = 0; e < QC_CPL; ++e) o[e] = v;
  }
}

// y: fl(1 / s) of the lane's 8 scales s; get_sc(sc) fetches the scales themselves (at the call, so that
// they hold no registers between tokens)
template <bool SUB_MU, typename GetScales>
__device__ __forceinline__ u32x2 quant8(u32x4 w, const float (&y)[QC_CPL], GetScales get_sc, const float (&mu)[QC_CPL]) {
  float x[QC_CPL], t[QC_CPL];
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[2 * j] = bf16_lo(wd[j]);
    x[2 * j + 1] = bf16_hi(wd[j]);
  }
  if (SUB_MU) {
#pragma unroll
    for (int e = 0; e < QC_CPL; ++e) x[e] = x[e] - mu[e];
  }
  float sc[QC_CPL];
  get_sc(sc);
#pragma unroll
  for (int e = 0; e < QC_CPL; ++e) t[e] = code_magic(x[e], sc[e], y[e]);
  return u32x2{pack_magic4(t[0], t[1], t[2], t[3]), pack_magic4(t[4], t[5], t[6], t[7])};
}

template <int D>
__global__ __launch_bounds__(QC_BLOCK) __attribute__((amdgpu_waves_per_eu(QC_WAVES))) void quant_cache_kernel(
    const uint16_t* __restrict__ key, int64_t key_st, int64_t key_sh, const uint16_t* __restrict__ value,
    int64_t val_st, int64_t val_sh, int8_t* __restrict__ kc, int64_t kc_sb, int64_t kc_sn, int64_t kc_sh,
    int8_t* __restrict__ vc, int64_t vc_sb, int64_t vc_sn, int64_t vc_sh, const int64_t* __restrict__ slots,
    int n, int H, int64_t num_slots, int lbs, const float* __restrict__ ks, int ks_pc,
    const float* __restrict__ vs, int vs_pc, const float* __restrict__ kmu) {
  constexpr int LPH = D / QC_CPL;                 // lanes per head
  const int ipt = H * LPH;                        // lanes per token
  const int tpb = QC_BLOCK / ipt;                 // tokens per block and step
  if ((int)threadIdx.x >= tpb * ipt) return;
  const int item = threadIdx.x % ipt;
  const int h = item / LPH, d0 = (item % LPH) * QC_CPL;
  const int64_t bmask = (int64_t(1) << lbs) - 1;
  const int stride = gridDim.x * tpb;
  const int t_first = blockIdx.x * tpb + threadIdx.x / ipt;
  if (t_first >= n) return;
  const int steps = (n - 1 - t_first) / stride + 1;  // tokens of this lane: t_first + k * stride
  int64_t slot[QC_PF];
  u32x4 kin[QC_PF], vin[QC_PF];
  auto fetch = [&](int j, int k) {  // k clamped: past the end it re-reads the lane's last token
    const int t = t_first + min(k, steps - 1) * stride;
    slot[j] = slots[t];
    kin[j] = qc_load(reinterpret_cast<const u32x4*>(key + t * key_st + h * key_sh + d0));
    vin[j] = qc_load(reinterpret_cast<const u32x4*>(value + t * val_st + h * val_sh + d0));
  };
  // scales first, then the first tokens' rows: all in flight before anything waits
  const float* kp = ks + (ks_pc ? h * D + d0 : h);
  const float* vp = vs + (vs_pc ? h * D + d0 : h);
  float kr[QC_CPL], vr[QC_CPL], mu[QC_CPL];
  load_scales8(kp, ks_pc, kr);
  load_scales8(vp, vs_pc, vr);
  load_scales8(kmu + h * D + d0, 1, mu);
  auto emit = [&](int j) {
    const int64_t sl = slot[j];
    if (sl < 0 || sl >= num_slots) return;   // padding (or out of range): skipped
    const int64_t blk = sl >> lbs, off = sl & bmask;
    qc_store(quant8<true>(kin[j], kr, [&](float (&sc)[QC_CPL]) { load_scales8(kp, ks_pc, sc); }, mu),
                                reinterpret_cast<u32x2*>(kc + blk * kc_sb + off * kc_sn + h * kc_sh + d0));
    qc_store(quant8<false>(vin[j], vr, [&](float (&sc)[QC_CPL]) { load_scales8(vp, vs_pc, sc); }, mu),
                                reinterpret_cast<u32x2*>(vc + blk * vc_sb + off * vc_sn + h * vc_sh + d0));
  };
  if (steps <= QC_PF - 1) {
    // all of the lane's tokens fit in flight at once (a step's worth of new tokens): load exactly
    // those, then write them -- no ring, no re-reads
#pragma unroll
    for (int j = 0; j < QC_PF - 1; ++j)
      if (j < steps) fetch(j, j);
#pragma unroll
    for (int e = 0; e < QC_CPL; ++e) {
      kr[e] = 1.f / kr[e];
      vr[e] = 1.f / vr[e];
    }
#pragma unroll
    for (int j = 0; j < QC_PF - 1; ++j)
      if (j < steps) emit(j);
    return;
  }
#pragma unroll
  for (int j = 0; j < QC_PF - 1; ++j) fetch(j, j);
#pragma unroll
  for (int e = 0; e < QC_CPL; ++e) {
    kr[e] = 1.f / kr[e];
    vr[e] = 1.f / vr[e];
  }
  for (int k0 = 0; k0 < steps; k0 += QC_PF) {
#pragma unroll
    for (int j = 0; j < QC_PF; ++j) {
      const int k = k0 + j;
      if (k >= steps) break;
      fetch((j + QC_PF - 1) % QC_PF, k + QC_PF - 1);
      emit(j);
    }
  }
}

// Wavefront-row variant, for shapes where a token's H * D channels are a whole number of wavefronts
// (H * D % 512 == 0: 8 channels per lane). Each wavefront owns 512 / D heads of a token, so the
// token, its slot and every row base are wave-uniform: the slot is a scalar load, the K/V rows are
// buffer loads (one descriptor per input, the token's byte offset as the scalar offset) and each
// cache row is a buffer store through a descriptor built in scalar registers from the block address
// -- no per-token vector address arithmetic. Same arithmetic per channel (quant8), same codes.
//
// The vector-memory counter (vmcnt) counts loads and stores in issue order, and a wait can only be
// as precise as the compiler's static count of what was issued: so nothing here issues a vector
// memory operation under a branch. A padded slot (or a ring entry past the wavefront's last token)
// still stores, through a descriptor with no records, which the hardware's range check drops; the
// scales come from LDS at each token. The ring's waits then leave QC_ROW_PF - 1 tokens' loads and
// the stores of earlier tokens in flight instead of draining them per token.
#ifndef QC_ROW_BLOCK
#define QC_ROW_BLOCK 256      // threads per workgroup of the wavefront-row kernel
#endif
#ifndef QC_ROW_PF
#define QC_ROW_PF 4           // ring of token loads per wavefront (QC_ROW_PF - 1 in flight ahead)
#endif
#ifndef QC_ROW_WAVES
#define QC_ROW_WAVES 6        // waves per SIMD (<= 80 VGPRs): more wavefronts share the arithmetic left
                              // after the last loads land
#endif
constexpr int QC_RSRC_WORD3 = 0x00020000;          // raw buffer, 32-bit dwords (gfx9 family)
constexpr int QC_LOAD_AUX = QC_NT_LOAD ? 2 : 0;    // 2: nontemporal
constexpr int QC_STORE_AUX = QC_NT_STORE ? 2 : 0;

template <int D>
__global__ __launch_bounds__(QC_ROW_BLOCK) __attribute__((amdgpu_waves_per_eu(QC_ROW_WAVES))) void quant_cache_rows_kernel(
    const uint16_t* __restrict__ key, int key_st, int key_sh, int key_bytes, const uint16_t* __restrict__ value,
    int val_st, int val_sh, int val_bytes, int8_t* __restrict__ kc, int64_t kc_sb, int64_t kc_sn, int kc_sh,
    int8_t* __restrict__ vc, int64_t vc_sb, int64_t vc_sn, int vc_sh, int row_bytes, const int64_t* __restrict__ slots,
    int n, int wpt, int64_t num_slots, int lbs, const float* __restrict__ ks, int ks_pc,
    const float* __restrict__ vs, int vs_pc, const float* __restrict__ kmu) {
  constexpr int LPH = D / QC_CPL;                 // lanes per head
  constexpr int HPW = WAVE / LPH;                 // heads per wavefront
  constexpr int CH = WAVE * QC_CPL;               // channels per wavefront
  constexpr int WPB = QC_ROW_BLOCK / WAVE;
  // a workgroup owns one part (HPW heads) of WPB tokens at a time; the grid is a multiple of wpt
  const int part = blockIdx.x % wpt;
  const int lane = threadIdx.x % WAVE;
  const int t_first = __builtin_amdgcn_readfirstlane((blockIdx.x / wpt) * WPB + threadIdx.x / WAVE);
  const int stride = (gridDim.x / wpt) * WPB;
  const int h = part * HPW + lane / LPH, d0 = (lane % LPH) * QC_CPL;

  // The part's scales, k_mu and the scales' reciprocals (IEEE division), made once per workgroup: every
  // wavefront of the grid reads the same few lines of these tables, so per-wavefront loads would pile
  // onto a few L2 channels, and a wavefront's own divisions would cost as much as its tokens' codes.
  // Each thread requests its table entries first, then its wavefront's first tokens, and builds its
  // entries once they (and only they: the loads return in order) have arrived; a barrier on LDS alone
  // then publishes the table while the tokens are still in flight.
  // k_scale, v_scale, k_mu, 1 / k_scale, 1 / v_scale of channels part * CH + c, each table in two halves:
  // tab[t][0][l] = channels 8 l .. 8 l + 3, tab[t][1][l] = channels 8 l + 4 .. 8 l + 7 -- lane l's two
  // 16-byte reads of a table are then at lane-contiguous addresses (a [t][2 l], [t][2 l + 1] layout puts
  // the lanes 32 bytes apart: 218,480 bank-conflict cycles per c1 call)
  __shared__ float4 tab[5][2][CH / 8];
  constexpr int NTAB = 3 * CH / 4, TPT = (NTAB + QC_ROW_BLOCK - 1) / QC_ROW_BLOCK;
  float tv[TPT][4];
  auto table_loads = [&] {
#pragma unroll
    for (int j = 0; j < TPT; ++j) {  // branch-free: an index past the table re-reads its last entry
      const int i = min((int)threadIdx.x + j * QC_ROW_BLOCK, NTAB - 1);
      // the table a wavefront's entries belong to is uniform (CH / 4 entries per table, a multiple of 64)
      const int t = __builtin_amdgcn_readfirstlane(i / (CH / 4)), ch = part * CH + (i % (CH / 4)) * 4;
      // (two-way selects: a three-way choice among the kernel's pointers became a lookup table in
      // scratch memory)
      const float* sb = t == 0 ? ks : vs;
      const bool spc = (t == 0 ? ks_pc : vs_pc) != 0;   // per head: the head's one scale (4 channels never straddle a head)
      const float* e0 = t == 2 ? kmu + ch : (spc ? sb + ch : sb + ch / D);
      const int step = (t == 2 || spc) ? 1 : 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) tv[j][k] = e0[k * step];
    }
  };
  auto tables = [&] {
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      const int i = (int)threadIdx.x + j * QC_ROW_BLOCK;
      if (i < NTAB) {
        const int t = i / (CH / 4), e = i % (CH / 4);   // entry e: channels 4 e .. 4 e + 3
        tab[t][e & 1][e >> 1] = float4{tv[j][0], tv[j][1], tv[j][2], tv[j][3]};
        if (t < 2)
          tab[3 + t][e & 1][e >> 1] = float4{1.f / tv[j][0], 1.f / tv[j][1], 1.f / tv[j][2], 1.f / tv[j][3]};
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // LDS writes done; token loads stay in flight
  };
  // tokens of this wavefront: tpw consecutive ones from t0, so that each workgroup streams a
  // contiguous run of key / value rows (the interleaved order -- token t_first + k * stride -- timed
  // 0.7% slower on c1). A wavefront past the last token still fetches (token n - 1, discarded) and
  // meets the table's barrier before it leaves.
  const int tpw = (n + stride - 1) / stride;
  const bool live = t_first * tpw < n;
  const int t0 = live ? t_first * tpw : n - 1;
  const int steps = live ? min(tpw, n - t0) : 1;
  const int64_t bmask = (int64_t(1) << lbs) - 1;
  // per-lane byte offsets within a token's rows (all extents < 2^31 bytes: host)
  const int koff = 2 * (h * key_sh + d0), voff = 2 * (h * val_sh + d0);
  const int kcoff = h * kc_sh + d0, vcoff = h * vc_sh + d0;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)key, 0, key_bytes, QC_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)value, 0, val_bytes, QC_RSRC_WORD3);
  int64_t slot[QC_ROW_PF];
  u32x4 kin[QC_ROW_PF], vin[QC_ROW_PF];
  // fetches are issued in ring order (scheduling barriers: the waits count on that order)
  auto fetch = [&](int j, int k) {  // k clamped: past the end it re-reads the wavefront's last token
    const int t = t0 + min(k, steps - 1);
    slot[j] = slots[t];
    __builtin_amdgcn_sched_barrier(0);
    kin[j] = __builtin_amdgcn_raw_buffer_load_b128(rk, koff, 2 * t * key_st, QC_LOAD_AUX);
    vin[j] = __builtin_amdgcn_raw_buffer_load_b128(rv, voff, 2 * t * val_st, QC_LOAD_AUX);
    __builtin_amdgcn_sched_barrier(0);
  };
  static_assert(QC_CPL == 8, "a lane's channels are one entry of each table half");
  auto tab8 = [&](int t, float (&o)[QC_CPL]) {   // this lane's 8 channels: tab[.][0][lane], tab[.][1][lane]
    const float4 a = tab[t][0][lane], b = tab[t][1][lane];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  };
  float kr[QC_CPL], vr[QC_CPL], mu[QC_CPL];
  auto emit = [&](int j, bool real) {
    const int64_t sl = slot[j];
    const bool ok = real && sl >= 0 && sl < num_slots;   // uniform; otherwise the stores are dropped
    const int64_t blk = ok ? sl >> lbs : 0, off = ok ? sl & bmask : 0;
    const int nrec = ok ? row_bytes : 0;
    const __amdgpu_buffer_rsrc_t wk =
        __builtin_amdgcn_make_buffer_rsrc((void*)(kc + blk * kc_sb + off * kc_sn), 0, nrec, QC_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t wv =
        __builtin_amdgcn_make_buffer_rsrc((void*)(vc + blk * vc_sb + off * vc_sn), 0, nrec, QC_RSRC_WORD3);
    __builtin_amdgcn_raw_buffer_store_b64(quant8<true>(kin[j], kr, [&](float (&sc)[QC_CPL]) { tab8(0, sc); }, mu),
                                          wk, kcoff, 0, QC_STORE_AUX);
    __builtin_amdgcn_raw_buffer_store_b64(quant8<false>(vin[j], vr, [&](float (&sc)[QC_CPL]) { tab8(1, sc); }, mu),
                                          wv, vcoff, 0, QC_STORE_AUX);
  };
  auto prepare = [&] {
    tab8(3, kr);
    tab8(4, vr);
    tab8(2, mu);
  };
  if (steps <= QC_ROW_PF - 1) {
    // all of the wavefront's tokens in flight at once (entries past the last re-read it, and drop
    // their stores)
    table_loads();
#pragma unroll
    for (int j = 0; j < QC_ROW_PF - 1; ++j) fetch(j, j);
    tables();
    if (!live) return;
    prepare();
#pragma unroll
    for (int j = 0; j < QC_ROW_PF - 1; ++j) emit(j, j < steps);
    return;
  }
  // (with a ring, the table first: holding its entries across the first fetches spills registers; its
  // latency is shared by more tokens here)
  table_loads();
  tables();
#pragma unroll
  for (int j = 0; j < QC_ROW_PF - 1; ++j) fetch(j, j);
  prepare();
  for (int k0 = 0; k0 < steps; k0 += QC_ROW_PF) {
#pragma unroll
    for (int j = 0; j < QC_ROW_PF; ++j) {
      const int k = k0 + j;
      fetch((j + QC_ROW_PF - 1) % QC_ROW_PF, k + QC_ROW_PF - 1);
      emit(j, k < steps);
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Standalone q quantization (reference kvq/cuda/int8_kv.cu:89-111). Half a wavefront (32 lanes x 4
// channels) per (token, q head) row; GROUP channels share a scale. Exact IEEE division: this op is
// tiny and its codes are compared bit for bit.
// ------------------------------------------------------------------------------------------------
template <int GROUP>
__global__ __launch_bounds__(256) void quant_q_kernel(const uint16_t* __restrict__ q, int64_t q_st, int64_t q_sh,
                                                      int T, int Hq, int G, const float* __restrict__ ks, int ks_pc,
                                                      int8_t* __restrict__ q_i8, float* __restrict__ q_scale) {
  constexpr int D = 128;
  const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
  const int lane = threadIdx.x & 31;
  if (row >= T * Hq) return;  // whole half-wavefronts leave together
  const int t = row / Hq, h = row % Hq, d0 = lane * 4;
  const uint2 raw = *reinterpret_cast<const uint2*>(q + t * q_st + h * q_sh + d0);
  float x[4] = {bf16_lo(raw.x), bf16_hi(raw.x), bf16_lo(raw.y), bf16_hi(raw.y)};
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (ks_pc) x[e] = x[e] * ks[(h / G) * D + d0 + e];
    amax = __builtin_fmaxf(amax, __builtin_fabsf(x[e]));
  }
#pragma unroll
  for (int o = 1; o < GROUP / 4; o <<= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, o, WAVE));
  const float s = __builtin_fmaxf(amax / 127.f, 1e-8f);
  const uint32_t w = pack_i8x4(code_exact(x[0], s), code_exact(x[1], s), code_exact(x[2], s), code_exact(x[3], s));
  *reinterpret_cast<uint32_t*>(q_i8 + (int64_t)row * D + d0) = w;
  if (lane % (GROUP / 4) == 0) q_scale[(int64_t)row * (D / GROUP) + d0 / GROUP] = s;
}

// ------------------------------------------------------------------------------------------------
// INT8 attention for short queries.
// ------------------------------------------------------------------------------------------------
struct AttnArgs {
  // What every workgroup reads first (the worker order and the plan), in the first 64 bytes of the
  // kernel arguments: one scalar-cache line, one memory round trip at launch.
  const int* cu_q;
  const int* seq_lens;
  int num_seqs, hkv, G, qmax;
  int max_splits;     // split buffers hold this many pieces per (token, q head); 1 = no split buffers
  int cut_rows;       // the split buffers' rows: tokens [0, cut_rows); a request with a token beyond is never cut
  int rt;             // row tiles per workgroup: consecutive 16-row tiles of one (request, kv head)
  int workers;        // workgroups of the attention grid
  int min_tiles;      // shortest piece of a cut segment, in 32-key tiles
  int seg_cost;       // work units a segment costs beyond its tiles (its fixed start and finish)
  int xcd_order;      // map workgroups to workers XCD by XCD
  int plan_fast_max;  // the plan's scans run in 32 bits on DPP while every request's units are below this
  const uint16_t* q;
  const int8_t* kc;
  const int8_t* vc;
  uint16_t* out;
  float* segm_out;
  float* segm_max;
  float* segm_sum;
  const int* block_table;
  const float* ks;
  const float* vs;
  int64_t q_st, q_sh, o_st, o_sh, k_sb, k_sn, k_sh, v_sb, v_sn, v_sh, seg_st, seg_sh, bt_stride;
  float sm_log2;      // softmax_scale * log2(e)
  int num_blocks, lbs, ks_pc, vs_pc;
  int ksplit;         // key splits per workgroup: wavefront (t, k) takes every ksplit-th key tile of row tile t
  int waves;          // rt * ksplit wavefronts per workgroup
  int lds_ring;       // 1: the workgroup's wavefronts are row tiles of the same rows (ksplit 1, rt >= 2)
                      // and share each K/V tile through an LDS ring of PF slots (the dynamic LDS)
};
static_assert(offsetof(AttnArgs, q) == 64, "the plan's arguments fill the first 64 bytes");

__device__ __forceinline__ long long uniform64(long long x) {
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)(x & 0xffffffffll));
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)((unsigned long long)x >> 32));
  return (long long)(((unsigned long long)hi << 32) | lo);
}

// What one request asks of the kernel: its 32-key tiles (at least one) and row groups (of `waves`
// 16-row tiles of (token, q head) rows per kv head). Requests with q_len outside [1, qmax] ask nothing.
struct ReqWork {
  int ntiles, rgroups, tok, qlen, len;   // len: the request's key count (seq_lens)
};
__device__ __forceinline__ ReqWork req_work(const AttnArgs& a, int r) {
  ReqWork w{0, 0, 0, 0, 0};
  w.tok = a.cu_q[r];
  w.qlen = a.cu_q[r + 1] - w.tok;
  w.len = a.seq_lens[r];
  if (w.qlen <= 0 || w.qlen > a.qmax) return w;
  w.ntiles = max(1, (w.len + TILE - 1) / TILE);
  const int rt = (w.qlen * a.G + 15) / 16;
  w.rgroups = (rt + a.rt - 1) / a.rt;
  return w;
}
// Whether the request's segments may be cut across workgroups: split buffers exist and hold rows for
// all of its tokens.
__device__ __forceinline__ bool cuttable(const AttnArgs& a, const ReqWork& w) {
  return a.max_splits > 1 && w.tok + w.qlen <= a.cut_rows;
}
// Length, in work units, of each of the request's (kv head, row group) segments: seg_cost units for
// its fixed cost (q load and quantization, the block-table walk's first round trips, the finish and
// output write -- latency a one-tile segment pays as much as a long one), then one unit per tile.
// Without split buffers segments are never cut, but the same lengths still balance the workers.
__device__ __forceinline__ int seg_units(const AttnArgs& a, const ReqWork& w) {
  return w.ntiles ? a.seg_cost + w.ntiles : 0;
}

// The batch as one line of work units: request by request, kv head by kv head, row group by row
// group. Workgroup w takes units [w * chunk, (w + 1) * chunk) (stream-K): every workgroup gets the
// same amount of work -- K/V to stream plus the segments' fixed costs -- however skewed the request
// lengths are. chunk is also long enough that no segment is cut into more than max_splits pieces.
// The merge kernel needs none of it: it reads each segment's piece count from the denominators.
// Segments that may not be cut (no split buffers, or none for the request's tokens) are run whole by the
// workgroup whose range holds their start.
struct Plan {
  long long total, chunk;
};
// a / b for 0 <= a, 0 < b: 32-bit division when both fit (every practical batch; a 64-bit division is a
// long instruction sequence, and the plan and each piece need a few)
__device__ __forceinline__ long long udiv_plan(long long a, long long b) {
  if (((unsigned long long)a | (unsigned long long)b) >> 32 == 0ull) return (long long)((unsigned)a / (unsigned)b);
  return a / b;
}

// Inclusive prefix sum / maximum of x over the wavefront's 64 lanes on DPP: row shifts by 1, 2, 4, 8
// within each 16-lane row, then lane 15's value added into rows 1 and 3 and lane 31's into rows 2
// and 3 -- VALU instructions only, no LDS round trips. max takes x >= 0.
__device__ __forceinline__ int wave_incl_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);   // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);   // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);   // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);   // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}
__device__ __forceinline__ int wave_incl_max(int x) {
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false));
  return x;
}
// Inclusive prefix sum of the lanes' v (>= 0): in 32 bits on DPP when every v < fast_max (at most 2^24:
// 64 of them cannot overflow), otherwise by 64-bit shuffles.
constexpr long long PLAN_FAST_MAX = 1ll << 24;
__device__ __forceinline__ long long wave_incl_sum64(long long v, int lane, long long fast_max) {
  if (__ballot(v >= fast_max) == 0ull) return (long long)wave_incl_sum((int)v);
  long long incl = v;
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) {
    const long long y = __shfl_up(incl, o, WAVE);
    if (lane >= o) incl += y;
  }
  return incl;
}
__device__ __forceinline__ long long lane_value64(long long x, int l) {
  const unsigned lo = __builtin_amdgcn_readlane((unsigned)(x & 0xffffffffll), l);
  const unsigned hi = __builtin_amdgcn_readlane((unsigned)((unsigned long long)x >> 32), l);
  return (long long)(((unsigned long long)hi << 32) | lo);
}

// The plan (total units, chunk) and the request holding unit pos0 = worker * chunk -- its index, the
// unit its segments start at and its work -- in two scans over the requests (their work is read once;
// up to PLAN_CACHE * 64 requests stay in registers). Every workgroup computes the same plan at once
// from the same few lines of cu_seqlens_q / seq_lens, so the scans run on DPP rather than through LDS
// permutes (the plan took ~7 us of a 62 us verification batch with 64-bit shuffle reductions).
constexpr int PLAN_CACHE = 4;
__device__ Plan plan_and_locate(const AttnArgs& a, int worker, int lane, int& r_out, long long& start_out,
                                ReqWork& w_out) {
  long long u[PLAN_CACHE];
  int tk[PLAN_CACHE], ql[PLAN_CACHE], ln[PLAN_CACHE];
  long long tot = 0;
  int nmax = 0;
  for (int c = 0; c * WAVE < a.num_seqs; ++c) {
    const int r = c * WAVE + lane;
    long long v = 0;
    int len = 0;
    ReqWork w{0, 0, 0, 0, 0};
    if (r < a.num_seqs) {
      w = req_work(a, r);
      const int units = seg_units(a, w);
      v = (long long)units * a.hkv * w.rgroups;
      if (cuttable(a, w)) len = units;
    }
    if (c < PLAN_CACHE) {
      u[c] = v; tk[c] = w.tok; ql[c] = w.qlen; ln[c] = w.len;
    }
    tot += lane_value64(wave_incl_sum64(v, lane, a.plan_fast_max), WAVE - 1);
    nmax = max(nmax, __builtin_amdgcn_readlane(wave_incl_max(len), WAVE - 1));
  }
  Plan p;
  p.total = tot;
  long long ch = udiv_plan(p.total + a.workers - 1, a.workers);
  if (nmax > 0) {
    ch = max(ch, (long long)((nmax + a.max_splits - 2) / (a.max_splits - 1)));
    ch = max(ch, (long long)a.min_tiles);
  }
  p.chunk = uniform64(max(ch, 1ll));
  const long long pos = (long long)worker * p.chunk;
  long long base = 0;
  r_out = a.num_seqs;
  start_out = p.total;
  w_out = ReqWork{0, 0, 0, 0, 0};
  for (int c = 0; c * WAVE < a.num_seqs && pos < p.total; ++c) {
    const int r = c * WAVE + lane;
    long long v = 0;
    ReqWork w{0, 0, 0, 0, 0};
    if (c < PLAN_CACHE) {
      v = u[c];
      w.tok = tk[c]; w.qlen = ql[c]; w.len = ln[c];
    } else if (r < a.num_seqs) {
      w = req_work(a, r);
      v = (long long)seg_units(a, w) * a.hkv * w.rgroups;
    }
    const long long incl = wave_incl_sum64(v, lane, a.plan_fast_max);
    const long long ctot = lane_value64(incl, WAVE - 1);
    if (base + ctot > pos) {
      const unsigned long long m = __ballot(base + incl > pos);
      const int idx = __builtin_amdgcn_readfirstlane(__builtin_ctzll(m));
      r_out = c * WAVE + idx;
      start_out = base + lane_value64(incl - v, idx);
      ReqWork f;
      f.tok = __builtin_amdgcn_readlane(w.tok, idx);
      f.qlen = __builtin_amdgcn_readlane(w.qlen, idx);
      f.len = __builtin_amdgcn_readlane(w.len, idx);
      f.ntiles = max(1, (f.len + TILE - 1) / TILE);
      f.rgroups = ((f.qlen * a.G + 15) / 16 + a.rt - 1) / a.rt;
      w_out = f;
      break;
    }
    base += ctot;
  }
  return p;
}

// K/V pages are streamed exactly once per launch: the non-temporal hint keeps them from evicting
// what is reused (block tables, q, scales) from L2 and the last-level cache (measured on c2:
// 771 -> 688 us).
__device__ __forceinline__ i32x4 ldk(const i32x4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ u32x2 ldv(const u32x2* p) { return __builtin_nontemporal_load(p); }

// s_waitcnt that waits until at most n vector-memory operations of this wavefront are outstanding
// (gfx9 encoding: vmcnt in bits 3:0 and 15:14; expcnt 6:4 and lgkmcnt 11:8 left at "no wait")
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// workgroup barrier for the LDS DMA rings below: this wavefront's LDS reads have returned, then
// s_barrier, with a compiler-level memory barrier around it. Each wavefront waits for its own DMAs
// (wait_vm) before it; a __syncthreads, or a release fence on LDS, would also wait for every DMA in
// flight (they write LDS), which the rings keep outstanding on purpose.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// code bytes of q: rint(x / s) saturated (code_magic, one IEEE division for the row's scale); x holds
// the lane's N channels. Codes are packed as they are made, so only x and the packed words are live at
// once.
template <int N>
__device__ __forceinline__ void q_codes(const float (&x)[N], float s, uint32_t (&out)[N / 4]) {
  const float y = 1.f / s;
#pragma unroll
  for (int u = 0; u < N / 4; ++u)
    out[u] = pack_magic4(code_magic(x[4 * u], s, y), code_magic(x[4 * u + 1], s, y), code_magic(x[4 * u + 2], s, y),
                         code_magic(x[4 * u + 3], s, y));
}

template <int D>
struct KVTile {
  i32x4 k[2][D / 64];     // QK A operands: keys 16b + m, bytes = channels (D/4) g + 16 s + j
  uint32_t v[8][D / 64];  // V rows: keys 16 (j / 4) + 4 g + j % 4, channels (D/16) m + 0..D/16-1
};

// 4x4 byte transpose: out[c] byte r = in[r] byte c.
__device__ __forceinline__ void transpose4x4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t& o0,
                                             uint32_t& o1, uint32_t& o2, uint32_t& o3) {
  const uint32_t lo01 = __builtin_amdgcn_perm(a1, a0, 0x05010400u);  // a0.b0 a1.b0 a0.b1 a1.b1
  const uint32_t hi01 = __builtin_amdgcn_perm(a1, a0, 0x07030602u);  // a0.b2 a1.b2 a0.b3 a1.b3
  const uint32_t lo23 = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
  const uint32_t hi23 = __builtin_amdgcn_perm(a3, a2, 0x07030602u);
  o0 = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);  // a0.b0 a1.b0 a2.b0 a3.b0
  o1 = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
  o2 = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
  o3 = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
}

// LDS of the key-split merge: wavefront (t, k >= 1) of a workgroup leaves its 16 rows' running max,
// denominator and accumulators in slot (k - 1) * rt + t, lane-major ([field][lane]: conflict-free).
constexpr int MERGE_FIELDS = 36;  // 32 accumulators (D = 128), max, denominator, 2 spare
constexpr int MERGE_SLOTS = MAX_ROW_TILES - 1;
// Shortest piece split across a workgroup's key splits, in tiles per key split: shorter pieces go
// whole to one key split in turn (no barrier, no merge). c4's decode rows: 2, 3, 4 all 117.8-118.0 us,
// 6 119.0, 8 119.3, 16 121.9 us.
#ifndef KVQ_COOP_TILES
#define KVQ_COOP_TILES 4
#endif
constexpr int COOP_TILES = KVQ_COOP_TILES;
constexpr float ATTN_SLACK = 8.f;  // log2 headroom of the attention's reference maximum

// One wavefront's share of one piece of a segment: its 16-row tile (rows row0..row0+15 of the
// (token, q head) rows of kv head kvh) over the key tiles c_begin + ks, c_begin + ks + KS, ... below
// c_end of request seq. The KS wavefronts of the row tile (ks = 0..KS-1) then merge through LDS, and
// wavefront ks = 0 finishes the piece, the segment's `part`-th of `nparts`: a whole segment writes
// bf16 out, a cut one an fp32 partial. Every wavefront of the workgroup calls this for every piece
// (inactive ones -- row tiles past the request's rows -- only join the barriers of the merge).
template <int D, int PF, bool SHARED>
__device__ __forceinline__ void attend_segment(const AttnArgs& a, int seq, int tok, int qlen, int seqlen, int kvh, int row0,
                                               int c_begin, int c_end, int ks, int KS, int rtile, bool active,
                                               int part, int nparts, float* lds, int lane) {
  constexpr int KPL = D / 4;        // K bytes per lane and key
  constexpr int KSTEPS = D / 64;    // x64 MFMAs per 16-key block
  constexpr int VT = D / 16;        // PV channel tiles = V bytes per lane and key
  constexpr int VW = D / 64;        // V dwords per lane and key
  // every argument is the same across the wavefront; make that explicit so that the block-table and
  // length reads and the loop bounds stay scalar (a vector page-id load would make every tile wait for
  // all K/V loads in flight)
  seq = __builtin_amdgcn_readfirstlane(seq);
  tok = __builtin_amdgcn_readfirstlane(tok);
  qlen = __builtin_amdgcn_readfirstlane(qlen);
  kvh = __builtin_amdgcn_readfirstlane(kvh);
  row0 = __builtin_amdgcn_readfirstlane(row0);
  c_begin = __builtin_amdgcn_readfirstlane(c_begin);
  c_end = __builtin_amdgcn_readfirstlane(c_end);
  part = __builtin_amdgcn_readfirstlane(part);
  nparts = __builtin_amdgcn_readfirstlane(nparts);
  ks = __builtin_amdgcn_readfirstlane(ks);
  KS = __builtin_amdgcn_readfirstlane(KS);
  const int n = lane & 15, g = lane >> 4;
  const int G = a.G;
  const int L = __builtin_amdgcn_readfirstlane(seqlen);
  // no keys (malformed): nothing is read. A wavefront with no rows reads nothing either -- except
  // with a shared LDS ring, where it still fetches its share of every tile and keeps the barriers
  constexpr bool shared = SHARED;  // launched with a.lds_ring set
  const bool work = L > 0 && active;
  if (L <= 0 || (!active && !shared)) c_end = c_begin;
  // this wavefront's tiles: c_begin + ks + j * KS, j < nt
  const int nt = c_begin + ks < c_end ? (c_end - c_begin - ks + KS - 1) / KS : 0;
  auto tile = [&](int j) { return c_begin + ks + j * KS; };
  const int* bt = a.block_table + (int64_t)seq * a.bt_stride;
  const int bs = 1 << a.lbs;

  i32x4 qop[KSTEPS];
  const int R = row0 + n, rtok = R / G, rh = R % G;
  float rs;
  int lim;
  // every row of this wavefront sees at least keys < lim_lo
  const int lim_lo = L - qlen + 1 + row0 / G;

  float m = -1e30f, l = 0.f, acc[VT][4];
#pragma unroll
  for (int t = 0; t < VT; ++t) acc[t][0] = acc[t][1] = acc[t][2] = acc[t][3] = 0.f;

  const int8_t* kbase = a.kc + (int64_t)kvh * a.k_sh;
  const int8_t* vbase = a.vc + (int64_t)kvh * a.v_sh;
  const int koff = n * (int)a.k_sn + g * KPL;            // lane offset of its K bytes inside a 16-key block
  const int voff = 4 * g * (int)a.v_sn + n * VT;         // lane offset of its first V row
  const int vsn = (int)a.v_sn;

  auto page_of = [&](int key) -> int {
    // a scalar load: the block table is read-only during the launch (constant address space), the
    // index is uniform; a vector load here would make each tile wait for every K/V load in flight
    const int idx = __builtin_amdgcn_readfirstlane(key >> a.lbs);
    const int p = __builtin_amdgcn_readfirstlane(((const __attribute__((address_space(4))) int*)bt)[idx]);
    return (p >= 0 && p < a.num_blocks) ? p : 0;
  };
  auto load = [&](KVTile<D>& r, int c) {
    const int n0 = c * TILE, n1 = n0 + 16;
    const int p0 = page_of(n0);
    const int p1 = n1 < L ? page_of(n1) : p0;
    const int o0 = n0 & (bs - 1), o1 = n1 < L ? (n1 & (bs - 1)) : o0;
    const int8_t* kb0 = kbase + (int64_t)p0 * a.k_sb + (int64_t)o0 * a.k_sn;
    const int8_t* kb1 = kbase + (int64_t)p1 * a.k_sb + (int64_t)o1 * a.k_sn;
    const int8_t* vb0 = vbase + (int64_t)p0 * a.v_sb + (int64_t)o0 * a.v_sn;
    const int8_t* vb1 = vbase + (int64_t)p1 * a.v_sb + (int64_t)o1 * a.v_sn;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      r.k[0][s] = ldk(reinterpret_cast<const i32x4*>(kb0 + koff + 16 * s));
      r.k[1][s] = ldk(reinterpret_cast<const i32x4*>(kb1 + koff + 16 * s));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (VW == 2) {
        const u32x2 w0 = ldv(reinterpret_cast<const u32x2*>(vb0 + voff + i * vsn));
        const u32x2 w1 = ldv(reinterpret_cast<const u32x2*>(vb1 + voff + i * vsn));
        r.v[i][0] = w0.x; r.v[i][1] = w0.y;
        r.v[4 + i][0] = w1.x; r.v[4 + i][1] = w1.y;
      } else {
        r.v[i][0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(vb0 + voff + i * vsn));
        r.v[4 + i][0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(vb1 + voff + i * vsn));
      }
    }
  };

  // ---- shared ring: a tile is DMA'd once (global_load_lds_dwordx4, 64 lanes x 16 bytes = RPI rows
  // per instruction; K rows, then V rows, each row's 16-byte chunks XOR-swizzled by row % CHR so
  // that the operand reads below spread over the banks); the rt wavefronts issue instruction
  // rtile + rt u of each tile (u < NIW; past NI an instruction is issued twice -- the same bytes to
  // the same place) ----
  constexpr int RB_ = D;                     // bytes per K (or V) row
  constexpr int CHR = RB_ / 16;              // 16-byte chunks per row
  constexpr int RPI = WAVE / CHR;            // rows per DMA instruction
  constexpr int NI = 2 * TILE / RPI;         // DMA instructions per tile (K rows, then V rows)
  constexpr int SLOT = 2 * TILE * RB_;       // bytes per ring slot
  uint8_t* lring = reinterpret_cast<uint8_t*>(lds);
  // lane part of a DMA source address: row lane / CHR of the instruction's RPI rows, chunk lc. The
  // swizzle row % CHR is (lane / CHR) % CHR whatever the instruction (RPI is a multiple of CHR), so the
  // offsets are the same for every instruction; the rest of the address is uniform (scalar base).
  const uint32_t lrow = lane / CHR, lch = 16 * ((lane % CHR) ^ (lrow % CHR));
  const uint32_t kdo = lrow * (uint32_t)a.k_sn + lch, vdo = lrow * (uint32_t)a.v_sn + lch;
  auto dma = [&](auto niw_t, int c, int st) {
    constexpr int NIW = decltype(niw_t)::value;
    const int n0 = c * TILE, n1 = n0 + 16;
    const int p0 = page_of(n0);
    const int p1 = n1 < L ? page_of(n1) : p0;
    const int o0 = n0 & (bs - 1), o1 = n1 < L ? (n1 & (bs - 1)) : o0;
#pragma unroll
    for (int u = 0; u < NIW; ++u) {
      int i = rtile + a.rt * u;
      if (i >= NI) i -= NI;
      const bool isv = i >= NI / 2;
      const int blk = i % (NI / 2);
      const bool hi = RPI * blk >= 16;  // rows of one instruction sit in one half of the tile
      const int p = hi ? p1 : p0, o = (hi ? o1 - 16 : o0) + RPI * blk;
      const int8_t* sb = isv ? vbase + (int64_t)p * a.v_sb + (int64_t)o * a.v_sn
                             : kbase + (int64_t)p * a.k_sb + (int64_t)o * a.k_sn;
      __builtin_amdgcn_global_load_lds((const void*)(sb + (uint64_t)(isv ? vdo : kdo)),
                                       (__attribute__((address_space(3))) void*)(lring + st * SLOT + (isv ? TILE * RB_ : 0) + 1024 * blk),
                                       16, 0, 0);
    }
  };
  // this lane's operands of slot st: K as load() would put them in registers (row 16 b + n, logical
  // chunk (KPL / 16) g + s), and the V^T operands themselves, read with ds_read_b64_tr_b8: within a
  // 16-lane group, lane 8 h + b receives byte b of the 8-byte chunks addressed by lanes h, h + 2, ...,
  // h + 14 (element j from lane h + 2 j). So lane (g, h, j = (lane % 16) / 2) addresses key row
  // 4 g + j (j < 4) or 16 + 4 g + j - 4 -- the key of P operand slot j of lane group g -- at bytes
  // 16 t + 8 h, and lane (m = 8 h + b, g) receives channel 16 t + m of its 8 keys: channel tile t is
  // channels 16 t .. 16 t + 15 here (the register path interleaves them, see the epilogue).
  // Inline assembly, each statement waiting for its own reads: the compiler would otherwise make the
  // reads wait for every DMA in flight (it cannot tell they read another slot).
  uint32_t ka0[2][KSTEPS], vta0[VT];  // slot 0's read addresses
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int s2 = 0; s2 < KSTEPS; ++s2) {
      const int row = 16 * b + n;
      ka0[b][s2] = (uint32_t)(uintptr_t)lring + row * RB_ + 16 * (((KPL / 16) * g + s2) ^ (row % CHR));
    }
  {
    const int j = (lane & 15) >> 1, h = lane & 1;
    const int row = j < 4 ? 4 * g + j : 16 + 4 * g + j - 4;
#pragma unroll
    for (int t = 0; t < VT; ++t)
      vta0[t] = (uint32_t)(uintptr_t)lring + TILE * RB_ + row * RB_ + 16 * (t ^ (row % CHR)) + 8 * h;
  }
  // st_t: the slot, an int or a std::integral_constant (then its offset is the reads' immediate)
  auto lds_tile = [&](auto st_t, KVTile<D>& r) {
    constexpr bool CT = !std::is_same_v<decltype(st_t), int>;
    uint32_t so;
    if constexpr (CT) so = 0;
    else so = (uint32_t)(st_t * SLOT);
    constexpr int IMM = [] {
      if constexpr (CT) return decltype(st_t)::value * SLOT;
      else return 0;
    }();
    typedef unsigned long long u64;
    u64 w[VT];
    if constexpr (D == 128) {
      asm volatile(
          "ds_read_b128 %0, %12 offset:%c24\n"
          "ds_read_b128 %1, %13 offset:%c24\n"
          "ds_read_b128 %2, %14 offset:%c24\n"
          "ds_read_b128 %3, %15 offset:%c24\n"
          "ds_read_b64_tr_b8 %4, %16 offset:%c24\n"
          "ds_read_b64_tr_b8 %5, %17 offset:%c24\n"
          "ds_read_b64_tr_b8 %6, %18 offset:%c24\n"
          "ds_read_b64_tr_b8 %7, %19 offset:%c24\n"
          "ds_read_b64_tr_b8 %8, %20 offset:%c24\n"
          "ds_read_b64_tr_b8 %9, %21 offset:%c24\n"
          "ds_read_b64_tr_b8 %10, %22 offset:%c24\n"
          "ds_read_b64_tr_b8 %11, %23 offset:%c24\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(r.k[0][0]), "=&v"(r.k[0][1]), "=&v"(r.k[1][0]), "=&v"(r.k[1][1]), "=&v"(w[0]), "=&v"(w[1]),
            "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]), "=&v"(w[6]), "=&v"(w[7])
          : "v"(ka0[0][0] + so), "v"(ka0[0][1] + so), "v"(ka0[1][0] + so), "v"(ka0[1][1] + so), "v"(vta0[0] + so),
            "v"(vta0[1] + so), "v"(vta0[2] + so), "v"(vta0[3] + so), "v"(vta0[4] + so), "v"(vta0[5] + so),
            "v"(vta0[6] + so), "v"(vta0[7] + so), "i"(IMM)
          : "memory");
    } else {
      asm volatile(
          "ds_read_b128 %0, %6 offset:%c12\n"
          "ds_read_b128 %1, %7 offset:%c12\n"
          "ds_read_b64_tr_b8 %2, %8 offset:%c12\n"
          "ds_read_b64_tr_b8 %3, %9 offset:%c12\n"
          "ds_read_b64_tr_b8 %4, %10 offset:%c12\n"
          "ds_read_b64_tr_b8 %5, %11 offset:%c12\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(r.k[0][0]), "=&v"(r.k[1][0]), "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3])
          : "v"(ka0[0][0] + so), "v"(ka0[1][0] + so), "v"(vta0[0] + so), "v"(vta0[1] + so), "v"(vta0[2] + so),
            "v"(vta0[3] + so), "i"(IMM)
          : "memory");
    }
    // the V^T operand of channel tile t, two dwords per tile, in r.v's storage
#pragma unroll
    for (int t = 0; t < VT; ++t) {
      r.v[(2 * t) / VW][(2 * t) % VW] = (uint32_t)w[t];
      r.v[(2 * t + 1) / VW][(2 * t + 1) % VW] = (uint32_t)(w[t] >> 32);
    }
  };
  const int niw = (NI + a.rt - 1) / a.rt;    // DMA instructions per wavefront and tile (uniform)
  auto with_niw = [&](auto f) {             // f(std::integral_constant<int, NIW>)
    if (niw == 1) f(std::integral_constant<int, 1>{});
    else if (niw == 2) f(std::integral_constant<int, 2>{});
    else if (niw == 3) f(std::integral_constant<int, 3>{});
    else f(std::integral_constant<int, 4>{});
  };

  KVTile<D> ring[SHARED ? 1 : PF];  // the register ring (unused with the LDS ring)
  // ---- q prologue, part 1: the q row and its K scales are requested before the first tiles' K/V, so
  // that waiting for them (vmcnt counts in issue order) does not wait for the tiles, and quantizing q
  // overlaps the tiles' flight ----
  const bool qrow = rtok < qlen;
  u32x4 qraw[KPL / 8];
  float ksc[KPL];
  if (qrow) {
    const u32x4* qp = reinterpret_cast<const u32x4*>(a.q + (int64_t)(tok + rtok) * a.q_st +
                                                     (int64_t)(kvh * G + rh) * a.q_sh + g * KPL);
#pragma unroll
    for (int u = 0; u < KPL / 8; ++u) qraw[u] = qp[u];
    if (a.ks_pc) {
      const float4* kp = reinterpret_cast<const float4*>(a.ks + kvh * D + g * KPL);
#pragma unroll
      for (int u = 0; u < KPL / 4; ++u) {
        const float4 f = kp[u];
        ksc[4 * u] = f.x; ksc[4 * u + 1] = f.y; ksc[4 * u + 2] = f.z; ksc[4 * u + 3] = f.w;
      }
    }
  }
  if (nt > 0) {
    if constexpr (SHARED) {
      with_niw([&](auto niw_t) {
#pragma unroll
        for (int j = 0; j < PF - 1; ++j) dma(niw_t, tile(min(j, nt - 1)), j);
      });
    } else {
#pragma unroll
      for (int j = 0; j < PF - 1; ++j) load(ring[j], tile(min(j, nt - 1)));
    }
  }

  // ---- q prologue, part 2: fold s_k, one scale per row, quantize (codes of rint(x / s), the rounding
  // shortcut of q_codes with exact division where a quotient nears a half-integer) ----
  {
    float x[KPL];
    float amax = 0.f;
    if (qrow) {
#pragma unroll
      for (int u = 0; u < KPL / 8; ++u) {
        const u32x4 w = qraw[u];
        x[8 * u + 0] = bf16_lo(w.x); x[8 * u + 1] = bf16_hi(w.x);
        x[8 * u + 2] = bf16_lo(w.y); x[8 * u + 3] = bf16_hi(w.y);
        x[8 * u + 4] = bf16_lo(w.z); x[8 * u + 5] = bf16_hi(w.z);
        x[8 * u + 6] = bf16_lo(w.w); x[8 * u + 7] = bf16_hi(w.w);
      }
      if (a.ks_pc) {
#pragma unroll
        for (int e = 0; e < KPL; ++e) x[e] = x[e] * ksc[e];
      }
#pragma unroll
      for (int e = 0; e < KPL; ++e) amax = __builtin_fmaxf(amax, __builtin_fabsf(x[e]));
    } else {
#pragma unroll
      for (int e = 0; e < KPL; ++e) x[e] = 0.f;
    }
    amax = group4_fmax(amax);
    const float s = __builtin_fmaxf(amax / 127.f, 1e-8f);
    uint32_t codes[KPL / 4];
    q_codes<KPL>(x, s, codes);
#pragma unroll
    for (int st = 0; st < KSTEPS; ++st)
      qop[st] = i32x4{(int)codes[4 * st], (int)codes[4 * st + 1], (int)codes[4 * st + 2], (int)codes[4 * st + 3]};
    rs = s * (a.ks_pc ? 1.f : a.ks[kvh]) * a.sm_log2;
    lim = rtok < qlen ? L - qlen + 1 + rtok : L;  // keys < lim are visible to this row
  }

  // One 32-key tile. MASKED: some key of the tile is at or past some row's limit (the last tiles of
  // a request, causal rows); other tiles skip the per-key limit test.
  auto compute = [&](auto masked_t, const KVTile<D>& r, int c) {
    constexpr bool MASKED = decltype(masked_t)::value;
    const int n0 = c * TILE;
    // ---- QK: S^T[key][row] for the tile's two 16-key blocks ----
    i32x4 sc[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      i32x4 z = {0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) z = __builtin_amdgcn_mfma_i32_16x16x64_i8(r.k[b][s], qop[s], z, 0, 0, 0);
      sc[b] = z;
    }
    // ---- V^T operands: 8x8 byte transpose per channel tile (the LDS ring reads them transposed) ----
    long vop[VT];
    if constexpr (SHARED) {
#pragma unroll
      for (int t = 0; t < VT; ++t)
        vop[t] = (long)(((uint64_t)r.v[(2 * t + 1) / VW][(2 * t + 1) % VW] << 32) | r.v[(2 * t) / VW][(2 * t) % VW]);
    } else if constexpr (VW == 2) {
      static_assert(VT == 8, "head_dim 128: two V dwords per lane and key, 8 channel tiles");
      uint32_t lo[8], hi[8];  // lo[t] = keys j 0..3 of channel tile t, hi[t] = keys j 4..7
      transpose4x4(r.v[0][0], r.v[1][0], r.v[2][0], r.v[3][0], lo[0], lo[1], lo[2], lo[3]);
      transpose4x4(r.v[0][1], r.v[1][1], r.v[2][1], r.v[3][1], lo[4], lo[5], lo[6], lo[7]);
      transpose4x4(r.v[4][0], r.v[5][0], r.v[6][0], r.v[7][0], hi[0], hi[1], hi[2], hi[3]);
      transpose4x4(r.v[4][1], r.v[5][1], r.v[6][1], r.v[7][1], hi[4], hi[5], hi[6], hi[7]);
#pragma unroll
      for (int t = 0; t < VT; ++t) vop[t] = (long)(((uint64_t)hi[t] << 32) | lo[t]);
    } else {
      static_assert(VW == 1 && VT == 4, "head_dim 64: one V dword per lane and key, 4 channel tiles");
      uint32_t lo[4], hi[4];
      transpose4x4(r.v[0][0], r.v[1][0], r.v[2][0], r.v[3][0], lo[0], lo[1], lo[2], lo[3]);
      transpose4x4(r.v[4][0], r.v[5][0], r.v[6][0], r.v[7][0], hi[0], hi[1], hi[2], hi[3]);
#pragma unroll
      for (int t = 0; t < VT; ++t) vop[t] = (long)(((uint64_t)hi[t] << 32) | lo[t]);
    }
    // ---- online softmax; key of accumulator (b, i) = n0 + 16 b + 4 g + i ----
    int mx = INT32_MIN;
    bool ok[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ok[b][i] = MASKED ? n0 + 16 * b + 4 * g + i < lim : true;
        mx = ok[b][i] ? max(mx, sc[b][i]) : mx;
      }
    mx = group4_max(mx);
    // an int8 dot product never reaches INT32_MIN: it marks a row with no visible key in the tile
    const float tmax = (MASKED && mx == INT32_MIN) ? -INFINITY : (float)mx * rs;
    // m is a reference maximum, raised only when a tile's maximum exceeds it by ATTN_SLACK (log2
    // units): P = 2^(s - m) <= 2^ATTN_SLACK, and acc / l are rescaled in few tiles. The P codes are
    // rint(127 P / max P) of the tile, the same for any reference; only ps carries it.
    const bool raise = tmax > m + ATTN_SLACK;
    const float mnew = raise ? tmax : m;
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);
    m = mnew;
    const float pm = __builtin_amdgcn_exp2f(tmax - mnew);  // max of this tile's P (exp2 is monotone)
    const float ps = __builtin_fmaxf(div127(pm), 1e-30f);
    const float ri = __builtin_amdgcn_rcpf(ps);
    // p_i8 = min(rint(P / ps), 127): fl(P * ri + 1.5 * 2^23) rounds to the nearest integer (ties to
    // even) and holds the code in its low byte; masked keys get code 0
    float t[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf((float)sc[b][i], rs, -mnew));
        const float v = __builtin_fminf(__builtin_fmaf(p, ri, QC_MAGIC), QC_MAGIC + 127.f);
        t[b][i] = ok[b][i] ? v : QC_MAGIC;
      }
    const uint32_t p0 = pack_magic4(t[0][0], t[0][1], t[0][2], t[0][3]);
    const uint32_t p1 = pack_magic4(t[1][0], t[1][1], t[1][2], t[1][3]);
    const long pop = (long)(((uint64_t)p1 << 32) | p0);
    // sum of the 8 codes (v_sad_u8: sum of |byte - 0|)
    const float psum = (float)__builtin_amdgcn_sad_u8(p1, 0u, __builtin_amdgcn_sad_u8(p0, 0u, 0u));
    l = __builtin_fmaf(psum, ps, l * alpha);
    if (__any(raise)) {
#pragma unroll
      for (int t = 0; t < VT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] *= alpha;
    }    // ---- PV: O^T[channel][row] += (V^T . P^T) * ps ----
#pragma unroll
    for (int t = 0; t < VT; ++t) {
      i32x4 z = {0, 0, 0, 0};
      z = __builtin_amdgcn_mfma_i32_16x16x32_i8(vop[t], pop, z, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][i] = __builtin_fmaf((float)z[i], ps, acc[t][i]);
    }
  };

  // ---- main loop: a ring of PF register tiles, PF - 1 of them in flight while one is computed.
  // Loads are never skipped (past the end they re-read the last tile, an L2 hit), so every wait
  // in the loop is for exactly the oldest tile. The first PF - 1 tiles were requested before the q
  // prologue. Tiles below full_end have no masked key for any row of the wavefront; the first loop
  // runs whole rounds of them (j < j_full), the second the rest -- both start rounds at j = k * PF,
  // so the ring slot of every tile is a compile-time index. ----
  if constexpr (SHARED) {
   if (nt > 0) {
    // one barrier per tile: this wavefront's DMA of tile j has landed (wait), everyone's has and
    // everyone is done reading tile j - 1 (barrier), so its slot takes tile j + PF - 1
    // tiles j < j_full have no masked key for any row of the wavefront: a loop of its own for them,
    // so that each loop body holds one variant of the tile arithmetic (with both in one body the
    // accumulators leave it in other registers than they entered, and are copied back every tile)
    const int full_end = lim_lo > 0 ? lim_lo / TILE : 0;
    const int j_full = min(nt, full_end > c_begin + ks ? (full_end - c_begin - ks + KS - 1) / KS : 0);
    with_niw([&](auto niw_t) {
      constexpr int NIW = decltype(niw_t)::value;
      KVTile<D> cur;
      // tile j sits in slot st = j % PF and its DMA goes to slot (j + PF - 1) % PF: ints, or
      // compile-time constants in the rounds below (the reads' slot offset is then an immediate)
      auto step = [&](auto masked_t, int j, auto st, auto dst) {
        wait_vm<(PF - 2) * NIW>();
        lds_barrier();
        dma(niw_t, tile(min(j + PF - 1, nt - 1)), (int)dst);
        if (work) {
          lds_tile(st, cur);
          compute(masked_t, cur, tile(j));
        }
      };
      int j = 0;
      // whole rounds of PF unmasked tiles (a round starts at a multiple of PF: slots 0 .. PF - 1)
      for (; j + PF <= j_full; j += PF) {
        auto round_step = [&](auto jj_t) {
          constexpr int JJ = decltype(jj_t)::value;
          if constexpr (JJ < PF)
            step(std::false_type{}, j + JJ, std::integral_constant<int, JJ>{},
                 std::integral_constant<int, (JJ + PF - 1) % PF>{});
        };
        round_step(std::integral_constant<int, 0>{});
        round_step(std::integral_constant<int, 1>{});
        round_step(std::integral_constant<int, 2>{});
        round_step(std::integral_constant<int, 3>{});
        round_step(std::integral_constant<int, 4>{});
        round_step(std::integral_constant<int, 5>{});
        static_assert(PF <= 6, "rounds are written for up to 6 slots");
      }
      for (; j < j_full; ++j) step(std::false_type{}, j, j % PF, (j + PF - 1) % PF);
      for (; j < nt; ++j) step(std::true_type{}, j, j % PF, (j + PF - 1) % PF);
    });
    wait_vm<0>();   // the ring is empty and read before the next piece refills it
    lds_barrier();
   }
  } else if (nt > 0) {
    const int full_end = lim_lo > 0 ? lim_lo / TILE : 0;
    const int j_full = min(nt, full_end > c_begin + ks ? (full_end - c_begin - ks + KS - 1) / KS : 0);
    int j0 = 0;
    for (; j0 + PF <= j_full; j0 += PF) {
#pragma unroll
      for (int jj = 0; jj < PF; ++jj) {
        load(ring[(jj + PF - 1) % PF], tile(min(j0 + jj + PF - 1, nt - 1)));
        compute(std::false_type{}, ring[jj], tile(j0 + jj));
      }
    }
    for (; j0 < nt; j0 += PF) {
#pragma unroll
      for (int jj = 0; jj < PF; ++jj) {
        const int j = j0 + jj;
        if (j >= nt) break;
        load(ring[(jj + PF - 1) % PF], tile(min(j + PF - 1, nt - 1)));
        compute(std::true_type{}, ring[jj], tile(j));
      }
    }
  }

  // ---- epilogue: lane (n, g) holds channels (D/4) g + (D/16) i + t of row n in acc[t][i] (register
  // path), or channels 16 t + 4 g + i (LDS ring path) ----
  l = group4_sum(l);
  if (KS > 1) {
    // key-split merge (the formula of split_reduce_kernel): wavefronts k >= 1 publish (m, l, acc),
    // wavefront 0 folds them in: M = max m_k, w_k = 2^(m_k - M), l = sum w_k l_k, acc = sum w_k acc_k
    static_assert(VT * 4 + 2 <= MERGE_FIELDS, "merge slot too small");
    // slot of wavefront (rtile, k >= 1): (k - 1) * rt + rtile
    auto slot = [&](int k) { return lds + (size_t)((k - 1) * a.rt + rtile) * MERGE_FIELDS * WAVE + lane; };
    if (ks > 0 && active) {
      float* sl = slot(ks);
#pragma unroll
      for (int t = 0; t < VT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) sl[(4 * t + i) * WAVE] = acc[t][i];
      sl[(4 * VT) * WAVE] = m;
      sl[(4 * VT + 1) * WAVE] = l;
    }
    __syncthreads();
    if (ks == 0 && active) {
      float M = m;
      for (int k = 1; k < KS; ++k) M = __builtin_fmaxf(M, slot(k)[(4 * VT) * WAVE]);
      const float w0 = __builtin_amdgcn_exp2f(m - M);
      l *= w0;
#pragma unroll
      for (int t = 0; t < VT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] *= w0;
      for (int k = 1; k < KS; ++k) {
        const float* src = slot(k);
        const float wk = __builtin_amdgcn_exp2f(src[(4 * VT) * WAVE] - M);
        l = __builtin_fmaf(wk, src[(4 * VT + 1) * WAVE], l);
#pragma unroll
        for (int t = 0; t < VT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[t][i] = __builtin_fmaf(wk, src[(4 * t + i) * WAVE], acc[t][i]);
      }
      m = M;
    }
    __syncthreads();  // the slots are rewritten by the next piece
  }
  if (ks > 0 || !active || rtok >= qlen) return;
  constexpr int OPL = D / 4;
  const int head = kvh * G + rh;
  const int qt = tok + rtok;
  if constexpr (SHARED) {
    float vsc[VT][4];
#pragma unroll
    for (int t = 0; t < VT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) vsc[t][i] = a.vs_pc ? a.vs[kvh * D + 16 * t + 4 * g + i] : a.vs[kvh];
    if (nparts == 1) {
      if (a.max_splits > 1 && qt < a.cut_rows && g == 0)
        a.segm_sum[(int64_t)qt * a.seg_st + (int64_t)head * a.seg_sh] = -1.f;
      const float inv = 1.f / __builtin_fmaxf(l, 1e-30f);
      uint16_t* orow = a.out + (int64_t)qt * a.o_st + (int64_t)head * a.o_sh + 4 * g;
#pragma unroll
      for (int t = 0; t < VT; ++t)
        *reinterpret_cast<u32x2*>(orow + 16 * t) =
            u32x2{pack_bf16x2((acc[t][0] * inv) * vsc[t][0], (acc[t][1] * inv) * vsc[t][1]),
                  pack_bf16x2((acc[t][2] * inv) * vsc[t][2], (acc[t][3] * inv) * vsc[t][3])};
    } else {
      const int64_t sidx = (int64_t)qt * a.seg_st + (int64_t)head * a.seg_sh + part;
      if (g == 0) {
        a.segm_max[sidx] = m;
        a.segm_sum[sidx] = part == nparts - 1 ? -2.f - l : l;
      }
      float* sp = a.segm_out + sidx * D + 4 * g;
#pragma unroll
      for (int t = 0; t < VT; ++t)
        *reinterpret_cast<float4*>(sp + 16 * t) =
            float4{acc[t][0] * vsc[t][0], acc[t][1] * vsc[t][1], acc[t][2] * vsc[t][2], acc[t][3] * vsc[t][3]};
    }
    return;
  }
  float vsc[OPL];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < VT; ++t) vsc[VT * i + t] = a.vs_pc ? a.vs[kvh * D + OPL * g + VT * i + t] : a.vs[kvh];
  if (nparts == 1) {
    // a row that is not cut tells the merge kernel so: -1 in its piece-0 denominator slot
    if (a.max_splits > 1 && qt < a.cut_rows && g == 0)
      a.segm_sum[(int64_t)qt * a.seg_st + (int64_t)head * a.seg_sh] = -1.f;
    const float inv = 1.f / __builtin_fmaxf(l, 1e-30f);
    uint32_t o[OPL / 2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int t = 0; t < VT; t += 2)
        o[(VT * i + t) / 2] = pack_bf16x2((acc[t][i] * inv) * vsc[VT * i + t], (acc[t + 1][i] * inv) * vsc[VT * i + t + 1]);
    u32x4* op = reinterpret_cast<u32x4*>(a.out + (int64_t)qt * a.o_st + (int64_t)head * a.o_sh + OPL * g);
#pragma unroll
    for (int u = 0; u < OPL / 8; ++u) op[u] = u32x4{o[4 * u], o[4 * u + 1], o[4 * u + 2], o[4 * u + 3]};
  } else {
    const int64_t sidx = (int64_t)qt * a.seg_st + (int64_t)head * a.seg_sh + part;
    if (g == 0) {
      a.segm_max[sidx] = m;
      a.segm_sum[sidx] = part == nparts - 1 ? -2.f - l : l;  // the last piece is marked (l >= 0)
    }
    float* sp = a.segm_out + sidx * D + OPL * g;
#pragma unroll
    for (int u = 0; u < OPL / 4; ++u) {
      float4 w;
      const int c0 = 4 * u;
      w.x = acc[(c0 + 0) % VT][(c0 + 0) / VT] * vsc[c0 + 0];
      w.y = acc[(c0 + 1) % VT][(c0 + 1) / VT] * vsc[c0 + 1];
      w.z = acc[(c0 + 2) % VT][(c0 + 2) / VT] * vsc[c0 + 2];
      w.w = acc[(c0 + 3) % VT][(c0 + 3) / VT] * vsc[c0 + 3];
      reinterpret_cast<float4*>(sp)[u] = w;
    }
  }
}

// Stream-K attention: workgroup w walks units [w * chunk, (w + 1) * chunk) of the batch (the plan of
// plan_and_locate), segment by segment. Its rt * ks wavefronts split each piece: rt consecutive
// 16-row tiles (they stream the same K/V tiles at the same time -- the second and later reads hit
// L1/L2), each over ks interleaved sets of key tiles merged through LDS at the end of the piece.
// Decode rows (one row tile) use 2 key splits, so a workgroup covers 2x the keys of one wavefront and
// a long request's (kv head) is cut across workgroups half as often. Pieces too short for every key
// split to stream COOP_TILES tiles are not split: the key splits take them in turn, each alone.
template <int D, int PF, bool SHARED = false>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
  // the wavefront index is uniform across the wavefront: keep it (and all row bookkeeping) scalar
  const int lane = threadIdx.x & (WAVE - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int rtile = wave % a.rt, kspl = wave / a.rt;  // row tile and key split of this wavefront
  extern __shared__ float merge_lds[];  // (ksplit - 1) * rt slots, sized at launch (none without key splits)
  // workgroups are dispatched round-robin over the XCDs: give each XCD a contiguous range of workers
  // (so one XCD's L2 sees whole requests' block-table rows and q); KVQ_XCD_ORDER=0 turns it off.
  // XCD x holds the blocks b = x (mod 8), q + (x < rem) of them for W = 8 q + rem, and takes the
  // workers [x q + min(x, rem), ...) -- consecutive ranges that tile [0, W) exactly.
  int worker = blockIdx.x;
  {  // no branch before the plan: its argument loads go out in one batch
    const int q = a.workers / NUM_XCDS, rem = a.workers % NUM_XCDS;
    const int wx = blockIdx.x % NUM_XCDS, wi = blockIdx.x / NUM_XCDS;
    worker = a.xcd_order ? wx * q + min(wx, rem) + wi : worker;
    worker = (int)blockIdx.x < a.workers ? worker : a.workers;   // past the grid's workers: no units
  }
  int r;
  long long rstart;
  ReqWork w;
  const Plan pl = plan_and_locate(a, worker, lane, r, rstart, w);
  long long pos = (long long)worker * pl.chunk;
  const long long end = min(pos + pl.chunk, pl.total);
  if (pos >= end || r >= a.num_seqs) return;
  int seglen = seg_units(a, w);
  int seg = (int)udiv_plan(pos - rstart, seglen), off = (int)(pos - rstart - (long long)seg * seglen);
  bool whole = !cuttable(a, w);
  int solo = 0;  // pieces run by a single wavefront so far (uniform across the workgroup)
  while (pos < end) {
    const long long seg_start = rstart + (long long)seg * seglen;
    const int take = (int)min((long long)(seglen - off), end - pos);
    // the segment's first seg_cost units stand for its fixed cost, the rest for its tiles: pieces are
    // the workers' shares of the tile units (a worker holding only fixed-cost units has no piece, and
    // the pieces are numbered from the worker holding the first tile). Uncut (whole): the worker where
    // the segment starts runs all of it, one piece.
    const int fc = a.seg_cost;
    const long long first = whole ? worker : udiv_plan(seg_start + fc, pl.chunk);
    const long long last = whole ? worker : udiv_plan(seg_start + seglen - 1, pl.chunk);
    const int kvh = seg / w.rgroups, rg = seg % w.rgroups;
    const int row0 = (rg * a.rt + rtile) * 16;
    const int c0 = whole ? 0 : max(off - fc, 0);
    const int c1 = whole ? (off == 0 ? w.ntiles : 0) : max(off + take - fc, 0);
    // a piece long enough for every key split to stream COOP_TILES tiles is split across them and
    // merged; shorter pieces go whole to one key split in turn (no barrier, no merge)
    if (c1 <= c0) {
      // fixed-cost units only: nothing to stream here (uniform across the workgroup)
    } else if (a.ksplit > 1 && c1 - c0 >= a.ksplit * COOP_TILES) {
      attend_segment<D, PF, SHARED>(a, r, w.tok, w.qlen, w.len, kvh, row0, c0, c1, kspl, a.ksplit, rtile, row0 < w.qlen * a.G,
                            (int)(worker - first), (int)(last - first + 1), merge_lds, lane);
    } else {
      if (solo % a.ksplit == kspl)
        attend_segment<D, PF, SHARED>(a, r, w.tok, w.qlen, w.len, kvh, row0, c0, c1, 0, 1, rtile, row0 < w.qlen * a.G,
                              (int)(worker - first), (int)(last - first + 1), merge_lds, lane);
      ++solo;
    }
    pos += take;
    off = 0;
    if (++seg == a.hkv * w.rgroups && pos < end) {  // on to the next request with work
      rstart += (long long)seglen * a.hkv * w.rgroups;
      seg = 0;
      do {
        if (++r >= a.num_seqs) return;
        w = req_work(a, r);
      } while (w.ntiles == 0);
      seglen = seg_units(a, w);
      whole = !cuttable(a, w);
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Verification-shape attention: more than 32 (token, q head) rows per (request, kv head), e.g. 8
// speculative tokens x 7 q heads = 56 rows. A workgroup of 2 x KS wavefronts takes a piece of one
// (request, kv head, group of 64 rows): row wavefront rw owns rows row0 = 32 rw .. 32 rw + 31 of the
// group, key split kw streams the piece's tiles kw, kw + KS, ...; the two row wavefronts of a key split
// share each 32-key K/V tile through the split's LDS ring (wavefront rw DMAs keys 16 rw .. 16 rw + 15 of
// it), and at the end of the piece key split 1 hands its running max, denominator and accumulators to
// key split 0 through LDS. Two key splits halve the pieces a batch is cut into at the same wavefront
// count -- and with them the fixed cost per piece (q prologue, first DMAs, finish) and the fp32 partials
// the merge kernel reads (c3: 68.8 -> 66.1 us).
// Per tile and wavefront, on the 32x32 int8 MFMA (lane l: n = l % 32, h = l / 32):
//   QK  S^T[key][row] = K . Q^T   v_mfma_i32_32x32x32_i8 x D/32, A = K (lane: key n, channel half h of
//       each 32-channel step), B = Q^T (lane: row n, same channels)
//   the accumulator leaves lane (n, h) with row n and keys 8 j + 4 h + i (j, i < 4; register 4 j + i);
//   those 16 P codes, packed in register order, are exactly the lane's B operand of
//   PV  O^T[chan][row] = V^T . P^T   v_mfma_i32_32x32x32_i8 x D/32, A = V^T (lane: channel n of the
//       32-channel tile, the same 16 keys in the same order, read transposed from LDS)
//   which leaves lane (n, h) with row n and channels 32 c + 8 j + 4 h + i.
// Against the 16x16 tiles of attn_kernel a wavefront covers twice the rows per tile, so every per-tile
// cost that is not per (row, key) or (row, channel) -- the row maximum's lane exchange, the tile scale,
// LDS addressing, the DMA issue, the barrier -- is paid once per 32 rows. The arithmetic per element is
// attn_kernel's (implementation B, p_tile 32), so results agree with it to the last bit of each row's
// fp32 sums in the same order.
// LDS rows are 16-byte chunks XOR-swizzled per key row (K: (row / 2) % chunks, V: bits 1 and 3 of the
// row, doubled) so that the K reads (16 rows, one chunk) and the transposing V reads (8 rows x 2
// chunks per 16 lanes) fall on distinct banks.
// ------------------------------------------------------------------------------------------------
constexpr int V32_GROUP_TILES = 4;
// verify_kernel's dynamic LDS: KS rings of PF slots (K then V rows of 32 keys), which the key-split
// merge reuses (2 row wavefronts x (16 D / 32 + 2) fields x 64 lanes of fp32) -- at least as large as
// either -- then the V scales of key split 0's two row wavefronts, then every wavefront's K scales
constexpr int64_t v32_vscale_offset(int64_t d, int64_t pf, int64_t ks) {
  const int64_t rings = ks * pf * 2 * TILE * d, merge = ks == 2 ? 2 * (16 * (d / 32) + 2) * WAVE * 4 : 0;
  return rings > merge ? rings : merge;
}
constexpr int64_t v32_lds_bytes(int64_t d, int64_t pf, int64_t ks) {
  return v32_vscale_offset(d, pf, ks) + (2 + 2 * ks) * d * 4;   // V scales of 2 wavefronts, K scales of all
}  // 16-row tiles per row group (the stream-K plan's unit of rows)

template <int CHR>
__device__ __forceinline__ int swz_k(int row) { return (row >> 1) & (CHR - 1); }
template <int CHR>
__device__ __forceinline__ int swz_v(int row) { return ((((row >> 1) & 1) | (((row >> 3) & 1) << 1)) << 1) & (CHR - 1); }

// QG: 0 = one q scale per (token, q head) row (implementation B's per-token-head q); 32 = one per 32
// channels (int8_ref's q_gran "group32"): QK step s then holds exactly group s's channels, its integer
// dot is scaled by that group's q scale and the groups' scores are summed in fp32.
// Wave priority over the issue of a step's tile DMA (after the step's barrier): the wavefront puts its
// share of the next tile's requests out ahead of the SIMD's other wavefronts' tile arithmetic, so the
// ring's loads start sooner (c3 60.1 -> 59.4 us, same box; priority over the QK block as well: no
// change). 0: off.
constexpr int V32_DMA_PRIO = 1;
template <int P>
__device__ __forceinline__ void v32_prio() {
  if constexpr (V32_DMA_PRIO != 0) {
    __builtin_amdgcn_sched_barrier(0);  // the priority brackets exactly the DMA issue
    __builtin_amdgcn_s_setprio(P);
    __builtin_amdgcn_sched_barrier(0);
  }
}
template <int D, int PF, int QG, int KS>
__device__ __forceinline__ void attend_rows32(const AttnArgs& a, int seq, int tok, int qlen, int seqlen, int kvh, int row0,
                                              int c_begin, int c_end, int wave, int kw, bool active, int part,
                                              int nparts, uint8_t* ring, float* vsl, float* ksl, float* merge,
                                              int lane) {
  constexpr int KST = D / 32;       // 32-channel QK steps = 32-channel PV tiles
  constexpr int CHR = D / 16;       // 16-byte chunks per K (or V) row
  constexpr int RPI = WAVE / CHR;   // rows per DMA instruction
  constexpr int IPH = 16 / RPI;     // DMA instructions per 16-key half of K (or V)
  constexpr int SLOT = 2 * TILE * D;
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  seq = __builtin_amdgcn_readfirstlane(seq);
  tok = __builtin_amdgcn_readfirstlane(tok);
  qlen = __builtin_amdgcn_readfirstlane(qlen);
  kvh = __builtin_amdgcn_readfirstlane(kvh);
  row0 = __builtin_amdgcn_readfirstlane(row0);
  c_begin = __builtin_amdgcn_readfirstlane(c_begin);
  c_end = __builtin_amdgcn_readfirstlane(c_end);
  part = __builtin_amdgcn_readfirstlane(part);
  nparts = __builtin_amdgcn_readfirstlane(nparts);
  wave = __builtin_amdgcn_readfirstlane(wave);
  kw = __builtin_amdgcn_readfirstlane(kw);
  const int n = lane & 31, h = lane >> 5;
  const int G = a.G;
  const int L = __builtin_amdgcn_readfirstlane(seqlen);
  // key split kw takes the piece's tiles kw, kw + KS, ...: ntk of them, in nsteps steps (the same count
  // for every wavefront of the workgroup -- a split with fewer tiles ends with an empty step); the two
  // wavefronts of a split fill its ring together, and all meet at one barrier per step
  if (L <= 0) c_end = c_begin;
  const int nt = c_end - c_begin;
  const int ntk = nt > kw ? (nt - kw + KS - 1) / KS : 0;
  const int nsteps = (nt + KS - 1) / KS;
  auto tile_of = [&](int i) { return c_begin + kw + i * KS; };   // the split's i-th tile
  const bool work = L > 0 && active;
  const int* bt = a.block_table + (int64_t)seq * a.bt_stride;
  const int bs = 1 << a.lbs;
  const int8_t* kbase = a.kc + (int64_t)kvh * a.k_sh;
  const int8_t* vbase = a.vc + (int64_t)kvh * a.v_sh;

  // ---- DMA: wavefront `wave` copies keys 16 wave .. 16 wave + 15 of a tile, K rows then V rows; lane L
  // of an instruction lands at byte 16 L of its RPI rows: row RPI u + L / CHR of the half, physical chunk
  // L % CHR, which holds logical chunk (L % CHR) ^ swz(row) ----
  uint32_t koff[IPH], voff[IPH];
#pragma unroll
  for (int u = 0; u < IPH; ++u) {
    const int rb = lane / CHR, pc = lane % CHR, row = 16 * wave + RPI * u + rb;
    koff[u] = (uint32_t)(rb * (int)a.k_sn + 16 * (pc ^ swz_k<CHR>(row)));
    voff[u] = (uint32_t)(rb * (int)a.v_sn + 16 * (pc ^ swz_v<CHR>(row)));
  }
  const int64_t kstep = (int64_t)RPI * a.k_sn, vstep = (int64_t)RPI * a.v_sn;
  // the half's first key; a half past the end re-reads the tile's first half (an in-bounds page)
  auto half_key = [&](int c) {
    const int key0 = c * TILE + 16 * wave;
    return key0 < L ? key0 : c * TILE;
  };
  auto page_of = [&](int c) {  // a scalar load of the block table
    const int idx = __builtin_amdgcn_readfirstlane(half_key(c) >> a.lbs);
    const int p = __builtin_amdgcn_readfirstlane(((const __attribute__((address_space(4))) int*)bt)[idx]);
    return (p >= 0 && p < a.num_blocks) ? p : 0;
  };
  auto dma_page = [&](int c, int st, int p) {
    const int key0 = half_key(c);
    const int o = key0 & (bs - 1);
    const int8_t* kb = kbase + (int64_t)p * a.k_sb + (int64_t)o * a.k_sn;
    const int8_t* vb = vbase + (int64_t)p * a.v_sb + (int64_t)o * a.v_sn;
    uint8_t* dst = ring + st * SLOT + (16 * wave) * D;
#pragma unroll
    for (int u = 0; u < IPH; ++u) {
      __builtin_amdgcn_global_load_lds((const void*)(kb + u * kstep + koff[u]),
                                       (__attribute__((address_space(3))) void*)(dst + RPI * u * D), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(vb + u * vstep + voff[u]),
                                       (__attribute__((address_space(3))) void*)(dst + TILE * D + RPI * u * D), 16,
                                       0, 0);
    }
  };
  auto dma = [&](int c, int st) { dma_page(c, st, page_of(c)); };
  constexpr int NIW = 2 * IPH;   // DMA instructions per wavefront and tile

  // ---- LDS read addresses (slot 0; a slot adds st * SLOT): K of QK step s for lane (key n, half h):
  // logical chunk 2 s + h of row n; V^T of channel tile c, read t: 16-lane group q = lane / 16,
  // addressing lane P = lane % 16 points at key 8 (2 t + (P / 2) / 4) + 4 (q / 2) + (P / 2) % 4, bytes
  // 32 c + 16 (q % 2) + 8 (P % 2): ds_read_b64_tr_b8 then hands lane 8 a + b (a, b < 8 ... of the group)
  // byte b of the chunks of lanes a, a + 2, ..., a + 14, i.e. channel 32 c + 16 (q % 2) + 8 a + b of
  // keys 8 (2 t + e / 4) + 4 h + e % 4, e = 0..7 -- the P codes' key order ----
  const uint32_t lbase = (uint32_t)(uintptr_t)ring;
  uint32_t ka[KST], va[KST][2];
#pragma unroll
  for (int s = 0; s < KST; ++s) ka[s] = lbase + n * D + 16 * ((2 * s + h) ^ swz_k<CHR>(n));
  {
    const int q = lane >> 4, P = lane & 15, e = P >> 1;
#pragma unroll
    for (int c = 0; c < KST; ++c)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int key = 8 * (2 * t + (e >> 2)) + 4 * (q >> 1) + (e & 3);
        va[c][t] = lbase + TILE * D + key * D + 16 * ((2 * c + (q & 1)) ^ swz_v<CHR>(key)) + 8 * (P & 1);
      }
  }

  // ---- q prologue: lane (row n, half h) holds channels 32 s + 16 h + b of row row0 + n; fold s_k,
  // one scale per row (the two halves exchange their maxima), quantize. Its loads -- the q row, the K
  // scales, and the V scales the epilogue reads (staged in this wavefront's LDS slice) -- are issued
  // before the first tiles' page ids and DMAs: vmcnt counts in issue order, so waiting for them does not
  // wait for the DMAs, and the three round trips overlap instead of adding up ----
  const int R = row0 + n, rtok = R / G, rh = R % G;
  static_assert(QG == 0 || QG == 32, "q scales per row or per 32 channels");
  i32x4 qop[KST];
  float rs;
  float rsg[QG ? KST : 1];   // per-group score scales (QG): q scale x K scale x softmax scale x log2 e
  int lim;
  {
    const bool qrow = rtok < qlen && active;
    u32x4 qw[2 * KST];
    if (qrow) {
      const uint16_t* qp = a.q + (int64_t)(tok + rtok) * a.q_st + (int64_t)(kvh * G + rh) * a.q_sh + 16 * h;
#pragma unroll
      for (int s = 0; s < KST; ++s) {
        qw[2 * s] = *reinterpret_cast<const u32x4*>(qp + 32 * s);
        qw[2 * s + 1] = *reinterpret_cast<const u32x4*>(qp + 32 * s + 8);
      }
    }
    // the K scales go through this wavefront's LDS slice too: 2 per lane here, 16 per lane read back
    // below (in registers they would hold 16 D / 32 VGPRs through the prologue)
    float2 ks2 = {0.f, 0.f};
    if (a.ks_pc && 2 * lane < D) ks2 = *reinterpret_cast<const float2*>(a.ks + kvh * D + 2 * lane);
    float2 vs2 = {0.f, 0.f};
    if (kw == 0 && a.vs_pc && 2 * lane < D) vs2 = *reinterpret_cast<const float2*>(a.vs + kvh * D + 2 * lane);
    if (nt > 0) {
      // groups past the split's last tile re-read the piece's last tile (in bounds, never read back)
      int pg[PF - 1];
#pragma unroll
      for (int j = 0; j < PF - 1; ++j) pg[j] = page_of(min(tile_of(j), c_end - 1));
#pragma unroll
      for (int j = 0; j < PF - 1; ++j) dma_page(min(tile_of(j), c_end - 1), j, pg[j]);
    }
    if (kw == 0 && a.vs_pc && 2 * lane < D) *reinterpret_cast<float2*>(vsl + 2 * lane) = vs2;
    if (a.ks_pc && 2 * lane < D) *reinterpret_cast<float2*>(ksl + 2 * lane) = ks2;
    float x[16 * KST];
    float amax = 0.f;
    if (qrow) {
#pragma unroll
      for (int s = 0; s < KST; ++s) {
        const u32x4 w0 = qw[2 * s], w1 = qw[2 * s + 1];
        const uint32_t wd[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          x[16 * s + 2 * j] = bf16_lo(wd[j]);
          x[16 * s + 2 * j + 1] = bf16_hi(wd[j]);
        }
      }
      if (a.ks_pc) {
#pragma unroll
        for (int s = 0; s < KST; ++s)
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const float4 f = *reinterpret_cast<const float4*>(ksl + 32 * s + 16 * h + 4 * u);
            x[16 * s + 4 * u] *= f.x; x[16 * s + 4 * u + 1] *= f.y;
            x[16 * s + 4 * u + 2] *= f.z; x[16 * s + 4 * u + 3] *= f.w;
          }
      }
#pragma unroll
      for (int e = 0; e < 16 * KST; ++e) amax = __builtin_fmaxf(amax, __builtin_fabsf(x[e]));
    } else {
#pragma unroll
      for (int e = 0; e < 16 * KST; ++e) x[e] = 0.f;
    }
    const float kpost = (a.ks_pc ? 1.f : a.ks[kvh]) * a.sm_log2;
    if constexpr (QG == 0) {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(amax), __float_as_uint(amax), false, false);
      amax = __builtin_fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      const float s = __builtin_fmaxf(amax / 127.f, 1e-8f);
      uint32_t codes[4 * KST];
      q_codes<16 * KST>(x, s, codes);
#pragma unroll
      for (int st = 0; st < KST; ++st) qop[st] = i32x4{(int)codes[4 * st], (int)codes[4 * st + 1],
                                                        (int)codes[4 * st + 2], (int)codes[4 * st + 3]};
      rs = s * kpost;
    } else {
      // group st: this lane's 16 channels and the other half's 16 (lane ^ 32)
#pragma unroll
      for (int st = 0; st < KST; ++st) {
        float ga = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) ga = __builtin_fmaxf(ga, __builtin_fabsf(x[16 * st + e]));
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ga), __float_as_uint(ga), false, false);
        ga = __builtin_fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        const float s = __builtin_fmaxf(ga / 127.f, 1e-8f);
        float xs[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) xs[e] = x[16 * st + e];
        uint32_t codes[4];
        q_codes<16>(xs, s, codes);
        qop[st] = i32x4{(int)codes[0], (int)codes[1], (int)codes[2], (int)codes[3]};
        rsg[st] = s * kpost;
      }
      rs = 0.f;
    }
    lim = rtok < qlen ? L - qlen + 1 + rtok : L;  // keys < lim are visible to this row
  }

  float m = -1e30f, l = 0.f, acc[KST][16];
#pragma unroll
  for (int c = 0; c < KST; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[c][v] = 0.f;

  // One 32-key tile from ring offset `so` (an int, or a compile-time constant: then the reads' immediate).
  // MASKED: some key of the tile is at or past some row's limit.
  auto tile = [&](auto masked_t, auto so_t, int c) {
    constexpr bool MASKED = decltype(masked_t)::value;
    constexpr bool CT = !std::is_same_v<decltype(so_t), int>;
    uint32_t so;
    if constexpr (CT) so = 0;
    else so = (uint32_t)so_t;
    constexpr int IMM = [] {
      if constexpr (CT) return decltype(so_t)::value;
      else return 0;
    }();
    const int n0 = c * TILE;
    // ---- QK ----
    i32x4 kop[KST];
    if constexpr (KST == 4) {
      asm volatile(
          "ds_read_b128 %0, %4 offset:%c8\n"
          "ds_read_b128 %1, %5 offset:%c8\n"
          "ds_read_b128 %2, %6 offset:%c8\n"
          "ds_read_b128 %3, %7 offset:%c8\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(kop[0]), "=&v"(kop[1]), "=&v"(kop[2]), "=&v"(kop[3])
          : "v"(ka[0] + so), "v"(ka[1] + so), "v"(ka[2] + so), "v"(ka[3] + so), "i"(IMM)
          : "memory");
    } else {
      asm volatile(
          "ds_read_b128 %0, %2 offset:%c4\n"
          "ds_read_b128 %1, %3 offset:%c4\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(kop[0]), "=&v"(kop[1])
          : "v"(ka[0] + so), "v"(ka[1] + so), "i"(IMM)
          : "memory");
    }
    i32x16 sc = {};
    float sf[QG ? 16 : 1];   // QG: the scores (log2 units), the groups' scaled dots summed in fp32
    if constexpr (QG == 0) {
#pragma unroll
      for (int s = 0; s < KST; ++s) sc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kop[s], qop[s], sc, 0, 0, 0);
    } else {
#pragma unroll
      for (int s = 0; s < KST; ++s) {
        const i32x16 zg = __builtin_amdgcn_mfma_i32_32x32x32_i8(kop[s], qop[s], i32x16{}, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 16; ++v) sf[v] = s == 0 ? (float)zg[v] * rsg[0] : __builtin_fmaf((float)zg[v], rsg[s], sf[v]);
      }
    }
    // ---- V^T operands (issued now, consumed after the softmax) ----
    typedef unsigned long long u64;
    u64 vw[KST][2];
    if constexpr (KST == 4) {
      asm volatile(
          "ds_read_b64_tr_b8 %0, %8 offset:%c16\n"
          "ds_read_b64_tr_b8 %1, %9 offset:%c16\n"
          "ds_read_b64_tr_b8 %2, %10 offset:%c16\n"
          "ds_read_b64_tr_b8 %3, %11 offset:%c16\n"
          "ds_read_b64_tr_b8 %4, %12 offset:%c16\n"
          "ds_read_b64_tr_b8 %5, %13 offset:%c16\n"
          "ds_read_b64_tr_b8 %6, %14 offset:%c16\n"
          "ds_read_b64_tr_b8 %7, %15 offset:%c16\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(vw[0][0]), "=&v"(vw[0][1]), "=&v"(vw[1][0]), "=&v"(vw[1][1]), "=&v"(vw[2][0]), "=&v"(vw[2][1]),
            "=&v"(vw[3][0]), "=&v"(vw[3][1])
          : "v"(va[0][0] + so), "v"(va[0][1] + so), "v"(va[1][0] + so), "v"(va[1][1] + so), "v"(va[2][0] + so),
            "v"(va[2][1] + so), "v"(va[3][0] + so), "v"(va[3][1] + so), "i"(IMM)
          : "memory");
    } else {
      asm volatile(
          "ds_read_b64_tr_b8 %0, %4 offset:%c8\n"
          "ds_read_b64_tr_b8 %1, %5 offset:%c8\n"
          "ds_read_b64_tr_b8 %2, %6 offset:%c8\n"
          "ds_read_b64_tr_b8 %3, %7 offset:%c8\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(vw[0][0]), "=&v"(vw[0][1]), "=&v"(vw[1][0]), "=&v"(vw[1][1])
          : "v"(va[0][0] + so), "v"(va[0][1] + so), "v"(va[1][0] + so), "v"(va[1][1] + so), "i"(IMM)
          : "memory");
    }
    // ---- online softmax; key of register v = n0 + 8 (v / 4) + 4 h + v % 4 ----
    bool ok[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) ok[v] = MASKED ? n0 + 8 * (v >> 2) + 4 * h + (v & 3) < lim : true;
    float tmax;
    if constexpr (QG == 0) {
      int mx = INT32_MIN;
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = ok[v] ? max(mx, sc[v]) : mx;
      const auto sw = __builtin_amdgcn_permlane32_swap((unsigned)mx, (unsigned)mx, false, false);
      mx = max((int)sw[0], (int)sw[1]);
      // an int8 dot product never reaches INT32_MIN: it marks a row with no visible key in the tile
      tmax = (MASKED && mx == INT32_MIN) ? -INFINITY : (float)mx * rs;
    } else {
      float fx = -INFINITY;
#pragma unroll
      for (int v = 0; v < 16; ++v) fx = ok[v] ? __builtin_fmaxf(fx, sf[v]) : fx;
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(fx), __float_as_uint(fx), false, false);
      tmax = __builtin_fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    const bool raise = tmax > m + ATTN_SLACK;
    const bool rescale = raise && m > -1e29f;   // a piece's first tile has nothing to rescale
    const float mnew = raise ? tmax : m;
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);
    m = mnew;
    const float pm = __builtin_amdgcn_exp2f(tmax - mnew);  // max of this tile's P (exp2 is monotone)
    const float ps = __builtin_fmaxf(div127(pm), 1e-30f);
    const float ri = __builtin_amdgcn_rcpf(ps);
    uint32_t pw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float t[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int v = 4 * j + i;
        const float p = QG ? __builtin_amdgcn_exp2f(sf[v] - mnew)
                           : __builtin_amdgcn_exp2f(__builtin_fmaf((float)sc[v], rs, -mnew));
        const float c2 = __builtin_fminf(__builtin_fmaf(p, ri, QC_MAGIC), QC_MAGIC + 127.f);
        t[i] = ok[v] ? c2 : QC_MAGIC;
      }
      pw[j] = pack_magic4(t[0], t[1], t[2], t[3]);
    }
    const i32x4 pop = i32x4{(int)pw[0], (int)pw[1], (int)pw[2], (int)pw[3]};
    const float psum = (float)__builtin_amdgcn_sad_u8(pw[3], 0u, __builtin_amdgcn_sad_u8(pw[2], 0u,
                           __builtin_amdgcn_sad_u8(pw[1], 0u, __builtin_amdgcn_sad_u8(pw[0], 0u, 0u))));
    l = __builtin_fmaf(psum, ps, l * alpha);
    if (__any(rescale)) {
#pragma unroll
      for (int c = 0; c < KST; ++c)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[c][v] *= alpha;
    }
    // ---- PV ----
#pragma unroll
    for (int c = 0; c < KST; ++c) {
      const i32x4 vop = i32x4{(int)(uint32_t)vw[c][0], (int)(uint32_t)(vw[c][0] >> 32), (int)(uint32_t)vw[c][1],
                              (int)(uint32_t)(vw[c][1] >> 32)};
      i32x16 z = {};
      z = __builtin_amdgcn_mfma_i32_32x32x32_i8(vop, pop, z, 0, 0, 0);
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[c][v] = __builtin_fmaf((float)z[v], ps, acc[c][v]);
    }
  };

  // ---- main loop: one barrier per step. The split's i-th tile sits in slot i % PF of its ring; after
  // the barrier (this wavefront's DMA of it has landed, everyone's has, and everyone is done with step
  // i - 1) slot (i + PF - 1) % PF takes the split's tile i + PF - 1. Tiles before j_full (piece-relative)
  // have no masked key for any row of this wavefront (a loop of whole rounds of PF of them, with
  // compile-time slots, then the rest); wavefronts may split their steps differently between the loops
  // but each meets exactly nsteps barriers. ----
  if (nt > 0) {
    const int lim_lo = L - qlen + 1 + row0 / G;          // every row of this wavefront sees keys < lim_lo
    const int full_end = lim_lo > 0 ? lim_lo / TILE : 0;
    const int j_full = work ? max(0, min(nt, full_end - c_begin)) : nt;
    const int i_full = j_full > kw ? (j_full - kw + KS - 1) / KS : 0;   // the split's unmasked tiles
    // Whole rounds keep PF - 2 of the split's tiles in flight behind the one they wait for. The last
    // PF - 1 steps issue no more DMAs and wait for exactly what is still in flight: groups g_0 .. g_{PF-2}
    // came from the prologue (past the split's end: re-reads), step i issued g_{i+PF-1} while
    // i + PF - 1 < ntk, so behind the split's tile i there are ahead = min(PF - 2, max(PF - 2, ntk - 1) - i)
    // groups; a step past the split's tiles (i >= ntk) only waits and meets the barrier.
    auto step = [&](auto masked_t, auto tail_t, int i, auto st_t) {
      if constexpr (decltype(tail_t)::value) {
        const int ahead = min(PF - 2, max(PF - 2, ntk - 1) - i);
        if (ahead <= 0) wait_vm<0>();
        else if (ahead == 1) wait_vm<NIW>();
        else wait_vm<(PF - 2) * NIW>();
      } else {
        wait_vm<(PF - 2) * NIW>();
      }
      lds_barrier();
      v32_prio<1>();
      if (!decltype(tail_t)::value || i + PF - 1 < ntk) dma(tile_of(i + PF - 1), (i + PF - 1) % PF);
      v32_prio<0>();
      if (work && (!decltype(tail_t)::value || i < ntk)) {
        if constexpr (std::is_same_v<decltype(st_t), int>) tile(masked_t, (int)(st_t * SLOT), tile_of(i));
        else tile(masked_t, std::integral_constant<int, decltype(st_t)::value * SLOT>{}, tile_of(i));
      }
    };
    int i = 0;
    // whole rounds end at least PF - 1 tiles before the split's end, so every step of them fetches a real tile
    const int i_round = min(i_full, ntk - (PF - 1));
    for (; i + PF <= i_round; i += PF) {
      step(std::false_type{}, std::false_type{}, i, std::integral_constant<int, 0>{});
      if constexpr (PF > 1) step(std::false_type{}, std::false_type{}, i + 1, std::integral_constant<int, 1 % PF>{});
      if constexpr (PF > 2) step(std::false_type{}, std::false_type{}, i + 2, std::integral_constant<int, 2 % PF>{});
      if constexpr (PF > 3) step(std::false_type{}, std::false_type{}, i + 3, std::integral_constant<int, 3 % PF>{});
      static_assert(PF >= 2 && PF <= 4, "rounds are written for 2 to 4 slots");
    }
    for (; i < min(i_full, ntk); ++i) step(std::false_type{}, std::true_type{}, i, i % PF);
    for (; i < nsteps; ++i) step(std::true_type{}, std::true_type{}, i, i % PF);
    wait_vm<0>();   // the ring is empty and read before the next piece refills it
    lds_barrier();
  }

  // ---- epilogue: lane (n, h) holds row n, channels 32 c + 8 j + 4 h + i in acc[c][4 j + i] ----
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    l = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if constexpr (KS == 2) {
    // key split 1 hands its (m, l, acc) to key split 0 of the same rows through LDS (the rings' space,
    // free now: lane-major [field][lane], conflict-free), which merges them:
    // M = max(m0, m1), acc = 2^(m0 - M) acc0 + 2^(m1 - M) acc1, l likewise
    constexpr int MF = 16 * KST + 2;
    float* mb = merge + (wave & 1) * MF * WAVE + lane;
    if (kw == 1) {
#pragma unroll
      for (int c = 0; c < KST; ++c)
#pragma unroll
        for (int v = 0; v < 16; ++v) mb[(16 * c + v) * WAVE] = acc[c][v];
      mb[16 * KST * WAVE] = m;
      mb[(16 * KST + 1) * WAVE] = l;
    }
    lds_barrier();
    if (kw == 0) {
      const float m1 = mb[16 * KST * WAVE], l1 = mb[(16 * KST + 1) * WAVE];
      const float M = __builtin_fmaxf(m, m1);
      const float a0 = __builtin_amdgcn_exp2f(m - M), a1 = __builtin_amdgcn_exp2f(m1 - M);
#pragma unroll
      for (int c = 0; c < KST; ++c)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[c][v] = __builtin_fmaf(acc[c][v], a0, mb[(16 * c + v) * WAVE] * a1);
      l = __builtin_fmaf(l, a0, l1 * a1);
      m = M;
    }
    lds_barrier();   // read before the next piece's DMAs refill the rings
    if (kw != 0) return;
  }
  if (!active || rtok >= qlen) return;
  const int head = kvh * G + rh;
  const int qt = tok + rtok;
  // the V scales of channels 32 c + 8 j + 4 h .. + 3, from the copy the prologue staged in LDS
  auto vscale4 = [&](int c, int j) -> float4 {
    if (a.vs_pc) return *reinterpret_cast<const float4*>(vsl + 32 * c + 8 * j + 4 * h);
    const float v = a.vs[kvh];
    return float4{v, v, v, v};
  };
  if (nparts == 1) {
    if (a.max_splits > 1 && qt < a.cut_rows && h == 0) a.segm_sum[(int64_t)qt * a.seg_st + (int64_t)head * a.seg_sh] = -1.f;
    const float inv = 1.f / __builtin_fmaxf(l, 1e-30f);
    uint16_t* orow = a.out + (int64_t)qt * a.o_st + (int64_t)head * a.o_sh + 4 * h;
#pragma unroll
    for (int c = 0; c < KST; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 f = vscale4(c, j);
        const float* ac = &acc[c][4 * j];
        *reinterpret_cast<u32x2*>(orow + 32 * c + 8 * j) =
            u32x2{pack_bf16x2((ac[0] * inv) * f.x, (ac[1] * inv) * f.y), pack_bf16x2((ac[2] * inv) * f.z, (ac[3] * inv) * f.w)};
      }
  } else {
    const int64_t sidx = (int64_t)qt * a.seg_st + (int64_t)head * a.seg_sh + part;
    if (h == 0) {
      a.segm_max[sidx] = m;
      a.segm_sum[sidx] = part == nparts - 1 ? -2.f - l : l;  // the last piece is marked (l >= 0)
    }
    float* sp = a.segm_out + sidx * D + 4 * h;
#pragma unroll
    for (int c = 0; c < KST; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 f = vscale4(c, j);
        const float* ac = &acc[c][4 * j];
        *reinterpret_cast<float4*>(sp + 32 * c + 8 * j) = float4{ac[0] * f.x, ac[1] * f.y, ac[2] * f.z, ac[3] * f.w};
      }
  }
}

// Stream-K over the batch as attn_kernel (plan_and_locate, the same units and pieces), for row groups
// of 64 rows run by 2 x KS wavefronts: row wavefront rw = wave % 2 (rows 32 rw .. 32 rw + 31 of the
// group) of key split kw = wave / 2. Dynamic LDS (v32_lds_bytes): KS rings of PF slots, then the V scales of the 2 row
// wavefronts of key split 0.
template <int D, int PF, int QG, int KS>
__global__ __launch_bounds__(WAVE * 2 * KS) void verify_kernel(AttnArgs a) {
  const int lane = threadIdx.x & (WAVE - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int rw = wave & 1, kw = wave >> 1;
  extern __shared__ float v32_lds[];
  constexpr int SLOT = 2 * TILE * D;
  uint8_t* rings = reinterpret_cast<uint8_t*>(v32_lds);
  uint8_t* ring = rings + kw * PF * SLOT;
  float* vsl = reinterpret_cast<float*>(rings + v32_vscale_offset(D, PF, KS)) + rw * D;
  float* ksl = reinterpret_cast<float*>(rings + v32_vscale_offset(D, PF, KS)) + (2 + wave) * D;
  float* merge = reinterpret_cast<float*>(rings);
  int worker = blockIdx.x;
  {  // no branch before the plan: its argument loads go out in one batch
    const int q = a.workers / NUM_XCDS, rem = a.workers % NUM_XCDS;
    const int wx = blockIdx.x % NUM_XCDS, wi = blockIdx.x / NUM_XCDS;
    worker = a.xcd_order ? wx * q + min(wx, rem) + wi : worker;
    worker = (int)blockIdx.x < a.workers ? worker : a.workers;   // past the grid's workers: no units
  }
  int r;
  long long rstart;
  ReqWork w;
  const Plan pl = plan_and_locate(a, worker, lane, r, rstart, w);
  long long pos = (long long)worker * pl.chunk;
  const long long end = min(pos + pl.chunk, pl.total);
  if (pos >= end || r >= a.num_seqs) return;
  int seglen = seg_units(a, w);
  int seg = (int)udiv_plan(pos - rstart, seglen), off = (int)(pos - rstart - (long long)seg * seglen);
  bool whole = !cuttable(a, w);
  while (pos < end) {
    const long long seg_start = rstart + (long long)seg * seglen;
    const int take = (int)min((long long)(seglen - off), end - pos);
    const int fc = a.seg_cost;
    const long long first = whole ? worker : udiv_plan(seg_start + fc, pl.chunk);
    const long long last = whole ? worker : udiv_plan(seg_start + seglen - 1, pl.chunk);
    const int kvh = seg / w.rgroups, rg = seg % w.rgroups;
    const int row0 = rg * (16 * V32_GROUP_TILES) + 32 * rw;
    const int c0 = whole ? 0 : max(off - fc, 0);
    const int c1 = whole ? (off == 0 ? w.ntiles : 0) : max(off + take - fc, 0);
    if (c1 > c0)
      attend_rows32<D, PF, QG, KS>(a, r, w.tok, w.qlen, w.len, kvh, row0, c0, c1, rw, kw, row0 < w.qlen * a.G,
                                   (int)(worker - first), (int)(last - first + 1), ring, vsl, ksl, merge, lane);
    pos += take;
    off = 0;
    if (++seg == a.hkv * w.rgroups && pos < end) {  // on to the next request with work
      rstart += (long long)seglen * a.hkv * w.rgroups;
      seg = 0;
      do {
        if (++r >= a.num_seqs) return;
        w = req_work(a, r);
      } while (w.ntiles == 0);
      seglen = seg_units(a, w);
      whole = !cuttable(a, w);
    }
  }
}

// Merge the pieces of the cut segments (reference kvq/cuda/int8_kv.cu:465-503):
//   o = sum_s 2^(m_s - M) acc_s / max(sum_s 2^(m_s - M) l_s, 1e-30)
// One wavefront per (request, q head, query token), RED_WAVES q heads per workgroup (fewer, larger
// workgroups: a row is a short chain of dependent loads, and one-wavefront workgroups ran into the
// per-CU workgroup limit before the wavefront limit); lane s holds piece s's weight; lanes own D / 64
// channels each. The piece count is read from the denominators (the last piece's is stored as
// -2 - l, a row that was not cut has -1 in slot 0 and was written by the attention kernel), so the
// merge needs neither the plan nor any buffer beyond the split buffers of the call.
constexpr int RED_WAVES = 4;
constexpr int MERGE_Z = 64;   // largest z extent of split_reduce_kernel's grid
// pieces of a row fetched together with its denominators (c3: 59.4 -> 59.0 us same box, c4 unchanged;
// 4 pieces: 61.4 us -- the extra reads of rows with fewer pieces cost more than the round trip saves)
constexpr int MERGE_SPEC = 2;
template <int D>
__device__ __forceinline__ void merge_row(const AttnArgs& a, int tok, int t, int h, int lane) {
  // denominators as the attention kernel left them: piece-0 slot -1 = not cut (already written);
  // otherwise pieces 0..S-2 hold l >= 0 and the last piece -2 - l
  const int64_t base = (int64_t)(tok + t) * a.seg_st + (int64_t)h * a.seg_sh;
  // the maxima and the first MERGE_SPEC pieces' partial outputs are fetched with the denominators (one
  // memory round trip for a row of up to MERGE_SPEC pieces), later pieces four at a time
  const bool held = lane < a.max_splits;
  constexpr int CPL = D / WAVE, UNR = 4;
  const float* po = a.segm_out + base * D + CPL * lane;
  const float enc = held ? a.segm_sum[base + lane] : -1.f;
  const float mraw = held ? a.segm_max[base + lane] : -INFINITY;
  float v0[MERGE_SPEC][CPL];
#pragma unroll
  for (int j = 0; j < MERGE_SPEC; ++j) {  // (in bounds: slots past the buffers' pieces re-read the last)
    const float* p = po + (int64_t)min(j, a.max_splits - 1) * D;
#pragma unroll
    for (int e = 0; e < CPL; ++e) v0[j][e] = p[e];
  }
  // keep those loads here, ahead of the test below (the compiler would otherwise sink them into it)
#pragma unroll
  for (int j = 0; j < MERGE_SPEC; ++j)
#pragma unroll
    for (int e = 0; e < CPL; ++e) asm volatile("" : "+v"(v0[j][e]));
  const unsigned long long neg = __ballot(enc < 0.f);
  if (neg == 0ull) return;
  const int last = __builtin_ctzll(neg);
  if (last == 0) return;  // not cut
  const int S = last + 1;
  const float ls = lane < last ? enc : (lane == last ? -2.f - enc : 0.f);
  const float ms = lane < S ? mraw : -INFINITY;
  const float M = wave_max(ms);
  const float wt = lane < S ? __builtin_amdgcn_exp2f(ms - M) : 0.f;
  const float den = wave_sum(wt * ls);
  const float inv = 1.f / __builtin_fmaxf(den, 1e-30f);
  float num[CPL];
#pragma unroll
  for (int e = 0; e < CPL; ++e) num[e] = 0.f;
#pragma unroll
  for (int j = 0; j < MERGE_SPEC; ++j) {
    const bool in = j < S;
    const float ws = __shfl(wt, min(j, S - 1), WAVE);
#pragma unroll
    for (int e = 0; e < CPL; ++e) num[e] = in ? __builtin_fmaf(ws, v0[j][e], num[e]) : num[e];
  }
  for (int s0 = MERGE_SPEC; s0 < S; s0 += UNR) {
    float v[UNR][CPL];
#pragma unroll
    for (int j = 0; j < UNR; ++j) {  // pieces past the last re-read it (in bounds), unused
      const float* p = po + (int64_t)min(s0 + j, S - 1) * D;
#pragma unroll
      for (int e = 0; e < CPL; ++e) v[j][e] = p[e];
    }
#pragma unroll
    for (int j = 0; j < UNR; ++j) {
      const bool in = s0 + j < S;
      const float ws = __shfl(wt, min(s0 + j, S - 1), WAVE);
#pragma unroll
      for (int e = 0; e < CPL; ++e) num[e] = in ? __builtin_fmaf(ws, v[j][e], num[e]) : num[e];
    }
  }
  uint16_t* op = a.out + (int64_t)(tok + t) * a.o_st + (int64_t)h * a.o_sh + CPL * lane;
  if constexpr (CPL == 2) {
    *reinterpret_cast<uint32_t*>(op) = pack_bf16x2(num[0] * inv, num[1] * inv);
  } else {
    op[0] = (uint16_t)bf16_rne(num[0] * inv);
  }
}
// Grid (request, group of RED_WAVES q heads, z): block z merges query tokens z, z + gridDim.z, ... of
// its request, so every short request's rows are covered whatever max_query_len the caller reported.
template <int D>
__global__ __launch_bounds__(WAVE * RED_WAVES) void split_reduce_kernel(AttnArgs a) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int seq = blockIdx.x;
  const int h = blockIdx.y * RED_WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int tok = a.cu_q[seq], qlen = a.cu_q[seq + 1] - tok;
  if (h >= a.G * a.hkv || qlen <= 0 || qlen > a.qmax) return;
  const int rows = min(qlen, a.cut_rows - tok);  // tokens past the split buffers' rows were not cut
  for (int t = blockIdx.z; t < rows; t += gridDim.z) merge_row<D>(a, tok, t, h, lane);
}

// ------------------------------------------------------------------------------------------------
// Page dequantization for the long-query path (reference kvq/cuda/int8_kv.cu:505-542): a lane converts
// 16 channels of one (token, head) -- a 16-byte int8 load, two 16-byte bf16 stores (bf16_rne(f32(code) *
// scale), v_cvt_pk_bf16_f32, round to nearest even).
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ float i8f(uint32_t w, int b) { return (float)(int8_t)(w >> (8 * b)); }

__device__ __forceinline__ u32x4 dq8(uint32_t w0, uint32_t w1, const float* s) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  u32x4 o;
  uint32_t r[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = j < 2 ? w0 : w1;
    bf2 h;
    h.x = (__bf16)(i8f(w, 2 * (j & 1)) * s[2 * j]);
    h.y = (__bf16)(i8f(w, 2 * (j & 1) + 1) * s[2 * j + 1]);
    r[j] = *reinterpret_cast<uint32_t*>(&h);
  }
  o.x = r[0]; o.y = r[1]; o.z = r[2]; o.w = r[3];
  return o;
}

// 8 codes (two dwords) -> 8 bf16 (one 16-byte store)
// 8 int8 codes -> 8 bf16 (exact: |code| <= 128)
__device__ __forceinline__ u32x4 cv8(uint32_t w0, uint32_t w1) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  uint32_t r[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = j < 2 ? w0 : w1;
    bf2 h;
    h.x = (__bf16)i8f(w, 2 * (j & 1));
    h.y = (__bf16)i8f(w, 2 * (j & 1) + 1);
    r[j] = *reinterpret_cast<uint32_t*>(&h);
  }
  u32x4 o;
  o.x = r[0]; o.y = r[1]; o.z = r[2]; o.w = r[3];
  return o;
}

__device__ __forceinline__ u32x4 dq8x(uint32_t w0, uint32_t w1, const float (&s)[8]) {
  const float tmp[8] = {s[0], s[1], s[2], s[3], s[4], s[5], s[6], s[7]};
  return dq8(w0, w1, tmp);
}

// One workgroup per output page (blockIdx.x) and group of heads (blockIdx.y): its page id chain (src_req,
// src_j, block table) is read once, by scalar loads. Thread tid owns combination k = tid % C of (head,
// K|V, 8-channel chunk) -- C = heads * 2 * D / 8 of them, chunks fastest -- and tokens tid / C, + TPC, ...
// of the page (TPC = threads / C), its 8 scales in registers; up to DQ_BATCH 8-byte code loads are in
// flight before they are converted and stored. A lane's 8 bf16 are one 16-byte store and consecutive
// lanes' stores are consecutive: each store instruction writes whole rows of the output [P, bs, H, D]
// (16 lanes per 256-byte K or V row at D = 128), never parts of lines.
constexpr int DQ_BATCH = 16;
template <int D>
__global__ __launch_bounds__(256) void dequant_pages_kernel(
    const int8_t* __restrict__ kc, int64_t k_sb, int64_t k_sn, int64_t k_sh, const int8_t* __restrict__ vc,
    int64_t v_sb, int64_t v_sn, int64_t v_sh, int num_blocks, int bs, int H, int heads_per_block,
    uint16_t* __restrict__ ko, uint16_t* __restrict__ vo, const int* __restrict__ bt, int64_t bt_stride,
    const int* __restrict__ src_req, const int* __restrict__ src_j, const float* __restrict__ ks, int ks_pc,
    const float* __restrict__ vs, int vs_pc) {
  constexpr int CPK = D / 8;                      // 8-channel chunks of one K (or V) row
  constexpr int CPH = 2 * CPK;                    // combinations per head: K and V chunks
  const int p = blockIdx.x;
  const int h0 = blockIdx.y * heads_per_block;
  const int nh = min(heads_per_block, H - h0);
  const int C = nh * CPH;
  const int tpc = blockDim.x / C;                 // threads per combination (token slices)
  const int tid = threadIdx.x;
  if (tid >= C * tpc) return;
  const int k = tid % C, t0 = tid / C;
  const int h = h0 + k / CPH, kv = (k % CPH) / CPK, d0 = 8 * (k % CPK);
  // page id: three dependent loads, uniform across the workgroup (scalar)
  const int r = __builtin_amdgcn_readfirstlane(((const __attribute__((address_space(4))) int*)src_req)[p]);
  const int j = __builtin_amdgcn_readfirstlane(((const __attribute__((address_space(4))) int*)src_j)[p]);
  int src = __builtin_amdgcn_readfirstlane(((const __attribute__((address_space(4))) int*)bt)[(int64_t)r * bt_stride + j]);
  if (src < 0 || src >= num_blocks) src = 0;
  float sc[8];
  const float* sp = kv ? vs : ks;
  if (kv ? vs_pc : ks_pc) {
    const float4 f0 = *reinterpret_cast<const float4*>(sp + h * D + d0);
    const float4 f1 = *reinterpret_cast<const float4*>(sp + h * D + d0 + 4);
    sc[0] = f0.x; sc[1] = f0.y; sc[2] = f0.z; sc[3] = f0.w; sc[4] = f1.x; sc[5] = f1.y; sc[6] = f1.z; sc[7] = f1.w;
  } else {
    const float v = sp[h];
#pragma unroll
    for (int e = 0; e < 8; ++e) sc[e] = v;
  }
  const int8_t* base = kv ? vc + (int64_t)src * v_sb + (int64_t)h * v_sh + d0 : kc + (int64_t)src * k_sb + (int64_t)h * k_sh + d0;
  const int64_t tstride = kv ? v_sn : k_sn;
  uint16_t* obase = (kv ? vo : ko) + ((int64_t)p * bs * H + h) * D + d0;
  for (int tb = t0; tb < bs; tb += DQ_BATCH * tpc) {
    u32x2 w[DQ_BATCH];
#pragma unroll
    for (int i = 0; i < DQ_BATCH; ++i) {
      const int t = tb + i * tpc;
      if (t < bs) w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(base + t * tstride));
    }
#pragma unroll
    for (int i = 0; i < DQ_BATCH; ++i) {
      const int t = tb + i * tpc;
      if (t >= bs) break;
      __builtin_nontemporal_store(dq8x(w[i].x, w[i].y, sc), reinterpret_cast<u32x4*>(obase + (int64_t)t * H * D));
    }
  }
}

// ------------------------------------------------------------------------------------------------
// bf16 paged prefill attention for the long-query requests: the consumer of dequant_pages' temporary
// bf16 cache, in place of the reference's vLLM FlashAttention call (kvq/cuda_kernels.py:106-131,
// flash_attn_varlen_func(q, kt, vt, ..., causal=True, block_table=plan.block_table)).
//   o = softmax(q k^T * scale, bottom-right causal) v   per (token, q head), fp32 softmax and
//   accumulation, bf16 operands -- P is rounded to bf16 for the PV product, as FlashAttention does.
// A workgroup takes 128 (token, q head) rows of one (request, kv head) (rows = token * G + head: the G
// q heads of a kv head share every K/V tile), 4 wavefronts x 2 blocks of 16 rows; every K and V operand
// read from LDS feeds the MFMAs of both blocks. 32-key K/V tiles are staged in
// LDS (double buffered, one barrier per tile), both row-major [key][channel] with padded rows: K rows
// of D + 8 elements (a quarter-wavefront's 16 rows of 16 bytes fall in 16 distinct bank quads), V rows
// of D + 16 (the 4 rows x 32 bytes of a transposing read in distinct banks). The V^T operand comes from
// ds_read_b64_tr_b16: within a 16-lane group, lane 4a + b receives element b of the 8-byte chunks
// addressed by lanes a, a + 4, a + 8, a + 12 -- pointing those lanes at 4 keys' rows gives every lane
// 4 keys of one channel. Per wavefront and tile:
//   QK  S^T[key][row]  = K . Q^T     v_mfma_f32_16x16x32_bf16, A = K (16 keys), B = q rows
//   PV  O^T[chan][row] = V^T . P^T   v_mfma_f32_16x16x32_bf16, K = the 32-key tile
// The QK accumulator lane (row n, group g) holds keys 16b + 4g + i -- the 8 key slots it feeds to the
// PV B operand (slot j: key 4g + j for j < 4, 16 + 4g + j - 4 after), so P stays in its lane; the
// V^T operand reads the same keys: two transposing 8-byte LDS reads per channel tile.
// ------------------------------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct PrefillArgs {
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  uint16_t* out;
  const int* cu_q;
  const int* seq_lens;
  const int* block_table;
  const int* tile_req;   // workgroup x: request and first row of its 64 rows
  const int* tile_row;
  int64_t q_st, q_sh, o_st, o_sh, k_sb, k_sn, k_sh, v_sb, v_sn, v_sh, bt_stride;  // elements
  float sm_log2;         // softmax_scale * log2(e)
  int G, lbs, num_blocks;
  uint32_t kpage, vpage;  // bytes per page (2 k_sb, 2 v_sb: below 2^32)
  uint32_t krow, vrow;    // bytes per slot (2 k_sn, 2 v_sn: a page's slots span below 2^31 bytes)
  int contig;             // a page is block_size slots (k_sb = block_size k_sn, v likewise)
  // INT8 pages read directly (prefill_i8_kernel): kc / vc are the int8 caches, the strides and the
  // page / slot sizes above are bytes, and these are the dequantization scales (per channel when *_pc)
  const float* ks;
  const float* vs;
  int ks_pc, vs_pc;
};

constexpr int PR_RB = 2;                    // 16-row blocks per wavefront
constexpr int PR_ROWS = 4 * 16 * PR_RB;     // rows per workgroup (4 wavefronts)
constexpr int PR_KEYS = 32;                 // keys per tile
constexpr float PR_SLACK = 8.f;             // log2 headroom of the reference maximum (general loop)
constexpr float PR_FAST_PSUM_MAX = 0x1p60f;  // largest per-lane denominator the fast pass takes (P <= 2^60)
constexpr int PR_STAGES = 3;                // LDS ring: tiles in flight + the one computed (3 x 16 KB: 3 workgroups per CU)
constexpr int PR_I8_STAGES = 2;             // INT8 pages: int8 ring stages (2 x 8 KB at D 128, + 2 bf16 stages)
// Wave priority over a tile's QK block (K operand reads + MFMAs): a wavefront with matrix work ready
// issues it ahead of the other wavefronts' softmax VALU on its SIMD, so the MFMA pipe idles less
// (c4 prefill 7.28-7.37 -> 7.16-7.19 ms, same box, identical output; priority over the PV block as well,
// or over the PV block alone, timed the same or slower, and over the softmax made no difference).
// 0: off.
constexpr int PR_QK_PRIO = 1;
template <int P>
__device__ __forceinline__ void pr_prio() {
  if constexpr (PR_QK_PRIO != 0) {
    __builtin_amdgcn_sched_barrier(0);  // the priority brackets exactly the QK block
    __builtin_amdgcn_s_setprio(P);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// two floats -> two bf16 (round to nearest even, v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float a, float b) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  bf2 h;
  h.x = (__bf16)a;
  h.y = (__bf16)b;
  return *reinterpret_cast<uint32_t*>(&h);
}


// Where the K / V tiles come from: the bf16 temporary cache, or the INT8 pages themselves
// (prefill_i8_kernel below), converted tile by tile either as dequant_pages converts them (bf16 of
// code x scale) or as exact bf16 codes with the scales folded into q (K) and the output (V).
constexpr int PR_SRC_BF16 = 0, PR_SRC_I8 = 1, PR_SRC_I8_FOLD = 2;

template <int D, int SRC>
__device__ __forceinline__ void prefill_body(const PrefillArgs& a) {
  constexpr bool I8 = SRC != PR_SRC_BF16;
  constexpr bool FOLD = SRC == PR_SRC_I8_FOLD;
  constexpr int DS = D / 32;                // 32-channel chunks of the QK contraction
  constexpr int VT = D / 16;                // PV channel tiles
  constexpr int RB = PR_RB;
  constexpr int CH = D / 8;                 // 16-byte chunks per key row
  constexpr int ROWB = 2 * D;               // bytes per key row
  constexpr int TILEB = PR_KEYS * ROWB;     // bytes per K (or V) tile
  constexpr int RPI = 1024 / ROWB;          // key rows per DMA instruction (64 lanes x 16 bytes)
  constexpr int IPW = TILEB / 1024 / 4;     // DMA instructions per wavefront per matrix and tile
  constexpr int NS = PR_STAGES;
  // XOR swizzles of the 16-byte chunks of a row: K by row % CH (the 16 rows of a K-operand read land
  // in distinct bank quads), V by 2 * row % CH (the 4 rows x 2 chunks of a transposing read do)
  auto kswz = [](int row) { return row % CH; };
  auto vswz = [](int row) { return (2 * row) % CH; };
  // I8: the DMA brings a tile's codes into a ring of NS8 int8 stages (rows of D bytes, unswizzled); the
  // workgroup converts the tile into one of two bf16 stages, laid out as the bf16 ring's stages
  constexpr int NB = I8 ? 2 : NS;           // bf16 stages
  constexpr int NS8 = PR_I8_STAGES;
  constexpr int TILE8B = PR_KEYS * D;       // bytes per int8 K (or V) tile
  constexpr int PPM = TILE8B / 1024;        // DMA instructions per int8 matrix and tile
  constexpr int IPW8 = 2 * PPM / 4;         // per wavefront and tile, K and V together
  constexpr int CPR8 = D / 16;              // 16-byte chunks per int8 key row
  constexpr int RPI8 = 1024 / D;            // int8 key rows per DMA instruction
  static_assert(NS8 >= 2 && IPW8 * 4 == 2 * PPM && RPI8 <= 16, "int8 ring");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NB][2][TILEB];
  __shared__ __attribute__((aligned(1024))) uint8_t ring8[I8 ? NS8 : 1][2][I8 ? TILE8B : 16];

  const int kvh = blockIdx.y;
  const int lane = threadIdx.x & (WAVE - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int n = lane & 15, g = lane >> 4;
  const int r = a.tile_req[blockIdx.x], row0 = a.tile_row[blockIdx.x];
  const int tok = a.cu_q[r], Q = a.cu_q[r + 1] - tok, L = a.seq_lens[r];
  const int G = a.G;
  const int* bt = a.block_table + (int64_t)r * a.bt_stride;

  const int wrow0 = row0 + wave * 16 * RB;
  int t[RB], hq[RB], lim[RB];
  bool valid[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int R = wrow0 + 16 * rb + n;
    t[rb] = R / G;
    hq[rb] = kvh * G + R % G;
    valid[rb] = t[rb] < Q;
    lim[rb] = L - Q + 1 + t[rb];
  }
  const int t_last = min(Q - 1, (row0 + PR_ROWS - 1) / G);
  const int kend = max(0, min(L, L - Q + 1 + t_last));
  const int ntiles = (kend + PR_KEYS - 1) / PR_KEYS;
  const int wt0 = wrow0 / G;
  const int lim_lo = L - Q + 1 + wt0;  // smallest limit of the wavefront's rows

  bf16x8 qop[RB][DS];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const uint16_t* qp = a.q + (int64_t)(tok + t[rb]) * a.q_st + (int64_t)hq[rb] * a.q_sh + 8 * g;
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (valid[rb]) w = *reinterpret_cast<const u32x4*>(qp + 32 * s);
      qop[rb][s] = *reinterpret_cast<bf16x8*>(&w);
    }
  }
  // FOLD: q' = bf16(q x k_scale) per channel (lane (n, g) holds channels 32 s + 8 g .. + 7), so that
  // q' . code = q . (code x k_scale) up to that one rounding
  if constexpr (FOLD) {
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      float sc[8];
      if (a.ks_pc) {
        const float4 f0 = *reinterpret_cast<const float4*>(a.ks + kvh * D + 32 * s + 8 * g);
        const float4 f1 = *reinterpret_cast<const float4*>(a.ks + kvh * D + 32 * s + 8 * g + 4);
        sc[0] = f0.x; sc[1] = f0.y; sc[2] = f0.z; sc[3] = f0.w; sc[4] = f1.x; sc[5] = f1.y; sc[6] = f1.z; sc[7] = f1.w;
      } else {
        const float v = a.ks[kvh];
#pragma unroll
        for (int e = 0; e < 8; ++e) sc[e] = v;
      }
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int e = 0; e < 8; ++e) qop[rb][s][e] = (__bf16)((float)qop[rb][s][e] * sc[e]);
    }
  }

  // ---- DMA of tile c into ring stage st: wavefront w's instruction i fills key rows
  // RPI * (IPW * w + i) .. + RPI - 1 of each matrix, lane l the physical chunk l % CH of row l / CH.
  // Those RPI rows lie in one page (32-key tiles start at multiples of 32, block size >= 16), so
  // the instruction's page and row are a scalar base and the lane's offset from it (row, swizzled
  // chunk) is fixed for the launch: an SGPR base plus a VGPR offset, no per-lane address arithmetic.
  // Rows past the last key read rows of a valid page; the causal mask drops them. ----
  const int bsm = (1 << a.lbs) - 1;
  uint32_t kvo[IPW], vvo[IPW];   // byte offsets of the lane's chunk from its instruction's first row
  uint32_t kro[IPW], vro[IPW];   // byte offsets of the instruction's first row from its half-tile's first
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int lr = lane / CH, row = RPI * (IPW * wave + i) + lr;
    kvo[i] = (uint32_t)(2 * lr * a.k_sn + 16 * ((lane % CH) ^ kswz(row)));
    vvo[i] = (uint32_t)(2 * lr * a.v_sn + 16 * ((lane % CH) ^ vswz(row)));
    const uint32_t r0 = RPI * (IPW * wave + i) % 16;
    kro[i] = r0 * a.krow;
    vro[i] = r0 * a.vrow;
  }
  // I8: wavefront w's instruction i is number j = w + 4 i of the tile's 2 PPM: matrix j / PPM (K, V),
  // key rows RPI8 (j % PPM) .. + RPI8 - 1, lane l the 16-byte chunk l % CPR8 of row l / CPR8, landing
  // at byte 16 l of the instruction's 1 KB (the int8 stage is row-major, D bytes per row)
  uint32_t o8[IPW8], r8[IPW8];
#pragma unroll
  for (int i = 0; i < IPW8; ++i) {
    const int j = wave + 4 * i, mat = j / PPM, part = j % PPM;
    o8[i] = (uint32_t)((lane / CPR8) * (mat ? a.v_sn : a.k_sn) + 16 * (lane % CPR8));
    r8[i] = (uint32_t)(RPI8 * part % 16) * (mat ? a.vrow : a.krow);
  }
  const char* kh = I8 ? (const char*)a.kc + (int64_t)kvh * a.k_sh : (const char*)(a.kc + (int64_t)kvh * a.k_sh);
  const char* vh = I8 ? (const char*)a.vc + (int64_t)kvh * a.v_sh : (const char*)(a.vc + (int64_t)kvh * a.v_sh);
  // Pages as one run: when the pages the workgroup reads are consecutive ids p_0, p_0 + 1, ... and a
  // page is bs slots (the layout dequant_pages writes), key k is slot p_0 bs + k of the head's cache:
  // the tiles' addresses need no block-table read (checked once, by every wavefront alike).
  bool linear = false;
  int pfirst = 0;
  if (ntiles > 0 && a.contig) {
    const int npg = ((kend - 1) >> a.lbs) + 1;
    pfirst = __builtin_amdgcn_readfirstlane(((const __attribute__((address_space(4))) int*)bt)[0]);
    bool bad = pfirst < 0 || pfirst > a.num_blocks - npg;
    for (int j = lane; j < npg && !bad; j += WAVE) bad = bt[j] != pfirst + j;
    linear = !__any(bad);
  }
  const char* klin = kh + (uint64_t)(uint32_t)pfirst * a.kpage;
  const char* vlin = vh + (uint64_t)(uint32_t)pfirst * a.vpage;
  // tile c: keys 0..15 sit in page p0 from slot (32 c) mod bs on, keys 16..31 right after them
  // (bs >= 32) or from slot 0 of page p1 (bs == 16); rows past the last key read a valid page
  // lin_t: std::true_type = the pages are one run (no block-table read), false_type = read the
  // table, bool = decide at run time
  auto issue = [&](int c, int st, auto lin_t) {
    c = min(c, max(ntiles - 1, 0));  // past the end: reload the last tile into the free stage
    const int kb0 = c * PR_KEYS, klast = max(kend - 1, 0);
    const char* kb[2];
    const char* vb[2];
    bool lin;
    if constexpr (std::is_same_v<decltype(lin_t), bool>) lin = lin_t;
    else lin = decltype(lin_t)::value;
    if (lin) {
      // the upper half as below: past the last page (bs == 16) it re-reads the lower half's page
      const uint32_t k1 = ((min(kb0 + 16, klast) >> a.lbs) << a.lbs) + ((kb0 + 16) & bsm);
      kb[0] = klin + (uint32_t)kb0 * a.krow;
      vb[0] = vlin + (uint32_t)kb0 * a.vrow;
      kb[1] = klin + k1 * a.krow;
      vb[1] = vlin + k1 * a.vrow;
    } else {
      const int i0 = kb0 >> a.lbs, i1 = min(kb0 + 16, klast) >> a.lbs;
      int p0 = __builtin_amdgcn_readfirstlane(((const __attribute__((address_space(4))) int*)bt)[i0]);
      int p1 = __builtin_amdgcn_readfirstlane(((const __attribute__((address_space(4))) int*)bt)[i1]);
      p0 = (p0 >= 0 && p0 < a.num_blocks) ? p0 : 0;
      p1 = (p1 >= 0 && p1 < a.num_blocks) ? p1 : 0;
      const uint32_t s0 = kb0 & bsm, s1 = (kb0 + 16) & bsm;
      // 32 x 32 -> 64-bit page offsets, 32-bit slot offsets
      kb[0] = kh + ((uint64_t)(uint32_t)p0 * a.kpage + s0 * a.krow);
      kb[1] = kh + ((uint64_t)(uint32_t)p1 * a.kpage + s1 * a.krow);
      vb[0] = vh + ((uint64_t)(uint32_t)p0 * a.vpage + s0 * a.vrow);
      vb[1] = vh + ((uint64_t)(uint32_t)p1 * a.vpage + s1 * a.vrow);
    }
    if constexpr (I8) {
#pragma unroll
      for (int i = 0; i < IPW8; ++i) {
        const int j = wave + 4 * i, mat = j / PPM, part = j % PPM;  // uniform
        const int half = RPI8 * part >= 16;
        const char* b = (mat ? vb[half] : kb[half]) + r8[i];
        asm volatile("" : "+s"(b));
        asm volatile("" : "+v"(o8[i]));
        __builtin_amdgcn_global_load_lds((const void*)(b + (uint64_t)o8[i]),
                                         (__attribute__((address_space(3))) void*)(ring8[st][mat] + 1024 * part), 16, 0, 0);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int half = RPI * (IPW * wave + i) >= 16;  // uniform
      // the instruction's first row, kept opaque so that the address stays an SGPR base plus the
      // lane's 32-bit offset (global_load_lds's saddr form)
      const char* kr = kb[half] + kro[i];
      const char* vr = vb[half] + vro[i];
      asm volatile("" : "+s"(kr), "+s"(vr));
      // the lane's offsets, too, are re-declared here: hoisted out of the tile loop as 64-bit values
      // (a different block), they made every address a 64-bit VGPR addition instead of the saddr form
      asm volatile("" : "+v"(kvo[i]), "+v"(vvo[i]));
      __builtin_amdgcn_global_load_lds((const void*)(kr + (uint64_t)kvo[i]),
                                       (__attribute__((address_space(3))) void*)(ring[st][0] + 1024 * (IPW * wave + i)), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(vr + (uint64_t)vvo[i]),
                                       (__attribute__((address_space(3))) void*)(ring[st][1] + 1024 * (IPW * wave + i)), 16, 0, 0);
    }
  };
  // V^T transposing reads: this lane supplies the address of row vr0 = 4 g + n / 4 (keys 0..15 half) and
  // vr0 + 16 (the other half: +16 rows = immediate offset), element chunk n % 4 of channel tile tt. With
  // V's swizzle (chunk c of row r at c ^ (2 r % CH)) that is byte 32 (tt ^ (vr0 % 8)) + 16 (n % 4 / 2)
  // + 8 (n % 2) of the row (D = 128; D = 64 the same with CH = 8).
  static_assert(CH == 16 || CH == 8, "head_dim 128 or 64");
  const int vr0 = 4 * g + n / 4;
  const uint32_t ring0 = (uint32_t)(uintptr_t)(&ring[0][0][0]);
  uint32_t vadr[VT];  // stage 0's V^T read addresses; stage st adds st * 2 * TILEB
#pragma unroll
  for (int tt = 0; tt < VT; ++tt)
    vadr[tt] = ring0 + TILEB + vr0 * ROWB + 16 * ((2 * tt + ((n % 4) >> 1)) ^ vswz(vr0)) + 8 * (n & 1);
  // stage 0's K operand read addresses of key row n, chunks 4 s + g; row 16 + n has the same swizzle
  // (row % CH, and CH divides 16), so its reads are the immediate offset 16 * ROWB away
  static_assert(16 % CH == 0, "rows n and 16 + n share their swizzle");
  uint32_t kadr[DS];
#pragma unroll
  for (int s = 0; s < DS; ++s) kadr[s] = ring0 + n * ROWB + 16 * ((4 * s + g) ^ kswz(n));
  // A ring stage is a run-time int (its byte offset added to the LDS read addresses) or a
  // std::integral_constant (the offset goes into the reads' immediate field: no VALU per tile).
  auto stage_vofs = [](auto st_t) -> uint32_t {
    if constexpr (std::is_same_v<decltype(st_t), int>) return (uint32_t)(st_t * 2 * TILEB);
    else return 0u;
  };
  auto stage_iofs = [](auto st_t) -> int {
    if constexpr (std::is_same_v<decltype(st_t), int>) return 0;
    else return decltype(st_t)::value * 2 * TILEB;
  };

  // ---- I8: conversion of a tile's codes into a bf16 stage by the whole workgroup. Thread x takes the
  // 8-channel chunk cc = x % CH of key rows x / CH + CR i (i < NPT), K and V, the 8 channels' scales in
  // registers; a value is (bf16)(code * scale), as dequant_pages computes it, so the MFMAs see the
  // operands the two-kernel path gives them. A half-wavefront's 8-byte reads cover 256 contiguous
  // bytes and a quarter-wavefront's 16-byte writes one bf16 row (its chunks permuted): no bank
  // conflicts. Rows x / CH and x / CH + CR share their swizzles (CR is a multiple of CH). ----
  constexpr int CR = 256 / CH;
  constexpr int NPT = PR_KEYS / CR;  // rows per thread: 2 (D 128) or 1 (D 64)
  static_assert(CR % CH == 0 && NPT * CR == PR_KEYS, "conversion share");
  // !FOLD: the kv head's scales in LDS, K then V (a per-head scale repeated), read with the codes
  // (registers for them would cost the kernel its third workgroup per CU). Channel 8 c + 4 h + e sits
  // at float (D / 2) h + 4 c + e of its matrix's D: a quarter-wavefront's 16-byte reads of the first
  // (or second) four scales of 16 chunks are 256 contiguous bytes (no bank conflicts).
  __shared__ __attribute__((aligned(16))) float scl[I8 && !FOLD ? 2 * D : 4];
  uint32_t cra = 0, cwk = 0, cwv = 0, csa = 0;  // int8 stage 0 read, bf16 stage 0 writes, scales
  if constexpr (I8) {
    const int cc = threadIdx.x % CH, crow = threadIdx.x / CH;
    if constexpr (!FOLD) {
      for (int i = threadIdx.x; i < 2 * D; i += 256) {  // before any DMA; the prologue's barrier publishes it
        const bool v = i >= D;
        const int ch = i % D;
        const float* sp = v ? a.vs : a.ks;
        scl[(v ? D : 0) + (D / 2) * ((ch >> 2) & 1) + 4 * (ch >> 3) + (ch & 3)] =
            (v ? a.vs_pc : a.ks_pc) ? sp[kvh * D + ch] : sp[kvh];
      }
      csa = (uint32_t)(uintptr_t)(&scl[0]) + 16 * cc;
    }
    cra = (uint32_t)(uintptr_t)(&ring8[0][0][0]) + crow * D + 8 * cc;
    cwk = ring0 + crow * ROWB + 16 * (cc ^ kswz(crow));
    cwv = ring0 + TILEB + crow * ROWB + 16 * (cc ^ vswz(crow));
  }
  auto stage8_vofs = [](auto st_t) -> uint32_t {
    if constexpr (std::is_same_v<decltype(st_t), int>) return (uint32_t)(st_t * 2 * TILE8B);
    else return 0u;
  };
  auto stage8_iofs = [](auto st_t) -> int {
    if constexpr (std::is_same_v<decltype(st_t), int>) return 0;
    else return decltype(st_t)::value * 2 * TILE8B;
  };
  // int8 stage s8 -> bf16 stage sb (each a run-time int or a std::integral_constant)
  auto convert = [&](auto s8_t, auto sb_t) {
    const uint32_t ra = cra + stage8_vofs(s8_t);
    const uint32_t wk = cwk + stage_vofs(sb_t), wv = cwv + stage_vofs(sb_t);
    const int RO = stage8_iofs(s8_t), WO = stage_iofs(sb_t);
    u32x2 kw[NPT], vw[NPT];
    f32x4 sk[2], sv[2];  // !FOLD: the chunk's 8 K and 8 V scales
    if constexpr (!FOLD && NPT == 2) {
      asm volatile(
          "ds_read_b64 %0, %8 offset:%c10\n"
          "ds_read_b64 %1, %8 offset:%c11\n"
          "ds_read_b64 %2, %8 offset:%c12\n"
          "ds_read_b64 %3, %8 offset:%c13\n"
          "ds_read_b128 %4, %9\n"
          "ds_read_b128 %5, %9 offset:%c14\n"
          "ds_read_b128 %6, %9 offset:%c15\n"
          "ds_read_b128 %7, %9 offset:%c16\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(kw[0]), "=&v"(kw[1]), "=&v"(vw[0]), "=&v"(vw[1]), "=&v"(sk[0]), "=&v"(sk[1]), "=&v"(sv[0]),
            "=&v"(sv[1])
          : "v"(ra), "v"(csa), "i"(RO), "i"(RO + CR * D), "i"(RO + TILE8B), "i"(RO + TILE8B + CR * D), "i"(2 * D),
            "i"(4 * D), "i"(6 * D)
          : "memory");
    } else if constexpr (!FOLD) {
      static_assert(NPT == 1, "rows per thread");
      asm volatile(
          "ds_read_b64 %0, %6 offset:%c8\n"
          "ds_read_b64 %1, %6 offset:%c9\n"
          "ds_read_b128 %2, %7\n"
          "ds_read_b128 %3, %7 offset:%c10\n"
          "ds_read_b128 %4, %7 offset:%c11\n"
          "ds_read_b128 %5, %7 offset:%c12\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(kw[0]), "=&v"(vw[0]), "=&v"(sk[0]), "=&v"(sk[1]), "=&v"(sv[0]), "=&v"(sv[1])
          : "v"(ra), "v"(csa), "i"(RO), "i"(RO + TILE8B), "i"(2 * D), "i"(4 * D), "i"(6 * D)
          : "memory");
    } else if constexpr (NPT == 2) {
      asm volatile(
          "ds_read_b64 %0, %4 offset:%c5\n"
          "ds_read_b64 %1, %4 offset:%c6\n"
          "ds_read_b64 %2, %4 offset:%c7\n"
          "ds_read_b64 %3, %4 offset:%c8\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(kw[0]), "=&v"(kw[1]), "=&v"(vw[0]), "=&v"(vw[1])
          : "v"(ra), "i"(RO), "i"(RO + CR * D), "i"(RO + TILE8B), "i"(RO + TILE8B + CR * D)
          : "memory");
    } else {
      static_assert(NPT == 1, "rows per thread");
      asm volatile(
          "ds_read_b64 %0, %2 offset:%c3\n"
          "ds_read_b64 %1, %2 offset:%c4\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(kw[0]), "=&v"(vw[0])
          : "v"(ra), "i"(RO), "i"(RO + TILE8B)
          : "memory");
    }
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      u32x4 kb, vb;
      if constexpr (FOLD) {
        kb = cv8(kw[i].x, kw[i].y);
        vb = cv8(vw[i].x, vw[i].y);
      } else {
        float kf[8], vf[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          kf[e] = sk[e / 4][e % 4];
          vf[e] = sv[e / 4][e % 4];
        }
        kb = dq8(kw[i].x, kw[i].y, kf);
        vb = dq8(vw[i].x, vw[i].y, vf);
      }
      asm volatile("ds_write_b128 %0, %1 offset:%c2" : : "v"(wk), "v"(kb), "i"(WO + i * CR * ROWB) : "memory");
      asm volatile("ds_write_b128 %0, %1 offset:%c2" : : "v"(wv), "v"(vb), "i"(WO + i * CR * ROWB) : "memory");
    }
  };

  float m[RB], l[RB];
  f32x4 acc[RB][VT];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m[rb] = -1e30f;
    l[rb] = 0.f;
#pragma unroll
    for (int tt = 0; tt < VT; ++tt) acc[rb][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // ---- per tile: scores (QK) and each row's largest, masked for the keys past a row's limit ----
  f32x4 sc[RB][2];
  float lmax[RB], top[RB];
  // K operand reads from inline assembly, each statement waiting for its own reads: as plain loads
  // the compiler makes them wait for every LDS DMA in flight (it cannot tell they read another ring
  // stage), which would empty the ring every tile
  // mask_t: std::false_type = no key of the tile is past any row's limit; true_type = test when the
  // tile reaches the causal edge of some row of the wavefront
  auto scores = [&](auto st_t, int c, auto mask_t) {
    pr_prio<1>();
    const int n0 = c * PR_KEYS;
    uint32_t ad[DS];
#pragma unroll
    for (int s = 0; s < DS; ++s) ad[s] = kadr[s] + stage_vofs(st_t);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int KOFS = b * 16 * ROWB + stage_iofs(st_t);  // key rows 16 + n: same swizzle, 16 rows on
      bf16x8 kop[DS];
      if constexpr (DS == 4) {
        asm volatile(
            "ds_read_b128 %0, %4 offset:%c8\n"
            "ds_read_b128 %1, %5 offset:%c8\n"
            "ds_read_b128 %2, %6 offset:%c8\n"
            "ds_read_b128 %3, %7 offset:%c8\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(kop[0]), "=&v"(kop[1]), "=&v"(kop[2]), "=&v"(kop[3])
            : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "i"(KOFS)
            : "memory");
      } else {
        static_assert(DS == 2, "head_dim 128 or 64");
        asm volatile(
            "ds_read_b128 %0, %2 offset:%c4\n"
            "ds_read_b128 %1, %3 offset:%c4\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(kop[0]), "=&v"(kop[1])
            : "v"(ad[0]), "v"(ad[1]), "i"(KOFS)
            : "memory");
      }
#pragma unroll
      for (int s = 0; s < DS; ++s)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          sc[rb][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[s], qop[rb][s], s == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : sc[rb][b],
                                                             0, 0, 0);
    }
    pr_prio<0>();
    if (decltype(mask_t)::value && n0 + PR_KEYS > lim_lo) {  // a tile on the causal edge of some row
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (n0 + 16 * b + 4 * g + i >= lim[rb]) sc[rb][b][i] = -INFINITY;
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)  // this lane's largest score of the row in the tile (raw units)
      lmax[rb] = __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(sc[rb][0][0], sc[rb][0][1]), sc[rb][0][2]),
                                 __builtin_fmaxf(__builtin_fmaxf(sc[rb][0][3], sc[rb][1][0]), __builtin_fmaxf(
                                     __builtin_fmaxf(sc[rb][1][1], sc[rb][1][2]), sc[rb][1][3])));
  };
  // the row's largest score of the tile, log2 units (the 4 lanes of a row agree)
  auto row_top = [&]() {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) top[rb] = group4_fmax(lmax[rb]) * a.sm_log2;
  };
  // m is a reference maximum (log2 units) raised only when a score exceeds it by more than PR_SLACK:
  // P = 2^(s c - m) <= 2^PR_SLACK (exact in fp32, in range for bf16), so acc / l are rescaled in a few
  // tiles only -- out of the tile loop below, which therefore never changes acc conditionally.
  auto needs_rescale = [&]() {
    bool any = false;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) any |= top[rb] > m[rb] + PR_SLACK;
    return __any(any);
  };
  auto rescale = [&]() {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const float mnew = top[rb] > m[rb] + PR_SLACK ? top[rb] : m[rb];
      const float alpha = __builtin_amdgcn_exp2f(m[rb] - mnew);
      m[rb] = mnew;
      l[rb] *= alpha;
#pragma unroll
      for (int tt = 0; tt < VT; ++tt) acc[rb][tt] *= alpha;
    }
  };
  auto softmax_pv = [&](auto st_t) {
    const uint32_t so = stage_vofs(st_t);
    const int SOI = stage_iofs(st_t);
    bf16x8 pop[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float p[2][4], psum = 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[b][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[rb][b][i], a.sm_log2, -m[rb]));
          psum += p[b][i];
        }
      l[rb] += psum;
      u32x4 pw;
      pw.x = pack_bf16x2_rne(p[0][0], p[0][1]);
      pw.y = pack_bf16x2_rne(p[0][2], p[0][3]);
      pw.z = pack_bf16x2_rne(p[1][0], p[1][1]);
      pw.w = pack_bf16x2_rne(p[1][2], p[1][3]);
      pop[rb] = *reinterpret_cast<bf16x8*>(&pw);
    }
    // V^T operands (lane (n, g): V[4g + k][16 tt + n] and V[16 + 4g + k][16 tt + n], k = 0..3). The
    // transposing reads are issued from inline assembly, 4 channel tiles per statement, each statement
    // waiting for its own reads: the compiler would otherwise make them wait for every LDS DMA in
    // flight (it cannot tell they read another ring stage), emptying the ring each tile.
    typedef unsigned long long u64;
#pragma unroll
    for (int t0 = 0; t0 < VT; t0 += 4) {
      u64 lo[4], hi[4];
      asm volatile(
          "ds_read_b64_tr_b16 %0, %8 offset:%c12\n"
          "ds_read_b64_tr_b16 %1, %8 offset:%c13\n"
          "ds_read_b64_tr_b16 %2, %9 offset:%c12\n"
          "ds_read_b64_tr_b16 %3, %9 offset:%c13\n"
          "ds_read_b64_tr_b16 %4, %10 offset:%c12\n"
          "ds_read_b64_tr_b16 %5, %10 offset:%c13\n"
          "ds_read_b64_tr_b16 %6, %11 offset:%c12\n"
          "ds_read_b64_tr_b16 %7, %11 offset:%c13\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(lo[0]), "=&v"(hi[0]), "=&v"(lo[1]), "=&v"(hi[1]), "=&v"(lo[2]), "=&v"(hi[2]), "=&v"(lo[3]), "=&v"(hi[3])
          : "v"(vadr[t0] + so), "v"(vadr[t0 + 1] + so), "v"(vadr[t0 + 2] + so), "v"(vadr[t0 + 3] + so), "i"(SOI),
            "i"(SOI + 16 * ROWB)
          : "memory");
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        u32x4 vw = {(uint32_t)lo[u], (uint32_t)(lo[u] >> 32), (uint32_t)hi[u], (uint32_t)(hi[u] >> 32)};
        const bf16x8 vop = *reinterpret_cast<bf16x8*>(&vw);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[rb][t0 + u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[rb], acc[rb][t0 + u], 0, 0, 0);
      }
    }
  };

  if (ntiles > 0) {
    // ring stages of tile c (scur) and of the tile DMA'd while c is computed (snext = stage of c - 1),
    // advanced after each tile (no division in the loop). I8: scur is tile c's bf16 stage (c % 2), s8
    // its int8 stage (c % NS8).
    // the first tiles' DMA; I8: NS8 tiles in flight, tile 0 converted once it has landed
    auto prologue = [&]() {
      if constexpr (I8) {
#pragma unroll
        for (int j = 0; j < NS8; ++j) issue(j, j, linear);
        wait_vm<IPW8 * (NS8 - 1)>();
        lds_barrier();
        convert(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
      } else {
#pragma unroll
        for (int j = 0; j < NS - 1; ++j) issue(j, j, linear);
      }
    };
    prologue();
    int scur = 0, snext = NS - 1, s8 = 0;
    auto next_tile = [&](int c, auto lin_t, auto mask_t) {
      if constexpr (I8) {
        wait_vm<IPW8 * (NS8 - 2)>();  // this wavefront's share of tile c + 1 has landed
        lds_barrier();                // everyone's has, tile c is converted, and the other bf16 stage
                                      // (tile c - 1) and tile c's int8 stage are free again
        issue(c + NS8, s8, lin_t);
      } else {
        wait_vm<2 * IPW * (NS - 2)>();  // this wavefront's share of tile c has landed
        lds_barrier();                  // everyone's share has; stage (c - 1) % NS is free again
        issue(c + NS - 1, snext, lin_t);
      }
      scores(scur, c, mask_t);
    };
    // the same for tile c in stage ST = c % NS (I8: bf16 stage c % 2; the int8 stage too when NS8 is 2,
    // else it is moved on here), known at compile time
    auto next_tile_ct = [&](int c, auto st_t, auto lin_t) {
      constexpr int ST = decltype(st_t)::value;
      if constexpr (I8) {
        wait_vm<IPW8 * (NS8 - 2)>();
        lds_barrier();
        issue(c + NS8, NS8 == 2 ? ST : s8, lin_t);
      } else {
        wait_vm<2 * IPW * (NS - 2)>();
        lds_barrier();
        issue(c + NS - 1, (ST + NS - 1) % NS, lin_t);
      }
      scores(st_t, c, std::false_type{});
      softmax_pv(st_t);
      if constexpr (I8) {  // tile c + 1 into the other bf16 stage
        if constexpr (NS8 == 2) {
          convert(std::integral_constant<int, 1 - ST>{}, std::integral_constant<int, 1 - ST>{});
        } else {
          s8 = s8 == NS8 - 1 ? 0 : s8 + 1;
          convert(s8, std::integral_constant<int, 1 - ST>{});
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // tiles of a round are not interleaved (register pressure)
    };
    // after tile c's softmax and PV (the fewest registers live); I8: tile c + 1 is converted into the
    // other bf16 stage (free since this tile's barrier; its int8 stage landed before that barrier)
    auto advance = [&]() {
      if constexpr (I8) {
        convert(s8 == NS8 - 1 ? 0 : s8 + 1, scur ^ 1);
        scur ^= 1;
        s8 = s8 == NS8 - 1 ? 0 : s8 + 1;
      } else {
        scur = scur == NS - 1 ? 0 : scur + 1;
        snext = snext == NS - 1 ? 0 : snext + 1;
      }
    };
    // Fast pass: tile 0 sets each row's reference maximum (acc is still zero), later tiles only
    // accumulate. P = 2^(s c - m) stays finite and keeps its relative precision as long as no score
    // exceeds the reference by more than 60 (log2 units). Every P is at most its lane's denominator
    // l (a sum of P >= 0), so a lane whose l ends at most 2^60 (and not NaN) saw no such score;
    // any other lane sends the workgroup to the general pass below -- acc is never changed under a
    // condition, which keeps the accumulators in place in registers. The tiles below J have no key
    // past any row's limit; with the page addressing fixed per loop, their loop body is one block
    // of straight-line code.
    const int J = min(ntiles, max(lim_lo, 0) / PR_KEYS);
    auto fast_pass = [&](auto lin_t) {
      next_tile(0, lin_t, std::true_type{});
      row_top();
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) m[rb] = __builtin_fmaxf(top[rb], -1e30f);
      softmax_pv(scur);
      advance();
      int c = 1;
      if constexpr (I8) {
        // unmasked tiles in rounds of 2, tile c in bf16 stage c % 2 (1, 0 from c = 1 on)
        for (; c + 2 <= J; c += 2) {
          next_tile_ct(c, std::integral_constant<int, 1>{}, lin_t);
          next_tile_ct(c + 1, std::integral_constant<int, 0>{}, lin_t);
        }
      } else {
        // unmasked tiles in rounds of NS, tile c in stage c % NS (1, 2, 0 from c = 1 on)
        static_assert(NS == 3, "the rounds below are written for a 3-stage ring");
        for (; c + NS <= J; c += NS) {
          next_tile_ct(c, std::integral_constant<int, 1>{}, lin_t);
          next_tile_ct(c + 1, std::integral_constant<int, 2>{}, lin_t);
          next_tile_ct(c + 2, std::integral_constant<int, 0>{}, lin_t);
        }
      }
      // the run-time stages still hold tile c's: a round moves c by the rings' period
      for (; c < J; ++c) {
        next_tile(c, lin_t, std::false_type{});
        softmax_pv(scur);
        advance();
      }
      for (; c < ntiles; ++c) {
        next_tile(c, lin_t, std::true_type{});
        softmax_pv(scur);
        advance();
      }
    };
    if (linear) fast_pass(std::true_type{});
    else fast_pass(std::false_type{});
    wait_vm<0>();
    bool jump = false;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) jump |= !(l[rb] <= PR_FAST_PSUM_MAX);
    // Rare: a score far above its row's first tile somewhere in the workgroup -- redo the workgroup's
    // tiles with a reference maximum raised (and acc / l rescaled) whenever a score exceeds it by
    // 2^PR_SLACK.
    if (__syncthreads_or(jump)) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        m[rb] = -1e30f;
        l[rb] = 0.f;
#pragma unroll
        for (int tt = 0; tt < VT; ++tt) acc[rb][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      prologue();
      scur = 0;
      snext = NS - 1;
      s8 = 0;
      for (int c = 0; c < ntiles; ++c) {
        next_tile(c, linear, std::true_type{});
        row_top();
        if (needs_rescale()) rescale();
        softmax_pv(scur);
        advance();
      }
      wait_vm<0>();  // the reloads past the end, before the wavefront exits
    }
  }

#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const float lr = group4_sum(l[rb]);
    if (!valid[rb]) continue;
    const float inv = lr > 0.f ? 1.f / lr : 0.f;
    uint16_t* orow = a.out + (int64_t)(tok + t[rb]) * a.o_st + (int64_t)hq[rb] * a.o_sh + 4 * g;
#pragma unroll
    for (int tt = 0; tt < VT; ++tt) {
      f32x4 o = acc[rb][tt] * inv;
      if constexpr (FOLD) {  // channels 16 tt + 4 g + i: the V scales, applied to the output
        if (a.vs_pc) {
          const float4 f = *reinterpret_cast<const float4*>(a.vs + kvh * D + 16 * tt + 4 * g);
          o[0] *= f.x; o[1] *= f.y; o[2] *= f.z; o[3] *= f.w;
        } else {
          o *= a.vs[kvh];
        }
      }
      u32x2 w;
      w.x = pack_bf16x2_rne(o[0], o[1]);
      w.y = pack_bf16x2_rne(o[2], o[3]);
      *reinterpret_cast<u32x2*>(orow + 16 * tt) = w;
    }
  }
}

template <int D>
__global__ __launch_bounds__(256, 3) void prefill_kernel(PrefillArgs a) {
  prefill_body<D, PR_SRC_BF16>(a);
}

// The same attention reading the INT8 pages themselves, in place of dequant_pages + prefill_kernel:
// no temporary bf16 cache (2 x 2 bytes per key, channel and kv head of the long requests). Each tile
// is converted in LDS. PR_SRC_I8: with dequant_pages' arithmetic, so the output is bit-identical to the
// two-kernel path's. PR_SRC_I8_FOLD: codes converted exactly, k_scale folded into q and v_scale applied
// to the output (one rounding of q x k_scale in place of one of code x scale per K and V element).
template <int D, int SRC>
__global__ __launch_bounds__(256, 3) void prefill_i8_kernel(PrefillArgs a) {
  prefill_body<D, SRC>(a);
}

// ------------------------------------------------------------------------------------------------
// Dense-bf16 MFMA probe (instrumentation, no counterpart in the reference): every wavefront runs 8
// independent accumulation chains of v_mfma_f32_16x16x32_bf16 (the prefill kernel's instruction) for
// `iters` rounds, on operands taken from `data` (1,024 16-byte vectors) and rotated every round, so the
// multipliers see changing values as the prefill's do; each lane stores a sum of its accumulators (no
// MFMA is dropped). What it sustains is the dense bf16 rate the box delivers, at the clock its power
// limit allows for such operands: the ceiling the prefill kernel is compared with.
__global__ __launch_bounds__(256) void mfma_probe_kernel(const bf16x8* __restrict__ data, int iters,
                                                         float* __restrict__ out) {
  const int t = threadIdx.x;
  bf16x8 x[4], y[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] = data[(t * 8 + i) & 1023];
    y[i] = data[(t * 8 + 4 + i + blockIdx.x) & 1023];
  }
  f32x4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; it += 4) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[j & 3], y[(j + u) & 3], acc[j], 0, 0, 0);
  }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) sum += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  out[(int64_t)blockIdx.x * 256 + t] = sum;
}

// ------------------------------------------------------------------------------------------------
// Streaming-read probe (instrumentation, no counterpart in the reference): reads n16 16-byte words
// once and stores each lane's XOR of what it read (so no load is dropped). Workgroup b streams the
// b-th contiguous share of the buffer, its wavefronts taking interleaved 1 KB blocks of it with 8
// non-temporal loads in flight per lane -- the way the attention kernel streams its pages. What it
// sustains is what HBM delivers to a read-only stream on the box at hand: the ceiling the decode
// attention kernel is compared with.
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, int64_t n16,
                                                          uint32_t* __restrict__ out) {
  constexpr int DEPTH = 8;
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
  const int64_t share = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t lo = min((int64_t)blockIdx.x * share, n16), hi = min(lo + share, n16);
  uint32_t acc = 0;
  int64_t i = lo + (int64_t)wave * WAVE + lane;
  constexpr int64_t STEP = 4 * WAVE;  // the 4 wavefronts' interleaved 1 KB blocks
  for (; i + (DEPTH - 1) * STEP < hi; i += DEPTH * STEP) {
    u32x4 v[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) v[d] = __builtin_nontemporal_load(p + i + d * STEP);
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) acc ^= v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
  }
  for (; i < hi; i += STEP) {
    const u32x4 a = __builtin_nontemporal_load(p + i);
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

// Streaming read + write probe, no counterpart in the reference: `src` (nr 16-byte chunks) is read
// once and `dst` (nw chunks) written once, in order, each workgroup a contiguous share of both, the
// two streams interleaved in the fixed ratio KR : KW (per round a lane reads KR chunks and writes KW,
// each value a function of what it read). Timed at a kernel's byte mix -- 2 : 1 for the fused cache
// write (bf16 K/V read, int8 codes written), 1 : 2 for page dequantization (int8 read, bf16 written) --
// it gives what a plain stream of that many bytes costs on the box, the floor that kernel is compared
// with.
template <int KR, int KW>
__global__ __launch_bounds__(256) void stream_rw_kernel(const u32x4* __restrict__ src, int64_t nr,
                                                        u32x4* __restrict__ dst, int64_t nw) {
  constexpr int64_t STEP = 256;   // the workgroup's 256 lanes, one chunk each
  const int64_t r0 = nr * blockIdx.x / gridDim.x, r1 = nr * (blockIdx.x + 1) / gridDim.x;
  const int64_t w0 = nw * blockIdx.x / gridDim.x, w1 = nw * (blockIdx.x + 1) / gridDim.x;
  const int64_t rounds = max((r1 - r0 + KR * STEP - 1) / (KR * STEP), (w1 - w0 + KW * STEP - 1) / (KW * STEP));
  uint32_t acc = threadIdx.x;
  for (int64_t rd = 0; rd < rounds; ++rd) {
    u32x4 v[KR];
#pragma unroll
    for (int k = 0; k < KR; ++k) {
      const int64_t i = r0 + (rd * KR + k) * STEP + threadIdx.x;
      v[k] = i < r1 ? __builtin_nontemporal_load(src + i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int k = 0; k < KR; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
#pragma unroll
    for (int k = 0; k < KW; ++k) {
      const int64_t i = w0 + (rd * KW + k) * STEP + threadIdx.x;
      const u32x4 w = v[k % KR];
      if (i < w1) __builtin_nontemporal_store(u32x4{w.x ^ acc, w.y, w.z ^ (uint32_t)k, w.w}, dst + i);
    }
  }
}

// Streaming scatter probe, no counterpart in the reference: the cache write's memory traffic without
// its arithmetic. For tokens t < n whose slot >= 0, each lane reads a 16-byte piece (8 bf16 channels) of
// key row t and of value row t and writes one byte per channel (the bf16's high byte, a byte shuffle)
// to cache row (slot / bs, slot % bs, head) of kc and vc -- the same bytes, addresses and scatter by slot
// as the fused quantize + cache write. Consecutive lanes take consecutive pieces of a row (16-byte
// loads contiguous across the wavefront, 8-byte stores filling whole 128-byte cache rows) and each lane
// keeps SC_TPL tokens in flight; the grid covers n_tokens * pieces lanes.
constexpr int SC_TPL = 4;
__global__ __launch_bounds__(256) void stream_scatter_kernel(
    const uint16_t* __restrict__ key, int64_t key_st, const uint16_t* __restrict__ value, int64_t val_st,
    int8_t* __restrict__ kc, int8_t* __restrict__ vc, int64_t sb, int64_t sn, int64_t sh, int pieces_per_head,
    int pieces, const int64_t* __restrict__ slots, int n_tokens, int lbs, int64_t num_slots) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int c = (int)(gid % pieces);
  const int64_t t0 = gid / pieces * SC_TPL;
  const int h = c / pieces_per_head, cc = c % pieces_per_head;
  u32x4 kw[SC_TPL], vw[SC_TPL];
  int64_t sl[SC_TPL];
#pragma unroll
  for (int i = 0; i < SC_TPL; ++i) {
    const int64_t t = t0 + i;
    sl[i] = t < n_tokens ? slots[t] : -1;
    if (t < n_tokens) {
      kw[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(key + t * key_st) + c);
      vw[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(value + t * val_st) + c);
    }
  }
#pragma unroll
  for (int i = 0; i < SC_TPL; ++i) {
    if (sl[i] < 0 || sl[i] >= num_slots) continue;
    const int64_t off = (sl[i] >> lbs) * sb + (sl[i] & ((1 << lbs) - 1)) * sn + (int64_t)h * sh + 8 * cc;
    const u32x2 kb{__builtin_amdgcn_perm(kw[i].y, kw[i].x, 0x07050301u), __builtin_amdgcn_perm(kw[i].w, kw[i].z, 0x07050301u)};
    const u32x2 vb{__builtin_amdgcn_perm(vw[i].y, vw[i].x, 0x07050301u), __builtin_amdgcn_perm(vw[i].w, vw[i].z, 0x07050301u)};
    __builtin_nontemporal_store(kb, reinterpret_cast<u32x2*>(kc + off));
    __builtin_nontemporal_store(vb, reinterpret_cast<u32x2*>(vc + off));
  }
}

// ------------------------------------------------------------------------------------------------
// Host side: argument checks, launches, error reporting.
// ------------------------------------------------------------------------------------------------
thread_local std::string g_err;
thread_local hipEvent_t g_ev_start = nullptr, g_ev_stop = nullptr;

int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return KVQ_ERR_ARG;
}

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_err = std::string(what) + ": " + hipGetErrorString(e);
    return KVQ_ERR_LAUNCH;
  }
  g_err.clear();
  return KVQ_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
int log2i(int64_t x) {
  int r = 0;
  while ((int64_t(1) << r) < x) ++r;
  return r;
}
// Work units (32-key tiles of one workgroup's streaming) charged per segment for its fixed cost in
// the stream-K partition, per kernel (KVQ_SEG_COST overrides both). Like the other tuning variables,
// read at every call.
int seg_cost_units(bool lds_ring, int v32_key_splits) {
  const int env = [] {
    const char* e = getenv("KVQ_SEG_COST");
    if (!e) return -1;
    const int v = atoi(e);
    return v < 0 ? 0 : (v > 64 ? 64 : v);
  }();
  // verify_kernel with 2 key splits streams a unit (one 32-key tile of the segment) in half the time, so
  // its fixed cost is more units (c3, 3-slot rings: 12 -> 24 units 68.5 -> 66.1 us, 36 units 67.3, 48
  // units 71.3; 2-slot rings: 16 units 65.1-65.3 us, 24 units 66.1-66.9; with the merge's speculative
  // loads, same box: 10, 12, 14, 16, 20 units 59.7, 59.3, 58.6, 59.0, 60.3 us -- a piece's measured fixed
  // cost, prologue + epilogue + the step between pieces, is ~6.5 us, about 10 tiles at 1.35 us per step of
  // 2 tiles; a little more than that balances best, as the plan's first piece of a worker also waits for
  // the plan)
  if (env >= 0) return env;
  if (v32_key_splits == 2) return DEFAULT_SEG_COST_V32_KS2;
  return lds_ring ? DEFAULT_SEG_COST_LDS_RING : DEFAULT_SEG_COST;
}

// slots of the attention's shared LDS ring (KVQ_LDS_PREFETCH: 3, 4 or 6)
int lds_prefetch_depth() {
  const char* e = getenv("KVQ_LDS_PREFETCH");
  const int v = e ? atoi(e) : DEFAULT_LDS_PREFETCH;
  return v <= 3 ? 3 : (v >= 6 ? 6 : 4);
}

// slots of verify_kernel's LDS ring (KVQ_V32_RING: 2, 3 or 4; 2 only with two key splits, where it is
// the fastest on verification batches: 3 or 4 slots took 66.5-67 against 62-64 us on c3)
int v32_ring_depth() {
  const char* e = getenv("KVQ_V32_RING");
  const int v = e ? atoi(e) : DEFAULT_V32_RING;
  return v <= 2 ? 2 : v == 3 ? 3 : 4;
}
// verify_kernel's key splits per workgroup (KVQ_V32_KSPLIT: 1 or 2)
int v32_key_splits() {
  const char* e = getenv("KVQ_V32_KSPLIT");
  const int v = e ? atoi(e) : DEFAULT_V32_KSPLIT;
  return v <= 1 ? 1 : 2;
}

// Register tiles per wavefront in the attention ring (KVQ_PREFETCH overrides the default; d128 is
// instantiated for 2, 3, 4, 6, 8 and d64 for 2, 3, 4 -- other values run depth 4).
int prefetch_depth() {
  const char* e = getenv("KVQ_PREFETCH");
  const int v = e ? atoi(e) : DEFAULT_PREFETCH;
  return v < 2 ? 2 : (v > 8 ? 8 : v);
}

int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return cus;
}

// workgroups of 256 threads of kernel K resident per CU at once (queried once); the environment
// variable `env`, when set to a positive count, overrides it on every call (a tuning and test knob)
template <auto K, int THREADS = QC_BLOCK>
int resident_blocks(const char* env) {
  if (const char* e = getenv(env)) {
    const int v = atoi(e);
    if (v > 0) return v;
  }
  static const int nb = [] {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, K, THREADS, 0) != hipSuccess || v <= 0) v = QC_WAVES;
    return v;
  }();
  return nb;
}

// wavefronts of kernel k resident per CU at once with `threads` per workgroup and `lds` bytes of
// dynamic LDS (queried once per shape); DEFAULT_WAVES_PER_CU if the runtime cannot tell
int resident_waves(const void* k, int threads, size_t lds) {
  static std::mutex mu;
  static std::map<std::tuple<const void*, int, size_t>, int> memo;
  std::lock_guard<std::mutex> guard(mu);
  const auto key = std::make_tuple(k, threads, lds);
  const auto it = memo.find(key);
  if (it != memo.end()) return it->second;
  int nb = 0;
  const int w = (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k, threads, lds) == hipSuccess && nb > 0)
                    ? nb * (threads / WAVE) : DEFAULT_WAVES_PER_CU;
  memo.emplace(key, w);
  return w;
}

// Split partials of kvq_int8_decode_attention_noalloc: [T, Hq, S, D] outputs, then [T, Hq, S] maxima
// and denominators, in the library's own device array (see `scratch` below). 64 MiB holds, e.g.,
// 128 tokens x 28 q heads x 35 splits, or 512 x 28 x 9, at head_dim 128.
constexpr int64_t NOALLOC_SCRATCH_BYTES = 64ll << 20;
constexpr int MAX_DEVICES = 64;
char* scratch_ptr();

int decode_attention(const void* q, int64_t q_st, int64_t q_sh, const int8_t* k_cache, int64_t k_sb, int64_t k_sn,
                     int64_t k_sh, const int8_t* v_cache, int64_t v_sb, int64_t v_sn, int64_t v_sh, int64_t num_blocks,
                     int64_t block_size, int64_t num_kv_heads, int64_t head_dim, void* out, int64_t o_st, int64_t o_sh,
                     const int32_t* cu_seqlens_q, const int32_t* seq_lens, const int32_t* block_table,
                     int64_t bt_stride, int64_t num_seqs, int64_t num_q_heads, const float* k_scale,
                     int64_t k_scale_cols, const float* v_scale, int64_t v_scale_cols, double softmax_scale,
                     float* segm_out, float* segm_max, float* segm_sum, int64_t seg_st, int64_t seg_sh,
                     int64_t num_splits, int64_t segm_rows, int64_t target_waves, int64_t max_query_len, int64_t qmax,
                     int64_t q_group, void* stream);

}  // namespace

// The allocation-free decode attention's split partials. Every GPU the library runs on holds one copy
// for the life of the process; all kvq_int8_decode_attention_noalloc calls on a GPU share it, so calls
// that overlap on one GPU (two streams, two threads) race. Nothing in it needs clearing between calls:
// the attention kernel writes every slot the merge kernel reads in the same call.
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {

// Device address of `scratch` on the current device, looked up once per device with that device
// current (each GPU holds its own copy at its own address; in host code the array's name is only a
// handle for this lookup). nullptr, with the error text set, if the runtime cannot tell.
char* scratch_ptr() {
  static std::mutex mu;
  static char* ptrs[MAX_DEVICES] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
    g_err = "int8_decode_attention_noalloc: no current HIP device";
    return nullptr;
  }
  std::lock_guard<std::mutex> guard(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      g_err = std::string("int8_decode_attention_noalloc: hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
      return nullptr;
    }
    ptrs[dev] = static_cast<char*>(p);
  }
  return ptrs[dev];
}

}  // namespace

extern "C" {

const char* kvq_last_error(void) { return g_err.c_str(); }

}  // extern "C"

namespace {

// Shared by the bf16 (dequant_pages' temporary cache) and the INT8 (the pages themselves) prefill:
// es = bytes per cache element (2 or 1); ks / vs only for the INT8 caches.
int prefill_launch(const char* nm, int es, const void* q, int64_t q_st, int64_t q_sh, const void* k_cache,
                   int64_t k_sb, int64_t k_sn, int64_t k_sh, const void* v_cache, int64_t v_sb, int64_t v_sn,
                   int64_t v_sh, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
                   void* out, int64_t o_st, int64_t o_sh, const int32_t* cu_seqlens_q, const int32_t* seq_lens,
                   const int32_t* block_table, int64_t bt_stride, int64_t num_q_heads, const int32_t* tile_req,
                   const int32_t* tile_row, int64_t num_tiles, int64_t rows_per_tile, double softmax_scale,
                   const float* k_scale, int64_t k_scale_cols, const float* v_scale, int64_t v_scale_cols,
                   int64_t fold_scales, void* stream) {
  if (head_dim != 64 && head_dim != 128) return fail("%s: head_dim must be 64 or 128, got %lld", nm, (long long)head_dim);
  if (block_size < 16 || !pow2(block_size)) return fail("%s: block_size must be a power of two >= 16", nm);
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads || num_kv_heads > 65535)
    return fail("%s: bad head counts Hq=%lld Hkv=%lld", nm, (long long)num_q_heads, (long long)num_kv_heads);
  if (num_tiles < 0 || num_tiles > INT32_MAX || num_blocks > INT32_MAX) return fail("%s: bad sizes", nm);
  if (es == 1 && ((k_scale_cols != 1 && k_scale_cols != head_dim) || (v_scale_cols != 1 && v_scale_cols != head_dim)))
    return fail("%s: scale columns must be 1 or head_dim", nm);
  if (num_tiles == 0) { g_err.clear(); return KVQ_OK; }
  // 16-byte rows: the DMA moves 16-byte chunks (8 bf16 or 16 int8 channels)
  const int64_t ea = 16 / es;
  if (!aligned16(q) || !aligned16(out) || !aligned16(k_cache) || !aligned16(v_cache) || (q_st | q_sh | o_st | o_sh) % 8 ||
      (k_sb | k_sn | k_sh | v_sb | v_sn | v_sh) % ea)
    return fail("%s: rows must be 16-byte aligned (base pointers and strides)", nm);
  if (es == 1 && ((k_scale_cols > 1 && !aligned16(k_scale)) || (v_scale_cols > 1 && !aligned16(v_scale))))
    return fail("%s: per-channel scale tables must be 16-byte aligned", nm);
  if (rows_per_tile != PR_ROWS) return fail("%s: work list tiles must be %d rows", nm, PR_ROWS);
  if (k_sb < 0 || v_sb < 0 || k_sn < 0 || v_sn < 0 || es * k_sb > UINT32_MAX || es * v_sb > UINT32_MAX ||
      es * block_size * k_sn > INT32_MAX || es * block_size * v_sn > INT32_MAX)
    return fail("%s: page too large for 32-bit page / slot offsets", nm);
  PrefillArgs a;
  a.q = (const uint16_t*)q; a.kc = (const uint16_t*)k_cache; a.vc = (const uint16_t*)v_cache; a.out = (uint16_t*)out;
  a.cu_q = cu_seqlens_q; a.seq_lens = seq_lens; a.block_table = block_table; a.tile_req = tile_req; a.tile_row = tile_row;
  a.q_st = q_st; a.q_sh = q_sh; a.o_st = o_st; a.o_sh = o_sh;
  a.k_sb = k_sb; a.k_sn = k_sn; a.k_sh = k_sh; a.v_sb = v_sb; a.v_sn = v_sn; a.v_sh = v_sh; a.bt_stride = bt_stride;
  a.sm_log2 = (float)(softmax_scale * 1.4426950408889634);
  a.G = (int)(num_q_heads / num_kv_heads); a.lbs = log2i(block_size); a.num_blocks = (int)num_blocks;
  a.kpage = (uint32_t)(es * k_sb); a.vpage = (uint32_t)(es * v_sb);
  a.krow = (uint32_t)(es * k_sn); a.vrow = (uint32_t)(es * v_sn);
  a.contig = (k_sb == block_size * k_sn && v_sb == block_size * v_sn) ? 1 : 0;
  a.ks = k_scale; a.vs = v_scale; a.ks_pc = k_scale_cols > 1; a.vs_pc = v_scale_cols > 1;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)num_tiles, (unsigned)num_kv_heads);
  if (es == 1 && fold_scales) {
    if (head_dim == 128) hipLaunchKernelGGL((prefill_i8_kernel<128, PR_SRC_I8_FOLD>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((prefill_i8_kernel<64, PR_SRC_I8_FOLD>), grid, dim3(256), 0, st, a);
  } else if (es == 1) {
    if (head_dim == 128) hipLaunchKernelGGL((prefill_i8_kernel<128, PR_SRC_I8>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((prefill_i8_kernel<64, PR_SRC_I8>), grid, dim3(256), 0, st, a);
  } else {
    if (head_dim == 128) hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(prefill_kernel<64>, grid, dim3(256), 0, st, a);
  }
  return launched(nm);
}

}  // namespace

extern "C" {

int kvq_paged_prefill_attention(const void* q, int64_t q_st, int64_t q_sh, const void* k_cache, int64_t k_sb,
                                int64_t k_sn, int64_t k_sh, const void* v_cache, int64_t v_sb, int64_t v_sn,
                                int64_t v_sh, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
                                int64_t head_dim, void* out, int64_t o_st, int64_t o_sh,
                                const int32_t* cu_seqlens_q, const int32_t* seq_lens, const int32_t* block_table,
                                int64_t bt_stride, int64_t num_q_heads, const int32_t* tile_req,
                                const int32_t* tile_row, int64_t num_tiles, int64_t rows_per_tile,
                                double softmax_scale, void* stream) {
  return prefill_launch("paged_prefill_attention", 2, q, q_st, q_sh, k_cache, k_sb, k_sn, k_sh, v_cache, v_sb, v_sn,
                        v_sh, num_blocks, block_size, num_kv_heads, head_dim, out, o_st, o_sh, cu_seqlens_q,
                        seq_lens, block_table, bt_stride, num_q_heads, tile_req, tile_row, num_tiles, rows_per_tile,
                        softmax_scale, nullptr, 1, nullptr, 1, 0, stream);
}

int kvq_int8_prefill_attention(const void* q, int64_t q_st, int64_t q_sh, const int8_t* k_cache, int64_t k_sb,
                               int64_t k_sn, int64_t k_sh, const int8_t* v_cache, int64_t v_sb, int64_t v_sn,
                               int64_t v_sh, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
                               int64_t head_dim, void* out, int64_t o_st, int64_t o_sh,
                               const int32_t* cu_seqlens_q, const int32_t* seq_lens, const int32_t* block_table,
                               int64_t bt_stride, int64_t num_q_heads, const int32_t* tile_req,
                               const int32_t* tile_row, int64_t num_tiles, int64_t rows_per_tile,
                               double softmax_scale, const float* k_scale, int64_t k_scale_cols,
                               const float* v_scale, int64_t v_scale_cols, int64_t fold_scales, void* stream) {
  if (fold_scales != 0 && fold_scales != 1) return fail("int8_prefill_attention: fold_scales must be 0 or 1");
  return prefill_launch("int8_prefill_attention", 1, q, q_st, q_sh, k_cache, k_sb, k_sn, k_sh, v_cache, v_sb, v_sn,
                        v_sh, num_blocks, block_size, num_kv_heads, head_dim, out, o_st, o_sh, cu_seqlens_q,
                        seq_lens, block_table, bt_stride, num_q_heads, tile_req, tile_row, num_tiles, rows_per_tile,
                        softmax_scale, k_scale, k_scale_cols, v_scale, v_scale_cols, fold_scales, stream);
}

int kvq_set_attention_events(void* start, void* stop) {
  g_ev_start = reinterpret_cast<hipEvent_t>(start);
  g_ev_stop = reinterpret_cast<hipEvent_t>(stop);
  return KVQ_OK;
}

int kvq_mfma_probe(const void* data, int64_t iters, float* out, int64_t workgroups, void* stream) {
  if (!data || !out || !aligned16(data) || iters < 4 || iters % 4 || iters > INT32_MAX || workgroups < 1 ||
      workgroups > INT32_MAX / 256)
    return fail("mfma_probe: need 16 KB of 16-byte aligned bf16 data, iters a positive multiple of 4, 1..2^23 workgroups");
  hipLaunchKernelGGL(mfma_probe_kernel, dim3((unsigned)workgroups), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const bf16x8*>(data), (int)iters, out);
  return launched("mfma_probe");
}

int kvq_stream_read(const void* data, int64_t bytes, uint32_t* out, int64_t workgroups, void* stream) {
  if (!data || !out || bytes < 16 || bytes % 16 || !aligned16(data) || workgroups < 1 || workgroups > INT32_MAX / 256)
    return fail("stream_read: need a 16-byte aligned buffer of a positive multiple of 16 bytes and 1..2^23 workgroups");
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)workgroups), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const u32x4*>(data), bytes / 16, out);
  return launched("stream_read");
}

int kvq_stream_rw(const void* src, int64_t read_bytes, void* dst, int64_t write_bytes, int64_t workgroups,
                  void* stream) {
  if (!src || !dst || read_bytes < 16 || write_bytes < 16 || read_bytes % 16 || write_bytes % 16 || !aligned16(src) ||
      !aligned16(dst) || workgroups < 1 || workgroups > INT32_MAX / 256)
    return fail("stream_rw: need 16-byte aligned buffers of positive multiples of 16 bytes and 1..2^23 workgroups");
  const int64_t nr = read_bytes / 16, nw = write_bytes / 16;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)workgroups), block(256);
  const u32x4* s = reinterpret_cast<const u32x4*>(src);
  u32x4* d = reinterpret_cast<u32x4*>(dst);
  if (nr == 2 * nw) hipLaunchKernelGGL((stream_rw_kernel<4, 2>), grid, block, 0, st, s, nr, d, nw);
  else if (2 * nr == nw) hipLaunchKernelGGL((stream_rw_kernel<2, 4>), grid, block, 0, st, s, nr, d, nw);
  else if (nr == nw) hipLaunchKernelGGL((stream_rw_kernel<4, 4>), grid, block, 0, st, s, nr, d, nw);
  else return fail("stream_rw: read : write must be 2 : 1, 1 : 1 or 1 : 2 (got %lld : %lld bytes)", (long long)read_bytes,
                   (long long)write_bytes);
  return launched("stream_rw");
}

int kvq_stream_scatter(const void* key, int64_t key_st, int64_t key_sh, const void* value, int64_t val_st,
                       int64_t val_sh, int8_t* k_cache, int8_t* v_cache, int64_t c_sb, int64_t c_sn, int64_t c_sh,
                       const int64_t* slot_mapping, int64_t n_tokens, int64_t num_heads, int64_t head_dim,
                       int64_t num_blocks, int64_t block_size, void* stream) {
  if (head_dim != 64 && head_dim != 128) return fail("stream_scatter: head_dim must be 64 or 128");
  if (n_tokens < 0 || n_tokens > INT32_MAX || num_heads <= 0 || !pow2(block_size)) return fail("stream_scatter: bad sizes");
  if (n_tokens == 0) { g_err.clear(); return KVQ_OK; }
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return fail("stream_scatter: null pointer");
  if (key_sh != head_dim || val_sh != head_dim || !aligned16(key) || !aligned16(value) || (key_st | val_st) % 8 ||
      ((uintptr_t)k_cache | (uintptr_t)v_cache | c_sb | c_sn | c_sh) % 8)
    return fail("stream_scatter: key / value rows [T, H, D] with contiguous heads, 16-byte aligned; 8-byte aligned caches");
  const int pph = (int)(head_dim / 8), pieces = (int)(num_heads * pph);
  const int64_t lanes = (n_tokens + SC_TPL - 1) / SC_TPL * pieces;
  if (lanes / 256 + 1 > INT32_MAX) return fail("stream_scatter: too many tokens");
  hipLaunchKernelGGL(stream_scatter_kernel, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), (const uint16_t*)key, key_st, (const uint16_t*)value, val_st,
                     k_cache, v_cache, c_sb, c_sn, c_sh, pph, pieces, slot_mapping, (int)n_tokens, log2i(block_size),
                     num_blocks * block_size);
  return launched("stream_scatter");
}

int kvq_abi_version(void) { return 11; }

int kvq_prefill_rows_per_tile(void) { return PR_ROWS; }

int kvq_quant_cache(const void* key, int64_t key_st, int64_t key_sh, const void* value, int64_t val_st,
                    int64_t val_sh, int8_t* k_cache, int64_t kc_sb, int64_t kc_sn, int64_t kc_sh, int8_t* v_cache,
                    int64_t vc_sb, int64_t vc_sn, int64_t vc_sh, const int64_t* slot_mapping, int64_t n_tokens,
                    int64_t num_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size,
                    const float* k_scale, int64_t k_scale_cols, const float* v_scale, int64_t v_scale_cols,
                    const float* k_mu, void* stream) {
  if (head_dim != 64 && head_dim != 128) return fail("quant_cache: head_dim must be 64 or 128, got %lld", (long long)head_dim);
  if (n_tokens < 0 || num_heads <= 0) return fail("quant_cache: bad sizes n=%lld H=%lld", (long long)n_tokens, (long long)num_heads);
  if (n_tokens == 0) { g_err.clear(); return KVQ_OK; }
  if (!pow2(block_size)) return fail("quant_cache: block_size must be a power of two, got %lld", (long long)block_size);
  if ((k_scale_cols != 1 && k_scale_cols != head_dim) || (v_scale_cols != 1 && v_scale_cols != head_dim))
    return fail("quant_cache: scale columns must be 1 or head_dim");
  if (!key || !value || !k_cache || !v_cache || !slot_mapping || !k_scale || !v_scale || !k_mu) return fail("quant_cache: null pointer");
  if ((k_scale_cols > 1 && !aligned16(k_scale)) || (v_scale_cols > 1 && !aligned16(v_scale)) || !aligned16(k_mu))
    return fail("quant_cache: per-channel scale tables and k_mu must be 16-byte aligned");
  if (!aligned16(key) || !aligned16(value) || !aligned16(k_cache) || !aligned16(v_cache) || (key_st | key_sh | val_st | val_sh) % 8 ||
      (kc_sb | kc_sn | kc_sh | vc_sb | vc_sn | vc_sh) % 16)
    return fail("quant_cache: rows must be 16-byte aligned (base pointers and strides)");
  if (n_tokens > INT32_MAX) return fail("quant_cache: too many tokens");
  const int H = (int)num_heads;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int lbs = log2i(block_size);
  const int64_t num_slots = num_blocks * block_size;
  const int ks_pc = k_scale_cols > 1, vs_pc = v_scale_cols > 1;
  // byte extents the wavefront-row kernel addresses with 32-bit offsets
  const int64_t key_bytes = 2 * ((n_tokens - 1) * key_st + (num_heads - 1) * key_sh + head_dim);
  const int64_t val_bytes = 2 * ((n_tokens - 1) * val_st + (num_heads - 1) * val_sh + head_dim);
  const int64_t row_bytes = (num_heads - 1) * std::max(kc_sh, vc_sh) + head_dim;
  // KVQ_QC_KERNEL=lanes: the lane kernel wherever a token's lanes fit one workgroup (a test knob)
  const char* qk = getenv("KVQ_QC_KERNEL");
  const bool lanes_only = qk && strcmp(qk, "lanes") == 0 && num_heads * (head_dim / QC_CPL) <= QC_BLOCK;
  if (!lanes_only && (num_heads * head_dim) % (WAVE * QC_CPL) == 0 && std::max({key_bytes, val_bytes, row_bytes}) <= INT32_MAX) {
    // whole wavefronts per token: the wavefront-row kernel; the grid holds a whole number of tokens'
    // wavefronts (wpt) and no more workgroups than are resident at once
    // a workgroup owns one of the token's wpt parts for QC_ROW_BLOCK / WAVE tokens at a time (the grid
    // is a multiple of wpt). Balanced: the fewest tokens per wavefront one resident round allows,
    // then just enough workgroups for n at that count -- a wavefront with fewer tokens than its
    // ring holds still issues (and drops) the rest
    const int wpt = (int)(num_heads * head_dim / (WAVE * QC_CPL));
    const int wpb = QC_ROW_BLOCK / WAVE;
    auto go = [&](auto kern, int resident) {
      const int64_t conc = std::max<int64_t>(1, (int64_t)device_cus() * resident / wpt) * wpb;  // tokens in flight
      const int64_t per = (n_tokens + conc - 1) / conc;                                        // tokens per wavefront
      const int64_t grid = (n_tokens + wpb * per - 1) / (wpb * per) * wpt;
      hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(QC_ROW_BLOCK), 0, st, (const uint16_t*)key, (int)key_st,
                         (int)key_sh, (int)key_bytes, (const uint16_t*)value, (int)val_st, (int)val_sh, (int)val_bytes,
                         k_cache, kc_sb, kc_sn, (int)kc_sh, v_cache, vc_sb, vc_sn, (int)vc_sh, (int)row_bytes,
                         slot_mapping, (int)n_tokens, wpt, num_slots, lbs, k_scale, ks_pc, v_scale, vs_pc, k_mu);
    };
    if (head_dim == 128) go(quant_cache_rows_kernel<128>, resident_blocks<quant_cache_rows_kernel<128>, QC_ROW_BLOCK>("KVQ_QC_WG_PER_CU"));
    else go(quant_cache_rows_kernel<64>, resident_blocks<quant_cache_rows_kernel<64>, QC_ROW_BLOCK>("KVQ_QC_WG_PER_CU"));
    return launched("quant_cache");
  }
  if (num_heads * (head_dim / QC_CPL) > QC_BLOCK) return fail("quant_cache: at most %d heads of dim %lld", (int)(QC_BLOCK * QC_CPL / head_dim), (long long)head_dim);
  const int ipt = H * (int)(head_dim / QC_CPL), tpb = QC_BLOCK / ipt;
  const int64_t want = (n_tokens + tpb - 1) / tpb;
  auto go = [&](auto kern, int resident) {
    // one round of resident workgroups, balanced: the fewest tokens per lane that round allows, then
    // just enough workgroups for n at that count
    const int64_t conc = (int64_t)device_cus() * resident * tpb;   // tokens in flight
    const int64_t per = (n_tokens + conc - 1) / conc;
    const int grid = (int)std::min<int64_t>(want, (n_tokens + tpb * per - 1) / (tpb * per));
    hipLaunchKernelGGL(kern, dim3(grid), dim3(QC_BLOCK), 0, st, (const uint16_t*)key, key_st, key_sh,
                       (const uint16_t*)value, val_st, val_sh, k_cache, kc_sb, kc_sn, kc_sh, v_cache, vc_sb, vc_sn,
                       vc_sh, slot_mapping, (int)n_tokens, H, num_slots, lbs, k_scale, ks_pc, v_scale, vs_pc, k_mu);
  };
  if (head_dim == 128) go(quant_cache_kernel<128>, resident_blocks<quant_cache_kernel<128>>("KVQ_QC_WG_PER_CU"));
  else go(quant_cache_kernel<64>, resident_blocks<quant_cache_kernel<64>>("KVQ_QC_WG_PER_CU"));
  return launched("quant_cache");
}

int kvq_quant_q(const void* q, int64_t q_st, int64_t q_sh, int64_t num_tokens, int64_t num_q_heads,
                int64_t head_dim, const float* k_scale, int64_t num_kv_heads, int64_t k_scale_cols,
                int64_t group, int8_t* q_i8, float* q_scale, void* stream) {
  if (head_dim != 128 || (group != 128 && group != 32)) return fail("standalone q quantization: head_dim 128, group 128 or 32");
  if (num_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads)
    return fail("quant_q: bad head counts Hq=%lld Hkv=%lld", (long long)num_q_heads, (long long)num_kv_heads);
  if (k_scale_cols != 1 && k_scale_cols != head_dim) return fail("quant_q: scale columns must be 1 or head_dim");
  if (num_tokens == 0) { g_err.clear(); return KVQ_OK; }
  if (((uintptr_t)q & 7u) || (q_st | q_sh) % 4) return fail("quant_q: q rows must be 8-byte aligned");
  const int64_t rows = num_tokens * num_q_heads;
  if (rows > INT32_MAX / 2) return fail("quant_q: too many rows");
  const int grid = (int)((rows + 7) / 8);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int G = (int)(num_q_heads / num_kv_heads);
  if (group == 128)
    hipLaunchKernelGGL(quant_q_kernel<128>, dim3(grid), dim3(256), 0, st, (const uint16_t*)q, q_st, q_sh, (int)num_tokens,
                       (int)num_q_heads, G, k_scale, (int)(k_scale_cols > 1), q_i8, q_scale);
  else
    hipLaunchKernelGGL(quant_q_kernel<32>, dim3(grid), dim3(256), 0, st, (const uint16_t*)q, q_st, q_sh, (int)num_tokens,
                       (int)num_q_heads, G, k_scale, (int)(k_scale_cols > 1), q_i8, q_scale);
  return launched("quant_q");
}

int kvq_int8_decode_attention(const void* q, int64_t q_st, int64_t q_sh, const int8_t* k_cache, int64_t k_sb,
                              int64_t k_sn, int64_t k_sh, const int8_t* v_cache, int64_t v_sb, int64_t v_sn,
                              int64_t v_sh, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
                              int64_t head_dim, void* out, int64_t o_st, int64_t o_sh, const int32_t* cu_seqlens_q,
                              const int32_t* seq_lens, const int32_t* block_table, int64_t bt_stride, int64_t num_seqs,
                              int64_t num_q_heads, const float* k_scale, int64_t k_scale_cols, const float* v_scale,
                              int64_t v_scale_cols, double softmax_scale, float* segm_out, float* segm_max,
                              float* segm_sum, int64_t seg_st, int64_t seg_sh, int64_t num_splits,
                              int64_t target_waves, int64_t max_query_len, int64_t qmax, void* stream) {
  return decode_attention(q, q_st, q_sh, k_cache, k_sb, k_sn, k_sh, v_cache, v_sb, v_sn, v_sh, num_blocks, block_size,
                          num_kv_heads, head_dim, out, o_st, o_sh, cu_seqlens_q, seq_lens, block_table, bt_stride,
                          num_seqs, num_q_heads, k_scale, k_scale_cols, v_scale, v_scale_cols, softmax_scale, segm_out,
                          segm_max, segm_sum, seg_st, seg_sh, num_splits, INT32_MAX, target_waves, max_query_len, qmax, 0,
                          stream);
}

int kvq_int8_decode_attention_ex(const void* q, int64_t q_st, int64_t q_sh, const int8_t* k_cache, int64_t k_sb,
                                 int64_t k_sn, int64_t k_sh, const int8_t* v_cache, int64_t v_sb, int64_t v_sn,
                                 int64_t v_sh, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
                                 int64_t head_dim, void* out, int64_t o_st, int64_t o_sh, const int32_t* cu_seqlens_q,
                                 const int32_t* seq_lens, const int32_t* block_table, int64_t bt_stride,
                                 int64_t num_seqs, int64_t num_q_heads, const float* k_scale, int64_t k_scale_cols,
                                 const float* v_scale, int64_t v_scale_cols, double softmax_scale, float* segm_out,
                                 float* segm_max, float* segm_sum, int64_t seg_st, int64_t seg_sh, int64_t num_splits,
                                 int64_t segm_rows, int64_t target_waves, int64_t max_query_len, int64_t qmax,
                                 int64_t q_group, void* stream) {
  if (q_group != 32 && q_group != head_dim)
    return fail("int8_decode_attention_ex: q_group must be 32 or head_dim (%lld), got %lld", (long long)head_dim,
                (long long)q_group);
  if (segm_rows < 0) return fail("int8_decode_attention_ex: segm_rows must be >= 0");
  return decode_attention(q, q_st, q_sh, k_cache, k_sb, k_sn, k_sh, v_cache, v_sb, v_sn, v_sh, num_blocks, block_size,
                          num_kv_heads, head_dim, out, o_st, o_sh, cu_seqlens_q, seq_lens, block_table, bt_stride,
                          num_seqs, num_q_heads, k_scale, k_scale_cols, v_scale, v_scale_cols, softmax_scale, segm_out,
                          segm_max, segm_sum, seg_st, seg_sh, num_splits, segm_rows, target_waves, max_query_len,
                          qmax, q_group == 32 ? 32 : 0, stream);
}

int kvq_int8_decode_attention_noalloc(const void* q, int64_t q_st, int64_t q_sh, int64_t num_tokens,
                                      const int8_t* k_cache, int64_t k_sb, int64_t k_sn, int64_t k_sh,
                                      const int8_t* v_cache, int64_t v_sb, int64_t v_sn, int64_t v_sh,
                                      int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
                                      void* out, int64_t o_st, int64_t o_sh, const int32_t* cu_seqlens_q,
                                      const int32_t* seq_lens, const int32_t* block_table, int64_t bt_stride,
                                      int64_t num_seqs, int64_t num_q_heads, const float* k_scale,
                                      int64_t k_scale_cols, const float* v_scale, int64_t v_scale_cols,
                                      double softmax_scale, int64_t num_splits, int64_t target_waves,
                                      int64_t max_query_len, int64_t qmax, void* stream) {
  if (num_splits < 1 || num_splits > MAX_SPLITS) return fail("int8_decode_attention_noalloc: at most %d split-KV segments", MAX_SPLITS);
  // (the head count is bounded here, before any product of sizes: decode_attention bounds it again)
  if (num_tokens < 0 || num_q_heads <= 0 || num_q_heads > 65535ll * RED_WAVES || (head_dim != 64 && head_dim != 128))
    return fail("int8_decode_attention_noalloc: bad sizes T=%lld Hq=%lld D=%lld", (long long)num_tokens,
                (long long)num_q_heads, (long long)head_dim);
  float *so = nullptr, *sm = nullptr, *ss = nullptr;
  int64_t st_t = 0, st_h = 0;
  if (num_splits > 1) {
    // [T, Hq, S, D] partial outputs, then [T, Hq, S] maxima and [T, Hq, S] denominators: compared by
    // division, so no product of caller sizes can overflow
    const int64_t per_token = num_q_heads * num_splits * (head_dim + 2) * (int64_t)sizeof(float);  // < 2^38
    if (num_tokens > INT32_MAX || num_tokens > (int64_t)NOALLOC_SCRATCH_BYTES / per_token)
      return fail("int8_decode_attention_noalloc: %lld tokens x %lld q heads x %lld splits need %lld bytes per token "
                  "of split partials, more than the library's %lld-byte scratch holds; pass fewer splits (1 needs none)",
                  (long long)num_tokens, (long long)num_q_heads, (long long)num_splits, (long long)per_token,
                  (long long)NOALLOC_SCRATCH_BYTES);
    const int64_t rows = num_tokens * num_q_heads * num_splits;
    char* base = scratch_ptr();
    if (!base) return KVQ_ERR_LAUNCH;  // g_err set by scratch_ptr
    so = reinterpret_cast<float*>(base);
    sm = so + rows * head_dim;
    ss = sm + rows;
    st_t = num_q_heads * num_splits;
    st_h = num_splits;
  }
  return decode_attention(q, q_st, q_sh, k_cache, k_sb, k_sn, k_sh, v_cache, v_sb, v_sn, v_sh, num_blocks, block_size,
                          num_kv_heads, head_dim, out, o_st, o_sh, cu_seqlens_q, seq_lens, block_table, bt_stride,
                          num_seqs, num_q_heads, k_scale, k_scale_cols, v_scale, v_scale_cols, softmax_scale, so, sm,
                          ss, st_t, st_h, num_splits, num_tokens, target_waves, max_query_len, qmax, 0, stream);
}

int kvq_noalloc_scratch_bytes(void) { return (int)NOALLOC_SCRATCH_BYTES; }

}  // extern "C"

namespace {

int decode_attention(const void* q, int64_t q_st, int64_t q_sh, const int8_t* k_cache, int64_t k_sb, int64_t k_sn,
                     int64_t k_sh, const int8_t* v_cache, int64_t v_sb, int64_t v_sn, int64_t v_sh, int64_t num_blocks,
                     int64_t block_size, int64_t num_kv_heads, int64_t head_dim, void* out, int64_t o_st, int64_t o_sh,
                     const int32_t* cu_seqlens_q, const int32_t* seq_lens, const int32_t* block_table,
                     int64_t bt_stride, int64_t num_seqs, int64_t num_q_heads, const float* k_scale,
                     int64_t k_scale_cols, const float* v_scale, int64_t v_scale_cols, double softmax_scale,
                     float* segm_out, float* segm_max, float* segm_sum, int64_t seg_st, int64_t seg_sh,
                     int64_t num_splits, int64_t segm_rows, int64_t target_waves, int64_t max_query_len, int64_t qmax,
                     int64_t q_group, void* stream) {
  if (head_dim != 64 && head_dim != 128) return fail("int8_decode_attention: head_dim must be 64 or 128, got %lld", (long long)head_dim);
  if (block_size < 16 || !pow2(block_size)) return fail("int8_decode_attention: block_size must be a power of two >= 16");
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return fail("int8_decode_attention: bad head counts Hq=%lld Hkv=%lld", (long long)num_q_heads, (long long)num_kv_heads);
  if (num_splits < 1 || num_splits > MAX_SPLITS) return fail("int8_decode_attention: at most %d split-KV segments", MAX_SPLITS);
  if (num_seqs < 0 || max_query_len < 0 || qmax < 1 || target_waves < 0) return fail("int8_decode_attention: bad sizes");
  if (num_seqs == 0) { g_err.clear(); return KVQ_OK; }
  if ((k_scale_cols != 1 && k_scale_cols != head_dim) || (v_scale_cols != 1 && v_scale_cols != head_dim))
    return fail("int8_decode_attention: scale columns must be 1 or head_dim");
  if (num_splits > 1 && segm_rows > 0 && (!segm_out || !segm_max || !segm_sum))
    return fail("int8_decode_attention: split buffers missing");
  if (!aligned16(q) || !aligned16(out) || !aligned16(k_cache) || !aligned16(v_cache) || (q_st | q_sh | o_st | o_sh) % 8 ||
      (k_sb | k_sn | k_sh | v_sb | v_sn | v_sh) % 16 || (segm_out && !aligned16(segm_out)))
    return fail("int8_decode_attention: rows must be 16-byte aligned (base pointers and strides)");
  if ((int64_t)block_size * k_sn > INT32_MAX || 16 * v_sn > INT32_MAX || num_blocks > INT32_MAX)
    return fail("int8_decode_attention: page too large for 32-bit lane offsets");
  const int G = (int)(num_q_heads / num_kv_heads);
  const int64_t maxq = std::min<int64_t>(std::max<int64_t>(max_query_len, 1), qmax);
  const int64_t row_tiles = ((int64_t)G * maxq + 15) / 16;
  const int rt = (int)std::min<int64_t>(MAX_ROW_TILES, row_tiles);
  // key splits fill up to DEFAULT_KSPLIT wavefronts per row tile, within the workgroup's 4
  // (KVQ_KSPLIT overrides, 1: none)
  const char* ks_env = getenv("KVQ_KSPLIT");
  // Without split buffers nothing is cut across workgroups: as many key splits as the workgroup
  // holds then run each segment
  const int ks_max = ks_env ? std::max(1, std::min(MAX_ROW_TILES, atoi(ks_env)))
                            : (num_splits == 1 ? MAX_ROW_TILES : DEFAULT_KSPLIT);
  const int ks = std::max(1, std::min(ks_max, MAX_ROW_TILES / rt));
  // more than 32 rows per (request, kv head): the 32-row wavefronts of verify_kernel (KVQ_ROWS32=0: off)
  // (per-32-channel q scales run there for every row count)
  const bool rows32 = q_group == 32 ||
                      ((int64_t)G * maxq > 32 && !(getenv("KVQ_ROWS32") && atoi(getenv("KVQ_ROWS32")) == 0));
  const int v32ks = rows32 ? v32_key_splits() : 1;
  const int waves = rows32 ? 2 * v32ks : rt * ks;
  if (num_seqs > INT32_MAX - 1 || num_kv_heads > 65535 || (num_q_heads + RED_WAVES - 1) / RED_WAVES > 65535 ||
      (int64_t)G * maxq > INT32_MAX / 2)
    return fail("int8_decode_attention: grid too large");
  AttnArgs a;
  a.q = (const uint16_t*)q; a.kc = k_cache; a.vc = v_cache; a.out = (uint16_t*)out;
  a.segm_out = segm_out; a.segm_max = segm_max; a.segm_sum = segm_sum;
  a.cu_q = cu_seqlens_q; a.seq_lens = seq_lens; a.block_table = block_table;
  a.ks = k_scale; a.vs = v_scale;
  a.q_st = q_st; a.q_sh = q_sh; a.o_st = o_st; a.o_sh = o_sh;
  a.k_sb = k_sb; a.k_sn = k_sn; a.k_sh = k_sh; a.v_sb = v_sb; a.v_sn = v_sn; a.v_sh = v_sh;
  a.seg_st = seg_st; a.seg_sh = seg_sh; a.bt_stride = bt_stride;
  a.sm_log2 = (float)(softmax_scale * 1.4426950408889634);
  a.num_blocks = (int)num_blocks; a.lbs = log2i(block_size); a.G = G;
  a.qmax = (int)std::min<int64_t>(qmax, INT32_MAX);
  a.ks_pc = k_scale_cols > 1; a.vs_pc = v_scale_cols > 1;
  a.num_seqs = (int)num_seqs; a.hkv = (int)num_kv_heads;
  a.max_splits = (int)num_splits;
  a.cut_rows = num_splits > 1 ? (int)std::min<int64_t>(segm_rows, INT32_MAX) : 0;
  a.rt = rows32 ? V32_GROUP_TILES : rt; a.ksplit = rows32 ? v32ks : ks; a.waves = waves;
  a.min_tiles = MIN_SPLIT_TILES * a.ksplit;
  a.xcd_order = getenv("KVQ_XCD_ORDER") ? atoi(getenv("KVQ_XCD_ORDER")) : 1;
  // KVQ_PLAN_FAST_MAX (tests): a lower bound on units sends the plan's scans down the 64-bit path
  a.plan_fast_max = getenv("KVQ_PLAN_FAST_MAX") ? (int)std::max(1ll, std::min(PLAN_FAST_MAX, atoll(getenv("KVQ_PLAN_FAST_MAX"))))
                                                : (int)PLAN_FAST_MAX;
  // row tiles of the same rows without key splits share each K/V tile through an LDS ring
  // (KVQ_LDS_RING=0: off), of lds_prefetch_depth() slots
  a.lds_ring = (rows32 || (ks == 1 && rt >= 2 && !(getenv("KVQ_LDS_RING") && atoi(getenv("KVQ_LDS_RING")) == 0))) ? 1 : 0;
  a.seg_cost = seg_cost_units(a.lds_ring != 0, rows32 ? v32ks : 0);
  // (verify_kernel has 2-slot rings only with key splits: the instantiated depth sizes the LDS below)
  const int pf = rows32 ? std::max(v32_ring_depth(), v32ks == 2 ? 2 : 3) : a.lds_ring ? lds_prefetch_depth() : prefetch_depth();
  const size_t lds = rows32     ? (size_t)v32_lds_bytes(head_dim, pf, v32ks)
                     : a.lds_ring ? (size_t)pf * 2 * TILE * head_dim
                                  : (size_t)(ks - 1) * rt * MERGE_FIELDS * WAVE * sizeof(float);
  void (*kern)(AttnArgs);
  if (rows32) {
    auto pick = [&](auto qg_t) -> void (*)(AttnArgs) {
      constexpr int QG = decltype(qg_t)::value;
      if (head_dim == 128) {
        if (v32ks == 2)
          return pf == 2 ? verify_kernel<128, 2, QG, 2> : pf == 3 ? verify_kernel<128, 3, QG, 2> : verify_kernel<128, 4, QG, 2>;
        return pf == 3 ? verify_kernel<128, 3, QG, 1> : verify_kernel<128, 4, QG, 1>;
      }
      if (v32ks == 2)
        return pf == 2 ? verify_kernel<64, 2, QG, 2> : pf == 3 ? verify_kernel<64, 3, QG, 2> : verify_kernel<64, 4, QG, 2>;
      return pf == 3 ? verify_kernel<64, 3, QG, 1> : verify_kernel<64, 4, QG, 1>;
    };
    kern = q_group == 32 ? pick(std::integral_constant<int, 32>{}) : pick(std::integral_constant<int, 0>{});
  } else if (a.lds_ring) {
    if (head_dim == 128) kern = pf == 3 ? attn_kernel<128, 3, true> : pf == 6 ? attn_kernel<128, 6, true> : attn_kernel<128, 4, true>;
    else kern = pf == 3 ? attn_kernel<64, 3, true> : pf == 6 ? attn_kernel<64, 6, true> : attn_kernel<64, 4, true>;
  } else if (head_dim == 128) {
    kern = pf == 2 ? attn_kernel<128, 2> : pf == 3 ? attn_kernel<128, 3> : pf == 6 ? attn_kernel<128, 6>
         : pf == 8 ? attn_kernel<128, 8> : attn_kernel<128, 4>;
  } else {
    kern = pf == 2 ? attn_kernel<64, 2> : pf == 3 ? attn_kernel<64, 3> : attn_kernel<64, 4>;
  }
  // Default grid. With split buffers: as many wavefronts as the chosen kernel keeps resident on the
  // device at once (stream-K cuts the segments to even shares). Without (nothing can be cut, every
  // segment runs whole in one workgroup): one workgroup per CU. With more workgroups than CUs the
  // segments land on every other worker or so, and the dispatch order then stacks two busy
  // workgroups on some CUs while others idle, and a long segment shares its CU; one per CU gives each
  // CU an equal run of segments to stream in turn (uniform batches of 1, 2, 2.5 and 3 segments per CU
  // 36%, 1%, 19% and 15% faster, 4 per CU alike, 1.5 per CU 3% slower; c4's decode rows in one pass
  // 405 -> 252 us, c3 in one pass 162 -> 154 us).
  const bool cuttable_any = num_splits > 1 && a.cut_rows > 0;
  const int64_t tw = target_waves > 0 ? target_waves
                   : cuttable_any     ? (int64_t)device_cus() * resident_waves((const void*)kern, WAVE * waves, lds)
                                      : (int64_t)device_cus() * waves;
  a.workers = (int)std::max<int64_t>(1, std::min<int64_t>(tw / waves, INT32_MAX));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)a.workers);
  hipEvent_t ev0 = g_ev_start, ev1 = g_ev_stop;
  g_ev_start = g_ev_stop = nullptr;
  if (ev0) (void)hipEventRecord(ev0, st);
  const dim3 block(WAVE * waves);
  hipLaunchKernelGGL(kern, grid, block, lds, st, a);
  int rc = launched("int8_decode_attention");
  if (ev1) (void)hipEventRecord(ev1, st);
  if (rc != KVQ_OK || num_splits == 1 || a.cut_rows == 0) return rc;
  // the merge's z blocks stride over a request's query tokens (split_reduce_kernel), so any query length
  // is covered with at most MERGE_Z of them
  const dim3 rgrid((unsigned)num_seqs, (unsigned)((num_q_heads + RED_WAVES - 1) / RED_WAVES),
                   (unsigned)std::min<int64_t>(maxq, MERGE_Z));
  if (head_dim == 128) hipLaunchKernelGGL(split_reduce_kernel<128>, rgrid, dim3(WAVE * RED_WAVES), 0, st, a);
  else hipLaunchKernelGGL(split_reduce_kernel<64>, rgrid, dim3(WAVE * RED_WAVES), 0, st, a);
  return launched("split_reduce");
}

}  // namespace

extern "C" {

int kvq_dequant_pages(const int8_t* k_cache, int64_t k_sb, int64_t k_sn, int64_t k_sh, const int8_t* v_cache,
                      int64_t v_sb, int64_t v_sn, int64_t v_sh, int64_t num_blocks, int64_t block_size,
                      int64_t num_heads, int64_t head_dim, void* k_out, void* v_out, const int32_t* block_table,
                      int64_t bt_stride, const int32_t* src_req, const int32_t* src_j, int64_t num_pages,
                      const float* k_scale, int64_t k_scale_cols, const float* v_scale, int64_t v_scale_cols,
                      void* stream) {
  if (head_dim != 64 && head_dim != 128) return fail("dequant_pages: head_dim must be 64 or 128, got %lld", (long long)head_dim);
  if (num_pages < 0 || num_heads <= 0 || block_size <= 0) return fail("dequant_pages: bad sizes");
  if (num_pages == 0) { g_err.clear(); return KVQ_OK; }
  if ((k_scale_cols != 1 && k_scale_cols != head_dim) || (v_scale_cols != 1 && v_scale_cols != head_dim))
    return fail("dequant_pages: scale columns must be 1 or head_dim");
  if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(k_out) || !aligned16(v_out) ||
      (k_sb | k_sn | k_sh | v_sb | v_sn | v_sh) % 16)
    return fail("dequant_pages: rows must be 16-byte aligned (base pointers and strides)");
  if ((k_scale_cols > 1 && !aligned16(k_scale)) || (v_scale_cols > 1 && !aligned16(v_scale)))
    return fail("dequant_pages: per-channel scale tables must be 16-byte aligned");
  if (num_pages > INT32_MAX || num_blocks > INT32_MAX) return fail("dequant_pages: too many pages");
  if (num_heads > 65535 * 4) return fail("dequant_pages: too many heads");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // heads per workgroup: as many as 256 threads' worth of (head, K|V, chunk) combinations; threads: the
  // largest multiple of those combinations up to 256
  const int cph = 2 * (int)head_dim / 8;
  const int hpb = (int)std::min<int64_t>(num_heads, 256 / cph);
  const int combos = hpb * cph;
  const int threads = (256 / combos) * combos;
  const dim3 grid((unsigned)num_pages, (unsigned)((num_heads + hpb - 1) / hpb));
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(threads), 0, st, k_cache, k_sb, k_sn, k_sh, v_cache, v_sb, v_sn, v_sh,
                       (int)num_blocks, (int)block_size, (int)num_heads, hpb, (uint16_t*)k_out, (uint16_t*)v_out,
                       block_table, bt_stride, src_req, src_j, k_scale, (int)(k_scale_cols > 1), v_scale,
                       (int)(v_scale_cols > 1));
  };
  if (head_dim == 128) go(dequant_pages_kernel<128>);
  else go(dequant_pages_kernel<64>);
  return launched("dequant_pages");
}

}  // extern "C"
