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

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <string>

#include "../../include/kvq_int8.h"

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int WAVE = 64;
constexpr int TILE = 32;          // keys per attention tile = P quantization tile
constexpr int MAX_SPLITS = 64;    // split_reduce_kernel keeps one split per lane
constexpr int MAX_ROW_TILES = 4;  // row tiles (wavefronts) per attention workgroup
constexpr int MIN_SPLIT_TILES = 4;  // shortest split: 4 tiles = 128 keys
constexpr int DEFAULT_WAVES_PER_CU = 8;
constexpr int DEFAULT_PREFETCH = 3;

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
// (kvq/quant.py:50-51). r is v_rcp_f32(s) (<= 1 ulp), so q0 = x * r is within |q0| * 2^-22 of
// fl(x / s); when q0 is farther than |q0| * 2^-19 from every half-integer, rint(q0) equals
// rint(fl(x / s)). `bad` is set for the rare element that needs the exact division instead.
// |q0| >= 128 saturates either way.
__device__ __forceinline__ float code_fast(float x, float r, bool& bad) {
  const float q0 = x * r;
  const float n = __builtin_rintf(q0);
  const float aq = __builtin_fabsf(q0);
  bad |= (__builtin_fabsf(q0 - n) >= __builtin_fmaf(aq, -0x1p-19f, 0.5f)) & (aq < 128.f);
  return sat127(n);
}
__device__ __forceinline__ float code_exact(float x, float s) { return sat127(__builtin_rintf(x / s)); }

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
// A wavefront covers whole tokens: each lane owns 8 channels of one head for the whole launch (their
// reciprocal scales and K means stay in registers), so a token's K and V rows are read as 1 KB
// contiguous runs (H = 4, D = 128) and each (token, head) writes its 128-byte K and V code rows with
// 16 consecutive lanes -- the 256-byte K|V run of a slot in vLLM's interleaved layout. Every lane
// issues the loads of QC_UNROLL tokens before converting any of them.
// ------------------------------------------------------------------------------------------------
constexpr int QC_CPL = 8;     // channels per lane
constexpr int QC_UNROLL = 4;  // tokens per lane and step
constexpr int QC_BLOCK = 256;

// Codes of 8 channels (one 16-byte bf16 run) packed little endian into 2 dwords; K subtracts mu.
// Fast path with v_rcp reciprocals; a lane whose quotient lies near a rounding boundary redoes its
// 8 channels with IEEE division (scales re-read from memory).
template <bool SUB_MU>
__device__ __forceinline__ u32x2 quant8(u32x4 w, const float (&r)[QC_CPL], const float (&mu)[QC_CPL],
                                        const float* __restrict__ s, int s_pc) {
  float x[QC_CPL], c[QC_CPL];
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
  bool bad = false;
#pragma unroll
  for (int e = 0; e < QC_CPL; ++e) c[e] = code_fast(x[e], r[e], bad);
  if (bad) {
#pragma unroll
    for (int e = 0; e < QC_CPL; ++e) c[e] = code_exact(x[e], s[s_pc ? e : 0]);
  }
  return u32x2{pack_i8x4(c[0], c[1], c[2], c[3]), pack_i8x4(c[4], c[5], c[6], c[7])};
}

template <int D>
__global__ __launch_bounds__(QC_BLOCK) void quant_cache_kernel(
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
  const float* ksp = ks + (ks_pc ? h * D + d0 : h);
  const float* vsp = vs + (vs_pc ? h * D + d0 : h);
  float kr[QC_CPL], vr[QC_CPL], mu[QC_CPL];
#pragma unroll
  for (int e = 0; e < QC_CPL; ++e) {
    kr[e] = __builtin_amdgcn_rcpf(ksp[ks_pc ? e : 0]);
    vr[e] = __builtin_amdgcn_rcpf(vsp[vs_pc ? e : 0]);
    mu[e] = kmu[h * D + d0 + e];
  }
  const int64_t bmask = (int64_t(1) << lbs) - 1;
  const int stride = gridDim.x * tpb;
  for (int t0 = blockIdx.x * tpb + threadIdx.x / ipt; t0 < n; t0 += QC_UNROLL * stride) {
    int64_t slot[QC_UNROLL];
    u32x4 kin[QC_UNROLL], vin[QC_UNROLL];
#pragma unroll
    for (int u = 0; u < QC_UNROLL; ++u) {
      const int t = t0 + u * stride;
      slot[u] = -1;
      if (t < n) {
        slot[u] = slots[t];
        kin[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(key + t * key_st + h * key_sh + d0));
        vin[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(value + t * val_st + h * val_sh + d0));
      }
    }
#pragma unroll
    for (int u = 0; u < QC_UNROLL; ++u) {
      if (slot[u] < 0 || slot[u] >= num_slots) continue;   // padding (or out of range): skipped
      const int64_t blk = slot[u] >> lbs, off = slot[u] & bmask;
      __builtin_nontemporal_store(quant8<true>(kin[u], kr, mu, ksp, ks_pc),
                                  reinterpret_cast<u32x2*>(kc + blk * kc_sb + off * kc_sn + h * kc_sh + d0));
      __builtin_nontemporal_store(quant8<false>(vin[u], vr, mu, vsp, vs_pc),
                                  reinterpret_cast<u32x2*>(vc + blk * vc_sb + off * vc_sn + h * vc_sh + d0));
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
  const uint16_t* q;
  const int8_t* kc;
  const int8_t* vc;
  uint16_t* out;
  float* segm_out;
  float* segm_max;
  float* segm_sum;
  const int* cu_q;
  const int* seq_lens;
  const int* block_table;
  const float* ks;
  const float* vs;
  int64_t q_st, q_sh, o_st, o_sh, k_sb, k_sn, k_sh, v_sb, v_sn, v_sh, seg_st, seg_sh, bt_stride;
  float sm_log2;      // softmax_scale * log2(e)
  int num_blocks, lbs, G, qmax, ks_pc, vs_pc;
  int num_seqs, hkv;
  int max_splits;     // splits per request in the grid (an upper bound: requests use what they need)
  int row_tiles;      // 16-row tiles of (token, q head) rows per (request, kv head)
  int waves;          // wavefronts per workgroup: consecutive row tiles of one (request, kv head, split)
  int min_tiles;      // shortest split, in 32-key tiles
  int64_t target_waves;  // the batch's tiles are spread over about this many wavefronts
};

// 32-key tiles per split of a request with `ntiles` tiles: at most max_splits splits, and long enough
// that the whole batch (its tiles x kv heads x row tiles) spreads over about target_waves wavefronts,
// never shorter than min_tiles. The attention kernel and the merge both evaluate it (one whole
// wavefront, identical integer arithmetic), so they agree on every request's split count.
__device__ int split_len(const AttnArgs& a, int ntiles, int lane) {
  if (a.max_splits == 1) return ntiles > 0 ? ntiles : 1;
  long long part = 0;
  for (int r = lane; r < a.num_seqs; r += WAVE) part += (a.seq_lens[r] + TILE - 1) / TILE;
#pragma unroll
  for (int o = 32; o; o >>= 1) part += __shfl_xor(part, o, WAVE);
  const long long units = part * a.hkv * a.row_tiles;
  const long long target = (units + a.target_waves - 1) / a.target_waves;
  const int per = (ntiles + a.max_splits - 1) / a.max_splits;
  // the reduction leaves every lane with the same value; say so, so that the loop bounds (and the
  // block-table reads they guard) stay scalar
  return __builtin_amdgcn_readfirstlane(
      (int)std::max<long long>(std::max<long long>(per, target), std::max(a.min_tiles, 1)));
}

// K/V pages are streamed exactly once per launch: the non-temporal hint keeps them from evicting
// what is reused (block tables, q, scales) from L2 and the last-level cache (measured on c2:
// 771 -> 688 us).
__device__ __forceinline__ i32x4 ldk(const i32x4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ u32x2 ldv(const u32x2* p) { return __builtin_nontemporal_load(p); }

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

// One wavefront = one 16-row tile of one (request, kv head, split); a workgroup holds `waves`
// consecutive row tiles of the same (request, kv head, split), which stream the same K/V tiles at
// the same time (the second and later reads hit L1/L2).
template <int D, int PF>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
  constexpr int KPL = D / 4;        // K bytes per lane and key
  constexpr int KSTEPS = D / 64;    // x64 MFMAs per 16-key block
  constexpr int VT = D / 16;        // PV channel tiles = V bytes per lane and key
  constexpr int VW = D / 64;        // V dwords per lane and key
  // the wavefront index is uniform across the wavefront: keep it (and all row bookkeeping) scalar
  const int lane = threadIdx.x & (WAVE - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int n = lane & 15, g = lane >> 4;
  const int seq = blockIdx.x, kvh = blockIdx.y;
  const int split = blockIdx.z % a.max_splits, rg = blockIdx.z / a.max_splits;
  const int tok = a.cu_q[seq], qlen = a.cu_q[seq + 1] - tok;
  const int G = a.G;
  const int row0 = (rg * a.waves + wave) * 16;  // first (token, q head) row of this wavefront
  if (qlen == 0 || qlen > a.qmax || row0 >= qlen * G) return;
  const int L = a.seq_lens[seq];
  const int ntiles = (L + TILE - 1) / TILE;
  const int per = split_len(a, ntiles, lane);
  const int nsplit = ntiles > 0 ? (ntiles + per - 1) / per : 1;
  if (split >= nsplit) return;
  const int c_begin = split * per, c_end = min(ntiles, c_begin + per);
  const int* bt = a.block_table + (int64_t)seq * a.bt_stride;
  const int bs = 1 << a.lbs;

  // ---- q prologue: fold s_k, one scale per row, quantize (exact division) ----
  i32x4 qop[KSTEPS];
  const int R = row0 + n, rtok = R / G, rh = R % G;
  float rs;
  int lim;
  {
    float x[KPL];
    float amax = 0.f;
    if (rtok < qlen) {
      const u32x4* qp = reinterpret_cast<const u32x4*>(a.q + (int64_t)(tok + rtok) * a.q_st +
                                                       (int64_t)(kvh * G + rh) * a.q_sh + g * KPL);
#pragma unroll
      for (int u = 0; u < KPL / 8; ++u) {
        const u32x4 w = qp[u];
        x[8 * u + 0] = bf16_lo(w.x); x[8 * u + 1] = bf16_hi(w.x);
        x[8 * u + 2] = bf16_lo(w.y); x[8 * u + 3] = bf16_hi(w.y);
        x[8 * u + 4] = bf16_lo(w.z); x[8 * u + 5] = bf16_hi(w.z);
        x[8 * u + 6] = bf16_lo(w.w); x[8 * u + 7] = bf16_hi(w.w);
      }
      if (a.ks_pc) {
#pragma unroll
        for (int e = 0; e < KPL; ++e) x[e] = x[e] * a.ks[kvh * D + g * KPL + e];
      }
#pragma unroll
      for (int e = 0; e < KPL; ++e) amax = __builtin_fmaxf(amax, __builtin_fabsf(x[e]));
    } else {
#pragma unroll
      for (int e = 0; e < KPL; ++e) x[e] = 0.f;
    }
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 16, WAVE));
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 32, WAVE));
    const float s = __builtin_fmaxf(amax / 127.f, 1e-8f);
#pragma unroll
    for (int st = 0; st < KSTEPS; ++st) {
      i32x4 w;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = 16 * st + 4 * u;
        w[u] = (int)pack_i8x4(code_exact(x[e], s), code_exact(x[e + 1], s), code_exact(x[e + 2], s),
                              code_exact(x[e + 3], s));
      }
      qop[st] = w;
    }
    rs = s * (a.ks_pc ? 1.f : a.ks[kvh]) * a.sm_log2;
    lim = rtok < qlen ? L - qlen + 1 + rtok : L;  // keys < lim are visible to this row
  }
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
    int p = bt[key >> a.lbs];
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

  auto compute = [&](const KVTile<D>& r, int c) {
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
    // ---- V^T operands: 8x8 byte transpose per channel tile ----
    long vop[VT];
    if constexpr (VW == 2) {
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
    const bool full = n0 + TILE <= lim_lo;  // no key of this tile is masked for any row
    int mx = INT32_MIN;
    bool ok[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ok[b][i] = full || n0 + 16 * b + 4 * g + i < lim;
        mx = ok[b][i] ? max(mx, sc[b][i]) : mx;
      }
    mx = max(mx, __shfl_xor(mx, 16, WAVE));
    mx = max(mx, __shfl_xor(mx, 32, WAVE));
    const float tmax = mx == INT32_MIN ? -INFINITY : (float)mx * rs;
    const float mnew = __builtin_fmaxf(m, tmax);
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);
    m = mnew;
    const float pm = __builtin_amdgcn_exp2f(tmax - mnew);  // max of this tile's P (exp2 is monotone)
    const float ps = __builtin_fmaxf(pm / 127.f, 1e-30f);
    const float ri = __builtin_amdgcn_rcpf(ps);
    float pc[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf((float)sc[b][i], rs, -mnew));
        pc[b][i] = ok[b][i] ? __builtin_fminf(__builtin_rintf(p * ri), 127.f) : 0.f;
      }
    const uint32_t p0 = pack_i8x4(pc[0][0], pc[0][1], pc[0][2], pc[0][3]);
    const uint32_t p1 = pack_i8x4(pc[1][0], pc[1][1], pc[1][2], pc[1][3]);
    const long pop = (long)(((uint64_t)p1 << 32) | p0);
    const float psum = (pc[0][0] + pc[0][1]) + (pc[0][2] + pc[0][3]) + (pc[1][0] + pc[1][1]) + (pc[1][2] + pc[1][3]);
    l = __builtin_fmaf(psum, ps, l * alpha);
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int t = 0; t < VT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] *= alpha;
    }
    // ---- PV: O^T[channel][row] += (V^T . P^T) * ps ----
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
  // in the loop is for exactly the oldest tile. ----
  if (c_begin < c_end) {
    KVTile<D> ring[PF];
    const int c_last = c_end - 1;
#pragma unroll
    for (int j = 0; j < PF - 1; ++j) load(ring[j], min(c_begin + j, c_last));
    for (int c0 = c_begin; c0 < c_end; c0 += PF) {
#pragma unroll
      for (int j = 0; j < PF; ++j) {
        const int c = c0 + j;
        if (c >= c_end) break;
        load(ring[(j + PF - 1) % PF], min(c + PF - 1, c_last));
        compute(ring[j], c);
      }
    }
  }

  // ---- epilogue: lane (n, g) holds channels (D/4) g + (D/16) i + t of row n ----
  l += __shfl_xor(l, 16, WAVE);
  l += __shfl_xor(l, 32, WAVE);
  if (rtok >= qlen) return;
  constexpr int OPL = D / 4;
  const int head = kvh * G + rh;
  const int qt = tok + rtok;
  float vsc[OPL];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < VT; ++t) vsc[VT * i + t] = a.vs_pc ? a.vs[kvh * D + OPL * g + VT * i + t] : a.vs[kvh];
  if (nsplit == 1) {
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
    const int64_t sidx = (int64_t)qt * a.seg_st + (int64_t)head * a.seg_sh + split;
    if (g == 0) {
      a.segm_max[sidx] = m;
      a.segm_sum[sidx] = l;
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

// Merge the split partials of the requests that used more than one split (reference
// kvq/cuda/int8_kv.cu:465-503): o = sum_s 2^(m_s - M) acc_s / max(sum_s 2^(m_s - M) l_s, 1e-30).
// One wavefront per (request, q head, query token); lane s holds split s's weight; lanes own D / 64
// channels each.
template <int D>
__global__ __launch_bounds__(WAVE) void split_reduce_kernel(AttnArgs a) {
  const int seq = blockIdx.x, h = blockIdx.y, r = blockIdx.z, lane = threadIdx.x;
  const int tok = a.cu_q[seq], qlen = a.cu_q[seq + 1] - tok;
  if (qlen == 0 || qlen > a.qmax || r >= qlen) return;
  const int ntiles = (a.seq_lens[seq] + TILE - 1) / TILE;
  const int per = split_len(a, ntiles, lane);
  const int S = ntiles > 0 ? (ntiles + per - 1) / per : 1;
  if (S <= 1) return;  // written directly by the attention kernel
  const int64_t base = (int64_t)(tok + r) * a.seg_st + (int64_t)h * a.seg_sh;
  const float ms = lane < S ? a.segm_max[base + lane] : -INFINITY;
  const float M = wave_max(ms);
  const float w = lane < S ? __builtin_amdgcn_exp2f(ms - M) : 0.f;
  const float den = wave_sum(lane < S ? w * a.segm_sum[base + lane] : 0.f);
  const float inv = 1.f / __builtin_fmaxf(den, 1e-30f);
  constexpr int CPL = D / WAVE;
  float num[CPL];
#pragma unroll
  for (int e = 0; e < CPL; ++e) num[e] = 0.f;
  for (int s = 0; s < S; ++s) {
    const float ws = __shfl(w, s, WAVE);
    const float* p = a.segm_out + (base + s) * D + CPL * lane;
#pragma unroll
    for (int e = 0; e < CPL; ++e) num[e] = __builtin_fmaf(ws, p[e], num[e]);
  }
  uint16_t* op = a.out + (int64_t)(tok + r) * a.o_st + (int64_t)h * a.o_sh + CPL * lane;
  if constexpr (CPL == 2) {
    *reinterpret_cast<uint32_t*>(op) = pack_bf16x2(num[0] * inv, num[1] * inv);
  } else {
    op[0] = (uint16_t)bf16_rne(num[0] * inv);
  }
}

// ------------------------------------------------------------------------------------------------
// Page dequantization for the long-query path (reference kvq/cuda/int8_kv.cu:505-542). Blocks walk
// the output pages with a grid stride; a lane converts 16 channels of one (token, head): a 16-byte
// int8 load, two 16-byte bf16 stores (v_cvt_pk_bf16_f32, round to nearest even). When the lanes of
// a token divide the block, each lane keeps its (head, channels) and their scales for the launch.
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

template <int D>
__global__ __launch_bounds__(256) void dequant_pages_kernel(
    const int8_t* __restrict__ kc, int64_t k_sb, int64_t k_sn, int64_t k_sh, const int8_t* __restrict__ vc,
    int64_t v_sb, int64_t v_sn, int64_t v_sh, int num_blocks, int bs, int H, uint16_t* __restrict__ ko,
    uint16_t* __restrict__ vo, const int* __restrict__ bt, int64_t bt_stride, const int* __restrict__ src_req,
    const int* __restrict__ src_j, int P, const float* __restrict__ ks, int ks_pc, const float* __restrict__ vs,
    int vs_pc) {
  constexpr int CPL = 16, LPR = D / CPL;
  const int ipt = H * LPR;                       // lanes per token
  const int items = bs * ipt;
  const bool fixed = (int)blockDim.x % ipt == 0;  // lane role invariant across items
  float kS[CPL], vS[CPL];
  auto load_scales = [&](int h, int d0) {
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      kS[e] = ks[ks_pc ? h * D + d0 + e : h];
      vS[e] = vs[vs_pc ? h * D + d0 + e : h];
    }
  };
  if (fixed) load_scales((threadIdx.x % ipt) / LPR, (threadIdx.x % LPR) * CPL);
  for (int p = blockIdx.x; p < P; p += gridDim.x) {
    int src = bt[(int64_t)src_req[p] * bt_stride + src_j[p]];
    if (src < 0 || src >= num_blocks) src = 0;
    for (int it = threadIdx.x; it < items; it += blockDim.x) {
      const int c = it % LPR, h = (it / LPR) % H, tkn = it / ipt;
      const int d0 = c * CPL;
      if (!fixed) load_scales(h, d0);
      const u32x4 kr = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kc + (int64_t)src * k_sb + tkn * k_sn + h * k_sh + d0));
      const u32x4 vr = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vc + (int64_t)src * v_sb + tkn * v_sn + h * v_sh + d0));
      const int64_t o = (((int64_t)p * bs + tkn) * H + h) * D + d0;
      __builtin_nontemporal_store(dq8(kr.x, kr.y, kS), reinterpret_cast<u32x4*>(ko + o));
      __builtin_nontemporal_store(dq8(kr.z, kr.w, kS + 8), reinterpret_cast<u32x4*>(ko + o) + 1);
      __builtin_nontemporal_store(dq8(vr.x, vr.y, vS), reinterpret_cast<u32x4*>(vo + o));
      __builtin_nontemporal_store(dq8(vr.z, vr.w, vS + 8), reinterpret_cast<u32x4*>(vo + o) + 1);
    }
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
// Register tiles per wavefront in the attention ring (2..4; KVQ_PREFETCH overrides the default).
int prefetch_depth() {
  static const int depth = [] {
    const char* e = getenv("KVQ_PREFETCH");
    const int v = e ? atoi(e) : DEFAULT_PREFETCH;
    return v < 2 ? 2 : (v > 8 ? 8 : v);
  }();
  return depth;
}

int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return cus;
}


}  // namespace

extern "C" {

const char* kvq_last_error(void) { return g_err.c_str(); }

int kvq_set_attention_events(void* start, void* stop) {
  g_ev_start = reinterpret_cast<hipEvent_t>(start);
  g_ev_stop = reinterpret_cast<hipEvent_t>(stop);
  return KVQ_OK;
}

int kvq_abi_version(void) { return 2; }

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
  if (num_heads * (head_dim / QC_CPL) > QC_BLOCK) return fail("quant_cache: at most %d heads of dim %lld", (int)(QC_BLOCK * QC_CPL / head_dim), (long long)head_dim);
  if ((k_scale_cols != 1 && k_scale_cols != head_dim) || (v_scale_cols != 1 && v_scale_cols != head_dim))
    return fail("quant_cache: scale columns must be 1 or head_dim");
  if (!key || !value || !k_cache || !v_cache || !slot_mapping || !k_scale || !v_scale || !k_mu) return fail("quant_cache: null pointer");
  if (!aligned16(key) || !aligned16(value) || !aligned16(k_cache) || !aligned16(v_cache) || (key_st | key_sh | val_st | val_sh) % 8 ||
      (kc_sb | kc_sn | kc_sh | vc_sb | vc_sn | vc_sh) % 16)
    return fail("quant_cache: rows must be 16-byte aligned (base pointers and strides)");
  if (n_tokens > INT32_MAX) return fail("quant_cache: too many tokens");
  const int H = (int)num_heads;
  const int ipt = H * (int)(head_dim / QC_CPL), tpb = QC_BLOCK / ipt;
  const int64_t want = (n_tokens + (int64_t)tpb * QC_UNROLL - 1) / ((int64_t)tpb * QC_UNROLL);
  const int grid = (int)std::min<int64_t>(want, (int64_t)device_cus() * 16);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int lbs = log2i(block_size);
  const int64_t num_slots = num_blocks * block_size;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(grid), dim3(QC_BLOCK), 0, st, (const uint16_t*)key, key_st, key_sh,
                       (const uint16_t*)value, val_st, val_sh, k_cache, kc_sb, kc_sn, kc_sh, v_cache, vc_sb, vc_sn,
                       vc_sh, slot_mapping, (int)n_tokens, H, num_slots, lbs, k_scale, (int)(k_scale_cols > 1),
                       v_scale, (int)(v_scale_cols > 1), k_mu);
  };
  if (head_dim == 128) go(quant_cache_kernel<128>);
  else go(quant_cache_kernel<64>);
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
  if (head_dim != 64 && head_dim != 128) return fail("int8_decode_attention: head_dim must be 64 or 128, got %lld", (long long)head_dim);
  if (block_size < 16 || !pow2(block_size)) return fail("int8_decode_attention: block_size must be a power of two >= 16");
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return fail("int8_decode_attention: bad head counts Hq=%lld Hkv=%lld", (long long)num_q_heads, (long long)num_kv_heads);
  if (num_splits < 1 || num_splits > MAX_SPLITS) return fail("int8_decode_attention: at most %d split-KV segments", MAX_SPLITS);
  if (num_seqs < 0 || max_query_len < 0 || qmax < 1 || target_waves < 0) return fail("int8_decode_attention: bad sizes");
  if (num_seqs == 0) { g_err.clear(); return KVQ_OK; }
  if ((k_scale_cols != 1 && k_scale_cols != head_dim) || (v_scale_cols != 1 && v_scale_cols != head_dim))
    return fail("int8_decode_attention: scale columns must be 1 or head_dim");
  if (num_splits > 1 && (!segm_out || !segm_max || !segm_sum)) return fail("int8_decode_attention: split buffers missing");
  if (!aligned16(q) || !aligned16(out) || !aligned16(k_cache) || !aligned16(v_cache) || (q_st | q_sh | o_st | o_sh) % 8 ||
      (k_sb | k_sn | k_sh | v_sb | v_sn | v_sh) % 16 || (segm_out && !aligned16(segm_out)))
    return fail("int8_decode_attention: rows must be 16-byte aligned (base pointers and strides)");
  if ((int64_t)block_size * k_sn > INT32_MAX || 16 * v_sn > INT32_MAX || num_blocks > INT32_MAX)
    return fail("int8_decode_attention: page too large for 32-bit lane offsets");
  const int G = (int)(num_q_heads / num_kv_heads);
  const int64_t maxq = std::min<int64_t>(std::max<int64_t>(max_query_len, 1), qmax);
  const int64_t row_tiles = ((int64_t)G * maxq + 15) / 16;
  const int waves = (int)std::min<int64_t>(MAX_ROW_TILES, row_tiles);
  const int64_t row_groups = (row_tiles + waves - 1) / waves;
  if (num_seqs > INT32_MAX || num_kv_heads > 65535 || row_groups * num_splits > 65535)
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
  a.max_splits = (int)num_splits; a.row_tiles = (int)row_tiles; a.waves = waves;
  a.min_tiles = MIN_SPLIT_TILES;
  a.target_waves = target_waves > 0 ? target_waves : (int64_t)device_cus() * DEFAULT_WAVES_PER_CU;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)num_seqs, (unsigned)num_kv_heads, (unsigned)(num_splits * row_groups));
  hipEvent_t ev0 = g_ev_start, ev1 = g_ev_stop;
  g_ev_start = g_ev_stop = nullptr;
  if (ev0) (void)hipEventRecord(ev0, st);
  const dim3 block(WAVE * waves);
  const int pf = prefetch_depth();
  if (head_dim == 128) {
    if (pf == 2) hipLaunchKernelGGL((attn_kernel<128, 2>), grid, block, 0, st, a);
    else if (pf == 3) hipLaunchKernelGGL((attn_kernel<128, 3>), grid, block, 0, st, a);
    else if (pf == 6) hipLaunchKernelGGL((attn_kernel<128, 6>), grid, block, 0, st, a);
    else if (pf == 8) hipLaunchKernelGGL((attn_kernel<128, 8>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((attn_kernel<128, 4>), grid, block, 0, st, a);
  } else {
    if (pf == 2) hipLaunchKernelGGL((attn_kernel<64, 2>), grid, block, 0, st, a);
    else if (pf == 3) hipLaunchKernelGGL((attn_kernel<64, 3>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((attn_kernel<64, 4>), grid, block, 0, st, a);
  }
  int rc = launched("int8_decode_attention");
  if (ev1) (void)hipEventRecord(ev1, st);
  if (rc != KVQ_OK || num_splits == 1) return rc;
  const dim3 rgrid((unsigned)num_seqs, (unsigned)num_q_heads, (unsigned)maxq);
  if (head_dim == 128) hipLaunchKernelGGL(split_reduce_kernel<128>, rgrid, dim3(WAVE), 0, st, a);
  else hipLaunchKernelGGL(split_reduce_kernel<64>, rgrid, dim3(WAVE), 0, st, a);
  return launched("split_reduce");
}

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
  if (num_pages > INT32_MAX || num_blocks > INT32_MAX) return fail("dequant_pages: too many pages");
  const int grid = (int)std::min<int64_t>(num_pages, (int64_t)device_cus() * 8);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, st, k_cache, k_sb, k_sn, k_sh, v_cache, v_sb, v_sn, v_sh,
                       (int)num_blocks, (int)block_size, (int)num_heads, (uint16_t*)k_out, (uint16_t*)v_out,
                       block_table, bt_stride, src_req, src_j, (int)num_pages, k_scale, (int)(k_scale_cols > 1),
                       v_scale, (int)(v_scale_cols > 1));
  };
  if (head_dim == 128) go(dequant_pages_kernel<128>);
  else go(dequant_pages_kernel<64>);
  return launched("dequant_pages");
}

}  // extern "C"
