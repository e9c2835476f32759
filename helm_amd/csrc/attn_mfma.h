// Split-K paged decode attention on the matrix cores (gfx950 MFMA), for
// 16-bit K/V pages with head_dim 128 — the hot configuration of HELM's
// perform_streaming_attention (helm/runtime/kv_cache.py:468-555 masked
// online-softmax loop, :562-568 Path 1, :584-662 Path 3) and of the batched
// decode of _decode_batched (helm/runtime/kv_offload.py:152-174).
//
// Decode attention is bound by HBM: every K/V byte is read once.  The matrix
// cores are used here only to take the arithmetic off the vector ALU, so that
// the ALU work per 16-token block stays far below the time its 8 KiB take to
// arrive, at any GQA group size up to 16 query rows per KV head.
//
// Work decomposition: grid.x = split (<= kMfmaMaxPps pages), grid.y = KV head
// + Hkv * row tile, grid.z = sequence; NW waves per workgroup, wave w takes
// the 16-token blocks w, w+NW, ... of the split.  Per block, with q4 = lane/16 and
// n = lane%16:
//   * scores: S^T = K . Q^T with four 16x16x32 MFMAs (k = head dims).  Lane l
//     loads K of token tau(n) = 4*(n%4) + n/4 at dims chunk 4i + q4 (16 B, i =
//     0..3); Q^T's operand holds query row n at the same chunks.  The result
//     gives lane l the scores of query row n for tokens 4r + q4 (r = 0..3).
//   * online softmax per row on those four scores, in natural-log units as
//     HELM's loop; the running max is refreshed (wave-uniformly) only when a
//     score exceeds it by more than kMfmaSlack, otherwise the stale max keeps
//     every weight <= e^kMfmaSlack and O, L exact relative to it.
//   * O += P . V with eight 16x16x32 MFMAs (one per dim e of each lane's
//     8-dim column group): P's operand is {hi(p_r), lo(p_r)} — each weight
//     split into two 16-bit values whose sum carries 16 mantissa bits — and
//     V's operand the same four tokens 4j + q4 twice, so one MFMA adds
//     (hi + lo) . v.  Lane (q4, n) loads V rows 4j + q4 at dims 8n..8n+7: a
//     wave load is 1 KiB contiguous.  Products are exact and accumulate in
//     fp32.
// No data moves between lanes in the loop; the split's per-wave states meet in
// LDS; the shared split epilogue (attn_kernel.h) merges the waves and then
// the splits.
#pragma once

#include <type_traits>

#include "attn_kernel.h"

namespace helm {

constexpr int kMfmaRows = 16;     // query rows per tile (MFMA M dimension)
// pages per split: page records live one per lane, in two windows of 64
constexpr int kMfmaMaxPps = 128;
constexpr int kMfmaMaxSplits = 4096;
constexpr float kMfmaSlack = 8.f;
// Register buffers of the block pipeline: with two, one block's loads are in
// flight while the wave computes the other (8 KiB per wave, 32 KiB per CU).
// Measured on the Qwen3-8B 32k call: 2 buffers 26.4-26.5 us, 3 buffers
// 26.7-27.0, 4 buffers 27.2-27.4 per call.
#ifndef HELM_MFMA_NBUF
#define HELM_MFMA_NBUF 2
#endif
constexpr int kMfmaBufs = HELM_MFMA_NBUF;

// kFeatMask16: the mask is 16-bit (bf16 / fp16); only the decode kernel
// reads it at that width (the chunk kernels read the element type at run time)
enum MfmaFeat { kFeatMask = 1, kFeatCap = 2, kFeatCausal = 4, kFeatMask16 = 8 };

typedef __bf16 mf_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 mf_f16x8 __attribute__((ext_vector_type(8)));
typedef float mf_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t mf_u32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct MfmaOps;

template <> struct MfmaOps<bf16_t> {
  __device__ static __forceinline__ mf_f32x4 mma(mf_u32x4 a, mf_u32x4 b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mf_bf16x8, a),
                                                   __builtin_bit_cast(mf_bf16x8, b), c, 0, 0, 0);
  }
  // Two weights as packed 16-bit hi and lo parts, hi = RNE(w), lo = RNE(w - hi)
  // (v_cvt_pk_bf16_f32 rounds to nearest even); element 0 in the low half.
  __device__ static __forceinline__ void split2(float w0, float w1, uint32_t& hi,
                                                uint32_t& lo) {
    hi = pk(w0, w1);
    lo = pk(w0 - __uint_as_float(hi << 16), w1 - __uint_as_float(hi & 0xffff0000u));
  }
  __device__ static __forceinline__ uint32_t pk(float a, float b) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, bf2));
  }
  // eight 16-bit ones (an MFMA operand)
  __device__ static __forceinline__ mf_u32x4 ones8() {
    return mf_u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  }
};

template <> struct MfmaOps<f16_t> {
  __device__ static __forceinline__ mf_f32x4 mma(mf_u32x4 a, mf_u32x4 b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mf_f16x8, a),
                                                  __builtin_bit_cast(mf_f16x8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pk(float a, float b) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, h2));
  }
  // eight 16-bit ones (an MFMA operand)
  __device__ static __forceinline__ mf_u32x4 ones8() {
    return mf_u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};
  }
  // hi = RNE(w), lo = RNE(w - hi) in fp16, packed two per word (v_cvt_pk_f16_f32)
  __device__ static __forceinline__ void split2(float w0, float w1, uint32_t& hi,
                                                uint32_t& lo) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    const h2 h = __builtin_convertvector((f2){w0, w1}, h2);
    hi = __builtin_bit_cast(uint32_t, h);
    const f2 back = __builtin_convertvector(h, f2);
    lo = __builtin_bit_cast(uint32_t,
                            __builtin_convertvector((f2){w0 - back[0], w1 - back[1]}, h2));
  }
};

// 16-byte buffer load with the non-temporal hint: K/V are read exactly once.
__device__ __forceinline__ mf_u32x4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, int off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
  return mf_u32x4{v[0], v[1], v[2], v[3]};
}

// LDS transpose read of 16-bit elements (ds_read_b64_tr_b16): within each
// 16-lane group, lane c = 4a + b receives element b of the 8 bytes that
// lanes a, a + 4, a + 8 and a + 12 address, in that order.
__device__ __forceinline__ uint2 ld_tr16(const char* lds_addr) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16*)(lds_addr));
  return __builtin_bit_cast(uint2, r);
}

// Low / high 16-bit halves of two words packed into one: (a.lo, b.lo), (a.hi, b.hi).
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// ---- page records held one per lane ------------------------------------------
// Lane i holds the record of page pg0 + i of the split; a block reads its
// page's record with v_readlane (a uniform lane index), so no memory access
// sits between a block's turn and the issue of its loads.
struct PoolLanes {
  int slot;
};
struct DescLanes {
  uint32_t klo, khi, vlo, vhi;
  int used, tok_off, head_stride;
};

// Issued before the sequence length is known: the pool's table row is read
// up to its declared width, so the first K/V loads wait for one memory trip.
__device__ __forceinline__ PoolLanes lane_pages(const PoolSrc& s, int b, int pg0, int lane) {
  PoolLanes L;
  L.slot = s.max_pages > 0
               ? s.table[(int64_t)b * s.table_stride + min(pg0 + lane, s.max_pages - 1)]
               : 0;
  return L;
}
__device__ __forceinline__ DescLanes lane_pages(const DescSrc& s, int b, int pg0, int lane) {
  const helm_page* base = s.base(b);
  const int cnt = s.n_pages(b);
  helm_page d{};
  if (cnt > 0) d = base[max(0, min(pg0 + lane, cnt - 1))];
  DescLanes L;
  L.klo = static_cast<uint32_t>(d.k);
  L.khi = static_cast<uint32_t>(d.k >> 32);
  L.vlo = static_cast<uint32_t>(d.v);
  L.vhi = static_cast<uint32_t>(d.v >> 32);
  L.used = s.used_of(d, b);
  L.tok_off = d.tok_off;
  L.head_stride = d.head_stride;
  return L;
}

// Page i of the split (uniform): head-hk K / V bases, used tokens, token offset.
__device__ __forceinline__ PageView lane_page_view(const PoolSrc& s, const PoolLanes& L, int b,
                                                   int pg, int i, int hk) {
  const int slot = __builtin_amdgcn_readlane(L.slot, i);
  const int T = sload(s.seq_lens + b);
  PageView pv;
  const int64_t off = (int64_t)slot * s.slot_stride_b + hk * s.head_stride_b;
  pv.k = s.k_pool + off;
  pv.v = s.v_pool + off;
  pv.tok_off = pg * s.page_size;
  pv.used = min(s.page_size, T - pv.tok_off);
  pv.head_stride_b = 0;
  return pv;
}
__device__ __forceinline__ PageView lane_page_view(const DescSrc& s, const DescLanes& L, int,
                                                   int, int i, int hk) {
  const uint64_t k = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(L.khi, i) << 32) |
                     (uint32_t)__builtin_amdgcn_readlane(L.klo, i);
  const uint64_t v = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(L.vhi, i) << 32) |
                     (uint32_t)__builtin_amdgcn_readlane(L.vlo, i);
  const int hs = __builtin_amdgcn_readlane(L.head_stride, i);
  // (head strides are >= 0: one 32 x 32 -> 64-bit product)
  const uint64_t off = (uint64_t)(uint32_t)hs * (uint32_t)(hk * s.elem_bytes);
  PageView pv;
  pv.k = reinterpret_cast<const char*>(k) + off;
  pv.v = reinterpret_cast<const char*>(v) + off;
  pv.used = __builtin_amdgcn_readlane(L.used, i);
  pv.tok_off = __builtin_amdgcn_readlane(L.tok_off, i);
  pv.head_stride_b = 0;
  return pv;
}

// Used tokens and token offset of page i of the split (uniform), without its
// addresses: what a walk needs for the blocks it does not load itself.
struct PageMeta {
  int used;
  int tok_off;
};
__device__ __forceinline__ PageMeta lane_page_meta(const PoolSrc& s, const PoolLanes&, int b,
                                                   int pg, int) {
  const int T = sload(s.seq_lens + b);
  PageMeta pm;
  pm.tok_off = pg * s.page_size;
  pm.used = min(s.page_size, T - pm.tok_off);
  return pm;
}
__device__ __forceinline__ PageMeta lane_page_meta(const DescSrc&, const DescLanes& L, int, int,
                                                   int i) {
  PageMeta pm;
  pm.used = __builtin_amdgcn_readlane(L.used, i);
  pm.tok_off = __builtin_amdgcn_readlane(L.tok_off, i);
  return pm;
}

// One 16-token block of the online-softmax recurrence on the matrix cores:
// k / v are the block's K and V operands (K token tau(n) at dim chunks
// q4 + 4i; V tokens q4 + 4j at dims 8n..8n+7), mk the additive mask of the
// lane's row for tokens 4r + q4, ntok the block's valid tokens, tok0 the
// HELM token cursor of its first token.  Updates the row max m, this lane's
// share of the row sum, and O (rows 4 q4 + r, dims 8n + e).
// q . k of the lane's row n for tokens 4r + q4 of a block (K operand k).
template <class Ops>
__device__ __forceinline__ mf_f32x4 mfma_qk(const mf_u32x4 (&k)[4], const mf_u32x4 (&qop)[4]) {
  mf_f32x4 sc = mf_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) sc = Ops::mma(k[i], qop[i], sc);
  return sc;
}

// Logits of those four tokens: scale, soft-cap, additive mask, causal limit
// (tokens past s_vis, the row's last visible token), and -inf past the
// block's ntok valid tokens.
template <bool kMask, bool kCap, bool kCausal>
__device__ __forceinline__ void mfma_logits(mf_f32x4 sc, const float (&mk)[4], int ntok, int tok0,
                                            float scale, float cap, float inv_cap, int s_vis,
                                            int q4, float (&x)[4]) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float val = sc[r] * scale;
    if constexpr (kCap) val = tanhf(val * inv_cap) * cap;
    if constexpr (kMask) val += mk[r];
    if constexpr (kCausal)
      if (tok0 + 4 * r + q4 > s_vis) val = -INFINITY;
    x[r] = val;
  }
  if (ntok < kBlockTok) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (4 * r + q4 >= ntok) x[r] = -INFINITY;
  }
}

// The lazy online-softmax reference update for a block max bm: when bm
// exceeds the row max by more than the slack anywhere in the wave, the row
// max is refreshed and l and the O rows rescaled.
__device__ __forceinline__ void mfma_refresh_max(float bm, float& m, float& lsum,
                                                 mf_f32x4 (&o)[8], int q4) {
  if (__builtin_amdgcn_ballot_w64(bm > m + kMfmaSlack)) {
    // refresh the row max (uniform across the row's four lanes)
    float rm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    rm = fmaxf(rm, __shfl_xor(rm, 32, 64));
    const float mn = fmaxf(m, rm);
    const float a = fexp(m - ((mn == -INFINITY) ? 0.f : mn));
    lsum *= a;
    m = mn;
    // O rows of this lane are 4*q4 + r: fetch their factors
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ar = __shfl(a, 4 * q4 + r, 64);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e][r] *= ar;
    }
  }
}

// Weights exp(x - m) of the four tokens into l and, as hi + lo 16-bit parts,
// P . V into O (V operand v: tokens q4 + 4j at dims 8n .. 8n + 7).
template <class Ops>
__device__ __forceinline__ void mfma_pv(const float (&x)[4], const mf_u32x4 (&v)[4], float m,
                                        float& lsum, mf_f32x4 (&o)[8]) {
  const float base = (m == -INFINITY) ? 0.f : m;
  float wt[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    wt[r] = fexp(x[r] - base);
    lsum += wt[r];
  }
  uint32_t h01, l01, h23, l23;
  Ops::split2(wt[0], wt[1], h01, l01);
  Ops::split2(wt[2], wt[3], h23, l23);
  const mf_u32x4 pop = mf_u32x4{h01, h23, l01, l23};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t a01 = pack_lo(v[0][w], v[1][w]);
    const uint32_t a23 = pack_lo(v[2][w], v[3][w]);
    const uint32_t b01 = pack_hi(v[0][w], v[1][w]);
    const uint32_t b23 = pack_hi(v[2][w], v[3][w]);
    o[2 * w] = Ops::mma(pop, mf_u32x4{a01, a23, a01, a23}, o[2 * w]);
    o[2 * w + 1] = Ops::mma(pop, mf_u32x4{b01, b23, b01, b23}, o[2 * w + 1]);
  }
}

// One 16-token block of the recurrence: q . k, logits, max refresh, P . V.
template <class Ops, bool kMask, bool kCap, bool kCausal>
__device__ __forceinline__ void mfma_block_step(const mf_u32x4 (&k)[4], const mf_u32x4 (&v)[4],
                                                const float (&mk)[4], int ntok, int tok0,
                                                const mf_u32x4 (&qop)[4], float& m, float& lsum,
                                                mf_f32x4 (&o)[8], float scale, float cap,
                                                float inv_cap, int s_vis, int q4) {
  float x[4];
  mfma_logits<kMask, kCap, kCausal>(mfma_qk<Ops>(k, qop), mk, ntok, tok0, scale, cap, inv_cap,
                                    s_vis, q4, x);
  mfma_refresh_max(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), m, lsum, o, q4);
  mfma_pv<Ops>(x, v, m, lsum, o);
}

template <class Src> struct LanesOf;
template <> struct LanesOf<PoolSrc> { using type = PoolLanes; };
template <> struct LanesOf<DescSrc> { using type = DescLanes; };

template <typename T, class Src, int FEAT, int NW>
__global__ __launch_bounds__(64 * NW) void decode_mfma_kernel(AttnParams p, Src src) {
  using Ops = MfmaOps<T>;
  constexpr int NT = 64 * NW;
  constexpr int kRow = 256;  // bytes per token row (128 dims x 2 B)
  constexpr bool kMask = (FEAT & kFeatMask) != 0;
  constexpr bool kCap = (FEAT & kFeatCap) != 0;
  constexpr bool kCausal = (FEAT & kFeatCausal) != 0;
  constexpr bool kMask16 = (FEAT & kFeatMask16) != 0;

  __shared__ Smem<NW, kMfmaRows, 128> sm;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int q4 = lane >> 4;
  const int n = lane & 15;
  // profiling stamps of this workgroup (helm_profile_workgroup_stamps)
  uint64_t* const stp =
      p.stamps ? p.stamps + 4 * (blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z))
               : nullptr;
  if (stp && tid == 0) {
    stp[0] = stamp_now();
    stp[3] = stamp_place();
  }

  int split_local = blockIdx.x, b = blockIdx.z;
  if (src.compact) {
    // the last sequence whose first split is at or before blockIdx.x
    int bb = 0;
#pragma unroll
    for (int j = 1; j < kSeqArgs; ++j)
      if (j < src.n_seq && (int)blockIdx.x >= src.seq_split0[j]) bb = j;
    b = bb;
    split_local = blockIdx.x - src.seq_split0[bb];
  }
  const int hk = blockIdx.y % p.Hkv;
  // the waves share one 16-row tile and split its blocks (query chunks with
  // more tiles run in chunk_mfma_kernel)
  const int qt = blockIdx.y / p.Hkv;
  const int tile = (b * p.Hkv + hk) * p.n_qtiles + qt;
  const int S = p.S;
  const int G = p.G;
  const int r0 = qt * kMfmaRows;
  const int nrows = min(kMfmaRows, G * S - r0);

  // ---- loads that need no sequence length: page records, query rows --------
  // (pg0 below equals this whenever the workgroup has pages to process)
  const typename LanesOf<Src>::type lanes =
      lane_pages(src, b, p.lo + split_local * p.pps, lane);
  // a split of more than 64 pages: the records of its pages 64 .. 127
  typename LanesOf<Src>::type lanes_hi{};
  if (p.pps > 64 && !p.dyn) lanes_hi = lane_pages(src, b, p.lo + split_local * p.pps + 64, lane);
  // ---- query operand: row n of the tile at dim chunks 4i + q4 ---------------
  const bool row_ok = n < nrows;
  const int rr = r0 + (row_ok ? n : 0);
  const RowCoord rc = row_coord(rr, G);
  const int g_row = rc.g;
  const int s_row = rc.s;
  // causal: query position s sees tokens 0 .. s + causal - 1
  const int s_vis = s_row + (kCausal ? p.causal - 1 : 0);
  mf_u32x4 qop[4];
  {
    const int h = hk * G + g_row;
    const char* qp = reinterpret_cast<const char*>(p.q) +
                     ((int64_t)(b * p.Hq + h) * S + s_row) * kRow;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(qp + 16 * (4 * i + q4));
      qop[i] = row_ok ? mf_u32x4{v.x, v.y, v.z, v.w} : mf_u32x4{0u, 0u, 0u, 0u};
    }
  }
  // ---- this workgroup's page range -------------------------------------------
  const int np = src.n_pages(b);
  const int lo = min(p.lo, np);
  const int hi = min(p.hi, np);
  const int nsplit_launch = (hi - lo + p.pps - 1) / p.pps;
  const int total = p.total_splits > 0 ? p.total_splits : nsplit_launch;
  // split 0 publishes the tile's split count; a tile without pages gets
  // zeros (HELM kv_cache.py:441-442): from split 0 in fused mode, from
  // merge_splits_kernel otherwise
  if (split_local == 0 && tid == 0) p.counts[tile] = total;
  const bool active = total > 0 && split_local < nsplit_launch;
  if (!active) {
    if (total == 0 && p.fused && split_local == 0) {
      for (int idx = tid; idx < nrows * 128; idx += NT) {
        const int zr = r0 + idx / 128;
        const RowCoord rc = row_coord(zr, G);
        const int h = hk * G + rc.g, s = rc.s;
        const int64_t o_off = ((int64_t)(b * p.Hq + h) * S + s) * 128 + idx % 128;
        store_elem<T>(reinterpret_cast<char*>(p.out) + o_off * 2, 0.f);
      }
    }
    if (stp && tid == 0) stp[1] = stp[2] = stamp_now();
    return;
  }
  const int split = p.split_base + split_local;
  const int pg0 = lo + split_local * p.pps;
  const int npg = min(pg0 + p.pps, hi) - pg0;  // 1..kMfmaMaxPps
  if constexpr (std::is_same<Src, DescSrc>::value) {
    // a call that carries the sequences' new tokens: each workgroup whose
    // split holds the sequence's last page writes its head's token into that
    // page's last used slot (16 lanes K, 16 lanes V, 16 bytes each), and the
    // stores are complete before any wave of the workgroup reads the page.
    // Workgroups of other query tiles of the same head write the same bytes.
    if (!p.dyn && b < src.app_n && pg0 + npg == np) {
      if (wave == 0) {
        const PageView tv = src.page(b, np - 1, hk);
        if (lane < 32 && tv.used > 0) {
          const int c = lane & 15;
          const bool isv = lane >= 16;
          const char* from = (isv ? src.app_v[b] : src.app_k[b]) + hk * src.app_hs[b] * 2 + 16 * c;
          char* to = const_cast<char*>(isv ? tv.v : tv.k) + (int64_t)(tv.used - 1) * kRow + 16 * c;
          *reinterpret_cast<uint4*>(to) = *reinterpret_cast<const uint4*>(from);
        }
        __builtin_amdgcn_s_waitcnt(0);
      }
      __syncthreads();
    }
  }

  MaskRow mrow{nullptr, HELM_F32};
  if constexpr (kMask) mrow = mask_row(p, b, hk * G + g_row, s_row);

  const float scale = p.scale;
  const float cap = p.softcap;
  const float inv_cap = kCap ? 1.f / cap : 0.f;

  float m = -INFINITY;  // running max of row n (same in the 4 lanes of the row)
  float lsum = 0.f;     // this lane's share of row n's weight sum
  mf_f32x4 o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = mf_f32x4{0.f, 0.f, 0.f, 0.f};

  const int bpp = p.bpp;
  const int nblk = npg * bpp;
  // lane offsets inside a block: K token tau(n) at chunk q4 (+64 B per i),
  // V token q4 at dims 8n (+1 KiB per j)
  const int voff_k = (4 * (n & 3) + (n >> 2)) * kRow + 16 * q4;
  const int voff_v = q4 * kRow + 16 * n;

  struct Blk {
    mf_u32x4 k[4];
    mf_u32x4 v[4];
    // mask elements as loaded, at their width (a 16-bit mask kept as 16-bit
    // values: zero-extending them would be an instruction on each loaded
    // register, placed where the next step's loads must have completed)
    typename std::conditional<kMask16, uint16_t, uint32_t>::type mk[4];
    int ntok;   // valid tokens of the block (0: past the end)
    int tok0;   // HELM token cursor of the block's first token
  };

  auto load_block = [&](int bi, Blk& B) {
    const bool valid = bi < nblk;
    const int pi = valid ? (p.bpp_log2 >= 0 ? bi >> p.bpp_log2 : bi / bpp) : 0;
    const int sub = valid ? bi - pi * bpp : 0;
    const PageView pv = pi < 64 ? lane_page_view(src, lanes, b, pg0 + pi, pi, hk)
                                : lane_page_view(src, lanes_hi, b, pg0 + pi, pi - 64, hk);
    const int tok_in = sub * kBlockTok;
    const int ntok = valid ? sclamp(pv.used - tok_in, 0, kBlockTok) : 0;
    B.ntok = ntok;
    B.tok0 = pv.tok_off + tok_in;
    const auto rk = make_rsrc(pv.k + tok_in * kRow, ntok * kRow);
    const auto rv = make_rsrc(pv.v + tok_in * kRow, ntok * kRow);
#pragma unroll
    for (int i = 0; i < 4; ++i) B.k[i] = buf_load16_nt(rk, voff_k + 64 * i);
#pragma unroll
    for (int j = 0; j < 4; ++j) B.v[j] = buf_load16_nt(rv, voff_v + 1024 * j);
    if constexpr (kMask) {
      // token 4r + q4 of the block for row n; clamped inside the block's
      // tokens (a block past its page's tokens reads the row's first key:
      // its scores are -inf whatever the mask holds)
      const int mbase = ntok > 0 ? B.tok0 : 0;
      const int last = max(ntok - 1, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        B.mk[r] = mrow.bits<kMask16>(mbase + min(4 * r + q4, last));
    }
  };

  auto compute_block = [&](const Blk& B) {
    float mk[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) mk[r] = kMask ? mrow.widen<kMask16>(B.mk[r]) : 0.f;
    mfma_block_step<Ops, kMask, kCap, kCausal>(B.k, B.v, mk, B.ntok, B.tok0, qop, m, lsum, o,
                                               scale, cap, inv_cap, s_vis, q4);
  };

  // ---- dynamic block claiming (p.dyn): the waves of every workgroup of the
  // tile share the tile's blocks through one counter -------------------------
  // Block k of the tile is page lo + k / bpp, 16-token block k % bpp of it.
  // The Wt waves of the tile's workgroups take blocks w, w + Wt, w + 2 Wt
  // first (w = the wave's index among them), then claim one block at a time
  // (block 3 Wt + the counter's old value), so a wave that streams faster
  // takes more blocks and every wave's last block ends at about the same
  // time.  Per step a wave reads the result of the claim it issued one step
  // before, issues the next claim, fetches the page record of the block two
  // ahead (scalar load) and the K / V of the block one ahead, then computes
  // the current block: each of the three latencies hides behind one step.
  // Claims only grow, so a wave is done at its first block past the tile.
  if (p.dyn) {
    const int Wt = nsplit_launch * NW;
    const int np_t = hi - lo;
    const int nblk_t = np_t * bpp;
    const int kbase = 3 * Wt;
    uint32_t* const ctr = p.claims + (int64_t)tile * kClaimStride;
    const int w0 = split_local * NW + wave;
    // the block whose last slot takes the step's new token (-1: none)
    int k_tok = -1;
    const char* tok_from = nullptr;
    if constexpr (std::is_same<Src, DescSrc>::value) {
      if (b < src.app_n && np_t > 0) {
        const PageView tv = src.page(b, hi - 1, hk);
        if (tv.used > 0) {
          k_tok = (np_t - 1) * bpp + (tv.used - 1) / kBlockTok;
          tok_from = (lane >= 16 ? src.app_v[b] : src.app_k[b]) + hk * src.app_hs[b] * 2 +
                     16 * (lane & 15);
        }
      }
    }
    // block k's page record, fetched a step before it is used (scalar loads
    // whose wait falls in the next step), and its view; past the tile: none
    struct Rec {
      typename Src::Raw r;
      int k;
    };
    const typename Src::Ctx sc = src.ctx(b);
    auto fetch = [&](int k) {
      Rec d;
      d.k = __builtin_amdgcn_readfirstlane(k);  // uniform: scalar loads, not vector ones
      // (past the tile: the last page's record, not used)
      const int kk = min(d.k, nblk_t - 1);
      const int pi = p.bpp_log2 >= 0 ? kk >> p.bpp_log2 : kk / bpp;
      d.r = src.raw(sc, lo + pi);
      return d;
    };
    auto view = [&](Rec d) {
      PageView pv;
      if (d.k < nblk_t) {
        const int pi = p.bpp_log2 >= 0 ? d.k >> p.bpp_log2 : d.k / bpp;
        Src::pin(d.r);
        pv = src.view(sc, d.r, lo + pi, hk);
        const int tok_in = (d.k - pi * bpp) * kBlockTok;
        pv.k += tok_in * kRow;
        pv.v += tok_in * kRow;
        pv.tok_off += tok_in;
        pv.used -= tok_in;
      } else {
        pv.k = pv.v = reinterpret_cast<const char*>(p.q);
        pv.used = 0;
        pv.tok_off = 0;
      }
      // (uniform; said so, so that the values stay in scalar registers)
      pv.k = reinterpret_cast<const char*>(uniform64(reinterpret_cast<uint64_t>(pv.k)));
      pv.v = reinterpret_cast<const char*>(uniform64(reinterpret_cast<uint64_t>(pv.v)));
      pv.used = __builtin_amdgcn_readfirstlane(pv.used);
      pv.tok_off = __builtin_amdgcn_readfirstlane(pv.tok_off);
      pv.head_stride_b = 0;
      return pv;
    };
    // K / V (and mask) loads of block k through its record
    auto load_dyn = [&](int k, const PageView& pv, Blk& B) {
      k = __builtin_amdgcn_readfirstlane(k);
      if constexpr (std::is_same<Src, DescSrc>::value) {
        if (k == k_tok) {
          // this wave is the one that reads the new token's block: write the
          // token into its slot first (16 lanes K, 16 lanes V)
          if (lane < 32) {
            char* to = const_cast<char*>(lane >= 16 ? pv.v : pv.k) +
                       (int64_t)(pv.used - 1) * kRow + 16 * (lane & 15);
            *reinterpret_cast<uint4*>(to) = *reinterpret_cast<const uint4*>(tok_from);
          }
          __builtin_amdgcn_s_waitcnt(0);
        }
      }
      const int ntok = sclamp(pv.used, 0, kBlockTok);
      B.ntok = ntok;
      B.tok0 = pv.tok_off;
      const auto rk = make_rsrc(pv.k, ntok * kRow);
      const auto rv = make_rsrc(pv.v, ntok * kRow);
#pragma unroll
      for (int i = 0; i < 4; ++i) B.k[i] = buf_load16_nt(rk, voff_k + 64 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) B.v[j] = buf_load16_nt(rv, voff_v + 1024 * j);
      if constexpr (kMask) {
        const int mbase = ntok > 0 ? B.tok0 : 0;
        const int last = max(ntok - 1, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) B.mk[r] = mrow.bits<kMask16>(mbase + min(4 * r + q4, last));
      }
    };
    auto claim = [&]() {
      uint32_t v = 0;
      if (lane == 0) v = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return v;
    };
    bool dry = kbase >= nblk_t;  // no block left to claim
    uint32_t cl = dry ? 0u : claim();
    int kc = w0, kn = w0 + Wt, kr = w0 + 2 * Wt;
    Rec rn = fetch(kn);
    Blk buf[2];
    load_dyn(kc, view(fetch(kc)), buf[0]);
    auto step = [&](Blk& cur, Blk& nxt) {
      int kq = nblk_t;
      if (!dry) {
        kq = kbase + (int)__builtin_amdgcn_readfirstlane(cl);
        if (kq >= nblk_t) {
          kq = nblk_t;
          dry = true;
        } else {
          cl = claim();
        }
      }
      // (the record fetch after the view of the one fetched a step before:
      // scalar loads return out of order, so a wait for that one would also
      // wait for this one)
      load_dyn(kn, view(rn), nxt);
      const Rec rr = fetch(kr);
      compute_block(cur);
      kc = kn;
      kn = kr;
      rn = rr;
      kr = kq;
    };
    while (kc < nblk_t) {
      step(buf[0], buf[1]);
      if (kc >= nblk_t) break;
      step(buf[1], buf[0]);
    }
    // the claim still in flight (its result is not needed)
    __builtin_amdgcn_s_waitcnt(0);
  } else
  // ---- main loop: a ring of kMfmaBufs register buffers, kMfmaBufs - 1
  // blocks' loads in flight while one block is computed ----------------------
  {
    constexpr int NB = kMfmaBufs;
    // this wave's blocks: wave, wave + NW, ...
    const int nmine = nblk > wave ? (nblk - wave + NW - 1) / NW : 0;
    Blk buf[NB];
#pragma unroll
    for (int i = 0; i < NB - 1; ++i) load_block(wave + i * NW, buf[i]);
    // Whole rounds of NB blocks, then the remaining blocks: an exit inside
    // the unrolled round would join register states the compiler can only
    // reconcile by waiting for every load in flight.  The scheduling barrier
    // keeps each step's loads ahead of its compute, so the wait for the
    // block computed covers that block's loads only.
    int k = 0;
    for (; k + NB <= nmine; k += NB) {
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        load_block(wave + (k + u + NB - 1) * NW, buf[(u + NB - 1) % NB]);
        __builtin_amdgcn_sched_barrier(0);
        compute_block(buf[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < NB - 1; ++u) {
      if (k + u >= nmine) break;
      load_block(wave + (k + u + NB - 1) * NW, buf[(u + NB - 1) % NB]);
      compute_block(buf[u]);
    }
  }

  // ---- per-wave state to LDS ---------------------------------------------------
  float lrow = lsum + __shfl_xor(lsum, 16, 64);
  lrow += __shfl_xor(lrow, 32, 64);
  if (q4 == 0) {
    sm.m[wave][n] = m;
    sm.l[wave][n] = lrow;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float* dst = &sm.o[wave][4 * q4 + r][8 * n];
    *reinterpret_cast<float4*>(dst) = make_float4(o[0][r], o[1][r], o[2][r], o[3][r]);
    *reinterpret_cast<float4*>(dst + 4) = make_float4(o[4][r], o[5][r], o[6][r], o[7][r]);
  }
  __syncthreads();
  if (stp && tid == 0) stp[1] = stamp_now();
  split_epilogue_d128<T, NW, kMfmaRows>(sm, p, tid, tile, split, total, nrows, r0, b, hk);
  if (stp && tid == 0) stp[2] = stamp_now();
}

// ---- query chunks: K/V blocks staged through LDS ----------------------------
// For q_len > 1 with more than one 16-row tile per KV head.  A workgroup of
// four waves owns four 16-row tiles (one per wave) and walks the split's
// blocks in stages of four: wave w loads block w of the stage (K and V,
// 4 KiB each) from HBM / L2 into registers one stage ahead, writes it to LDS,
// and after one barrier every wave computes all four blocks from LDS.  K and
// V sit in LDS as 16-byte chunks with chunk c of token t at slot c ^ (t % 16),
// so the operand reads of a wave (16 tokens x one chunk for K, one token x
// 16 chunks for V) are free of bank conflicts.  The per-block arithmetic is
// mfma_block_step, as in the decode kernel.  A split may span any number of
// pages: the page records sit one per lane in windows of 64 pages, the next
// window loaded when the current one is entered.  Each wave writes its own
// split partial (merged by merge_splits_d128_kernel), or, when the call has a
// single split (p.direct_out), its normalized output rows.
constexpr int kChunkStage = 4;        // blocks per stage = waves per workgroup
constexpr int kRecWindow = 64;        // page records held per lane window

template <typename T, class Src, int FEAT>
__global__ __launch_bounds__(256) void chunk_mfma_kernel(AttnParams p, Src src) {
  using Ops = MfmaOps<T>;
  constexpr int kRow = 256;            // bytes per token row (128 dims x 2 B)
  constexpr int kBlk = kBlockTok * kRow;  // 4 KiB per block of K (or V)
  constexpr bool kMask = (FEAT & kFeatMask) != 0;
  constexpr bool kCap = (FEAT & kFeatCap) != 0;
  constexpr bool kCausal = (FEAT & kFeatCausal) != 0;
  // [buffer][K, V][block of the stage][16-byte chunk]
  __shared__ mf_u32x4 lds[2][2][kChunkStage][kBlk / 16];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int q4 = lane >> 4;
  const int n = lane & 15;

  const int split_local = blockIdx.x;
  const int hk = blockIdx.y % p.Hkv;
  const int qt_w = (blockIdx.y / p.Hkv) * kChunkStage + wave;
  const bool wave_rows = qt_w < p.n_qtiles;
  const int qt = wave_rows ? qt_w : p.n_qtiles - 1;
  const int b = blockIdx.z;
  const int tile = (b * p.Hkv + hk) * p.n_qtiles + qt;
  const int S = p.S;
  const int G = p.G;
  const int r0 = qt * kMfmaRows;
  const int nrows = min(kMfmaRows, G * S - r0);

  // output row of this lane's accumulator row 4 q4 + r (direct output)
  auto out_row = [&](int r) -> char* {
    const RowCoord c = row_coord(r0 + 4 * q4 + r, G);
    return reinterpret_cast<char*>(p.out) +
           (((int64_t)(b * p.Hq + hk * G + c.g) * S + c.s) * 128 + n) * 2;
  };

  const int np = src.n_pages(b);
  const int lo = min(p.lo, np);
  const int hi = min(p.hi, np);
  const int nsplit_launch = (hi - lo + p.pps - 1) / p.pps;
  const int total = p.total_splits > 0 ? p.total_splits : nsplit_launch;
  if (split_local == 0 && lane == 0 && wave_rows) p.counts[tile] = total;
  if (!(total > 0 && split_local < nsplit_launch)) {      // uniform per workgroup
    if (p.direct_out && total == 0 && split_local == 0 && wave_rows) {
      // no keys: HELM's zeros
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (4 * q4 + r < nrows) {
          uint16_t* dst = reinterpret_cast<uint16_t*>(out_row(r));
#pragma unroll
          for (int e = 0; e < 8; ++e) dst[16 * e] = 0;
        }
    }
    return;
  }
  const int split = p.split_base + split_local;
  const int pg0 = lo + split_local * p.pps;
  const int npg = min(pg0 + p.pps, hi) - pg0;

  const bool row_ok = n < nrows;
  const int rr = r0 + (row_ok ? n : 0);
  const RowCoord rc = row_coord(rr, G);
  const int g_row = rc.g;
  const int s_row = rc.s;
  // causal: query position s sees tokens 0 .. s + causal - 1
  const int s_vis = s_row + (kCausal ? p.causal - 1 : 0);
  mf_u32x4 qop[4];
  {
    const int h = hk * G + g_row;
    const char* qp = reinterpret_cast<const char*>(p.q) +
                     ((int64_t)(b * p.Hq + h) * S + s_row) * kRow;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(qp + 16 * (4 * i + q4));
      qop[i] = row_ok ? mf_u32x4{v.x, v.y, v.z, v.w} : mf_u32x4{0u, 0u, 0u, 0u};
    }
  }
  MaskRow mrow{nullptr, HELM_F32};
  if constexpr (kMask) mrow = mask_row(p, b, hk * G + g_row, s_row);
  const float scale = p.scale;
  const float cap = p.softcap;
  const float inv_cap = kCap ? 1.f / cap : 0.f;

  float m = -INFINITY;
  float lsum = 0.f;
  mf_f32x4 o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = mf_f32x4{0.f, 0.f, 0.f, 0.f};

  const int bpp = p.bpp;
  const int nblk = npg * bpp;
  const int nstage = (nblk + kChunkStage - 1) / kChunkStage;

  // page records: window [win, win + 64) of the split's pages, and the next
  typename LanesOf<Src>::type lanes = lane_pages(src, b, pg0, lane);
  typename LanesOf<Src>::type lanes_next = lane_pages(src, b, pg0 + kRecWindow, lane);
  int win = 0;
  // the page (relative to pg0) and sub-block of the next block to be viewed
  int cur_pi = 0, cur_sub = 0;

  // The four blocks of a stage, viewed once, in order: valid tokens and HELM
  // token cursor of each (uniform), and this wave's own block's K / V bases.
  struct StageView {
    int ntok[kChunkStage], tok0[kChunkStage];
    int own_ntok;
    const char *kb, *vb;
  };
  auto view_stage = [&](int st, StageView& sv) {
#pragma unroll
    for (int j = 0; j < kChunkStage; ++j) {
      if (cur_pi - win >= kRecWindow) {   // uniform: the page lies in the next window
        lanes = lanes_next;
        win += kRecWindow;
        lanes_next = lane_pages(src, b, pg0 + win + kRecWindow, lane);
      }
      const PageView pv = lane_page_view(src, lanes, b, pg0 + cur_pi, cur_pi - win, hk);
      const int tok_in = cur_sub * kBlockTok;
      const int nt = st * kChunkStage + j < nblk ? sclamp(pv.used - tok_in, 0, kBlockTok) : 0;
      sv.ntok[j] = nt;
      sv.tok0[j] = pv.tok_off + tok_in;
      if (j == wave) {
        sv.own_ntok = nt;
        sv.kb = pv.k + tok_in * kRow;
        sv.vb = pv.v + tok_in * kRow;
      }
      if (++cur_sub == bpp) {
        cur_sub = 0;
        ++cur_pi;
      }
    }
  };

  // additive mask of the lane's row for the four blocks of a stage (tokens
  // 4r + q4 of each block), loaded a stage ahead like the K/V chunks
  float mcur[kChunkStage][4], mnext[kChunkStage][4];
  auto load_mask = [&](const StageView& sv, float (&mk)[kChunkStage][4]) {
    if constexpr (kMask) {
#pragma unroll
      for (int j = 0; j < kChunkStage; ++j) {
        const int last = max(sv.ntok[j] - 1, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          mk[j][r] = sv.ntok[j] > 0 ? mrow[sv.tok0[j] + min(4 * r + q4, last)] : 0.f;
      }
    }
  };

  // this wave's share of a stage: block (stage * 4 + wave), 4 chunks of K and
  // 4 of V per lane (chunk lane + 64 u of the block)
  mf_u32x4 gk[4], gv[4];
  auto load_stage = [&](const StageView& sv) {
    const auto rk = make_rsrc(sv.kb, sv.own_ntok * kRow);
    const auto rv = make_rsrc(sv.vb, sv.own_ntok * kRow);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      gk[u] = buf_load16_nt(rk, (lane + 64 * u) * 16);
      gv[u] = buf_load16_nt(rv, (lane + 64 * u) * 16);
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = lane + 64 * u;          // chunk index in the block
      const int t = c >> 4;                 // token
      const int slot = t * 16 + ((c & 15) ^ t);
      lds[buf][0][wave][slot] = gk[u];
      lds[buf][1][wave][slot] = gv[u];
    }
  };

  // LDS address this lane supplies to the transpose read of V dim group e of
  // block j: token 4 (n >> 2) + q4, dims 16 e + 4 (n & 3) .. + 3 (8 bytes of
  // the swizzled row); the read hands lane n dim 16 e + n of the four tokens
  // 4r + q4 supplied by lanes n >> 2, + 4, + 8, + 12 of its 16-lane group
  const int vt = 4 * (n >> 2) + q4;
  auto vaddr = [&](int buf, int j, int e) -> const char* {
    const int chunk = 2 * e + ((n & 3) >> 1);
    return reinterpret_cast<const char*>(&lds[buf][1][j][vt * 16 + (chunk ^ vt)]) + 8 * (n & 1);
  };
  const int tau = 4 * (n & 3) + (n >> 2);   // K token of this lane in a block
  StageView sv_cur, sv_next;
  if (nstage > 0) {
    view_stage(0, sv_cur);
    load_stage(sv_cur);
    if (wave_rows) load_mask(sv_cur, mcur);
  }
  for (int st = 0; st < nstage; ++st) {
    const int buf = st & 1;
    store_stage(buf);
    if (st + 1 < nstage) {
      view_stage(st + 1, sv_next);
      load_stage(sv_next);
      if (wave_rows) load_mask(sv_next, mnext);
    }
    __syncthreads();
    if (wave_rows) {
      // blocks in pairs: one P . V MFMA takes 32 tokens (block jp's four of
      // this lane in k 0-3, block jp + 1's in k 4-7), once with the hi parts
      // of the weights and once with the lo parts, against the same V
      // operand; an empty block of a pair holds zeros (bounded loads) and
      // -inf logits, so it adds nothing
#pragma unroll
      for (int jp = 0; jp < kChunkStage; jp += 2) {
        if (sv_cur.ntok[jp] == 0 && sv_cur.ntok[jp + 1] == 0) continue;   // uniform
        float x[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int j = jp + h;
          mf_u32x4 k[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) k[i] = lds[buf][0][j][tau * 16 + ((q4 + 4 * i) ^ tau)];
          float mk[4] = {0.f, 0.f, 0.f, 0.f};
          if constexpr (kMask) {
#pragma unroll
            for (int r = 0; r < 4; ++r) mk[r] = mcur[j][r];
          }
          mfma_logits<kMask, kCap, kCausal>(mfma_qk<Ops>(k, qop), mk, sv_cur.ntok[j],
                                            sv_cur.tok0[j], scale, cap, inv_cap, s_vis, q4, x[h]);
        }
        mfma_refresh_max(fmaxf(fmaxf(fmaxf(x[0][0], x[0][1]), fmaxf(x[0][2], x[0][3])),
                               fmaxf(fmaxf(x[1][0], x[1][1]), fmaxf(x[1][2], x[1][3]))),
                         m, lsum, o, q4);
        const float base = (m == -INFINITY) ? 0.f : m;
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float wt[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            wt[r] = fexp(x[h][r] - base);
            lsum += wt[r];
          }
          Ops::split2(wt[0], wt[1], hw[2 * h], lw[2 * h]);
          Ops::split2(wt[2], wt[3], hw[2 * h + 1], lw[2 * h + 1]);
        }
        const mf_u32x4 phi = mf_u32x4{hw[0], hw[1], hw[2], hw[3]};
        const mf_u32x4 plo = mf_u32x4{lw[0], lw[1], lw[2], lw[3]};
        // V operand of dim group e: lane n gets dim 16 e + n of tokens
        // 4r + q4 (r = 0..3) of each block, by the LDS transpose read
        mf_u32x4 vop[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint2 a = ld_tr16(vaddr(buf, jp, e));
          const uint2 c = ld_tr16(vaddr(buf, jp + 1, e));
          vop[e] = mf_u32x4{a.x, a.y, c.x, c.y};
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = Ops::mma(phi, vop[e], o[e]);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = Ops::mma(plo, vop[e], o[e]);
      }
    }
    sv_cur = sv_next;
    if constexpr (kMask) {
#pragma unroll
      for (int j = 0; j < kChunkStage; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) mcur[j][r] = mnext[j][r];
    }
  }

  if (!wave_rows) return;
  float lrow = lsum + __shfl_xor(lsum, 16, 64);
  lrow += __shfl_xor(lrow, 32, 64);
  if (p.direct_out) {
    // the call's only split: normalized rows straight to the output
    // (HELM's final out / max(sum, 1e-12), kv_cache.py:554-555)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float l = __shfl(lrow, 4 * q4 + r, 64);   // lane 4 q4 + r holds that row's sum
      const float inv = 1.f / fmaxf(l, 1e-12f);
      if (4 * q4 + r < nrows) {
        uint16_t* dst = reinterpret_cast<uint16_t*>(out_row(r));
#pragma unroll
        for (int e = 0; e < 8; ++e)                              // dim 16 e + n
          dst[16 * e] = static_cast<uint16_t>(Ops::pk(o[e][r] * inv, 0.f));
      }
    }
    return;
  }
  // the wave's own partial (m, l, o[128]) per row, straight from registers
  const int64_t part = ((int64_t)tile * p.max_splits + split) * p.rows_per_tile;
  if (q4 == 0 && n < nrows)
    *reinterpret_cast<float2*>(&p.ws_ml[(part + n) * 2]) = make_float2(m, lrow);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = 4 * q4 + r;
    if (row < nrows) {
      float* dst = &p.ws_o[(part + row) * 128 + n];
#pragma unroll
      for (int e = 0; e < 8; ++e) dst[16 * e] = o[e][r];      // dim 16 e + n
    }
  }
}

}  // namespace helm
