// Query chunks on 32 x 32 matrix-core tiles (v_mfma_f32_32x32x16_{bf16,f16}).
//
// The same page walk and LDS staging as chunk_mfma_kernel (stages of four
// 16-token blocks swizzled into LDS, two stage buffers, one barrier per stage;
// here the blocks go from memory straight into LDS by buffer loads with the
// LDS destination, shared out over the workgroup's waves), but each wave owns
// 32 query rows (two 16-row tiles of the partial layout) and computes 32
// tokens (two blocks) per step, so the softmax of a step covers 1024 scores
// instead of 256 and its fixed costs (max refresh check, weight rounding,
// scalar bookkeeping) are shared by four times the matrix work.  A workgroup
// has four waves (128 rows; two workgroups per CU) or eight (256 rows; one
// per CU, half the stage loads per row).
//
// Lane l = 32 hh + j (j = l % 32):
//   q . k   S^T = K Q^T: A = K (row m = token tau(m), dims 16i + 8hh .. + 7),
//           B = Q^T (column j = query row j), eight MFMAs over the 128 dims.
//           The result gives lane l, for its query row j, register
//           r = 4g + t <-> output row m = 8g + 4hh + t, and with
//           tau(8g + 4h + t) = 16 (g >> 1) + 8h + 4 (g & 1) + t register r holds
//           token 8hh + (r & 7) of block r >> 3 of the step.
//   P . V   O += P V: A = the weights of row j for tokens 8hh .. 8hh + 7 of a
//           block (exactly registers 8u .. 8u + 7 above), rounded once to the
//           16-bit type; B = V of those tokens at dim 32e + j, fetched by LDS
//           transpose reads; O register 4g + t of dim group e is row
//           8g + 4hh + t, dim 32e + j.  A fifth MFMA per block multiplies the
//           same weights by a column of ones: the row sums of exactly the
//           weights P . V used, so that each output row is an exact weighted
//           mean of V under the rounded weights (their rounding perturbs the
//           weights by <= 2^-9 relative, bf16, and the mean by that times the
//           spread of V).  HELM_CHUNK32_HILO=1 builds the split into hi and lo
//           16-bit parts instead (weights to ~2^-17, one more MFMA per group).
// Online softmax per query row with the lazy rescale of the decode kernel, in
// base-2 units (logits scaled by log2(e) with the softmax scale, weights
// 2^(x - m); the partials' max goes out in natural units).
#pragma once

#include <type_traits>

#include "attn_mfma.h"

namespace helm {

typedef float mf_f32x16 __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma32;
template <> struct Mfma32<bf16_t> {
  __device__ static __forceinline__ mf_f32x16 mma(mf_u32x4 a, mf_u32x4 b, mf_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(mf_bf16x8, a),
                                                   __builtin_bit_cast(mf_bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma32<f16_t> {
  __device__ static __forceinline__ mf_f32x16 mma(mf_u32x4 a, mf_u32x4 b, mf_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(mf_f16x8, a),
                                                  __builtin_bit_cast(mf_f16x8, b), c, 0, 0, 0);
  }
};

constexpr int kChunk32Rows = 32;   // query rows per wave

// LDS swizzle of a staged block: chunk c (16 B) of token t (0..15) sits at
// slot c ^ swz(t) of the token's 256-byte row, swz(4a + b) = 4b + a.  The
// q . k reads (one chunk, 16 tokens per 16 lanes) meet 16 distinct slots
// mod 16, and so do the V transpose reads (chunks c0 .. c0 + 3, c0 a
// multiple of 4, of four consecutive tokens 4a .. 4a + 3 per 32 lanes): each
// group of accesses covers every 16-byte bank group once.
__device__ __forceinline__ int swz(int t) { return ((t & 3) << 2) | (t >> 2); }
// P . V with the weights split into 16-bit hi and lo parts (1) or rounded
// once to 16 bits (0: the default — a query chunk is bound by the matrix
// cores, and the single rounding stays far inside the tolerance)
#ifndef HELM_CHUNK32_HILO
#define HELM_CHUNK32_HILO 0
#endif
constexpr float kLog2E = 1.4426950408889634f;   // log2(e)
constexpr float kLn2 = 0.6931471805599453f;     // ln(2)

// 16 bytes per lane from a buffer straight into LDS: lane i writes
// lds_dst + 16 i (the address must be the same in every lane); loads past the
// buffer's size write zeros
__device__ __forceinline__ void buf_load16_lds(__amdgpu_buffer_rsrc_t r, void* lds_dst, int off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_dst, 16,
                                           off, 0, 0, 0);
}

// NW waves per workgroup (4: two workgroups per CU; 8: one, which halves the
// stage loads per query row), 32 query rows each.
template <typename T, class Src, int FEAT, int NW>
__global__ __launch_bounds__(NW * 64, 2) void chunk32_mfma_kernel(AttnParams p, Src src) {
  static_assert(NW == 4 || NW == 8, "waves per workgroup");
  constexpr int SB = kChunkStage;   // 16-token blocks per stage
  using Ops = MfmaOps<T>;
  using M32 = Mfma32<T>;
  constexpr int kRow = 256;                // bytes per token row (128 dims x 2 B)
  constexpr int kBlk = kBlockTok * kRow;   // 4 KiB per 16-token block of K (or V)
  constexpr bool kMask = (FEAT & kFeatMask) != 0;
  constexpr bool kCap = (FEAT & kFeatCap) != 0;
  constexpr bool kCausal = (FEAT & kFeatCausal) != 0;
  // 16-byte-per-lane loads (1 KiB each) a wave issues per stage: a stage is
  // SB blocks of K and of V, 4 loads each, shared out over the NW waves in
  // order (wave w takes loads w * kLoads ..), all in one block per wave
  constexpr int kLoads = 8 * SB / NW;
  // two stage buffers as two objects, so that the compiler sees that the
  // loads filling one never touch the reads of the other:
  // [K, V][block of the stage][16-byte chunk], chunk c of token t at slot
  // t * 16 + (c ^ swz(t)) (see swz)
  typedef mf_u32x4 StageBuf[2][SB][kBlk / 16];
  __shared__ StageBuf lds0, lds1;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int jr = lane & 31;
  const int hh = lane >> 5;

  const int split_local = blockIdx.x;
  const int hk = blockIdx.y % p.Hkv;
  const int n32 = (p.n_qtiles + 1) / 2;                 // 32-row groups of the head
  const int wt = (blockIdx.y / p.Hkv) * NW + wave;
  const bool wave_rows = wt < n32;
  const int wtc = wave_rows ? wt : n32 - 1;
  const int b = blockIdx.z;
  const int S = p.S;
  const int G = p.G;
  const int rbase = wtc * kChunk32Rows;
  const int nrows = min(kChunk32Rows, G * S - rbase);
  const int tile0 = (b * p.Hkv + hk) * p.n_qtiles + 2 * wtc;   // this wave's first 16-row tile
  const bool two_tiles = 2 * wtc + 1 < p.n_qtiles;

  // output element of O register 4g + t of dim group e
  auto out_elem = [&](int g, int t, int e) -> uint16_t* {
    const RowCoord c = row_coord(rbase + 8 * g + 4 * hh + t, G);
    return reinterpret_cast<uint16_t*>(p.out) +
           ((int64_t)(b * p.Hq + hk * G + c.g) * S + c.s) * 128 + 32 * e + jr;
  };

  const int np = src.n_pages(b);
  const int lo = min(p.lo, np);
  const int hi = min(p.hi, np);
  const int nsplit_launch = (hi - lo + p.pps - 1) / p.pps;
  const int total = p.total_splits > 0 ? p.total_splits : nsplit_launch;
  if (split_local == 0 && lane == 0 && wave_rows) {
    p.counts[tile0] = total;
    if (two_tiles) p.counts[tile0 + 1] = total;
  }
  if (!(total > 0 && split_local < nsplit_launch)) {        // uniform per workgroup
    if (p.direct_out && total == 0 && split_local == 0 && wave_rows) {
      // no keys: HELM's zeros
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (8 * g + 4 * hh + t < nrows)
#pragma unroll
            for (int e = 0; e < 4; ++e) *out_elem(g, t, e) = 0;
    }
    return;
  }
  const int split = p.split_base + split_local;
  const int pg0 = lo + split_local * p.pps;
  const int npg = min(pg0 + p.pps, hi) - pg0;

  // ---- query operand: row jr of the wave, dims 16i + 8hh .. + 7 ----------------
  const bool row_ok = jr < nrows;
  const RowCoord rc = row_coord(rbase + (row_ok ? jr : 0), G);
  const int s_row = rc.s;
  // causal: query position s sees tokens 0 .. s + coff (coff = causal - 1)
  const int coff = kCausal ? p.causal - 1 : 0;
  const int s_vis = s_row + coff;                      // row jr's last visible token
  const int s_last = (rbase + nrows - 1) / G + coff;   // the wave's last visible token
  const int s_first = rbase / G + coff;                // and its first row's
  mf_u32x4 qop[8];
  {
    const char* qp = reinterpret_cast<const char*>(p.q) +
                     ((int64_t)(b * p.Hq + hk * G + rc.g) * S + s_row) * kRow;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(qp + 16 * (2 * i + hh));
      qop[i] = row_ok ? mf_u32x4{v.x, v.y, v.z, v.w} : mf_u32x4{0u, 0u, 0u, 0u};
    }
  }
  MaskRow mrow{nullptr, HELM_F32};
  if constexpr (kMask) mrow = mask_row(p, b, hk * G + rc.g, s_row);
  const float scale = p.scale;
  const float cap = p.softcap;
  const float inv_cap = kCap ? 1.f / cap : 0.f;
  // logits, running max and weights in base-2 units: one multiply per score
  // turns q . k into x = s * scale * log2(e), and each weight is 2^(x - m)
  const float scale2 = scale * kLog2E;
  const float cap2 = cap * kLog2E;
  auto sexp = [](float v) { return __builtin_amdgcn_exp2f(v); };

  float m = -INFINITY;   // running max of row jr (same in both halves)
#if HELM_CHUNK32_HILO
  float lsum = 0.f;      // this lane's share of the row's weight sum
#else
  // the rows' weight sums on the matrix cores: P times a column of ones, so
  // the sum takes exactly the 16-bit weights that P . V takes; register
  // 4g + t holds row 8g + 4hh + t (the same value in every lane of a half)
  mf_f32x16 osum;
#pragma unroll
  for (int r = 0; r < 16; ++r) osum[r] = 0.f;
  const mf_u32x4 ones = Ops::ones8();
#endif
  mf_f32x16 o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[e][r] = 0.f;

  const int bpp = p.bpp;
  const int nblk = npg * bpp;
  const int nstage = (nblk + SB - 1) / SB;

  // page records: window [win, win + 64) of the split's pages (the next
  // window is read when the walk enters it, once per 64 pages)
  typename LanesOf<Src>::type lanes = lane_pages(src, b, pg0, lane);
  int win = 0;
  int cur_pi = 0, cur_sub = 0;   // page (relative to pg0) and sub-block of the next view

  // a stage's blocks: valid tokens and first token offset of each (kept for
  // the stage's compute, one stage after its loads were issued), and the
  // block this wave loads
  int vnt[2][SB], vt0[2][SB];
  struct OwnBlock {
    int ntok;
    const char *kb, *vb;
  };
  const int own_blk = (wave * kLoads) >> 3;
  // (a stage never straddles two record windows: window w starts at block
  // 64 w bpp of the split, a multiple of the stage's SB = 4 blocks, so the
  // window is entered at a stage's first block; blocks past the split's end
  // have no tokens and their views are never dereferenced)
  static_assert(kRecWindow % SB == 0, "record windows start at stage boundaries");
  auto view_stage = [&](int st, int (&ntok)[SB], int (&tok0)[SB], OwnBlock& ob) {
    if (cur_pi - win >= kRecWindow) {   // uniform: the stage lies in the next window
      win += kRecWindow;
      lanes = lane_pages(src, b, pg0 + win, lane);
    }
    int own_pi = cur_pi, own_tok_in = 0;
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const PageMeta pm = lane_page_meta(src, lanes, b, pg0 + cur_pi, cur_pi - win);
      const int tok_in = cur_sub * kBlockTok;
      const int nt = st * SB + j < nblk ? sclamp(pm.used - tok_in, 0, kBlockTok) : 0;
      ntok[j] = nt;
      tok0[j] = pm.tok_off + tok_in;
      if (j == own_blk) {
        ob.ntok = nt;
        own_pi = cur_pi;
        own_tok_in = tok_in;
      }
      if (++cur_sub == bpp) {
        cur_sub = 0;
        ++cur_pi;
      }
    }
    // the addresses of the one block this wave loads
    const PageView pv = lane_page_view(src, lanes, b, pg0 + own_pi, own_pi - win, hk);
    ob.kb = pv.k + own_tok_in * kRow;
    ob.vb = pv.v + own_tok_in * kRow;
  };

  // this wave's loads of a stage straight from memory into LDS (no VGPRs):
  // load i = wave * kLoads + k covers K (bit 2 of i clear) or V of the
  // wave's block, slots 64u .. 64u + 63 with u = i % 4, lane l slot 64u + l,
  // which holds chunk (l & 15) ^ swz(t) of token t = 4u + (l >> 4) (the
  // swizzle), so each lane fetches that chunk; loads past the block's tokens
  // write zeros
  auto dma_stage = [&](const OwnBlock& ob, StageBuf& dst) {
    const auto rk = make_rsrc(ob.kb, ob.ntok * kRow);
    const auto rv = make_rsrc(ob.vb, ob.ntok * kRow);
#pragma unroll
    for (int k = 0; k < kLoads; ++k) {
      const int i = wave * kLoads + k;
      const int u = i & 3;
      const int t = 4 * u + (lane >> 4);
      const int off = t * kRow + 16 * ((lane & 15) ^ swz(t));
      if ((i >> 2) & 1)
        buf_load16_lds(rv, &dst[1][own_blk][64 * u], off);
      else
        buf_load16_lds(rk, &dst[0][own_blk][64 * u], off);
    }
  };

  // K row this lane supplies to the q . k MFMAs: token tau(jr) of the step
  const int g_a = jr >> 3, h_a = (jr >> 2) & 1, t_a = jr & 3;
  const int tau = 16 * (g_a >> 1) + 8 * h_a + 4 * (g_a & 1) + t_a;
  const int kblk = tau >> 4, ktok = tau & 15;
  // transpose-read address of V: token 8hh + 4z + (n >> 2) of a block, dims
  // 32e + 16 (jr >> 4) + 4 (n & 3) .. + 3, with n = lane % 16
  const int nl = lane & 15;
  auto vaddr = [&](const StageBuf& cur, int blk, int z, int e) -> const char* {
    const int vtok = 8 * hh + 4 * z + (nl >> 2);
    const int chunk = 4 * e + 2 * (jr >> 4) + ((nl & 3) >> 1);
    return reinterpret_cast<const char*>(&cur[1][blk][vtok * 16 + (chunk ^ swz(vtok))]) +
           8 * (nl & 1);
  };

  // additive mask of row jr for the step of blocks bp, bp + 1 of a stage:
  // tokens 8hh .. 8hh + 7 of each block, bounded by its valid tokens
  float mk_next[16];
  auto load_step_mask = [&](const int (&ntok)[SB], const int (&tok0)[SB], int bp) {
    if constexpr (kMask) {
      // (plain loads: the row differs between lanes; past the block's last
      // valid token the index is clamped to it)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int nt = ntok[bp + u];
        const int last = max(nt - 1, 0);
        const MaskRow mb = mrow + tok0[bp + u];
#pragma unroll
        for (int i = 0; i < 8; ++i) mk_next[8 * u + i] = nt > 0 ? mb[min(8 * hh + i, last)] : 0.f;
      }
    }
  };

  // the first stage's loads
  {
    OwnBlock ob;
    if (nstage > 0) {
      view_stage(0, vnt[0], vt0[0], ob);
      dma_stage(ob, lds0);
      if (wave_rows) load_step_mask(vnt[0], vt0[0], 0);
    }
  }
  // causal: the workgroup's last query position; stages starting past it
  // add nothing for any of its rows (a causal call lists a launch's pages in
  // token order, so tokens only grow along the walk), and the walk ends
  // there (uniform across the workgroup)
  const int qrow_end = min(G * S, (int)(blockIdx.y / p.Hkv + 1) * NW * kChunk32Rows);
  const int s_last_wg = (qrow_end - 1) / G + coff;
  bool done = false;
  // stage st (view slot K = st % 2) computes from `cur` while the loads of
  // stage st + 1 go into `nxt` (the buffer stage st - 1 computed from)
  auto stage = [&](int st, auto kslot, const StageBuf& cur, StageBuf& nxt) {
    constexpr int K = decltype(kslot)::value;
    const int (&ntok_c)[SB] = vnt[K];
    const int (&tok0_c)[SB] = vt0[K];
    if constexpr (kCausal) {
      if (tok0_c[0] > s_last_wg) {
        __builtin_amdgcn_s_waitcnt(0x0F70);   // this stage's loads land before the exit
        done = true;
        return;
      }
    }
    // stage st is in LDS (this wave's loads done, then everyone's), and every
    // wave is done with the other buffer, which the next stage's loads fill
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();
    if (st + 1 < nstage) {
      OwnBlock ob;
      view_stage(st + 1, vnt[K ^ 1], vt0[K ^ 1], ob);
      dma_stage(ob, nxt);
    }
    if (wave_rows) {
      // q . k of the step of blocks bp, bp + 1: S^T for the wave's 32 rows
      auto qk = [&](int bp) -> mf_f32x16 {
        mf_f32x16 sc;
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] = 0.f;
        // every K operand read issued before the first MFMA (one LDS wait,
        // then the eight MFMAs back to back), registers allowing: with a mask
        // operand its prefetched values take them, and the compiler's order
        // stays
        mf_u32x4 ka[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          ka[i] = cur[0][bp + kblk][ktok * 16 + ((2 * i + hh) ^ swz(ktok))];
        if constexpr (!kMask)
          __builtin_amdgcn_sched_barrier(0);   // (keeps the reads ahead of the MFMAs)
#pragma unroll
        for (int i = 0; i < 8; ++i) sc = M32::mma(ka[i], qop[i], sc);
        return sc;
      };
      // steps that add exactly nothing for any row of the wave are skipped
      // (uniform tests): both blocks empty (an empty block holds zeros and
      // -inf logits), or, causal, every token past the wave's last query
      // position
      auto idle_step = [&](int bp) -> bool {
        const int nt0 = ntok_c[bp], nt1 = ntok_c[bp + 1];
        if (nt0 == 0 && nt1 == 0) return true;
        if constexpr (kCausal)
          return (nt0 == 0 || tok0_c[bp] > s_last) &&
                 (nt1 == 0 || tok0_c[bp + 1] > s_last);
        return false;
      };
      // logits, online softmax and P . V of one step
      auto finish = [&](int bp, const mf_f32x16& sc, const float* mk) {
        const int nt0 = ntok_c[bp], nt1 = ntok_c[bp + 1];
        float x[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float val;
          if constexpr (kCap)
            val = tanhf(sc[r] * scale * inv_cap) * cap2;
          else
            val = sc[r] * scale2;
          // finfo.min masks stay finite, as in natural units (a row masked
          // everywhere gets equal weights, as HELM's loop gives it)
          if constexpr (kMask) val = fmaxf(fmaf(mk[r], kLog2E, val), -__FLT_MAX__);
          x[r] = val;
        }
        // the per-token limits, only where a step reaches them (uniform tests):
        // the causal limit when a block's last token is past the wave's first
        // query position, the valid-token limit when a block is partial
        if constexpr (kCausal) {
          if (__builtin_expect(max(tok0_c[bp], tok0_c[bp + 1]) + kBlockTok - 1 > s_first, 0)) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if (tok0_c[bp + (r >> 3)] + 8 * hh + (r & 7) > s_vis) x[r] = -INFINITY;
          }
        }
        if (__builtin_expect(nt0 < kBlockTok || nt1 < kBlockTok, 0)) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (8 * hh + (r & 7) >= ((r >> 3) ? nt1 : nt0)) x[r] = -INFINITY;
        }
        float bm = x[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) bm = fmaxf(bm, x[r]);
        if (__builtin_expect(__builtin_amdgcn_ballot_w64(bm > m + kMfmaSlack) != 0, 0)) {
          // refresh the row max (both halves of the row agree)
          const float mn = fmaxf(m, fmaxf(bm, __shfl_xor(bm, 32, 64)));
          const float a = sexp(m - ((mn == -INFINITY) ? 0.f : mn));
#if HELM_CHUNK32_HILO
          lsum *= a;
#else
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int t = 0; t < 4; ++t) osum[4 * g + t] *= __shfl(a, 8 * g + 4 * hh + t, 64);
#endif
          m = mn;
          // O register 4g + t is row 8g + 4hh + t: that row's factor
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const float ar = __shfl(a, 8 * g + 4 * hh + t, 64);
#pragma unroll
              for (int e = 0; e < 4; ++e) o[e][4 * g + t] *= ar;
            }
        }
        const float base = (m == -INFINITY) ? 0.f : m;
        uint32_t hw[8], lw[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const float w0 = sexp(x[2 * q] - base), w1 = sexp(x[2 * q + 1] - base);
#if HELM_CHUNK32_HILO
          lsum += w0 + w1;
          Ops::split2(w0, w1, hw[q], lw[q]);
#else
          hw[q] = Ops::pk(w0, w1);
          lw[q] = 0u;
#endif
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const mf_u32x4 phi = mf_u32x4{hw[4 * u], hw[4 * u + 1], hw[4 * u + 2], hw[4 * u + 3]};
          const mf_u32x4 plo = mf_u32x4{lw[4 * u], lw[4 * u + 1], lw[4 * u + 2], lw[4 * u + 3]};
          mf_u32x4 vop[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint2 a0 = ld_tr16(vaddr(cur, bp + u, 0, e));
            const uint2 a1 = ld_tr16(vaddr(cur, bp + u, 1, e));
            vop[e] = mf_u32x4{a0.x, a0.y, a1.x, a1.y};
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = M32::mma(phi, vop[e], o[e]);
#if HELM_CHUNK32_HILO
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = M32::mma(plo, vop[e], o[e]);
#else
          (void)plo;
          osum = M32::mma(phi, ones, osum);
#endif
        }
      };
      {
#pragma unroll
        for (int bp = 0; bp < SB; bp += 2) {     // the step's blocks bp, bp + 1
          // the mask of the next step is loaded now, one step ahead of its use
          float mk[16];
          if constexpr (kMask) {
#pragma unroll
            for (int r = 0; r < 16; ++r) mk[r] = mk_next[r];
            if (bp + 2 < SB)
              load_step_mask(ntok_c, tok0_c, bp + 2);
            else if (st + 1 < nstage)
              load_step_mask(vnt[K ^ 1], vt0[K ^ 1], 0);
          }
          if (__builtin_expect(idle_step(bp), 0)) continue;
          // masked, a step whose every mask value is <= -1e30 while every
          // row's max is already above -1e20 adds exactly nothing (each
          // weight underflows to 0 and the max stays)
          if constexpr (kMask) {
            float mm = mk[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) mm = fmaxf(mm, mk[r]);
            if (!__builtin_amdgcn_ballot_w64(mm > -1e30f) &&
                !__builtin_amdgcn_ballot_w64(m <= -1e20f))
              continue;
          }
          finish(bp, qk(bp), mk);
        }
      }
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  for (int st = 0; st < nstage && !done; st += 2) {
    stage(st, I0{}, lds0, lds1);
    if (st + 1 < nstage && !done) stage(st + 1, I1{}, lds1, lds0);
  }

  if (!wave_rows) return;
#if HELM_CHUNK32_HILO
  const float lrow = lsum + __shfl_xor(lsum, 32, 64);     // row jr's sum
#else
  // row jr's sum: held by the half hh = (jr >> 2) & 1, register 4 (jr >> 3) + (jr & 3)
  float lself = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r)
    if (r == 4 * (jr >> 3) + (jr & 3)) lself = osum[r];
  const float lother = __shfl_xor(lself, 32, 64);
  const float lrow = (((jr >> 2) & 1) == hh) ? lself : lother;
#endif
  if (p.direct_out) {
    // the call's only split: normalized rows straight to the output
    // (HELM's final out / max(sum, 1e-12), kv_cache.py:554-555)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int i = 8 * g + 4 * hh + t;
#if HELM_CHUNK32_HILO
        const float inv = 1.f / fmaxf(__shfl(lrow, i, 64), 1e-12f);
#else
        const float inv = 1.f / fmaxf(osum[4 * g + t], 1e-12f);
#endif
        if (i < nrows)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            *out_elem(g, t, e) = static_cast<uint16_t>(Ops::pk(o[e][4 * g + t] * inv, 0.f));
      }
    return;
  }
  // partials (m, l, o[128]) of the wave's rows in their 16-row tiles
  auto part_row = [&](int i) -> int64_t {
    return ((int64_t)(tile0 + (i >> 4)) * p.max_splits + split) * p.rows_per_tile + (i & 15);
  };
  const float m_nat = m * kLn2;   // the partials' max in natural units
  if (hh == 0 && jr < nrows)
    *reinterpret_cast<float2*>(&p.ws_ml[part_row(jr) * 2]) = make_float2(m_nat, lrow);
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int i = 8 * g + 4 * hh + t;
      if (i < nrows) {
        float* dst = &p.ws_o[part_row(i) * 128 + jr];
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[32 * e] = o[e][4 * g + t];
      }
    }
}

}  // namespace helm
