// Split-K paged decode attention for gfx950 (CDNA4, wave64).
//
// Computes, for every sequence b, KV head hk and query row r of that head's
// group, softmax(q . K^T * scale [softcap] [+ mask]) . V over the sequence's
// pages — the arithmetic of HELM's perform_streaming_attention
// (helm/runtime/kv_cache.py:468-555 masked/online-softmax loop, :562-568 Path 1,
// :584-662 Path 3) with fp32 accumulation.
//
// Work decomposition
//   grid.x = split (a run of `pps` pages), grid.y = hk + Hkv * query-row tile,
//   grid.z = sequence.  256 threads = 4 waves; wave w takes the 16-token blocks
//   w, w+4, w+8 ... of its split.  Within a wave, DPP row r (16 lanes) owns
//   token 4j + r of the block (j = 0..3) and lane c of the row owns head dims
//   [c*EPL, c*EPL+EPL).  One 128-bit load per lane per j covers 1 KiB of a
//   page tile contiguously, so a 4 KiB (16 tok x 128 dim x bf16) tile is four
//   fully coalesced wave loads.
//   q.k partial sums are reduced across the 16 lanes of a row with four DPP
//   adds; every lane of the row then holds the exact same score, so each lane
//   keeps an online-softmax state (m, l, o[EPL]) over the tokens of its row
//   with no cross-row traffic in the loop.  All query heads of the GQA group
//   reuse every K/V tile from registers.
//   At the end the 16 row states are merged (shuffles, then LDS), each
//   workgroup writes one partial (m, l, o[D]) per row to the workspace, and
//   the last workgroup of a (sequence, head, tile) to arrive — found with an
//   agent-scope atomic ticket — merges all splits and writes the output.  The
//   ticket is reset by that workgroup, so the workspace needs zeroing once.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "helm_amd.h"

namespace helm {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kRowLanes = 16;   // lanes per token row (one DPP row)
constexpr int kBlockTok = 16;   // tokens per wave block (4 rows x 4 j)
constexpr int kMaxPps = 256;    // pages per split held in LDS

// ---- element types ----------------------------------------------------------
struct f16_t { uint16_t x; };
struct bf16_t { uint16_t x; };

template <typename T> struct ElemBytes;
template <> struct ElemBytes<f16_t> { static constexpr int v = 2; };
template <> struct ElemBytes<bf16_t> { static constexpr int v = 2; };
template <> struct ElemBytes<float> { static constexpr int v = 4; };

// Raw register image of NB bytes (NB >= 2).
template <int NB> struct Raw { uint32_t w[(NB + 3) / 4]; };

template <int NB>
__device__ __forceinline__ Raw<NB> load_raw(const char* p) {
  Raw<NB> r;
  if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      uint4 v = *reinterpret_cast<const uint4*>(p + 16 * i);
      r.w[4 * i + 0] = v.x; r.w[4 * i + 1] = v.y;
      r.w[4 * i + 2] = v.z; r.w[4 * i + 3] = v.w;
    }
  } else if constexpr (NB == 8) {
    uint2 v = *reinterpret_cast<const uint2*>(p);
    r.w[0] = v.x; r.w[1] = v.y;
  } else if constexpr (NB == 4) {
    r.w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else {
    static_assert(NB == 2, "unsupported raw width");
    r.w[0] = *reinterpret_cast<const uint16_t*>(p);
  }
  return r;
}

template <int NB>
__device__ __forceinline__ Raw<NB> zero_raw() {
  Raw<NB> r;
#pragma unroll
  for (int i = 0; i < (NB + 3) / 4; ++i) r.w[i] = 0u;
  return r;
}

// Element e of a raw image, widened to fp32 (exact for all three types).
template <typename T, int NB>
__device__ __forceinline__ float elem_f32(const Raw<NB>& r, int e) {
  if constexpr (ElemBytes<T>::v == 4) {
    return __uint_as_float(r.w[e]);
  } else {
    const uint32_t word = r.w[e >> 1];
    const uint32_t h = (e & 1) ? (word >> 16) : (word & 0xffffu);
    if constexpr (sizeof(T) == 2 && __is_same(T, bf16_t)) {
      return __uint_as_float(h << 16);
    } else {
      _Float16 hv = __builtin_bit_cast(_Float16, static_cast<uint16_t>(h));
      return static_cast<float>(hv);
    }
  }
}

// Loads element-by-element (any alignment, any D) into a raw image.
template <typename T, int EPL>
__device__ __forceinline__ Raw<EPL * ElemBytes<T>::v> load_elems(
    const char* p, int n_valid) {
  constexpr int EB = ElemBytes<T>::v;
  Raw<EPL * EB> r = zero_raw<EPL * EB>();
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    if (e < n_valid) {
      if constexpr (EB == 4) {
        r.w[e] = *reinterpret_cast<const uint32_t*>(p + 4 * e);
      } else {
        const uint32_t h = *reinterpret_cast<const uint16_t*>(p + 2 * e);
        r.w[e >> 1] |= (e & 1) ? (h << 16) : h;
      }
    }
  }
  return r;
}

template <typename T>
__device__ __forceinline__ void store_elem(char* p, float v);
template <>
__device__ __forceinline__ void store_elem<float>(char* p, float v) {
  *reinterpret_cast<float*>(p) = v;
}
template <>
__device__ __forceinline__ void store_elem<f16_t>(char* p, float v) {
  _Float16 h = static_cast<_Float16>(v);  // round to nearest even
  *reinterpret_cast<uint16_t*>(p) = __builtin_bit_cast(uint16_t, h);
}
template <>
__device__ __forceinline__ void store_elem<bf16_t>(char* p, float v) {
  // round to nearest even; NaN kept quiet
  uint32_t u = __float_as_uint(v);
  uint32_t out;
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
    out = (u >> 16) | 0x40u;
  } else {
    out = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  }
  *reinterpret_cast<uint16_t*>(p) = static_cast<uint16_t>(out);
}

// ---- packed dot products (exact products, fp32 accumulate) ---------------
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc);
template <>
__device__ __forceinline__ float dot2<bf16_t>(uint32_t a, uint32_t b,
                                              float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc,
                                         false);
}
template <>
__device__ __forceinline__ float dot2<f16_t>(uint32_t a, uint32_t b,
                                             float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a),
                                __builtin_bit_cast(f16x2_t, b), acc, false);
}

// ---- DPP row (16-lane) sum -------------------------------------------------
// quad_perm[1,0,3,2], quad_perm[2,3,0,1], row_half_mirror, row_mirror: after
// the four steps every lane of the row holds the same (commutative) sum.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(
      __builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row_sum16(float x) {
  x += dpp_mov<0xB1>(x);
  x += dpp_mov<0x4E>(x);
  x += dpp_mov<0x141>(x);
  x += dpp_mov<0x140>(x);
  return x;
}

// exp(x) for x <= 0 or -inf (returns 0 for -inf).
__device__ __forceinline__ float fexp(float x) { return __expf(x); }

// ---- page sources -----------------------------------------------------------
struct PageView {
  const char* k;     // head hk, token 0
  const char* v;
  int used;
  int tok_off;
  int head_stride_b;  // unused once the head offset is folded in
};

// vLLM-style pool: slot s at base + s*slot_stride (bytes), int32 page table.
struct PoolSrc {
  const char* k_pool;
  const char* v_pool;
  int64_t slot_stride_b;
  int64_t head_stride_b;
  const int32_t* table;
  int table_stride;
  const int32_t* seq_lens;
  int page_size;
  int max_pages;  // table columns the caller declared; bounds every walk

  __device__ __forceinline__ int n_pages(int b) const {
    const int T = seq_lens[b];
    return T > 0 ? min((T + page_size - 1) / page_size, max_pages) : 0;
  }
  __device__ __forceinline__ PageView page(int b, int p, int hk) const {
    const int slot = table[(int64_t)b * table_stride + p];
    const int T = seq_lens[b];
    PageView pv;
    const int64_t off = (int64_t)slot * slot_stride_b + hk * head_stride_b;
    pv.k = k_pool + off;
    pv.v = v_pool + off;
    pv.tok_off = p * page_size;
    pv.used = min(page_size, T - pv.tok_off);
    pv.head_stride_b = 0;
    return pv;
  }
};

// Explicit page descriptors (device addresses), sequence b owns
// pages[seq_off[b] .. seq_off[b+1]).
struct DescSrc {
  const helm_page* pages;
  const int32_t* seq_off;
  int elem_bytes;

  __device__ __forceinline__ int n_pages(int b) const {
    return seq_off[b + 1] - seq_off[b];
  }
  __device__ __forceinline__ PageView page(int b, int p, int hk) const {
    const helm_page d = pages[seq_off[b] + p];
    PageView pv;
    const int64_t off = (int64_t)hk * d.head_stride * elem_bytes;
    pv.k = reinterpret_cast<const char*>(d.k) + off;
    pv.v = reinterpret_cast<const char*>(d.v) + off;
    pv.used = d.used;
    pv.tok_off = d.tok_off;
    pv.head_stride_b = 0;
    return pv;
  }
};

// ---- launch parameters ------------------------------------------------------
struct AttnParams {
  const void* q;
  void* out;
  int B, Hq, Hkv, G, S, D;
  int rows_per_tile;  // query rows per workgroup tile (= GM)
  int n_qtiles;
  float scale;
  float softcap;      // <= 0: off
  const float* mask;  // may be null
  int64_t mask_bstride, mask_hstride, mask_qstride;
  int causal;         // top-left causal over key positions
  int pps;            // pages per split
  int bpp;            // 16-token blocks per page
  int lo, hi;         // page range of this launch within every sequence
  int split_base;     // global index of this launch's first split
  int total_splits;   // > 0: splits of the whole call (chained launches)
  int max_splits;     // stride of the partial buffers
  int full_d;         // D == 16*EPL and 16-byte friendly addresses
  float* ws_o;        // [tiles][max_splits][GM][D]
  float* ws_ml;       // [tiles][max_splits][GM][2]
  uint32_t* tickets;  // [tiles]
};

// Per-workgroup LDS.
template <int GM, int DMAX>
struct Smem {
  const char* pk[kMaxPps];
  const char* pv[kMaxPps];
  int used[kMaxPps];
  int tok_off[kMaxPps];
  float o[kWaves][GM][DMAX];
  float m[kWaves][GM];
  float l[kWaves][GM];
  int last;
};

template <typename TKV, typename TQ, int EPL, int GM, bool DOT2, class Src>
__global__ __launch_bounds__(kThreads) void paged_attn_kernel(AttnParams p,
                                                               Src src) {
  constexpr int EB = ElemBytes<TKV>::v;
  constexpr int QB = ElemBytes<TQ>::v;
  constexpr int NB = EPL * EB;       // bytes per lane per token row
  constexpr int DMAX = kRowLanes * EPL;
  static_assert(!DOT2 || (EB == 2 && QB == 2), "dot2 needs 16-bit q and kv");

  __shared__ Smem<GM, DMAX> sm;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int row = lane >> 4;
  const int col = lane & 15;

  const int split_local = blockIdx.x;
  const int hk = blockIdx.y % p.Hkv;
  const int qt = blockIdx.y / p.Hkv;
  const int b = blockIdx.z;
  const int tile = (b * p.Hkv + hk) * p.n_qtiles + qt;

  const int D = p.D;
  const int S = p.S;
  const int G = p.G;
  const int nrows_total = G * S;
  const int r0 = qt * GM;
  const int nrows = min(GM, nrows_total - r0);

  // ---- this workgroup's page range -----------------------------------------
  const int np = src.n_pages(b);
  const int lo = min(p.lo, np);
  const int hi = min(p.hi, np);
  const int nsplit_launch = (hi - lo + p.pps - 1) / p.pps;
  const int total = p.total_splits > 0 ? p.total_splits : nsplit_launch;

  if (total == 0) {
    // Sequence without active tokens: zeros (HELM kv_cache.py:441-442).
    if (split_local == 0) {
      for (int idx = tid; idx < nrows * D; idx += kThreads) {
        const int rr = r0 + idx / D;
        const int g = rr / S, s = rr % S;
        const int h = hk * G + g;
        const int64_t o_off = ((int64_t)(b * p.Hq + h) * S + s) * D + idx % D;
        store_elem<TQ>(reinterpret_cast<char*>(p.out) + o_off * QB, 0.f);
      }
    }
    return;
  }
  if (split_local >= nsplit_launch) return;
  const int split = p.split_base + split_local;
  const int pg0 = lo + split_local * p.pps;
  const int pg1 = min(pg0 + p.pps, hi);
  const int npg = pg1 - pg0;

  // ---- page addresses of the split into LDS --------------------------------
  for (int i = tid; i < npg; i += kThreads) {
    PageView pv = src.page(b, pg0 + i, hk);
    sm.pk[i] = pv.k;
    sm.pv[i] = pv.v;
    sm.used[i] = pv.used;
    sm.tok_off[i] = pv.tok_off;
  }

  // ---- query rows into registers -------------------------------------------
  const int d0 = col * EPL;
  const int dvalid = max(0, min(EPL, D - d0));
  Raw<EPL * QB> qraw[GM];
  float qf[DOT2 ? 1 : GM][DOT2 ? 1 : EPL];
  int64_t mrow[GM];
  int srow[GM];
#pragma unroll
  for (int g = 0; g < GM; ++g) {
    const int rr = r0 + (g < nrows ? g : 0);
    const int gg = rr / S, s = rr % S;
    const int h = hk * G + gg;
    srow[g] = s;
    mrow[g] = (int64_t)b * p.mask_bstride + (int64_t)h * p.mask_hstride +
              (int64_t)s * p.mask_qstride;
    const char* qp = reinterpret_cast<const char*>(p.q) +
                     (((int64_t)(b * p.Hq + h) * S + s) * D + d0) * QB;
    if (p.full_d) {
      qraw[g] = load_raw<EPL * QB>(qp);
    } else {
      qraw[g] = load_elems<TQ, EPL>(qp, dvalid);
    }
    if constexpr (!DOT2) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) qf[g][e] = elem_f32<TQ>(qraw[g], e);
    }
  }

  float m[GM], l[GM], o[GM][EPL];
#pragma unroll
  for (int g = 0; g < GM; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[g][e] = 0.f;
  }

  __syncthreads();

  const bool has_mask = p.mask != nullptr;
  const bool has_cap = p.softcap > 0.f;
  const float scale = p.scale;
  const float cap = p.softcap;
  const float inv_cap = has_cap ? 1.f / cap : 0.f;
  const int64_t row_bytes = (int64_t)D * EB;
  const int nblk = npg * p.bpp;

  auto load_block = [&](int bi, Raw<NB> (&kr)[4], Raw<NB> (&vr)[4]) {
    const int pi = bi / p.bpp;
    const int sub = bi - pi * p.bpp;
    const int used = sm.used[pi];
    const char* kb = sm.pk[pi];
    const char* vb = sm.pv[pi];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = sub * kBlockTok + 4 * j + row;
      if (t < used) {
        const int64_t off = (int64_t)t * row_bytes + (int64_t)d0 * EB;
        if (p.full_d) {
          kr[j] = load_raw<NB>(kb + off);
          vr[j] = load_raw<NB>(vb + off);
        } else {
          kr[j] = load_elems<TKV, EPL>(kb + off, dvalid);
          vr[j] = load_elems<TKV, EPL>(vb + off, dvalid);
        }
      } else {
        kr[j] = zero_raw<NB>();
        vr[j] = zero_raw<NB>();
      }
    }
  };

  auto compute_block = [&](int bi, const Raw<NB> (&kr)[4],
                           const Raw<NB> (&vr)[4]) {
    const int pi = bi / p.bpp;
    const int sub = bi - pi * p.bpp;
    const int used = sm.used[pi];
    const int tok_base = sm.tok_off[pi];
    float sc[GM][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DOT2) {
#pragma unroll
        for (int g = 0; g < GM; ++g) {
          float acc = 0.f;
#pragma unroll
          for (int w = 0; w < NB / 4; ++w)
            acc = dot2<TKV>(kr[j].w[w], qraw[g].w[w], acc);
          sc[g][j] = acc;
        }
      } else {
        float kf[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) kf[e] = elem_f32<TKV>(kr[j], e);
#pragma unroll
        for (int g = 0; g < GM; ++g) {
          float acc = 0.f;
#pragma unroll
          for (int e = 0; e < EPL; ++e) acc = fmaf(qf[g][e], kf[e], acc);
          sc[g][j] = acc;
        }
      }
    }
#pragma unroll
    for (int g = 0; g < GM; ++g)
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[g][j] = row_sum16(sc[g][j]);

    float vf[4][EPL];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < EPL; ++e) vf[j][e] = elem_f32<TKV>(vr[j], e);

#pragma unroll
    for (int g = 0; g < GM; ++g) {
      float s4[4];
      float bm = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = sub * kBlockTok + 4 * j + row;
        float s = sc[g][j] * scale;
        if (has_cap) s = tanhf(s * inv_cap) * cap;
        // clamp keeps the mask read inside the page's tokens
        const int tpos = tok_base + min(t, used - 1);
        if (has_mask) s += p.mask[mrow[g] + tpos];
        if (p.causal && tpos > srow[g]) s = -INFINITY;
        if (t >= used) s = -INFINITY;
        s4[j] = s;
        bm = fmaxf(bm, s);
      }
      const float mn = fmaxf(m[g], bm);
      const float base = (mn == -INFINITY) ? 0.f : mn;
      const float alpha = fexp(m[g] - base);
      float ps = 0.f;
      float pj[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pj[j] = fexp(s4[j] - base);
        ps += pj[j];
      }
      l[g] = l[g] * alpha + ps;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        float acc = o[g][e] * alpha;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = fmaf(pj[j], vf[j][e], acc);
        o[g][e] = acc;
      }
      m[g] = mn;
    }
  };

  // ---- main loop: two register buffers, next block's loads in flight ------
  {
    Raw<NB> ka[4], va[4], kb2[4], vb2[4];
    int bi = wave;
    if (bi < nblk) load_block(bi, ka, va);
    while (bi < nblk) {
      const int bn = bi + kWaves;
      if (bn < nblk) load_block(bn, kb2, vb2);
      compute_block(bi, ka, va);
      bi = bn;
      if (bi >= nblk) break;
      const int bn2 = bi + kWaves;
      if (bn2 < nblk) load_block(bn2, ka, va);
      compute_block(bi, kb2, vb2);
      bi = bn2;
    }
  }

  // ---- merge the 4 row states of the wave (lanes xor 16, xor 32) ----------
#pragma unroll
  for (int step = 16; step <= 32; step <<= 1) {
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      const float m2 = __shfl_xor(m[g], step, 64);
      const float l2 = __shfl_xor(l[g], step, 64);
      const float mn = fmaxf(m[g], m2);
      const float base = (mn == -INFINITY) ? 0.f : mn;
      const float a1 = fexp(m[g] - base);
      const float a2 = fexp(m2 - base);
      l[g] = l[g] * a1 + l2 * a2;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float o2 = __shfl_xor(o[g][e], step, 64);
        o[g][e] = o[g][e] * a1 + o2 * a2;
      }
      m[g] = mn;
    }
  }
  if (row == 0) {
#pragma unroll
    for (int g = 0; g < GM; ++g) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) sm.o[wave][g][d0 + e] = o[g][e];
      if (col == 0) {
        sm.m[wave][g] = m[g];
        sm.l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();

  // ---- merge the 4 waves, write this split's partial ------------------------
  const int64_t part = ((int64_t)tile * p.max_splits + split) * GM;
  for (int idx = tid; idx < nrows * D; idx += kThreads) {
    const int g = idx / D;
    const int d = idx - g * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm.m[w][g]);
    const float base = (M == -INFINITY) ? 0.f : M;
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float a = fexp(sm.m[w][g] - base);
      L += a * sm.l[w][g];
      O += a * sm.o[w][g][d];
    }
    p.ws_o[(part + g) * D + d] = O;
    if (d == 0) {
      p.ws_ml[(part + g) * 2 + 0] = M;
      p.ws_ml[(part + g) * 2 + 1] = L;
    }
  }

  // ---- ticket: the last split of the tile merges -----------------------------
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = atomicAdd(&p.tickets[tile], 1u);
    sm.last = (prev == static_cast<uint32_t>(total - 1)) ? 1 : 0;
  }
  __syncthreads();
  if (!sm.last) return;
  __threadfence();

  const int64_t part0 = (int64_t)tile * p.max_splits * GM;
  for (int idx = tid; idx < nrows * D; idx += kThreads) {
    const int g = idx / D;
    const int d = idx - g * D;
    float M = -INFINITY;
    for (int sp = 0; sp < total; ++sp)
      M = fmaxf(M, p.ws_ml[(part0 + (int64_t)sp * GM + g) * 2]);
    const float base = (M == -INFINITY) ? 0.f : M;
    float L = 0.f, O = 0.f;
    for (int sp = 0; sp < total; ++sp) {
      const int64_t pi = part0 + (int64_t)sp * GM + g;
      const float ms = p.ws_ml[pi * 2];
      const float ls = p.ws_ml[pi * 2 + 1];
      const float os = p.ws_o[pi * D + d];
      const float a = fexp(ms - base);
      L += a * ls;
      O += a * os;
    }
    const int rr = r0 + g;
    const int gg = rr / S, s = rr % S;
    const int h = hk * G + gg;
    const int64_t o_off = ((int64_t)(b * p.Hq + h) * S + s) * D + d;
    store_elem<TQ>(reinterpret_cast<char*>(p.out) + o_off * QB,
                   O / fmaxf(L, 1e-12f));
  }
  if (tid == 0) p.tickets[tile] = 0u;
}

// ---- host-side launch description -------------------------------------------
struct LaunchSpec {
  AttnParams p;
  int mode;           // 0 = pool, 1 = descriptors
  PoolSrc pool;
  DescSrc desc;
  int kv_dtype, q_dtype;
  int epl;            // elements per lane (D <= 16*epl)
  int gm;             // rows per tile
  int fast;           // exact-G dot2 kernel
  dim3 grid;
};

// Implemented per KV dtype in attn_f16.hip / attn_bf16.hip / attn_f32.hip.
hipError_t launch_attn_f16(const LaunchSpec& s, hipStream_t st);
hipError_t launch_attn_bf16(const LaunchSpec& s, hipStream_t st);
hipError_t launch_attn_f32(const LaunchSpec& s, hipStream_t st);

}  // namespace helm
