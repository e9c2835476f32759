// Streaming attention on the host CPU: the attention of HELM's CPU-stage
// layers, a query on the CPU over KV pages in host memory.
//
// HELM computes it with PyTorch on the CPU.  With a mask or soft-cap it runs
// the per-page fp32 online-softmax loop (helm/runtime/kv_cache.py:468-555, the
// CPU branch :531-552).  Without them it takes Path 2: concatenate every page,
// widen to fp32, repeat the KV heads up to the query heads, one fp32 SDPA
// (:573-577).  A first prompt chunk runs SDPA over its own K/V
// (helm/runtime/kv_offload.py:330-338).  All of them are
// softmax(q k^T * scale [soft-cap] [+ mask]) v with fp32 arithmetic.  Here:
//
// * one pass over a KV head's pages serves every query row that reads it (the
//   G = Hq / Hkv query heads of the group times the query positions), so the
//   K/V bytes are read once per tile of rows rather than G times after a
//   repeat, and are widened to fp32 only a 16-token block at a time (L1);
// * per block and row: 16 dot products (vector FMAs over D; the 16 sums are
//   reduced together so that lane j holds token j's logit), scale, soft-cap,
//   additive mask, the online max / exp / sum update with exp evaluated on
//   16 lanes at once, and the P.V accumulation into the row's fp32 output;
// * work items are (sequence, KV head, tile of up to 32 rows, split of the
//   sequence's pages) on OpenMP threads; a decode call (few rows per KV head)
//   splits each sequence's pages so that it still occupies the cores, and the
//   splits' partial (max, sum, output) rows are merged at the end;
// * AVX-512 where the CPU has it (16 lanes), else AVX2 + F16C + FMA (two
//   8-lane halves); the algorithm (attn_core.inc) is compiled once per set.
//
// Bound: host DRAM bandwidth in decode (each K/V byte read once per call);
// the FMA units for long prompt chunks (4 * rows * D flops per token).
#include "helm_cpu.h"
#include "common.h"

#include <immintrin.h>
#include <omp.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

namespace {

using helm_cpu_internal::fail;

constexpr int kMaxD = 512;
constexpr int kTileRows = 32;

constexpr size_t dtsize(int dt) { return dt == HELM_CPU_F32 ? 4 : 2; }

struct Job {
  const void* q;
  void* out;
  int B, Hq, Hkv, S, D, Dp, G, R, RT, ntiles, nsplit;
  const helm_cpu_page* pages;
  const int32_t* seq_off;
  float scale, softcap;
  const float* mask;
  int64_t mbs, mhs, mqs;
  int causal, kv_dtype, q_dtype;
  float* part;   // split partials (nsplit > 1): per item RT rows of m, RT of l, RT x Dp of o
};

// Rows of KV head kvh are ordered r = g * S + s: query head kvh * G + g,
// query position s.  Returns the row's index in the [B, Hq, S] query.
inline int64_t row_index(const Job& J, int b, int kvh, int r) {
  const int g = r / J.S, s = r - g * J.S;
  return ((int64_t)b * J.Hq + (int64_t)kvh * J.G + g) * J.S + s;
}

__attribute__((target("f16c"))) inline float widen1(const char* p, int d, int dt) {
  if (dt == HELM_CPU_F32) return reinterpret_cast<const float*>(p)[d];
  const uint16_t h = reinterpret_cast<const uint16_t*>(p)[d];
  if (dt == HELM_CPU_F16) return _cvtsh_ss(h);
  const uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// fp32 -> bf16, round to nearest even (a NaN stays a quiet NaN)
inline uint16_t to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__attribute__((target("f16c"))) void narrow_row(const float* src, void* out, int64_t off, int D,
                                                int dt) {
  if (dt == HELM_CPU_F32) {
    std::memcpy(static_cast<float*>(out) + off, src, (size_t)D * 4);
  } else if (dt == HELM_CPU_F16) {
    uint16_t* o = static_cast<uint16_t*>(out) + off;
    for (int d = 0; d < D; ++d) o[d] = _cvtss_sh(src[d], _MM_FROUND_TO_NEAREST_INT);
  } else {
    uint16_t* o = static_cast<uint16_t*>(out) + off;
    for (int d = 0; d < D; ++d) o[d] = to_bf16(src[d]);
  }
}

// exp(x) on vector lanes, from the Cody-Waite reduction x = n ln2 + r
// (|r| <= ln2 / 2; ln2 split into a 15-bit head, exact times any n here, and
// its remainder) and the degree-7 Taylor polynomial of e^r, whose truncation
// error (r^8 / 8! <= 5.1e-9) is below fp32 rounding; e^x = 2^n e^r.  Lanes
// below ln(FLT_MIN) (and -inf) give 0.
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2Hi = 0.693145751953125f;
constexpr float kLn2Lo = 1.4286068203094173e-6f;
constexpr float kExpLow = -87.33654475f;
constexpr float kInvFact[8] = {1.f,           1.f,           0.5f,          1.f / 6.f,
                               1.f / 24.f,    1.f / 120.f,   1.f / 720.f,   1.f / 5040.f};

}  // namespace

// ---- AVX-512: F is one 16-lane register ------------------------------------------
#pragma GCC push_options
#pragma GCC target("avx512f,avx512bw,avx512vl,avx2,f16c,fma")
namespace isa_avx512 {
namespace {

struct F {
  __m512 v;
};
inline F f_zero() { return {_mm512_setzero_ps()}; }
inline F f_set1(float x) { return {_mm512_set1_ps(x)}; }
inline F f_load(const float* p) { return {_mm512_loadu_ps(p)}; }
inline void f_store(float* p, F a) { _mm512_storeu_ps(p, a.v); }
inline F f_fma(F a, F b, F c) { return {_mm512_fmadd_ps(a.v, b.v, c.v)}; }
inline F f_mul(F a, F b) { return {_mm512_mul_ps(a.v, b.v)}; }
inline F f_add(F a, F b) { return {_mm512_add_ps(a.v, b.v)}; }
inline F f_sub(F a, F b) { return {_mm512_sub_ps(a.v, b.v)}; }
inline float f_hmax(F a) { return _mm512_reduce_max_ps(a.v); }
inline float f_hsum(F a) { return _mm512_reduce_add_ps(a.v); }
inline __mmask16 first(int n) { return n >= 16 ? (__mmask16)0xffff : (__mmask16)((1u << n) - 1u); }
// lanes >= n replaced by `fill`
inline F f_keep(F a, int n, float fill) {
  return {_mm512_mask_blend_ps(first(n), _mm512_set1_ps(fill), a.v)};
}
// lanes < n from p (nothing past p + n is read), the rest 0
inline F f_load_n(const float* p, int n) { return {_mm512_maskz_loadu_ps(first(n), p)}; }

// lane j of the result = the sum of acc[j]'s 16 lanes
inline F f_reduce16(const F* acc) {
  __m512 b[8], c[4];
  for (int i = 0; i < 8; ++i) {   // 128-bit lanes: [a.0+a.2, a.1+a.3, b.0+b.2, b.1+b.3]
    const __m512 x = acc[2 * i].v, y = acc[2 * i + 1].v;
    b[i] = _mm512_add_ps(_mm512_shuffle_f32x4(x, y, 0x44), _mm512_shuffle_f32x4(x, y, 0xEE));
  }
  for (int i = 0; i < 4; ++i)     // 128-bit lane k: four partial sums of acc[4i + k]
    c[i] = _mm512_add_ps(_mm512_shuffle_f32x4(b[2 * i], b[2 * i + 1], 0x88),
                         _mm512_shuffle_f32x4(b[2 * i], b[2 * i + 1], 0xDD));
  const __m512 d0 = _mm512_add_ps(_mm512_unpacklo_ps(c[0], c[1]), _mm512_unpackhi_ps(c[0], c[1]));
  const __m512 d1 = _mm512_add_ps(_mm512_unpacklo_ps(c[2], c[3]), _mm512_unpackhi_ps(c[2], c[3]));
  // lane 4k + m holds acc[4m + k]
  const __m512 e = _mm512_add_ps(_mm512_shuffle_ps(d0, d1, 0x44), _mm512_shuffle_ps(d0, d1, 0xEE));
  const __m512i idx = _mm512_setr_epi32(0, 4, 8, 12, 1, 5, 9, 13, 2, 6, 10, 14, 3, 7, 11, 15);
  return {_mm512_permutexvar_ps(idx, e)};
}

inline F f_exp(F x) {
  const __m512 t = _mm512_mul_ps(x.v, _mm512_set1_ps(kLog2e));
  const __m512 n = _mm512_roundscale_ps(t, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  __m512 r = _mm512_fnmadd_ps(n, _mm512_set1_ps(kLn2Hi), x.v);
  r = _mm512_fnmadd_ps(n, _mm512_set1_ps(kLn2Lo), r);
  __m512 p = _mm512_set1_ps(kInvFact[7]);
  for (int k = 6; k >= 0; --k) p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(kInvFact[k]));
  const __m512 e = _mm512_scalef_ps(p, n);
  const __mmask16 low = _mm512_cmp_ps_mask(x.v, _mm512_set1_ps(kExpLow), _CMP_LT_OQ);
  return {_mm512_mask_blend_ps(low, e, _mm512_setzero_ps())};
}

template <int DT>
inline F f_widen(const char* p) {
  if constexpr (DT == HELM_CPU_F32) {
    return {_mm512_loadu_ps(reinterpret_cast<const float*>(p))};
  } else {
    const __m256i h = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(p));
    if constexpr (DT == HELM_CPU_F16) return {_mm512_cvtph_ps(h)};
    return {_mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu16_epi32(h), 16))};
  }
}

#include "attn_core.inc"

}  // namespace

void run(const Job& J, int nt) {
  if (J.kv_dtype == HELM_CPU_F16) return run_all<HELM_CPU_F16>(J, nt);
  if (J.kv_dtype == HELM_CPU_BF16) return run_all<HELM_CPU_BF16>(J, nt);
  return run_all<HELM_CPU_F32>(J, nt);
}

}  // namespace isa_avx512
#pragma GCC pop_options

// ---- AVX2: F is two 8-lane halves ------------------------------------------------
#pragma GCC push_options
#pragma GCC target("avx2,f16c,fma")
namespace isa_avx2 {
namespace {

struct F {
  __m256 lo, hi;
};
inline F f_zero() { return {_mm256_setzero_ps(), _mm256_setzero_ps()}; }
inline F f_set1(float x) { return {_mm256_set1_ps(x), _mm256_set1_ps(x)}; }
inline F f_load(const float* p) { return {_mm256_loadu_ps(p), _mm256_loadu_ps(p + 8)}; }
inline void f_store(float* p, F a) {
  _mm256_storeu_ps(p, a.lo);
  _mm256_storeu_ps(p + 8, a.hi);
}
inline F f_fma(F a, F b, F c) {
  return {_mm256_fmadd_ps(a.lo, b.lo, c.lo), _mm256_fmadd_ps(a.hi, b.hi, c.hi)};
}
inline F f_mul(F a, F b) { return {_mm256_mul_ps(a.lo, b.lo), _mm256_mul_ps(a.hi, b.hi)}; }
inline F f_add(F a, F b) { return {_mm256_add_ps(a.lo, b.lo), _mm256_add_ps(a.hi, b.hi)}; }
inline F f_sub(F a, F b) { return {_mm256_sub_ps(a.lo, b.lo), _mm256_sub_ps(a.hi, b.hi)}; }
inline float hmax8(__m256 v) {
  __m128 s = _mm_max_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_max_ps(s, _mm_movehl_ps(s, s));
  s = _mm_max_ss(s, _mm_movehdup_ps(s));
  return _mm_cvtss_f32(s);
}
inline float hsum8(__m256 v) {
  __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_movehdup_ps(s));
  return _mm_cvtss_f32(s);
}
inline float f_hmax(F a) { return hmax8(_mm256_max_ps(a.lo, a.hi)); }
inline float f_hsum(F a) { return hsum8(_mm256_add_ps(a.lo, a.hi)); }
inline __m256 lanes_below(int n, int base) {
  const __m256i i = _mm256_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7);
  return _mm256_castsi256_ps(_mm256_cmpgt_epi32(_mm256_set1_epi32(n - base), i));
}
inline F f_keep(F a, int n, float fill) {
  const __m256 f = _mm256_set1_ps(fill);
  return {_mm256_blendv_ps(f, a.lo, lanes_below(n, 0)), _mm256_blendv_ps(f, a.hi, lanes_below(n, 8))};
}
inline F f_load_n(const float* p, int n) {
  if (n >= 16) return f_load(p);
  return {_mm256_maskload_ps(p, _mm256_castps_si256(lanes_below(n, 0))),
          _mm256_maskload_ps(p + 8, _mm256_castps_si256(lanes_below(n, 8)))};
}
// 8 vectors -> one vector of their 8 lane-sums
inline __m256 reduce8(const __m256* a) {
  const __m256 t0 = _mm256_hadd_ps(a[0], a[1]), t1 = _mm256_hadd_ps(a[2], a[3]);
  const __m256 t2 = _mm256_hadd_ps(a[4], a[5]), t3 = _mm256_hadd_ps(a[6], a[7]);
  const __m256 u0 = _mm256_hadd_ps(t0, t1), u1 = _mm256_hadd_ps(t2, t3);
  return _mm256_add_ps(_mm256_permute2f128_ps(u0, u1, 0x20), _mm256_permute2f128_ps(u0, u1, 0x31));
}
inline F f_reduce16(const F* acc) {
  __m256 h[16];
  for (int j = 0; j < 16; ++j) h[j] = _mm256_add_ps(acc[j].lo, acc[j].hi);
  return {reduce8(h), reduce8(h + 8)};
}
inline __m256 exp8(__m256 x) {
  const __m256 t = _mm256_mul_ps(x, _mm256_set1_ps(kLog2e));
  const __m256 n = _mm256_round_ps(t, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  __m256 r = _mm256_fnmadd_ps(n, _mm256_set1_ps(kLn2Hi), x);
  r = _mm256_fnmadd_ps(n, _mm256_set1_ps(kLn2Lo), r);
  __m256 p = _mm256_set1_ps(kInvFact[7]);
  for (int k = 6; k >= 0; --k) p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(kInvFact[k]));
  // 2^n from the exponent field; lanes below ln(FLT_MIN) are replaced by 0
  const __m256 low = _mm256_cmp_ps(x, _mm256_set1_ps(kExpLow), _CMP_LT_OQ);
  const __m256 nn = _mm256_blendv_ps(n, _mm256_setzero_ps(), low);
  const __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(nn), _mm256_set1_epi32(127)), 23);
  return _mm256_blendv_ps(_mm256_mul_ps(p, _mm256_castsi256_ps(e)), _mm256_setzero_ps(), low);
}
inline F f_exp(F x) { return {exp8(x.lo), exp8(x.hi)}; }

template <int DT>
inline F f_widen(const char* p) {
  if constexpr (DT == HELM_CPU_F32) {
    const float* f = reinterpret_cast<const float*>(p);
    return {_mm256_loadu_ps(f), _mm256_loadu_ps(f + 8)};
  } else {
    const __m128i a = _mm_loadu_si128(reinterpret_cast<const __m128i*>(p));
    const __m128i b = _mm_loadu_si128(reinterpret_cast<const __m128i*>(p + 16));
    if constexpr (DT == HELM_CPU_F16) return {_mm256_cvtph_ps(a), _mm256_cvtph_ps(b)};
    return {_mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(a), 16)),
            _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(b), 16))};
  }
}

#include "attn_core.inc"

}  // namespace

void run(const Job& J, int nt) {
  if (J.kv_dtype == HELM_CPU_F16) return run_all<HELM_CPU_F16>(J, nt);
  if (J.kv_dtype == HELM_CPU_BF16) return run_all<HELM_CPU_BF16>(J, nt);
  return run_all<HELM_CPU_F32>(J, nt);
}

}  // namespace isa_avx2
#pragma GCC pop_options

extern "C" int helm_cpu_stream_attn(const void* q, void* out, int B, int Hq, int Hkv, int q_len,
                                    int D, const helm_cpu_page* pages, const int32_t* seq_off,
                                    float scale, float softcap, const float* mask,
                                    int64_t mask_bstride, int64_t mask_hstride,
                                    int64_t mask_qstride, int causal, int kv_dtype, int q_dtype,
                                    int threads) {
  if (B < 0 || Hq < 1 || Hkv < 1 || q_len < 1 || D < 1)
    return fail(HELM_CPU_E_INVALID, "B must be >= 0; Hq, Hkv, q_len and D >= 1");
  if (B == 0) return HELM_CPU_OK;
  if (!q || !out || !seq_off) return fail(HELM_CPU_E_INVALID, "null q, out or seq_off");
  if (Hq % Hkv) return fail(HELM_CPU_E_INVALID, "Hq must be a multiple of Hkv");
  if (D > kMaxD) return fail(HELM_CPU_E_UNSUPPORTED, "head_dim above 512");
  if (kv_dtype < 0 || kv_dtype > 2 || q_dtype < 0 || q_dtype > 2)
    return fail(HELM_CPU_E_INVALID, "dtype must be HELM_CPU_F16, _BF16 or _F32");
  if (causal < 0) return fail(HELM_CPU_E_INVALID, "causal must be >= 0");
  if (seq_off[0] != 0) return fail(HELM_CPU_E_INVALID, "seq_off[0] must be 0");
  int max_pages = 0;
  for (int b = 0; b < B; ++b) {
    const int np = seq_off[b + 1] - seq_off[b];
    if (np < 0) return fail(HELM_CPU_E_INVALID, "seq_off must be non-decreasing");
    max_pages = np > max_pages ? np : max_pages;
  }
  const int n_pages = seq_off[B];
  if (n_pages > 0 && !pages) return fail(HELM_CPU_E_INVALID, "null pages");
  for (int i = 0; i < n_pages; ++i) {
    const helm_cpu_page& p = pages[i];
    if (p.used > 0 && (!p.k || !p.v || p.tok_off < 0 || p.head_stride < 0 ||
                       (Hkv > 1 && p.head_stride < (int64_t)p.used * D)))
      return fail(HELM_CPU_E_INVALID, "page " + std::to_string(i) +
                                          ": null K/V, negative token offset or head stride "
                                          "shorter than its tokens");
  }
  const int isa = helm_cpu_internal::detect_isa();
  if (isa == HELM_CPU_ISA_NONE)
    return fail(HELM_CPU_E_UNSUPPORTED, "this CPU lacks AVX2 + F16C + FMA");

  Job J{};
  J.q = q;
  J.out = out;
  J.B = B;
  J.Hq = Hq;
  J.Hkv = Hkv;
  J.S = q_len;
  J.D = D;
  J.Dp = (D + 15) / 16 * 16;
  J.G = Hq / Hkv;
  J.R = J.G * q_len;
  J.RT = J.R < kTileRows ? J.R : kTileRows;
  J.ntiles = (J.R + J.RT - 1) / J.RT;
  J.pages = pages;
  J.seq_off = seq_off;
  J.scale = scale;
  J.softcap = softcap;
  J.mask = mask;
  J.mbs = mask_bstride;
  J.mhs = mask_hstride;
  J.mqs = mask_qstride;
  J.causal = causal;
  J.kv_dtype = kv_dtype;
  J.q_dtype = q_dtype;
  const int nt = threads > 0 ? threads : omp_get_max_threads();
  // split each sequence's pages so that there are about two items per
  // thread, keeping at least 4 pages in a split
  const int base = B * Hkv * J.ntiles;
  int nsplit = 1;
  if (base < 2 * nt) {
    nsplit = (2 * nt + base - 1) / base;
    const int cap = max_pages / 4 > 1 ? max_pages / 4 : 1;
    nsplit = nsplit < cap ? nsplit : cap;
  }
  J.nsplit = nsplit;
  if (nsplit > 1) {
    // the splits' partial rows: this calling thread's buffer, kept between
    // calls (every row is written before the merge reads it)
    thread_local std::vector<float> part;
    const size_t need = (size_t)base * nsplit * J.RT * (J.Dp + 2);
    if (part.size() < need) part.resize(need);
    J.part = part.data();
  }
  if (isa == HELM_CPU_ISA_AVX512)
    isa_avx512::run(J, nt);
  else
    isa_avx2::run(J, nt);
  return HELM_CPU_OK;
}
