// fp16 GEMV for HELM's CPU stages, built for the host CPU of an MI355X node.
//
// y = fp16(W x + b): W [N, K] and x [K] in fp16, products and sums in fp32,
// bias added in fp32, one round-to-nearest-even to fp16 at the end — the
// arithmetic of helm_fp16_linear's decode fast path
// (helm/kernels/fp16_gemv.cpp:115-155).  Its design here:
//
// * One vector (the decode step of one sequence): each thread streams its
//   rows of W one at a time with four accumulator chains (one_avx512 below).
// * 2 to 8 vectors (a batched decode step): several rows per step share each
//   x load and the vectors share each W load, so W is read once per call
//   whatever the batch (batch_avx512 below).  The two kernels sum in
//   different orders (four chains, one chain): a batch gives each vector the
//   same bits at every batch size from 2 to 8, a single call its own, both
//   within the float32 bound of the exact result.
// * AVX-512F on CPUs that have it (16 lanes: 32 B of W per FMA), else AVX2
//   (8 lanes); the path is chosen at run time from CPUID, since the library is
//   built on one machine and run on another.  Each path is compiled with its
//   own target attribute; nothing else in the library assumes those ISAs.
// * Rows split over OpenMP threads in contiguous blocks (static schedule), so
//   each thread streams one contiguous region of W; results do not depend on
//   the thread count.  Each thread writes its rows' results (bias added in
//   fp32, rounded) straight to y.
//
// The operation is bound by DRAM bandwidth: N*K*2 bytes of W per call against
// N*K FMAs.
#include "helm_cpu.h"
#include "common.h"

#include <immintrin.h>
#include <omp.h>

#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace helm_cpu_internal {

namespace {
thread_local std::string g_err;
}  // namespace

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

const char* last_error() { return g_err.c_str(); }

int detect_isa() {
  __builtin_cpu_init();
  if (!__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("fma") ||
      !__builtin_cpu_supports("f16c"))
    return HELM_CPU_ISA_NONE;
  const char* cap = std::getenv("HELM_CPU_ISA");
  if (cap && !std::strcmp(cap, "avx2")) return HELM_CPU_ISA_AVX2;
  return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                 __builtin_cpu_supports("avx512vl")
             ? HELM_CPU_ISA_AVX512
             : HELM_CPU_ISA_AVX2;
}

}  // namespace helm_cpu_internal

namespace {

using helm_cpu_internal::detect_isa;
using helm_cpu_internal::fail;

constexpr int kRows = 4;   // rows per thread-block granule

// fp32 sum + bias (fp32) -> fp16, round to nearest even
__attribute__((target("avx2,f16c,fma"))) inline uint16_t finish(float v, const void* bias,
                                                                int bias_dtype, int64_t i) {
  if (bias_dtype == 1)
    v += _cvtsh_ss(static_cast<const uint16_t*>(bias)[i]);
  else if (bias_dtype == 2)
    v += static_cast<const float*>(bias)[i];
  return _cvtss_sh(v, _MM_FROUND_TO_NEAREST_INT);
}

// ---- one vector: one weight row per step ----------------------------------
//
// Each thread streams its rows of W one after another (a single forward
// stream per thread: on the MI355X hosts' EPYC cores this reads DRAM faster
// than several interleaved row streams, which split the hardware
// prefetchers), with four independent accumulators so that the FMA latency
// never limits the stream; x is converted in the loop (it is read from L1).
// A sum's order depends only on K: lanes accumulate the 4L-element chunks
// j = 4L t + L u into accumulator u (L = 16 or 8 lanes), leftover L-element
// chunks go to accumulator 0, then (a0 + a1) + (a2 + a3), then the lanes, then
// the scalar tail.

__attribute__((target("avx2,f16c,fma"))) inline float hsum8(__m256 v) {
  __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_movehdup_ps(s));
  return _mm_cvtss_f32(s);
}

__attribute__((target("avx2,f16c,fma"))) void one_avx2(const uint16_t* W, const uint16_t* x,
                                                        const void* bias, int bias_dtype,
                                                        uint16_t* y, int64_t r0, int64_t r1,
                                                        int64_t K) {
  const int64_t K32 = K & ~int64_t(31), K8 = K & ~int64_t(7);
  for (int64_t i = r0; i < r1; ++i) {
    const uint16_t* wr = W + i * K;
    __m256 a[4];
#pragma GCC unroll 4
    for (int u = 0; u < 4; ++u) a[u] = _mm256_setzero_ps();
    for (int64_t j = 0; j < K32; j += 32) {
#pragma GCC unroll 4
      for (int u = 0; u < 4; ++u)
        a[u] = _mm256_fmadd_ps(
            _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(wr + j + 8 * u))),
            _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(x + j + 8 * u))), a[u]);
    }
    for (int64_t j = K32; j < K8; j += 8)
      a[0] = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(wr + j))),
                             _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(x + j))), a[0]);
    float s = hsum8(_mm256_add_ps(_mm256_add_ps(a[0], a[1]), _mm256_add_ps(a[2], a[3])));
    for (int64_t j = K8; j < K; ++j) s += _cvtsh_ss(wr[j]) * _cvtsh_ss(x[j]);
    y[i] = finish(s, bias, bias_dtype, i);
  }
}

__attribute__((target("avx512f,avx2,f16c,fma"))) void one_avx512(
    const uint16_t* W, const uint16_t* x, const void* bias, int bias_dtype, uint16_t* y,
    int64_t r0, int64_t r1, int64_t K) {
  const int64_t K64 = K & ~int64_t(63), K16 = K & ~int64_t(15);
  for (int64_t i = r0; i < r1; ++i) {
    const uint16_t* wr = W + i * K;
    __m512 a[4];
#pragma GCC unroll 4
    for (int u = 0; u < 4; ++u) a[u] = _mm512_setzero_ps();
    for (int64_t j = 0; j < K64; j += 64) {
#pragma GCC unroll 4
      for (int u = 0; u < 4; ++u)
        a[u] = _mm512_fmadd_ps(
            _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(wr + j + 16 * u))),
            _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(x + j + 16 * u))), a[u]);
    }
    for (int64_t j = K64; j < K16; j += 16)
      a[0] = _mm512_fmadd_ps(_mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(wr + j))),
                             _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(x + j))), a[0]);
    float s = _mm512_reduce_add_ps(_mm512_add_ps(_mm512_add_ps(a[0], a[1]),
                                                 _mm512_add_ps(a[2], a[3])));
    for (int64_t j = K16; j < K; ++j) s += _cvtsh_ss(wr[j]) * _cvtsh_ss(x[j]);
    y[i] = finish(s, bias, bias_dtype, i);
  }
}

// ---- 2 to 8 vectors: several rows per step share each x load --------------
//
// x is widened to fp32 once per call; R rows per step share every x load and
// the G vectors of a group share every W load (R * G accumulators); vectors
// come in groups of at most four, and for more than four a block of rows is
// computed for the first group and then for the second while it is still in
// L2, so W crosses from DRAM once.  Each (row, vector) sum runs over the
// L-element chunks in ascending order in one accumulator, then the lanes,
// then the scalar tail: the same for every batch size from 2 to 8, grouping,
// R and thread count.
constexpr int kBlockRows = 16;   // rows per block when vectors come in two groups

template <int R, int G>
__attribute__((target("avx2,f16c,fma"))) void batch_avx2(const uint16_t* W, const float* xf,
                                                          const void* bias, int bias_dtype,
                                                          uint16_t* y, int64_t N, int64_t r0,
                                                          int64_t r1, int64_t K, int m0) {
  const int64_t K8 = K & ~int64_t(7);
  const float* xg = xf + m0 * K;
  int64_t i = r0;
  for (; i + R <= r1; i += R) {
    __m256 a[R][G];
#pragma GCC unroll 4
    for (int r = 0; r < R; ++r)
#pragma GCC unroll 4
      for (int m = 0; m < G; ++m) a[r][m] = _mm256_setzero_ps();
    for (int64_t j = 0; j < K8; j += 8) {
      __m256 w[R];
#pragma GCC unroll 4
      for (int r = 0; r < R; ++r)
        w[r] = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(W + (i + r) * K + j)));
#pragma GCC unroll 4
      for (int m = 0; m < G; ++m) {
        const __m256 xv = _mm256_loadu_ps(xg + m * K + j);
#pragma GCC unroll 4
        for (int r = 0; r < R; ++r) a[r][m] = _mm256_fmadd_ps(w[r], xv, a[r][m]);
      }
    }
#pragma GCC unroll 4
    for (int r = 0; r < R; ++r) {
      const uint16_t* wr = W + (i + r) * K;
#pragma GCC unroll 4
      for (int m = 0; m < G; ++m) {
        float s = hsum8(a[r][m]);
        for (int64_t j = K8; j < K; ++j) s += _cvtsh_ss(wr[j]) * xg[m * K + j];
        y[(m0 + m) * N + i + r] = finish(s, bias, bias_dtype, i + r);
      }
    }
  }
  if (R > 1 && i < r1) batch_avx2<1, G>(W, xf, bias, bias_dtype, y, N, i, r1, K, m0);
}

template <int R, int G>
__attribute__((target("avx512f,avx2,f16c,fma"))) void batch_avx512(
    const uint16_t* W, const float* xf, const void* bias, int bias_dtype, uint16_t* y,
    int64_t N, int64_t r0, int64_t r1, int64_t K, int m0) {
  const int64_t K16 = K & ~int64_t(15);
  const float* xg = xf + m0 * K;
  int64_t i = r0;
  for (; i + R <= r1; i += R) {
    __m512 a[R][G];
#pragma GCC unroll 4
    for (int r = 0; r < R; ++r)
#pragma GCC unroll 4
      for (int m = 0; m < G; ++m) a[r][m] = _mm512_setzero_ps();
    for (int64_t j = 0; j < K16; j += 16) {
      __m512 w[R];
#pragma GCC unroll 4
      for (int r = 0; r < R; ++r)
        w[r] = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(W + (i + r) * K + j)));
#pragma GCC unroll 4
      for (int m = 0; m < G; ++m) {
        const __m512 xv = _mm512_loadu_ps(xg + m * K + j);
#pragma GCC unroll 4
        for (int r = 0; r < R; ++r) a[r][m] = _mm512_fmadd_ps(w[r], xv, a[r][m]);
      }
    }
#pragma GCC unroll 4
    for (int r = 0; r < R; ++r) {
      const uint16_t* wr = W + (i + r) * K;
#pragma GCC unroll 4
      for (int m = 0; m < G; ++m) {
        float s = _mm512_reduce_add_ps(a[r][m]);
        for (int64_t j = K16; j < K; ++j) s += _cvtsh_ss(wr[j]) * xg[m * K + j];
        y[(m0 + m) * N + i + r] = finish(s, bias, bias_dtype, i + r);
      }
    }
  }
  if (R > 1 && i < r1) batch_avx512<1, G>(W, xf, bias, bias_dtype, y, N, i, r1, K, m0);
}

// one group of G vectors over rows [r0, r1): 4 rows per step with AVX-512
// (32 registers: 16 accumulators), 2 with AVX2 (16 registers: 8)
template <int G>
void batch_g(int isa, const uint16_t* W, const float* xf, const void* bias, int bias_dtype,
             uint16_t* y, int64_t N, int64_t r0, int64_t r1, int64_t K, int m0) {
  if (isa == HELM_CPU_ISA_AVX512)
    batch_avx512<4, G>(W, xf, bias, bias_dtype, y, N, r0, r1, K, m0);
  else
    batch_avx2<2, G>(W, xf, bias, bias_dtype, y, N, r0, r1, K, m0);
}

void batch_group(int isa, int G, const uint16_t* W, const float* xf, const void* bias,
                 int bias_dtype, uint16_t* y, int64_t N, int64_t r0, int64_t r1, int64_t K,
                 int m0) {
  switch (G) {
    case 1: return batch_g<1>(isa, W, xf, bias, bias_dtype, y, N, r0, r1, K, m0);
    case 2: return batch_g<2>(isa, W, xf, bias, bias_dtype, y, N, r0, r1, K, m0);
    case 3: return batch_g<3>(isa, W, xf, bias, bias_dtype, y, N, r0, r1, K, m0);
    default: return batch_g<4>(isa, W, xf, bias, bias_dtype, y, N, r0, r1, K, m0);
  }
}

// x [n] fp16 -> fp32 (exact)
__attribute__((target("avx2,f16c,fma"))) void widen(const uint16_t* x, float* xf, int64_t n) {
  int64_t j = 0;
  for (; j + 8 <= n; j += 8)
    _mm256_storeu_ps(xf + j, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(x + j))));
  for (; j < n; ++j) xf[j] = _cvtsh_ss(x[j]);
}

}  // namespace

extern "C" {

int helm_cpu_isa(void) { return detect_isa(); }

const char* helm_cpu_last_error(void) { return helm_cpu_internal::last_error(); }

int helm_cpu_fp16_gemv(const uint16_t* x, const uint16_t* W, const void* bias, int bias_dtype,
                       uint16_t* y, int64_t N, int64_t K, int threads) {
  return helm_cpu_fp16_gemv_batch(x, W, bias, bias_dtype, y, 1, N, K, threads);
}

int helm_cpu_fp16_gemv_batch(const uint16_t* x, const uint16_t* W, const void* bias,
                             int bias_dtype, uint16_t* y, int M, int64_t N, int64_t K,
                             int threads) {
  if (!x || !W || !y) return fail(HELM_CPU_E_INVALID, "null pointer argument");
  if (N < 1 || K < 1) return fail(HELM_CPU_E_INVALID, "N and K must be positive");
  if (M < 1 || M > HELM_CPU_GEMV_MAX_BATCH)
    return fail(HELM_CPU_E_INVALID, "M must be in [1, 8]");
  if (bias_dtype < 0 || bias_dtype > 2 || (bias_dtype != 0 && !bias))
    return fail(HELM_CPU_E_INVALID, "bias_dtype must be 0 (none), 1 (fp16) or 2 (fp32)");
  const int isa = detect_isa();
  if (isa == HELM_CPU_ISA_NONE)
    return fail(HELM_CPU_E_UNSUPPORTED, "this CPU lacks AVX2 + F16C + FMA");
  const int nt = threads > 0 ? threads : omp_get_max_threads();
  // contiguous blocks of 4-row groups per thread
  const int64_t groups = (N + kRows - 1) / kRows;
  if (M == 1) {
#pragma omp parallel num_threads(nt)
    {
      const int t = omp_get_thread_num(), n = omp_get_num_threads();
      const int64_t g0 = groups * t / n, g1 = groups * (t + 1) / n;
      const int64_t r0 = g0 * kRows, r1 = g1 * kRows < N ? g1 * kRows : N;
      if (r0 < r1) {
        if (isa == HELM_CPU_ISA_AVX512)
          one_avx512(W, x, bias, bias_dtype, y, r0, r1, K);
        else
          one_avx2(W, x, bias, bias_dtype, y, r0, r1, K);
      }
    }
    return HELM_CPU_OK;
  }
  // x widened once per call, in parallel, into the calling thread's buffer
  // (kept between calls: no allocation once it has reached 8 x K)
  static thread_local std::vector<float> xbuf;
  const int64_t nx = (int64_t)M * K;
  if ((int64_t)xbuf.size() < nx) xbuf.resize(nx);
  float* xf = xbuf.data();
#pragma omp parallel num_threads(nt)
  {
    const int t = omp_get_thread_num(), n = omp_get_num_threads();
    widen(x + nx * t / n, xf + nx * t / n, nx * (t + 1) / n - nx * t / n);
#pragma omp barrier
    const int64_t g0 = groups * t / n, g1 = groups * (t + 1) / n;
    const int64_t r0 = g0 * kRows, r1 = g1 * kRows < N ? g1 * kRows : N;
    if (M <= 4) {
      if (r0 < r1) batch_group(isa, M, W, xf, bias, bias_dtype, y, N, r0, r1, K, 0);
    } else {
      for (int64_t b = r0; b < r1; b += kBlockRows) {
        const int64_t e = b + kBlockRows < r1 ? b + kBlockRows : r1;
        batch_group(isa, 4, W, xf, bias, bias_dtype, y, N, b, e, K, 0);
        batch_group(isa, M - 4, W, xf, bias, bias_dtype, y, N, b, e, K, 4);
      }
    }
  }
  return HELM_CPU_OK;
}

}  // extern "C"
