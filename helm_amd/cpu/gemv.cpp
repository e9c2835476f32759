// fp16 GEMV for HELM's CPU stages, built for the host CPU of an MI355X node.
//
// y = fp16(W x + b): W [N, K] and x [K] in fp16, products and sums in fp32,
// bias added in fp32, one round-to-nearest-even to fp16 at the end — the
// arithmetic of helm_fp16_linear's decode fast path
// (helm/kernels/fp16_gemv.cpp:115-155).  Its design here:
//
// * x is widened to fp32 once per call (K floats, cache resident), so the
//   inner loop converts only W: one fp16 -> fp32 conversion and one FMA per
//   weight element.
// * Several rows per step share each x load (four W streams per thread for
//   one vector), and up to 8 vectors (a batched decode step) share each W
//   load, so W is read once per call whatever the batch.
// * AVX-512F on CPUs that have it (16 lanes: 32 B of W per FMA), else AVX2
//   (8 lanes); the path is chosen at run time from CPUID, since the library is
//   built on one machine and run on another.  Each path is compiled with its
//   own target attribute; nothing else in the library assumes those ISAs.
// * Rows split over OpenMP threads in contiguous blocks (static schedule), so
//   each thread streams one contiguous region of W.
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

// ---- AVX2 + F16C + FMA: 8 lanes --------------------------------------------
__attribute__((target("avx2,f16c,fma"))) inline float hsum8(__m256 v) {
  __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_movehdup_ps(s));
  return _mm_cvtss_f32(s);
}

__attribute__((target("avx2,f16c,fma"))) void widen_avx2(const uint16_t* x, float* xf,
                                                          int64_t K) {
  int64_t j = 0;
  for (; j + 8 <= K; j += 8)
    _mm256_storeu_ps(xf + j, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(x + j))));
  for (; j < K; ++j) xf[j] = _cvtsh_ss(x[j]);
}

// Rows [r0, r1) against M vectors: R rows per step share each x load, the M
// vectors share each W load; R * M accumulator chains.  Each sum runs over j
// in ascending order in vector lanes, then the lanes are added, then the
// scalar tail: the same order for every M, R and thread count.
template <int M, int R>
__attribute__((target("avx2,f16c,fma"))) void rows_avx2(const uint16_t* W, const float* xf,
                                                         float* acc, int64_t N, int64_t r0,
                                                         int64_t r1, int64_t K) {
  const int64_t K8 = K & ~int64_t(7);
  int64_t i = r0;
  for (; i + R <= r1; i += R) {
    __m256 a[R][M];
#pragma GCC unroll 8
    for (int r = 0; r < R; ++r)
#pragma GCC unroll 8
      for (int m = 0; m < M; ++m) a[r][m] = _mm256_setzero_ps();
    for (int64_t j = 0; j < K8; j += 8) {
      __m256 w[R];
#pragma GCC unroll 8
      for (int r = 0; r < R; ++r)
        w[r] = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(W + (i + r) * K + j)));
#pragma GCC unroll 8
      for (int m = 0; m < M; ++m) {
        const __m256 xv = _mm256_loadu_ps(xf + m * K + j);
#pragma GCC unroll 8
        for (int r = 0; r < R; ++r) a[r][m] = _mm256_fmadd_ps(w[r], xv, a[r][m]);
      }
    }
#pragma GCC unroll 8
    for (int r = 0; r < R; ++r) {
      const uint16_t* wr = W + (i + r) * K;
#pragma GCC unroll 8
      for (int m = 0; m < M; ++m) {
        float s = hsum8(a[r][m]);
        for (int64_t j = K8; j < K; ++j) s += _cvtsh_ss(wr[j]) * xf[m * K + j];
        acc[m * N + i + r] = s;
      }
    }
  }
  if (R > 1 && i < r1) rows_avx2<M, 1>(W, xf, acc, N, i, r1, K);
}

template <int M, int R>
__attribute__((target("avx512f,avx2,f16c,fma"))) void rows_avx512(const uint16_t* W,
                                                                   const float* xf, float* acc,
                                                                   int64_t N, int64_t r0,
                                                                   int64_t r1, int64_t K) {
  const int64_t K16 = K & ~int64_t(15);
  int64_t i = r0;
  for (; i + R <= r1; i += R) {
    __m512 a[R][M];
#pragma GCC unroll 8
    for (int r = 0; r < R; ++r)
#pragma GCC unroll 8
      for (int m = 0; m < M; ++m) a[r][m] = _mm512_setzero_ps();
    for (int64_t j = 0; j < K16; j += 16) {
      __m512 w[R];
#pragma GCC unroll 8
      for (int r = 0; r < R; ++r)
        w[r] = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(W + (i + r) * K + j)));
#pragma GCC unroll 8
      for (int m = 0; m < M; ++m) {
        const __m512 xv = _mm512_loadu_ps(xf + m * K + j);
#pragma GCC unroll 8
        for (int r = 0; r < R; ++r) a[r][m] = _mm512_fmadd_ps(w[r], xv, a[r][m]);
      }
    }
#pragma GCC unroll 8
    for (int r = 0; r < R; ++r) {
      const uint16_t* wr = W + (i + r) * K;
#pragma GCC unroll 8
      for (int m = 0; m < M; ++m) {
        float s = _mm512_reduce_add_ps(a[r][m]);
        for (int64_t j = K16; j < K; ++j) s += _cvtsh_ss(wr[j]) * xf[m * K + j];
        acc[m * N + i + r] = s;
      }
    }
  }
  if (R > 1 && i < r1) rows_avx512<M, 1>(W, xf, acc, N, i, r1, K);
}

// rows per step for M vectors: at most 16 accumulators (AVX-512 has 32
// vector registers) or 8 (AVX2 has 16)
template <int M>
void rows_m(int isa, const uint16_t* W, const float* xf, float* acc, int64_t N, int64_t r0,
            int64_t r1, int64_t K) {
  if (isa == HELM_CPU_ISA_AVX512)
    rows_avx512<M, (M <= 4 ? 4 : 2)>(W, xf, acc, N, r0, r1, K);
  else
    rows_avx2<M, (M <= 2 ? 4 : (M <= 4 ? 2 : 1))>(W, xf, acc, N, r0, r1, K);
}

void rows(int isa, int M, const uint16_t* W, const float* xf, float* acc, int64_t N, int64_t r0,
          int64_t r1, int64_t K) {
  switch (M) {
    case 1: return rows_m<1>(isa, W, xf, acc, N, r0, r1, K);
    case 2: return rows_m<2>(isa, W, xf, acc, N, r0, r1, K);
    case 3: return rows_m<3>(isa, W, xf, acc, N, r0, r1, K);
    case 4: return rows_m<4>(isa, W, xf, acc, N, r0, r1, K);
    case 5: return rows_m<5>(isa, W, xf, acc, N, r0, r1, K);
    case 6: return rows_m<6>(isa, W, xf, acc, N, r0, r1, K);
    case 7: return rows_m<7>(isa, W, xf, acc, N, r0, r1, K);
    default: return rows_m<8>(isa, W, xf, acc, N, r0, r1, K);
  }
}

// fp32 sums + bias (fp32) -> fp16, round to nearest even
__attribute__((target("avx2,f16c,fma"))) void finish(const float* acc, const void* bias,
                                                      int bias_dtype, uint16_t* y, int64_t i0,
                                                      int64_t i1, int64_t N) {
  for (int64_t t = i0; t < i1; ++t) {
    const int64_t i = t % N;
    float v = acc[t];
    if (bias_dtype == 1)
      v += _cvtsh_ss(static_cast<const uint16_t*>(bias)[i]);
    else if (bias_dtype == 2)
      v += static_cast<const float*>(bias)[i];
    y[t] = _cvtss_sh(v, _MM_FROUND_TO_NEAREST_INT);
  }
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
  std::vector<float> xf((size_t)M * K), acc((size_t)M * N);
  widen_avx2(x, xf.data(), (int64_t)M * K);
  const int nt = threads > 0 ? threads : omp_get_max_threads();
  // contiguous blocks of 4-row groups per thread
  const int64_t groups = (N + kRows - 1) / kRows;
#pragma omp parallel num_threads(nt)
  {
    const int t = omp_get_thread_num(), n = omp_get_num_threads();
    const int64_t g0 = groups * t / n, g1 = groups * (t + 1) / n;
    const int64_t r0 = g0 * kRows, r1 = g1 * kRows < N ? g1 * kRows : N;
    if (r0 < r1) {
      rows(isa, M, W, xf.data(), acc.data(), N, r0, r1, K);
      for (int m = 0; m < M; ++m)
        finish(acc.data(), bias, bias_dtype, y, m * N + r0, m * N + r1, N);
    }
  }
  return HELM_CPU_OK;
}

}  // extern "C"
