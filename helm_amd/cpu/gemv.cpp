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
// * Four rows per step share each x load: four independent W streams per
//   thread, four accumulator chains (W is read once, sequentially per row).
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

#include <immintrin.h>
#include <omp.h>

#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

constexpr int kRows = 4;   // rows per step sharing one x load

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

__attribute__((target("avx2,f16c,fma"))) void rows_avx2(const uint16_t* W, const float* xf,
                                                         float* acc, int64_t r0, int64_t r1,
                                                         int64_t K) {
  const int64_t K8 = K & ~int64_t(7);
  int64_t i = r0;
  for (; i + kRows <= r1; i += kRows) {
    const uint16_t* w0 = W + i * K;
    const uint16_t* w1 = w0 + K;
    const uint16_t* w2 = w1 + K;
    const uint16_t* w3 = w2 + K;
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (int64_t j = 0; j < K8; j += 8) {
      const __m256 xv = _mm256_loadu_ps(xf + j);
      a0 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(w0 + j))), xv, a0);
      a1 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(w1 + j))), xv, a1);
      a2 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(w2 + j))), xv, a2);
      a3 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(w3 + j))), xv, a3);
    }
    float s0 = hsum8(a0), s1 = hsum8(a1), s2 = hsum8(a2), s3 = hsum8(a3);
    for (int64_t j = K8; j < K; ++j) {
      s0 += _cvtsh_ss(w0[j]) * xf[j];
      s1 += _cvtsh_ss(w1[j]) * xf[j];
      s2 += _cvtsh_ss(w2[j]) * xf[j];
      s3 += _cvtsh_ss(w3[j]) * xf[j];
    }
    acc[i] = s0;
    acc[i + 1] = s1;
    acc[i + 2] = s2;
    acc[i + 3] = s3;
  }
  for (; i < r1; ++i) {
    const uint16_t* w0 = W + i * K;
    __m256 a0 = _mm256_setzero_ps();
    for (int64_t j = 0; j < K8; j += 8)
      a0 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(w0 + j))),
                           _mm256_loadu_ps(xf + j), a0);
    float s0 = hsum8(a0);
    for (int64_t j = K8; j < K; ++j) s0 += _cvtsh_ss(w0[j]) * xf[j];
    acc[i] = s0;
  }
}

// ---- AVX-512F: 16 lanes -----------------------------------------------------
__attribute__((target("avx512f,avx2,f16c,fma"))) void rows_avx512(const uint16_t* W,
                                                                   const float* xf, float* acc,
                                                                   int64_t r0, int64_t r1,
                                                                   int64_t K) {
  const int64_t K16 = K & ~int64_t(15);
  int64_t i = r0;
  for (; i + kRows <= r1; i += kRows) {
    const uint16_t* w0 = W + i * K;
    const uint16_t* w1 = w0 + K;
    const uint16_t* w2 = w1 + K;
    const uint16_t* w3 = w2 + K;
    __m512 a0 = _mm512_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (int64_t j = 0; j < K16; j += 16) {
      const __m512 xv = _mm512_loadu_ps(xf + j);
      a0 = _mm512_fmadd_ps(_mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(w0 + j))), xv, a0);
      a1 = _mm512_fmadd_ps(_mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(w1 + j))), xv, a1);
      a2 = _mm512_fmadd_ps(_mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(w2 + j))), xv, a2);
      a3 = _mm512_fmadd_ps(_mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(w3 + j))), xv, a3);
    }
    float s0 = _mm512_reduce_add_ps(a0), s1 = _mm512_reduce_add_ps(a1);
    float s2 = _mm512_reduce_add_ps(a2), s3 = _mm512_reduce_add_ps(a3);
    for (int64_t j = K16; j < K; ++j) {
      s0 += _cvtsh_ss(w0[j]) * xf[j];
      s1 += _cvtsh_ss(w1[j]) * xf[j];
      s2 += _cvtsh_ss(w2[j]) * xf[j];
      s3 += _cvtsh_ss(w3[j]) * xf[j];
    }
    acc[i] = s0;
    acc[i + 1] = s1;
    acc[i + 2] = s2;
    acc[i + 3] = s3;
  }
  for (; i < r1; ++i) {
    const uint16_t* w0 = W + i * K;
    __m512 a0 = _mm512_setzero_ps();
    for (int64_t j = 0; j < K16; j += 16)
      a0 = _mm512_fmadd_ps(_mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(w0 + j))),
                           _mm512_loadu_ps(xf + j), a0);
    float s0 = _mm512_reduce_add_ps(a0);
    for (int64_t j = K16; j < K; ++j) s0 += _cvtsh_ss(w0[j]) * xf[j];
    acc[i] = s0;
  }
}

// fp32 sums + bias (fp32) -> fp16, round to nearest even
__attribute__((target("avx2,f16c,fma"))) void finish(const float* acc, const void* bias,
                                                      int bias_dtype, uint16_t* y, int64_t r0,
                                                      int64_t r1) {
  for (int64_t i = r0; i < r1; ++i) {
    float v = acc[i];
    if (bias_dtype == 1)
      v += _cvtsh_ss(static_cast<const uint16_t*>(bias)[i]);
    else if (bias_dtype == 2)
      v += static_cast<const float*>(bias)[i];
    y[i] = _cvtss_sh(v, _MM_FROUND_TO_NEAREST_INT);
  }
}

int detect_isa() {
  __builtin_cpu_init();
  if (!__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("fma") ||
      !__builtin_cpu_supports("f16c"))
    return HELM_CPU_ISA_NONE;
  const char* cap = std::getenv("HELM_CPU_ISA");
  if (cap && !std::strcmp(cap, "avx2")) return HELM_CPU_ISA_AVX2;
  return __builtin_cpu_supports("avx512f") ? HELM_CPU_ISA_AVX512 : HELM_CPU_ISA_AVX2;
}

}  // namespace

extern "C" {

int helm_cpu_isa(void) { return detect_isa(); }

const char* helm_cpu_last_error(void) { return g_err.c_str(); }

int helm_cpu_fp16_gemv(const uint16_t* x, const uint16_t* W, const void* bias, int bias_dtype,
                       uint16_t* y, int64_t N, int64_t K, int threads) {
  if (!x || !W || !y) return fail(HELM_CPU_E_INVALID, "null pointer argument");
  if (N < 1 || K < 1) return fail(HELM_CPU_E_INVALID, "N and K must be positive");
  if (bias_dtype < 0 || bias_dtype > 2 || (bias_dtype != 0 && !bias))
    return fail(HELM_CPU_E_INVALID, "bias_dtype must be 0 (none), 1 (fp16) or 2 (fp32)");
  const int isa = detect_isa();
  if (isa == HELM_CPU_ISA_NONE)
    return fail(HELM_CPU_E_UNSUPPORTED, "this CPU lacks AVX2 + F16C + FMA");
  std::vector<float> xf(K), acc(N);
  widen_avx2(x, xf.data(), K);
  const int nt = threads > 0 ? threads : omp_get_max_threads();
  // contiguous blocks of 4-row groups per thread
  const int64_t groups = (N + kRows - 1) / kRows;
#pragma omp parallel num_threads(nt)
  {
    const int t = omp_get_thread_num(), n = omp_get_num_threads();
    const int64_t g0 = groups * t / n, g1 = groups * (t + 1) / n;
    const int64_t r0 = g0 * kRows, r1 = g1 * kRows < N ? g1 * kRows : N;
    if (r0 < r1) {
      if (isa == HELM_CPU_ISA_AVX512)
        rows_avx512(W, xf.data(), acc.data(), r0, r1, K);
      else
        rows_avx2(W, xf.data(), acc.data(), r0, r1, K);
      finish(acc.data(), bias, bias_dtype, y, r0, r1);
    }
  }
  return HELM_CPU_OK;
}

}  // extern "C"
