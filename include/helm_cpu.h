/* helm_cpu.h — C-ABI of libhelm_cpu.so: the fp16 GEMV of HELM's CPU stages.
 *
 * Host-CPU code (no GPU): the decode-step linear y = W x + b with fp16 W and x,
 * fp32 accumulation, bias added in fp32, result rounded to fp16 (round to
 * nearest even).  Replaces helm_fp16_linear's GEMV fast path
 * (helm/kernels/fp16_gemv.cpp:115-155) and its row dot product
 * (:45-96, :101-108).  Plain pointers and sizes; no torch types. */
#ifndef HELM_CPU_H
#define HELM_CPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (0 = ok). */
#define HELM_CPU_OK 0
#define HELM_CPU_E_INVALID 1
#define HELM_CPU_E_UNSUPPORTED 2

/* Instruction-set paths, as returned by helm_cpu_isa(). */
#define HELM_CPU_ISA_NONE 0     /* no F16C + FMA: helm_cpu_fp16_gemv refuses */
#define HELM_CPU_ISA_AVX2 1     /* AVX2 + F16C + FMA, 8 lanes */
#define HELM_CPU_ISA_AVX512 2   /* AVX-512F (+ F16C + FMA), 16 lanes */

/* The path helm_cpu_fp16_gemv takes on this CPU (the best one the CPU
 * supports; environment HELM_CPU_ISA=avx2 caps it at AVX2). */
int helm_cpu_isa(void);

/* y[i] = fp16( sum_j W[i*K + j] * x[j]  +  bias[i] ),  i in [0, N).
 * W: N x K fp16 row-major (IEEE binary16 bits); x: K fp16; bias: N values of
 * bias_dtype (0 = none, 1 = fp16, 2 = fp32), may be null when bias_dtype = 0;
 * y: N fp16.  Products and sums in fp32 (FMA), bias added in fp32, one
 * rounding to fp16 at the end — as helm_fp16_linear (fp16_gemv.cpp:137-151).
 * Rows are split over `threads` OpenMP threads (<= 0: the OpenMP default).
 * Returns HELM_CPU_E_INVALID for null pointers, N or K < 1 or a bad
 * bias_dtype, HELM_CPU_E_UNSUPPORTED when helm_cpu_isa() is NONE. */
int helm_cpu_fp16_gemv(const uint16_t* x, const uint16_t* W, const void* bias,
                       int bias_dtype, uint16_t* y, int64_t N, int64_t K,
                       int threads);

/* Up to HELM_CPU_GEMV_MAX_BATCH vectors per call: y[m*N + i] =
 * fp16( sum_j W[i*K + j] * x[m*K + j]  +  bias[i] ), m in [0, M) — a decode
 * step of M tokens, each vector rounded exactly as helm_cpu_fp16_gemv rounds it
 * (the same summation order: a batch equals M single calls bit for bit),
 * with W read from memory once.  HELM runs more than one token through
 * F.linear in float32 (helm/kernels/__init__.py:78-82): the same arithmetic
 * (float32 sums, one rounding), its weight widened to float32 every call.
 * M outside [1, HELM_CPU_GEMV_MAX_BATCH] is HELM_CPU_E_INVALID. */
#define HELM_CPU_GEMV_MAX_BATCH 8
int helm_cpu_fp16_gemv_batch(const uint16_t* x, const uint16_t* W, const void* bias,
                             int bias_dtype, uint16_t* y, int M, int64_t N, int64_t K,
                             int threads);

/* Message of the last failed call on this thread. */
const char* helm_cpu_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* HELM_CPU_H */
