/* helm_cpu.h — C-ABI of libhelm_cpu.so: the host-CPU compute of HELM's CPU
 * stages.
 *
 * Host-CPU code (no GPU), plain pointers and sizes, no torch types:
 *  - the decode-step linear y = W x + b with fp16 W and x, fp32
 *    accumulation, bias added in fp32, result rounded to fp16 (round to
 *    nearest even).  Replaces helm_fp16_linear's GEMV fast path
 *    (helm/kernels/fp16_gemv.cpp:115-155) and its row dot product
 *    (:45-96, :101-108);
 *  - streaming attention of a query on the CPU over KV pages in host memory,
 *    the attention of HELM's CPU-stage layers (perform_streaming_attention's
 *    CPU branches, helm/runtime/kv_cache.py:531-555 and :573-577). */
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

/* Element types of helm_cpu_stream_attn (the codes of helm_amd.h). */
#define HELM_CPU_F16 0
#define HELM_CPU_BF16 1
#define HELM_CPU_F32 2

/* One KV page in host memory, laid out as helm_amd.h's helm_page (32 bytes):
 * `k` / `v` address the page's head-0, token-0 element; KV head h starts
 * h * head_stride elements further on and token j of a head j * D elements
 * after its start; `tok_off` is the position of the page's first token among
 * the sequence's active tokens (HELM's token_cursor); `flags` is ignored. */
typedef struct helm_cpu_page {
  uint64_t k;
  uint64_t v;
  int32_t used;
  int32_t tok_off;
  int32_t head_stride;
  int32_t flags;
} helm_cpu_page;

/* Streaming attention on the host CPU, for a query on the CPU:
 *   out[b, h, s] = sum_t softmax_t(l_t) v_t,
 *   l_t = cap(q[b, h, s] . k_t * scale) + mask[b, h, s, t]
 * over the tokens t of sequence b's pages pages[seq_off[b] .. seq_off[b+1])
 * (in order, t counted from 0 across them), with KV head h / (Hq / Hkv) for
 * query head h (HELM's repeat_interleave).  cap(x) = tanh(x / softcap) *
 * softcap when softcap > 0, else x.  mask (additive fp32, may be NULL) holds
 * element (b, h, s, t) at mask + b*mask_bstride + h*mask_hstride +
 * s*mask_qstride + t.  causal = c > 0 excludes key t from position s unless
 * t <= s + c - 1 (c = 1: top-left causal; c = 1 + past: a prompt chunk after
 * `past` cached tokens).  fp32 arithmetic throughout; the online-softmax
 * recurrence of HELM's loop (running max, rescale by exp(old - new) with a
 * -inf max giving 0, running sum) and its final out / max(sum, 1e-12).  Keys
 * whose logit is -inf contribute nothing; a row that sees no key, or a
 * sequence with no pages, gives zeros (HELM's zeros_like for no pages,
 * kv_cache.py:441-442).
 *   query / out: [B, Hq, q_len, D] dense, dtype q_dtype; pages: kv_dtype.
 * Replaces, for a CPU query over host pages, HELM's masked / soft-capped loop
 * (helm/runtime/kv_cache.py:468-555), Path 2 (:573-577, the same formula
 * unmasked) and the first prompt chunk's SDPA over its own K/V
 * (helm/runtime/kv_offload.py:330-338).  Work is spread over `threads`
 * OpenMP threads (<= 0: the OpenMP default).  D <= 512.  Returns
 * HELM_CPU_E_INVALID for bad shapes, dtypes, null pointers or a page with a
 * null K/V, HELM_CPU_E_UNSUPPORTED for D > 512 or a CPU without AVX2. */
int helm_cpu_stream_attn(const void* q, void* out, int B, int Hq, int Hkv, int q_len, int D,
                         const helm_cpu_page* pages, const int32_t* seq_off, float scale,
                         float softcap, const float* mask, int64_t mask_bstride,
                         int64_t mask_hstride, int64_t mask_qstride, int causal,
                         int kv_dtype, int q_dtype, int threads);

/* Message of the last failed call on this thread. */
const char* helm_cpu_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* HELM_CPU_H */
