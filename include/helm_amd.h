/*
 * helm_amd.h — C-ABI of the MI355X (gfx950) paged-KV decode-attention and
 * cold-page offload library (libhelm_amd.so).
 *
 * Every entry point takes plain pointers, integers and a hipStream_t passed as
 * `void*`.  No torch types cross this boundary.  The caller owns every buffer
 * it passes in; the library never frees caller memory.  The only memory the
 * library owns is held by a `helm_engine` (workspace, staging ring, pinned
 * descriptor-upload buffers, one side stream) and is released by
 * helm_engine_destroy().
 *
 * Status convention: 0 = success; a positive value is the hipError_t that
 * failed; a negative value is an argument/contract error (HELM_E_*).  On any
 * non-zero status helm_last_error_string() returns a thread-local message.
 *
 * Element types: HELM_F16 (IEEE binary16), HELM_BF16, HELM_F32.
 *
 * Layouts (all row-major, innermost dimension last and contiguous):
 *   query / out      [B, Hq, q_len, D]  (dense)
 *   one page's K, V  [Hkv, page_tokens, D] — the [1,Hkv,page,D] tensors that
 *                    HELM's KVPage.k_tensor / v_tensor hold.  head_stride is the
 *                    element distance between consecutive KV heads of a page
 *                    (= page capacity * D for a dense page).
 *   mask             additive, of element type mask_dtype (HELM_F32, HELM_BF16
 *                    or HELM_F16: HELM's pipeline builds its masks in the
 *                    model's dtype and widens them to fp32 before adding,
 *                    helm/runtime/kv_cache.py:519, :535; a 16-bit element
 *                    widens exactly, so it is read as given), element
 *                    (b, h, s, t) at element index
 *                    b*mask_bstride + h*mask_hstride + s*mask_qstride + t
 *                    where t is the position of the key among the sequence's
 *                    active tokens (HELM's token_cursor).
 *
 * GQA: query head h reads KV head h / (Hq / Hkv) (HELM repeat_interleave).
 */
#ifndef HELM_AMD_H
#define HELM_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HELM_AMD_ABI_VERSION 2

enum helm_dtype { HELM_F16 = 0, HELM_BF16 = 1, HELM_F32 = 2 };

enum helm_status {
  HELM_OK = 0,
  HELM_E_INVALID = -1,     /* bad argument (shape, pointer, size)          */
  HELM_E_UNSUPPORTED = -2, /* valid request the library does not implement */
  HELM_E_WORKSPACE = -3,   /* caller workspace smaller than required        */
};

/* One KV page as the streaming entry point sees it.  `k`/`v` point at the
 * page's head-0, token-0 element (device memory, or pinned host memory when
 * HELM_PAGE_HOST is set).  `tok_off` is the position of the page's first token
 * among the sequence's active tokens.  32 bytes. */
typedef struct helm_page {
  uint64_t k;
  uint64_t v;
  int32_t used;        /* tokens in the page (> 0)                          */
  int32_t tok_off;     /* HELM token_cursor of the page's first token       */
  int32_t head_stride; /* elements between KV heads inside the page         */
  int32_t flags;       /* HELM_PAGE_HOST: page lives in pinned host memory  */
} helm_page;

#define HELM_PAGE_HOST 1

/* One run of tokens appended into one page (helm_page_append).  The source
 * holds `n_tok` tokens for every KV head: element (h, s, d) of the source K at
 * src_k + h*src_head_stride + s*src_tok_stride + d; the destination token s
 * lands at page row dst_tok + s. */
typedef struct helm_append_seg {
  uint64_t dst_k;
  uint64_t dst_v;
  uint64_t src_k;
  uint64_t src_v;
  int64_t src_head_stride; /* elements */
  int64_t src_tok_stride;  /* elements */
  int32_t dst_head_stride; /* elements */
  int32_t dst_tok;
  int32_t n_tok;
  int32_t pad;
} helm_append_seg;

typedef struct helm_engine helm_engine;

/* ---- library ------------------------------------------------------------ */

/* Thread-local message for the last non-zero status on this thread. */
const char* helm_last_error_string(void);
int helm_abi_version(void);

/* ---- engine: per-device state (side stream, workspace, staging ring) ----- */

/* Creates the per-device engine.  chunk_bytes / ring_slots size the device
 * staging ring that cold pages are prefetched through (0 = defaults:
 * 64 MiB x 2).  Its side stream replaces the per-device copy stream of
 * helm/runtime/kv_cache.py:383-391 (_get_kv_copy_stream). */
int helm_engine_create(int device, size_t chunk_bytes, int ring_slots,
                       helm_engine** out);
int helm_engine_destroy(helm_engine* eng);
/* The engine's side stream (hipStream_t). */
void* helm_engine_copy_stream(helm_engine* eng);

/* ---- attention ------------------------------------------------------------ */

/* Workspace (bytes) helm_paged_decode_attn needs for this shape: per-tile
 * merge tickets and block-claim counters (a fixed region at its start,
 * 64 KiB, used for nothing else), split counts, and the split partials
 * (m, l, o[D]) of every query row.  It must be zero before its first use;
 * every completed call leaves the ticket region zero again, so one workspace
 * serves calls of any shapes. */
size_t helm_query_workspace_bytes(int B, int Hq, int Hkv, int q_len, int D,
                                  int max_pages, int page_size,
                                  int pages_per_split);

/* Batched paged decode attention over a slot pool with an int32 page table.
 * Replaces perform_streaming_attention (helm/runtime/kv_cache.py:405-662) and
 * the batched all-GPU branch of _decode_batched (helm/runtime/kv_offload.py:
 * 152-174) for the vLLM-style layout: slot s of the K pool starts at
 * k_pool + s*slot_stride elements, the page of sequence b at position p is
 * slot page_table[b*table_stride + p], sequence b holds seq_lens[b] tokens
 * (device array), every page but the last is full (page_size tokens).
 * pages_per_split <= 0 picks the split automatically; total_pages is an
 * optional hint (sum over b of pages, 0 = unknown) for that choice.
 * seq_lens_host (may be NULL) holds the same B lengths as seq_lens in host
 * memory: a batch of 2..16 sequences then gets a split length chosen from
 * every sequence's page count and a grid of exactly its splits (no
 * workgroup of a short sequence without a split).  Lengths that differ from
 * seq_lens give wrong results (never an access outside the buffers).
 * softcap <= 0 disables the tanh soft-cap; mask may be NULL. */
int helm_paged_decode_attn(const void* q, void* out,
                           const void* k_pool, const void* v_pool,
                           int64_t slot_stride, int64_t head_stride,
                           const int32_t* page_table, int table_stride,
                           const int32_t* seq_lens,
                           int B, int Hq, int Hkv, int q_len, int D,
                           int page_size, int max_pages, int total_pages,
                           const int32_t* seq_lens_host, float scale, float softcap,
                           const void* mask, int64_t mask_bstride,
                           int64_t mask_hstride, int64_t mask_qstride, int mask_dtype,
                           int kv_dtype, int q_dtype, int pages_per_split,
                           void* workspace, size_t ws_bytes, void* stream);

/* The call of helm_paged_decode_attn without a workspace argument, for
 * callers that cannot allocate device memory: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  It has no
 * counterpart in the reference.  Its split-merge tickets, split counts and
 * partials live in a fixed array of HELM_STATIC_SCRATCH_BYTES in the
 * library's device memory (one per GPU, held from the library's load to the
 * end of the process); the call allocates nothing, so a shape whose plan
 * needs more scratch is refused with HELM_E_WORKSPACE.  The caller still
 * passes every input and output.  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other host threads)
 * race and must be ordered by the caller.  The first call on a GPU (and the
 * next call after one whose launch failed) first clears the ticket region
 * with a small kernel on `stream`. */
#define HELM_STATIC_SCRATCH_BYTES (16u << 20)
int helm_paged_decode_attn_static(const void* q, void* out,
                                  const void* k_pool, const void* v_pool,
                                  int64_t slot_stride, int64_t head_stride,
                                  const int32_t* page_table, int table_stride,
                                  const int32_t* seq_lens,
                                  int B, int Hq, int Hkv, int q_len, int D,
                                  int page_size, int max_pages, int total_pages,
                                  const int32_t* seq_lens_host, float scale, float softcap,
                                  const void* mask, int64_t mask_bstride,
                                  int64_t mask_hstride, int64_t mask_qstride, int mask_dtype,
                                  int kv_dtype, int q_dtype, int pages_per_split,
                                  void* stream);

/* Streaming attention over explicit page lists with mixed residency — the
 * drop-in for perform_streaming_attention (helm/runtime/kv_cache.py:405-662),
 * all four paths.  `pages` (host array) holds the active pages of every
 * sequence, sequence b owning pages[seq_off[b] .. seq_off[b+1]) (host array of
 * B+1).  A page flagged HELM_PAGE_HOST whose K and V each lie in one pinned
 * host allocation that the device maps at the same address (hipHostMalloc,
 * torch pin_memory) can be read in place by the attention kernel over the
 * host link, like a device page (see helm_host_pages_in_place); it is, unless
 * B == 1 and the call's host pages coalesce into large address runs (mean
 * >= 2 MiB), which copy faster.  Other host pages
 * are copied into the engine's device staging ring with hipMemcpyAsync on
 * `stream` (runs of adjacent host pages become one copy, up to chunk_bytes
 * per chunk), each chunk's attention launch queued right behind its copy,
 * after the launch over the resident pages; the split merge follows, all on
 * `stream`.  causal = c > 0 applies a causal mask with offset c - 1 (key t
 * visible to query position s iff t <= s + c - 1): c = 1 is the top-left
 * causal mask of HELM's is_causal=q_len>1 (Path 1); c = 1 + past is the
 * chunk mask of a prefill chunk after `past` cached tokens
 * (helm/runtime/pipeline_runtime.py:94-113) without reading it; causal < 0
 * is HELM_E_INVALID.  Under causal masking the pages of each sequence are
 * attended in token-offset order whatever their order in `pages`.  A sequence
 * with no pages yields zeros.  Staged host pages require B == 1
 * (HELM_E_UNSUPPORTED otherwise).  Environment HELM_AMD_HOST_READ=copy stages
 * every host page, =direct reads every readable one in place.
 * HELM_AMD_STAGE_STREAM=side issues the staging copies on the engine's side
 * stream instead, each chunk's launch waiting for its copies by event; once
 * the engine has evicted pages (helm_evict_pages) those copies wait only for
 * the last eviction and for the launches that last read their ring slots, so
 * host pages written by any other means must then be complete when the call
 * is made; before the first eviction they wait for all earlier work on
 * `stream`.  A call of that mode with staged pages first waits on the host
 * until the call of that mode HELM_AMD_SIDE_AHEAD (0..4, default 2, 0 = no
 * wait) such calls earlier has completed on its stream. */
int helm_stream_attn(helm_engine* eng, const void* q, void* out,
                     int B, int Hq, int Hkv, int q_len, int D,
                     const helm_page* pages, const int32_t* seq_off,
                     float scale, float softcap,
                     const void* mask, int64_t mask_bstride,
                     int64_t mask_hstride, int64_t mask_qstride, int mask_dtype, int causal,
                     int kv_dtype, int q_dtype, void* stream);

/* Decode / chunk attention over page records that already sit in device
 * memory, one record array per sequence — the batched all-GPU call of
 * _decode_batched (helm/runtime/kv_offload.py:152-174) for caches whose page
 * lists persist between steps.  Sequence b's records are the device array
 * seq_pages[b] (an address, host array of B) of seq_npages[b] records in
 * token order (tok_off ascending, each page but the last holding exactly its
 * `used` tokens); it holds seq_tokens[b] tokens, so the last record may keep
 * the page's capacity in `used` while tokens are appended (a page's tokens
 * are min(used, seq_tokens[b] - tok_off)).  page_tokens bounds `used`.
 * Every page must be readable by the device: device memory, or pinned host
 * memory mapped at the same address (helm_host_pages_in_place); records are
 * not read on the host (the Python runtime's validation mode,
 * HELM_AMD_CHECK_RECORDS=1, checks them and their device copy against the
 * pages before every launch).  aligned16 != 0 promises 16-byte aligned K/V bases and head
 * strides.  B <= 16 (HELM_E_UNSUPPORTED otherwise).  Same semantics as
 * helm_stream_attn otherwise; the engine's workspace serves the split
 * partials, so calls on one engine are ordered on one stream. */
int helm_paged_attn_seqs(helm_engine* eng, const void* q, void* out, int B,
                         int Hq, int Hkv, int q_len, int D,
                         const uint64_t* seq_pages, const int32_t* seq_npages,
                         const int32_t* seq_tokens, int page_tokens,
                         int aligned16, float scale, float softcap,
                         const void* mask, int64_t mask_bstride,
                         int64_t mask_hstride, int64_t mask_qstride, int mask_dtype, int causal,
                         int kv_dtype, int q_dtype, void* stream);

/* One decode step of _decode_batched (helm/runtime/kv_offload.py:145-174):
 * each sequence's new token written into its pages (KVCacheManager.
 * append_decode's copy_, kv_cache.py:164-165) and the attention over every
 * page, in one kernel.  Arguments as helm_paged_attn_seqs with q_len = 1
 * and q in the KV dtype; tokens[b] is sequence b's token:
 * src_k / src_v its head-0 K / V (16-byte aligned), src_head_stride elements
 * between heads, n_tok = 1 — the destination is the last used slot of the
 * sequence's last record (the bookkeeping has counted the token in
 * seq_tokens[b]), so the dst_* fields are not read.  The split that holds the
 * last page writes the token before reading it.  Returns HELM_E_UNSUPPORTED,
 * launching nothing, when the call's shape does not run on the matrix-core
 * decode kernel (16-bit KV, D = 128) or a token source is not 16-byte
 * aligned: write the tokens
 * with helm_page_append and call helm_paged_attn_seqs then. */
int helm_paged_attn_seqs_append(helm_engine* eng, const void* q, void* out, int B,
                                int Hq, int Hkv, int D, const uint64_t* seq_pages,
                                const int32_t* seq_npages, const int32_t* seq_tokens,
                                int page_tokens, int aligned16, float scale, float softcap,
                                const void* mask, int64_t mask_bstride,
                                int64_t mask_hstride, int64_t mask_qstride, int mask_dtype, int kv_dtype,
                                const helm_append_seg* tokens, void* stream);

/* One decode step of one layer for up to HELM_DECODE_MAX_SEQS sequences, its
 * arguments in one struct (a serving loop keeps it and rewrites only what
 * changes: q, out, token counts, mask, token sources), so that a step costs
 * one native call.  Same call as helm_paged_attn_seqs_append (append != 0:
 * sequence b's token at tok_k[b] / tok_v[b], heads tok_head_stride[b]
 * elements apart, written into the last used slot of its last record) or
 * helm_paged_attn_seqs with q_len = 1 (append == 0).  Replaces, with the
 * runtime's slot bookkeeping, the per-layer attention of _decode_batched
 * (helm/runtime/kv_offload.py:145-174) and its append_decode copy
 * (helm/runtime/kv_cache.py:164-165).  Returns HELM_E_UNSUPPORTED, launching
 * nothing, where helm_paged_attn_seqs_append would. */
#define HELM_DECODE_MAX_SEQS 16
typedef struct helm_decode_args {
  uint64_t q;                 /* [B, Hq, 1, D] in the KV dtype                  */
  uint64_t out;               /* [B, Hq, 1, D]                                  */
  uint64_t mask;              /* additive mask of mask_dtype, or 0              */
  uint64_t stream;            /* hipStream_t                                     */
  int64_t mask_bstride, mask_hstride, mask_qstride;
  uint64_t seq_pages[HELM_DECODE_MAX_SEQS];   /* device record arrays            */
  uint64_t tok_k[HELM_DECODE_MAX_SEQS];       /* the step's tokens (append)      */
  uint64_t tok_v[HELM_DECODE_MAX_SEQS];
  int64_t tok_head_stride[HELM_DECODE_MAX_SEQS];
  int32_t seq_npages[HELM_DECODE_MAX_SEQS];
  int32_t seq_tokens[HELM_DECODE_MAX_SEQS];
  int32_t B, Hq, Hkv, D;
  int32_t page_tokens, aligned16, mask_dtype, kv_dtype;
  int32_t append, pad;
  float scale, softcap;
} helm_decode_args;
int helm_decode_step(helm_engine* eng, const helm_decode_args* a);

/* Copies `bytes` from host memory `src` to device memory `dst` in the order
 * of `stream`, through the engine's pinned staging ring (src may be reused
 * as soon as the call returns).  Keeps device-resident page records current
 * (the page-list bookkeeping of helm/runtime/kv_cache.py:77-86). */
int helm_upload(helm_engine* eng, void* dst, const void* src, size_t bytes,
                void* stream);

/* For each of n page records: in_place[i] = 1 when page i is flagged
 * HELM_PAGE_HOST and helm_stream_attn would read it in place (its K and V
 * regions, Hkv heads of head_stride elements, each inside one pinned host
 * allocation mapped at the same address; a B == 1 call may still stage such
 * pages when they form large runs), else 0.  Queries the HIP runtime
 * only; launches nothing.  Reports what perform_streaming_attention's host
 * pages cost (kv_cache.py:584-662): read over the link, or staged. */
int helm_host_pages_in_place(helm_engine* eng, const helm_page* pages, int n,
                             int Hkv, int D, int kv_dtype, uint8_t* in_place);

/* ---- page movement -------------------------------------------------------- */

/* Writes K/V tokens into pages (device memory), one kernel launch for all
 * segments.  Replaces the per-token / per-chunk copy_ of
 * KVCacheManager.append_decode and append_prefill
 * (helm/runtime/kv_cache.py:135-136, :164-165).  Bit-exact copy. */
int helm_page_append(const helm_append_seg* segs, int n_segs, int Hkv, int D,
                     int dtype, void* stream);

/* Decode front end, one launch for B sequences of one token each.  Row b of
 * q_proj / k_proj / v_proj (q_stride / kv_stride elements apart, heads of D
 * contiguous elements) gets, per head: RMSNorm with weights q_norm_w /
 * k_norm_w and epsilon eps (norm_mode 1: per head, D weights, rounded before
 * the weight multiply like Qwen3RMSNorm; 2: over the whole row, Hq*D or
 * Hkv*D weights, rounded after it like Olmo2RMSNorm; 0: none), then the
 * rotary embedding x*cos + rotate_half(x)*sin with cos / sin rows of D
 * elements cs_stride apart (cs_dtype: dtype, every op rounded to dtype as
 * eager torch does, or HELM_F32, computed in fp32 and rounded once).  q goes
 * to q_out [B, Hq, D]; k and v (v unchanged) go to token dst[b].dst_tok of the
 * page at dst[b].dst_k / dst_v (heads dst_head_stride elements apart; the
 * src_* and n_tok fields are unused).  D even, <= 256.  Replaces the q_norm /
 * k_norm / apply_rotary_pos_emb steps and the append_decode copy of the
 * patched attention forwards (helm/runtime/kv_offload.py:365-373,
 * helm/runtime/kv_cache.py:145-171). */
int helm_decode_front(const void* q_proj, const void* k_proj, const void* v_proj,
                      int64_t q_stride, int64_t kv_stride, const void* q_norm_w,
                      const void* k_norm_w, int norm_mode, float eps, const void* cos,
                      const void* sin, int64_t cs_stride, int cs_dtype, void* q_out,
                      const helm_append_seg* dst, int B, int Hq, int Hkv, int D, int dtype,
                      void* stream);

/* Eviction copies: n regions of bytes[i] from device src[i] to pinned host
 * dst[i], issued with hipMemcpyAsync on `stream` after everything already
 * queued there; regions adjacent on both sides are merged into one copy.
 * With sync != 0 the call returns after the copies completed (HELM's
 * synchronous move_page, helm/runtime/kv_allocator.py:104-116); otherwise
 * later work on `stream` is ordered after them, and so are the engine's
 * side-stream staging copies (an event recorded after them; an eviction on
 * another stream than the previous one first waits for it).  Replaces
 * KVAllocator.move_page GPU->CPU. */
int helm_evict_pages(helm_engine* eng, int n, const uint64_t* src_dev,
                     const uint64_t* dst_host, const uint64_t* bytes,
                     int sync, void* stream);

/* Prefetch copies: the host->device mirror of helm_evict_pages (pinned host
 * src -> device dst).  Replaces KVAllocator.move_page CPU->GPU
 * (helm/runtime/kv_allocator.py:95-121). */
int helm_prefetch_pages(helm_engine* eng, int n, const uint64_t* src_host,
                        const uint64_t* dst_dev, const uint64_t* bytes,
                        int sync, void* stream);

/* ---- device profile ------------------------------------------------------- */

/* Bandwidths of one device, as HELM's device profiler measures them for its
 * planner (helm/compiler/optimization/device_profiler.py:188-240: _bench_gpu's
 * stream copy, counted as 2 x bytes per copy; _bench_pcie's pinned H2D / D2H
 * copies), in bytes per second, each the mean of `iters` timed repetitions
 * on a stream of the probe's own, after untimed ones (at least three, and at
 * least 20 ms of them: the host link reads low for the first milliseconds of
 * a process). */
typedef struct helm_bandwidth {
  double device_copy_bytes_per_s; /* HBM: a streaming-copy kernel, read + write */
  double h2d_bytes_per_s;         /* pinned host -> device, hipMemcpyAsync       */
  double d2h_bytes_per_s;         /* device -> pinned host, hipMemcpyAsync       */
  int64_t copy_mismatched_words;  /* the copy checked word by word: 0 expected   */
} helm_bandwidth;

/* Measures `device` (made current for the call, then restored): a device copy
 * of stream_bytes (HELM: 256 MB) and host-link copies of link_bytes (HELM:
 * 64 MB).  Allocates its buffers (device, pinned host) and frees them before
 * returning.  Byte counts >= 4096 and multiples of 16, iters >= 1. */
int helm_measure_bandwidth(int device, uint64_t stream_bytes, uint64_t link_bytes,
                           int iters, helm_bandwidth* out);

/* No counterpart in HELM: the floor a decode call is measured against.  Times
 * `iters` passes on `stream` (after three untimed ones), pass i reading
 * bufs[i % nbufs][0, bytes) once with a kernel that does nothing else
 * (`workgroups` workgroups of 256 threads, each reading its own contiguous
 * run with 16-byte non-temporal loads, eight in flight per thread) and,
 * when tail_bytes > 0, then
 * bufs[(i + 1) % nbufs][0, tail_bytes) with a second such kernel of
 * tail_workgroups workgroups (a split merge's reads after the page walk).
 * Writes the mean microseconds per pass to *us_per_iter.  Allocates (and
 * frees) a small result buffer; byte counts are multiples of 16. */
int helm_profile_read_pass(const void* const* bufs, int nbufs, uint64_t bytes, int workgroups,
                           uint64_t tail_bytes, int tail_workgroups, int iters, void* stream,
                           float* us_per_iter);

/* ---- split-kernel timing ----------------------------------------------------- */

/* No counterpart in HELM: a profiling hook for callers that time the
 * attention kernel itself (the bench's roofline) rather than the whole call.
 * Arms HIP-event timing of the split (attention) kernel launches of the next
 * n calls of helm_paged_decode_attn, helm_paged_decode_attn_static and
 * helm_paged_attn_seqs[_append] in this process: a start and a stop event are
 * attached to that launch (hipExtLaunchKernelGGL), so the interval is the
 * kernel's own and the split merge that follows is outside it.  n = 0 disarms
 * and frees the events.  Process-wide; arm, run and read from one thread. */
int helm_profile_split_kernels(int n);

/* No counterpart in HELM: a profiling hook that shows how the decode
 * kernel's workgroups share a call.  Arms the next matrix-core decode-kernel
 * launch of helm_paged_decode_attn[_static] or helm_paged_attn_seqs[_append]
 * whose grid has at most max_workgroups
 * workgroups to write, for workgroup w (blockIdx.x + gridDim.x * (blockIdx.y
 * + gridDim.y * blockIdx.z)), four uint64 at dev_buf + 32 w: the s_memrealtime
 * counter (100 MHz) at its start, after its page loop (every wave done), at
 * its end, and (XCD id << 32) | HW_ID (its CU, SIMD and shader engine).  The
 * launch disarms it.  dev_buf is device memory the caller owns and reads
 * after the launch completes.  max_workgroups = 0 disarms.  Process-wide. */
int helm_profile_workgroup_stamps(void* dev_buf, int max_workgroups);

/* Waits for the armed calls' events and writes the split-kernel durations of
 * the calls timed so far (microseconds, call order) to us_out[0 .. max_n);
 * returns how many were written (>= 0), or an error (< 0 / HIP code). */
int helm_profile_split_read(float* us_out, int max_n);

#ifdef __cplusplus
}
#endif

#endif /* HELM_AMD_H */
