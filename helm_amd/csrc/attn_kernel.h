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
//   At the end the 16 row states are merged (shuffles, then LDS) and each
//   workgroup writes one partial (m, l, o[D]) per row to the workspace;
//   merge_splits_kernel, launched after the split kernels, combines the
//   partials of every (sequence, head, tile) and writes the output.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "helm_amd.h"

namespace helm {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kRowLanes = 16;   // lanes per token row (one DPP row)
constexpr int kBlockTok = 16;   // tokens per wave block (4 rows x 4 j)
constexpr int kMaxPps = 256;    // pages per split held in LDS
constexpr int kMaxSplits = 256; // splits per (sequence, head, tile) merged
constexpr int kMergeBatch = 8;  // split partials a merging thread loads at once
constexpr float kRescaleSlack = 8.f;  // lazy online-softmax rescale threshold

// Query row rr of a KV head's G * S rows is query position rr / G of group
// head rr % G: the G heads that share a KV head and one position sit in
// adjacent rows, so the rows of a tile read one mask row (and have one causal
// limit) per position instead of one per row.  Decode (S = 1) has row = head.
struct RowCoord { int g, s; };
__device__ __forceinline__ RowCoord row_coord(int rr, int G) { return {rr % G, rr / G}; }

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

// ---- buffer loads (SGPR resource + VGPR offset) ----------------------------
// Raw (untyped) buffer resource word 3 for CDNA: 32-bit data format.
constexpr int kBufFlags = 0x00020000;

__device__ __forceinline__ uint64_t uniform64(uint64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// clamp(x, lo, hi) on the scalar ALU.  Written out so the compiler cannot
// fold it into a VALU med3 whose VGPR temporary may alias the destination of
// a load still in flight (which would force a full vmcnt(0) wait).
__device__ __forceinline__ int sclamp(int x, int lo, int hi) {
  int r;
  asm volatile("s_max_i32 %0, %1, %2\n\ts_min_i32 %0, %0, %3"
               : "=&s"(r)
               : "s"(x), "s"(lo), "s"(hi)
               : "scc");
  return r;
}

// Resource over [base, base + bytes); loads past `bytes` return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes,
                                           kBufFlags);
}

template <int NB>
__device__ __forceinline__ Raw<NB> buf_load(__amdgpu_buffer_rsrc_t r, int off) {
  Raw<NB> out;
  if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, 0);
      out.w[4 * i + 0] = v[0]; out.w[4 * i + 1] = v[1];
      out.w[4 * i + 2] = v[2]; out.w[4 * i + 3] = v[3];
    }
  } else if constexpr (NB == 8) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    out.w[0] = v[0]; out.w[1] = v[1];
  } else if constexpr (NB == 4) {
    out.w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  } else {
    static_assert(NB == 2, "unsupported raw width");
    out.w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  }
  return out;
}

// Element-wise buffer loads of the first n_valid elements (any D).
template <typename T, int EPL>
__device__ __forceinline__ Raw<EPL * ElemBytes<T>::v> buf_load_elems(
    __amdgpu_buffer_rsrc_t r, int off, int n_valid) {
  constexpr int EB = ElemBytes<T>::v;
  Raw<EPL * EB> out = zero_raw<EPL * EB>();
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    if (e < n_valid) {
      if constexpr (EB == 4) {
        out.w[e] = __builtin_amdgcn_raw_buffer_load_b32(r, off + 4 * e, 0, 0);
      } else {
        const uint32_t h = __builtin_amdgcn_raw_buffer_load_b16(r, off + 2 * e, 0, 0);
        out.w[e >> 1] |= (e & 1) ? (h << 16) : h;
      }
    }
  }
  return out;
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
// update_dpp with old = 0 and bound_ctrl lets the compiler fold the move
// into the following add (v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float row_sum16(float x) {
  x += dpp_mov<0xB1>(x);
  x += dpp_mov<0x4E>(x);
  x += dpp_mov<0x141>(x);
  x += dpp_mov<0x140>(x);
  return x;
}

// ---- agent-scope (cross-XCD coherent) partial-result accesses -------------
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_ml(float* p, float m, float l) {
  const unsigned long long u = (unsigned long long)__float_as_uint(m) |
                               ((unsigned long long)__float_as_uint(l) << 32);
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), u,
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 ld_agent_ml(const float2* p) {
  const unsigned long long u =
      __hip_atomic_load(reinterpret_cast<const unsigned long long*>(p),
                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((unsigned)u),
                     __uint_as_float((unsigned)(u >> 32)));
}
__device__ __forceinline__ float4 ld_agent4(const float* p) {
  const unsigned long long* q = reinterpret_cast<const unsigned long long*>(p);
  const unsigned long long a =
      __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long b =
      __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float4(__uint_as_float((unsigned)a), __uint_as_float((unsigned)(a >> 32)),
                     __uint_as_float((unsigned)b), __uint_as_float((unsigned)(b >> 32)));
}

// exp(x) for x <= 0 or -inf (returns 0 for -inf).
__device__ __forceinline__ float fexp(float x) { return __expf(x); }

// Load through the constant address space: a wave-uniform address becomes a
// scalar (SMEM) load whose wait never involves the vector loads in flight.
template <typename T>
__device__ __forceinline__ T sload(const T* p) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef const __attribute__((address_space(4))) T ConstT;
  return *(ConstT*)(reinterpret_cast<uintptr_t>(p));
#else
  return *p;  // host pass only parses device code
#endif
}

// ---- page sources -----------------------------------------------------------
struct PageView {
  const char* k;     // head hk, token 0
  const char* v;
  int used;
  int tok_off;
  int head_stride_b;  // unused once the head offset is folded in
};

// vLLM-style pool: slot s at base + s*slot_stride (bytes), int32 page table.
// Sequences a call that numbers its splits compactly carries (PoolSrc,
// DescSrc).
constexpr int kSeqArgs = 16;

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
  // compact numbering (decode kernel, sequence lengths known on the host):
  // blockIdx.x runs over every sequence's splits in turn, sequence b's first
  // at seq_split0[b] (b < n_seq, ascending); no workgroup lacks a split
  int compact, n_seq;
  int seq_split0[kSeqArgs];

  __device__ __forceinline__ int n_pages(int b) const {
    const int T = sload(seq_lens + b);
    return T > 0 ? min((T + page_size - 1) / page_size, max_pages) : 0;
  }
  // Dynamic claiming (decode kernel): a sequence's loop-invariant part, a
  // page's record (its slot) fetched a step ahead, and the page's view
  struct Ctx {
    const int32_t* row;  // the sequence's page-table row
    int T;               // its tokens
  };
  __device__ __forceinline__ Ctx ctx(int b) const {
    return Ctx{table + (int64_t)b * table_stride, sload(seq_lens + b)};
  }
  struct Raw {
    int slot;
  };
  __device__ __forceinline__ Raw raw(const Ctx& c, int p) const { return Raw{sload(c.row + p)}; }
  // the record as loaded, read where it is used: the compiler then does not
  // start computing with it (and wait for its load) where it is fetched
  __device__ __forceinline__ static void pin(Raw& r) {
    r.slot = __builtin_amdgcn_readfirstlane(r.slot);
  }
  __device__ __forceinline__ PageView view(const Ctx& c, const Raw& r, int p, int hk) const {
    PageView pv;
    const int64_t off = (int64_t)r.slot * slot_stride_b + hk * head_stride_b;
    pv.k = k_pool + off;
    pv.v = v_pool + off;
    pv.tok_off = p * page_size;
    pv.used = min(page_size, c.T - pv.tok_off);
    pv.head_stride_b = 0;
    return pv;
  }
  __device__ __forceinline__ PageView page(int b, int p, int hk) const {
    const int slot = sload(table + (int64_t)b * table_stride + p);
    const int T = sload(seq_lens + b);
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

// Explicit page descriptors (device addresses).  Either sequence b owns
// pages[seq_off[b] .. seq_off[b+1]) (both device arrays), or (by_value) the
// launch carries each sequence's own record array, page count and token count
// in its arguments: then a page's used tokens are capped at the tokens the
// sequence holds past the page's offset, so the last page's record may keep
// its full capacity while tokens are appended to it.

struct DescSrc {
  const helm_page* pages;
  const int32_t* seq_off;
  int elem_bytes;
  int by_value;
  const helm_page* seq_pages[kSeqArgs];
  int seq_n[kSeqArgs];
  int seq_tokens[kSeqArgs];
  // decode calls that also write each sequence's new token (by_value only):
  // for b < app_n, head h of sequence b's token (D = 128, 16-bit) is at
  // app_k[b] / app_v[b] + h * app_hs[b] elements and goes to the last used
  // slot of the sequence's last page (decode_mfma_kernel)
  int app_n;
  const char* app_k[kSeqArgs];
  const char* app_v[kSeqArgs];
  int64_t app_hs[kSeqArgs];
  // compact numbering (by_value, decode kernel): blockIdx.x runs over every
  // sequence's splits in turn, sequence b's first at seq_split0[b] (b < n_seq,
  // ascending); no workgroup lacks a split
  int compact, n_seq;
  int seq_split0[kSeqArgs];

  __device__ __forceinline__ const helm_page* base(int b) const {
    return by_value ? seq_pages[b] : pages + sload(seq_off + b);
  }
  __device__ __forceinline__ int n_pages(int b) const {
    return by_value ? seq_n[b] : sload(seq_off + b + 1) - sload(seq_off + b);
  }
  __device__ __forceinline__ int used_of(const helm_page& d, int b) const {
    return by_value ? min(d.used, seq_tokens[b] - d.tok_off) : d.used;
  }
  // Dynamic claiming (decode kernel): as PoolSrc's
  struct Ctx {
    const helm_page* base;  // the sequence's records
    int tokens;             // its tokens (by_value; else no cap)
  };
  __device__ __forceinline__ Ctx ctx(int b) const {
    return Ctx{base(b), by_value ? seq_tokens[b] : 0x7fffffff};
  }
  struct Raw {
    helm_page d;
  };
  __device__ __forceinline__ Raw raw(const Ctx& c, int p) const { return Raw{sload(c.base + p)}; }
  __device__ __forceinline__ static void pin(Raw& r) {
    r.d.k = uniform64(r.d.k);
    r.d.v = uniform64(r.d.v);
    r.d.used = __builtin_amdgcn_readfirstlane(r.d.used);
    r.d.tok_off = __builtin_amdgcn_readfirstlane(r.d.tok_off);
    r.d.head_stride = __builtin_amdgcn_readfirstlane(r.d.head_stride);
  }
  __device__ __forceinline__ PageView view(const Ctx& c, const Raw& r, int, int hk) const {
    PageView pv;
    const int64_t off = (int64_t)hk * r.d.head_stride * elem_bytes;
    pv.k = reinterpret_cast<const char*>(r.d.k) + off;
    pv.v = reinterpret_cast<const char*>(r.d.v) + off;
    pv.used = min(r.d.used, c.tokens - r.d.tok_off);
    pv.tok_off = r.d.tok_off;
    pv.head_stride_b = 0;
    return pv;
  }
  __device__ __forceinline__ PageView page(int b, int p, int hk) const {
    const helm_page d = sload(base(b) + p);
    PageView pv;
    const int64_t off = (int64_t)hk * d.head_stride * elem_bytes;
    pv.k = reinterpret_cast<const char*>(d.k) + off;
    pv.v = reinterpret_cast<const char*>(d.v) + off;
    pv.used = used_of(d, b);
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
  const void* mask;   // may be null; additive, in the element type mask_dt
  int64_t mask_bstride, mask_hstride, mask_qstride;
  int mask_dt;        // HELM_F32, HELM_BF16 or HELM_F16
  int causal;         // 0: off; c > 0: position s sees tokens 0 .. s + c - 1
                      // (1: top-left causal)
  int pps;            // pages per split
  int bpp;            // 16-token blocks per page
  int lo, hi;         // page range of this launch within every sequence
  int split_base;     // global index of this launch's first split
  int total_splits;   // > 0: splits of the whole call (chained launches)
  int max_splits;     // stride of the partial buffers
  int full_d;         // D == 16*EPL and 16-byte friendly addresses
  float* ws_o;        // [tiles][max_splits][rows_per_tile][D]
  float* ws_ml;       // [tiles][max_splits][rows_per_tile][2]
  int* counts;        // [tiles] splits of each tile (merge-kernel mode)
  uint32_t* tickets;  // [tiles] arrivals (fused mode; zero between calls)
  int fused;          // 1: the last split of a tile merges in-kernel
  int row_waves;      // query chunks: 16-row tiles per wave (1 or 2; 0: decode kernel)
  int direct_out;     // 1: the call has one split; the chunk kernel writes the output
  int bpp_log2;       // log2 of bpp when bpp is a power of two, else -1
  // profiling (helm_profile_workgroup_stamps): per workgroup of the decode
  // kernel {start, page loop end, end, XCD << 32 | HW_ID}; null: off
  uint64_t* stamps;
  // dynamic block claiming (decode kernel): one counter per tile at
  // claims[tile * kClaimStride], zero before the call, zeroed again by the
  // tile's merge (merge kernel, or the last split in fused mode)
  int dyn;
  uint32_t* claims;
};

// Counter spacing of the dynamic block claims (128 bytes: one tile's
// counter per line).
constexpr int kClaimStride = 32;

// Zeroes tile's claim counter once its merge runs (every claim is done).
__device__ __forceinline__ void reset_claims(const AttnParams& p, int tile) {
  if (p.claims) p.claims[(int64_t)tile * kClaimStride] = 0u;
}

// The s_memrealtime counter (100 MHz) and the workgroup's XCD and HW_ID
// (CU, SIMD, shader engine) for the profiling stamps.
__device__ __forceinline__ uint64_t stamp_now() { return __builtin_amdgcn_s_memrealtime(); }
__device__ __forceinline__ uint64_t stamp_place() {
  uint32_t xcc, hw;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
  return ((uint64_t)xcc << 32) | hw;
}

// One row of the additive mask, in the element type the caller built it in
// (HELM's pipeline builds its masks in the model's dtype and adds them to the
// fp32 scores after .to(float32), kv_cache.py:519, :535): a 16-bit element
// widens to fp32 exactly, so reading it here equals converting the mask
// first.  The element type is uniform, so the branch is a scalar one.
struct MaskRow {
  const char* base;  // element 0 of the row
  int dt;            // HELM_F32, HELM_BF16 or HELM_F16

  __device__ __forceinline__ float operator[](int64_t i) const {
    if (dt == HELM_F32) return reinterpret_cast<const float*>(base)[i];
    const uint32_t h = reinterpret_cast<const uint16_t*>(base)[i];
    if (dt == HELM_BF16) return __uint_as_float(h << 16);
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
  }
  __device__ __forceinline__ MaskRow operator+(int64_t i) const {
    return MaskRow{base + i * (dt == HELM_F32 ? 4 : 2), dt};
  }
  // element i's bits, for an element type known at compile time (K16: a
  // 16-bit mask); widened where the value is used
  template <bool K16>
  __device__ __forceinline__ typename std::conditional<K16, uint16_t, uint32_t>::type bits(
      int64_t i) const {
    if constexpr (K16) return reinterpret_cast<const uint16_t*>(base)[i];
    else return reinterpret_cast<const uint32_t*>(base)[i];
  }
  template <bool K16>
  __device__ __forceinline__ float widen(uint32_t x) const {
    if constexpr (!K16) return __uint_as_float(x);
    return dt == HELM_BF16 ? __uint_as_float(x << 16)
                           : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x)));
  }
};

// Row (b, h, s) of the call's mask.
__device__ __forceinline__ MaskRow mask_row(const AttnParams& p, int b, int h, int s) {
  return MaskRow{reinterpret_cast<const char*>(p.mask), p.mask_dt} +
         ((int64_t)b * p.mask_bstride + (int64_t)h * p.mask_hstride +
          (int64_t)s * p.mask_qstride);
}

// Per-workgroup LDS: per-wave online-softmax states of the tile's rows, and
// the cross-thread reduction of the in-kernel split merge.
template <int NW, int GM, int DMAX>
struct Smem {
  float o[NW][GM][DMAX];
  float m[NW][GM];
  float l[NW][GM];
  float4 red[64 * NW];
  float2 redml[64 * NW];
  int last;
};

// Agent-coherent 16-byte accesses (sc1: coherent across XCDs) to the split
// partials of the in-kernel merge, through one resource over the partial
// buffer (uniform base, per-lane byte offsets).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t partials_rsrc(const AttnParams& p) {
  return make_rsrc(p.ws_o, 0x7ffffff0);
}
__device__ __forceinline__ void st_coherent16(__amdgpu_buffer_rsrc_t r, int64_t elem, float4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(
      __builtin_bit_cast(__attribute__((ext_vector_type(4))) uint32_t, v), r,
      static_cast<int>(elem * 4), 0, 16);
}
__device__ __forceinline__ float4 ld_coherent16(__amdgpu_buffer_rsrc_t r, int64_t elem) {
  return __builtin_bit_cast(float4,
                            __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(elem * 4), 0, 16));
}

// Fused mode's end of a split (its partials already written agent-coherently):
// an atomic ticket counts the tile's arrivals and the last split to arrive
// merges all of them and writes the output.  Callers branch to it as the
// unlikely case, so the common (non-fused) end of a split stays a short
// straight run of code: every workgroup executes it once, from a cold
// instruction cache.
template <typename TQ, int NW, int GM, int DMAX>
__device__ __forceinline__ void fused_merge_tail(Smem<NW, GM, DMAX>& sm,
                                                            const AttnParams& p, int tid,
                                                            int tile, int total, int nrows,
                                                            int r0, int b, int hk) {
  constexpr int NT = 64 * NW;
  constexpr int QB = ElemBytes<TQ>::v;
  const int D = p.D;
  const int RS = p.rows_per_tile;
  const int cw = (D % 4 == 0) ? 4 : 1;
  const int ncol_all = nrows * (D / cw);
  const auto pr = partials_rsrc(p);
  // ---- ticket: the last split of the tile merges -----------------------------
  // The barrier waits (vmcnt(0)) for every wave's coherent stores before the
  // agent-scope ticket increment; the merging workgroup reads the partials
  // with coherent loads issued after it has seen the ticket.
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = atomicAdd(&p.tickets[tile], 1u);
    sm.last = (prev == static_cast<uint32_t>(total - 1)) ? 1 : 0;
  }
  __syncthreads();
  if (!sm.last) return;

  // Thread (sub, c) owns column chunk c of the tile's rows and the splits
  // sub, sub + nsub, ...: every load of a batch is in flight at once.
  constexpr int kBatch = 16;
  const int64_t part0 = (int64_t)tile * p.max_splits * RS;
  const int ncol = ncol_all;
  const int nsub = ncol >= NT ? 1 : NT / ncol;
  const int sub = ncol >= NT ? 0 : tid / ncol;
  const int cstep = ncol >= NT ? NT : ncol * nsub;
  const int S = p.S, G = p.G;
  for (int c = (ncol >= NT ? tid : tid % ncol); c < ncol && sub < nsub; c += cstep) {
    const int g = c / (D / cw);
    const int d0 = (c - g * (D / cw)) * cw;
    float M = -INFINITY, L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = sub; s0 < total; s0 += nsub * kBatch) {
      float2 ml[kBatch];
      float4 v[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int sp = s0 + k * nsub;
        if (sp < total) {
          const int64_t pi = part0 + (int64_t)sp * RS + g;
          ml[k] = ld_agent_ml(reinterpret_cast<const float2*>(p.ws_ml) + pi);
          v[k] = (cw == 4) ? ld_coherent16(pr, pi * D + d0)
                           : make_float4(ld_agent(p.ws_o + pi * D + d0), 0.f, 0.f, 0.f);
        } else {
          ml[k] = make_float2(-INFINITY, 0.f);
          v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
      float mb = M;
#pragma unroll
      for (int k = 0; k < kBatch; ++k) mb = fmaxf(mb, ml[k].x);
      const float base = (mb == -INFINITY) ? 0.f : mb;
      const float a0 = fexp(M - base);
      L *= a0;
      acc.x *= a0; acc.y *= a0; acc.z *= a0; acc.w *= a0;
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const float wgt = fexp(ml[k].x - base);
        L = fmaf(wgt, ml[k].y, L);
        acc.x = fmaf(wgt, v[k].x, acc.x);
        acc.y = fmaf(wgt, v[k].y, acc.y);
        acc.z = fmaf(wgt, v[k].z, acc.z);
        acc.w = fmaf(wgt, v[k].w, acc.w);
      }
      M = mb;
    }
    if (nsub > 1) {
      sm.red[tid] = acc;
      sm.redml[tid] = make_float2(M, L);
    } else {
      const int rr = r0 + g;
      const RowCoord rc = row_coord(rr, G);
      const int h = hk * G + rc.g, s = rc.s;
      char* orow = reinterpret_cast<char*>(p.out) + ((int64_t)(b * p.Hq + h) * S + s) * D * QB;
      const float inv = 1.f / fmaxf(L, 1e-12f);
      const float a[4] = {acc.x, acc.y, acc.z, acc.w};
      for (int j = 0; j < cw; ++j) store_elem<TQ>(orow + (d0 + j) * QB, a[j] * inv);
    }
  }
  if (nsub > 1) {
    __syncthreads();
    if (tid < ncol) {
      float M = -INFINITY;
      for (int j = 0; j < nsub; ++j) M = fmaxf(M, sm.redml[tid + j * ncol].x);
      const float base = (M == -INFINITY) ? 0.f : M;
      float L = 0.f;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int j = 0; j < nsub; ++j) {
        const float2 ml = sm.redml[tid + j * ncol];
        const float4 t = sm.red[tid + j * ncol];
        const float wgt = fexp(ml.x - base);
        L = fmaf(wgt, ml.y, L);
        acc.x = fmaf(wgt, t.x, acc.x);
        acc.y = fmaf(wgt, t.y, acc.y);
        acc.z = fmaf(wgt, t.z, acc.z);
        acc.w = fmaf(wgt, t.w, acc.w);
      }
      const int g = tid / (D / cw);
      const int d0 = (tid - g * (D / cw)) * cw;
      const int rr = r0 + g;
      const RowCoord rc = row_coord(rr, G);
      const int h = hk * G + rc.g, s = rc.s;
      char* orow = reinterpret_cast<char*>(p.out) + ((int64_t)(b * p.Hq + h) * S + s) * D * QB;
      const float inv = 1.f / fmaxf(L, 1e-12f);
      const float a[4] = {acc.x, acc.y, acc.z, acc.w};
      for (int j = 0; j < cw; ++j) store_elem<TQ>(orow + (d0 + j) * QB, a[j] * inv);
    }
  }
  if (tid == 0) {
    p.tickets[tile] = 0u;
    reset_claims(p, tile);
  }
}

// Shared end of a split for the vector-ALU decode kernels (NW waves per
// workgroup).  On entry sm.o / sm.m / sm.l hold the per-wave online-softmax
// states of the tile's `nrows` rows (a barrier has been passed).  Merges the waves and
// writes the split's partial (m, l, o[D]) per row.  In fused mode the
// partials are written agent-coherently, an atomic ticket counts the tile's
// arrivals and the last split to arrive merges all of them and writes the
// output; otherwise merge_splits_kernel does that after the kernel.
template <typename TQ, int NW, int GM, int DMAX>
__device__ __forceinline__ void split_epilogue(Smem<NW, GM, DMAX>& sm, const AttnParams& p,
                                               int tid, int tile, int split, int total,
                                               int nrows, int r0, int b, int hk) {
  constexpr int NT = 64 * NW;
  const int D = p.D;
  const int RS = p.rows_per_tile;  // workspace rows per (tile, split)
  const int64_t part = ((int64_t)tile * p.max_splits + split) * RS;
  const int cw = (D % 4 == 0) ? 4 : 1;
  const int ncol_all = nrows * (D / cw);
  const auto pr = partials_rsrc(p);
  for (int idx = tid; idx < ncol_all; idx += NT) {
    const int g = idx / (D / cw);
    const int d0 = (idx - g * (D / cw)) * cw;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm.m[w][g]);
    const float base = (M == -INFINITY) ? 0.f : M;
    float L = 0.f;
    float O[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float a = fexp(sm.m[w][g] - base);
      L += a * sm.l[w][g];
      for (int j = 0; j < cw; ++j) O[j] += a * sm.o[w][g][d0 + j];
    }
    float* dst = &p.ws_o[(part + g) * D + d0];
    if (p.fused) {
      if (cw == 4) st_coherent16(pr, (part + g) * D + d0, make_float4(O[0], O[1], O[2], O[3]));
      else st_agent(dst, O[0]);
      if (d0 == 0) st_agent_ml(&p.ws_ml[(part + g) * 2], M, L);
    } else {
      for (int j = 0; j < cw; ++j) dst[j] = O[j];
      if (d0 == 0) *reinterpret_cast<float2*>(&p.ws_ml[(part + g) * 2]) = make_float2(M, L);
    }
  }
  if (__builtin_expect(p.fused, 0))
    fused_merge_tail<TQ, NW, GM, DMAX>(sm, p, tid, tile, total, nrows, r0, b, hk);
}

// The same end of a split for the matrix-core kernel (D = 128, GM rows): the
// waves' row states are merged and each row's partial goes out as 16-byte
// stores, with the column arithmetic fixed at compile time.
template <typename TQ, int NW, int GM>
__device__ __forceinline__ void split_epilogue_d128(Smem<NW, GM, 128>& sm, const AttnParams& p,
                                                    int tid, int tile, int split, int total,
                                                    int nrows, int r0, int b, int hk) {
  constexpr int NT = 64 * NW;
  const int64_t part = ((int64_t)tile * p.max_splits + split) * p.rows_per_tile;
  const auto pr = partials_rsrc(p);
  for (int idx = tid; idx < nrows * 32; idx += NT) {
    const int g = idx >> 5;
    const int d0 = (idx & 31) * 4;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm.m[w][g]);
    const float base = (M == -INFINITY) ? 0.f : M;
    float L = 0.f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float a = fexp(sm.m[w][g] - base);
      L += a * sm.l[w][g];
      const float4 v = *reinterpret_cast<const float4*>(&sm.o[w][g][d0]);
      O.x += a * v.x; O.y += a * v.y; O.z += a * v.z; O.w += a * v.w;
    }
    if (p.fused) {
      st_coherent16(pr, (part + g) * 128 + d0, O);
      if (d0 == 0) st_agent_ml(&p.ws_ml[(part + g) * 2], M, L);
    } else {
      *reinterpret_cast<float4*>(&p.ws_o[(part + g) * 128 + d0]) = O;
      if (d0 == 0) *reinterpret_cast<float2*>(&p.ws_ml[(part + g) * 2]) = make_float2(M, L);
    }
  }
  if (__builtin_expect(p.fused, 0)) {
    // ticket: the last split of the tile to arrive merges (as fused_merge_tail)
    __syncthreads();
    if (tid == 0) {
      const uint32_t prev = atomicAdd(&p.tickets[tile], 1u);
      sm.last = (prev == static_cast<uint32_t>(total - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (!sm.last) return;
    constexpr int QB = ElemBytes<TQ>::v;
    const int items = nrows * 32;               // (row, float4 column chunk)
    const int nsub = items >= NT ? 1 : NT / items;
    const int sub = tid / items;
    const int it = tid - sub * items;
    const int64_t part0 = (int64_t)tile * p.max_splits * p.rows_per_tile;
    for (int i = it; i < items && sub < nsub; i += NT) {
      const int g = i >> 5;
      const int d0 = (i & 31) * 4;
      float M = -INFINITY, L = 0.f;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      constexpr int kB = 16;  // one trip for up to 16 * nsub splits
      for (int s0 = sub; s0 < total; s0 += nsub * kB) {
        float2 ml[kB];
        float4 v[kB];
#pragma unroll
        for (int k = 0; k < kB; ++k) {
          const int sp = s0 + k * nsub;
          if (sp < total) {
            const int64_t pi = part0 + (int64_t)sp * p.rows_per_tile + g;
            ml[k] = ld_agent_ml(reinterpret_cast<const float2*>(p.ws_ml) + pi);
            v[k] = ld_coherent16(pr, pi * 128 + d0);
          } else {
            ml[k] = make_float2(-INFINITY, 0.f);
            v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
        float mb = M;
#pragma unroll
        for (int k = 0; k < kB; ++k) mb = fmaxf(mb, ml[k].x);
        const float base = (mb == -INFINITY) ? 0.f : mb;
        const float a0 = fexp(M - base);
        L *= a0;
        acc.x *= a0; acc.y *= a0; acc.z *= a0; acc.w *= a0;
#pragma unroll
        for (int k = 0; k < kB; ++k) {
          const float wgt = fexp(ml[k].x - base);
          L = fmaf(wgt, ml[k].y, L);
          acc.x = fmaf(wgt, v[k].x, acc.x);
          acc.y = fmaf(wgt, v[k].y, acc.y);
          acc.z = fmaf(wgt, v[k].z, acc.z);
          acc.w = fmaf(wgt, v[k].w, acc.w);
        }
        M = mb;
      }
      if (nsub == 1) {
        // one thread per item: write the output row chunk directly
        const float inv = 1.f / fmaxf(L, 1e-12f);
        const int rr = r0 + g;
        const RowCoord rc = row_coord(rr, p.G);
        const int h = hk * p.G + rc.g, sq = rc.s;
        char* orow =
            reinterpret_cast<char*>(p.out) + ((int64_t)(b * p.Hq + h) * p.S + sq) * 128 * QB;
        store_elem<TQ>(orow + (d0 + 0) * QB, acc.x * inv);
        store_elem<TQ>(orow + (d0 + 1) * QB, acc.y * inv);
        store_elem<TQ>(orow + (d0 + 2) * QB, acc.z * inv);
        store_elem<TQ>(orow + (d0 + 3) * QB, acc.w * inv);
      } else {
        sm.red[tid] = acc;
        sm.redml[tid] = make_float2(M, L);
      }
    }
    __syncthreads();
    for (int i = tid; i < items && nsub > 1; i += NT) {
      float Mx = -INFINITY;
      for (int j = 0; j < nsub; ++j) Mx = fmaxf(Mx, sm.redml[i + j * items].x);
      const float base = (Mx == -INFINITY) ? 0.f : Mx;
      float Lx = 0.f;
      float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int j = 0; j < nsub; ++j) {
        const float2 ml = sm.redml[i + j * items];
        const float4 t = sm.red[i + j * items];
        const float wgt = fexp(ml.x - base);
        Lx = fmaf(wgt, ml.y, Lx);
        o.x = fmaf(wgt, t.x, o.x);
        o.y = fmaf(wgt, t.y, o.y);
        o.z = fmaf(wgt, t.z, o.z);
        o.w = fmaf(wgt, t.w, o.w);
      }
      const float inv = 1.f / fmaxf(Lx, 1e-12f);
      const int g = i >> 5;
      const int d0 = (i & 31) * 4;
      const int rr = r0 + g;
      const RowCoord rc = row_coord(rr, p.G);
      const int h = hk * p.G + rc.g, sq = rc.s;
      char* orow = reinterpret_cast<char*>(p.out) + ((int64_t)(b * p.Hq + h) * p.S + sq) * 128 * QB;
      store_elem<TQ>(orow + (d0 + 0) * QB, o.x * inv);
      store_elem<TQ>(orow + (d0 + 1) * QB, o.y * inv);
      store_elem<TQ>(orow + (d0 + 2) * QB, o.z * inv);
      store_elem<TQ>(orow + (d0 + 3) * QB, o.w * inv);
    }
    if (tid == 0) {
      p.tickets[tile] = 0u;
      reset_claims(p, tile);
    }
  }
}


// Combines the split partials of one (tile, row) and writes the output row:
// out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s, M = max_s m_s — the
// final normalisation of HELM's loop, out / clamp(sum, 1e-12)
// (helm/runtime/kv_cache.py:554-555).  grid = (tiles, rows_per_tile, column
// groups): a workgroup merges one group of the row's column chunks, so the
// partials are read by many CUs at once.  A tile whose sequence has no pages
// (split count 0) gets zeros (kv_cache.py:441-442).  Thread (sub, c) owns
// column chunk c and the splits sub, sub + nsub, ...; all of its loads of a
// batch are in flight at once, and the nsub partial results of a column meet
// in LDS.

template <typename TQ>
__global__ __launch_bounds__(kThreads) void merge_splits_kernel(AttnParams p) {
  constexpr int QB = ElemBytes<TQ>::v;
  __shared__ float4 red[kThreads];
  __shared__ float2 redml[kThreads];
  const int tile = blockIdx.x;
  // every split of the tile has finished claiming blocks
  if (blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0) reset_claims(p, tile);
  const int row = blockIdx.y;
  const int tid = threadIdx.x;
  const int D = p.D, S = p.S, G = p.G;
  const int RS = p.rows_per_tile;
  const int qt = tile % p.n_qtiles;
  const int hk = (tile / p.n_qtiles) % p.Hkv;
  const int b = tile / (p.n_qtiles * p.Hkv);
  const int r0 = qt * RS;
  if (r0 + row >= G * S) return;
  const int rr = r0 + row;
  const RowCoord rc = row_coord(rr, G);
  const int h = hk * G + rc.g, s = rc.s;
  char* out_row = reinterpret_cast<char*>(p.out) + ((int64_t)(b * p.Hq + h) * S + s) * D * QB;
  const int total = p.counts[tile];

  const int cw = (D % 4 == 0) ? 4 : 1;
  const int ncol_all = D / cw;
  const int per_group = (ncol_all + gridDim.z - 1) / gridDim.z;
  const int cbeg = blockIdx.z * per_group;
  const int ncol = min(per_group, ncol_all - cbeg);
  if (ncol <= 0) return;
  const int nsub = ncol >= kThreads ? 1 : kThreads / ncol;
  const int sub = tid / ncol;
  const int c0 = cbeg + tid % ncol;
  const int64_t base_part = (int64_t)tile * p.max_splits * RS + row;
  for (int c = c0; c < cbeg + ncol && sub < nsub; c += kThreads) {
    float M = -INFINITY, L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    // The first batch is loaded before the split count arrives (bounded by
    // the workspace's split capacity) and masked afterwards: one memory trip
    // instead of two.
    const int bound = p.max_splits;
    for (int s0 = sub; s0 < bound; s0 += nsub * kMergeBatch) {
      if (s0 > sub && s0 >= total) break;
      float2 ml[kMergeBatch];
      float4 v[kMergeBatch];
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k) {
        const int sp = s0 + k * nsub;
        if (sp < bound) {
          const int64_t pi = base_part + (int64_t)sp * RS;
          ml[k] = *reinterpret_cast<const float2*>(p.ws_ml + pi * 2);
          const float* src = p.ws_o + pi * D + c * cw;
          v[k] = (cw == 4) ? *reinterpret_cast<const float4*>(src)
                           : make_float4(*src, 0.f, 0.f, 0.f);
        } else {
          ml[k] = make_float2(-INFINITY, 0.f);
          v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k) {
        if (s0 + k * nsub >= total) {
          ml[k] = make_float2(-INFINITY, 0.f);
          v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
      float mb = M;
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k) mb = fmaxf(mb, ml[k].x);
      const float base = (mb == -INFINITY) ? 0.f : mb;
      const float a0 = fexp(M - base);
      L *= a0;
      acc.x *= a0; acc.y *= a0; acc.z *= a0; acc.w *= a0;
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k) {
        const float wgt = fexp(ml[k].x - base);
        L = fmaf(wgt, ml[k].y, L);
        acc.x = fmaf(wgt, v[k].x, acc.x);
        acc.y = fmaf(wgt, v[k].y, acc.y);
        acc.z = fmaf(wgt, v[k].z, acc.z);
        acc.w = fmaf(wgt, v[k].w, acc.w);
      }
      M = mb;
    }
    if (nsub > 1) {
      red[tid] = acc;
      redml[tid] = make_float2(M, L);
    } else {
      const float inv = 1.f / fmaxf(L, 1e-12f);
      const float a[4] = {acc.x, acc.y, acc.z, acc.w};
      for (int j = 0; j < cw; ++j) store_elem<TQ>(out_row + (c * cw + j) * QB, a[j] * inv);
    }
  }
  if (nsub > 1) {
    __syncthreads();
    if (tid < ncol) {
      float M = -INFINITY;
      for (int j = 0; j < nsub; ++j) M = fmaxf(M, redml[tid + j * ncol].x);
      const float base = (M == -INFINITY) ? 0.f : M;
      float L = 0.f;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int j = 0; j < nsub; ++j) {
        const float2 ml = redml[tid + j * ncol];
        const float4 t = red[tid + j * ncol];
        const float wgt = fexp(ml.x - base);
        L = fmaf(wgt, ml.y, L);
        acc.x = fmaf(wgt, t.x, acc.x);
        acc.y = fmaf(wgt, t.y, acc.y);
        acc.z = fmaf(wgt, t.z, acc.z);
        acc.w = fmaf(wgt, t.w, acc.w);
      }
      const float inv = 1.f / fmaxf(L, 1e-12f);
      const float a[4] = {acc.x, acc.y, acc.z, acc.w};
      for (int j = 0; j < cw; ++j)
        store_elem<TQ>(out_row + ((cbeg + tid) * cw + j) * QB, a[j] * inv);
    }
  }
}

// merge_splits_kernel for D = 128 with one column group, the arithmetic fixed
// at compile time: thread (sub, c) = (tid / 32, tid % 32) owns float4 column
// chunk c and splits sub, sub + 8, ...; the 8 subs meet in LDS.  A short,
// division-free kernel: it runs once per call with a cold instruction cache.
template <typename TQ>
__global__ __launch_bounds__(kThreads) void merge_splits_d128_kernel(AttnParams p) {
  constexpr int QB = ElemBytes<TQ>::v;
  constexpr int kSub = kThreads / 32;
  __shared__ float4 red[kThreads];
  __shared__ float2 redml[kThreads];
  const int tile = blockIdx.x;
  // every split of the tile has finished claiming blocks
  if (blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0) reset_claims(p, tile);
  const int row = blockIdx.y;
  const int tid = threadIdx.x;
  const int RS = p.rows_per_tile;
  const int qt = tile % p.n_qtiles;
  const int hk = (tile / p.n_qtiles) % p.Hkv;
  const int b = tile / (p.n_qtiles * p.Hkv);
  const int rr = qt * RS + row;
  if (rr >= p.G * p.S) return;
  const int total = p.counts[tile];
  const int sub = tid >> 5;
  const int c = tid & 31;
  const int64_t base_part = (int64_t)tile * p.max_splits * RS + row;
  float M = -INFINITY, L = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  // the first batch is loaded before the split count arrives (bounded by the
  // workspace's split capacity) and masked afterwards
  const int bound = p.max_splits;
  for (int s0 = sub; s0 < bound; s0 += kSub * kMergeBatch) {
    if (s0 > sub && s0 >= total) break;
    float2 ml[kMergeBatch];
    float4 v[kMergeBatch];
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const int sp = s0 + k * kSub;
      if (sp < bound) {
        const int64_t pi = base_part + (int64_t)sp * RS;
        ml[k] = *reinterpret_cast<const float2*>(p.ws_ml + pi * 2);
        v[k] = *reinterpret_cast<const float4*>(p.ws_o + pi * 128 + c * 4);
      } else {
        ml[k] = make_float2(-INFINITY, 0.f);
        v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    float mb = M;
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      if (s0 + k * kSub >= total) {
        ml[k] = make_float2(-INFINITY, 0.f);
        v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
      mb = fmaxf(mb, ml[k].x);
    }
    const float base = (mb == -INFINITY) ? 0.f : mb;
    const float a0 = fexp(M - base);
    L *= a0;
    acc.x *= a0; acc.y *= a0; acc.z *= a0; acc.w *= a0;
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const float wgt = fexp(ml[k].x - base);
      L = fmaf(wgt, ml[k].y, L);
      acc.x = fmaf(wgt, v[k].x, acc.x);
      acc.y = fmaf(wgt, v[k].y, acc.y);
      acc.z = fmaf(wgt, v[k].z, acc.z);
      acc.w = fmaf(wgt, v[k].w, acc.w);
    }
    M = mb;
  }
  red[tid] = acc;
  redml[tid] = make_float2(M, L);
  __syncthreads();
  if (tid < 32) {
    float Mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kSub; ++j) Mx = fmaxf(Mx, redml[tid + 32 * j].x);
    const float base = (Mx == -INFINITY) ? 0.f : Mx;
    float Lx = 0.f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < kSub; ++j) {
      const float2 ml = redml[tid + 32 * j];
      const float4 t = red[tid + 32 * j];
      const float wgt = fexp(ml.x - base);
      Lx = fmaf(wgt, ml.y, Lx);
      o.x = fmaf(wgt, t.x, o.x);
      o.y = fmaf(wgt, t.y, o.y);
      o.z = fmaf(wgt, t.z, o.z);
      o.w = fmaf(wgt, t.w, o.w);
    }
    const float inv = 1.f / fmaxf(Lx, 1e-12f);
    const RowCoord rc = row_coord(rr, p.G);
    const int h = hk * p.G + rc.g, sq = rc.s;
    char* orow = reinterpret_cast<char*>(p.out) + ((int64_t)(b * p.Hq + h) * p.S + sq) * 128 * QB;
    store_elem<TQ>(orow + (tid * 4 + 0) * QB, o.x * inv);
    store_elem<TQ>(orow + (tid * 4 + 1) * QB, o.y * inv);
    store_elem<TQ>(orow + (tid * 4 + 2) * QB, o.z * inv);
    store_elem<TQ>(orow + (tid * 4 + 3) * QB, o.w * inv);
  }
}

// The merge for calls with many query rows and few splits (query chunks):
// thread (r, c) = (tid / 32, tid % 32) of workgroup (tile, y) owns row
// 8 y + r of the tile and its float4 column chunk c, and walks the splits
// itself (no reduction across threads), eight partials in flight at a time
// (the first eight issued before the split count arrives, bounded by the
// workspace's split capacity).  Same arithmetic as merge_splits_d128_kernel
// per split, in split order.
template <typename TQ>
__global__ __launch_bounds__(kThreads) void merge_rows_d128_kernel(AttnParams p) {
  constexpr int QB = ElemBytes<TQ>::v;
  const int tile = blockIdx.x;
  // every split of the tile has finished claiming blocks
  if (blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0) reset_claims(p, tile);
  const int tid = threadIdx.x;
  const int RS = p.rows_per_tile;
  const int row = blockIdx.y * (kThreads / 32) + (tid >> 5);
  const int c = tid & 31;
  const int qt = tile % p.n_qtiles;
  const int hk = (tile / p.n_qtiles) % p.Hkv;
  const int b = tile / (p.n_qtiles * p.Hkv);
  const int rr = qt * RS + row;
  if (row >= RS || rr >= p.G * p.S) return;
  const int total = p.counts[tile];
  const int64_t base_part = (int64_t)tile * p.max_splits * RS + row;
  float M = -INFINITY, L = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  const int bound = p.max_splits;
  for (int s0 = 0; s0 < bound; s0 += kMergeBatch) {
    if (s0 > 0 && s0 >= total) break;
    float2 ml[kMergeBatch];
    float4 v[kMergeBatch];
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const int sp = s0 + k;
      if (sp < bound) {
        const int64_t pi = base_part + (int64_t)sp * RS;
        ml[k] = *reinterpret_cast<const float2*>(p.ws_ml + pi * 2);
        v[k] = *reinterpret_cast<const float4*>(p.ws_o + pi * 128 + c * 4);
      } else {
        ml[k] = make_float2(-INFINITY, 0.f);
        v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    float mb = M;
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      if (s0 + k >= total) {
        ml[k] = make_float2(-INFINITY, 0.f);
        v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
      mb = fmaxf(mb, ml[k].x);
    }
    const float base = (mb == -INFINITY) ? 0.f : mb;
    const float a0 = fexp(M - base);
    L *= a0;
    acc.x *= a0; acc.y *= a0; acc.z *= a0; acc.w *= a0;
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const float wgt = fexp(ml[k].x - base);
      L = fmaf(wgt, ml[k].y, L);
      acc.x = fmaf(wgt, v[k].x, acc.x);
      acc.y = fmaf(wgt, v[k].y, acc.y);
      acc.z = fmaf(wgt, v[k].z, acc.z);
      acc.w = fmaf(wgt, v[k].w, acc.w);
    }
    M = mb;
  }
  const float inv = 1.f / fmaxf(L, 1e-12f);
  const RowCoord rc = row_coord(rr, p.G);
  const int h = hk * p.G + rc.g;
  char* orow = reinterpret_cast<char*>(p.out) + ((int64_t)(b * p.Hq + h) * p.S + rc.s) * 128 * QB;
  store_elem<TQ>(orow + (4 * c + 0) * QB, acc.x * inv);
  store_elem<TQ>(orow + (4 * c + 1) * QB, acc.y * inv);
  store_elem<TQ>(orow + (4 * c + 2) * QB, acc.z * inv);
  store_elem<TQ>(orow + (4 * c + 3) * QB, acc.w * inv);
}

template <typename TKV, typename TQ, int EPL, int GM, bool DOT2, class Src>
__global__ __launch_bounds__(kThreads) void paged_attn_kernel(AttnParams p,
                                                               Src src) {
  constexpr int EB = ElemBytes<TKV>::v;
  constexpr int QB = ElemBytes<TQ>::v;
  constexpr int NB = EPL * EB;       // bytes per lane per token row
  constexpr int DMAX = kRowLanes * EPL;
  static_assert(!DOT2 || (EB == 2 && QB == 2), "dot2 needs 16-bit q and kv");

  __shared__ Smem<kWaves, GM, DMAX> sm;

  const int tid = threadIdx.x;
  // wave index made scalar so block indices / page bases live in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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

  // split 0 publishes the tile's split count; a tile without pages gets
  // zeros (HELM kv_cache.py:441-442), from split 0 in fused mode and from
  // merge_splits_kernel otherwise
  if (split_local == 0 && tid == 0) p.counts[tile] = total;
  if (total == 0) {
    if (p.fused && split_local == 0) {
      for (int idx = tid; idx < nrows * D; idx += kThreads) {
        const int rr = r0 + idx / D;
        const RowCoord rc = row_coord(rr, G);
        const int h = hk * G + rc.g, s = rc.s;
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
    const RowCoord rc = row_coord(rr, G);
    const int gg = rc.g, s = rc.s;
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

  // A block's registers: 4 token rows of K and V for this lane, and the
  // shared decode-mask value of each of those rows.
  struct Blk {
    Raw<NB> k[4];
    Raw<NB> v[4];
    float mk[4];
    int used;      // tokens in the block's page (0: past the end)
    int tok_base;  // HELM token cursor of the page's first token
    int tok0;      // first token of the block inside its page
  };
  // the mask row is shared by every query row of the tile (decode mask)
  const bool mask_shared = has_mask && p.mask_hstride == 0 && S == 1;
  // fast kernels always have full 128-dim rows in 16-byte-aligned pages
  const bool full = DOT2 || p.full_d;

  // Issues the loads of block bi.  Blocks past the end get a zero-byte
  // resource: the loads return 0 without touching memory, so every
  // iteration issues the same loads and waits stay exact.
  auto load_block = [&](int bi, Blk& B) {
    const bool valid = bi < nblk;
    const int pi = valid ? (p.bpp_log2 >= 0 ? bi >> p.bpp_log2 : bi / p.bpp) : 0;
    const int sub = valid ? bi - pi * p.bpp : 0;
    const PageView pv = src.page(b, pg0 + pi, hk);
    const int used = valid ? pv.used : 0;
    const int tok0 = sub * kBlockTok;
    B.used = used;
    B.tok_base = pv.tok_off;
    B.tok0 = tok0;
    const int ntok = sclamp(used - tok0, 0, kBlockTok);
    const char* kb = pv.k;
    const char* vb = pv.v;
    const int nbytes = ntok * (int)row_bytes;
    const auto rk = make_rsrc(kb + tok0 * row_bytes, nbytes);
    const auto rv = make_rsrc(vb + tok0 * row_bytes, nbytes);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int off = (4 * j + row) * (int)row_bytes + d0 * EB;
      if constexpr (DOT2) {
        B.k[j] = buf_load<NB>(rk, off);
        B.v[j] = buf_load<NB>(rv, off);
      } else {
        if (full) {
          B.k[j] = buf_load<NB>(rk, off);
          B.v[j] = buf_load<NB>(rv, off);
        } else {
          B.k[j] = buf_load_elems<TKV, EPL>(rk, off, dvalid);
          B.v[j] = buf_load_elems<TKV, EPL>(rv, off, dvalid);
        }
      }
    }
    if (mask_shared) {
      const MaskRow mr = MaskRow{reinterpret_cast<const char*>(p.mask), p.mask_dt} +
                         (mrow[0] + pv.tok_off + tok0);
      const char* mb = reinterpret_cast<const char*>(
          uniform64(reinterpret_cast<uint64_t>(mr.base)));
      if (p.mask_dt == HELM_F32) {
        const auto rm = make_rsrc(mb, ntok * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          B.mk[j] = __uint_as_float(
              __builtin_amdgcn_raw_buffer_load_b32(rm, (4 * j + row) * 4, 0, 0));
      } else {
        // 16-bit mask: zero past the block's tokens, as the fp32 loads
        const auto rm = make_rsrc(mb, ntok * 2);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t h = __builtin_amdgcn_raw_buffer_load_b16(rm, (4 * j + row) * 2, 0, 0);
          B.mk[j] = p.mask_dt == HELM_BF16
                        ? __uint_as_float(h << 16)
                        : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
        }
      }
    }
  };

  auto compute_block = [&](const Blk& B) {
    const int used = B.used;
    const int tok_base = B.tok_base;
    // q . k of this lane's 4 token rows, reduced across the 16-lane row
    float sc[GM][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DOT2) {
#pragma unroll
        for (int g = 0; g < GM; ++g) {
          float acc = 0.f;
#pragma unroll
          for (int w = 0; w < NB / 4; ++w)
            acc = dot2<TKV>(B.k[j].w[w], qraw[g].w[w], acc);
          sc[g][j] = acc;
        }
      } else {
        float kf[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) kf[e] = elem_f32<TKV>(B.k[j], e);
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

    // logits: scale, then the optional features, each one uniform branch per
    // block rather than per (row, token)
#pragma unroll
    for (int g = 0; g < GM; ++g)
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[g][j] *= scale;
    if (has_cap) {
#pragma unroll
      for (int g = 0; g < GM; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[g][j] = tanhf(sc[g][j] * inv_cap) * cap;
    }
    if (mask_shared) {
#pragma unroll
      for (int g = 0; g < GM; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[g][j] += B.mk[j];
    } else if (has_mask) {
      // per-row mask rows (prefill chunks, per-head masks); the clamp keeps
      // the read inside the page's tokens
#pragma unroll
      for (int g = 0; g < GM; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          sc[g][j] += MaskRow{reinterpret_cast<const char*>(p.mask), p.mask_dt}
              [mrow[g] + tok_base + min(B.tok0 + 4 * j + row, used - 1)];
    }
    if (p.causal) {
#pragma unroll
      for (int g = 0; g < GM; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (tok_base + B.tok0 + 4 * j + row > srow[g] + p.causal - 1) sc[g][j] = -INFINITY;
    }
    // online-softmax update; sc becomes the probabilities.  The reference
    // max m is refreshed only when a block max exceeds it by more than
    // kRescaleSlack (checked across the wave, so the branch is uniform);
    // otherwise p = exp(s - m) <= e^kRescaleSlack and O, L stay exact
    // relative to the stale m.
    float bm[GM];
    bool need = false;
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      bm[g] = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (B.tok0 + 4 * j + row >= used) sc[g][j] = -INFINITY;
        bm[g] = fmaxf(bm[g], sc[g][j]);
      }
      need = need || (bm[g] > m[g] + kRescaleSlack);
    }
    if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
      for (int g = 0; g < GM; ++g) {
        const float mn = fmaxf(m[g], bm[g]);
        const float base = (mn == -INFINITY) ? 0.f : mn;
        const float a = fexp(m[g] - base);
        l[g] *= a;
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[g][e] *= a;
        m[g] = mn;
      }
    }
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      const float base = (m[g] == -INFINITY) ? 0.f : m[g];
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sc[g][j] = fexp(sc[g][j] - base);
        ps += sc[g][j];
      }
      l[g] += ps;
    }
    // P . V, one token row of V widened at a time
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float vf[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) vf[e] = elem_f32<TKV>(B.v[j], e);
#pragma unroll
      for (int g = 0; g < GM; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[g][e] = fmaf(sc[g][j], vf[e], o[g][e]);
    }
  };

  // ---- main loop: three register buffers, two blocks' loads in flight ------
  {
    constexpr int W = kWaves;
    const int nmine = nblk > wave ? (nblk - wave + W - 1) / W : 0;
    Blk ba, bb, bc;
    load_block(wave, ba);
    load_block(wave + W, bb);
    for (int k = 0; k < nmine; k += 3) {
      load_block(wave + (k + 2) * W, bc);
      compute_block(ba);
      if (k + 1 >= nmine) break;
      load_block(wave + (k + 3) * W, ba);
      compute_block(bb);
      if (k + 2 >= nmine) break;
      load_block(wave + (k + 4) * W, bb);
      compute_block(bc);
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

  split_epilogue<TQ, kWaves, GM, DMAX>(sm, p, tid, tile, split, total, nrows, r0, b, hk);
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
  int mfma;           // matrix-core kernel (attn_mfma.h)
  int feat;           // its feature bits (MfmaFeat)
  int nw;             // its waves per workgroup (4 or 8)
  dim3 grid;
  hipEvent_t ev_start = nullptr;   // events of the launch (helm_profile_split_kernels)
  hipEvent_t ev_stop = nullptr;
};

// Implemented per KV dtype in attn_f16.hip / attn_bf16.hip / attn_f32.hip.
hipError_t launch_attn_f16(const LaunchSpec& s, hipStream_t st);
hipError_t launch_attn_bf16(const LaunchSpec& s, hipStream_t st);
hipError_t launch_attn_f32(const LaunchSpec& s, hipStream_t st);

}  // namespace helm
