// Decode front end: one token per sequence, from the q / k / v projection
// rows to the attention inputs, in one launch.
//
// For every sequence b and head, the kernel takes the head's slice of the
// projection row, applies (optionally) RMSNorm and then the rotary embedding
// q * cos + rotate_half(q) * sin, and writes q to a [B, Hq, D] buffer and k
// (with v copied alongside) into the token's slot of the sequence's page.
// This is the work of HF's q_norm / k_norm, apply_rotary_pos_emb and HELM's
// append_decode in the patched attention forwards (helm/runtime/
// kv_offload.py:365-373, kv_cache.py:145-171).
//
// Rounding follows the eager torch ops those forwards run, element by element:
//   norm 1 (per head, Qwen3RMSNorm):   y = rnd(x * r), out = rnd(w * y)
//   norm 2 (whole row, Olmo2RMSNorm):  out = rnd(w * (x * r))
//   with r = rsqrt(mean(x^2) + eps) over the head (1) or the row (2), in fp32;
//   rotary with cos / sin of the element type: rnd(rnd(x c) + rnd(rot(x) s)),
//   with fp32 cos / sin (OLMo-2): rnd(x c + rot(x) s) in fp32 (no fma).
// rnd() rounds to the element type (nearest even); it is the identity for
// fp32.  Only the sum of squares is accumulated in an order of its own.
//
// Grid (sequence, Hq + Hkv heads), one wave per head: rows of up to 256
// elements, 64 lanes x up to 4 elements; the rotate_half partner of each
// element comes through LDS.
#pragma once

#include "attn_kernel.h"

namespace helm {

constexpr int kFrontMaxSeqs = 64;   // sequences per launch (kernel arguments)
constexpr int kFrontMaxD = 256;

struct FrontArgs {
  const char* q;
  const char* k;
  const char* v;
  int64_t q_stride;    // elements between sequences' q rows
  int64_t kv_stride;   // elements between sequences' k (and v) rows
  const char* qw;      // RMSNorm weights (norm != 0)
  const char* kw;
  float eps;
  int norm;            // 0 none, 1 per head (D weights), 2 whole row (H * D weights)
  const char* cos;
  const char* sin;
  int64_t cs_stride;   // elements between sequences' cos / sin rows (0: shared)
  char* q_out;         // [B, Hq, D]
  int b0;              // first sequence of this launch
  int Hq, Hkv, D;
  uint64_t dst_k[kFrontMaxSeqs];
  uint64_t dst_v[kFrontMaxSeqs];
  int32_t dst_head_stride[kFrontMaxSeqs];
  int32_t dst_tok[kFrontMaxSeqs];
};

template <typename T> __device__ __forceinline__ float front_ld(const char* p, int64_t i) {
  if constexpr (__is_same(T, float)) {
    return reinterpret_cast<const float*>(p)[i];
  } else if constexpr (__is_same(T, bf16_t)) {
    return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16);
  } else {
    return static_cast<float>(reinterpret_cast<const _Float16*>(p)[i]);
  }
}

// Rounded to T and widened back (nearest even; identity for fp32).
template <typename T> __device__ __forceinline__ float front_rnd(float x) {
  if constexpr (__is_same(T, float)) {
    return x;
  } else if constexpr (__is_same(T, bf16_t)) {
    return static_cast<float>(static_cast<__bf16>(x));
  } else {
    return static_cast<float>(static_cast<_Float16>(x));
  }
}

template <typename T> __device__ __forceinline__ void front_st(char* p, int64_t i, float x) {
  if constexpr (__is_same(T, float)) {
    reinterpret_cast<float*>(p)[i] = x;
  } else if constexpr (__is_same(T, bf16_t)) {
    reinterpret_cast<__bf16*>(p)[i] = static_cast<__bf16>(x);
  } else {
    reinterpret_cast<_Float16*>(p)[i] = static_cast<_Float16>(x);
  }
}

template <typename T, typename TC>
__global__ __launch_bounds__(64) void decode_front_kernel(FrontArgs a) {
  // every product and sum rounds on its own, as torch's separate ops do
#pragma clang fp contract(off)
  __shared__ float row[kFrontMaxD];
  constexpr int EB = ElemBytes<T>::v;
  const int bl = blockIdx.x;                 // sequence within the launch
  const int b = a.b0 + bl;
  const int hh = blockIdx.y;
  const bool is_q = hh < a.Hq;
  const int h = is_q ? hh : hh - a.Hq;
  const int H = is_q ? a.Hq : a.Hkv;
  const int D = a.D;
  const int t = threadIdx.x;
  const char* src = is_q ? a.q : a.k;
  const int64_t base = (int64_t)b * (is_q ? a.q_stride : a.kv_stride);

  // every load of the head is issued up front: the row, cos / sin, weights
  const int64_t cs = (int64_t)b * a.cs_stride;
  const char* w = is_q ? a.qw : a.kw;
  float x[4], c[4], s[4], wt[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = t + 64 * i;
    const bool in = d < D;
    x[i] = in ? front_ld<T>(src, base + (int64_t)h * D + d) : 0.f;
    c[i] = in ? front_ld<TC>(a.cos, cs + d) : 0.f;
    s[i] = in ? front_ld<TC>(a.sin, cs + d) : 0.f;
    wt[i] = in && a.norm ? front_ld<T>(w, (a.norm == 2 ? (int64_t)h * D : 0) + d) : 0.f;
  }
  if (a.norm) {
    float ss = 0.f;
    if (a.norm == 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) ss += x[i] * x[i];
    } else {
      for (int e = t; e < H * D; e += 64) {
        const float y = front_ld<T>(src, base + e);
        ss += y * y;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const int n = a.norm == 1 ? D : H * D;
    // torch's mean multiplies the sum by 1 / n
    const float r = rsqrtf(ss * (1.f / (float)n) + a.eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (a.norm == 1)
        x[i] = front_rnd<T>(wt[i] * front_rnd<T>(x[i] * r));
      else
        x[i] = front_rnd<T>(wt[i] * (x[i] * r));
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = t + 64 * i;
    if (d < D) row[d] = x[i];
  }
  __syncthreads();
  const int half = D / 2;
  char* dk = is_q ? nullptr
                  : reinterpret_cast<char*>(a.dst_k[bl]) +
                        ((int64_t)h * a.dst_head_stride[bl] + (int64_t)a.dst_tok[bl] * D) * EB;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = t + 64 * i;
    if (d >= D) continue;
    const float rot = d < half ? -row[d + half] : row[d - half];
    float out;
    if constexpr (__is_same(TC, float))
      out = front_rnd<T>(x[i] * c[i] + rot * s[i]);
    else
      out = front_rnd<T>(front_rnd<T>(x[i] * c[i]) + front_rnd<T>(rot * s[i]));
    if (is_q)
      front_st<T>(a.q_out, ((int64_t)b * a.Hq + h) * D + d, out);
    else
      front_st<T>(dk, d, out);
  }
  if (!is_q) {
    // v is copied as it is
    char* dv = reinterpret_cast<char*>(a.dst_v[bl]) +
               ((int64_t)h * a.dst_head_stride[bl] + (int64_t)a.dst_tok[bl] * D) * EB;
    const char* vs = a.v + (base + (int64_t)h * D) * EB;
    for (int e = t; e < D * EB / 2; e += 64)
      reinterpret_cast<uint16_t*>(dv)[e] = reinterpret_cast<const uint16_t*>(vs)[e];
  }
}

}  // namespace helm
