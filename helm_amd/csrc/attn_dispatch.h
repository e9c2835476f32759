// Kernel instantiation + dispatch for one KV element type.  Each including
// file defines HELM_TKV (the KV element type), HELM_TKV_IS_16BIT and
// HELM_LAUNCH_NAME, so the instantiations compile in parallel per dtype.
#pragma once

#include "attn_kernel.h"
#include "attn_mfma.h"
#include "attn_chunk32.h"

#include <hip/hip_ext.h>

namespace helm {
namespace {

// A launch timed by helm_profile_split_kernels goes through
// hipExtLaunchKernelGGL with the spec's start / stop events, which then carry
// the kernel's own start and end; every other launch is a plain launch.
#define HELM_ATTN_LAUNCH(KERNEL, GRID, BLOCK, ...)                                       \
  do {                                                                                   \
    if (s.ev_start)                                                                      \
      hipExtLaunchKernelGGL(KERNEL, GRID, BLOCK, 0, st, s.ev_start, s.ev_stop, 0,        \
                            __VA_ARGS__);                                                \
    else                                                                                 \
      hipLaunchKernelGGL(KERNEL, GRID, BLOCK, 0, st, __VA_ARGS__);                       \
  } while (0)

template <typename TKV, typename TQ, int EPL, int GM, bool DOT2>
hipError_t launch_one(const LaunchSpec& s, hipStream_t st) {
  if (s.mode == 0) {
    HELM_ATTN_LAUNCH((paged_attn_kernel<TKV, TQ, EPL, GM, DOT2, PoolSrc>), s.grid, dim3(kThreads),
                     s.p, s.pool);
  } else {
    HELM_ATTN_LAUNCH((paged_attn_kernel<TKV, TQ, EPL, GM, DOT2, DescSrc>), s.grid, dim3(kThreads),
                     s.p, s.desc);
  }
  return hipGetLastError();
}

// Generic kernels: any D <= 16*EPL, runtime G tiled by 4 rows.
template <typename TKV, typename TQ>
hipError_t launch_generic(const LaunchSpec& s, hipStream_t st) {
  switch (s.epl) {
    case 1: return launch_one<TKV, TQ, 1, 4, false>(s, st);
    case 2: return launch_one<TKV, TQ, 2, 4, false>(s, st);
    case 4: return launch_one<TKV, TQ, 4, 4, false>(s, st);
    case 8: return launch_one<TKV, TQ, 8, 4, false>(s, st);
    case 16: return launch_one<TKV, TQ, 16, 4, false>(s, st);
    default: return hipErrorInvalidValue;
  }
}

#if HELM_TKV_IS_16BIT
// Matrix-core kernels: D = 128, q and KV of the same 16-bit type.
template <typename T, class Src, int FEAT>
hipError_t launch_mfma_feat(const LaunchSpec& s, const Src& src, hipStream_t st) {
  // the chunk kernels read a mask's element type at run time
  constexpr int CF = FEAT & ~kFeatMask16;
  if (s.p.row_waves == 2) {
    if (s.nw == 8)
      HELM_ATTN_LAUNCH((chunk32_mfma_kernel<T, Src, CF, 8>), s.grid, dim3(512), s.p, src);
    else
      HELM_ATTN_LAUNCH((chunk32_mfma_kernel<T, Src, CF, 4>), s.grid, dim3(256), s.p, src);
  } else if (s.p.row_waves)
    HELM_ATTN_LAUNCH((chunk_mfma_kernel<T, Src, CF>), s.grid, dim3(256), s.p, src);
  else if (s.nw == 8)
    HELM_ATTN_LAUNCH((decode_mfma_kernel<T, Src, FEAT, 8>), s.grid, dim3(512), s.p, src);
  else
    HELM_ATTN_LAUNCH((decode_mfma_kernel<T, Src, FEAT, 4>), s.grid, dim3(256), s.p, src);
  return hipGetLastError();
}

template <typename T, class Src>
hipError_t launch_mfma_src(const LaunchSpec& s, const Src& src, hipStream_t st) {
  switch (s.feat) {
    case 0: return launch_mfma_feat<T, Src, 0>(s, src, st);
    case 1: return launch_mfma_feat<T, Src, 1>(s, src, st);
    case 2: return launch_mfma_feat<T, Src, 2>(s, src, st);
    case 3: return launch_mfma_feat<T, Src, 3>(s, src, st);
    case 4: return launch_mfma_feat<T, Src, 4>(s, src, st);
    case 5: return launch_mfma_feat<T, Src, 5>(s, src, st);
    case 6: return launch_mfma_feat<T, Src, 6>(s, src, st);
    case 7: return launch_mfma_feat<T, Src, 7>(s, src, st);
    case 9: return launch_mfma_feat<T, Src, 9>(s, src, st);
    case 11: return launch_mfma_feat<T, Src, 11>(s, src, st);
    case 13: return launch_mfma_feat<T, Src, 13>(s, src, st);
    case 15: return launch_mfma_feat<T, Src, 15>(s, src, st);
    default: return hipErrorInvalidValue;
  }
}

template <typename T>
hipError_t launch_mfma(const LaunchSpec& s, hipStream_t st) {
  if (s.mode == 0) return launch_mfma_src<T, PoolSrc>(s, s.pool, st);
  return launch_mfma_src<T, DescSrc>(s, s.desc, st);
}

// Fast kernels: D = 128, q and KV of the same 16-bit type, exact G rows.
template <typename T>
hipError_t launch_fast(const LaunchSpec& s, hipStream_t st) {
  switch (s.gm) {
    case 1: return launch_one<T, T, 8, 1, true>(s, st);
    case 2: return launch_one<T, T, 8, 2, true>(s, st);
    case 3: return launch_one<T, T, 8, 3, true>(s, st);
    case 4: return launch_one<T, T, 8, 4, true>(s, st);
    case 5: return launch_one<T, T, 8, 5, true>(s, st);
    case 6: return launch_one<T, T, 8, 6, true>(s, st);
    case 7: return launch_one<T, T, 8, 7, true>(s, st);
    case 8: return launch_one<T, T, 8, 8, true>(s, st);
    default: return hipErrorInvalidValue;
  }
}
#endif

}  // namespace

hipError_t HELM_LAUNCH_NAME(const LaunchSpec& s, hipStream_t st) {
#if HELM_TKV_IS_16BIT
  if (s.mfma) return launch_mfma<HELM_TKV>(s, st);
  if (s.fast) return launch_fast<HELM_TKV>(s, st);
#endif
  if (s.q_dtype == HELM_F32) return launch_generic<HELM_TKV, float>(s, st);
  return launch_generic<HELM_TKV, HELM_TKV>(s, st);
}

}  // namespace helm
