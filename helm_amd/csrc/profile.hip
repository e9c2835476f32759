// Device and host-link bandwidth probes: the GPU and PCIe halves of HELM's
// device profiler (helm/compiler/optimization/device_profiler.py:188-240,
// _bench_gpu's stream copy and _bench_pcie's pinned copies), measured with a
// native streaming-copy kernel and hipMemcpyAsync between pinned host memory
// and the device, timed with HIP events on a stream of the probe's own.
#include <hip/hip_runtime.h>

#include <chrono>

#include <string>

#include "helm_amd.h"

namespace helm {
int report_error(int code, const std::string& msg);
}

namespace {

// dst = src in 16-byte elements, grid-stride, non-temporal (each byte is
// read and written once)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ void stream_copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                   size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// a word pattern that names its own index
__global__ void fill_index_kernel(uint32_t* p, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    p[i] = (uint32_t)(i * 2654435761u);
}

__global__ void zero_u64_kernel(unsigned long long* p) { *p = 0ull; }

// count of words where a differs from b
__global__ void count_mismatch_kernel(const uint32_t* a, const uint32_t* b, size_t n,
                                      unsigned long long* bad) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  unsigned long long local = 0;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    local += a[i] != b[i];
  if (local) atomicAdd(bad, local);
}

// Bare read pass: every 16-byte element of src[0, n) read once with the
// non-temporal hint and folded by XOR into one word per workgroup in sink (so
// that no load can be removed).  Workgroup w reads its own contiguous run of
// elements, as a decode workgroup walks its split; each thread keeps eight
// 16-byte loads in flight (a wave reads 1 KiB contiguous per load).
__global__ __launch_bounds__(256) void read_pass_kernel(const u32x4* __restrict__ src, size_t n,
                                                        uint32_t* __restrict__ sink) {
  __shared__ uint32_t red[256];
  constexpr size_t kStep = 256 * 8;
  const size_t per = (n + gridDim.x - 1) / gridDim.x;
  const size_t lo = min(n, (size_t)blockIdx.x * per);
  const size_t hi = min(n, lo + per);
  uint32_t acc = 0;
  for (size_t i = lo + threadIdx.x; i < hi; i += kStep) {
    u32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const size_t e = i + 256 * j;
      v[j] = e < hi ? __builtin_nontemporal_load(src + e) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= v[j][0] ^ v[j][1] ^ v[j][2] ^ v[j][3];
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t x = 0;
    for (int t = 0; t < 256; ++t) x ^= red[t];
    sink[blockIdx.x] = x;
  }
}

struct Probe {
  hipStream_t st = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  void *src = nullptr, *dst = nullptr, *pin = nullptr;
  unsigned long long* bad = nullptr;
  ~Probe() {   // teardown: statuses are not reported from here
    if (st) (void)hipStreamSynchronize(st);
    if (src) (void)hipFree(src);
    if (dst) (void)hipFree(dst);
    if (bad) (void)hipFree(bad);
    if (pin) (void)hipHostFree(pin);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
  }
};

#define PROBE_HIP(call)                                                            \
  do {                                                                             \
    hipError_t e_ = (call);                                                        \
    if (e_ != hipSuccess)                                                          \
      return helm::report_error((int)e_, std::string(#call) + ": " + hipGetErrorString(e_)); \
  } while (0)

}  // namespace

extern "C" int helm_measure_bandwidth(int device, uint64_t stream_bytes, uint64_t link_bytes,
                                      int iters, helm_bandwidth* out) {
  if (!out || iters < 1 || stream_bytes < 4096 || link_bytes < 4096 ||
      stream_bytes % 16 || link_bytes % 16)
    return helm::report_error(HELM_E_INVALID,
                              "need out, iters >= 1 and byte counts >= 4096, multiples of 16");
  int prev = 0;
  PROBE_HIP(hipGetDevice(&prev));
  PROBE_HIP(hipSetDevice(device));
  int rc = HELM_OK;
  {
    Probe pr;
    auto run = [&]() -> int {
      PROBE_HIP(hipStreamCreateWithFlags(&pr.st, hipStreamNonBlocking));
      PROBE_HIP(hipEventCreate(&pr.e0));
      PROBE_HIP(hipEventCreate(&pr.e1));
      // the device buffers also serve the link copies
      const uint64_t dev_bytes = stream_bytes > link_bytes ? stream_bytes : link_bytes;
      PROBE_HIP(hipMalloc(&pr.src, dev_bytes));
      PROBE_HIP(hipMalloc(&pr.dst, dev_bytes));
      PROBE_HIP(hipMalloc(&pr.bad, sizeof(unsigned long long)));
      PROBE_HIP(hipHostMalloc(&pr.pin, link_bytes, hipHostMallocDefault));
      const size_t words = stream_bytes / 4;
      hipLaunchKernelGGL(fill_index_kernel, dim3(1024), dim3(256), 0, pr.st,
                         static_cast<uint32_t*>(pr.src), words);
      PROBE_HIP(hipGetLastError());
      int cus = 0;
      PROBE_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
      const dim3 grid(8 * (cus > 0 ? cus : 256)), block(256);
      // op() issues one copy and returns its launch status.  Untimed copies
      // first: at least three (HELM's two warm-ups and its probe call,
      // device_profiler.py:94-107) and at least 20 ms of them — the host link
      // reads well below its rate for the first milliseconds of a process
      // (23-37 GB/s against 57 GB/s in the same run on the same machine).
      auto timed = [&](auto&& op, double* secs) -> int {
        const auto w0 = std::chrono::steady_clock::now();
        for (int w = 0;; ++w) {
          PROBE_HIP(op());
          PROBE_HIP(hipStreamSynchronize(pr.st));
          const double el = std::chrono::duration<double>(std::chrono::steady_clock::now() -
                                                          w0).count();
          if (w >= 2 && el >= 0.02) break;
        }
        PROBE_HIP(hipEventRecord(pr.e0, pr.st));
        for (int i = 0; i < iters; ++i) PROBE_HIP(op());
        PROBE_HIP(hipEventRecord(pr.e1, pr.st));
        PROBE_HIP(hipEventSynchronize(pr.e1));
        float ms = 0.f;
        PROBE_HIP(hipEventElapsedTime(&ms, pr.e0, pr.e1));
        *secs = ms / 1e3 / iters;
        return HELM_OK;
      };
      double t = 0.0;
      // device memory: a read and a write of every byte per copy
      int r = timed([&] {
        hipLaunchKernelGGL(stream_copy_kernel, grid, block, 0, pr.st,
                           static_cast<const u32x4*>(pr.src), static_cast<u32x4*>(pr.dst),
                           (size_t)(stream_bytes / 16));
        return hipGetLastError();
      }, &t);
      if (r != HELM_OK) return r;
      out->device_copy_bytes_per_s = 2.0 * (double)stream_bytes / t;
      hipLaunchKernelGGL(zero_u64_kernel, dim3(1), dim3(1), 0, pr.st, pr.bad);
      hipLaunchKernelGGL(count_mismatch_kernel, dim3(1024), dim3(256), 0, pr.st,
                         static_cast<const uint32_t*>(pr.src), static_cast<const uint32_t*>(pr.dst),
                         words, pr.bad);
      PROBE_HIP(hipGetLastError());
      unsigned long long bad = 0;
      PROBE_HIP(hipMemcpyAsync(&bad, pr.bad, sizeof(bad), hipMemcpyDeviceToHost, pr.st));
      PROBE_HIP(hipStreamSynchronize(pr.st));
      out->copy_mismatched_words = (int64_t)bad;
      // host link: pinned host memory to the device and back
      r = timed([&] {
        return hipMemcpyAsync(pr.dst, pr.pin, link_bytes, hipMemcpyHostToDevice, pr.st);
      }, &t);
      if (r != HELM_OK) return r;
      out->h2d_bytes_per_s = (double)link_bytes / t;
      r = timed([&] {
        return hipMemcpyAsync(pr.pin, pr.src, link_bytes, hipMemcpyDeviceToHost, pr.st);
      }, &t);
      if (r != HELM_OK) return r;
      out->d2h_bytes_per_s = (double)link_bytes / t;
      return HELM_OK;
    };
    rc = run();
  }
  const hipError_t e = hipSetDevice(prev);
  if (rc == HELM_OK && e != hipSuccess)
    return helm::report_error((int)e, std::string("hipSetDevice: ") + hipGetErrorString(e));
  return rc;
}

extern "C" int helm_profile_read_pass(const void* const* bufs, int nbufs, uint64_t bytes,
                                      int workgroups, uint64_t tail_bytes, int tail_workgroups,
                                      int iters, void* stream, float* us_per_iter) {
  if (!bufs || nbufs < 1 || !us_per_iter || iters < 1 || bytes < 16 || bytes % 16 ||
      workgroups < 1 || tail_bytes % 16 || tail_bytes > bytes ||
      (tail_bytes && tail_workgroups < 1))
    return helm::report_error(HELM_E_INVALID,
                              "need buffers, iters >= 1, byte counts multiples of 16 (tail <= "
                              "bytes) and workgroups >= 1");
  for (int i = 0; i < nbufs; ++i)
    if (!bufs[i]) return helm::report_error(HELM_E_INVALID, "null buffer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int sink_words = workgroups > tail_workgroups ? workgroups : tail_workgroups;
  uint32_t* sink = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  auto run = [&]() -> int {
    PROBE_HIP(hipMalloc(&sink, (size_t)sink_words * 4));
    PROBE_HIP(hipEventCreate(&e0));
    PROBE_HIP(hipEventCreate(&e1));
    auto pass = [&](int i) -> hipError_t {
      hipLaunchKernelGGL(read_pass_kernel, dim3(workgroups), dim3(256), 0, st,
                         static_cast<const u32x4*>(bufs[i % nbufs]), (size_t)(bytes / 16), sink);
      if (tail_bytes)
        hipLaunchKernelGGL(read_pass_kernel, dim3(tail_workgroups), dim3(256), 0, st,
                           static_cast<const u32x4*>(bufs[(i + 1) % nbufs]),
                           (size_t)(tail_bytes / 16), sink);
      return hipGetLastError();
    };
    for (int i = 0; i < 3; ++i) PROBE_HIP(pass(i));
    PROBE_HIP(hipEventRecord(e0, st));
    for (int i = 0; i < iters; ++i) PROBE_HIP(pass(i));
    PROBE_HIP(hipEventRecord(e1, st));
    PROBE_HIP(hipEventSynchronize(e1));
    float ms = 0.f;
    PROBE_HIP(hipEventElapsedTime(&ms, e0, e1));
    *us_per_iter = ms * 1e3f / iters;
    return HELM_OK;
  };
  const int rc = run();
  if (st) (void)hipStreamSynchronize(st);
  if (sink) (void)hipFree(sink);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  return rc;
}
