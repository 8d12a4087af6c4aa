// Streaming-read rate of the device memory: the measured ceiling that the
// benchmark sets beside each decode line (the decode layers read their
// factors and write almost nothing, so a copy, which also writes, is not
// their ceiling).  Built as its own library (libhbmread.so), outside the
// SVD-MLP C ABI.
//
// Every thread reads 16-byte words grid-stride, eight loads in flight, folds
// them with XOR and stores one word, so no load can be dropped.  On MI355X a
// 1 GiB buffer read by 8192 blocks of 256 threads this way takes ~180 us
// (5.9-6.0 TB/s); 1024-4096 blocks or 4 / 16 loads in flight read at
// 5.0-5.9 TB/s.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256, kInFlight = 8;

__global__ __launch_bounds__(kThreads) void read_words_kernel(const u32x4* __restrict__ p, int64_t n, unsigned* out) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + (kInFlight - 1) * stride < n; i += kInFlight * stride) {
    u32x4 v[kInFlight];
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) acc ^= v[u];
  }
  for (; i < n; i += stride) acc ^= p[i];
  out[(int64_t)blockIdx.x * kThreads + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

}  // namespace

// Reads nbytes (a multiple of 16, 16-byte aligned) at p with `blocks` blocks
// on `stream` (a hipStream_t, null for the default stream); out receives
// blocks * 256 words (out_bytes at least that).  0 on success, -1 for an
// invalid argument, -2 if the launch failed.
extern "C" int hbm_read_words(const void* p, int64_t nbytes, void* out, int64_t out_bytes, int32_t blocks,
                              void* stream) {
  if (!p || !out || nbytes <= 0 || nbytes % 16 != 0 || ((uintptr_t)p & 15u) != 0 || blocks <= 0 ||
      (int64_t)blocks * kThreads * 4 > out_bytes)
    return -1;
  hipLaunchKernelGGL(read_words_kernel, dim3(blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(p), nbytes / 16, static_cast<unsigned*>(out));
  return hipGetLastError() == hipSuccess ? 0 : -2;
}
