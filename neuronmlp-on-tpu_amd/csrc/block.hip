// RMSNorm prologue and residual epilogue of the MLP block
// y = x + svd_mlp(rmsnorm(x) * gain)  (models/modeling_llama.py:253-262,
// bench/e2e_block.py:268-278).  Both are single HBM passes over (T, d).
#include <algorithm>

#include "dispatch.hpp"

namespace svdmlp {

namespace {

// One 256-thread block per row: mean of squares in fp32, then
// y = act(gain * (x * (1 / sqrt(mean + eps)))), the order of LlamaRMSNorm.
template <bool BF16>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const void* x, const float* gain, void* y, int64_t d,
                                                      float eps) {
  __shared__ float part[8];
  const int64_t row = blockIdx.x;
  float ss = 0.f;
  if constexpr (BF16) {
    const uint16_t* xr = static_cast<const uint16_t*>(x) + row * d;
    for (int64_t j = threadIdx.x; j < d; j += 256) {
      const float v = bf16_bits_to_f32(xr[j]);
      ss += v * v;
    }
  } else {
    const float* xr = static_cast<const float*>(x) + row * d;
    for (int64_t j = threadIdx.x; j < d; j += 256) ss += xr[j] * xr[j];
  }
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  const float rstd = 1.0f / sqrtf(tot / (float)d + eps);
  if constexpr (BF16) {
    const uint16_t* xr = static_cast<const uint16_t*>(x) + row * d;
    uint16_t* yr = static_cast<uint16_t*>(y) + row * d;
    for (int64_t j = threadIdx.x; j < d; j += 256)
      yr[j] = (uint16_t)f32_to_bf16_bits(gain[j] * (bf16_bits_to_f32(xr[j]) * rstd));
  } else {
    const float* xr = static_cast<const float*>(x) + row * d;
    float* yr = static_cast<float*>(y) + row * d;
    for (int64_t j = threadIdx.x; j < d; j += 256) yr[j] = gain[j] * (xr[j] * rstd);
  }
}

// y = act(x + y), the residual add rounded to the activation dtype.
template <bool BF16>
__global__ void residual_add_kernel(const void* x, void* y, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    if constexpr (BF16) {
      const uint16_t* xs = static_cast<const uint16_t*>(x);
      uint16_t* ys = static_cast<uint16_t*>(y);
      ys[i] = (uint16_t)f32_to_bf16_bits(bf16_bits_to_f32(xs[i]) + bf16_bits_to_f32(ys[i]));
    } else {
      static_cast<float*>(y)[i] += static_cast<const float*>(x)[i];
    }
  }
}

}  // namespace

hipError_t launch_rmsnorm(const void* x, const float* gain, void* y, int64_t T, int64_t d, float eps, bool bf16,
                          hipStream_t st) {
  if (T <= 0) return hipSuccess;
  if (bf16)
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3((unsigned)T), dim3(256), 0, st, x, gain, y, d, eps);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3((unsigned)T), dim3(256), 0, st, x, gain, y, d, eps);
  return hipGetLastError();
}

hipError_t launch_residual_add(const void* x, void* y, int64_t n, bool bf16, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const unsigned blocks = (unsigned)std::min<int64_t>((n + 255) / 256, 4096);
  if (bf16)
    hipLaunchKernelGGL(residual_add_kernel<true>, dim3(blocks), dim3(256), 0, st, x, y, n);
  else
    hipLaunchKernelGGL(residual_add_kernel<false>, dim3(blocks), dim3(256), 0, st, x, y, n);
  return hipGetLastError();
}

}  // namespace svdmlp
