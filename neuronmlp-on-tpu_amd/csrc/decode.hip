// Decode-shape instances and the small elementwise kernels.
#include "dispatch.hpp"

namespace svdmlp {

namespace {

template <int MT, int SRCA, int SRCB, bool BK>
hipError_t go(const DecodeParams& p, int blocks, hipStream_t st) {
  // Keep 8*U weight rows of 1 KB in flight per wave; fewer when the token
  // tiles already need many accumulator registers.
  constexpr int U = MT <= 1 ? 4 : 2;
  hipLaunchKernelGGL((decode_kernel<MT, U, SRCA, SRCB, true, BK>), dim3(blocks), dim3(256), 0, st, p);
  return hipGetLastError();
}

template <int MT, int SRCA>
hipError_t go_b(const DecodeDesc& d, const DecodeParams& p, int blocks, hipStream_t st, const char** why) {
  if (d.srcb == SRC_BF16) return d.b_kc ? go<MT, SRCA, SRC_BF16, true>(p, blocks, st)
                                        : go<MT, SRCA, SRC_BF16, false>(p, blocks, st);
  if (d.srcb == SRC_FP8 && !d.b_kc) return go<MT, SRCA, SRC_FP8, false>(p, blocks, st);
  *why = "decode: unsupported weight type/layout";
  return hipErrorInvalidValue;
}

template <int MT>
hipError_t go_a(const DecodeDesc& d, const DecodeParams& p, int blocks, hipStream_t st, const char** why) {
  switch (d.srca) {
    case SRC_BF16: return go_b<MT, SRC_BF16>(d, p, blocks, st, why);
    case SRC_F32: return go_b<MT, SRC_F32>(d, p, blocks, st, why);
    case SRC_SWIGLU: return go_b<MT, SRC_SWIGLU>(d, p, blocks, st, why);
    default: *why = "decode: unsupported activation source"; return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_decode(const DecodeDesc& d, const DecodeParams& p, int blocks, hipStream_t st,
                         const char** why) {
  switch (d.mt) {
    case 1: return go_a<1>(d, p, blocks, st, why);
    case 2: return go_a<2>(d, p, blocks, st, why);
    case 4: return go_a<4>(d, p, blocks, st, why);
    default: *why = "decode: token tile count must be 1, 2 or 4"; return hipErrorInvalidValue;
  }
}

__global__ void fill_zero_kernel(float* p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * 4;
  for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < n; i += stride) {
    if (i + 3 < n) {
      *reinterpret_cast<f32x4*>(p + i) = f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
      for (int64_t t = i; t < n; ++t) p[t] = 0.0f;
    }
  }
}

// out[i] = bf16(in[i]), eight elements per thread and step.
__global__ void cvt_bf16_kernel(const float* in, uint16_t* out, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * 8;
  for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8; i < n; i += stride) {
    if (i + 7 < n) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(in + i);
      const f32x4 b = *reinterpret_cast<const f32x4*>(in + i + 4);
      *reinterpret_cast<u32x4*>(out + i) = u32x4{pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w),
                                                 pack_bf16x2(b.x, b.y), pack_bf16x2(b.z, b.w)};
    } else {
      for (int64_t t = i; t < n; ++t) out[t] = (uint16_t)f32_to_bf16_bits(in[t]);
    }
  }
}

hipError_t launch_cvt_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const int blocks = (int)std::min<int64_t>((n / 8 + 255) / 256 + 1, 2048);
  hipLaunchKernelGGL(cvt_bf16_kernel, dim3(blocks), dim3(256), 0, st, in, out, n);
  return hipGetLastError();
}

// out[i] = bf16(sum over split-K slices), eight elements per thread and step;
// slices are summed in order, so the result is deterministic.
__global__ void reduce_bf16_kernel(const float* in, int slices, int64_t stride, uint16_t* out, int64_t n) {
  const int64_t step = (int64_t)gridDim.x * blockDim.x * 8;
  for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8; i < n; i += step) {
    if (i + 7 < n) {
      f32x4 a = *reinterpret_cast<const f32x4*>(in + i);
      f32x4 b = *reinterpret_cast<const f32x4*>(in + i + 4);
      for (int s = 1; s < slices; ++s) {
        a += *reinterpret_cast<const f32x4*>(in + s * stride + i);
        b += *reinterpret_cast<const f32x4*>(in + s * stride + i + 4);
      }
      *reinterpret_cast<u32x4*>(out + i) = u32x4{pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w),
                                                 pack_bf16x2(b.x, b.y), pack_bf16x2(b.z, b.w)};
    } else {
      for (int64_t t = i; t < n; ++t) {
        float v = in[t];
        for (int s = 1; s < slices; ++s) v += in[s * stride + t];
        out[t] = (uint16_t)f32_to_bf16_bits(v);
      }
    }
  }
}

hipError_t launch_reduce_bf16(const float* in, int slices, int64_t stride, uint16_t* out, int64_t n,
                              hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const int blocks = (int)std::min<int64_t>((n / 8 + 255) / 256 + 1, 4096);
  hipLaunchKernelGGL(reduce_bf16_kernel, dim3(blocks), dim3(256), 0, st, in, slices, stride, out, n);
  return hipGetLastError();
}

hipError_t launch_fill_zero(float* p, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const int64_t vec = (n + 3) / 4;
  int blocks = (int)std::min<int64_t>((vec + 255) / 256, 4096);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, st, p, n);
  return hipGetLastError();
}

hipError_t launch_finalize(const float* g, const float* u, int64_t ldi, uint16_t* out, int64_t ldo, int rows,
                           int cols, bool swiglu, bool out_t, hipStream_t st) {
  const int64_t total = (int64_t)rows * cols;
  if (total <= 0) return hipSuccess;
  int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
  if (swiglu) {
    if (out_t)
      hipLaunchKernelGGL((finalize_bf16_kernel<true, true>), dim3(blocks), dim3(256), 0, st, g, u, ldi, out, ldo,
                         rows, cols);
    else
      hipLaunchKernelGGL((finalize_bf16_kernel<true, false>), dim3(blocks), dim3(256), 0, st, g, u, ldi, out, ldo,
                         rows, cols);
  } else {
    hipLaunchKernelGGL((finalize_bf16_kernel<false, false>), dim3(blocks), dim3(256), 0, st, g, u, ldi, out, ldo,
                       rows, cols);
  }
  return hipGetLastError();
}

}  // namespace svdmlp
