// RMSNorm prologue and residual epilogue of the MLP block
// y = x + svd_mlp(rmsnorm(x) * gain)  (models/modeling_llama.py:253-262,
// bench/e2e_block.py:268-278).  Both are single HBM passes over (T, d),
// moved in 16-byte pieces (8 bf16 or 4 fp32 per lane access).
#include <algorithm>

#include "dispatch.hpp"

namespace svdmlp {

namespace {

// One 256-thread block per row: mean of squares in fp32, then
// y = act(gain * (x * (1 / sqrt(mean + eps)))), the order of LlamaRMSNorm.
// VEC: d is a multiple of 8 (bf16) / 4 (fp32) and the rows are 16-byte
// aligned, so each thread moves whole 16-byte pieces; the row is read once
// into registers (up to PER pieces per thread) and written from them.
template <bool BF16, bool VEC>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const void* x, const float* gain, void* y, int64_t d,
                                                      float eps) {
  __shared__ float part[4];
  const int64_t row = blockIdx.x;
  constexpr int E = BF16 ? 8 : 4;  // elements per 16-byte piece
  constexpr int PER = 4;           // pieces per thread kept in registers (rows up to 256 * 4 * E)
  float ss = 0.f;
  u32x4 keep[PER];
  const int64_t pieces = d / E;
  if constexpr (VEC) {
    const u32x4* xr = reinterpret_cast<const u32x4*>(static_cast<const char*>(x) + row * d * (BF16 ? 2 : 4));
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int64_t i = threadIdx.x + 256 * q;
      keep[q] = i < pieces ? xr[i] : u32x4{0u, 0u, 0u, 0u};
    }
    for (int64_t i = threadIdx.x + 256 * PER; i < pieces; i += 256) {  // rows longer than the register copy
      const u32x4 v = xr[i];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        if constexpr (BF16) {
          const float a = bf16_bits_to_f32(v[w] & 0xffffu), b = bf16_bits_to_f32(v[w] >> 16);
          ss += a * a + b * b;
        } else {
          const float a = __uint_as_float(v[w]);
          ss += a * a;
        }
      }
    }
#pragma unroll
    for (int q = 0; q < PER; ++q)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        if constexpr (BF16) {
          const float a = bf16_bits_to_f32(keep[q][w] & 0xffffu), b = bf16_bits_to_f32(keep[q][w] >> 16);
          ss += a * a + b * b;
        } else {
          const float a = __uint_as_float(keep[q][w]);
          ss += a * a;
        }
      }
  } else if constexpr (BF16) {
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
  if constexpr (VEC) {
    const char* xb = static_cast<const char*>(x) + row * d * (BF16 ? 2 : 4);
    u32x4* yr = reinterpret_cast<u32x4*>(static_cast<char*>(y) + row * d * (BF16 ? 2 : 4));
    auto norm = [&](u32x4 v, int64_t i) {
      const f32x4* g = reinterpret_cast<const f32x4*>(gain + i * E);
      u32x4 o;
      if constexpr (BF16) {
        const f32x4 g0 = g[0], g1 = g[1];
        const float gl[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
        for (int w = 0; w < 4; ++w)
          o[w] = pack_bf16x2(gl[2 * w] * (bf16_bits_to_f32(v[w] & 0xffffu) * rstd),
                             gl[2 * w + 1] * (bf16_bits_to_f32(v[w] >> 16) * rstd));
      } else {
        const f32x4 g0 = g[0];
        const float gl[4] = {g0.x, g0.y, g0.z, g0.w};
#pragma unroll
        for (int w = 0; w < 4; ++w) o[w] = __float_as_uint(gl[w] * (__uint_as_float(v[w]) * rstd));
      }
      return o;
    };
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int64_t i = threadIdx.x + 256 * q;
      if (i < pieces) yr[i] = norm(keep[q], i);
    }
    for (int64_t i = threadIdx.x + 256 * PER; i < pieces; i += 256)
      yr[i] = norm(reinterpret_cast<const u32x4*>(xb)[i], i);
  } else if constexpr (BF16) {
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

// y = act(x + y), the residual add rounded to the activation dtype; VEC: n is
// a multiple of the 16-byte piece and both buffers are 16-byte aligned.
template <bool BF16, bool VEC>
__global__ void residual_add_kernel(const void* x, void* y, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if constexpr (VEC) {
    const u32x4* xs = static_cast<const u32x4*>(x);
    u32x4* ys = static_cast<u32x4*>(y);
    const int64_t pieces = n / (BF16 ? 8 : 4);
    for (int64_t i = t0; i < pieces; i += stride) {
      const u32x4 a = xs[i], b = ys[i];
      u32x4 o;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        if constexpr (BF16)
          o[w] = pack_bf16x2(bf16_bits_to_f32(a[w] & 0xffffu) + bf16_bits_to_f32(b[w] & 0xffffu),
                             bf16_bits_to_f32(a[w] >> 16) + bf16_bits_to_f32(b[w] >> 16));
        else
          o[w] = __float_as_uint(__uint_as_float(a[w]) + __uint_as_float(b[w]));
      }
      ys[i] = o;
    }
  } else {
    for (int64_t i = t0; i < n; i += stride) {
      if constexpr (BF16) {
        const uint16_t* xs = static_cast<const uint16_t*>(x);
        uint16_t* ys = static_cast<uint16_t*>(y);
        ys[i] = (uint16_t)f32_to_bf16_bits(bf16_bits_to_f32(xs[i]) + bf16_bits_to_f32(ys[i]));
      } else {
        static_cast<float*>(y)[i] += static_cast<const float*>(x)[i];
      }
    }
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

// out[c][r] = in[r][c] (bf16, r < rows, c < cols): 64 x 64 tiles through
// LDS, 256 threads; a quarter-wave group moves 64 consecutive elements (128
// contiguous bytes) of one row per access on both sides.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const uint16_t* in, int64_t ldi, uint16_t* out,
                                                             int64_t ldo, int rows, int cols) {
  __shared__ uint16_t tile[64][65];  // odd pitch: the column reads of the store side hit distinct banks
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int t = threadIdx.x & 63, q = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = 4 * i + q, c = t;
    if (r0 + r < rows && c0 + c < cols) tile[r][c] = in[(int64_t)(r0 + r) * ldi + c0 + c];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = 4 * i + q, r = t;
    if (c0 + c < cols && r0 + r < rows) out[(int64_t)(c0 + c) * ldo + r0 + r] = tile[r][c];
  }
}

// The same transpose in 16-byte pieces on both global sides, for rows, cols
// and both pitches multiples of 8 and 16-byte aligned buffers (a piece is then
// wholly inside or wholly outside the matrix).  Thread t moves piece t % 8 of
// rows (t / 8) and (t / 8 + 32): two 16-byte loads in flight, 8 LDS stores of
// one element each; the store side gathers 8 elements of one column from 8
// consecutive tile rows into one 16-byte store.  (The 2-byte version spent
// 8.2 us on the (128 x 14336) h of an 8B layer: 0.9 TB/s.)
__global__ __launch_bounds__(256) void transpose_bf16_v8_kernel(const uint16_t* in, int64_t ldi, uint16_t* out,
                                                                int64_t ldo, int rows, int cols) {
  // pitch 65: a store-side wave's lanes (8 pieces x 8 columns) fall on 32
  // distinct 4-byte words per element read
  __shared__ uint16_t tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int t = threadIdx.x, k = t & 7, j = t >> 3;
  u32x4 v[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int r = r0 + j + 32 * s, c = c0 + 8 * k;
    v[s] = (r < rows && c < cols) ? *reinterpret_cast<const u32x4*>(in + (int64_t)r * ldi + c) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const uint32_t w[4] = {v[s].x, v[s].y, v[s].z, v[s].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[j + 32 * s][8 * k + e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int c = j + 32 * s, r = 8 * k;
    if (c0 + c >= cols || r0 + r >= rows) continue;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = (uint32_t)tile[r + 2 * e][c] | ((uint32_t)tile[r + 2 * e + 1][c] << 16);
    *reinterpret_cast<u32x4*>(out + (int64_t)(c0 + c) * ldo + r0 + r) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

hipError_t launch_rmsnorm(const void* x, const float* gain, void* y, int64_t T, int64_t d, float eps, bool bf16,
                          hipStream_t st) {
  if (T <= 0) return hipSuccess;
  const bool vec = d % (bf16 ? 8 : 4) == 0 && aligned16(x) && aligned16(y) && aligned16(gain);
  const dim3 grid((unsigned)T), block(256);
  if (bf16 && vec)
    hipLaunchKernelGGL((rmsnorm_kernel<true, true>), grid, block, 0, st, x, gain, y, d, eps);
  else if (bf16)
    hipLaunchKernelGGL((rmsnorm_kernel<true, false>), grid, block, 0, st, x, gain, y, d, eps);
  else if (vec)
    hipLaunchKernelGGL((rmsnorm_kernel<false, true>), grid, block, 0, st, x, gain, y, d, eps);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<false, false>), grid, block, 0, st, x, gain, y, d, eps);
  return hipGetLastError();
}

hipError_t launch_residual_add(const void* x, void* y, int64_t n, bool bf16, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const bool vec = n % (bf16 ? 8 : 4) == 0 && aligned16(x) && aligned16(y);
  const int64_t work = vec ? n / (bf16 ? 8 : 4) : n;
  const unsigned blocks = (unsigned)std::min<int64_t>((work + 255) / 256, 4096);
  if (bf16 && vec)
    hipLaunchKernelGGL((residual_add_kernel<true, true>), dim3(blocks), dim3(256), 0, st, x, y, n);
  else if (bf16)
    hipLaunchKernelGGL((residual_add_kernel<true, false>), dim3(blocks), dim3(256), 0, st, x, y, n);
  else if (vec)
    hipLaunchKernelGGL((residual_add_kernel<false, true>), dim3(blocks), dim3(256), 0, st, x, y, n);
  else
    hipLaunchKernelGGL((residual_add_kernel<false, false>), dim3(blocks), dim3(256), 0, st, x, y, n);
  return hipGetLastError();
}

hipError_t launch_transpose_bf16(const uint16_t* in, int64_t ldi, uint16_t* out, int64_t ldo, int rows, int cols,
                                 hipStream_t st) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  dim3 grid((cols + 63) / 64, (rows + 63) / 64);
  if (grid.y > 65535) return hipErrorInvalidValue;
  const bool v8 = rows % 8 == 0 && cols % 8 == 0 && ldi % 8 == 0 && ldo % 8 == 0 && aligned16(in) && aligned16(out);
  if (v8)
    hipLaunchKernelGGL(transpose_bf16_v8_kernel, grid, dim3(256), 0, st, in, ldi, out, ldo, rows, cols);
  else
    hipLaunchKernelGGL(transpose_bf16_kernel, grid, dim3(256), 0, st, in, ldi, out, ldo, rows, cols);
  return hipGetLastError();
}

}  // namespace svdmlp
