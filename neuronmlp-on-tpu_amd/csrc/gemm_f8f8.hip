// Launchers of the fp8 x fp8 GEMM and the e4m3 row quantisation.
#include "dispatch.hpp"
#include "gemm_f8f8.hpp"

namespace svdmlp {

namespace {

// Row quantisation to e4m3fn: row m of h (bf16, pitch ldh) -> q (pitch ldq
// bytes) with s[m] = amax / 448 and q = e4m3(h * (448 / amax)) (round to
// nearest even, the hardware conversion; a zero row gets s = 1 and zeros).
// One block per row; each thread keeps its 8-element pieces in registers
// between the amax and the conversion pass (n <= 8 * kF8Threads * kF8QPieces).
__global__ __launch_bounds__(kF8Threads) void quant_rows_e4m3_kernel(const uint16_t* h, int64_t ldh, uint8_t* q,
                                                                     int64_t ldq, float* s, int n, int blk) {
  __shared__ float part[kF8Threads / 64];
  const int64_t row = blockIdx.x;
  const uint16_t* hr = h + row * ldh;
  u32x4 v[kF8QPieces];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < kF8QPieces; ++i) {
    const int e = 8 * ((int)threadIdx.x + kF8Threads * i);
    v[i] = e < n ? *reinterpret_cast<const u32x4*>(hr + e) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int w = 0; w < 4; ++w)
      amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(v[i][w] << 16)), fabsf(__uint_as_float(v[i][w] & 0xffff0000u))));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = part[0];
#pragma unroll
  for (int w = 1; w < kF8Threads / 64; ++w) amax = fmaxf(amax, part[w]);
  const float inv = amax > 0.f ? 448.0f / amax : 1.0f;
  if (threadIdx.x == 0) s[row] = amax > 0.f ? amax / 448.0f : 1.0f;
  // row-major, or 16 x 128 blocks (2 KB each; a thread's 8 bytes never cross one)
  uint8_t* qr = blk ? q + (row >> 4) * (int64_t)(n >> 7) * 2048 + (row & 15) * 128 : q + row * ldq;
#pragma unroll
  for (int i = 0; i < kF8QPieces; ++i) {
    const int e = 8 * ((int)threadIdx.x + kF8Threads * i);
    if (e < n) {
      u32x2 o;
      const u32x4 x = v[i];
      o.x = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(x.x << 16) * inv,
                                                        __uint_as_float(x.x & 0xffff0000u) * inv, 0, false);
      o.x = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(x.y << 16) * inv,
                                                        __uint_as_float(x.y & 0xffff0000u) * inv, (int)o.x, true);
      o.y = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(x.z << 16) * inv,
                                                        __uint_as_float(x.z & 0xffff0000u) * inv, 0, false);
      o.y = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(x.w << 16) * inv,
                                                        __uint_as_float(x.w & 0xffff0000u) * inv, (int)o.y, true);
      *reinterpret_cast<u32x2*>(qr + (blk ? (e >> 7) * 2048 + (e & 127) : e)) = o;
    }
  }
}

}  // namespace

hipError_t launch_f8_gemm(const F8Params& p, int splits, int nw, hipStream_t st, const char** why) {
  if ((nw != 4 && nw != 8) || p.K % kF8BK || p.k_split % kF8BK || p.N % 16 || p.lda % 16 || p.ldb % 16 || splits < 1 ||
      ((uintptr_t)p.sb & 15u)) {
    *why = "fp8 x fp8 GEMM: K and K per split multiples of 128, N and pitches multiples of 16, aligned scales";
    return hipErrorInvalidValue;
  }
  if (p.tile0 < 0 || p.tiles < 1 || p.tile0 + p.tiles > p.mtiles * p.ntiles) {
    *why = "fp8 x fp8 GEMM: the launch's tiles must lie within the mtiles x ntiles";
    return hipErrorInvalidValue;
  }
  const dim3 grid(p.tiles, splits);
  if (nw == 4) {
    if (splits > 1)
      hipLaunchKernelGGL((f8_gemm_kernel<true, 4>), grid, dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((f8_gemm_kernel<false, 4>), grid, dim3(256), 0, st, p);
  } else {
    if (splits > 1)
      hipLaunchKernelGGL((f8_gemm_kernel<true, 8>), grid, dim3(512), 0, st, p);
    else
      hipLaunchKernelGGL((f8_gemm_kernel<false, 8>), grid, dim3(512), 0, st, p);
  }
  return hipGetLastError();
}

hipError_t launch_quant_rows_e4m3(const uint16_t* h, int64_t ldh, uint8_t* q, int64_t ldq, float* s, int rows, int n,
                                  hipStream_t st, const char** why, bool blk) {
  if (n % 8 || n > 8 * kF8Threads * kF8QPieces || ldh % 8 || ldq % 8 || (blk && n % 128)) {
    *why = "e4m3 row quantisation: row length a multiple of 8 (of 128 in blocks) and at most 32768, pitches multiples of 8";
    return hipErrorInvalidValue;
  }
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(quant_rows_e4m3_kernel, dim3(rows), dim3(kF8Threads), 0, st, h, ldh, q, ldq, s, n, blk ? 1 : 0);
  return hipGetLastError();
}

}  // namespace svdmlp
