// Shared device helpers for the SVD-MLP kernels (gfx950 / CDNA4).
//
// Element types on the path: bf16 activations and weights (the headline),
// fp32 (the reference's `mixed_precision=False` arm) and fp8 e4m3fn weights
// with per-output-channel fp32 scales.  All arithmetic accumulates in fp32 on
// MFMA; bf16 values are produced by round-to-nearest-even.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace svdmlp {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Scalar conversions
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h16) {
  return __uint_as_float(h16 << 16);
}

// fp32 -> bf16, round to nearest even, NaN stays NaN: gfx950's
// v_cvt_pk_bf16_f32, two values per instruction (the vector conversion
// compiles to it).  It equals the integer form -- u += 0x7fff + ((u >> 16) & 1),
// keep the high half -- on every non-NaN input, denormals included (checked
// on MI355X over 2^28 value pairs: every exponent, halfway and near-halfway
// mantissas); the integer form took ~6 instructions per value in the
// epilogues.
typedef float f32x2_cvt __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_cvt __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_cvt{lo, hi}, bf16x2_cvt));
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return pack_bf16x2(f, 0.0f) & 0xffffu; }

// fp8 e4m3fn (OCP, no infinities, 0x7f/0xff = NaN, max 448) -> fp32, exact.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t s = (b & 0x80u) << 24;
  const uint32_t e = (b >> 3) & 0xfu;
  const uint32_t m = b & 0x7u;
  if (e == 0xfu && m == 0x7u) return __uint_as_float(0x7fc00000u | s);
  if (e == 0) {  // subnormal: m * 2^-9
    return __uint_as_float(s) + (s ? -1.0f : 1.0f) * (float)m * 0.001953125f;
  }
  return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}

// Branch-stable SiLU in fp32 (kernels/reference.py:37-51): every exp
// argument is <= 0, so 1 + z lies in [1, 2] and the hardware reciprocal
// (v_rcp_f32, 1 ulp) stands in for an IEEE division, whose scale / fma /
// fixup sequence made the SwiGLU epilogue of the 8B layer ~4 us slower; the
// result is rounded to bf16 (8 bits of mantissa) afterwards.
__device__ __forceinline__ float silu_f32(float x) {
  const float z = __expf(-fabsf(x));
  const float r = __builtin_amdgcn_rcpf(1.0f + z);
  return x * ((x >= 0.0f) ? r : z * r);
}

// ---------------------------------------------------------------------------
// MFMA wrappers.  One "k-step" consumes four 16-byte chunks of K per lane
// group (lane / 16 selects the chunk), i.e. 32 bf16 or 16 fp32 values of K.
// D[row][col] lands in lane (row / 4) * 16 + col, register row % 4.
// ---------------------------------------------------------------------------

__device__ __forceinline__ f32x4 mfma_chunk(u32x4 a, u32x4 b, f32x4 c, __bf16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_chunk(u32x4 a, u32x4 b, f32x4 c, float) {
  // A 16-byte chunk holds four consecutive k; the hardware k index of
  // 16x16x4f32 is lane / 16, so the j-th call covers k = 4 * (lane / 16) + j.
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
  return c;
}

// ---------------------------------------------------------------------------
// Global memory helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ u32x4 ldg128(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ u32x2 ldg64(const void* p) {
  return *reinterpret_cast<const u32x2*>(p);
}

// Blocks are dispatched round-robin over the 8 XCDs (each with its own L2).
// Remap the hardware block id so that logically consecutive tiles (which
// share an operand panel) run on the same XCD.  Bijective for any count.
__device__ __forceinline__ int xcd_remap(int w, int count) {
  constexpr int kXcd = 8;
  const int q = count / kXcd, rem = count % kXcd;
  const int xcd = w % kXcd, slot = w / kXcd;
  return (xcd < rem) ? xcd * (q + 1) + slot : rem * (q + 1) + (xcd - rem) * q + slot;
}

}  // namespace svdmlp
