// Instances of the large-tile prefill GEMM (bf16 operands).
#include "dispatch.hpp"
#include "gemm_big.hpp"

namespace svdmlp {

namespace {

template <int FN, bool BK, int EPI, bool F32 = false, bool F8 = false, int NW = 8, int NS = 4, int KG = 1, bool TR = false>
hipError_t go(const BigParams& p, int splits, int batch, hipStream_t st) {
  using C = BigCfg<FN, BK, EPI, F32, F8, NW, NS, KG, TR>;
  dim3 grid(p.tiles > 0 ? p.tiles : p.mtiles * p.ntiles, splits, batch);
  hipLaunchKernelGGL(big_gemm_kernel<C>, grid, dim3(C::THREADS), 0, st, p);
  return hipGetLastError();
}

// 256 x 128 tiles with natural-layout bf16 B keep 6 LDS stages (8 KB of B
// each in 256-byte rows), the others 4.
template <int FN, int EPI, bool F32 = false>
hipError_t go_b(const BigDesc& d, const BigParams& p, int splits, int batch, hipStream_t st) {
  // K groups (128-row tiles), natural-layout bf16 B, store epilogues: five
  // 32 KB stages at 128 columns, four 40 KB stages at 192 (384-byte B rows):
  // three or two stages in flight (with three 48 KB stages of 512-byte rows
  // the 192-column tiles waited on their operands)
  if constexpr ((FN == 4 || FN == 6) && EPI == BEPI_STORE) {
    if (d.kg == 2) return go<FN, false, EPI, F32, false, 8, FN == 4 ? 5 : 4, 2>(p, splits, batch, st);
  }
  if constexpr (FN == 8 && EPI == BEPI_STORE) {
    // tile ranges (the X.U split tail): 256 x 256, natural-layout bf16 B, 8 waves
    if (p.tiles > 0) return go<FN, false, EPI, F32, false, 8, 4, 1, true>(p, splits, batch, st);
    // 4-wave instances: natural layout, STORE
    if (d.nw == 4 && !d.b_kc)
      return d.fp8 ? go<FN, false, EPI, F32, true, 4>(p, splits, batch, st)
                   : go<FN, false, EPI, F32, false, 4>(p, splits, batch, st);
  }
  if (d.fp8) return go<FN, false, EPI, F32, true>(p, splits, batch, st);  // fp8 B: natural layout only
  return d.b_kc ? go<FN, true, EPI, F32>(p, splits, batch, st) : go<FN, false, EPI, F32, false, 8, FN == 4 ? 6 : 4>(p, splits, batch, st);
}

// FN 6 (256 x 192 tiles, the rank stages' X.U products) has the store
// epilogues only.
template <int FN>
hipError_t go_e(const BigDesc& d, const BigParams& p, int splits, int batch, hipStream_t st, const char** why) {
  switch (d.epi) {
    case BEPI_STORE:
      if (d.out_f32) return go_b<FN, BEPI_STORE, true>(d, p, splits, batch, st);
      return go_b<FN, BEPI_STORE>(d, p, splits, batch, st);
    case BEPI_SWIGLU_MEM:
      if constexpr (FN != 6) return go_b<FN, BEPI_SWIGLU_MEM>(d, p, splits, batch, st);
      break;
    case BEPI_STORE_FRAG:
      if constexpr (FN != 6) return go_b<FN, BEPI_STORE_FRAG>(d, p, splits, batch, st);
      break;
    case BEPI_GU_DUAL:  // natural-layout B (bf16 or fp8), 8 waves
      if constexpr (FN == 4 || FN == 7 || FN == 8) {
        if (!d.b_kc && d.nw == 8) {
          // 128 x 128 K-group tiles (bf16 B) for 129-256 token rows
          if (d.kg == 2) {
            if constexpr (FN == 4)
              if (!d.fp8) return go<FN, false, BEPI_GU_DUAL, false, false, 8, 5, 2>(p, splits, batch, st);
            break;
          }
          return d.fp8 ? go<FN, false, BEPI_GU_DUAL, false, true>(p, splits, batch, st)
                       : go<FN, false, BEPI_GU_DUAL, false, false, 8, FN == 4 ? 6 : 4>(p, splits, batch, st);
        }
      }
      break;
    case BEPI_DUAL_F32:  // the split passes' fp32 slices; natural-layout B, 8 waves
      if constexpr (FN == 4 || FN == 8) {
        if (!d.b_kc && d.nw == 8 && d.out_f32) {
          // 128 x 128 K-group tiles (bf16 B) for up to 128 token rows
          if (d.kg == 2) {
            if constexpr (FN == 4)
              if (!d.fp8) return go<FN, false, BEPI_DUAL_F32, true, false, 8, 5, 2>(p, splits, batch, st);
            break;
          }
          return d.fp8 ? go<FN, false, BEPI_DUAL_F32, true, true>(p, splits, batch, st)
                       : go<FN, false, BEPI_DUAL_F32, true, false, 8, FN == 4 ? 6 : 4>(p, splits, batch, st);
        }
      }
      break;
    default: break;
  }
  *why = "big GEMM: unsupported epilogue for this tile";
  return hipErrorInvalidValue;
}

// One block per wave tile (16*FM x 16*FN, FM*FN*256 floats contiguous in
// fragment order) of one batch entry: the splits are summed with coalesced
// 16-byte reads, the bf16 tile is staged in LDS and written as whole row
// pieces (16 bytes per lane).  Lane L of fragment (i, j) holds rows
// 16i + L%16, columns 16j + 4*(L/16) .. +3 of the wave tile.
template <int FM, int FN>
__global__ __launch_bounds__(256) void reduce_frag_bf16_kernel(const float* in, int splits, int64_t sstride,
                                                               int64_t bstride, uint16_t* out, int64_t ldo,
                                                               int64_t obstride, int M, int N, int mtiles, int nw,
                                                               const uint16_t* gate, const uint16_t* resid,
                                                               const float* gsl, int gsplits) {
  // tiles of (nw / 2) x 2 wave tiles: 256 rows (8 waves of 64, 4 of 128) or
  // 128 (the K-group tiles' four wave tiles of 64)
  constexpr int ROWS = 16 * FM, COLS = 16 * FN, PITCH = COLS + 8;  // staged row pitch (elements)
  constexpr int Q = FM * FN * 64;                                   // float4s per wave tile
  __shared__ __attribute__((aligned(16))) uint16_t tile[ROWS * PITCH];
  const int zb = blockIdx.y;
  const int unit = blockIdx.x, wave = unit % nw, t_lin = unit / nw;
  const int m0 = (t_lin % mtiles) * ((nw >> 1) * ROWS) + (wave >> 1) * ROWS;
  const int n0 = (t_lin / mtiles) * (2 * COLS) + (wave & 1) * COLS;
  const float* src = in + (int64_t)zb * bstride + (int64_t)unit * Q * 4 + 4 * threadIdx.x;
  static_assert(Q % 256 == 0, "whole rounds");
  constexpr int PER = Q / 256;  // float4s per thread, all loaded per split before any is summed
  f32x4 a[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) a[k] = *reinterpret_cast<const f32x4*>(src + 1024 * k);
  for (int s = 1; s < splits; ++s) {
    f32x4 b[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) b[k] = *reinterpret_cast<const f32x4*>(src + (int64_t)s * sstride + 1024 * k);
#pragma unroll
    for (int k = 0; k < PER; ++k) a[k] += b[k];
  }
  if (gsl) {  // SwiGLU with the gate as fp32 slices: g = bf16(sum in split order), then out = SiLU(g) * sum
    const float* gp = gsl + (int64_t)zb * bstride + (int64_t)unit * Q * 4 + 4 * threadIdx.x;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      f32x4 g = *reinterpret_cast<const f32x4*>(gp + 1024 * k);
      for (int s = 1; s < gsplits; ++s) g += *reinterpret_cast<const f32x4*>(gp + s * sstride + 1024 * k);
      const uint32_t g01 = pack_bf16x2(g.x, g.y), g23 = pack_bf16x2(g.z, g.w);
      a[k].x *= silu_f32(bf16_bits_to_f32(g01 & 0xffffu));
      a[k].y *= silu_f32(bf16_bits_to_f32(g01 >> 16));
      a[k].z *= silu_f32(bf16_bits_to_f32(g23 & 0xffffu));
      a[k].w *= silu_f32(bf16_bits_to_f32(g23 >> 16));
    }
  } else if (gate) {  // SwiGLU: out = SiLU(g) * sum, g bf16 in the same fragment order
    const uint16_t* gp = gate + (int64_t)zb * bstride + (int64_t)unit * Q * 4 + 4 * threadIdx.x;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const u32x2 g = *reinterpret_cast<const u32x2*>(gp + 1024 * k);
      a[k].x *= silu_f32(bf16_bits_to_f32(g.x & 0xffffu));
      a[k].y *= silu_f32(bf16_bits_to_f32(g.x >> 16));
      a[k].z *= silu_f32(bf16_bits_to_f32(g.y & 0xffffu));
      a[k].w *= silu_f32(bf16_bits_to_f32(g.y >> 16));
    }
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int q = threadIdx.x + 256 * k, fi = q >> 6, l = q & 63;
    const int r = 16 * (fi / FN) + (l & 15), c = 16 * (fi % FN) + 4 * (l >> 4);
    *reinterpret_cast<u32x2*>(tile + r * PITCH + c) = u32x2{pack_bf16x2(a[k].x, a[k].y), pack_bf16x2(a[k].z, a[k].w)};
  }
  __syncthreads();
  uint16_t* dst = out + (int64_t)zb * obstride;
  for (int k = threadIdx.x; k < ROWS * (COLS / 8); k += 256) {
    const int r = k / (COLS / 8), c = 8 * (k % (COLS / 8));
    const int m = m0 + r, n = n0 + c;
    if (m < M && n < N) {  // N % 8 == 0
      u32x4 o = *reinterpret_cast<const u32x4*>(tile + r * PITCH + c);
      if (resid) {  // the MLP block's residual add, same layout as out (batch entry 0)
        const u32x4 xr = *reinterpret_cast<const u32x4*>(resid + (int64_t)m * ldo + n);
        o = u32x4{add_bf16x2(xr.x, o.x), add_bf16x2(xr.y, o.y), add_bf16x2(xr.z, o.z), add_bf16x2(xr.w, o.w)};
      }
      *reinterpret_cast<u32x4*>(dst + (int64_t)m * ldo + n) = o;
    }
  }
}

template <int FM, int FN>
hipError_t go_reduce(const float* in, int splits, int64_t sstride, int64_t bstride, uint16_t* out, int64_t ldo,
                     int64_t obstride, int M, int N, int mtiles, int ntiles, int nw, int batch, const uint16_t* gate,
                     const uint16_t* resid, hipStream_t st, const float* gsl, int gsplits) {
  hipLaunchKernelGGL((reduce_frag_bf16_kernel<FM, FN>), dim3(mtiles * ntiles * nw, batch), dim3(256), 0, st, in,
                     splits, sstride, bstride, out, ldo, obstride, M, N, mtiles, nw, gate, resid, gsl, gsplits);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_reduce_frag_bf16(const float* in, int splits, int64_t sstride, int64_t bstride, uint16_t* out,
                                   int64_t ldo, int64_t obstride, int M, int N, int mtiles, int ntiles, int fn, int nw,
                                   int batch, hipStream_t st, const uint16_t* gate, const uint16_t* resid, int kg,
                                   const float* gsl, int gsplits) {
  if (kg == 2) {  // 128-row K-group tiles: four 64-row wave tiles per tile
    if (nw != 8) return hipErrorInvalidValue;
    if (fn == 4) return go_reduce<4, 4>(in, splits, sstride, bstride, out, ldo, obstride, M, N, mtiles, ntiles, 4, batch, gate, resid, st, gsl, gsplits);
    if (fn == 6) return go_reduce<4, 6>(in, splits, sstride, bstride, out, ldo, obstride, M, N, mtiles, ntiles, 4, batch, gate, resid, st, gsl, gsplits);
    return hipErrorInvalidValue;
  }
  if (kg != 1) return hipErrorInvalidValue;
  if (nw == 8 && fn == 8) return go_reduce<4, 8>(in, splits, sstride, bstride, out, ldo, obstride, M, N, mtiles, ntiles, nw, batch, gate, resid, st, gsl, gsplits);
  if (nw == 8 && fn == 7) return go_reduce<4, 7>(in, splits, sstride, bstride, out, ldo, obstride, M, N, mtiles, ntiles, nw, batch, gate, resid, st, gsl, gsplits);
  if (nw == 8 && fn == 6) return go_reduce<4, 6>(in, splits, sstride, bstride, out, ldo, obstride, M, N, mtiles, ntiles, nw, batch, gate, resid, st, gsl, gsplits);
  if (nw == 8 && fn == 4) return go_reduce<4, 4>(in, splits, sstride, bstride, out, ldo, obstride, M, N, mtiles, ntiles, nw, batch, gate, resid, st, gsl, gsplits);
  if (nw == 4 && fn == 4) return go_reduce<8, 4>(in, splits, sstride, bstride, out, ldo, obstride, M, N, mtiles, ntiles, nw, batch, gate, resid, st, gsl, gsplits);
  if (nw == 4 && fn == 8) return go_reduce<8, 8>(in, splits, sstride, bstride, out, ldo, obstride, M, N, mtiles, ntiles, nw, batch, gate, resid, st, gsl, gsplits);
  return hipErrorInvalidValue;
}

hipError_t launch_big(const BigDesc& d, const BigParams& p, int splits, int batch, hipStream_t st,
                      const char** why) {
  if (p.tiles < 0 || (p.tiles > 0 && (p.tile0 < 0 || p.tile0 + p.tiles > p.mtiles * p.ntiles))) {
    *why = "big GEMM: the launch's tiles must lie within the mtiles x ntiles";
    return hipErrorInvalidValue;
  }
  if (p.tiles > 0 && !(d.fn == 8 && d.epi == BEPI_STORE && !d.fp8 && !d.b_kc && d.nw == 8 && d.kg == 1)) {
    *why = "big GEMM: tile ranges take 256 x 256 tiles of natural-layout bf16 B with 8 waves and a store epilogue";
    return hipErrorInvalidValue;
  }
  if (d.kg != 1 && !(d.kg == 2 && !d.fp8 && !d.b_kc && d.nw == 8 &&
                     (((d.fn == 4 || d.fn == 6) && d.epi == BEPI_STORE) ||
                      (d.fn == 4 && (d.epi == BEPI_DUAL_F32 || d.epi == BEPI_GU_DUAL))))) {
    *why = "big GEMM: K groups take natural-layout bf16 B, store (or dual) epilogues and 128 x 128 or 128 x 192 tiles";
    return hipErrorInvalidValue;
  }
  if (d.fn == 8) return go_e<8>(d, p, splits, batch, st, why);
  if (d.fn == 7) return go_e<7>(d, p, splits, batch, st, why);
  if (d.fn == 6) return go_e<6>(d, p, splits, batch, st, why);
  if (d.fn == 4) return go_e<4>(d, p, splits, batch, st, why);
  *why = "big GEMM: no compiled instance for this tile";
  return hipErrorInvalidValue;
}

}  // namespace svdmlp
