// fp8 x fp8 large-tile GEMM on the CDNA4 fp8 MFMA, for the down projection's
// h . Ud stage with fp8 activations:
//
//   C[M x N] = diag(sa) . Aq[M x K] . Bq[K x N] . diag(sb)
//
// Aq: e4m3fn (M, K) row-major with one fp32 scale per row (the activations,
// quantised per token row by quant_rows_e4m3_kernel); Bq: e4m3fn natural
// (K, N) layout with one fp32 scale per column (the factor's per-output-
// channel scale).  v_mfma_scale_f32_16x16x128_f8f6f4 with unit E8M0 block
// scales (127 = 2^0), fp32 accumulation; both scales multiply the fp32
// accumulator in the epilogue.
//
// Block: 8 waves in a 4 (M) x 2 (N) grid of 64 x 64 wave tiles, or 4 waves
// in a 2 x 2 grid of 128 x 64; the block tile is 256 x 128 either way, and
// the fragment order of split-K slices is the large-tile bf16 kernel's at
// fn = 4 with the same wave count, summed by the same reduction.
//
// One k-step is 128 k (one MFMA deep).  LDS holds 3 stages of 48 KB:
//  * A: 256 rows x 128 bytes, 16-byte chunks XOR-swizzled by row & 7; a
//    fragment (16 rows x 128 k, lane l: row l % 16, 32 bytes) is two
//    ds_read_b128, chunks l / 16 and l / 16 + 4;
//  * B: 128 k-rows x 128 bytes (128 columns) as they lie in HBM, chunks
//    XOR-swizzled by f8b_swz(k); a fragment (16 columns x 128 k, lane l:
//    column l % 16, the same 32 k as A) is four ds_read_b64_tr_b8.
// The MFMA contracts the k of its two operands position by position, so
// any k order works as long as A and B share it.  The one used here: byte
// b of lane group g = l / 16 is k = 16 g + b for b < 16 and 64 + 16 g +
// (b - 16) above.  With it each A read takes chunk g (or g + 4) of its row,
// which an LDS probe measured at the rate of a linear read; chunks 2 g and
// 2 g + 1 (k = 32 g + b) took 1.65 times as long.  Operands go global ->
// LDS by direct DMA (buffer_load ... lds), 1 KB instructions (per wave and
// stage: 8 A and 4 B with 4 waves, 4 and 2 with 8); the DMA of stage
// kt + 3 and the fragment reads of stage kt + 1 are interleaved with the
// MFMAs of stage kt, as in the bf16 kernel.
#pragma once

#include "gemm_big.hpp"

namespace svdmlp {

struct F8Params {
  const uint8_t* a;  // (M, K) e4m3fn, row pitch lda bytes
  const uint8_t* b;  // (K, N) e4m3fn, row pitch ldb bytes
  uint32_t a_bytes, b_bytes;
  int64_t lda, ldb;
  const float* sa;   // M row scales
  const float* sb;   // N column scales
  void* out;         // splits == 1: bf16 (M, N), row pitch ldo; else fp32 fragment-order slices
  int64_t ldo;
  int64_t out_sstride;  // floats between split-K slices
  int M, N, K;
  int mtiles, ntiles;
  // this launch's tiles: tile0 .. tile0 + tiles - 1 of the mtiles x ntiles
  // (tile = m-tile + mtiles * n-tile), each in every split
  int tile0, tiles;
  int k_split;  // K per split, a multiple of 128
  // A in 16 x 128 blocks: (m, k) at ((m/16)*(K/128) + k/128)*2048 + (m%16)*128
  // + k%128 (lda unused; a_bytes covers whole 16-row blocks).  A stage's 16
  // rows are then one 2 KB run instead of 16 lines at the row pitch.
  int a_blk;
};

constexpr int kF8Threads = 512;  // the row quantisation's block
constexpr int kF8BM = 256, kF8BN = 128, kF8BK = 128;
constexpr int kF8Stages = 3;
constexpr int kF8ABytes = kF8BM * kF8BK;  // 32 KB
constexpr int kF8BBytes = kF8BK * kF8BN;  // 16 KB
constexpr int kF8Stage = kF8ABytes + kF8BBytes;
static_assert(kF8Stages * kF8Stage <= 160 * 1024, "LDS budget");

// Chunk swizzle of B k-row k (128-byte rows: two per 64-bank row).  A
// transposing read's lanes 0-15 touch rows k0..k0+7 and lanes 16-31 rows
// k0+16..k0+23, served in the same pass: k & 7 places each group's rows on
// 8 distinct 16-byte bank groups (even rows in one half of the banks, odd
// in the other) and k & 16 flips the chunk's low bit, so the second group
// takes the 16 bank groups the first leaves free.
__device__ __forceinline__ int f8b_swz(int k) { return (k & 7) ^ ((k >> 4) & 1); }

// 16 e4m3 x 16 e4m3 over 128 k into a 16x16 fp32 block (unit E8M0 scales).
__device__ __forceinline__ f32x4 mfma_f8(const u32x4 (&b)[2], const u32x4 (&a)[2], f32x4 c) {
  typedef int v8i __attribute__((ext_vector_type(8)));
  const v8i bv = v8i{(int)b[0].x, (int)b[0].y, (int)b[0].z, (int)b[0].w, (int)b[1].x, (int)b[1].y, (int)b[1].z, (int)b[1].w};
  const v8i av = v8i{(int)a[0].x, (int)a[0].y, (int)a[0].z, (int)a[0].w, (int)a[1].x, (int)a[1].y, (int)a[1].z, (int)a[1].w};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bv, av, c, 0, 0, 0, 127, 0, 127);
}

// NW waves in an (NW / 2) x 2 grid: 8 waves of 64 x 64 (two per SIMD) or 4
// of 128 x 64 (one per SIMD, accumulators in AGPRs), which read a quarter
// less from LDS per MFMA.
template <bool SLICES, int NW>
__global__ __launch_bounds__(NW * 64, 1) void f8_gemm_kernel(F8Params p) {
  constexpr int FM = 32 / NW, FN = 4, NS = kF8Stages;
  constexpr int A_UNITS = kF8ABytes / 1024 / NW, B_UNITS = kF8BBytes / 1024 / NW;  // 4, 2
  constexpr int NDMA = A_UNITS + B_UNITS;
  constexpr int B_REGION = NS * kF8ABytes;
  __shared__ __attribute__((aligned(1024))) char lds[NS * kF8Stage];

  const int nblk = gridDim.x * gridDim.y;
  const int vb = xcd_remap(blockIdx.x + gridDim.x * blockIdx.y, nblk);
  const int tile = p.tile0 + vb % p.tiles;
  const int split = vb / p.tiles;
  const int m0 = (tile % p.mtiles) * kF8BM;
  const int n0 = (tile / p.mtiles) * kF8BN;
  const int kbeg = split * p.k_split;
  const int kend = min(p.K, kbeg + p.k_split);
  const int nk = (kend - kbeg + kF8BK - 1) / kF8BK;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;
  const int wm0 = (wave >> 1) * 16 * FM, wn0 = (wave & 1) * 64;

  const i32x4 ra = make_rsrc_sgpr(p.a, p.a_bytes);
  const i32x4 rb = make_rsrc_sgpr(p.b, p.b_bytes);
  const i32x4 r_none = make_rsrc_sgpr(p.a, 0);
  const uint32_t lbase = lds_addr(lds);

  // DMA geometry: instruction i of this wave fills 8 rows (A: m rows, B: k
  // rows) 8 * (wave + NW * i) + lane / 8 of 128 bytes (whole 128-byte
  // lines); lane slot lane % 8 holds logical chunk (lane % 8) ^ (A: row & 7,
  // B: f8b_swz(row)).  Rows or columns outside the matrix take an offset past
  // the records and fetch zeros; the stage's k goes into the scalar offset
  // (stages wholly past kend use r_none).
  uint32_t a_voff[A_UNITS], b_voff[B_UNITS];
#pragma unroll
  for (int i = 0; i < A_UNITS; ++i) {
    const int row = 8 * (wave + NW * i) + (lane >> 3);
    const int lc = (lane & 7) ^ (row & 7);
    const int m = m0 + row;
    const uint32_t base = p.a_blk ? (uint32_t)((m >> 4) * (int64_t)(p.K >> 7) * 2048 + (m & 15) * 128)
                                  : (uint32_t)((int64_t)m * p.lda);
    a_voff[i] = m < p.M ? base + 16u * (uint32_t)lc : kOOB;
  }
#pragma unroll
  for (int i = 0; i < B_UNITS; ++i) {
    const int kr = 8 * (wave + NW * i) + (lane >> 3);
    const int col = 16 * ((lane & 7) ^ f8b_swz(kr));
    b_voff[i] = n0 + col < p.N ? (uint32_t)((int64_t)kr * p.ldb) + (uint32_t)(n0 + col) : kOOB;
  }
  const uint32_t a_kshift = p.a_blk ? 4u : 0u;  // k0 (a multiple of 128) -> its block's offset, k0 / 128 * 2048
  auto dma_one = [&](int kt, int s, int d) {
    const int k0 = kbeg + kt * kF8BK;
    const bool live = k0 < kend;  // uniform
    if (d < A_UNITS)
      dma16(live ? ra : r_none, a_voff[d], (uint32_t)k0 << a_kshift, lbase + s * kF8ABytes + (wave + NW * d) * 1024);
    else
      dma16(live ? rb : r_none, b_voff[d - A_UNITS], (uint32_t)((int64_t)k0 * p.ldb),
            lbase + B_REGION + s * kF8BBytes + (wave + NW * (d - A_UNITS)) * 1024);
  };

  // Fragment addresses within a stage.  A fragment i: row wm0 + 16 i + lr,
  // chunks lg (k 16 lg ..) and lg + 4 (k 64 + 16 lg ..); row & 7 is lr & 7
  // for every i.  B fragment j, read q: lane lr points at k-row 16 lg +
  // 8 (q & 1) + 64 (q >> 1) + lr / 2, byte 8 (lr & 1) of column chunk
  // c = (wn0 + 16 j) / 16, giving the lane bytes 8 q .. 8 q + 7 of its k
  // order.
  const lds_cptr l0 = (lds_cptr)lds;
  const lds_cptr a_rd0 = l0 + (wm0 + lr) * 128 + ((lg ^ (lr & 7)) << 4);
  const lds_cptr a_rd1 = l0 + (wm0 + lr) * 128 + (((lg + 4) ^ (lr & 7)) << 4);
  const int bk = 16 * lg + (lr >> 1);
  lds_cptr b_rd[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int cc = (wn0 >> 4) + j;
    b_rd[j] = l0 + B_REGION + bk * 128 + ((cc ^ f8b_swz(bk)) << 4) + ((lr & 1) << 3);
  }

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  struct Frags {
    u32x4 a[FM][2];
    u32x2 b[FN][4];
  };
  constexpr int NREAD = 2 * FM + 4 * FN;  // 24 (NW 8) or 32 (NW 4)
  // read r of stage slot s: A halves first, then B pieces
  auto read_one = [&](int s, int r, Frags& f) {
    if (r < 2 * FM) {
      const int i = r >> 1;
      f.a[i][r & 1] = lds_read_b128((r & 1 ? a_rd1 : a_rd0) + s * kF8ABytes + 16 * 128 * i);
    } else {
      const int j = (r - 2 * FM) >> 2, q = (r - 2 * FM) & 3;
      // the row offsets 8 and 64 keep k-row & 7 and k-row & 16 (k-row % 16
      // + 8 < 16), so the swizzle is that of q = 0
      f.b[j][q] = lds_read_tr8(b_rd[j] + s * kF8BBytes + 128 * (8 * (q & 1) + 64 * (q >> 1)));
    }
  };
  constexpr int NMFMA = FM * FN;  // 16 or 32
  auto mfma_one = [&](int m, const Frags& f) {
    const int i = m / FN, j = m % FN;
    const u32x4 bb[2] = {u32x4{f.b[j][0].x, f.b[j][0].y, f.b[j][1].x, f.b[j][1].y},
                         u32x4{f.b[j][2].x, f.b[j][2].y, f.b[j][3].x, f.b[j][3].y}};
    acc[i][j] = mfma_f8(bb, f.a[i], acc[i][j]);
  };

  // Step kt: the MFMAs of stage kt (fragments read in step kt - 1), with the
  // fragment reads of stage kt + 1 (two per MFMA slot) and the DMAs of stage
  // kt + NS into slot kt % NS (free: every wave read stage kt before the
  // barrier that ended step kt - 1) interleaved; then wait until stage
  // kt + 2 landed (stage kt + NS may still fly) and meet at the barrier.
  Frags f0, f1;
  // reads per MFMA slot: 2 with 8 waves (24 reads, 16 MFMAs), 1 with 4
  constexpr int RPS = (NREAD + NMFMA - 1) / NMFMA;
  static_assert(NDMA + 2 <= NMFMA, "interleave slots");
  auto step = [&](int kt, int s, const Frags& cur, Frags& nxt) {
#pragma unroll
    for (int m = 0; m < NMFMA; ++m) {
#pragma unroll
      for (int q = 0; q < RPS; ++q)
        if (RPS * m + q < NREAD) read_one((s + 1) % NS, RPS * m + q, nxt);
      if (m >= 2 && m - 2 < NDMA) dma_one(kt + NS, s, m - 2);
      mfma_one(m, cur);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_dma<(NS - 2) * NDMA>();
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };

  if (nk > 0) {
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int d = 0; d < NDMA; ++d) dma_one(s, s, d);
    wait_dma<(NS - 1) * NDMA>();  // stage 0 landed
    __syncthreads();
#pragma unroll
    for (int r = 0; r < NREAD; ++r) read_one(0, r, f0);
    wait_dma<(NS - 2) * NDMA>();  // stage 1 landed: step 0 reads it
    __syncthreads();  // ... and every wave holds stage 0 before step 0 refills its slot
    __builtin_amdgcn_sched_barrier(0);
  }
  constexpr int UNROLL = 2 * NS;  // slot cycle x f0/f1 alternation
  for (int kt = 0; kt < nk; kt += UNROLL) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (kt + u < nk) {
        if (u % 2 == 0)
          step(kt + u, u % NS, f0, f1);
        else
          step(kt + u, u % NS, f1, f0);
      }
    }
  }
  wait_dma<0>();  // drain DMAs of stages past the end before the block exits

  // ---- epilogue: lane holds D[n = 4 lg + t][m = lr] of each 16x16 block ----
  const int64_t frag0 =
      ((((int64_t)(m0 / kF8BM) + (int64_t)p.mtiles * (n0 / kF8BN)) * NW + wave) * FM * FN) * 256 + 4 * lane;
  float* slice = reinterpret_cast<float*>(p.out) + (int64_t)split * p.out_sstride;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = m0 + wm0 + 16 * i + lr;
    const float sa = m < p.M ? p.sa[m] : 0.f;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn0 + 16 * j + 4 * lg;
      f32x4 v = acc[i][j];
      if (n < p.N) v *= sa * *reinterpret_cast<const f32x4*>(p.sb + n);
      if constexpr (SLICES) {
        // whole tiles in fragment order (padded rows / columns hold zeros)
        *reinterpret_cast<f32x4*>(slice + frag0 + (int64_t)(i * FN + j) * 256) = n < p.N ? v : f32x4{0.f, 0.f, 0.f, 0.f};
      } else if (m < p.M && n < p.N) {
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.out) + (int64_t)m * p.ldo + n) =
            u32x2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
      }
    }
  }
}

// Pieces of 8 elements per thread of the e4m3 row quantisation (gemm_f8f8.hip):
// rows of at most 8 * kF8Threads * kF8QPieces elements.
constexpr int kF8QPieces = 8;

}  // namespace svdmlp
