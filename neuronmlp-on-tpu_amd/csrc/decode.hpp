// Decode-shape (T <= 64 tokens) projections: memory-bound weight streaming.
//
//   OUT[T x N] += A[T x K] . W[K x N]      (fp32 accumulation target)
//
// At decode shapes the factors (311 MB per LLaMA3-8B layer in bf16) dominate
// every byte moved, so the kernel is built to keep HBM busy:
//  * No LDS staging for W.  Each lane streams 16-byte rows of W straight into
//    registers: lane (lr = lane % 16, lg = lane / 16) reads, for one k-step of
//    32, the rows k + 8*lg + 0..7 at columns n0 + 8*lr .. +7 (natural (in, out)
//    layout), i.e. 16 lanes cover 256 contiguous bytes of a row.  The 8x8
//    bf16 block is transposed in registers into eight MFMA B fragments; MFMA
//    column label lr of fragment j is the real column n0 + 8*lr + j.
//  * Weights stored (out, in) (PyTorch Linear) need no transpose: fragment j
//    covers column n0 + 16*j + lr.
//  * A (the T activation rows, zero-padded to 16) is tiny and L2-resident; it
//    may be bf16, an fp32 partial-sum workspace, or the fp32 gate/up pair
//    (then h = bf16(silu(g) * u) is formed on load, so h never hits HBM).
//  * Split-K: the 4 waves of a block take interleaved k-steps of one K slice,
//    reduce through LDS float atomics, then one coalesced pass of fp32
//    global atomics adds the block's partial sums into OUT.
//  * Each wave issues all loads of U k-steps before its first MFMA, so every
//    wave keeps 8*U 1 KB requests in flight.
#pragma once

#include "gemm.hpp"

namespace svdmlp {

struct DecodeSeg {
  const void* w;       // weight base
  const float* scale;  // per output column scale (fp8) or null
  float* out;          // fp32 accumulation target
  int64_t ldw;         // weight leading dimension (elements)
  int64_t ldo;         // output leading dimension (elements)
  int N;               // columns in this segment
  int ntiles;          // ceil(N / 128)
};

struct DecodeParams {
  Operand a[2];  // A operand per segment
  DecodeSeg seg[2];
  int nseg;
  int T, K;
  int k_split;  // K elements per block (multiple of 32)
};

constexpr int kDecTileN = 128;

template <int SRCA, bool VEC>
__device__ __forceinline__ u32x4 dec_load_a(const Operand& op, int m, int T, int k, int kend) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (m < T) {
    const int64_t off = (int64_t)m * op.ld + k;
    if constexpr (VEC) {
      if (k < kend) v = load8_as_bf16<SRCA>(op, off);
    } else {
      float e[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) e[t] = (k + t < kend) ? load_elem_f32<SRCA>(op, off + t) : 0.0f;
      v = u32x4{pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3]), pack_bf16x2(e[4], e[5]),
                pack_bf16x2(e[6], e[7])};
    }
  }
  return v;
}

// One k-step worth of B data for this lane: 8 fragments (u32x4 each).
template <int SRCB, bool VEC, bool B_KCONTIG>
__device__ __forceinline__ void dec_load_b(const DecodeSeg& s, int n0, int k, int kend, int lr, int lg,
                                           u32x4 raw[8]) {
  Operand op{s.w, nullptr, s.ldw};
  if constexpr (!B_KCONTIG) {
    const int n = n0 + 8 * lr;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int kk = k + 8 * lg + jj;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (kk < kend && n < s.N) {
        const int64_t off = (int64_t)kk * s.ldw + n;
        if constexpr (VEC) {
          v = load8_as_bf16<SRCB>(op, off);
        } else {
          float e[8];
#pragma unroll
          for (int t = 0; t < 8; ++t) e[t] = (n + t < s.N) ? load_elem_f32<SRCB>(op, off + t) : 0.0f;
          v = u32x4{pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3]), pack_bf16x2(e[4], e[5]),
                    pack_bf16x2(e[6], e[7])};
        }
      }
      raw[jj] = v;
    }
  } else {
    const int kk = k + 8 * lg;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int n = n0 + 16 * j + lr;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (n < s.N && kk < kend) {
        const int64_t off = (int64_t)n * s.ldw + kk;
        if constexpr (VEC) {
          v = load8_as_bf16<SRCB>(op, off);
        } else {
          float e[8];
#pragma unroll
          for (int t = 0; t < 8; ++t) e[t] = (kk + t < kend) ? load_elem_f32<SRCB>(op, off + t) : 0.0f;
          v = u32x4{pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3]), pack_bf16x2(e[4], e[5]),
                    pack_bf16x2(e[6], e[7])};
        }
      }
      raw[j] = v;
    }
  }
}

// raw[jj] = row (k + 8*lg + jj), 8 columns packed in pairs.  Fragment j wants
// column j, rows 0..7 packed in pairs: dword p = (row 2p, row 2p+1).
__device__ __forceinline__ u32x4 dec_transpose(const u32x4 raw[8], int j) {
  const int p = j >> 1;
  u32x4 r;
  if (j & 1) {
    r.x = (raw[0][p] >> 16) | (raw[1][p] & 0xffff0000u);
    r.y = (raw[2][p] >> 16) | (raw[3][p] & 0xffff0000u);
    r.z = (raw[4][p] >> 16) | (raw[5][p] & 0xffff0000u);
    r.w = (raw[6][p] >> 16) | (raw[7][p] & 0xffff0000u);
  } else {
    r.x = (raw[0][p] & 0xffffu) | (raw[1][p] << 16);
    r.y = (raw[2][p] & 0xffffu) | (raw[3][p] << 16);
    r.z = (raw[4][p] & 0xffffu) | (raw[5][p] << 16);
    r.w = (raw[6][p] & 0xffffu) | (raw[7][p] << 16);
  }
  return r;
}

template <int MT, int U, int SRCA, int SRCB, bool VEC, bool B_KCONTIG>
__global__ __launch_bounds__(256) void decode_kernel(DecodeParams p) {
  __shared__ float red[16 * MT * kDecTileN];

  const int tiles = p.seg[0].ntiles + (p.nseg > 1 ? p.seg[1].ntiles : 0);
  const int split = blockIdx.x / tiles;
  int tile = blockIdx.x % tiles;
  int si = 0;
  if (tile >= p.seg[0].ntiles) {
    tile -= p.seg[0].ntiles;
    si = 1;
  }
  const DecodeSeg& s = p.seg[si];
  const Operand& a = p.a[si];
  const int n0 = tile * kDecTileN;
  const int kbeg = split * p.k_split;
  const int kend = min(p.K, kbeg + p.k_split);

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lr = lane & 15, lg = lane >> 4;

  for (int i = threadIdx.x; i < 16 * MT * kDecTileN; i += 256) red[i] = 0.0f;

  f32x4 acc[MT][8];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nsteps = (kend - kbeg + 31) / 32;
  for (int st0 = wave; st0 < nsteps; st0 += 4 * U) {
    u32x4 raw[U][8];
    u32x4 fa[U][MT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = st0 + 4 * u;
      const int k = kbeg + 32 * st;
      if (st < nsteps) {
        dec_load_b<SRCB, VEC, B_KCONTIG>(s, n0, k, kend, lr, lg, raw[u]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) fa[u][mt] = dec_load_a<SRCA, VEC>(a, 16 * mt + lr, p.T, k + 8 * lg, kend);
      } else {
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) raw[u][jj] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) fa[u][mt] = u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const u32x4 fb = B_KCONTIG ? raw[u][j] : dec_transpose(raw[u], j);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][j] = mfma_chunk(fa[u][mt], fb, acc[mt][j], __bf16{});
      }
    }
  }

  __syncthreads();  // red[] zeroed by all threads
  // D[m = 4*lg + t][label = lr]; label lr of fragment j is column
  // 8*lr + j (natural layout) or 16*j + lr (Linear layout).
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int nl = B_KCONTIG ? 16 * j + lr : 8 * lr + j;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int m = 16 * mt + 4 * lg + t;
        if (m < p.T) atomicAdd(&red[m * kDecTileN + nl], acc[mt][j][t]);
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < p.T * kDecTileN; i += 256) {
    const int m = i / kDecTileN, nl = i % kDecTileN;
    const int n = n0 + nl;
    if (n < s.N) {
      float v = red[i];
      if (s.scale) v *= s.scale[n];
      unsafeAtomicAdd(s.out + (int64_t)m * s.ldo + n, v);
    }
  }
}

// ---------------------------------------------------------------------------
// Small elementwise kernels
// ---------------------------------------------------------------------------

// out[m][n] = bf16(in[m][n])  or  bf16(silu(g[m][n]) * u[m][n]); optionally
// written transposed (out[n][m]).
template <bool SWIGLU, bool OUT_T>
__global__ void finalize_bf16_kernel(const float* g, const float* u, int64_t ldi, uint16_t* out, int64_t ldo,
                                     int rows, int cols) {
  const int64_t total = (int64_t)rows * cols;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int r = (int)(i / cols), c = (int)(i % cols);
    const int64_t off = (int64_t)r * ldi + c;
    const float v = SWIGLU ? silu_f32(g[off]) * u[off] : g[off];
    if (OUT_T) {
      out[(int64_t)c * ldo + r] = (uint16_t)f32_to_bf16_bits(v);
    } else {
      out[(int64_t)r * ldo + c] = (uint16_t)f32_to_bf16_bits(v);
    }
  }
}

}  // namespace svdmlp
