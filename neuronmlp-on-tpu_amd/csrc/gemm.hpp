// Tiled MFMA GEMM for the prefill (compute-bound) shapes of the SVD-MLP path.
//
//   C[M x N] = A[M x K] . B[K x N]       (one or two independent branches)
//
// Design (gfx950):
//  * 256 threads = 4 waves of 64; each wave owns a (BM/WM) x (BN/WN) sub-tile
//    built from 16x16 MFMA blocks (v_mfma_f32_16x16x32_bf16, fp32 accumulate).
//  * Both operands live in LDS "K-contiguous": one 128-byte row per M (or N)
//    index holding 8 16-byte chunks of K, XOR-swizzled by row so that the
//    MFMA fragment reads (16 rows x 1 chunk) and the loader writes are free of
//    bank conflicts.  A fragment is one ds_read_b128.
//  * Operands stored row-major with K contiguous (activations, PyTorch-Linear
//    weights) are copied chunk by chunk.  Operands stored with N contiguous
//    (the reference's natural (in, out) weights) are loaded as 4(k) x 8(n)
//    blocks with 16-byte global loads and transposed in registers before the
//    LDS write; no extra HBM pass, no host-side transpose.
//  * The A operand may be an fp32 workspace (split-K partial sums) or a pair
//    of fp32 gate/up sums; it is rounded to bf16 on the way into LDS, which is
//    exactly the rounding the reference applies at each GEMM boundary.
//  * Two LDS stages: global loads for tile k+1 are in flight while tile k is
//    multiplied; one barrier per K tile.
//  * Epilogues: bf16 store, fp32 store, fp32 atomic add (split-K), and the
//    dual-branch SiLU(g) * u epilogue that never writes g or u to HBM.
//  * Tiles are numbered N-major and remapped so that tiles sharing a B panel
//    run on the same XCD (own L2).
#pragma once

#include <type_traits>

#include "common.hpp"

namespace svdmlp {

enum SrcKind : int { SRC_BF16 = 0, SRC_F32 = 1, SRC_FP8 = 2, SRC_SWIGLU = 3 };
// EPI_STORE: plain store (bf16 or fp32 by OUT_F32); EPI_ATOMIC: fp32 atomic
// add of a split-K partial; EPI_SWIGLU: out = silu(g) * u over two branches.
enum EpiKind : int { EPI_STORE = 0, EPI_ATOMIC = 2, EPI_SWIGLU = 3 };

struct Operand {
  const void* p;   // element (row, k) or (k, row) base pointer
  const void* p2;  // SRC_SWIGLU: the "up" half (same layout as p)
  int64_t ld;      // leading dimension in elements
};

struct GemmParams {
  Operand a[2];
  Operand b[2];
  const float* scale[2];  // per output column scale (fp8 weights) or null
  void* out;
  int64_t ldo;
  int64_t out_bstride;  // elements between the outputs of batch entries (blockIdx.z)
  int M, N, K;
  int mtiles, ntiles;
  int k_split;  // K elements per split (multiple of the K tile)
};

template <typename TM> struct MfmaTraits;
template <> struct MfmaTraits<__bf16> { static constexpr int kChunk = 8; };
template <> struct MfmaTraits<float> { static constexpr int kChunk = 4; };

__device__ __forceinline__ int lds_swz(int row) { return (row ^ (row >> 3)) & 7; }

__device__ __forceinline__ u32x4 lds_read_chunk(const char* base, int row, int chunk) {
  return *reinterpret_cast<const u32x4*>(base + row * 128 + ((chunk ^ lds_swz(row)) << 4));
}

// ---------------------------------------------------------------------------
// Element loads with conversion to the MFMA type (bounds already checked).
// ---------------------------------------------------------------------------

template <int SRC>
__device__ __forceinline__ float load_elem_f32(const Operand& op, int64_t off) {
  if constexpr (SRC == SRC_BF16) {
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(op.p)[off]);
  } else if constexpr (SRC == SRC_F32) {
    return reinterpret_cast<const float*>(op.p)[off];
  } else if constexpr (SRC == SRC_FP8) {
    return e4m3_to_f32(reinterpret_cast<const uint8_t*>(op.p)[off]);
  } else {
    const float g = reinterpret_cast<const float*>(op.p)[off];
    const float u = reinterpret_cast<const float*>(op.p2)[off];
    return silu_f32(g) * u;
  }
}

// Eight consecutive elements starting at `off` (16B-aligned in VEC mode),
// returned as four packed bf16 pairs.
template <int SRC>
__device__ __forceinline__ u32x4 load8_as_bf16(const Operand& op, int64_t off) {
  if constexpr (SRC == SRC_BF16) {
    return ldg128(reinterpret_cast<const uint16_t*>(op.p) + off);
  } else if constexpr (SRC == SRC_F32) {
    const float* f = reinterpret_cast<const float*>(op.p) + off;
    const f32x4 lo = *reinterpret_cast<const f32x4*>(f);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(f + 4);
    return u32x4{pack_bf16x2(lo.x, lo.y), pack_bf16x2(lo.z, lo.w),
                 pack_bf16x2(hi.x, hi.y), pack_bf16x2(hi.z, hi.w)};
  } else if constexpr (SRC == SRC_FP8) {
    const u32x2 w = ldg64(reinterpret_cast<const uint8_t*>(op.p) + off);
    u32x4 r;
    // e4m3 values are exact in bf16: take the top half of the fp32 value.
    r.x = (__float_as_uint(e4m3_to_f32(w.x & 0xff)) >> 16) |
          (__float_as_uint(e4m3_to_f32((w.x >> 8) & 0xff)) & 0xffff0000u);
    r.y = (__float_as_uint(e4m3_to_f32((w.x >> 16) & 0xff)) >> 16) |
          (__float_as_uint(e4m3_to_f32(w.x >> 24)) & 0xffff0000u);
    r.z = (__float_as_uint(e4m3_to_f32(w.y & 0xff)) >> 16) |
          (__float_as_uint(e4m3_to_f32((w.y >> 8) & 0xff)) & 0xffff0000u);
    r.w = (__float_as_uint(e4m3_to_f32((w.y >> 16) & 0xff)) >> 16) |
          (__float_as_uint(e4m3_to_f32(w.y >> 24)) & 0xffff0000u);
    return r;
  } else {
    const float* g = reinterpret_cast<const float*>(op.p) + off;
    const float* u = reinterpret_cast<const float*>(op.p2) + off;
    const f32x4 g0 = *reinterpret_cast<const f32x4*>(g), g1 = *reinterpret_cast<const f32x4*>(g + 4);
    const f32x4 u0 = *reinterpret_cast<const f32x4*>(u), u1 = *reinterpret_cast<const f32x4*>(u + 4);
    return u32x4{pack_bf16x2(silu_f32(g0.x) * u0.x, silu_f32(g0.y) * u0.y),
                 pack_bf16x2(silu_f32(g0.z) * u0.z, silu_f32(g0.w) * u0.w),
                 pack_bf16x2(silu_f32(g1.x) * u1.x, silu_f32(g1.y) * u1.y),
                 pack_bf16x2(silu_f32(g1.z) * u1.z, silu_f32(g1.w) * u1.w)};
  }
}

// ---------------------------------------------------------------------------
// Loader for operands stored with K contiguous: element (row, k) at
// p[row * ld + k].  The tile is R rows x 8 chunks.
// ---------------------------------------------------------------------------
template <int R, typename TM, int SRC, bool VEC>
struct RowLoader {
  static constexpr int kC = MfmaTraits<TM>::kChunk;
  static constexpr int kChunks = R * 8;
  static constexpr int kPer = (kChunks + 255) / 256;
  u32x4 r[kPer];

  __device__ __forceinline__ void load(const Operand& op, int row0, int nrows, int k0, int kend) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = threadIdx.x + 256 * i;
      const int row = idx >> 3, c = idx & 7;
      u32x4 v = {0u, 0u, 0u, 0u};
      const int grow = row0 + row;
      const int k = k0 + c * kC;
      if (idx < kChunks && grow < nrows) {
        const int64_t off = (int64_t)grow * op.ld + k;
        if constexpr (VEC) {
          if (k < kend) {
            if constexpr (sizeof(TM) == 2) {
              v = load8_as_bf16<SRC>(op, off);
            } else {
              v = ldg128(reinterpret_cast<const float*>(op.p) + off);
            }
          }
        } else {
          if constexpr (sizeof(TM) == 2) {
            float e[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) e[t] = (k + t < kend) ? load_elem_f32<SRC>(op, off + t) : 0.0f;
            v = u32x4{pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3]),
                      pack_bf16x2(e[4], e[5]), pack_bf16x2(e[6], e[7])};
          } else {
            float e[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) e[t] = (k + t < kend) ? load_elem_f32<SRC>(op, off + t) : 0.0f;
            v = u32x4{__float_as_uint(e[0]), __float_as_uint(e[1]), __float_as_uint(e[2]),
                      __float_as_uint(e[3])};
          }
        }
      }
      r[i] = v;
    }
  }

  __device__ __forceinline__ void store(char* lds) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = threadIdx.x + 256 * i;
      if (idx < kChunks) {
        const int row = idx >> 3, c = idx & 7;
        *reinterpret_cast<u32x4*>(lds + row * 128 + ((c ^ lds_swz(row)) << 4)) = r[i];
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Loader for operands stored with the tile's row index contiguous: element
// (row, k) at p[k * ld + row].  bf16 MFMA: blocks of 4(k) x 8(rows); fp32
// MFMA: blocks of 4(k) x 4(rows).  Each block is loaded with one 16-byte (or
// 8-byte for fp8) global load per k and transposed in registers.
// ---------------------------------------------------------------------------
template <int R, typename TM, int SRC, bool VEC>
struct ColLoader;

template <int R, int SRC, bool VEC>
struct ColLoader<R, __bf16, SRC, VEC> {
  static constexpr int kGroups = R / 8;
  static constexpr int kBlocks = kGroups * 16;  // 16 groups of 4 k = 64 k
  static constexpr int kPer = (kBlocks + 255) / 256;
  u32x4 in[kPer][4];  // [block][k row] = 8 bf16 along rows, packed in pairs

  __device__ __forceinline__ void load(const Operand& op, int row0, int nrows, int k0, int kend) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = threadIdx.x + 256 * i;
      const int g = idx % kGroups, q = idx / kGroups;
      const int grow = row0 + 8 * g;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = k0 + 4 * q + j;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (idx < kBlocks && k < kend && grow < nrows) {
          const int64_t off = (int64_t)k * op.ld + grow;
          if constexpr (VEC) {
            v = load8_as_bf16<SRC>(op, off);
          } else {
            float e[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) e[t] = (grow + t < nrows) ? load_elem_f32<SRC>(op, off + t) : 0.0f;
            v = u32x4{pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3]),
                      pack_bf16x2(e[4], e[5]), pack_bf16x2(e[6], e[7])};
          }
        }
        in[i][j] = v;
      }
    }
  }

  __device__ __forceinline__ void store(char* lds) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = threadIdx.x + 256 * i;
      if (idx >= kBlocks) continue;
      const int g = idx % kGroups, q = idx / kGroups;
      const int chunk = q >> 1, half = q & 1;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int p = t >> 1;
        uint32_t d0, d1;
        if (t & 1) {
          d0 = (in[i][0][p] >> 16) | (in[i][1][p] & 0xffff0000u);
          d1 = (in[i][2][p] >> 16) | (in[i][3][p] & 0xffff0000u);
        } else {
          d0 = (in[i][0][p] & 0xffffu) | (in[i][1][p] << 16);
          d1 = (in[i][2][p] & 0xffffu) | (in[i][3][p] << 16);
        }
        const int row = 8 * g + t;
        *reinterpret_cast<u32x2*>(lds + row * 128 + ((chunk ^ lds_swz(row)) << 4) + half * 8) =
            u32x2{d0, d1};
      }
    }
  }
};

template <int R, int SRC, bool VEC>
struct ColLoader<R, float, SRC, VEC> {
  static_assert(SRC == SRC_F32, "fp32 MFMA path takes fp32 operands");
  static constexpr int kGroups = R / 4;
  static constexpr int kBlocks = kGroups * 8;  // 8 groups of 4 k = 32 k
  static constexpr int kPer = (kBlocks + 255) / 256;
  u32x4 in[kPer][4];

  __device__ __forceinline__ void load(const Operand& op, int row0, int nrows, int k0, int kend) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = threadIdx.x + 256 * i;
      const int g = idx % kGroups, q = idx / kGroups;
      const int grow = row0 + 4 * g;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = k0 + 4 * q + j;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (idx < kBlocks && k < kend && grow < nrows) {
          const int64_t off = (int64_t)k * op.ld + grow;
          const float* f = reinterpret_cast<const float*>(op.p) + off;
          if constexpr (VEC) {
            v = ldg128(f);
          } else {
            float e[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) e[t] = (grow + t < nrows) ? f[t] : 0.0f;
            v = u32x4{__float_as_uint(e[0]), __float_as_uint(e[1]), __float_as_uint(e[2]),
                      __float_as_uint(e[3])};
          }
        }
        in[i][j] = v;
      }
    }
  }

  __device__ __forceinline__ void store(char* lds) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int idx = threadIdx.x + 256 * i;
      if (idx >= kBlocks) continue;
      const int g = idx % kGroups, q = idx / kGroups;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = 4 * g + t;
        *reinterpret_cast<u32x4*>(lds + row * 128 + ((q ^ lds_swz(row)) << 4)) =
            u32x4{in[i][0][t], in[i][1][t], in[i][2][t], in[i][3][t]};
      }
    }
  }
};

template <int R, typename TM, int SRC, bool VEC, bool KCONTIG>
using Loader = typename std::conditional<KCONTIG, RowLoader<R, TM, SRC, VEC>, ColLoader<R, TM, SRC, VEC>>::type;

// ---------------------------------------------------------------------------
// Kernel configuration
// ---------------------------------------------------------------------------
template <int BM_, int BN_, int WM_, int WN_, typename TM_, int SRCA_, int SRCB_, bool A_KCONTIG_,
          bool B_KCONTIG_, int NBR_, int EPI_, bool OUT_T_, bool OUT_F32_, bool VEC_>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  using TM = TM_;
  static constexpr int SRCA = SRCA_, SRCB = SRCB_;
  static constexpr bool A_KCONTIG = A_KCONTIG_, B_KCONTIG = B_KCONTIG_;
  static constexpr int NBR = NBR_, EPI = EPI_;
  static constexpr bool OUT_T = OUT_T_, OUT_F32 = OUT_F32_, VEC = VEC_;
  static constexpr int BK = 8 * MfmaTraits<TM>::kChunk;
  static constexpr int FM = BM / WM / 16, FN = BN / WN / 16;
  static constexpr int kStageBytes = NBR * (BM + BN) * 128;
  static_assert(WM * WN == 4, "4 waves per block");
  static_assert(FM >= 1 && FN >= 1, "wave tile must hold at least one 16x16 block");
  static_assert(2 * kStageBytes <= 160 * 1024, "LDS budget");
  static_assert(!(OUT_T && EPI == EPI_ATOMIC), "split-K partials are row-major");
  static_assert(EPI != EPI_SWIGLU || NBR == 2, "SiLU(g) * u needs both branches");
};

template <class C>
__device__ __forceinline__ void store_out4(const GemmParams& p, void* outp, int m, int n, const float v[4]) {
  // Four consecutive outputs along N (row-major output) or along M (transposed).
  if constexpr (C::EPI == EPI_ATOMIC) {
    float* o = reinterpret_cast<float*>(outp);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (m < p.M && n + t < p.N) unsafeAtomicAdd(o + (int64_t)m * p.ldo + n + t, v[t]);
    return;
  }
  const int r = C::OUT_T ? n : m;   // output row
  const int c0 = C::OUT_T ? m : n;  // first output column
  const int rows = C::OUT_T ? p.N : p.M;
  const int cols = C::OUT_T ? p.M : p.N;
  if (r >= rows) return;
  if constexpr (C::OUT_F32) {
    float* o = reinterpret_cast<float*>(outp) + (int64_t)r * p.ldo + c0;
    if (C::VEC && c0 + 3 < cols) {
      *reinterpret_cast<f32x4*>(o) = f32x4{v[0], v[1], v[2], v[3]};
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (c0 + t < cols) o[t] = v[t];
    }
  } else {
    uint16_t* o = reinterpret_cast<uint16_t*>(outp) + (int64_t)r * p.ldo + c0;
    if (C::VEC && c0 + 3 < cols) {
      *reinterpret_cast<u32x2*>(o) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (c0 + t < cols) o[t] = (uint16_t)f32_to_bf16_bits(v[t]);
    }
  }
}

template <class C>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
  using TM = typename C::TM;
  constexpr int BM = C::BM, BN = C::BN, BK = C::BK, FM = C::FM, FN = C::FN, NBR = C::NBR;
  constexpr bool SWAP = !C::OUT_T;  // put B in the MFMA "A" slot -> lane holds 4 consecutive n

  __shared__ __attribute__((aligned(16))) char lds[2 * C::kStageBytes];

  const int ntile_total = p.mtiles * p.ntiles;
  const int tile = xcd_remap(blockIdx.x, ntile_total);
  const int m0 = (tile % p.mtiles) * BM;
  const int n0 = (tile / p.mtiles) * BN;
  // NBR == 1 launches may carry two independent problems in blockIdx.z
  // (gate and up share X but not U).
  const int zb = (NBR == 1) ? (int)blockIdx.z : 0;
  const int kbeg = blockIdx.y * p.k_split;
  const int kend = min(p.K, kbeg + p.k_split);
  const int nk = (kend - kbeg + BK - 1) / BK;

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lr = lane & 15, lg = lane >> 4;
  const int wm0 = (wave / C::WN) * (BM / C::WM);
  const int wn0 = (wave % C::WN) * (BN / C::WN);

  Loader<BM, TM, C::SRCA, C::VEC, C::A_KCONTIG> la[NBR];
  Loader<BN, TM, C::SRCB, C::VEC, C::B_KCONTIG> lb[NBR];

  f32x4 acc[NBR][FM][FN];
#pragma unroll
  for (int b = 0; b < NBR; ++b)
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[b][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto stage_ptr = [&](int s, int b) { return lds + s * C::kStageBytes + b * (BM + BN) * 128; };

  if (nk > 0) {
#pragma unroll
    for (int b = 0; b < NBR; ++b) {
      la[b].load(p.a[zb + b], m0, p.M, kbeg, kend);
      lb[b].load(p.b[zb + b], n0, p.N, kbeg, kend);
    }
#pragma unroll
    for (int b = 0; b < NBR; ++b) {
      la[b].store(stage_ptr(0, b));
      lb[b].store(stage_ptr(0, b) + BM * 128);
    }
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      const int k0 = kbeg + (kt + 1) * BK;
#pragma unroll
      for (int b = 0; b < NBR; ++b) {
        la[b].load(p.a[zb + b], m0, p.M, k0, kend);
        lb[b].load(p.b[zb + b], n0, p.N, k0, kend);
      }
    }
#pragma unroll
    for (int b = 0; b < NBR; ++b) {
      const char* sa = stage_ptr(cur, b);
      const char* sb = sa + BM * 128;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        u32x4 fa[FM], fb[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[i] = lds_read_chunk(sa, wm0 + 16 * i + lr, 4 * s + lg);
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[j] = lds_read_chunk(sb, wn0 + 16 * j + lr, 4 * s + lg);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[b][i][j] = SWAP ? mfma_chunk(fb[j], fa[i], acc[b][i][j], TM{})
                                : mfma_chunk(fa[i], fb[j], acc[b][i][j], TM{});
      }
    }
    if (more) {
#pragma unroll
      for (int b = 0; b < NBR; ++b) {
        la[b].store(stage_ptr(cur ^ 1, b));
        lb[b].store(stage_ptr(cur ^ 1, b) + BM * 128);
      }
    }
    __syncthreads();
  }

  // Epilogue.  SWAP: lane holds D[n = 4*lg + t][m = lr] of each 16x16 block.
  // !SWAP: lane holds D[m = 4*lg + t][n = lr].
  const float* sc0 = p.scale[zb];
  const float* sc1 = p.scale[1];
  char* outp = reinterpret_cast<char*>(p.out) +
               (int64_t)zb * p.out_bstride * ((C::OUT_F32 || C::EPI == EPI_ATOMIC) ? 4 : 2);
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      int m, n;
      if (SWAP) {
        m = m0 + wm0 + 16 * i + lr;
        n = n0 + wn0 + 16 * j + 4 * lg;
      } else {
        m = m0 + wm0 + 16 * i + 4 * lg;
        n = n0 + wn0 + 16 * j + lr;
      }
      float v[4];
      if constexpr (C::EPI == EPI_SWIGLU) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int nn = SWAP ? n + t : n;
          float g = acc[0][i][j][t], u = acc[1][i][j][t];
          if (sc0 && nn < p.N) g *= sc0[nn];
          if (sc1 && nn < p.N) u *= sc1[nn];
          v[t] = silu_f32(g) * u;
        }
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int nn = SWAP ? n + t : n;
          float x = acc[0][i][j][t];
          if (sc0 && nn < p.N) x *= sc0[nn];
          v[t] = x;
        }
      }
      store_out4<C>(p, outp, m, n, v);
    }
  }
}

}  // namespace svdmlp
