// The SVD-MLP layer at 1 or 2 tokens as four weight-streaming GEMV phases in
// one persistent launch.
//
// At T <= 2 every factor element is used at most twice, so the layer is
// a pure stream of the 311 MB of bf16 factors (LLaMA3-8B, r = 2816) and the
// arithmetic is a few VALU FMAs per element.  The design keeps HBM busy:
//  * one block of 8 waves per CU (grid = CU count);
//  * weights go straight from HBM into registers: a wave's load covers RW
//    rows x (512 / RW) columns of a natural-layout (K x N) factor, i.e. rows
//    of 512 or 1024 contiguous bytes, and every lane keeps kGvDepth 16-byte
//    loads in flight (128 KB per CU);
//  * a phase's work is the list of "groups" (8 * RW consecutive rows of one
//    column strip of one matrix) in (matrix, strip, row) order, and block b
//    takes the contiguous range [b * groups / G, (b + 1) * groups / G)
//    (stream-K); a range covers few strips, and at the end of each the
//    block's partial column sums are reduced through LDS and added with fp32
//    atomics;
//  * phases: 0 zero the fp32 sums; 1 XU_g, XU_u += X . [Ug | Uu];
//    2 G, U += XU_g . Vg, XU_u . Vu; 3 XU_d += bf16(SiLU(G) * U) . Ud;
//    4 Y32 += XU_d . Vd, separated by grid barriers; then the last block to
//    finish phase 4 (a done counter) writes y = bf16(Y32).  The rank sums
//    accumulate in fp32 and are rounded to bf16 where the next phase stages
//    them (as the MFMA layers and the prefill path round the rank-r
//    intermediates); h is rounded to bf16 as the reference casts it between
//    the two halves;
//  * the load stream runs on across phases: the last loads a wave issues in
//    a phase are the first of the next one, so they are in flight during the
//    phase-end atomics, the grid barrier and the activation staging.
// Cross-block data moves only through device-coherent accesses (fp32
// atomics, device-scope zero stores and loads), as in the MFMA decode layer,
// whose two-level grid barrier and barrier words this kernel shares.
#pragma once

#include "decode_layer.hpp"

namespace svdmlp {

struct GvParams {
  const uint16_t* x;  // (T, d) bf16
  const uint16_t* ug;
  const uint16_t* vg;
  const uint16_t* uu;
  const uint16_t* vu;
  const uint16_t* ud;
  const uint16_t* vd;
  uint16_t* y;     // (T, d) bf16
  const uint16_t* resid;  // MLP block: y = bf16(resid + bf16(MLP)) (row pitch d), else null
  float* xu32;     // (2, T, r_gu)
  float* gu32;     // (2, T, ff)
  float* xd32;     // (T, r_d)
  float* y32;      // (T, d)
  uint64_t* sync;  // barrier words (kDl* layout)
  int T, d, ff, r_gu, r_d;
  int ld_u, ld_v, ld_ud, ld_vd;  // row pitch (elements) of ug and uu, vg and vu, ud, vd
};

constexpr int kGvThreads = 512;
constexpr int kGvDepth = 16;             // 16-byte loads in flight per lane
// Highest token count: above it the MFMA decode layer is faster (8B layer on
// MI355X: 78 / 81 / 86 / 87 us here at T = 1..4, 83 us there for each).
constexpr int kGvMaxT = 2;
constexpr int kGvAFloats = 12 * 1024;    // activation slice capacity (floats)

// Phase geometry: Y_m += A_m . W_m (m < nm), W_m of K x N, natural layout.
struct GvPhase {
  const uint16_t* w0;
  const uint16_t* w1;
  float* o0;
  float* o1;
  int K, N, L, S, KG, nm, groups;  // L: row pitch of w0 and w1 (elements)
};

template <int RW>
__device__ __forceinline__ GvPhase gv_phase(const GvParams& p, int ph) {
  GvPhase P;
  const int T = p.T;
  if (ph == 1) {
    P.w0 = p.ug; P.w1 = p.uu; P.o0 = p.xu32; P.o1 = p.xu32 + (int64_t)T * p.r_gu; P.K = p.d; P.N = p.r_gu; P.nm = 2;
    P.L = p.ld_u;
  } else if (ph == 2) {
    P.w0 = p.vg; P.w1 = p.vu; P.o0 = p.gu32; P.o1 = p.gu32 + (int64_t)T * p.ff; P.K = p.r_gu; P.N = p.ff; P.nm = 2;
    P.L = p.ld_v;
  } else if (ph == 3) {
    P.w0 = P.w1 = p.ud; P.o0 = P.o1 = p.xd32; P.K = p.ff; P.N = p.r_d; P.nm = 1;
    P.L = p.ld_ud;
  } else {
    P.w0 = P.w1 = p.vd; P.o0 = P.o1 = p.y32; P.K = p.r_d; P.N = p.d; P.nm = 1;
    P.L = p.ld_vd;
  }
  constexpr int STRIP = 512 / RW, GROUP = 8 * RW;
  P.S = (P.N + STRIP - 1) / STRIP;
  P.KG = P.K / GROUP;
  P.groups = P.nm * P.S * P.KG;
  return P;
}

// Device-scope zero fill of n floats (n even, 8-byte aligned) by the
// threads [tid0, tid0 + stride) of a grid-stride loop.
__device__ __forceinline__ void gv_zero(float* q, int64_t n, int64_t tid, int64_t stride) {
  const u32x2 z = {0u, 0u};
  for (int64_t i = tid; i < n / 2; i += stride) dl_store8(q + 2 * i, z);
}

// Issue cursor of a wave over a phase's group range (wave-uniform).
struct GvCursor {
  int mat, s, kg, left;
};

__device__ __forceinline__ GvCursor gv_cursor(const GvPhase& P, int g, int n) {
  GvCursor c;
  const int per = P.S * P.KG;
  c.mat = g / per;
  const int r = g - c.mat * per;
  c.s = r / P.KG;
  c.kg = r - c.s * P.KG;
  c.left = n;
  return c;
}

__device__ __forceinline__ void gv_advance(GvCursor& c, const GvPhase& P) {
  if (++c.kg == P.KG) {
    c.kg = 0;
    if (++c.s == P.S) {
      c.s = 0;
      ++c.mat;
    }
  }
}

// 16-byte buffer load into registers.  The caller waits for it with gv_wait
// before the value is read or the register is written again.
__device__ __forceinline__ u32x4 gv_load(i32x4 rs, uint32_t voff, uint32_t soff) {
  u32x4 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(rs), "s"(soff) : "memory");
  return v;
}

// Wait until at most N vector-memory operations are outstanding; ties the
// wait to the register of the load it completes.
template <int N>
__device__ __forceinline__ void gv_wait(u32x4& v) {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%1)" : "+v"(v) : "n"(N) : "memory");
}

// vmcnt(n + 1) for a runtime n in [0, kGvDepth): the count of loads issued
// after a wave's last atomics of a phase.
template <int J>
__device__ __forceinline__ void gv_wait_after(int n) {
  if constexpr (J < kGvDepth) {
    if (n == J) {
      dl_wait_vm<J + 1>();
      return;
    }
    gv_wait_after<J + 1>(n);
  } else {
    dl_wait_vm<0>();
  }
}

// Next load of the wave's stream.  Past its range (left == 0) the load has a
// descriptor with no records: it returns zeros and moves no data.
template <int RW>
__device__ __forceinline__ u32x4 gv_issue(const GvPhase& P, GvCursor& c, int lrow, int lcol) {
  constexpr int STRIP = 512 / RW, GROUP = 8 * RW;
  const bool live = c.left > 0;
  const uint16_t* w = c.mat ? P.w1 : P.w0;
  const i32x4 rs = make_rsrc_sgpr(w, live ? (uint32_t)P.K * (uint32_t)P.L * 2u : 0u);
  const int col = STRIP * c.s + lcol;
  const uint32_t voff = col < P.N ? ((uint32_t)lrow * (uint32_t)P.L + (uint32_t)col) * 2u : kOOB;
  const uint32_t soff = (uint32_t)__builtin_amdgcn_readfirstlane((int)((uint32_t)(GROUP * c.kg) * (uint32_t)P.L * 2u));
  const u32x4 v = gv_load(rs, voff, soff);
  if (live) {
    gv_advance(c, P);
    --c.left;
  }
  return v;
}

// Activation rows of a block's group range into LDS: a_lds[i * T + t] is
// token t of local row i (group i / GROUP, row i % GROUP of it).  Phase 1
// reads X (bf16); 2 the gate/up rank sums rounded to bf16; 3
// h = bf16(SiLU(G) * U); 4 the down rank sums rounded to bf16 (device-scope
// loads of other blocks' atomics).  The rank-r intermediates are rounded as
// the MFMA decode layer and the prefill path round them (the reference casts
// XU to the activation dtype, test_speedup.py:430-437).  Loads go
// out in batches of SB per thread before any is used; lanes past the end
// load element 0 and discard it, so no branch splits a batch.
template <int PH, int T, int RW>
__device__ __forceinline__ void gv_stage(const GvParams& p, const GvPhase& P, int g0, int n, float* a_lds) {
  constexpr int GROUP = 8 * RW, SB = 8;
  const int total = GROUP * n * T;
  const int per = P.S * P.KG;
  for (int i0 = threadIdx.x; i0 < total; i0 += SB * kGvThreads) {
    float v[SB], v2[SB];
#pragma unroll
    for (int q = 0; q < SB; ++q) {
      const int i = i0 + q * kGvThreads;
      const bool in = i < total;
      const int li = i / T, t = i - li * T;
      const int g = g0 + li / GROUP;
      const int mat = g / per;
      const int k = GROUP * ((g - mat * per) % P.KG) + li % GROUP;
      if constexpr (PH == 1) {
        v[q] = bf16_bits_to_f32(p.x[in ? (int64_t)t * p.d + k : 0]);
      } else if constexpr (PH == 2) {
        v[q] = __hip_atomic_load(p.xu32 + (in ? ((int64_t)mat * p.T + t) * p.r_gu + k : 0), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
      } else if constexpr (PH == 3) {
        v[q] = __hip_atomic_load(p.gu32 + (in ? (int64_t)t * p.ff + k : 0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        v2[q] = __hip_atomic_load(p.gu32 + (in ? ((int64_t)p.T + t) * p.ff + k : 0), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
      } else {
        v[q] = __hip_atomic_load(p.xd32 + (in ? (int64_t)t * p.r_d + k : 0), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
      }
    }
#pragma unroll
    for (int q = 0; q < SB; ++q) {
      const int i = i0 + q * kGvThreads;
      if (i < total) {
        if constexpr (PH == 3)
          a_lds[i] = bf16_bits_to_f32(f32_to_bf16_bits(silu_f32(v[q]) * v2[q]));
        else if constexpr (PH == 1)
          a_lds[i] = v[q];
        else
          a_lds[i] = bf16_bits_to_f32(f32_to_bf16_bits(v[q]));
      }
    }
  }
}

template <int T, int RW>
__global__ __launch_bounds__(kGvThreads, 1) void gemv_layer_kernel(GvParams p) {
  constexpr int D = kGvDepth;
  constexpr int STRIP = 512 / RW, GROUP = 8 * RW;
  __shared__ __attribute__((aligned(16))) float a_lds[kGvAFloats];
  __shared__ __attribute__((aligned(16))) float red[8 * T * STRIP];

  const int G = gridDim.x, b = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int lrow = RW * wave + (RW == 2 ? (lane >> 5) : 0);  // row within a group
  const int lcol = 8 * (RW == 2 ? (lane & 31) : lane);      // first column within a strip
  const bool writer = RW == 1 || lane < 32;                  // holds the wave's column sums after the fold
  uint32_t nbar = 0;
  const uint64_t gen0 = __hip_atomic_load(&p.sync[kDlGen], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t spin = dl_spin_limit(p.sync);
  __shared__ int s_bad;  // a barrier wait of this block gave up (the done counter carries it to the last block)
  if (threadIdx.x == 0) s_bad = 0;
  const int64_t gtid = (int64_t)b * kGvThreads + threadIdx.x, gstride = (int64_t)G * kGvThreads;

  auto range = [&](const GvPhase& P, int& g0, int& n) {
    g0 = (int)((int64_t)b * P.groups / G);
    n = (int)((int64_t)(b + 1) * P.groups / G) - g0;
  };

  u32x4 ring[D];
  // ---- phase 0: zero the fp32 sums; first loads of phase 1 ----
  gv_zero(p.xu32, (int64_t)2 * p.T * p.r_gu, gtid, gstride);
  gv_zero(p.gu32, (int64_t)2 * p.T * p.ff, gtid, gstride);
  gv_zero(p.xd32, (int64_t)p.T * p.r_d, gtid, gstride);
  gv_zero(p.y32, (int64_t)p.T * p.d, gtid, gstride);
  GvCursor ic;
  {
    const GvPhase P1 = gv_phase<RW>(p, 1);
    int g0, n;
    range(P1, g0, n);
    ic = gv_cursor(P1, g0, n);
#pragma unroll
    for (int u = 0; u < D; ++u) ring[u] = gv_issue<RW>(P1, ic, lrow, lcol);
  }
  dl_wait_vm<D>();  // the zero stores, issued before the D loads, are done
  dl_grid_sync(p.sync, gen0, ++nbar, spin, nullptr, &s_bad);

#pragma unroll 1
  for (int ph = 1; ph <= 4; ++ph) {
    const GvPhase P = gv_phase<RW>(p, ph);
    int g0, n;
    range(P, g0, n);
    const int npad = n > 0 ? (n + D - 1) / D * D : D;

    // ---- stage this block's activation rows: a_lds[i * T + t] ----
    switch (ph) {
      case 1: gv_stage<1, T, RW>(p, P, g0, n, a_lds); break;
      case 2: gv_stage<2, T, RW>(p, P, g0, n, a_lds); break;
      case 3: gv_stage<3, T, RW>(p, P, g0, n, a_lds); break;
      default: gv_stage<4, T, RW>(p, P, g0, n, a_lds); break;
    }
    dl_block_sync();

    // Next phase's cursor (its first D loads are issued in this phase's tail).
    GvPhase PN = P;
    GvCursor nc;
    nc.mat = nc.s = nc.kg = 0;
    nc.left = 0;
    if (ph < 4) {
      PN = gv_phase<RW>(p, ph + 1);
      int gn, nn;
      range(PN, gn, nn);
      nc = gv_cursor(PN, gn, nn);
    }

    // consume cursor: current piece (matrix, strip) and its remaining groups
    GvCursor cc = gv_cursor(P, g0, n);
    int piece_left = min(n, P.KG - cc.kg);
    float acc[T][8];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[t][c] = 0.0f;
    int after_flush = -1;  // loads issued after the wave's last atomics

    auto flush = [&]() {
      if constexpr (RW == 2) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int c = 0; c < 8; ++c) acc[t][c] += __shfl_xor(acc[t][c], 32);
      }
      if (writer) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
          float* r = red + (wave * T + t) * STRIP + lcol;
          *reinterpret_cast<f32x4*>(r) = f32x4{acc[t][0], acc[t][1], acc[t][2], acc[t][3]};
          *reinterpret_cast<f32x4*>(r + 4) = f32x4{acc[t][4], acc[t][5], acc[t][6], acc[t][7]};
        }
      }
      dl_block_sync();
      float* out = cc.mat ? P.o1 : P.o0;
      for (int i = threadIdx.x; i < T * STRIP; i += kGvThreads) {
        const int t = i / STRIP, c = i - t * STRIP;
        const int col = STRIP * cc.s + c;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < 8; ++w) s += red[(w * T + t) * STRIP + c];
        if (col < P.N) dl_atomic_add(out + (int64_t)t * P.N + col, s);
      }
      dl_block_sync();
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[t][c] = 0.0f;
    };

    for (int j = 0; j < npad; j += D) {
#pragma unroll
      for (int u = 0; u < D; ++u) {
        const int jj = j + u;
        gv_wait<D - 1>(ring[u]);
        if (jj < n) {
          const float* ar = a_lds + (GROUP * jj + lrow) * T;
          float a[T];
#pragma unroll
          for (int t = 0; t < T; ++t) a[t] = ar[t];
          const u32x4 w = ring[u];
          float wf[8];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            wf[2 * q] = __uint_as_float(w[q] << 16);
            wf[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
          }
#pragma unroll
          for (int t = 0; t < T; ++t)
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[t][c] = fmaf(a[t], wf[c], acc[t][c]);
          if (--piece_left == 0) {
            flush();
            after_flush = 0;
            // next piece of the range
            cc.kg = 0;
            if (++cc.s == P.S) {
              cc.s = 0;
              ++cc.mat;
            }
            piece_left = min(n - 1 - jj, P.KG);
          }
        }
        // the stream's load jj + D: this phase's (no records past its
        // range), then in the last round the next phase's first D
        if (jj + D >= npad)
          ring[u] = gv_issue<RW>(PN, nc, lrow, lcol);
        else
          ring[u] = gv_issue<RW>(P, ic, lrow, lcol);
        if (after_flush >= 0) ++after_flush;
      }
    }
    // The wave's atomics must be complete before its block arrives; the
    // loads issued after them may stay in flight.
    if (after_flush >= 1)
      gv_wait_after<0>(after_flush - 1);
    ic = nc;
    if (ph < 4) dl_grid_sync(p.sync, gen0, ++nbar, spin, nullptr, &s_bad);
  }
  // drain the run-out loads (no records) before the registers are released
#pragma unroll
  for (int u = 0; u < D; ++u) gv_wait<0>(ring[u]);

  // ---- phase 5: the last block to finish phase 4 writes y = bf16(Y32)
  // (MLP block: y = bf16(resid + bf16(Y32))) ----
  // Every wave has waited for its own atomics; a block counts itself done
  // once all of its waves have.  A block whose barrier wait gave up set
  // kGvDoneBad before its own arrival, so the last arrival sees it and
  // writes NaN instead (the sums may be incomplete).
  __shared__ int s_last;
  dl_block_sync();
  if (threadIdx.x == 0) {
    const uint64_t done =
        __hip_atomic_fetch_add(&p.sync[kGvDone], (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
    s_last = ((done & ~kGvDoneBad) % (uint64_t)G == 0) ? ((done & kGvDoneBad) ? 2 : 1) : 0;
  }
  dl_block_sync();
  if (s_last == 2) {
    uint32_t* yw = reinterpret_cast<uint32_t*>(p.y);
    for (int64_t i = threadIdx.x; i < (int64_t)p.T * p.d / 2; i += kGvThreads) yw[i] = 0x7fc07fc0u;  // bf16 NaN pairs
  } else if (s_last) {
    constexpr int SB = 8;
    const int64_t n = (int64_t)p.T * p.d / 2;
    for (int64_t i0 = threadIdx.x; i0 < n; i0 += SB * kGvThreads) {
      u32x2 v[SB];
#pragma unroll
      for (int q = 0; q < SB; ++q) {
        const int64_t i = i0 + q * kGvThreads;
        v[q] = dl_load8(p.y32 + 2 * (i < n ? i : 0));
      }
#pragma unroll
      for (int q = 0; q < SB; ++q) {
        const int64_t i = i0 + q * kGvThreads;
        if (i >= n) continue;
        uint32_t o = pack_bf16x2(__uint_as_float(v[q].x), __uint_as_float(v[q].y));
        if (p.resid) {
          const uint32_t xr = reinterpret_cast<const uint32_t*>(p.resid)[i];
          o = pack_bf16x2(__uint_as_float(xr << 16) + __uint_as_float(o << 16),
                          __uint_as_float(xr & 0xffff0000u) + __uint_as_float(o & 0xffff0000u));
        }
        reinterpret_cast<uint32_t*>(p.y)[i] = o;
      }
    }
  }
}

}  // namespace svdmlp
