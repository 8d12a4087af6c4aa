// Runtime -> template dispatch for the SVD-MLP kernels.  Each launcher
// returns hipSuccess, or hipErrorInvalidValue (with *why set) when the
// requested combination has no compiled instance.
#pragma once

#include <atomic>

#include "decode.hpp"

namespace svdmlp {

struct GemmDesc {
  bool tm_f32;   // MFMA type: fp32 (true) or bf16 (false)
  int srca;      // SrcKind of A
  int srcb;      // SrcKind of B
  bool a_kc;     // A stored (M, K) with K contiguous; else (K, M)
  bool b_kc;     // B stored (N, K) with K contiguous (Linear); else (K, N)
  int nbr;       // 1 or 2 branches
  int epi;       // EpiKind
  bool out_t;    // transposed output
  bool out_f32;  // fp32 output (EPI_STORE / EPI_SWIGLU)
  bool vec;      // 16-byte vector path (aligned, multiples of 8)
};

struct DecodeDesc {
  int mt;        // 16-row token tiles: 1, 2 or 4
  int srca;      // SRC_BF16, SRC_F32 or SRC_SWIGLU
  int srcb;      // SRC_BF16 or SRC_FP8
  bool b_kc;     // Linear-layout weights
};

struct BigDesc {
  int fn;        // block tile = 256 x 32*fn (8 waves, each 64 x 16*fn)
  bool b_kc;     // Linear-layout B
  int epi;       // BigEpi
  bool out_f32;  // fp32 output (split-K partial slices)
  bool fp8 = false;  // fp8 e4m3fn B (natural layout) with per-column scales
  int nw = 8;        // waves per block: 8, or 4 (natural-layout fn-8 STORE tiles)
  int kg = 1;        // K groups: 1 (256-row tiles), or 2 (128-row tiles, two 32-k halves per stage)
};

struct BigParams;
struct DecLayerParams;

// Block tile of the prefill GEMM (rows x cols of C per 256-thread block).
constexpr int kGemmBM = 128;
constexpr int kGemmBN = 128;

hipError_t launch_gemm_bf16(const GemmDesc& d, const GemmParams& p, int splits, int batch, hipStream_t st,
                            const char** why);
hipError_t launch_gemm_fp8(const GemmDesc& d, const GemmParams& p, int splits, int batch, hipStream_t st,
                           const char** why);
hipError_t launch_gemm_f32(const GemmDesc& d, const GemmParams& p, int splits, int batch, hipStream_t st,
                           const char** why);
hipError_t launch_big(const BigDesc& d, const BigParams& p, int splits, int batch, hipStream_t st,
                      const char** why);
hipError_t launch_decode(const DecodeDesc& d, const DecodeParams& p, int blocks, hipStream_t st,
                         const char** why);
hipError_t launch_fill_zero(float* p, int64_t n, hipStream_t st);
// MLP block prologue / epilogue: y = act(gain * rmsnorm(x)), y = act(x + y).
hipError_t launch_rmsnorm(const void* x, const float* gain, void* y, int64_t T, int64_t d, float eps, bool bf16,
                          hipStream_t st);
hipError_t launch_residual_add(const void* x, void* y, int64_t n, bool bf16, hipStream_t st);
// out[c][r] = in[r][c] for a (rows x cols) bf16 matrix (row pitches ldi, ldo
// elements): the transposed operands of the reference's TPU launchers.
hipError_t launch_transpose_bf16(const uint16_t* in, int64_t ldi, uint16_t* out, int64_t ldo, int rows, int cols,
                                 hipStream_t st);
// Persistent decode layer (T <= 128): token tiles of 16 * MT rows (MT = 1,
// 2, 4 or 8), grid = CU count (at most kDlMaxGrid) when the kernel fits one
// block per CU, else 0.
int decode_layer_mt(int T);
int decode_layer_grid(int mt);
// contract: the contracted instance (phases 2 and 3 fused, h kept in LDS),
// grid = decode_layer_contract_grid().
int decode_layer_contract_grid();
hipError_t launch_decode_layer(const DecLayerParams& p, int mt, int grid, hipStream_t st, const char** why,
                               bool contract = false);
// Streaming-GEMV decode layer (T <= 2): rows per wave load rw (1 or 2),
// grid = CU count when the kernel fits one block per CU, else 0.
struct GvParams;
int gemv_layer_grid(int rw);
int gemv_layer_a_floats();
hipError_t launch_gemv_layer(const GvParams& p, int rw, int grid, hipStream_t st, const char** why);
hipError_t launch_cvt_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t st);
// out[i] = bf16(sum_s in[s * stride + i]) for s < slices.
hipError_t launch_reduce_bf16(const float* in, int slices, int64_t stride, uint16_t* out, int64_t n,
                              hipStream_t st);
// Split-K slices of the large-tile kernel in fragment order (out_frag):
// out[m][n] = bf16(sum_s in[s * sstride + zb * bstride + frag(m, n)]) for
// tiles of 256 x 32*fn with nw waves (kg 1) or 128 x 32*fn with K groups
// (kg 2, nw 8: four wave tiles), batch entries zb (out batch stride
// obstride elements); with `gate` (bf16 in the same fragment order),
// out = bf16(SiLU(gate) * sum); with `gsl` (gsplits fp32 slices of the gate
// in the same layout and slice stride), the gate is bf16(sum of its slices
// in order) first, as launch_reduce_bf16 would round it; with `resid` (bf16,
// row pitch ldo, batch entry 0), out = bf16(resid + bf16(sum)), the MLP
// block's residual add.
hipError_t launch_reduce_frag_bf16(const float* in, int splits, int64_t sstride, int64_t bstride, uint16_t* out,
                                   int64_t ldo, int64_t obstride, int M, int N, int mtiles, int ntiles, int fn, int nw,
                                   int batch, hipStream_t st, const uint16_t* gate = nullptr,
                                   const uint16_t* resid = nullptr, int kg = 1, const float* gsl = nullptr,
                                   int gsplits = 0);
// fp8 x fp8 GEMM (gemm_f8f8.hpp), nw = 8 or 4 waves: splits > 1 writes fp32
// fragment-order slices (256 x 128 tiles) for launch_reduce_frag_bf16 (fn 4, nw).
struct F8Params;
hipError_t launch_f8_gemm(const F8Params& p, int splits, int nw, hipStream_t st, const char** why);
// e4m3fn row quantisation: q[m] = e4m3(h[m] * 448 / amax_m), s[m] = amax_m / 448.
// blk: q in 16 x 128 blocks ((m, k) at ((m/16)*(n/128) + k/128)*2048 +
// (m%16)*128 + k%128; n a multiple of 128, ldq unused), the fp8 GEMM's a_blk.
hipError_t launch_quant_rows_e4m3(const uint16_t* h, int64_t ldh, uint8_t* q, int64_t ldq, float* s, int rows, int n,
                                  hipStream_t st, const char** why, bool blk = false);
hipError_t launch_finalize(const float* g, const float* u, int64_t ldi, uint16_t* out, int64_t ldo, int rows,
                           int cols, bool swiglu, bool out_t, hipStream_t st);

// A per-device constant (a persistent kernel's grid size) computed once per
// device and slot: the lookups behind it (device attributes, occupancy) cost
// host time on every decode call otherwise.
enum DeviceConst : int { DC_DL1 = 0, DC_DL2, DC_DL4, DC_DL8, DC_DL_CONTRACT, DC_GV1, DC_GV2, DC_COUNT };
template <class F>
inline int cached_per_device(int slot, F compute) {
  static std::atomic<int> cache[64][DC_COUNT];  // value + 1; 0 = not yet computed
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return compute();
  int v = cache[dev][slot].load(std::memory_order_relaxed);
  if (v == 0) {
    v = compute() + 1;
    cache[dev][slot].store(v, std::memory_order_relaxed);
  }
  return v - 1;
}

inline hipError_t gemm_launch(const GemmDesc& d, const GemmParams& p, int splits, int batch, hipStream_t st,
                              const char** why) {
  if (d.tm_f32) return launch_gemm_f32(d, p, splits, batch, st, why);
  if (d.srcb == SRC_FP8) return launch_gemm_fp8(d, p, splits, batch, st, why);
  return launch_gemm_bf16(d, p, splits, batch, st, why);
}

// Compile-time bool expansion helper.
template <class F>
inline hipError_t expand_bool(bool b, F&& f) {
  return b ? f(std::true_type{}) : f(std::false_type{});
}

template <class Cfg>
inline hipError_t run_gemm(const GemmParams& p, int splits, int batch, hipStream_t st) {
  dim3 grid(p.mtiles * p.ntiles, splits, batch);
  hipLaunchKernelGGL(gemm_kernel<Cfg>, grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace svdmlp
