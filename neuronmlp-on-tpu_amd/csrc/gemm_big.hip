// Instances of the large-tile prefill GEMM (bf16 operands).
#include "dispatch.hpp"
#include "gemm_big.hpp"

namespace svdmlp {

namespace {

template <int FN, bool BK, int EPI, bool F32 = false, bool F8 = false, int NW = 8, int NS = 4>
hipError_t go(const BigParams& p, int splits, int batch, hipStream_t st) {
  using C = BigCfg<FN, BK, EPI, F32, F8, NW, NS>;
  dim3 grid(p.mtiles * p.ntiles, splits, batch);
  hipLaunchKernelGGL(big_gemm_kernel<C>, grid, dim3(C::THREADS), 0, st, p);
  return hipGetLastError();
}

template <int FN, int EPI, bool F32 = false>
hipError_t go_b(const BigDesc& d, const BigParams& p, int splits, int batch, hipStream_t st) {
  if constexpr (FN == 8 && EPI == BEPI_STORE) {  // 4-wave instances: natural layout, STORE
    if (d.nw == 4 && !d.b_kc)
      return d.fp8 ? go<FN, false, EPI, F32, true, 4>(p, splits, batch, st)
                   : go<FN, false, EPI, F32, false, 4>(p, splits, batch, st);
  }
  if (d.fp8) return go<FN, false, EPI, F32, true>(p, splits, batch, st);  // fp8 B: natural layout only
  return d.b_kc ? go<FN, true, EPI, F32>(p, splits, batch, st) : go<FN, false, EPI, F32>(p, splits, batch, st);
}

template <int FN>
hipError_t go_e(const BigDesc& d, const BigParams& p, int splits, int batch, hipStream_t st, const char** why) {
  switch (d.epi) {
    case BEPI_STORE:
      if (d.out_f32) {
        if constexpr (FN != 7) return go_b<FN, BEPI_STORE, true>(d, p, splits, batch, st);
        break;
      }
      return go_b<FN, BEPI_STORE>(d, p, splits, batch, st);
    case BEPI_SWIGLU_MEM:
      return go_b<FN, BEPI_SWIGLU_MEM>(d, p, splits, batch, st);
    case BEPI_STORE_FRAG:
      return go_b<FN, BEPI_STORE_FRAG>(d, p, splits, batch, st);
    default: break;
  }
  *why = "big GEMM: unsupported epilogue for this tile";
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_big(const BigDesc& d, const BigParams& p, int splits, int batch, hipStream_t st,
                      const char** why) {
  if (d.fn == 8) return go_e<8>(d, p, splits, batch, st, why);
  if (d.fn == 7) return go_e<7>(d, p, splits, batch, st, why);
  if (d.fn == 4) return go_e<4>(d, p, splits, batch, st, why);
  *why = "big GEMM: no compiled instance for this tile";
  return hipErrorInvalidValue;
}

}  // namespace svdmlp
