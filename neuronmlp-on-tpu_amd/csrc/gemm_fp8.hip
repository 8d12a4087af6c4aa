// bf16-MFMA GEMM instances with fp8 e4m3fn weights (natural layout).  The
// weights are widened to bf16 exactly in registers; the per-output-column
// scale is applied to the fp32 accumulator in the epilogue.
#include "dispatch.hpp"

namespace svdmlp {

namespace {

template <int SRCA, int NBR, int EPI, bool AK, bool OT>
hipError_t go(const GemmParams& p, int splits, int batch, hipStream_t st) {
  using C = GemmCfg<kGemmBM, kGemmBN, 2, 2, __bf16, SRCA, SRC_FP8, AK, false, NBR, EPI, OT, false, true>;
  return run_gemm<C>(p, splits, batch, st);
}

}  // namespace

hipError_t launch_gemm_fp8(const GemmDesc& d, const GemmParams& p, int splits, int batch, hipStream_t st,
                           const char** why) {
  if (d.tm_f32 || d.srcb != SRC_FP8 || d.out_f32 || d.b_kc || !d.vec) {
    *why = "fp8 GEMM: weights must be natural layout, aligned, with bf16 activations";
    return hipErrorInvalidValue;
  }
  if (d.nbr == 1 && !d.out_t) {
    if (d.srca == SRC_BF16 && d.epi == EPI_STORE)
      return d.a_kc ? go<SRC_BF16, 1, EPI_STORE, true, false>(p, splits, batch, st)
                    : go<SRC_BF16, 1, EPI_STORE, false, false>(p, splits, batch, st);
    if (d.srca == SRC_BF16 && d.epi == EPI_ATOMIC)
      return d.a_kc ? go<SRC_BF16, 1, EPI_ATOMIC, true, false>(p, splits, batch, st)
                    : go<SRC_BF16, 1, EPI_ATOMIC, false, false>(p, splits, batch, st);
    if (d.srca == SRC_F32 && d.epi == EPI_STORE && d.a_kc)
      return go<SRC_F32, 1, EPI_STORE, true, false>(p, splits, batch, st);
  }
  if (d.nbr == 2 && d.epi == EPI_SWIGLU && d.a_kc) {
    if (d.srca == SRC_BF16)
      return d.out_t ? go<SRC_BF16, 2, EPI_SWIGLU, true, true>(p, splits, batch, st)
                     : go<SRC_BF16, 2, EPI_SWIGLU, true, false>(p, splits, batch, st);
    if (d.srca == SRC_F32)
      return d.out_t ? go<SRC_F32, 2, EPI_SWIGLU, true, true>(p, splits, batch, st)
                     : go<SRC_F32, 2, EPI_SWIGLU, true, false>(p, splits, batch, st);
  }
  *why = "fp8 GEMM: no compiled instance for this stage";
  return hipErrorInvalidValue;
}

}  // namespace svdmlp
