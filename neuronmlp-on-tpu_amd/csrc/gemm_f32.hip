// fp32-MFMA GEMM instances (v_mfma_f32_16x16x4_f32): the reference's
// mixed_precision=False / float32 arm, computed without any rounding to bf16.
#include "dispatch.hpp"

namespace svdmlp {

namespace {

template <int NBR, int EPI, bool AK, bool BK, bool OT, bool VEC>
hipError_t go(const GemmParams& p, int splits, int batch, hipStream_t st) {
  using C = GemmCfg<kGemmBM, kGemmBN, 2, 2, float, SRC_F32, SRC_F32, AK, BK, NBR, EPI, OT, true, VEC>;
  return run_gemm<C>(p, splits, batch, st);
}

template <int NBR, int EPI, bool AK, bool OT>
hipError_t go2(const GemmDesc& d, const GemmParams& p, int splits, int batch, hipStream_t st) {
  return expand_bool(d.b_kc, [&](auto bk) {
    return expand_bool(d.vec, [&](auto vec) {
      return go<NBR, EPI, AK, decltype(bk)::value, OT, decltype(vec)::value>(p, splits, batch, st);
    });
  });
}

}  // namespace

hipError_t launch_gemm_f32(const GemmDesc& d, const GemmParams& p, int splits, int batch, hipStream_t st,
                           const char** why) {
  if (!d.tm_f32 || d.srca != SRC_F32 || d.srcb != SRC_F32) {
    *why = "fp32 GEMM: all operands must be fp32";
    return hipErrorInvalidValue;
  }
  if (d.nbr == 1 && !d.out_t && (d.out_f32 || d.epi == EPI_ATOMIC)) {
    if (d.epi == EPI_STORE)
      return d.a_kc ? go2<1, EPI_STORE, true, false>(d, p, splits, batch, st)
                    : go2<1, EPI_STORE, false, false>(d, p, splits, batch, st);
    if (d.epi == EPI_ATOMIC)
      return d.a_kc ? go2<1, EPI_ATOMIC, true, false>(d, p, splits, batch, st)
                    : go2<1, EPI_ATOMIC, false, false>(d, p, splits, batch, st);
  }
  if (d.nbr == 2 && d.epi == EPI_SWIGLU && d.a_kc && d.out_f32) {
    return d.out_t ? go2<2, EPI_SWIGLU, true, true>(d, p, splits, batch, st)
                   : go2<2, EPI_SWIGLU, true, false>(d, p, splits, batch, st);
  }
  *why = "fp32 GEMM: no compiled instance for this stage";
  return hipErrorInvalidValue;
}

}  // namespace svdmlp
