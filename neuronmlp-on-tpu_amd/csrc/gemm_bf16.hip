// bf16-MFMA GEMM instances with bf16 weights.
#include "dispatch.hpp"

namespace svdmlp {

namespace {

template <int SRCA, int NBR, int EPI, bool AK, bool BK, bool OT, bool VEC>
hipError_t go(const GemmParams& p, int splits, int batch, hipStream_t st) {
  using C = GemmCfg<kGemmBM, kGemmBN, 2, 2, __bf16, SRCA, SRC_BF16, AK, BK, NBR, EPI, OT, false, VEC>;
  return run_gemm<C>(p, splits, batch, st);
}

template <int SRCA, int NBR, int EPI, bool AK, bool OT>
hipError_t go2(const GemmDesc& d, const GemmParams& p, int splits, int batch, hipStream_t st) {
  return expand_bool(d.b_kc, [&](auto bk) {
    return expand_bool(d.vec, [&](auto vec) {
      return go<SRCA, NBR, EPI, AK, decltype(bk)::value, OT, decltype(vec)::value>(p, splits, batch, st);
    });
  });
}

}  // namespace

hipError_t launch_gemm_bf16(const GemmDesc& d, const GemmParams& p, int splits, int batch, hipStream_t st,
                            const char** why) {
  if (d.tm_f32 || d.srcb != SRC_BF16 || d.out_f32) {
    *why = "bf16 GEMM: unsupported type combination";
    return hipErrorInvalidValue;
  }
  if (d.nbr == 1 && !d.out_t) {
    if (d.srca == SRC_BF16 && d.epi == EPI_STORE)
      return d.a_kc ? go2<SRC_BF16, 1, EPI_STORE, true, false>(d, p, splits, batch, st)
                    : go2<SRC_BF16, 1, EPI_STORE, false, false>(d, p, splits, batch, st);
    if (d.srca == SRC_BF16 && d.epi == EPI_ATOMIC)
      return d.a_kc ? go2<SRC_BF16, 1, EPI_ATOMIC, true, false>(d, p, splits, batch, st)
                    : go2<SRC_BF16, 1, EPI_ATOMIC, false, false>(d, p, splits, batch, st);
    if (d.srca == SRC_F32 && d.epi == EPI_STORE && d.a_kc)
      return go2<SRC_F32, 1, EPI_STORE, true, false>(d, p, splits, batch, st);
  }
  if (d.nbr == 2 && d.epi == EPI_SWIGLU && d.a_kc) {
    if (d.srca == SRC_BF16)
      return d.out_t ? go2<SRC_BF16, 2, EPI_SWIGLU, true, true>(d, p, splits, batch, st)
                     : go2<SRC_BF16, 2, EPI_SWIGLU, true, false>(d, p, splits, batch, st);
    if (d.srca == SRC_F32)
      return d.out_t ? go2<SRC_F32, 2, EPI_SWIGLU, true, true>(d, p, splits, batch, st)
                     : go2<SRC_F32, 2, EPI_SWIGLU, true, false>(d, p, splits, batch, st);
  }
  *why = "bf16 GEMM: no compiled instance for this stage";
  return hipErrorInvalidValue;
}

}  // namespace svdmlp
