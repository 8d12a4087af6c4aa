// Launcher of the streaming-GEMV decode layer (1 or 2 tokens).  Grid = CU
// count (at most kDlMaxGrid, the MFMA decode layer's grid: both layers share
// the workspace's barrier counters, which need one grid size), one block per
// CU, plain launch; the grid barriers' polls are bounded, as in the MFMA
// decode layer.
#include <algorithm>

#include "decode_gemv.hpp"
#include "dispatch.hpp"

namespace svdmlp {

namespace {

template <int T, int RW>
hipError_t go(const GvParams& p, int grid, hipStream_t st) {
  hipLaunchKernelGGL((gemv_layer_kernel<T, RW>), dim3(grid), dim3(kGvThreads), 0, st, p);
  return hipGetLastError();
}

template <int RW>
hipError_t go_t(const GvParams& p, int grid, hipStream_t st) {
  switch (p.T) {
    case 1: return go<1, RW>(p, grid, st);
    case 2: return go<2, RW>(p, grid, st);
    default: return hipErrorInvalidValue;
  }
}

int resident(const void* k) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kGvThreads, 0) != hipSuccess) return 0;
  return n;
}

}  // namespace

int gemv_layer_grid(int rw) {
  auto compute = [rw]() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    const void* k = rw == 1 ? reinterpret_cast<const void*>(&gemv_layer_kernel<kGvMaxT, 1>)
                            : reinterpret_cast<const void*>(&gemv_layer_kernel<kGvMaxT, 2>);
    return resident(k) >= 1 ? std::min(cus, kDlMaxGrid) : 0;
  };
  return cached_per_device(rw == 1 ? DC_GV1 : DC_GV2, compute);
}

int gemv_layer_a_floats() { return kGvAFloats; }

hipError_t launch_gemv_layer(const GvParams& p, int rw, int grid, hipStream_t st, const char** why) {
  if (grid <= 0) {
    *why = "decode GEMV layer: the kernel cannot be resident on this device";
    return hipErrorInvalidValue;
  }
  if (p.T < 1 || p.T > kGvMaxT) {
    *why = "decode GEMV layer: no instance for this token count";
    return hipErrorInvalidValue;
  }
  const hipError_t e = rw == 1 ? go_t<1>(p, grid, st) : go_t<2>(p, grid, st);
  if (e != hipSuccess) *why = "decode GEMV layer: launch failed";
  return e;
}

}  // namespace svdmlp
