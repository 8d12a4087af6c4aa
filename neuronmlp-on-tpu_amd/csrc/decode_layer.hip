// Launcher of the persistent decode-layer kernel.  Grid = CU count (at most
// kDlMaxGrid, the units the workspace's slice area holds) with one block per
// CU (its LDS takes most of a CU), so on an otherwise idle device every block
// is resident at once.  A plain launch is used: a cooperative
// launch guarantees residency but costs ~20 us per launch on this stack
// (~2.3 us for a plain one).  If other work holds CUs, late blocks only delay
// the barriers; the bounded barrier spin turns a true deadlock into a flagged
// error instead of a hang.
#include <algorithm>

#include "decode_layer.hpp"
#include "dispatch.hpp"

namespace svdmlp {

namespace {

// p.gain set: the MLP block's instance, whose phase 0 applies the RMSNorm.
template <int MT, bool CONTRACT = false>
hipError_t coop(const DecLayerParams& p, int grid, hipStream_t st) {
  if (p.gain)
    hipLaunchKernelGGL((decode_layer_kernel<MT, CONTRACT, true>), dim3(grid), dim3(kDlThreads), 0, st, p);
  else
    hipLaunchKernelGGL((decode_layer_kernel<MT, CONTRACT>), dim3(grid), dim3(kDlThreads), 0, st, p);
  return hipGetLastError();
}

template <int MT, bool CONTRACT = false>
int blocks_per_cu() {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &n, reinterpret_cast<const void*>(&decode_layer_kernel<MT, CONTRACT>), kDlThreads, 0) != hipSuccess)
    return 0;
  return n;
}

}  // namespace

int decode_layer_mt(int T) { return T <= 16 ? 1 : (T <= 32 ? 2 : (T <= 64 ? 4 : 8)); }

namespace {

template <int MT, bool CONTRACT = false>
int grid_of() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return blocks_per_cu<MT, CONTRACT>() >= 1 ? std::min(cus, kDlMaxGrid) : 0;
}

}  // namespace

int decode_layer_grid(int mt) {
  if (mt == 1) return cached_per_device(DC_DL1, grid_of<1>);
  if (mt == 2) return cached_per_device(DC_DL2, grid_of<2>);
  if (mt == 4) return cached_per_device(DC_DL4, grid_of<4>);
  return cached_per_device(DC_DL8, grid_of<8>);
}

int decode_layer_contract_grid() { return cached_per_device(DC_DL_CONTRACT, grid_of<1, true>); }

hipError_t launch_decode_layer(const DecLayerParams& p, int mt, int grid, hipStream_t st, const char** why,
                               bool contract) {
  if (grid <= 0) {
    *why = "decode layer: the kernel cannot be resident on this device";
    return hipErrorInvalidValue;
  }
  if (p.gain && (p.d > 8 * kDlThreads * kDlNormPieces || p.T > grid || !p.xn || !p.resid)) {
    *why = "decode layer: the RMSNorm instance takes d <= 16384, a block per token and the block's buffers";
    return hipErrorInvalidValue;
  }
  if (p.p2split && (contract || p.ff % 128 || p.units2 > grid || p.units2 != 2 * (p.ff / 128) ||
                    p.r_gu / 128 + p.r_up / 128 + p.r_d / 128 + p.d / 128 + p.ff / 128 > kDlMaxTiles)) {
    *why = "decode layer: one-branch phase 2 takes ff % 128 == 0, a block per unit and a counter per column tile";
    return hipErrorInvalidValue;
  }
  if (p.r_up != p.r_gu && (!p.p2split || contract)) {
    *why = "decode layer: distinct gate and up ranks need the one-branch phase 2 (not the contracted layer)";
    return hipErrorInvalidValue;
  }
  hipError_t e;
  if (contract) {
    // one unit per h strip plus one combining block per XU_d tile
    // ... and a gate/up rank of at least NS - 1 ring stages, whose run-out
    // brings in the down half's first stages
    if (mt != 1 || p.units2 + p.r_d / 128 > grid || !p.cslices ||
        p.r_gu < 32 * DlDepth<1>::KC * (DlDepth<1>::NS - 1)) {
      *why = "contracted decode layer: one 16-row tile, a block per h strip and per XU_d tile, gate/up rank >= 320";
      return hipErrorInvalidValue;
    }
    e = coop<1, true>(p, grid, st);
  } else if (mt == 1)
    e = coop<1>(p, grid, st);
  else if (mt == 2)
    e = coop<2>(p, grid, st);
  else if (mt == 4)
    e = coop<4>(p, grid, st);
  else if (mt == 8)
    e = coop<8>(p, grid, st);
  else {
    *why = "decode layer: no instance for this token count";
    return hipErrorInvalidValue;
  }
  if (e != hipSuccess) *why = "decode layer: launch failed";
  return e;
}

}  // namespace svdmlp
