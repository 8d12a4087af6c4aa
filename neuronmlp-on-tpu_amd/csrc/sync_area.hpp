// The workspace's 4096-byte sync area: cross-block words of the kernels that
// wait on other blocks (the persistent decode layers' grid barriers and
// split-K tile counters, the large-tile GEMM's in-kernel split-K fixup), the
// timeout flag and the bounded-wait override.  All words start at zero (the
// caller zeroes the area once) and every launch leaves them valid for the next
// one on the same workspace.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace svdmlp {

// Default bound of a grid-barrier wait, in polls (~1 us each with the
// device-scope load): seconds, far beyond any barrier of a resident grid.
constexpr uint32_t kDlSpinLimit = 1u << 22;
// Barrier words in the workspace's sync area, one 128-byte line each (in
// uint64 units): kDlGroups group counters, then root, generation, and the
// timeout line: word kDlFlag is nonzero once a bounded wait gave up (sticky
// until the caller zeroes the area), word kDlSpin, if nonzero, replaces
// kDlSpinLimit (failure tests set a tiny bound so that waits give up at once).
constexpr int kDlGroups = 16;
constexpr int kDlLine = 16;
constexpr int kDlRoot = kDlGroups * kDlLine;
constexpr int kDlGen = kDlRoot + kDlLine;
constexpr int kDlFlag = kDlGen + kDlLine;
constexpr int kDlSpin = kDlFlag + 1;
// Block-done counter of the streaming-GEMV decode layer (monotone, like the
// barrier counters: the last of every G arrivals finishes the launch); bit
// kGvDoneBad is set with the timeout flag, so the last block learns of a
// timeout from its own arrival.
constexpr int kGvDone = kDlFlag + kDlLine;
constexpr uint64_t kGvDoneBad = (uint64_t)1 << 63;
// 32-bit arrival counters of the split-K tiles of phases 1, 3 and 4 (in
// that order) fill the rest of the 4 KB area, kDlTileLines 128-byte lines.
// Tile t's counter is word t / kDlTileLines of line t % kDlTileLines, so
// neighbouring tiles, whose units finish together, hit different lines
// (packed consecutively, ~100 blocks' atomics on 3 lines cost ~2 us per
// layer).  The last arrival of a launch resets its tile's counter to zero.
constexpr int kDlTileWords = kGvDone + kDlLine;
constexpr int kDlTileLines = (512 - kDlTileWords) / kDlLine;
constexpr int kDlMaxTiles = kDlTileLines * 32;
constexpr int kDlSyncBytes = kDlTileWords * 8 + kDlMaxTiles * 4;
__device__ __forceinline__ uint32_t* dl_tile_counter(uint64_t* sync, int t) {
  return reinterpret_cast<uint32_t*>(sync + kDlTileWords) + (t % kDlTileLines) * 32 + t / kDlTileLines;
}


// Ready flags of the decode layer's XU_d tiles and RMSNorm rows (in place of
// the grid barriers before its phases 4 and 1): words 1..15 of the 16 group-counter lines, which the
// barrier's counters (word 0) leave free; tile t at line t % 16, word
// 1 + t / 16, so the pollers of different tiles read different lines.  A
// flag holds the epoch of the launch that wrote its tile (its generation at
// launch start plus one: every launch that uses the flags still passes a
// grid barrier, so the generation, read before any block's first barrier
// arrival, differs from launch to launch and is the same for all blocks of
// one).
constexpr int kDlMaxFlags = kDlGroups * (kDlLine - 1);
// Flags kDlRowFlag0 + m: row m of the MLP block's RMSNorm output written
// (phase 0); XU_d tiles use the flags below kDlRowFlag0.
constexpr int kDlRowFlag0 = kDlMaxFlags - 128;
__device__ __forceinline__ uint64_t* dl_ready_flag(uint64_t* sync, int t) {
  return sync + (t % kDlGroups) * kDlLine + 1 + t / kDlGroups;
}

// Cache-policy bits of a device-scope (sc1) buffer access: coherent across
// XCDs without cache maintenance.
constexpr int kDlSc1 = 16;

// Bound of this launch's barrier waits: the workspace's override, if set.
__device__ __forceinline__ uint32_t dl_spin_limit(uint64_t* sync) {
  const uint64_t o = __hip_atomic_load(&sync[kDlSpin], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return o ? (uint32_t)o : kDlSpinLimit;
}

}  // namespace svdmlp
