// The whole SVD-MLP layer at decode shapes (T <= 128 tokens) in one
// persistent launch (a plain launch of one block per CU; see the launcher).
//
// At these shapes the layer is a stream of 311 MB of bf16 factors (LLaMA3-8B,
// r = 2816) against a few KB of activations, so the design goal is to keep
// HBM busy from the first byte to the last:
//  * one block per CU (grid = CU count; the LDS footprint keeps it to one);
//  * weights go global -> LDS by direct DMA through a ring of 4 to 6 stages
//    of one or two 32-k chunks (by token count: the activation tile shares
//    the ring).  A chunk is 32 k x 128 columns, stored as two 64-column
//    sub-tiles of 128-byte rows whose 32-byte units are XOR-swizzled by
//    dl_wswz(k), and read with the transposing ds_read_b64_tr_b16, so no
//    register transpose exists;
//  * the activation rows (zero-padded to 16 * MT) follow in the same ring;
//  * the layer runs as four phases separated by three grid barriers:
//      1  XU_g, XU_u = X . [Ug | Uu]                (split-K)
//      2  h = bf16(SiLU(XU_g . Vg) * (XU_u . Vu))    (whole rank, no split: a
//         block owns 64 columns of both branches at one token tile, else
//         128 columns of one branch, the g and u units of a column tile
//         meeting through its counter)
//      3  XU_d = h . Ud                              (split-K)
//      4  y = XU_d . Vd                              (split-K)
//  * split-K tiles (128 columns) are combined without atomics or a zero
//    fill: every unit stores its fp32 accumulators, in register order, as a
//    slice of the workspace and counts its arrival on the tile's counter;
//    the block whose arrival completes the count sums every slice, its own
//    included, in split order (so replays are bitwise identical) and rounds
//    the tile to bf16 once: XU and XU_d (the
//    reference rounds the rank-r intermediate to the activation dtype) and y
//    itself, so phases 2 to 4 stream bf16 activations and no barrier
//    follows phase 4 (fp32 atomics onto shared sums cost ~20 us per phase at
//    64 tokens);
//  * at a barrier, once its arrival is counted, every block issues the
//    weight DMAs of its first stages of the next phase (weights do not depend
//    on the barrier), so barrier latency overlaps the weight stream.
// Data crosses blocks through device-scope (sc1) stores (slices, bf16
// tiles), device-scope loads (slices) and the counters' atomics.  Each wave
// waits for its own writes (vmcnt(0)) before its block arrives at a barrier,
// so the barriers need no cache write-back or invalidation (with agent-scope
// fences a barrier costs ~9 us, without ~2 us).  The bf16 activation tiles
// (XU, h, XU_d) are read back through the caches (plain DMAs) when the
// workspace is 128-byte aligned: every 128-byte line of them has one writing
// block, no CU reads a line of them in a launch before the barrier that
// follows its write (so no cache holds a copy older than the write from this
// launch), and copies from earlier launches are not served (a kernel sees
// the writes of the kernels before it, which needs exactly that).  One copy
// per XCD's L2 then serves its CUs: 8B layer at 32 tokens 82.9 -> 78.4 us.
// With a workspace aligned to less, lines could have two writers, and the
// activation DMAs stay device-scope.
// Grid barriers are two-level: blocks arrive on one of 16 group counters,
// the last of a group arrives on a root counter, and the last root arrival
// advances a generation word that every block polls (a single counter for
// all blocks serialises 256 device-scope atomics, ~15 us).  The 64-bit
// counters only ever grow: a launch reads the generation at its start and
// waits for start + k at barrier k, and group / root completion is taken
// modulo the group size, so no reset is needed as long as every launch on a
// workspace uses the same grid.  Polls are bounded.  A block whose wait
// gives up sets the workspace's timeout flag, remembers it, and runs to its
// end with whatever data it finds (every access stays in bounds, and every
// block still arrives once at every barrier, so the counters stay
// consistent); whoever writes y then writes NaN instead wherever the data
// could be incomplete: a block that timed out itself, and every split-K
// combination that finds the flag set after its last slice arrived (any
// incomplete input reached it only after the flag was set).
#pragma once

#include "gemm_big.hpp"
#include "sync_area.hpp"

namespace svdmlp {

struct DecLayerParams {
  const void* x;  // (T, d) bf16
  const void* ug;
  const void* vg;
  const void* uu;
  const void* vu;
  const void* ud;
  const void* vd;
  void* y;         // (T, d) bf16
  uint16_t* xu16;  // bf16 gate/up rank intermediates: (T, r_gu) gate, then (T, r_up) up
  uint16_t* h;     // (T, ff) bf16
  uint16_t* xd16;  // (T, r_d) bf16 down rank intermediate
  float* slices;   // split-K partial sums: dl_slice_banks(MT) banks of kDlMaxGrid units, MT * 2048 floats each
  float* cslices;  // contracted layer: partial XU_d tiles, (r_d / 128, units2, T, 128) fp32
  uint64_t* sync;  // barrier words, one per 128-byte line (kDl*), then split-K tile counters
  int T, d, ff, r_gu, r_d;
  int r_up;                            // up-branch rank (r_gu is the gate's); distinct ranks need p2split
  int ks1, ks3, ks4;                   // K per split, phases 1, 3, 4 (multiples of 32)
  int units1, units2, units3, units4;  // tiles x splits
  int splits1, splits3, splits4;       // splits per tile, phases 1, 3 and 4
  int ld_u, ld_v, ld_ud, ld_vd;        // row pitch (elements) of ug, vg, ud, vd
  int ld_uu, ld_vu;                    // ... of uu and vu
  int a_cached;                        // activation DMAs through the caches (workspace 128-byte aligned)
  // Phase 2 with one branch per unit: unit u = 2 t + b computes g (b = 0) or
  // u (b = 1) over 128 columns 128 t..; the pair meets through a tile
  // counter after phases 1, 3 and 4's.  Otherwise a unit computes both over
  // 64 columns.
  int p2split;
  // Phase 4 waits for its XU_d tiles' ready flags (kDlMaxFlags tiles at
  // most) instead of a grid barrier: the contracted layer, one token tile,
  // and from two tiles up with the tiles written by all their splits (dist).
  int xd_ready;
  // Phase 2 waits for the XU tiles' ready flags (flags xu_flag0 .. xu_flag0 +
  // tiles - 1) instead of a grid barrier
  int xu_ready, xu_flag0;
  // Phase 4 at one token tile as 16-column units over the whole rank, one per
  // block (dl_narrow_unit): grid == d / 16, r_d a multiple of 32, at most
  // kDlNarrowMaxChunks 32-k chunks, with the XU_d tiles' ready flags
  int p4narrow;  // xu_ready: 0 barrier, 1 a flag per XU tile, 2 one flag for all of XU
  // First of the second-round tile counters of dl_combine_dist with ready
  // flags: phase 1's XU tiles, then phase 3's XU_d tiles.
  int cnt2;
  // Phase 3 waits for one flag per K split (flag hf0 + split), set by the
  // last of the phase-2 units writing h columns of that split to count down
  // on counter hc0 + split, instead of a grid barrier (eight token tiles,
  // one-branch pairs writing h half each, per-tile XU flags); the launch's
  // one grid-barrier generation then comes from an arrival-only barrier
  // after phase 1.
  int h_ready, hf0, hc0;
  // dl_combine_dist: a split that waits for the others issues the next
  // phase's first weight stages before it waits (bit 0: phase 1, bit 1:
  // phase 3), else once its share of the tile is written
  int pre_wait;
  // Token tiles of 32 rows and more: split-K tiles combined by all their
  // splits (dl_combine_dist), the phase-2 pairs' h written half by each
  // unit (dl_swiglu_pair_dist).
  int dist;
  // The weight prefetch at a grid barrier fills all NS ring slots (the last
  // one where the unit has that many stages), not NS - 1 (DlDepth::PF_FULL
  // instances only).
  int pf_full;
  // MLP block (null otherwise): y = bf16(resid + bf16(MLP)); with `gain`
  // (NORM instances) a phase 0 writes RMSNorm(x) to xn, which phase 1 reads
  // instead of x.
  const void* resid;  // (T, d) bf16, row pitch d
  const float* gain;  // (d) fp32
  uint16_t* xn;       // (T, d) bf16
  float eps;
};

constexpr int kDlThreads = 512;
// Largest grid: a split-K phase has at most one unit per block, so a slice
// bank holds kDlMaxGrid units (MT * 2048 floats each).
constexpr int kDlMaxGrid = 256;
// Slice banks: unit u's slice is slice u of its phase's bank.  From two
// token tiles up phases 2 and 4 use bank 1, phases 1 and 3 bank 0: their
// units start on ready flags (not a grid barrier) while the previous phase's
// slices may still be read (a split sums its share after the others move
// on), and the grid barrier before phase 3 separates every reuse of a bank.
// At one token tile one bank: phase 2 starts on the single "XU complete"
// flag or a grid barrier, and phase 4 also waits for the flag of the tile
// its block's phase-3 unit stored a slice for.  (8B layer, against one bank
// without those waits, same box: T=48 / 64 / 100 79.2 / 83.4 / 107.7 ->
// 77.8 / 82.5 / 107.0 us; the MLP block -0.5 to -1.3 us.)
template <int MT>
constexpr int kDlBank24 = MT >= 2 ? 1 : 0;
__host__ __device__ constexpr int dl_slice_banks(int mt) { return mt >= 2 ? 2 : 1; }
constexpr int kDlWStage = 8192;    // 32 k x 128 columns bf16
// Ring geometry by token tile: a ring stage holds KC 32-k chunks (more
// weight bytes per block barrier) and the ring holds NS stages, as far as
// the activation tile, which shares the ring, leaves room.  From 2 tiles up
// the k loop is bound by its per-stage chain (wait, block barrier, LDS
// fragment reads, MFMAs) rather than by the bytes in flight: 8B layer at 64
// tokens 101.4 us with (KC 1, NS 6), 95.8 with (2, 4), 102.6 with (3, 3);
// at 32 tokens (2, 4) 78.8, (3, 4) 83.7, (2, 5) 79.4; at 128 tokens (1, 4)
// 141.3, (2, 3) 143.1.
template <int MT>
struct DlDepth {
  static constexpr int KC = MT == 8 ? 1 : 2;
  static constexpr int NS = MT == 1 ? 6 : 4;
  // The weight prefetch at a grid barrier fills all NS ring slots rather
  // than NS - 1 (DecLayerParams::pf_full): 8B layer at 128 tokens 119.7 ->
  // 118.5 us; at 1-64 tokens 0.2-0.4 us slower, so only eight token tiles.
  static constexpr bool PF_FULL = MT == 8;
};

// fp32 -> bf16 round to nearest even in integer form (NaN stays NaN): the
// same bits as the hardware conversion that the other kernels use, which
// here raised the 4- and 8-tile instances' scalar-register spills from ~62 to
// ~91 and the 8B layer at 64 tokens from 112 to 115 us.
__device__ __forceinline__ uint32_t dl_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t dl_pack_bf16x2(float lo, float hi) {
  return dl_bf16_bits(lo) | (dl_bf16_bits(hi) << 16);
}

template <int N>
__device__ __forceinline__ void dl_wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Block barrier that publishes LDS writes (ds, and DMA after the issuing
// wave's vmcnt wait) without a global-memory fence.
__device__ __forceinline__ void dl_block_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Grid barrier k of this launch (gen0: generation at launch start).  The
// bound of the wait (dl_spin_limit) comes from spin_lds when non-null, else
// spin_reg: where it lives changes the register allocation of the whole
// layer kernel (8B layer: the 1-tile instance is 0.5 us faster with it in a
// register, the 4-tile instance ~4 us faster with it in LDS).  Every wave
// has completed its own global writes (vmcnt(0)) before calling.  If the
// wait gives up, thread 0 sets the timeout flag (and the GEMV layer's
// done bit), waits for both to complete, and sets *bad (LDS) for the block;
// *bad is never cleared within a launch.  (Polling the root counter itself,
// one atomic hop shorter, was ~2.4 us slower per layer: the polls then share
// a line with the group completions' atomics.)  `pre`, run by every wave
// once its block's arrival atomics have returned and before the first poll,
// issues the wave's share of the next phase's first weight DMAs.  Issued
// before the arrival, they delay it: the block's own 80 KB burst sits
// ahead of its arrival atomic at the memory side (8B layer: T=1 70.0 ->
// 68.6 us, T=8 72.0 -> 68.8 us).
struct DlNoPre {
  __device__ void operator()() const {}
};
template <class Pre = DlNoPre>
__device__ __forceinline__ void dl_grid_sync(uint64_t* sync, uint64_t gen0, uint32_t k, uint32_t spin_reg,
                                             const uint32_t* spin_lds, int* bad, const Pre& pre = Pre{}) {
  dl_block_sync();
  if (threadIdx.x == 0) {
    const uint32_t G = gridDim.x, b = blockIdx.x;
    const uint32_t g = b % kDlGroups;
    const uint32_t gsize = G / kDlGroups + (g < G % kDlGroups ? 1u : 0u);
    const uint32_t ngroups = G < (uint32_t)kDlGroups ? G : (uint32_t)kDlGroups;
    const uint64_t a = __hip_atomic_fetch_add(&sync[g * kDlLine], (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((a + 1) % gsize == 0) {
      const uint64_t r = __hip_atomic_fetch_add(&sync[kDlRoot], (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((r + 1) % ngroups == 0)
        __hip_atomic_fetch_add(&sync[kDlGen], (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  dl_block_sync();
  pre();
  if (threadIdx.x == 0) {
    const uint32_t spin = spin_lds ? *spin_lds : spin_reg;
    uint32_t polls = 0;
    while ((int64_t)(__hip_atomic_load(&sync[kDlGen], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - gen0 - k) < 0) {
      __builtin_amdgcn_s_sleep(1);
      if (++polls >= spin) {
        __hip_atomic_fetch_or(&sync[kDlFlag], (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_or(&sync[kGvDone], kGvDoneBad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        dl_wait_vm<0>();  // both flags complete before anything this block writes next
        *bad = 1;
        break;
      }
    }
  }
  dl_block_sync();
}

// Arrival at the launch's next grid barrier without waiting for it (the
// caller counts it in its barrier number): the generation still advances once
// every block has arrived.  For a launch whose blocks wait on ready flags
// only, whose epoch is the generation at launch start plus one: no block's
// read of that generation can see this launch's advance, which needs its own
// arrival.
__device__ __forceinline__ void dl_grid_arrive(uint64_t* sync) {
  if (threadIdx.x == 0) {
    const uint32_t G = gridDim.x, b = blockIdx.x;
    const uint32_t g = b % kDlGroups;
    const uint32_t gsize = G / kDlGroups + (g < G % kDlGroups ? 1u : 0u);
    const uint32_t ngroups = G < (uint32_t)kDlGroups ? G : (uint32_t)kDlGroups;
    const uint64_t a = __hip_atomic_fetch_add(&sync[g * kDlLine], (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((a + 1) % gsize == 0) {
      const uint64_t r = __hip_atomic_fetch_add(&sync[kDlRoot], (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((r + 1) % ngroups == 0)
        __hip_atomic_fetch_add(&sync[kDlGen], (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Tile t's ready flag set to `epoch` by thread 0, once every wave of the
// block has completed its stores of the tile (vmcnt(0) then the barrier).
__device__ __forceinline__ void dl_set_ready(uint64_t* flag, uint64_t epoch) {
  dl_wait_vm<0>();
  dl_block_sync();
  if (threadIdx.x == 0) __hip_atomic_store(flag, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void dl_set_ready(uint64_t* sync, int t, uint64_t epoch) {
  dl_set_ready(dl_ready_flag(sync, t), epoch);
}

// Bounded wait until the ready flags of tiles t0..t1 (at most 128), and of
// tile tx unless negative, hold `epoch`: lane i of wave 0 polls tiles t0 + i
// and t0 + 64 + i, lane 0 also tx.  A wait that gives up sets the timeout
// flags as a grid-barrier wait does.
__device__ __forceinline__ void dl_wait_ready(uint64_t* sync, int t0, int t1, uint64_t epoch, uint32_t spin,
                                              int* bad, int tx = -1) {
  if (threadIdx.x < 64) {
    const int t = t0 + (int)threadIdx.x;
    bool done = t > t1, done2 = t + 64 > t1, done3 = threadIdx.x != 0 || tx < 0;
    uint32_t polls = 0;
    while (true) {
      if (!done)
        done = __hip_atomic_load(dl_ready_flag(sync, t), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == epoch;
      if (!done2)
        done2 = __hip_atomic_load(dl_ready_flag(sync, t + 64), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == epoch;
      if (!done3)
        done3 = __hip_atomic_load(dl_ready_flag(sync, tx), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == epoch;
      done = done && done2 && done3;
      if (__builtin_amdgcn_read_exec() == __ballot(done)) break;  // every lane's tile is ready
      __builtin_amdgcn_s_sleep(1);
      if (++polls >= spin) {
        if (threadIdx.x == 0) {
          __hip_atomic_fetch_or(&sync[kDlFlag], (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_fetch_or(&sync[kGvDone], kGvDoneBad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          dl_wait_vm<0>();
          *bad = 1;
        }
        break;
      }
    }
  }
  dl_block_sync();
}

// Buffer descriptor of the split-K slice area (kDlMaxGrid units of MT
// 16-row blocks, 2048 floats each), the cache-policy bits of a device-scope
// (sc1) buffer access, and an offset past every record.
constexpr uint32_t kDlPastSlices = 0xfffffff0u;
template <int MT>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dl_slice_rsrc(float* slices) {
  return __builtin_amdgcn_make_buffer_rsrc(slices, 0, kDlMaxGrid * MT * 2048 * 4, 0x00020000);
}

// Device-scope 8-byte store / load (sc1): coherent across XCDs without cache
// maintenance.
__device__ __forceinline__ void dl_store8(void* p, u32x2 v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u32x2 dl_load8(const void* p) {
  return __builtin_bit_cast(u32x2, __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<void*>(p)), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void dl_atomic_add(float* p, float v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One unit of a phase: an output tile of 16*MT rows x 128 columns over the
// k range [kb, ke).  DUAL: sub-tile 0 is branch g (A = a0, B = b0), sub-tile
// 1 branch u (A = a1, B = b1), both over columns n0..n0+63; otherwise both
// sub-tiles read B = b0 (columns n0..n0+127) against A = a0.
struct DlUnit {
  const void* a0;
  const void* a1;
  int64_t lda;  // elements
  const void* b0;
  const void* b1;
  int64_t ldb;  // elements
  uint32_t a_bytes, b_bytes;
  int n0, kb, ke;
  uint16_t* dst;  // bf16 result (row-major, ldo)
  int64_t ldo;
};

// Compile-time shape of a unit (bf16 activations).
template <int MT, bool DUAL>
struct DlShape {
  static constexpr int A_ROW = 64;                          // bytes per 32-k activation row
  static constexpr int A_SUB = 16 * MT * A_ROW;             // one branch of one stage
  static constexpr int NA = (DUAL ? 2 : 1) * A_SUB / 1024;  // 1 KB DMA instructions per stage
  static constexpr int CNT_A = (NA + 7) / 8;                // per wave per chunk (padded with dummies)
  static constexpr int KC = DlDepth<MT>::KC;
  static constexpr int P = KC * (1 + CNT_A);                // DMA instructions per wave per stage
};

template <int MT>
struct DlLds {
  static constexpr int NS = DlDepth<MT>::NS;
  static constexpr int KC = DlDepth<MT>::KC;
  static constexpr int A_CHUNK = MT * 16 * 64 * 2;  // one 32-k chunk: bf16, two branches (the largest case)
  static constexpr int W_SLOT = KC * kDlWStage;
  static constexpr int A_SLOT = KC * A_CHUNK;
  static constexpr int W_OFF = 0;
  static constexpr int A_OFF = NS * W_SLOT;
  static constexpr int DUMMY_OFF = A_OFF + NS * A_SLOT;
  static constexpr int FLAG_OFF = DUMMY_OFF + 1024;  // int: "this block finishes the tile"
  static constexpr int BAD_OFF = FLAG_OFF + 4;       // int: "a barrier wait of this block gave up"
  static constexpr int SPIN_OFF = FLAG_OFF + 8;      // uint32: bound of the grid-barrier waits (MT >= 4)
  static constexpr int BYTES = FLAG_OFF + 16;
  static_assert(BYTES <= 160 * 1024, "LDS budget");
};

struct DlCtx {
  uint32_t lbase;  // LDS byte address of the block's array
  lds_cptr l0;
  int wave, lane, lr, lg, T;
  int a_cached;  // DecLayerParams::a_cached
  int pf_full;   // DecLayerParams::pf_full
};

// 32-byte unit swizzle of weight row k (128-byte rows, two per 64-bank
// row): a transposing read's lanes 0-15 touch rows k0..k0+3 and lanes 16-31
// rows k0+8..k0+11 in the same pass; k & 3 spreads each group's rows over
// distinct units and k & 8 flips the low bit, so the second group takes the
// units of each half of the banks that the first leaves free.
__device__ __forceinline__ int dl_wswz(int k) { return (k & 3) ^ ((k >> 3) & 1); }

// Weight DMA of stage j into ring slot `slot` (one instruction per wave):
// rows 8*(wave%4)..+7 of sub-tile wave/4; lane L takes row 8*(wave%4) + L/8,
// physical chunk L%8 of 32-byte unit pu = (L%8)/2, which holds logical unit
// pu ^ dl_wswz(row).
template <int MT, bool DUAL>
__device__ __forceinline__ void dl_dma_w(const DlCtx& c, const DlUnit& U, int j, int slot) {
  using L = DlLds<MT>;
  const int sub = c.wave >> 2;
  const int row = 8 * (c.wave & 3) + (c.lane >> 3);
  const int col = (DUAL ? 0 : 64 * sub) + 16 * (((c.lane & 7) >> 1) ^ dl_wswz(row)) + 8 * (c.lane & 1);
  const void* bp = (DUAL && sub) ? U.b1 : U.b0;
  const uint32_t voff = (uint32_t)row * (uint32_t)U.ldb * 2u + (uint32_t)(U.n0 + col) * 2u;
#pragma unroll
  for (int kc = 0; kc < L::KC; ++kc) {
    const int k0 = U.kb + 32 * (L::KC * j + kc);
    const bool live = k0 < U.ke;
    const i32x4 rs = make_rsrc_sgpr(bp, live ? U.b_bytes : 0u);
    dma16(rs, voff, live ? (uint32_t)k0 * (uint32_t)U.ldb * 2u : 0u,
          c.lbase + L::W_OFF + slot * L::W_SLOT + kc * kDlWStage + sub * 4096 + (c.wave & 3) * 1024);
  }
}

// Stages of unit U in the ring (KC 32-k chunks each).
template <int MT>
__device__ __forceinline__ int dl_stages(const DlUnit& U) {
  return (U.ke - U.kb + 32 * DlLds<MT>::KC - 1) / (32 * DlLds<MT>::KC);
}

// The weight DMAs of a stage that was issued already (KC per wave, as
// dl_dma_w), fetching nothing into the dummy slot: the memory counter then
// counts the same operations per step.
template <int MT>
__device__ __forceinline__ void dl_dma_w_none(const DlCtx& c, const void* any) {
  using L = DlLds<MT>;
#pragma unroll
  for (int kc = 0; kc < L::KC; ++kc) dma16(make_rsrc_sgpr(any, 0u), kOOB, 0u, c.lbase + L::DUMMY_OFF);
}

// Activation DMAs of stage j into ring slot `slot` (CNT_A per wave):
// instruction q holds rows 16q..16q+15 (64 bytes each, 16-byte chunk XOR
// a_swz(row)) of branch q / (NA/2) when DUAL.  Instructions past NA are
// dummies (no records) into a scratch slot, keeping the per-wave count.
template <int MT, bool DUAL>
__device__ __forceinline__ void dl_dma_a(const DlCtx& c, const DlUnit& U, int j, int slot) {
  using S = DlShape<MT, DUAL>;
  using L = DlLds<MT>;
#pragma unroll
  for (int kc = 0; kc < L::KC; ++kc) {
    const int k0 = U.kb + 32 * (L::KC * j + kc);
    const bool live = k0 < U.ke;
#pragma unroll
    for (int ci = 0; ci < S::CNT_A; ++ci) {
      const int q = c.wave + 8 * ci;
      if (q < S::NA) {
        constexpr int PER = DUAL ? S::NA / 2 : S::NA;
        const int br = DUAL ? q / PER : 0, qq = q % PER;
        const void* ap = br ? U.a1 : U.a0;
        const i32x4 rs = make_rsrc_sgpr(ap, live ? U.a_bytes : 0u);
        const int row = 16 * qq + (c.lane >> 2);
        const int lchunk = (c.lane & 3) ^ a_swz(row);
        const uint32_t voff = row < c.T ? (uint32_t)row * (uint32_t)U.lda * 2u + (uint32_t)lchunk * 16u : kOOB;
        const uint32_t soff = live ? (uint32_t)k0 * 2u : 0u;
        const uint32_t dst = c.lbase + L::A_OFF + slot * L::A_SLOT + kc * L::A_CHUNK + br * S::A_SUB + qq * 1024;
        if (c.a_cached)
          dma16(rs, voff, soff, dst);
        else
          dma16_dev(rs, voff, soff, dst);
      } else {
        dma16_dev(make_rsrc_sgpr(U.a0, 0u), kOOB, 0u, c.lbase + L::DUMMY_OFF);
      }
    }
  }
}

// vmcnt wait for stage j in the first NS-2 steps (KC chunks per stage,
// CNT_A activation DMAs per chunk): the activation DMAs of stages
// j+1..NS-2 and the j steps' (W, A) DMAs were issued after it:
// (NS-2) * KC * CNT_A + j * KC in all (B + J * STEP).
template <int B, int STEP, int J, int NMAX>
__device__ __forceinline__ void dl_wait_head(int j) {
  if constexpr (J < NMAX) {
    if (j == J) {
      dl_wait_vm<B + J * STEP>();
      return;
    }
    dl_wait_head<B, STEP, J + 1, NMAX>(j);
  }
}

// No weight DMAs in the run-out steps (stages past the unit's K): the
// default of dl_run, whose dl_dma_w then fetches nothing.
struct DlNoRunOut {
  static constexpr bool kActive = false;
  __device__ void operator()(int, int) const {}
};

// Runs one unit: returns the accumulators (lane: D[n = 4*lg + t][m = lr] of
// each 16-row block mt).  `prefetched`: every wave already issued its
// weight DMAs of stages 0..NS-2 (at the grid barrier), so every wave's order
// is W(0..NS-2), A(0..NS-2), then (W, A) per step; with c.pf_full and more
// than NS - 1 stages it also issued W(NS-1) there, and step 0 issues KC
// DMAs that fetch nothing in its place (the same count, so the same waits,
// which only ever need the A of their stage: every W is issued before it).
// Otherwise the first
// stages go out as (W, A) pairs, so stage 0 is usable as soon as its own
// pair lands rather than after every CU's whole first burst (8B layer: T=8
// 74.6 -> 72.0 us, T=64 103.7 -> 102.7 us), and every wait is the steady
// count.  `run_out(i, slot)`, when
// active, issues the weight DMAs (KC per wave) of what follows the unit in
// place of the empty stages past its K: stage nk + i goes to `slot`.
template <int MT, bool DUAL, class RunOut = DlNoRunOut>
__device__ __forceinline__ void dl_run(const DlCtx& c, const DlUnit& U, bool prefetched, f32x4 (&acc)[MT],
                                       const RunOut& run_out = RunOut{}) {
  using S = DlShape<MT, DUAL>;
  using L = DlLds<MT>;
  constexpr int NS = L::NS, KC = L::KC;
  const int nk = (U.ke - U.kb + 32 * KC - 1) / (32 * KC);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (!prefetched) {
    for (int s = 0; s < NS - 1; ++s) {
      dl_dma_w<MT, DUAL>(c, U, s, s);
      dl_dma_a<MT, DUAL>(c, U, s, s);
    }
  } else {
    for (int s = 0; s < NS - 1; ++s) dl_dma_a<MT, DUAL>(c, U, s, s);
  }

  // fragment addresses within a slot
  const int sub = c.wave >> 2, lu = c.wave & 3;
  const int k_lo = 8 * c.lg + (c.lr >> 2);
  const int b_off = L::W_OFF + sub * 4096 + k_lo * 128 + ((lu ^ dl_wswz(k_lo)) << 5) + ((c.lr & 3) << 3);
  const int abr = DUAL ? sub : 0;

  for (int j = 0; j < nk; ++j) {
    if (prefetched && j < NS - 2)
      dl_wait_head<(NS - 2) * KC * S::CNT_A, KC, 0, NS - 2>(j);
    else
      dl_wait_vm<(NS - 2) * S::P>();
    dl_block_sync();
    const int sn = j + NS - 1, slot_n = sn % NS;
    if (DlDepth<MT>::PF_FULL && j == 0 && prefetched && c.pf_full && sn < nk)
      dl_dma_w_none<MT>(c, U.b0);  // issued with the prefetch at the grid barrier
    else if (RunOut::kActive && sn >= nk)
      run_out(sn - nk, slot_n);
    else
      dl_dma_w<MT, DUAL>(c, U, sn, slot_n);
    dl_dma_a<MT, DUAL>(c, U, sn, slot_n);

    const int slot = j % NS;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const lds_cptr wb = c.l0 + slot * L::W_SLOT + kc * kDlWStage + b_off;
      const u32x2 lo = lds_read_tr(wb), hi = lds_read_tr(wb + 512);
      const u32x4 fb = u32x4{lo.x, lo.y, hi.x, hi.y};
      const lds_cptr ab = c.l0 + L::A_OFF + slot * L::A_SLOT + kc * L::A_CHUNK + abr * S::A_SUB;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int row = 16 * mt + c.lr;
        const u32x4 fa = lds_read_b128(ab + row * 64 + ((c.lg ^ a_swz(row)) << 4));
        acc[mt] = mfma_chunk(fb, fa, acc[mt], __bf16{});
      }
    }
  }
  dl_wait_vm<0>();  // drain run-out DMAs before the ring is reused
  dl_block_sync();
}

// Phase 2 with one branch per unit (DecLayerParams::p2split): unit u holds
// g (u even) or u (u odd) of 128 columns from U.n0 in acc (the lane layout
// of dl_combine).  It stores its rows < T as slice u and counts its arrival
// on the column tile's counter; the second of the pair resets the counter,
// loads the other unit's slice and writes h = bf16(SiLU(g) * u) -- the same
// fp32 operands, so the same bits, as a unit that computes both branches.
template <int MT>
__device__ __forceinline__ void dl_swiglu_pair(const DlCtx& c, const DlUnit& U, const f32x4 (&acc)[MT], int u,
                                               uint32_t* cnt, float* slices, int* flag, uint16_t* h) {
  const int n = U.n0 + 64 * (c.wave >> 2) + 16 * (c.wave & 3) + 4 * c.lg;
  const __amdgpu_buffer_rsrc_t rs = dl_slice_rsrc<MT>(slices);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const uint32_t off = 16 * mt + c.lr < c.T ? (uint32_t)(((u * MT + mt) * 2048 + 4 * threadIdx.x) * 4) : kDlPastSlices;
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(acc[mt].x), __float_as_uint(acc[mt].y),
                                                 __float_as_uint(acc[mt].z), __float_as_uint(acc[mt].w)},
                                           rs, off, 0, kDlSc1);
  }
  dl_wait_vm<0>();
  dl_block_sync();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + 1 == 2u;
    if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  dl_block_sync();
  if (!*flag) return;
  u32x4 v[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const uint32_t off =
        16 * mt + c.lr < c.T ? (uint32_t)((((u ^ 1) * MT + mt) * 2048 + 4 * threadIdx.x) * 4) : kDlPastSlices;
    v[mt] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kDlSc1);
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + c.lr;
    if (m < c.T) {
      const f32x4 o = f32x4{__uint_as_float(v[mt].x), __uint_as_float(v[mt].y), __uint_as_float(v[mt].z),
                            __uint_as_float(v[mt].w)};
      const f32x4 g = (u & 1) ? o : acc[mt], uv = (u & 1) ? acc[mt] : o;
      dl_store8(h + (int64_t)m * U.ldo + n, u32x2{dl_pack_bf16x2(silu_f32(g.x) * uv.x, silu_f32(g.y) * uv.y),
                                                  dl_pack_bf16x2(silu_f32(g.z) * uv.z, silu_f32(g.w) * uv.w)});
    }
  }
}

// Bounded wait of thread 0 until the tile counter `cnt` reads zero (the
// last split's reset: see dl_combine_dist); a wait that gives up sets the
// timeout flags as a grid-barrier wait does.
__device__ __forceinline__ void dl_wait_reset(uint32_t* cnt, uint64_t* sync, uint32_t spin, int* bad) {
  uint32_t polls = 0;
  while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
    __builtin_amdgcn_s_sleep(1);
    if (++polls >= spin) {
      __hip_atomic_fetch_or(&sync[kDlFlag], (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_or(&sync[kGvDone], kGvDoneBad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      dl_wait_vm<0>();
      *bad = 1;
      break;
    }
  }
}

// Arrival on a counter that `n` units share per launch: one atomic
// increment that wraps to zero at the n-th arrival (global_atomic_inc with
// limit n - 1), so the last arrival leaves the counter at zero for the next
// use with no store of its own.  Returns whether this was the last arrival.
__device__ __forceinline__ bool dl_arrive_wrap(uint32_t* cnt, int n) {
  return __builtin_amdgcn_atomic_inc32(cnt, (uint32_t)n - 1u, __ATOMIC_RELAXED, "agent") == (uint32_t)n - 1u;
}

// dl_swiglu_pair with the pair's work halved (token tiles of 32 rows and
// more): the g unit writes h for the first MT/2 16-row blocks, the u unit for
// the rest.  Each unit stores the half of its tile that its partner writes
// (slice u, the same offsets), arrives on the pair's counter (the second
// arrival wraps it to zero, which releases the first, dl_wait_reset), loads
// its partner's half of its own rows and writes them: the same fp32
// operands, so the same bits.  (The first to arrive issuing the next
// phase's first weight DMAs before it waits, as dl_combine_dist does, cost
// 0.3-0.5 us at 32-128 tokens.)  8B layer, against dl_swiglu_pair, with
// dl_combine_dist for the split phases: T=64 86.9 -> 86.3 us, T=128 121.1
// -> 120.2 us.
template <int MT>
__device__ __forceinline__ void dl_swiglu_pair_dist(const DlCtx& c, const DlUnit& U, const f32x4 (&acc)[MT], int u,
                                                    uint32_t* cnt, float* slices, int* flag, uint16_t* h,
                                                    uint64_t* sync, uint32_t spin, int* bad) {
  static_assert(MT >= 2 && MT % 2 == 0, "whole 16-row blocks per half");
  constexpr int HALF = MT / 2;
  const int own = u & 1;  // this unit writes blocks own * HALF ..
  const int n = U.n0 + 64 * (c.wave >> 2) + 16 * (c.wave & 3) + 4 * c.lg;
  const __amdgpu_buffer_rsrc_t rs = dl_slice_rsrc<MT>(slices);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if ((mt >= HALF) == (own != 0)) continue;  // the partner's blocks only
    const uint32_t off = 16 * mt + c.lr < c.T ? (uint32_t)(((u * MT + mt) * 2048 + 4 * threadIdx.x) * 4) : kDlPastSlices;
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(acc[mt].x), __float_as_uint(acc[mt].y),
                                                 __float_as_uint(acc[mt].z), __float_as_uint(acc[mt].w)},
                                           rs, off, 0, kDlSc1);
  }
  dl_wait_vm<0>();
  dl_block_sync();
  if (threadIdx.x == 0) *flag = dl_arrive_wrap(cnt, 2);
  dl_block_sync();
  if (!*flag) {
    if (threadIdx.x == 0) dl_wait_reset(cnt, sync, spin, bad);
    dl_block_sync();
  }
  // this unit's blocks own * HALF .. own * HALF + HALF - 1, with compile-time
  // indices into acc (a runtime index would put acc in scratch memory)
  auto finish = [&](auto base) {
    constexpr int B0 = decltype(base)::value;
    u32x4 v[HALF];
#pragma unroll
    for (int i = 0; i < HALF; ++i) {
      const int mt = B0 + i;
      const uint32_t off =
          16 * mt + c.lr < c.T ? (uint32_t)((((u ^ 1) * MT + mt) * 2048 + 4 * threadIdx.x) * 4) : kDlPastSlices;
      v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kDlSc1);
    }
#pragma unroll
    for (int i = 0; i < HALF; ++i) {
      const int m = 16 * (B0 + i) + c.lr;
      if (m < c.T) {
        const f32x4 o = f32x4{__uint_as_float(v[i].x), __uint_as_float(v[i].y), __uint_as_float(v[i].z),
                              __uint_as_float(v[i].w)};
        const f32x4 g = B0 ? o : acc[B0 + i], uv = B0 ? acc[B0 + i] : o;
        dl_store8(h + (int64_t)m * U.ldo + n, u32x2{dl_pack_bf16x2(silu_f32(g.x) * uv.x, silu_f32(g.y) * uv.y),
                                                    dl_pack_bf16x2(silu_f32(g.z) * uv.z, silu_f32(g.w) * uv.w)});
      }
    }
  };
  if (own)
    finish(std::integral_constant<int, HALF>{});
  else
    finish(std::integral_constant<int, 0>{});
}

// Split-K combination of unit u = tile + split * nt (splits per tile) into
// the bf16 tile at `dst` (row pitch U.ldo, columns from U.n0).  Lane layout
// of acc: D[n = 4*lg + t][m = lr] of each 16-row block mt.
//  * one split: the accumulators are rounded straight to dst;
//  * otherwise the unit stores its rows < T as slice u (16 bytes per lane
//    and block mt, in register order) and, once every wave's stores have
//    completed, counts its arrival on the tile's counter; the block that
//    completes the count resets the counter and sums every split's slice,
//    its own included, in split order, 0 + s_0 + s_1 + ..., so the result
//    does not depend on which unit came last; then it rounds to dst.  (Its
//    own slice from registers, selected into the sum, cost ~0.4 us more per
//    layer than the extra load.)
// `out_y`: dst is the layer output; it receives NaN instead if this block
// gave up a barrier wait (`bad`) or, after the last arrival, the timeout
// flag is set.  With `resid` (the MLP block) it receives bf16(resid + the
// bf16 MLP output), the residual add of the block.
// Units of a split phase never exceed the grid (at most one per block).
template <int MT>
__device__ __forceinline__ void dl_combine(const DlCtx& c, const DlUnit& U, f32x4 (&acc)[MT], int u, int nt,
                                           int splits, uint32_t* cnt, float* slices, int* flag, uint16_t* dst,
                                           bool out_y, bool bad, uint64_t* sync, const uint16_t* resid = nullptr) {
  const int n = U.n0 + 64 * (c.wave >> 2) + 16 * (c.wave & 3) + 4 * c.lg;
  bool poison = out_y && bad;
  if (splits > 1) {
    // Slices move as one 16-byte device-scope (sc1) buffer access per lane
    // and 16-row block; rows >= T take an offset past the records, which
    // stores drop and loads read as zeros.  (Pairs of 8-byte atomic accesses
    // cost 2 us at 1-8 tokens and 21 us at 128 in the 8B layer.)
    const __amdgpu_buffer_rsrc_t rs = dl_slice_rsrc<MT>(slices);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint32_t off = 16 * mt + c.lr < c.T ? (uint32_t)(((u * MT + mt) * 2048 + 4 * threadIdx.x) * 4) : kDlPastSlices;
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(acc[mt].x), __float_as_uint(acc[mt].y),
                                                   __float_as_uint(acc[mt].z), __float_as_uint(acc[mt].w)},
                                             rs, off, 0, kDlSc1);
    }
    dl_wait_vm<0>();
    dl_block_sync();
    if (threadIdx.x == 0) {
      const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = old + 1 == (uint32_t)splits;
      if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *flag = last;
    }
    dl_block_sync();
    if (!*flag) return;
    // issued with the first slices, after every split's arrival was seen
    const uint64_t tflag = out_y ? __hip_atomic_load(&sync[kDlFlag], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
    const int tile = u % nt;
    // slices in flight (registers: SB * MT * 4); at MT 4, 8 in flight cost
    // ~4 us per layer at 64 tokens against 4 (scalar-register spills)
    constexpr int SB = MT >= 8 ? 2 : (MT >= 4 ? 4 : 8);
    f32x4 sum[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sum[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < splits; s0 += SB) {
      u32x4 v[SB][MT];
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const int s = s0 + i;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const bool live = s < splits && 16 * mt + c.lr < c.T;
          const uint32_t off =
              live ? (uint32_t)((((tile + s * nt) * MT + mt) * 2048 + 4 * threadIdx.x) * 4) : kDlPastSlices;
          v[i][mt] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kDlSc1);
        }
      }
#pragma unroll
      for (int i = 0; i < SB; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          sum[mt].x += __uint_as_float(v[i][mt].x);
          sum[mt].y += __uint_as_float(v[i][mt].y);
          sum[mt].z += __uint_as_float(v[i][mt].z);
          sum[mt].w += __uint_as_float(v[i][mt].w);
        }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = sum[mt];
    poison = poison || tflag != 0;
  }
  constexpr uint32_t kNaN2 = 0x7fc07fc0u;  // two bf16 quiet NaNs
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + c.lr;
    if (m < c.T) {
      u32x2 v = u32x2{dl_pack_bf16x2(acc[mt].x, acc[mt].y), dl_pack_bf16x2(acc[mt].z, acc[mt].w)};
      if (resid && !poison) {
        const u32x2 xr = *reinterpret_cast<const u32x2*>(resid + (int64_t)m * U.ldo + n);
        v = u32x2{dl_pack_bf16x2(__uint_as_float(xr.x << 16) + __uint_as_float(v.x << 16),
                                 __uint_as_float(xr.x & 0xffff0000u) + __uint_as_float(v.x & 0xffff0000u)),
                  dl_pack_bf16x2(__uint_as_float(xr.y << 16) + __uint_as_float(v.y << 16),
                                 __uint_as_float(xr.y & 0xffff0000u) + __uint_as_float(v.y & 0xffff0000u))};
      }
      dl_store8(dst + (int64_t)m * U.ldo + n, poison ? u32x2{kNaN2, kNaN2} : v);
    }
  }
}

// Split-K combination shared by all splits of the tile (token tiles of 32
// rows and more, whose slices are 16 KB and larger: one block summing every
// split took 3-5 us per phase at 64 rows).  Every unit stores its slice and
// counts its arrival on the tile's counter, as in dl_combine; the last
// arrival wraps the counter to zero, and that zero releases the tile's
// other splits, which poll for it (the counter receives no other arrival in
// the launch, so it stays zero).  Split s then sums share s of the tile's
// float4 elements (16 * MT rows x 128 columns, in slice order) over every
// split in split order, 0 + s_0 + s_1 + ..., the same additions as one block
// summing the whole tile, so the result is bitwise that of dl_combine, and
// rounds them to dst.  `pre()` is run by every split but the last before it
// polls: it may issue the next phase's first weight DMAs, so the weight
// stream goes on while the split waits, and returns whether it did, which
// this function returns (the grid barrier then issues none).  y (`out_y`) is poisoned as in
// dl_combine: this block's own give-ups (`bad`, read after the wait) and the
// timeout flag read after the release.
template <int MT, class Pre>
__device__ __forceinline__ bool dl_combine_dist(const DlCtx& c, const DlUnit& U, const f32x4 (&acc)[MT], int u,
                                                int nt, int splits, uint32_t* cnt, float* slices, int* flag,
                                                uint16_t* dst, bool out_y, int* bad, uint64_t* sync, uint32_t spin,
                                                const uint16_t* resid, const Pre& pre, uint64_t* ready = nullptr,
                                                uint64_t epoch = 0, uint32_t* cnt2 = nullptr) {
  const __amdgpu_buffer_rsrc_t rs = dl_slice_rsrc<MT>(slices);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const uint32_t off = 16 * mt + c.lr < c.T ? (uint32_t)(((u * MT + mt) * 2048 + 4 * threadIdx.x) * 4) : kDlPastSlices;
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(acc[mt].x), __float_as_uint(acc[mt].y),
                                                 __float_as_uint(acc[mt].z), __float_as_uint(acc[mt].w)},
                                           rs, off, 0, kDlSc1);
  }
  dl_wait_vm<0>();
  dl_block_sync();
  if (threadIdx.x == 0) *flag = dl_arrive_wrap(cnt, splits);
  dl_block_sync();
  bool issued = false;
  if (!*flag) {
    issued = pre();
    if (threadIdx.x == 0) dl_wait_reset(cnt, sync, spin, bad);
    dl_block_sync();
  }
  const bool poison = out_y && (*bad != 0 || __hip_atomic_load(&sync[kDlFlag], __ATOMIC_RELAXED,
                                                               __HIP_MEMORY_SCOPE_AGENT) != 0);
  const int tile = u % nt, s = u / nt;
  constexpr int TOTAL = MT * 512;  // float4 elements of a tile
  const int share = (TOTAL + splits - 1) / splits;
  const int e1 = min(TOTAL, (s + 1) * share);
  constexpr int SB = 8;  // slices in flight per element
  for (int e = s * share + (int)threadIdx.x; e < e1; e += kDlThreads) {
    const int mt = e >> 9, t = e & 511;  // element e: the lane t of block mt in every slice
    const int m = 16 * mt + (t & 15);
    if (m >= c.T) continue;
    f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < splits; s0 += SB) {
      u32x4 v[SB];
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const uint32_t off =
            s0 + i < splits ? (uint32_t)((((tile + (s0 + i) * nt) * MT + mt) * 2048 + 4 * t) * 4) : kDlPastSlices;
        v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kDlSc1);
      }
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        if (s0 + i < splits) {
          sum.x += __uint_as_float(v[i].x);
          sum.y += __uint_as_float(v[i].y);
          sum.z += __uint_as_float(v[i].z);
          sum.w += __uint_as_float(v[i].w);
        }
      }
    }
    // column of lane t: wave t / 64, lane group (t % 64) / 16
    const int w = t >> 6;
    const int n = U.n0 + 64 * (w >> 2) + 16 * (w & 3) + 4 * ((t & 63) >> 4);
    u32x2 v = u32x2{dl_pack_bf16x2(sum.x, sum.y), dl_pack_bf16x2(sum.z, sum.w)};
    if (resid && !poison) {
      const u32x2 xr = *reinterpret_cast<const u32x2*>(resid + (int64_t)m * U.ldo + n);
      v = u32x2{dl_pack_bf16x2(__uint_as_float(xr.x << 16) + __uint_as_float(v.x << 16),
                               __uint_as_float(xr.x & 0xffff0000u) + __uint_as_float(v.x & 0xffff0000u)),
                dl_pack_bf16x2(__uint_as_float(xr.y << 16) + __uint_as_float(v.y << 16),
                               __uint_as_float(xr.y & 0xffff0000u) + __uint_as_float(v.y & 0xffff0000u))};
    }
    constexpr uint32_t kNaN2 = 0x7fc07fc0u;
    dl_store8(dst + (int64_t)m * U.ldo + n, poison ? u32x2{kNaN2, kNaN2} : v);
  }
  if (ready) {
    // a second round of arrivals, each after the split's share is stored,
    // the last of which marks the tile ready: on a counter of its own (on
    // `cnt` a split could arrive again before a slower one saw the first
    // round's zero, which that one would then never see)
    dl_wait_vm<0>();
    dl_block_sync();
    if (threadIdx.x == 0 && dl_arrive_wrap(cnt2, splits))
      __hip_atomic_store(ready, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return issued;
}

// ---------------------------------------------------------------------------
// Phase 4 at one token tile without a K split (DecLayerParams::p4narrow):
// block b owns 16 columns of y over the whole rank, so no block waits for
// another's partial sums at the end.  Its Vd strip (r_d k-rows x 32 bytes,
// 88 KB at the 8B shape) is brought into LDS whole, by DMAs issued as soon
// as the block's previous phase ends; once the XU_d tiles' ready flags are
// set, each wave loads its 1/8 of the k range of XU_d straight into
// registers (16 bytes per lane and 32-k chunk, the MFMA's B operand: rows
// past T are zeros, not loaded) and runs its MFMAs, and the 8 waves' sums
// are added through LDS in wave order.
// ---------------------------------------------------------------------------

// Columns of block b: 16-column tile c = 4q + r, where the four tiles of a
// 64-column group q (one 128-byte piece of a Vd row) go to blocks on one XCD
// (block b runs on XCD b % 8), so that XCD's L2 fetches each line once.
__device__ __forceinline__ int dl_narrow_tile(int b, int G) {
  if (G != 256) return b;
  const int x = b % 8, rest = b / 8, r = rest % 4, qh = rest / 4;
  return 4 * (x + 8 * qh) + r;
}

// LDS byte of (k-row, 16-byte half) of the strip: 32-byte rows, 1 KB per
// 32-k chunk, bit 7 flipped for rows whose bit 3 is set.  A transposing
// read's lanes 0-15 touch rows k0..k0+3 and lanes 16-31 rows k0+8..k0+11:
// 128 bytes each, which the flip puts on the two halves of the 64 banks.
__device__ __forceinline__ uint32_t dl_narrow_swz(uint32_t o) { return o ^ (((o >> 8) & 1u) << 7); }

constexpr int kDlNarrowMaxChunks = 128;  // r_d <= 4096

// DMAs of the strip of columns n0..n0+15 into LDS bytes [0, r_d * 32):
// chunk ch (32 k-rows) by wave ch % 8, one 1 KB instruction each.
__device__ __forceinline__ void dl_narrow_dma(const DlCtx& c, const DecLayerParams& p, int n0) {
  const int nch = p.r_d / 32;
  const i32x4 rs = make_rsrc_sgpr(p.vd, (uint32_t)((int64_t)p.r_d * p.ld_vd * 2));
  const uint32_t ol = dl_narrow_swz(16u * (uint32_t)c.lane);  // logical byte of the lane's LDS slot
  const uint32_t row = ol >> 5, half = (ol >> 4) & 1u;
  const uint32_t voff = row * (uint32_t)p.ld_vd * 2u + (uint32_t)(n0 + 8 * (int)half) * 2u;
  for (int ch = c.wave; ch < nch; ch += 8)
    dma16(rs, voff, (uint32_t)(32 * ch) * (uint32_t)p.ld_vd * 2u, c.lbase + 1024u * (uint32_t)ch);
}

// The unit: the strip's DMAs were issued (dl_narrow_dma) and the XU_d
// tiles are ready.  y (row pitch d) = bf16 of the sum, with `resid` added
// as in dl_combine; NaN where `poison`.  The wave's chunks go in batches of
// NB, whose MT * NB activation loads per lane (16) are in flight at once.
template <int MT>
__device__ __forceinline__ void dl_narrow_unit(const DlCtx& c, const DecLayerParams& p, char* lds, int n0,
                                               bool poison, const uint16_t* resid) {
  constexpr int NB = 16 / MT;
  const int nch = p.r_d / 32, per = (nch + 7) / 8;
  const int ch0 = c.wave * per;
  // XU_d rows through the caches where the workspace is 128-byte aligned (as
  // the ring's activation DMAs), device-scope otherwise; rows past T and
  // chunks past the wave's range read zeros (an offset past the records)
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc(p.xd16, 0, (int)((int64_t)c.T * p.r_d * 2), 0x00020000);
  // transposing reads: lane s of group lg points at row 8 lg + s / 4 (+ 4 for
  // the upper half) of the chunk, bytes 8 (s % 4)
  const uint32_t lo_off = (uint32_t)(8 * c.lg + (c.lr >> 2)) * 32u + 8u * (uint32_t)(c.lr & 3);
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int i0 = 0; i0 < per; i0 += NB) {
    u32x4 fa[NB][MT];
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int ch = ch0 + i0 + i, m = 16 * mt + c.lr;
        const uint32_t off = (i0 + i < per && ch < nch && m < c.T)
                                 ? (uint32_t)(((int64_t)m * p.r_d + 32 * ch + 8 * c.lg) * 2)
                                 : kDlPastSlices;
        fa[i][mt] = c.a_cached ? __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0)
                               : __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, kDlSc1);
      }
    dl_wait_vm<0>();  // (the first batch: the strip's DMAs too)
    if (i0 == 0) dl_block_sync();
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int ch = ch0 + i0 + i;
      if (i0 + i < per && ch < nch) {
        const lds_cptr base = c.l0 + 1024 * ch;
        const u32x2 lo = lds_read_tr(base + dl_narrow_swz(lo_off)), hi = lds_read_tr(base + dl_narrow_swz(lo_off + 128u));
        const u32x4 fb = u32x4{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma_chunk(fb, fa[i][mt], acc[mt], __bf16{});
      }
    }
  }
  // the 8 waves' sums, added in wave order through LDS (the strip is read)
  dl_block_sync();
  f32x4* part = reinterpret_cast<f32x4*>(lds);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) part[(c.wave * MT + mt) * 64 + c.lane] = acc[mt];
  dl_block_sync();
  // wave w finishes 16-row blocks w, w + 8, ... (MT <= 8: at most one)
  for (int mt = c.wave; mt < MT; mt += 8) {
    const int m = 16 * mt + c.lr;
    if (m >= c.T) continue;
    f32x4 tot = part[mt * 64 + c.lane];
#pragma unroll
    for (int w = 1; w < 8; ++w) tot += part[(w * MT + mt) * 64 + c.lane];
    const int n = n0 + 4 * c.lg;
    u32x2 v = u32x2{dl_pack_bf16x2(tot.x, tot.y), dl_pack_bf16x2(tot.z, tot.w)};
    if (resid && !poison) {
      const u32x2 xr2 = *reinterpret_cast<const u32x2*>(resid + (int64_t)m * p.d + n);
      v = u32x2{dl_pack_bf16x2(__uint_as_float(xr2.x << 16) + __uint_as_float(v.x << 16),
                               __uint_as_float(xr2.x & 0xffff0000u) + __uint_as_float(v.x & 0xffff0000u)),
                dl_pack_bf16x2(__uint_as_float(xr2.y << 16) + __uint_as_float(v.y << 16),
                               __uint_as_float(xr2.y & 0xffff0000u) + __uint_as_float(v.y & 0xffff0000u))};
    }
    constexpr uint32_t kNaN2 = 0x7fc07fc0u;
    dl_store8(static_cast<uint16_t*>(p.y) + (int64_t)m * p.d + n, poison ? u32x2{kNaN2, kNaN2} : v);
  }
}

// Phase 0 of the MLP block: row `row` of x normalised into xn,
// bf16(gain * (x * rsqrt(mean(x^2) + eps))), LlamaRMSNorm's fp32 formula
// (models/modeling_llama.py:257-262) rounded once.  Each thread holds 8
// elements per 4096 (d <= 4096 * kDlNormPieces), the sum of squares is
// reduced over the block in a fixed order (waves, then the 8 wave sums in
// order, through `part` in LDS), and the row goes out with device-scope
// stores, which phase 1 reads after the next grid barrier.
constexpr int kDlNormPieces = 4;
__device__ __forceinline__ void dl_norm_row(const DecLayerParams& p, char* part_lds, int row) {
  const uint16_t* xr = static_cast<const uint16_t*>(p.x) + (int64_t)row * p.d;
  u32x4 v[kDlNormPieces];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kDlNormPieces; ++i) {
    const int e = 8 * ((int)threadIdx.x + kDlThreads * i);
    v[i] = e < p.d ? *reinterpret_cast<const u32x4*>(xr + e) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float lo = __uint_as_float(v[i][w] << 16), hi = __uint_as_float(v[i][w] & 0xffff0000u);
      ss = fmaf(lo, lo, ss);
      ss = fmaf(hi, hi, ss);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  float* part = reinterpret_cast<float*>(part_lds);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  dl_block_sync();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kDlThreads / 64; ++w) tot += part[w];
  const float rstd = 1.0f / sqrtf(tot / (float)p.d + p.eps);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(p.xn, 0, (int)((int64_t)p.T * p.d * 2), 0x00020000);
#pragma unroll
  for (int i = 0; i < kDlNormPieces; ++i) {
    const int e = 8 * ((int)threadIdx.x + kDlThreads * i);
    if (e < p.d) {
      const f32x4 g0 = *reinterpret_cast<const f32x4*>(p.gain + e), g1 = *reinterpret_cast<const f32x4*>(p.gain + e + 4);
      const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
      u32x4 o;
#pragma unroll
      for (int w = 0; w < 4; ++w)
        o[w] = dl_pack_bf16x2(g[2 * w] * (__uint_as_float(v[i][w] << 16) * rstd),
                              g[2 * w + 1] * (__uint_as_float(v[i][w] & 0xffff0000u) * rstd));
      __builtin_amdgcn_raw_buffer_store_b128(o, rs, (uint32_t)(((int64_t)row * p.d + e) * 2), 0, kDlSc1);
    }
  }
}

// ---------------------------------------------------------------------------
// Contracted layer (phases 2 and 3 fused): unit u computes its 64-column
// strip of h as in phase 2 and keeps it in LDS as the A operand of
// XU_d += h[:, strip] . Ud[strip, :], so h never leaves the block; the
// (T, r_d) partial of every unit goes to the workspace as one fp32 slice per
// 128-column tile, and one otherwise idle block per tile sums the units'
// slices in unit order into bf16 XU_d while the units still stream.
// ---------------------------------------------------------------------------

// LDS byte offset of the h tile (two 32-k chunks of 16 * MT rows of 64
// bytes, A-operand layout) within the activation region, after the 4 KB *
// MT exchange area of the SwiGLU epilogue.
template <int MT>
struct DlH {
  static constexpr int XCH = 4 * MT * 64 * 16;
  static constexpr int OFF = XCH;
  static constexpr int CHUNK = MT * 16 * 64;
  static_assert(OFF + 2 * CHUNK <= DlLds<MT>::NS * DlLds<MT>::A_SLOT, "h tile fits the activation region");
};

// h = bf16(SiLU(g) * u) of the unit's strip into LDS (waves 0..3 hold g,
// waves 4..7 u, for the same lanes' (m, n)).  Column n = 16 * wave + 4 * lg
// + t of the strip is k = n of the down projection: chunk n / 32, 16-byte
// piece (n % 32) / 8 at slot piece ^ a_swz(m) of row m.
template <int MT>
__device__ __forceinline__ void dl_contract_h(const DlCtx& c, char* lds, const f32x4 (&acc)[MT]) {
  using L = DlLds<MT>;
  using H = DlH<MT>;
  f32x4* xch = reinterpret_cast<f32x4*>(lds + L::A_OFF);
  if (c.wave >= 4) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xch[((c.wave - 4) * MT + mt) * 64 + c.lane] = acc[mt];
  }
  dl_block_sync();
  if (c.wave < 4) {
    char* hl = lds + L::A_OFF + H::OFF + (c.wave >> 1) * H::CHUNK;
    const int piece = 2 * (c.wave & 1) + (c.lg >> 1);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + c.lr;
      const f32x4 uv = xch[(c.wave * MT + mt) * 64 + c.lane], g = acc[mt];
      *reinterpret_cast<u32x2*>(hl + m * 64 + ((piece ^ a_swz(m)) << 4) + (c.lg & 1) * 8) =
          u32x2{dl_pack_bf16x2(silu_f32(g.x) * uv.x, silu_f32(g.y) * uv.y),
                dl_pack_bf16x2(silu_f32(g.z) * uv.z, silu_f32(g.w) * uv.w)};
    }
  }
  dl_block_sync();
}

// Byte size of the contracted slices: nt tiles x units x T rows x 128 fp32.
__host__ __device__ constexpr int64_t dl_contract_bytes(int64_t nt, int64_t units, int64_t T) {
  return nt * units * T * 128 * 4;
}

// Weight DMAs (KC = 2 per wave) of stage j of unit u's down half -- tile j:
// 128 columns of Ud's rows 64u .. 64u+63 -- into ring slot `slot`, with
// dl_dma_w's lane geometry (non-DUAL: row 8 * (wave % 4) + lane / 8 of each
// 32-k chunk); stages past the last tile fetch nothing and keep the count.
template <int MT>
__device__ __forceinline__ void dl_contract_dma(const DlCtx& c, const void* ud, int ld_ud, int ff, int u, int NT,
                                                int j, int slot) {
  using L = DlLds<MT>;
  static_assert(L::KC == 2, "one 64-k strip per ring stage");
  const int sub = c.wave >> 2, lu = c.wave & 3;
  const int row = 8 * lu + (c.lane >> 3);
  const int col = 64 * sub + 16 * (((c.lane & 7) >> 1) ^ dl_wswz(row)) + 8 * (c.lane & 1);
  const uint32_t ldb2 = (uint32_t)ld_ud * 2u;
  const uint32_t voff = (uint32_t)row * ldb2 + (uint32_t)col * 2u;
  const bool live = j < NT;  // uniform
  const i32x4 rs = make_rsrc_sgpr(ud, live ? (uint32_t)((int64_t)ff * ld_ud * 2) : 0u);
  const uint32_t k_base = (uint32_t)(64 * u) * ldb2;
#pragma unroll
  for (int kc = 0; kc < 2; ++kc)
    dma16(rs, voff, live ? k_base + (uint32_t)(32 * kc) * ldb2 + (uint32_t)(128 * j) * 2u : 0u,
          c.lbase + L::W_OFF + slot * L::W_SLOT + kc * kDlWStage + sub * 4096 + lu * 1024);
}

// dl_run's run-out hook of a contracted unit: stage nk + i is the down
// half's stage i.
template <int MT>
struct DlContractRunOut {
  static constexpr bool kActive = true;
  DlCtx c;
  const void* ud;
  int ld_ud, ff, u, nt;
  __device__ __forceinline__ void operator()(int i, int slot) const {
    dl_contract_dma<MT>(c, ud, ld_ud, ff, u, nt, i, slot);
  }
};

// The down half of unit u: stage j of the ring (slot (s0 + j) % NS) is tile
// j, multiplied by the h fragments held in registers; the tile's partial is
// stored as slice (j, u) (rows < T, one 16-byte device-scope store per lane
// and 16-row block).  Stages 0..NS-2 were issued during the gate/up run-out
// and have landed (that run ends with a full drain).  Per wave and stage:
// MT stores, then the weight DMAs of stage j + NS - 1, so waiting for stage
// j (NS - 2 stages of MT + 2 operations issued after it) also completes the
// stores of tile j - NS + 1, whose arrival is counted then; the last NS - 1
// tiles arrive after a final drain.  The counter of tile j is cnt0 + j.
template <int MT>
__device__ __forceinline__ void dl_contract_down(const DlCtx& c, const DecLayerParams& p, char* lds, int u, int U2,
                                                 int NT, int cnt0, int s0) {
  using L = DlLds<MT>;
  using H = DlH<MT>;
  constexpr int NS = L::NS, P = MT + 2;
  const int sub = c.wave >> 2, lu = c.wave & 3;
  // h fragments: chunk kc, rows 16 * mt + lr
  u32x4 fa[2][MT];
#pragma unroll
  for (int kc = 0; kc < 2; ++kc)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + c.lr;
      fa[kc][mt] = lds_read_b128(c.l0 + L::A_OFF + H::OFF + kc * H::CHUNK + m * 64 + ((c.lg ^ a_swz(m)) << 4));
    }
  const int k_lo = 8 * c.lg + (c.lr >> 2);
  const int b_off = L::W_OFF + sub * 4096 + k_lo * 128 + ((lu ^ dl_wswz(k_lo)) << 5) + ((c.lr & 3) << 3);
  const int colo = 64 * sub + 16 * lu + 4 * c.lg;
  const __amdgpu_buffer_rsrc_t rs_sl =
      __builtin_amdgcn_make_buffer_rsrc(p.cslices, 0, (int)dl_contract_bytes(NT, U2, c.T), 0x00020000);

  for (int j = 0; j < NT; ++j) {
    dl_wait_vm<(NS - 2) * P>();
    dl_block_sync();
    if (j >= NS - 1 && threadIdx.x == 0)
      __hip_atomic_fetch_add(dl_tile_counter(p.sync, cnt0 + j - (NS - 1)), 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    const int slot = (s0 + j) % NS;
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const lds_cptr wb = c.l0 + slot * L::W_SLOT + kc * kDlWStage + b_off;
      const u32x2 lo = lds_read_tr(wb), hi = lds_read_tr(wb + 512);
      const u32x4 fb = u32x4{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma_chunk(fb, fa[kc][mt], acc[mt], __bf16{});
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + c.lr;
      const uint32_t off =
          m < c.T ? (uint32_t)(((((int64_t)j * U2 + u) * c.T + m) * 128 + colo) * 4) : kDlPastSlices;
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(acc[mt].x), __float_as_uint(acc[mt].y),
                                                   __float_as_uint(acc[mt].z), __float_as_uint(acc[mt].w)},
                                             rs_sl, off, 0, kDlSc1);
    }
    dl_contract_dma<MT>(c, p.ud, p.ld_ud, p.ff, u, NT, j + NS - 1, (s0 + j + NS - 1) % NS);
  }
  dl_wait_vm<0>();
  dl_block_sync();
  if (threadIdx.x < NS - 1) {
    const int t = NT - (NS - 1) + (int)threadIdx.x;
    if (t >= 0)
      __hip_atomic_fetch_add(dl_tile_counter(p.sync, cnt0 + t), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Tile j of XU_d from the U2 units' slices: the block waits (bounded, as at
// a grid barrier) until all U2 units have counted their slice of the tile,
// resets the counter, and sums in a fixed order: with R the power of two
// >= T and G = 16 / R, thread i takes float4 column q = i % 32 of row
// m = (i / 32) / G and units g, g + G, g + 2G, ... (g = (i / 32) % G), 16
// loads in flight, then the G partial sums of each (m, q) are added in g
// order through LDS; XU_d is rounded to bf16 once.
constexpr uint32_t kDlFarArrivals = 16;
template <int MT>
__device__ __forceinline__ void dl_contract_combine(const DlCtx& c, const DecLayerParams& p, char* lds, int j, int U2,
                                                    int cnt0, uint32_t spin_reg, const uint32_t* spin_lds, int* bad,
                                                    uint64_t epoch) {
  using L = DlLds<MT>;
  static_assert(kDlThreads == 512, "16 groups of 32 threads");
  if (threadIdx.x == 0) {
    uint32_t* cnt = dl_tile_counter(p.sync, cnt0 + j);
    const uint32_t spin = spin_lds ? *spin_lds : spin_reg;
    uint32_t polls = 0;
    uint32_t seen;
    while ((seen = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) < (uint32_t)U2) {
      __builtin_amdgcn_s_sleep(1);
      // Polls slow the units' weight stream (8B layer at T=1: the slowest
      // unit 2.7 us later with a poll every ~0.1 us from all 22 combining
      // blocks), so poll every ~1 us while more than kDlFarArrivals are
      // missing: 68.7 -> 67.2 us per layer.
      if ((uint32_t)U2 - seen > kDlFarArrivals)
        for (int z = 0; z < 4; ++z) __builtin_amdgcn_s_sleep(8);
      if (++polls >= spin) {
        __hip_atomic_fetch_or(&p.sync[kDlFlag], (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_or(&p.sync[kGvDone], kGvDoneBad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        dl_wait_vm<0>();
        *bad = 1;
        break;
      }
    }
    // every arrival of this launch is in (or the wait gave up): back to zero
    // for the next launch (a late arrival after a give-up leaves it nonzero,
    // as the timeout flag does; the caller resets the area)
    __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  dl_block_sync();
  const int R = c.T <= 1 ? 1 : (c.T <= 2 ? 2 : (c.T <= 4 ? 4 : (c.T <= 8 ? 8 : 16)));
  const int G = 16 / R;
  const int q = threadIdx.x & 31, grp = threadIdx.x >> 5, m = grp / G, g = grp % G;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(p.cslices, 0, (int)dl_contract_bytes(p.r_d / 128, U2, c.T), 0x00020000);
  f32x4* red = reinterpret_cast<f32x4*>(lds + L::A_OFF);  // 16 x 32 partial sums
  f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
  if (m < c.T) {
    constexpr int B = 16;  // loads in flight per thread
    for (int u0 = g; u0 < U2; u0 += B * G) {
      u32x4 v[B];
#pragma unroll
      for (int i = 0; i < B; ++i) {
        const int uu = u0 + G * i;
        const uint32_t off =
            uu < U2 ? (uint32_t)(((((int64_t)j * U2 + uu) * c.T + m) * 128 + 4 * q) * 4) : kDlPastSlices;
        v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kDlSc1);
      }
#pragma unroll
      for (int i = 0; i < B; ++i) {
        sum.x += __uint_as_float(v[i].x);
        sum.y += __uint_as_float(v[i].y);
        sum.z += __uint_as_float(v[i].z);
        sum.w += __uint_as_float(v[i].w);
      }
    }
  }
  red[grp * 32 + q] = sum;
  dl_block_sync();
  if (g == 0 && m < c.T) {
    f32x4 tot = red[grp * 32 + q];
    for (int gg = 1; gg < G; ++gg) tot += red[(grp + gg) * 32 + q];
    dl_store8(p.xd16 + (int64_t)m * p.r_d + 128 * j + 4 * q,
              u32x2{dl_pack_bf16x2(tot.x, tot.y), dl_pack_bf16x2(tot.z, tot.w)});
  }
  if (epoch) dl_set_ready(p.sync, j, epoch);
}

template <int MT, bool CONTRACT = false, bool NORM = false>
__global__ __launch_bounds__(kDlThreads, 1) void decode_layer_kernel(DecLayerParams p) {
  using L = DlLds<MT>;
  __shared__ __attribute__((aligned(1024))) char lds[L::BYTES];
  DlCtx c;
  c.lbase = lds_addr(lds);
  c.l0 = (lds_cptr)lds;
  c.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  c.lane = threadIdx.x & 63;
  c.lr = c.lane & 15;
  c.lg = c.lane >> 4;
  c.T = p.T;
  c.a_cached = p.a_cached;
  c.pf_full = p.pf_full;
  int* const flag = reinterpret_cast<int*>(lds + L::FLAG_OFF);
  int* const bad = reinterpret_cast<int*>(lds + L::BAD_OFF);
  uint32_t* const spin_lds = MT >= 4 ? reinterpret_cast<uint32_t*>(lds + L::SPIN_OFF) : nullptr;
  uint32_t spin = 0;
  if constexpr (MT < 4) spin = dl_spin_limit(p.sync);
  if (threadIdx.x == 0) {  // published by the block barriers ahead of their first reads
    *bad = 0;
    if constexpr (MT >= 4) *spin_lds = dl_spin_limit(p.sync);
  }
  const int G = gridDim.x, b = blockIdx.x;
  const int T = p.T;
  constexpr int NS = L::NS;
  uint32_t nbar = 0;
  // Generation at launch start: it cannot advance before every block has
  // arrived at barrier 1, which each block does only after this read.
  const uint64_t gen0 = __hip_atomic_load(&p.sync[kDlGen], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // XU_d tiles' ready flags in place of the grid barrier before phase 4
  // (DecLayerParams::xd_ready): this launch's epoch, else 0
  const uint64_t epoch = p.xd_ready ? gen0 + 1 : 0;
  // XU tiles' ready flags in place of the grid barrier before phase 2
  // (DecLayerParams::xu_ready)
  // 1: one flag per XU tile (from two token tiles up), 2: one flag for all
  // of XU, stored by the last of the tiles' writers to count down (one tile)
  const uint64_t xu_epoch = ((MT >= 2 && p.xu_ready == 1) || (MT == 1 && !CONTRACT && p.xu_ready == 2)) ? gen0 + 1 : 0;
  // phase 3's K splits' h flags in place of the grid barrier before phase 3
  // (DecLayerParams::h_ready)
  const uint64_t h_epoch = (MT >= 2 && !CONTRACT && p.h_ready && xu_epoch) ? gen0 + 1 : 0;

  auto unit_of = [&](int phase, int u, DlUnit& U) {
    if (phase == 1) {
      // tiles 0 .. r_gu/128 - 1 of XU_g, then those of XU_u
      const int pg = p.r_gu / 128, nt = pg + p.r_up / 128;
      const int tile = u % nt, split = u / nt, br = tile >= pg;
      U.a0 = U.a1 = NORM ? static_cast<const void*>(p.xn) : p.x;
      U.lda = p.d;
      U.a_bytes = (uint32_t)((int64_t)T * p.d * 2);
      U.b0 = U.b1 = br ? p.uu : p.ug;
      U.ldb = br ? p.ld_uu : p.ld_u;
      U.b_bytes = (uint32_t)((int64_t)p.d * U.ldb * 2);
      U.n0 = (br ? tile - pg : tile) * 128;
      U.kb = split * p.ks1;
      U.ke = min(p.d, U.kb + p.ks1);
      U.dst = p.xu16 + (br ? (int64_t)T * p.r_gu : 0);
      U.ldo = br ? p.r_up : p.r_gu;
    } else if (phase == 2 && p.p2split) {
      // each branch over its own rank
      const int br = u & 1, rk = br ? p.r_up : p.r_gu;
      U.a0 = U.a1 = p.xu16 + (br ? (int64_t)T * p.r_gu : 0);
      U.lda = rk;
      U.a_bytes = (uint32_t)((int64_t)T * rk * 2);
      U.b0 = U.b1 = br ? p.vu : p.vg;
      U.ldb = br ? p.ld_vu : p.ld_v;
      U.b_bytes = (uint32_t)((int64_t)rk * U.ldb * 2);
      U.n0 = (u >> 1) * 128;
      U.kb = 0;
      U.ke = rk;
      U.dst = p.h;
      U.ldo = p.ff;
    } else if (phase == 2) {  // both branches of 64 columns: one rank (r_up == r_gu), one V pitch
      U.a0 = p.xu16;
      U.a1 = p.xu16 + (int64_t)T * p.r_gu;
      U.lda = p.r_gu;
      U.a_bytes = (uint32_t)((int64_t)T * p.r_gu * 2);
      U.b0 = p.vg;
      U.b1 = p.vu;
      U.ldb = p.ld_v;
      U.b_bytes = (uint32_t)((int64_t)p.r_gu * p.ld_v * 2);
      U.n0 = u * 64;
      U.kb = 0;
      U.ke = p.r_gu;
      U.dst = p.h;
      U.ldo = p.ff;
    } else if (phase == 3) {
      const int nt = p.r_d / 128;
      const int tile = u % nt, split = u / nt;
      U.a0 = U.a1 = p.h;
      U.lda = p.ff;
      U.a_bytes = (uint32_t)((int64_t)T * p.ff * 2);
      U.b0 = U.b1 = p.ud;
      U.ldb = p.ld_ud;
      U.b_bytes = (uint32_t)((int64_t)p.ff * p.ld_ud * 2);
      U.n0 = tile * 128;
      U.kb = split * p.ks3;
      U.ke = min(p.ff, U.kb + p.ks3);
      U.dst = p.xd16;
      U.ldo = p.r_d;
    } else {
      const int nt = p.d / 128;
      const int tile = u % nt, split = u / nt;
      U.a0 = U.a1 = p.xd16;
      U.lda = p.r_d;
      U.a_bytes = (uint32_t)((int64_t)T * p.r_d * 2);
      U.b0 = U.b1 = p.vd;
      U.ldb = p.ld_vd;
      U.b_bytes = (uint32_t)((int64_t)p.r_d * p.ld_vd * 2);
      U.n0 = tile * 128;
      U.kb = split * p.ks4;
      U.ke = min(p.r_d, U.kb + p.ks4);
      U.dst = static_cast<uint16_t*>(p.y);
      U.ldo = p.d;
    }
  };
  const int units[5] = {0, p.units1, p.units2, p.units3, p.units4};
  // The first NS - 1 weight stages of this block's first unit of `phase`,
  // issued at the barrier ahead of it, once the block has arrived.
  // phase 4's first weights: the narrow unit's whole strip (p4narrow), else
  // the ring's first stages
  const bool narrow4 = MT == 1 && p.p4narrow;  // (from two tiles up every unit would load all of XU_d: T=64 +5 us)
  auto prefetch_w_ring = [&](int phase) {
    if (b < units[phase]) {
      DlUnit U;
      unit_of(phase, b, U);
      // the last ring slot too (pf_full) where the unit has that stage: dl_run
      // then issues no weights at its step 0
      const int ns = DlDepth<MT>::PF_FULL && p.pf_full && NS - 1 < dl_stages<MT>(U) ? NS : NS - 1;
      for (int s = 0; s < ns; ++s) {
        if (phase == 2 && !p.p2split)
          dl_dma_w<MT, true>(c, U, s, s);
        else
          dl_dma_w<MT, false>(c, U, s, s);
      }
    }
  };
  auto prefetch_w = [&](int phase) {
    if (phase == 4 && narrow4)
      dl_narrow_dma(c, p, 16 * dl_narrow_tile(b, G));
    else
      prefetch_w_ring(phase);
  };
  auto prefetch4 = [&] { prefetch_w(4); };
  // pre_done: the block already issued those DMAs (dl_combine_dist)
  auto grid_sync = [&](int next_phase, bool pre_done = false) {
    dl_grid_sync(p.sync, gen0, ++nbar, spin, spin_lds, bad, [&] {
      if (!pre_done) prefetch_w(next_phase);
    });
  };
  // Split-K combination of unit u of a split phase: by all the tile's
  // splits (dl_combine_dist) or by its last one (dl_combine); `next` is the
  // phase whose first weight stages a waiting split issues (0: none).
  // `ready`: the tile's ready flag, set to `rep` once the tile is written; a
  // tile that all its splits write counts their second arrivals on the
  // counters from `cnt2` (phase 1: the XU tiles, phase 3: the XU_d tiles).
  // `bank`: the phase's slice bank (kDlBank24 for phases 2 and 4, else 0).
  auto combine = [&](const DlUnit& U, f32x4(&acc)[MT], int u, int nt, int splits, int cnt_base, bool out_y,
                     int next, int bank, uint64_t* ready = nullptr, uint64_t rep = 0, int cnt2 = 0) -> bool {
    uint32_t* cnt = dl_tile_counter(p.sync, cnt_base + u % nt);
    float* const slices = p.slices + (size_t)bank * kDlMaxGrid * MT * 2048;
    const uint16_t* resid = out_y ? static_cast<const uint16_t*>(p.resid) : nullptr;
    if constexpr (MT >= 2) {
      if (p.dist && splits > 1)
        return dl_combine_dist<MT>(c, U, acc, u, nt, splits, cnt, slices, flag, U.dst, out_y, bad, p.sync,
                                   spin_lds ? *spin_lds : spin, resid, [&] {
                                     if (next == 0 || u + G < units[next - 1] || !((p.pre_wait >> (next == 2 ? 0 : 1)) & 1))
                                       return false;
                                     prefetch_w(next);
                                     return true;
                                   }, ready, rep, dl_tile_counter(p.sync, cnt2 + u % nt));
    }
    dl_combine<MT>(c, U, acc, u, nt, splits, cnt, slices, flag, U.dst, out_y, out_y && *bad != 0, p.sync, resid);
    if (ready && (splits == 1 || *flag)) {  // this block wrote the tile
      if (MT == 1 && p.xu_ready == 2) {
        // one flag for all tiles: the last writer to arrive stores it
        dl_wait_vm<0>();
        dl_block_sync();
        if (threadIdx.x == 0 && dl_arrive_wrap(dl_tile_counter(p.sync, p.cnt2), nt))
          __hip_atomic_store(ready, xu_epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        dl_set_ready(ready, xu_epoch);
      }
    }
    return false;
  };

  const int nt1 = p.r_gu / 128 + p.r_up / 128, nt3 = p.r_d / 128, nt4 = p.d / 128;

  // ---- phase 0 (the MLP block): xn = RMSNorm(x), row b by block b, which
  // sets the row's ready flag; phase 1's first weight stages stream in while
  // its units wait for the T rows' flags (instead of a grid barrier: T=1
  // block 70.0 -> 68.x us) ----
  if constexpr (NORM) {
    if (b < T) {
      dl_norm_row(p, lds + L::A_OFF, b);
      dl_set_ready(p.sync, kDlRowFlag0 + b, gen0 + 1);
    }
    prefetch_w(1);
  }

  // ---- phase 1: XU_g, XU_u = X . [Ug | Uu] -> bf16 XU ----
  bool pre2 = false;
  for (int u = b; u < units[1]; u += G) {
    DlUnit U;
    unit_of(1, u, U);
    f32x4 acc[MT];
    if (NORM && u == b) dl_wait_ready(p.sync, kDlRowFlag0, kDlRowFlag0 + T - 1, gen0 + 1, spin_lds ? *spin_lds : spin, bad);
    dl_run<MT, false>(c, U, NORM && u == b, acc);
    pre2 = combine(U, acc, u, nt1, p.splits1, 0, false, 2, 0,
                   xu_epoch ? dl_ready_flag(p.sync, p.xu_flag0 + (MT == 1 ? 0 : u % nt1)) : nullptr, xu_epoch,
                   p.cnt2);
  }
  dl_wait_vm<0>();
  if (xu_epoch) {
    if (!pre2) prefetch_w(2);
    if (h_epoch) {  // no grid barrier in this launch: arrive at one for the generation
      ++nbar;
      dl_grid_arrive(p.sync);
    }
  } else {
    grid_sync(2, pre2);
  }
  // phase 2's units read every XU tile of their branch (both branches: -1):
  // wait for their ready flags instead of a grid barrier, once per branch
  int xu_seen = 0;
  auto wait_xu = [&](int br) {
    if (!xu_epoch) return;
    const int need = br < 0 ? 3 : 1 << br;
    if ((xu_seen & need) == need) return;
    const int pg = p.r_gu / 128;
    if (MT == 1)
      dl_wait_ready(p.sync, p.xu_flag0, p.xu_flag0, xu_epoch, spin_lds ? *spin_lds : spin, bad);
    else
      dl_wait_ready(p.sync, p.xu_flag0 + (br == 1 ? pg : 0), p.xu_flag0 + (br == 0 ? pg : nt1) - 1, xu_epoch,
                    spin_lds ? *spin_lds : spin, bad);
    xu_seen |= need;
  };

  if constexpr (CONTRACT) {
    // ---- phases 2 and 3 contracted: unit b < units2 keeps its h strip in
    // LDS and stores partial XU_d tiles; blocks units2 .. units2 + nt3 - 1
    // each sum one tile (the launcher checks that the grid holds both) ----
    const int U2 = units[2];
    if (b < U2) {
      DlUnit U;
      unit_of(2, b, U);
      wait_xu(-1);
      f32x4 acc[MT];
      // the down half's first NS - 1 stages stream in during the gate/up
      // run-out (the launcher checks that the gate/up rank has >= NS - 1 stages)
      const DlContractRunOut<MT> run_out{c, p.ud, p.ld_ud, p.ff, b, nt3};
      dl_run<MT, true>(c, U, true, acc, run_out);
      const int nk = (U.ke - U.kb + 32 * L::KC - 1) / (32 * L::KC);
      dl_contract_h<MT>(c, lds, acc);
      dl_contract_down<MT>(c, p, lds, b, U2, nt3, nt1, nk % NS);
    } else if (b < U2 + nt3) {
      dl_contract_combine<MT>(c, p, lds, b - U2, U2, nt1, spin, spin_lds, bad, epoch);
    }
    dl_wait_vm<0>();
    if (epoch)
      prefetch4();  // phase 4 waits for its XU_d tiles' ready flags instead of a grid barrier
    else
      grid_sync(4);
  } else {
  if (p.p2split) {
    // ---- phase 2, one branch per unit: g or u of 128 columns; the second
    // unit of each pair to finish writes h = bf16(SiLU(g) * u) ----
    for (int u = b; u < units[2]; u += G) {
      DlUnit U;
      unit_of(2, u, U);
      wait_xu(u & 1);
      f32x4 acc[MT];
      dl_run<MT, false>(c, U, u == b, acc);
      uint32_t* pcnt = dl_tile_counter(p.sync, nt1 + nt3 + nt4 + (u >> 1));
      if constexpr (MT >= 2) {
        if (p.dist) {
          dl_swiglu_pair_dist<MT>(c, U, acc, u, pcnt, p.slices + kDlBank24<MT> * kDlMaxGrid * MT * 2048, flag, p.h,
                                  p.sync, spin_lds ? *spin_lds : spin, bad);
          if (h_epoch) {
            // count down on the phase-3 K splits whose columns this pair's h
            // covers (both units of a pair write h); the last of a split
            // sets its flag
            dl_wait_vm<0>();
            dl_block_sync();
            if (threadIdx.x == 0) {
              for (int s = U.n0 / p.ks3; s < p.splits3 && s * p.ks3 < U.n0 + 128; ++s) {
                const int kb = s * p.ks3, ke = min(p.ff, kb + p.ks3);
                if (dl_arrive_wrap(dl_tile_counter(p.sync, p.hc0 + s), 2 * ((ke - 1) / 128 - kb / 128 + 1)))
                  __hip_atomic_store(dl_ready_flag(p.sync, p.hf0 + s), h_epoch, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
              }
            }
          }
          continue;
        }
      }
      dl_swiglu_pair<MT>(c, U, acc, u, pcnt, p.slices + kDlBank24<MT> * kDlMaxGrid * MT * 2048, flag, p.h);
    }
  } else {
  // ---- phase 2: h = bf16(SiLU(XU_g . Vg) * (XU_u . Vu)) ----
  for (int u = b; u < units[2]; u += G) {
    DlUnit U;
    unit_of(2, u, U);
    wait_xu(-1);
    f32x4 acc[MT];
    dl_run<MT, true>(c, U, u == b, acc);
    // waves 4..7 hold u, waves 0..3 g, for the same lanes' (m, n)
    f32x4* xch = reinterpret_cast<f32x4*>(lds + L::A_OFF);
    if (c.wave >= 4) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xch[((c.wave - 4) * MT + mt) * 64 + c.lane] = acc[mt];
    }
    dl_block_sync();
    if (c.wave < 4) {
      const int n = U.n0 + 16 * c.wave + 4 * c.lg;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + c.lr;
        const f32x4 uv = xch[(c.wave * MT + mt) * 64 + c.lane];
        if (m < T) {
          const f32x4 g = acc[mt];
          dl_store8(p.h + (int64_t)m * p.ff + n, u32x2{dl_pack_bf16x2(silu_f32(g.x) * uv.x, silu_f32(g.y) * uv.y),
                                                        dl_pack_bf16x2(silu_f32(g.z) * uv.z, silu_f32(g.w) * uv.w)});
        }
      }
    }
    dl_block_sync();
  }
  }
  dl_wait_vm<0>();
  if (h_epoch)
    prefetch_w(3);
  else
    grid_sync(3);

  // ---- phase 3: XU_d = h . Ud -> bf16 XU_d ----
  bool pre4 = false;
  for (int u = b; u < units[3]; u += G) {
    DlUnit U;
    unit_of(3, u, U);
    if (h_epoch) dl_wait_ready(p.sync, p.hf0 + u / nt3, p.hf0 + u / nt3, h_epoch, spin_lds ? *spin_lds : spin, bad);
    f32x4 acc[MT];
    dl_run<MT, false>(c, U, u == b, acc);
    // from two token tiles up every split writes a share of the tile: the
    // last of their second arrivals sets its flag
    const bool shared = MT >= 2 && p.dist && p.splits3 > 1;
    pre4 = combine(U, acc, u, nt3, p.splits3, nt1, false, 4, 0,
                   epoch && shared ? dl_ready_flag(p.sync, u % nt3) : nullptr, epoch, p.cnt2 + nt1);
    if (epoch && !shared && (p.splits3 == 1 || *flag)) dl_set_ready(p.sync, u % nt3, epoch);  // this block wrote the tile
  }
  dl_wait_vm<0>();
  if (epoch) {
    if (!pre4) prefetch4();
  } else {
    grid_sync(4, pre4);
  }
  }

  // ---- phase 4: y = bf16(XU_d . Vd) ----
  if (narrow4) {
    if (epoch) dl_wait_ready(p.sync, 0, nt3 - 1, epoch, spin_lds ? *spin_lds : spin, bad);
    // (read after every XU_d tile's flag or the barrier: any wait that gave up set it before)
    const bool poison = *bad != 0 || __hip_atomic_load(&p.sync[kDlFlag], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    dl_narrow_unit<MT>(c, p, lds, 16 * dl_narrow_tile(b, G), poison, static_cast<const uint16_t*>(p.resid));
  } else
  for (int u = b; u < units[4]; u += G) {
    DlUnit U;
    unit_of(4, u, U);
    // with the XU_d tiles' flags at one token tile (one slice bank), also
    // that of the tile this block's phase-3 unit stored a slice for: its flag
    // is set once the tile's last split has read every slice, and this
    // unit's slice reuses slice u
    if (epoch)
      dl_wait_ready(p.sync, U.kb / 128, (U.ke - 1) / 128, epoch, spin_lds ? *spin_lds : spin, bad,
                    MT == 1 && !CONTRACT && u == b && b < units[3] ? b % nt3 : -1);
    f32x4 acc[MT];
    dl_run<MT, false>(c, U, u == b, acc);
    combine(U, acc, u, nt4, p.splits4, nt1 + nt3, true, 0, kDlBank24<MT>);
  }
}

}  // namespace svdmlp
