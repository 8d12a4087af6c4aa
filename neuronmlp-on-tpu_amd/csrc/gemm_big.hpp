// Large-tile bf16 MFMA GEMM for the prefill shapes (the hot kernel).
//
//   C[M x N] (+)= A[M x K] . B[K x N]
//
// Block: 512 threads = 8 waves (2 per SIMD) in a 4 (M) x 2 (N) grid; each
// wave owns a 64 x (16*FN) tile of 16x16 MFMA blocks
// (v_mfma_f32_16x16x32_bf16, fp32 accumulate), so the block tile is
// 256 x 32*FN (256 x 224 or 256 x 256).  While one wave of a SIMD waits on
// LDS, its sibling issues MFMAs.
//
// LDS holds 4 stages of 32 k (one MFMA k-step each).  The DMA of a stage
// is issued four steps before its MFMAs, its fragments are read into
// registers one step before, and both are interleaved one instruction per
// MFMA with the current step's MFMAs (sched_barrier-pinned), so a wave
// never holds its MFMAs behind a burst of memory instructions:
//  * A (K contiguous): one 64-byte row per m (four 16-byte chunks), chunk
//    XOR-swizzled by (row >> 1) & 3; an MFMA fragment is one ds_read_b128,
//    free of bank conflicts.
//  * B in the reference's natural (in, out) layout (N contiguous): stored
//    as it lies in HBM, one 512-byte row per k (256 bytes for tiles of at
//    most 128 columns, so no DMA lane fetches past the tile and the freed
//    LDS holds more stages), its 32-byte units XOR-swizzled by bnat_swz(k):
//    the rows a transposing read touches land on distinct banks.  A fragment (16 columns
//    x 8 k) is two ds_read_b64_tr_b16: in each 16-lane group, lane i
//    receives element i % 4 of the 8-byte pieces addressed by lanes
//    i/4 + 4j, so pointing lane s at row k + s/4, columns n + 4*(s % 4)
//    delivers column n + i, rows k..k+3 -- the MFMA operand layout -- with
//    no transpose pass anywhere.
//  * B in PyTorch Linear layout (K contiguous): same as A.
// Global -> LDS is direct (buffer_load ... lds): each lane fetches the
// 16-byte unit that belongs at its LDS slot under the swizzle, so no
// registers hold staged tiles.  Out-of-range lanes use an offset past the
// buffer end and fetch zeros.  The swizzle of a lane's slot does not change
// along K, so each lane keeps one base offset per operand.  Every wave
// issues exactly four 1 KB DMA instructions per stage, so "all but the two
// youngest stages landed" is the constant wait vmcnt(8).
#pragma once

#include <type_traits>

#include "gemm.hpp"

namespace svdmlp {

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
#define SVDMLP_LDS __attribute__((address_space(3)))

constexpr uint32_t kOOB = 0x80000000u;  // offset past any buffer: reads return 0

// Raw buffer descriptor (base, stride 0, num_records = bytes) in SGPRs.
__device__ __forceinline__ i32x4 make_rsrc_sgpr(const void* p, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
  r.z = __builtin_amdgcn_readfirstlane((int)bytes);
  r.w = 0x00020000;
  return r;
}

// LDS byte address of a __shared__ pointer.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)((const SVDMLP_LDS char*)p);
}

// 16 bytes per lane from global (buffer offset `voff` + scalar `soff`,
// past-the-end -> 0) straight into LDS at lds_base + 16 * lane.  Volatile inline asm without a
// memory clobber: the compiler neither serialises it against LDS traffic it
// cannot prove disjoint nor waits on it; ordering comes from the program
// order of volatile asm around s_barrier, and completion is awaited
// explicitly (wait_dma) before the barrier that publishes the stage.
// GFX9 needs one wait state between an SALU write of M0 and an LDS DMA that
// reads it (s_nop 0); the compiler's hazard pass does not look inside asm.
// The descriptor, scalar offset and LDS base are wave-uniform by
// construction; readfirstlane keeps them in SGPRs whatever the compiler's
// uniformity analysis concludes.
__device__ __forceinline__ i32x4 uniform4(i32x4 v) {
  return i32x4{__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
               __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w)};
}

__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
  rsrc = uniform4(rsrc);
  soff = (uint32_t)__builtin_amdgcn_readfirstlane((int)soff);
  lds_base = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_base);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff));
}

// As dma16, but a device-scope (sc1) load: it bypasses the non-coherent
// caches, so it sees data that other XCDs wrote with device-scope stores or
// atomics without any cache maintenance.
__device__ __forceinline__ void dma16_dev(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
  rsrc = uniform4(rsrc);
  soff = (uint32_t)__builtin_amdgcn_readfirstlane((int)soff);
  lds_base = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_base);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen sc1 lds"
               :
               : "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff));
}

template <int N>
__device__ __forceinline__ void wait_dma() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// A-tile chunk swizzle for 64-byte rows.  A ds_read_b128 serves 8 lanes
// (128 bytes, all 32 banks) per cycle; lanes 8q..8q+7 read the same logical
// chunk of 8 consecutive rows.  Rows r and r+2 lie 128 bytes apart (same
// banks), so the XOR must differ between them: (row >> 1) & 3 places the 8
// rows on 8 distinct 16-byte bank groups.
__device__ __forceinline__ int a_swz(int row) { return (row >> 1) & 3; }


typedef const SVDMLP_LDS char* lds_cptr;  // 32-bit LDS address

__device__ __forceinline__ u32x2 lds_read_tr(lds_cptr p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((SVDMLP_LDS bf16x4*)(p)));
}

__device__ __forceinline__ u32x4 lds_read_b128(lds_cptr p) { return *reinterpret_cast<const SVDMLP_LDS u32x4*>(p); }

typedef int i32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

// ds_read_b64_tr_b8: in each 16-lane group, lane i receives byte i % 8 of the
// 8-byte pieces addressed by lanes 2j + i/8 (j = 0..7).  Pointing lane s at
// k-row k + s/2, bytes n + 8*(s % 2) gives lane i column n + i, rows
// k..k+7: the fp8 MFMA operand, 8 consecutive k of one column.
__device__ __forceinline__ u32x2 lds_read_tr8(lds_cptr p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((SVDMLP_LDS i32x2v*)(p)));
}

// 8 fp8 e4m3fn values (k order, bytes of v.x then v.y) widened exactly to 8
// bf16 packed in pairs (every e4m3 value, subnormals and NaN included, is a
// bf16 value; the hardware conversion with scale 1 is exact).
__device__ __forceinline__ u32x4 fp8x8_to_bf16x8(u32x2 v) {
  return u32x4{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v.x, 1.0f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v.x, 1.0f, true)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v.y, 1.0f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v.y, 1.0f, true))};
}

// bf16(a + b) of four bf16 pairs (the residual add of the MLP block).
__device__ __forceinline__ uint32_t add_bf16x2(uint32_t a, uint32_t b) {
  return pack_bf16x2(__uint_as_float(a << 16) + __uint_as_float(b << 16),
                     __uint_as_float(a & 0xffff0000u) + __uint_as_float(b & 0xffff0000u));
}
__device__ __forceinline__ u32x2 add_bf16x4(u32x2 a, u32x2 b) { return u32x2{add_bf16x2(a.x, b.x), add_bf16x2(a.y, b.y)}; }

// LDS on gfx950: 64 banks of 4 bytes; a 64-bit read (ds_read_b64_tr_b16 /
// _b8 included) serves 32 lanes per pass, so lanes 0-15 and 16-31 of a
// transposing read must not share banks (with the k & 3 / k & 7 swizzles
// alone they did, and every such read took two passes: SQ_LDS_BANK_CONFLICT
// equal to the conflict-free active cycles in a probe of the pattern).
//
// 32-byte unit swizzle of a natural-layout bf16 B row k (512- or 256-byte
// rows, which all start at bank 0).  A transposing read's lanes 0-15 touch
// rows k0..k0+3 and lanes 16-31 rows k0+8..k0+11: bits 0-1 put the four
// rows of a group on distinct units of one 128-byte half of the banks, bit
// 2 (k & 8) moves the second group to the other half.
__device__ __forceinline__ int bnat_swz(int k) { return (k & 3) | (((k >> 3) & 1) << 2); }

// 32-byte unit swizzle of a natural-layout bf16 B row k of 384 bytes (the
// 192-column K-group tiles: 12 units, so that four 40 KB stages fit LDS).
// Row k starts at bank group 4 * (k & 1) (of eight 32-byte groups), and
// physical unit p of row k lies in group (4k + p) mod 8.  A transposing
// read's 32 lanes read one logical unit u of rows k0 + {0..3, 8..11}
// (k0 a multiple of 4): XOR with s(k) in 0..3 keeps u inside its aligned
// group of four (a permutation of the 12 units), and s takes four distinct
// values over the even rows and over the odd rows of that set, so the eight
// pieces land on eight distinct bank groups.  s(k + 4) = s(k) and
// s(k + 32) = s(k), as the upper-half and second-K-group reads need.
__device__ __forceinline__ int b384_swz(int k) { return ((k >> 1) & 1) | (((k >> 3) & 1) << 1); }

// 16-byte chunk swizzle of an fp8 natural B row k of 256 bytes (one full
// bank row): lanes 0-15 of a transposing read touch rows k0..k0+7 (bits 0-2
// spread them over 8 chunks) and lanes 16-31 rows k0+8..k0+15 (bit 3, k & 8,
// moves them to the other 8 chunks).
__device__ __forceinline__ int f8nat_swz(int k) { return (k & 7) | (((k >> 3) & 1) << 3); }

// BEPI_STORE_FRAG writes bf16 in fragment order: the 16x16 block (i, j) of
// wave w of output tile t = m_tile + mtiles * n_tile is 512 contiguous bytes
// at element ((t * NW + w) * FM * FN + i * FN + j) * 256 + 4 * lane, so every
// store (and the SwiGLU epilogue's matching load, with p.gfrag) moves one
// contiguous 512-byte piece.  Padded tiles are written too (zeros): the
// buffer holds mtiles * 256 x ntiles * BN elements.
// BEPI_GU_DUAL: the gate/up XU.V passes of one tile in one block, entry 0
// (XU_g . Vg, bf16 g stored to gmem in fragment order) then entry 1 (XU_u .
// Vu, SwiGLU epilogue reading those gate values back): one launch instead of
// two, the same arithmetic.  BEPI_DUAL_F32: the same two passes of one tile
// and K split, each storing its fp32 split-K slice (fragment order; entry 1's
// slices out_bstride elements after entry 0's).
enum BigEpi : int {
  BEPI_STORE = 0,
  BEPI_ATOMIC = 1,
  BEPI_SWIGLU_MEM = 2,
  BEPI_STORE_FRAG = 3,
  BEPI_GU_DUAL = 4,
  BEPI_DUAL_F32 = 5
};

struct BigParams {
  const void* a[2];  // per batch entry
  const void* b[2];
  uint32_t a_bytes[2], b_bytes[2];
  int64_t lda;        // elements
  int64_t ldb[2];     // per batch entry, elements
  void* out;
  int64_t ldo[2];     // per batch entry, elements
  int64_t out_bstride;   // elements from batch entry 0's output to entry 1's
  int64_t out_sstride;   // elements between split-K partial slices (fp32 output)
  const uint16_t* gmem;  // BEPI_SWIGLU_MEM: bf16 gate values, same layout as out
  const float* scale[2]; // fp8 B: one fp32 scale per output column, per batch entry
  const uint16_t* resid; // bf16 STORE epilogue, batch entry 0 (the MLP block's last stage): out = bf16(resid + bf16(C)), row pitch ldo[0]
  int gfrag;             // BEPI_SWIGLU_MEM: gmem holds g in fragment order (BEPI_STORE_FRAG)
  // 16 x 16 block-major bf16 (element (m, n) of a matrix with `cols` columns
  // at ((m / 16) * (cols / 16) + n / 16) * 256 + (m % 16) * 16 + n % 16):
  // out_blk -- the SwiGLU output h (cols = N[0]; one 512-byte block per
  // fragment store); a_blk -- the A operand (cols = K), whose 16-row,
  // 32-k DMA pieces are then 1 KB contiguous
  int out_blk, a_blk;
  int out_frag;          // fp32 output (split-K slices) in fragment order, padded tiles included
  int M, K;
  int N[2];    // output columns per batch entry
  int K1;      // dual launches: entry 1's K (the up rank; K is the gate rank)
  int64_t lda1;  // dual launches: entry 1's A row pitch (elements)
  int k_split1;  // BEPI_DUAL_F32: entry 1's K per split (its split count is entry 0's)
  int mtiles, ntiles;
  // 0: the batch entry is blockIdx.z and both entries have ntiles column
  // tiles; > 0: the grid's z is 1, entry 0 has the first nt0 of the ntiles
  // column tiles and entry 1 the rest (entries of different widths).
  int nt0;
  // tiles > 0: this launch runs tiles tile0 .. tile0 + tiles - 1 (tile = m-tile
  // + mtiles * column tile, both entries' column tiles counted) in every
  // split, its fragment-order outputs compact from tile0; 0: all mtiles x ntiles
  int tile0, tiles;
  int k_split;
};

template <int FN_, bool B_KC_, int EPI_, bool OUT_F32_, bool FP8_B_ = false, int NW_ = 8, int NS_ = 4, int KG_ = 1,
          bool TR_ = false>
struct BigCfg {
  // NW waves per block.  KG = 1: a 2 (n) x NW/2 (m) arrangement over a
  // 256-row tile: a wave's tile is (BM / (NW/2)) x 16*FN, i.e. 64 x 16*FN
  // with 8 waves (two per SIMD) or 128 x 16*FN with 4 (one per SIMD,
  // accumulators in AGPRs), which reads a third less from LDS per MFMA.
  // KG = 2 (K groups): a 128-row tile; the 8 waves form two groups of four
  // 64 x 16*FN wave tiles (2 x 2), group g taking the g-th 32-k half of
  // every 64-k stage, and the two groups' sums are added through LDS at the
  // end.  Each wave keeps the 8-wave tiles' MFMAs and fragment reads per
  // step, while the block tile halves: twice the output tiles, so the rank
  // stages need fewer K splits (or none).
  static constexpr int NW = NW_;
  static constexpr int KG = KG_;
  // TR: the launch may run a tile range (BigParams::tiles).  A separate
  // instance: its block-to-tile arithmetic, compiled into every instance,
  // cost the fp8-B ones ~20 VGPRs and the 256 x 256 fp8-B ones a spill.
  static constexpr bool TR = TR_;
  static constexpr int WT = NW / KG;                 // wave tiles per block
  static constexpr int THREADS = 64 * NW;
  static constexpr int BM = KG == 2 ? 128 : 256;
  static constexpr int FM = BM / (WT / 2) / 16, FN = FN_;  // per wave: 16*FM x 16*FN
  static constexpr bool B_KC = B_KC_;
  static constexpr int EPI = EPI_;
  static constexpr bool DUAL = EPI_ == BEPI_GU_DUAL || EPI_ == BEPI_DUAL_F32;
  static constexpr bool OUT_F32 = OUT_F32_;
  // fp8 e4m3fn B in natural layout: 1-byte elements staged as they lie in
  // HBM, widened to bf16 after the transposing LDS read.
  static constexpr bool FP8_B = FP8_B_;
  static constexpr int BN = 32 * FN, BK = 32 * KG;  // BK: k per stage
  static constexpr int STAGES = NS_;  // LDS stages: NS-2 in flight while one is read
  // A: BM rows of 64 bytes (32 k) per K group: 16 KB either way
  static constexpr int A_SUB = BM * 64;
  static constexpr int A_BYTES = A_SUB * KG;
  // natural-layout B row per k: 256 bytes for fp8 and for bf16 tiles of at most 128 columns, 384 for the
  // 192-column K-group tiles (b384_swz), else 512
  static constexpr int B_PITCH = (FP8_B || (!B_KC && BN <= 128)) ? 256 : ((KG == 2 && BN == 192) ? 384 : 512);
  static constexpr int B_BYTES = B_KC ? 256 * 64 : BK * B_PITCH;  // 16 KB (256-byte rows: 8 KB; Linear: rows >= BN read zeros)
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int A_UNITS = A_BYTES / 1024 / NW;  // DMA instructions per wave: 2 (NW 4: 4)
  static constexpr int B_UNITS = B_BYTES / 1024 / NW;  // 2 (256-byte rows: 1); NW 4: 4 (2); KG 2: twice
  static_assert(NW == 8 || NW == 4, "8 or 4 waves");
  static_assert(KG == 1 || (KG == 2 && NW == 8 && !B_KC && !FP8_B && (EPI == BEPI_STORE || DUAL)),
                "K groups: 8 waves, natural-layout bf16 B, store epilogues (the dual launches' included)");
  static_assert(A_UNITS * NW == 16 && B_UNITS * NW * 1024 == B_BYTES, "DMA instructions per wave and stage");
  static_assert(!(FP8_B && B_KC), "fp8 B is read in natural layout only");
  static_assert(B_KC || BN <= 256, "natural-layout B rows hold at most 256 columns");
  static_assert(B_KC ? BN <= 256 : true, "Linear-layout B tile holds at most 256 rows");
  static_assert(STAGES >= 3 && STAGES * STAGE <= 160 * 1024, "LDS budget");
  // K groups add their sums through LDS: half of each wave's fragments
  static_assert(KG == 1 || NW * (FM / 2) * FN * 1024 <= STAGES * STAGE, "K-group exchange fits the stages' LDS");
};

template <class C>
__global__ __launch_bounds__(C::THREADS, 1) void big_gemm_kernel(BigParams p) {
  constexpr int FM = C::FM, FN = C::FN, BM = C::BM, BN = C::BN, BK = C::BK, NW = C::NW;
  constexpr int NS = C::STAGES;
  // LDS: the A tiles of the NS stages, then their B tiles, so that every
  // fragment read of any stage is one base register plus an immediate offset
  // (16-bit: within 64 KB for 4 stages).
  constexpr int B_REGION = NS * C::A_BYTES;
  __shared__ __attribute__((aligned(1024))) char lds[NS * (C::A_BYTES + C::B_BYTES)];

  // Blocks are dispatched round-robin over the 8 XCDs (each with its own
  // L2).  Remap the linear block id so that each XCD holds a contiguous run
  // of work ordered m-tile fastest, then n-tile, then K split, then batch
  // entry: the blocks of one XCD then share K-range slices of A (same m) and
  // B (same n) in its L2.
  const int nblk = gridDim.x * gridDim.y * gridDim.z;
  int vb = xcd_remap(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z), nblk);
  int m0, nt, t = 0;
  if constexpr (C::TR) {  // tile t = m-tile + mtiles * column tile, from tile0 (tiles 0: all of them)
    const int ntl = p.tiles > 0 ? p.tiles : p.mtiles * p.ntiles;
    t = p.tile0 + vb % ntl;
    vb /= ntl;
    m0 = (t % p.mtiles) * BM;
    nt = t / p.mtiles;
  } else {
    m0 = (vb % p.mtiles) * BM;
    vb /= p.mtiles;
    nt = vb % p.ntiles;
    vb /= p.ntiles;
  }
  const int split = vb % gridDim.y;
  int zb = vb / gridDim.y;
  if (p.nt0 > 0 && nt >= p.nt0) {
    zb = 1;
    nt -= p.nt0;
  }
  // One pass: the tile's k-loop over batch entry zb (K = Kp) and the
  // epilogue EP; a BEPI_GU_DUAL block runs two (below).
  auto run_pass = [&](const int zb, const int Kp, auto epi_c) {
    constexpr int EP = decltype(epi_c)::value;
    const int n0 = nt * BN;
    const int N = p.N[zb];
    const int64_t ldb = p.ldb[zb], ldo = p.ldo[zb];
    const int ksp = C::EPI == BEPI_DUAL_F32 && zb ? p.k_split1 : p.k_split;
    const int kbeg = split * ksp;
    const int kend = min(Kp, kbeg + ksp);
    const int nk = (kend - kbeg + BK - 1) / BK;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lr = lane & 15, lg = lane >> 4;
    // wave tile wt of the block; K group kg (0 with KG = 1)
    constexpr int WT = C::WT;
    const int wt = wave % WT, kg = wave / WT;
    const int wm0 = (wt >> 1) * (16 * FM);
    const int wn0 = (wt & 1) * (BN / 2);

    const i32x4 ra = make_rsrc_sgpr(p.a[zb], p.a_bytes[zb]);
    const i32x4 rb = make_rsrc_sgpr(p.b[zb], p.b_bytes[zb]);
    const uint32_t lda2 = (uint32_t)(C::DUAL && zb ? p.lda1 : p.lda) * 2u, ldb2 = (uint32_t)ldb * 2u;
    const uint32_t lbase = lds_addr(lds);

    // ---- per-lane DMA geometry (constant along K) ----
    // The lane's byte offset without the stage's k (which goes into the
    // instruction's scalar offset), or kOOB for rows / columns outside the
    // matrix.  K and the split length are whole 32-k stages, so a stage lies
    // either below kend or wholly past it; stages past it (the pipeline's
    // run-out) use a descriptor with no records and fetch zeros.
    // A: instruction i of this wave fills LDS rows 16*(wave + NW*i) + lane/4;
    // slot lane%4 holds logical chunk (lane%4) ^ a_swz(row).  With K groups
    // the A region of a stage is KG sub-tiles of BM = 128 rows (16 * NW), one
    // per 32-k half: instruction i fills rows 16*wave + lane/4 of half i.
    const i32x4 r_none = make_rsrc_sgpr(p.a[zb], 0);
    const int a_row0 = 16 * wave + (lane >> 2);
    const int a_kk = 8 * ((lane & 3) ^ a_swz(a_row0));  // k within the stage
    uint32_t a_voff[C::A_UNITS];
#pragma unroll
    for (int i = 0; i < C::A_UNITS; ++i) {
      const int row = m0 + a_row0 + (C::KG == 1 ? 16 * NW * i : 0);
      if (p.a_blk) {  // block (row / 16, k / 16), row % 16, k % 16 (k = a_kk within the stage)
        const uint32_t blk = (uint32_t)(row >> 4) * (uint32_t)(Kp >> 4) + (uint32_t)(a_kk >> 4);
        a_voff[i] = row < p.M ? (blk * 256u + (uint32_t)(row & 15) * 16u + (uint32_t)(a_kk & 15)) * 2u : kOOB;
      } else {
        a_voff[i] = row < p.M ? (uint32_t)row * lda2 + (uint32_t)(a_kk * 2) : kOOB;
      }
    }
    // B natural: instruction i fills LDS k-row 2*(wave + NW*i) + lane/32, slot
    // lane%32 -> logical column 16*((slot/2) ^ swz(row)) + 8*(slot%2).
    // B Linear: like A with rows n.
    uint32_t b_voff[C::B_UNITS];
    if constexpr (C::B_KC) {
      const int row0 = 16 * wave + (lane >> 2);
      const int kk = 8 * ((lane & 3) ^ a_swz(row0));
#pragma unroll
      for (int i = 0; i < C::B_UNITS; ++i) {
        const int row = row0 + 16 * NW * i;
        b_voff[i] = (row < BN && n0 + row < N) ? (uint32_t)(n0 + row) * ldb2 + (uint32_t)(kk * 2) : kOOB;
      }
    } else if constexpr (C::FP8_B) {
      // fp8 natural: instruction i fills k-rows 4*(wave + NW*i) + lane/16
      // (256 bytes each); slot lane%16 holds logical 16-byte chunk
      // (lane%16) ^ f8nat_swz(row), i.e. columns 16 * that chunk .. +15.
#pragma unroll
      for (int i = 0; i < C::B_UNITS; ++i) {
        const int kk = 4 * (wave + NW * i) + (lane >> 4);
        const int col = 16 * ((lane & 15) ^ f8nat_swz(kk));
        b_voff[i] = (col < BN && n0 + col < N) ? (uint32_t)kk * (uint32_t)ldb + (uint32_t)(n0 + col) : kOOB;
      }
    } else if constexpr (C::B_PITCH == 384) {
      // 384-byte rows: instruction i fills bytes (wave + NW*i) KB .. +1 KB of
      // the stage's B tile; the lane's 16 bytes are half (byte >> 4) & 1 of
      // physical unit byte >> 5 of row byte_pos / 384
#pragma unroll
      for (int i = 0; i < C::B_UNITS; ++i) {
        const int pos = (wave + NW * i) * 1024 + 16 * lane;
        const int kk = pos / 384, byte = pos % 384;
        const int col = 16 * ((byte >> 5) ^ b384_swz(kk)) + 8 * ((byte >> 4) & 1);
        b_voff[i] = n0 + col < N ? (uint32_t)kk * ldb2 + (uint32_t)((n0 + col) * 2) : kOOB;
      }
    } else {
      // instruction i fills RPI k-rows from RPI * (wave + NW * i), LPR lanes per
      // row (512-byte rows: 2 rows of 32 lanes; 256-byte rows: 4 of 16)
      // (with 4 waves and 512-byte rows the rows of successive instructions
      // differ by 8, which changes bnat_swz: one column per instruction)
      constexpr int RPI = 1024 / C::B_PITCH, LPR = C::B_PITCH / 16;
      const int q = lane % LPR;
#pragma unroll
      for (int i = 0; i < C::B_UNITS; ++i) {
        const int kk = RPI * (wave + NW * i) + lane / LPR;
        const int col = 16 * ((q >> 1) ^ bnat_swz(kk)) + 8 * (q & 1);
        b_voff[i] = (col < BN && n0 + col < N) ? (uint32_t)kk * ldb2 + (uint32_t)((n0 + col) * 2) : kOOB;
      }
    }

    // DMA instruction d (0, 1: A; 2, 3: B) of stage kt into LDS stage slot s.
    auto dma_one = [&](int kt, int s, int d) {
      const int k0 = kbeg + kt * BK;
      const bool live = k0 < kend;  // uniform
      if (d < C::A_UNITS) {
        // k0 * 2 bytes along a row-major row, k0 * 32 (two 512-byte blocks per 32 k) in block-major A
        const uint32_t kshift = p.a_blk ? 5u : 1u;
        const uint32_t ksub = C::KG == 2 ? (uint32_t)(d * 32) << kshift : 0u;  // 32-k half of the stage (bytes)
        dma16(live ? ra : r_none, a_voff[d], ((uint32_t)k0 << kshift) + ksub, lbase + s * C::A_BYTES + (wave + NW * d) * 1024);
      } else {
        const int i = d - C::A_UNITS;
        const uint32_t soff = C::B_KC ? (uint32_t)k0 * 2u : (C::FP8_B ? (uint32_t)k0 * (uint32_t)ldb : (uint32_t)k0 * ldb2);
        dma16(live ? rb : r_none, b_voff[i], soff, lbase + B_REGION + s * C::B_BYTES + (wave + NW * i) * 1024);
      }
    };
    constexpr int NDMA = C::A_UNITS + C::B_UNITS;

    // ---- fragment read addresses (constant over stages) ----
    // A: rows wm0 + 16i + lr share one swizzle; fragment i of stage s is at
    // a_rd + s * A_BYTES + 1 KB * i.
    const lds_cptr l0 = (lds_cptr)lds;
    // K group kg reads its 32-k half: A sub-tile kg, B k-rows 32*kg ..
    const lds_cptr a_rd = l0 + kg * C::A_SUB + (wm0 + lr) * 64 + ((lg ^ a_swz(wm0 + lr)) << 4);
    // B natural: the lane reads k rows k_lo = 8*lg + lr/4 (and k_lo + 4 for
    // the upper half, same swizzle) in 32-byte unit U = wn0/16 + j for
    // fragment j, stored at unit U ^ bnat_swz(k_lo): fragment j of stage s is
    // at b_rd[j] + s * B_BYTES (+ 2 KB for the upper half).
    // B Linear: like A, fragment j of stage s at b_rd[0] + s * B_BYTES + 1 KB * j.
    lds_cptr b_rd[FN];
    if constexpr (C::B_KC) {
      const int row0 = wn0 + lr;
      b_rd[0] = l0 + B_REGION + row0 * 64 + ((lg ^ a_swz(row0)) << 4);
    } else {
      const int k_lo = 8 * lg + (lr >> 2);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int u = (wn0 >> 4) + j;
        const int pu = C::B_PITCH == 384 ? (u ^ b384_swz(k_lo)) : (u ^ bnat_swz(k_lo));
        b_rd[j] = l0 + B_REGION + (kg * 32 + k_lo) * C::B_PITCH + (pu << 5) + ((lr & 3) << 3);
      }
    }
    // fp8 B: lane s = lr of group lg points at k-row 8*lg + lr/2, bytes
    // 8*(lr & 1) of 16-byte chunk c = wn0/16 + j (fragment j's 16 columns),
    // stored at chunk c ^ f8nat_swz(row); one base per fragment.
    lds_cptr b8[C::FP8_B ? FN : 1];
    if constexpr (C::FP8_B) {
      const int row = 8 * lg + (lr >> 1);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int cc = (wn0 >> 4) + j;
        b8[j] = l0 + B_REGION + row * C::B_PITCH + ((cc ^ f8nat_swz(row)) << 4) + ((lr & 1) << 3);
      }
    }

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Fragment registers: A as one 16-byte read per 16-row block; B as two
    // 8-byte halves (k rows 0-3 and 4-7 of each lane's 8) so that natural and
    // Linear layouts share one schedule (a Linear fragment is one 16-byte
    // read split across the pair).
    struct Frags {
      u32x4 a[FM];
      u32x2 b[2 * FN];
    };
    // Read number r of stage slot s's fragments: A blocks first, then B.
    auto read_one = [&](int s, int r, Frags& f) {
      if (r < FM) {
        f.a[r] = lds_read_b128(a_rd + s * C::A_BYTES + 1024 * r);
      } else if constexpr (C::FP8_B) {
        f.b[r - FM] = lds_read_tr8(b8[r - FM] + s * C::B_BYTES);
      } else if constexpr (C::B_KC) {
        const u32x4 v = lds_read_b128(b_rd[0] + s * C::B_BYTES + 1024 * (r - FM));
        f.b[2 * (r - FM)] = u32x2{v.x, v.y};
        f.b[2 * (r - FM) + 1] = u32x2{v.z, v.w};
      } else {
        const int j = (r - FM) >> 1, hi = (r - FM) & 1;
        f.b[2 * j + hi] = lds_read_tr(b_rd[j] + s * C::B_BYTES + hi * 4 * C::B_PITCH);
      }
    };
    constexpr int NREAD = FM + ((C::B_KC || C::FP8_B) ? FN : 2 * FN);
    // fp8 B: fragment j widened to bf16 once per step (fbw[j]), interleaved
    // with the first FN MFMAs, which are the first to use them.
    u32x4 fbw[C::FP8_B ? FN : 1];
    auto mfma_one = [&](int m, const Frags& f) {
      const int i = m / FN, j = m % FN;
      if constexpr (C::FP8_B) {
        if (m < FN) fbw[j] = fp8x8_to_bf16x8(f.b[j]);
        acc[i][j] = mfma_chunk(fbw[j], f.a[i], acc[i][j], __bf16{});
      } else {
        const u32x2 lo = f.b[2 * j], hi = f.b[2 * j + 1];
        acc[i][j] = mfma_chunk(u32x4{lo.x, lo.y, hi.x, hi.y}, f.a[i], acc[i][j], __bf16{});
      }
    };

    // Stage kt sits in slot kt % NS.  Step kt runs the MFMAs of stage kt
    // (fragments already in registers, read in step kt-1) and, interleaved
    // one per MFMA so that no wave holds its MFMAs behind a burst of memory
    // instructions:
    //  * the fragment reads of stage kt+1;
    //  * the DMA of stage kt+NS into slot kt % NS, free since every wave's
    //    reads of stage kt completed before the barrier that ended step kt-1.
    // Then it waits until stage kt+2 landed (stages kt+3 .. kt+NS may still be
    // in flight: (NS-2) * NDMA instructions) and meets the other waves at the
    // barrier.  DMAs past kend fetch zeros and keep the per-wave count
    // constant.  The sched_barriers pin this instruction order.
    Frags f0, f1;
    constexpr int NMFMA = FM * FN;
    static_assert(NREAD <= NMFMA && NDMA <= NMFMA / 2, "one fragment read per MFMA slot");
    auto step = [&](int kt, int s, const Frags& cur, Frags& nxt) {
#pragma unroll
      for (int m = 0; m < NMFMA; ++m) {
        if (m < NREAD) read_one((s + 1) % NS, m, nxt);
#pragma unroll
        for (int d = 0; d < NDMA; ++d)
          if (m == d * NMFMA / NDMA + 1) dma_one(kt + NS, s, d);
        mfma_one(m, cur);
        __builtin_amdgcn_sched_barrier(0);
      }
      wait_dma<(NS - 2) * NDMA>();
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
    };

    if (nk > 0) {
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int d = 0; d < NDMA; ++d) dma_one(s, s, d);
      wait_dma<(NS - 2) * NDMA>();  // stages 0 and 1 landed
      __syncthreads();
#pragma unroll
      for (int r = 0; r < NREAD; ++r) read_one(0, r, f0);
      __syncthreads();  // every wave holds stage 0 before step 0 refills its slot
      __builtin_amdgcn_sched_barrier(0);
    }
    // unrolled over the slot cycle and the f0/f1 alternation
    constexpr int UNROLL = NS % 2 ? 2 * NS : NS;
    for (int kt = 0; kt < nk; kt += UNROLL) {
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        if (kt + u < nk) {
          if (u % 2 == 0)
            step(kt + u, u % NS, f0, f1);
          else
            step(kt + u, u % NS, f1, f0);
        }
      }
    }
    wait_dma<0>();  // drain DMAs of stages past the end before the block exits

    // K groups: add the two groups' sums.  Group g finishes fragment rows
    // [g * FM/2, (g+1) * FM/2) of its wave tile: it stores the other half to
    // LDS (1 KB per fragment, lane-contiguous) for its partner wave (same wave
    // tile, other group) and adds the partner's half of its own rows.  fp32
    // addition commutes, so both sides of a pair compute the same bits.
    if constexpr (C::KG == 2) {
      constexpr int H = FM / 2;
      __syncthreads();  // every wave's reads of the last stages are done
      SVDMLP_LDS char* const lw = (SVDMLP_LDS char*)lds;
      SVDMLP_LDS char* const xw = lw + ((wt * 2 + kg) * H * FN) * 1024 + 16 * lane;  // this wave's outgoing half
      const lds_cptr xr = l0 + ((wt * 2 + (kg ^ 1)) * H * FN) * 1024 + 16 * lane;     // the partner's
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          if ((i / H) != kg) *reinterpret_cast<SVDMLP_LDS f32x4*>(xw + ((i % H) * FN + j) * 1024) = acc[i][j];
      __syncthreads();
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          if ((i / H) == kg) acc[i][j] += *reinterpret_cast<const SVDMLP_LDS f32x4*>(xr + ((i % H) * FN + j) * 1024);
    }

    // ---- epilogue: lane holds D[n = 4*lg + t][m = lr] of each 16x16 block ----
    const size_t esz = (C::OUT_F32 || EP == BEPI_ATOMIC) ? 4 : 2;
    char* outp = reinterpret_cast<char*>(p.out) + ((int64_t)zb * p.out_bstride + (int64_t)split * p.out_sstride) * esz;
    constexpr bool FRAG = EP == BEPI_STORE_FRAG;
    // fp32 split-K slices in fragment order: every lane's 16 bytes of a
    // fragment are contiguous with its neighbours' (the row-major stores write
    // 16 rows x 64 bytes per instruction; 8B layer: epilogue 9.1K -> 6K cycles)
    const bool ffrag = C::OUT_F32 && p.out_frag;
    // fragment-order element offset of this lane's block (0, 0): tiles in
    // (m-tile, column tile) order per batch entry, or, in a tile-range launch,
    // the launch's tiles in order from its first (entries included, out_bstride 0)
    const int64_t ftl = C::TR && p.tiles > 0 ? (int64_t)(t - p.tile0) : (int64_t)(m0 / BM) + (int64_t)p.mtiles * (n0 / BN);
    const int64_t frag0 = ((ftl * WT + wt) * FM * FN) * 256 + 4 * lane;
    // SwiGLU: every gate value of the wave's tile is loaded before the first
    // h store (the stores could alias the loads as far as the compiler knows,
    // which would serialise one load round trip per fragment); the main
    // loop's fragment registers are free by now.
    u32x2 gv[EP == BEPI_SWIGLU_MEM ? FM : 1][EP == BEPI_SWIGLU_MEM ? FN : 1];
    if constexpr (EP == BEPI_SWIGLU_MEM) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int m = m0 + wm0 + 16 * i + lr;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int n = n0 + wn0 + 16 * j + 4 * lg;
          // Unconditional loads (fragment order covers the padded tile; a
          // row-major g is read at a clamped in-bounds address) so that all of
          // them issue before the first store: a load under a branch left a
          // vmcnt(0) per fragment, which also waited for every earlier h store.
          const int64_t fo = frag0 + (int64_t)(i * FN + j) * 256;
          const bool in = m < p.M && n < N;
          const u32x2 g = *reinterpret_cast<const u32x2*>(p.gmem + (p.gfrag ? fo : (in ? (int64_t)m * ldo + n : 0)));
          gv[i][j] = in ? g : u32x2{0u, 0u};
        }
      }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if (C::KG == 2 && (i / (FM / 2)) != kg) continue;  // the partner wave's rows
      const int m = m0 + wm0 + 16 * i + lr;
      if (!FRAG && !ffrag && m >= p.M) continue;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn0 + 16 * j + 4 * lg;
        if (!FRAG && !ffrag && n >= N) continue;  // N % 8 == 0: n < N implies n + 3 < N
        f32x4 v = acc[i][j];
        if constexpr (C::FP8_B)
          if (n < N) v *= *reinterpret_cast<const f32x4*>(p.scale[zb] + n);  // per-column dequant
        const int64_t fo = frag0 + (int64_t)(i * FN + j) * 256;
        if constexpr (FRAG) {
          // (a dual block's gate values go to gmem, its own buffer)
          uint16_t* const fout = C::EPI == BEPI_GU_DUAL ? const_cast<uint16_t*>(p.gmem) : reinterpret_cast<uint16_t*>(p.out);
          *reinterpret_cast<u32x2*>(fout + fo) = u32x2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
          continue;
        }
        const int64_t o = (int64_t)m * ldo + n;
        if constexpr (EP == BEPI_ATOMIC) {
          float* op = reinterpret_cast<float*>(outp) + o;
          unsafeAtomicAdd(op + 0, v.x);
          unsafeAtomicAdd(op + 1, v.y);
          unsafeAtomicAdd(op + 2, v.z);
          unsafeAtomicAdd(op + 3, v.w);
        } else if constexpr (C::OUT_F32) {
          *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(outp) + (ffrag ? fo : o)) = v;
        } else if constexpr (EP == BEPI_SWIGLU_MEM) {
          const u32x2 g = gv[i][j];
          const float g0 = bf16_bits_to_f32(g.x & 0xffffu), g1 = bf16_bits_to_f32(g.x >> 16);
          const float g2 = bf16_bits_to_f32(g.y & 0xffffu), g3 = bf16_bits_to_f32(g.y >> 16);
          const int64_t ob = p.out_blk ? (((int64_t)(m >> 4) * (N >> 4) + (n >> 4)) * 256 + (m & 15) * 16 + (n & 15)) : o;
          *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(outp) + ob) =
              u32x2{pack_bf16x2(silu_f32(g0) * v.x, silu_f32(g1) * v.y),
                    pack_bf16x2(silu_f32(g2) * v.z, silu_f32(g3) * v.w)};
        } else {
          u32x2 ov = u32x2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
          if (p.resid) ov = add_bf16x4(*reinterpret_cast<const u32x2*>(p.resid + o), ov);
          *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(outp) + o) = ov;
        }
      }
    }
  };
  if constexpr (C::DUAL) {
    constexpr bool F = C::EPI == BEPI_DUAL_F32;
    run_pass(0, p.K, std::integral_constant<int, F ? BEPI_STORE : BEPI_STORE_FRAG>{});
    // every wave's LDS reads of the first pass are complete before the
    // second pass's first DMAs refill the ring; its gate-value stores are
    // read back by the same lanes
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();
    run_pass(1, p.K1, std::integral_constant<int, F ? BEPI_STORE : BEPI_SWIGLU_MEM>{});
  } else {
    run_pass(zb, p.K, std::integral_constant<int, C::EPI>{});
  }
}

}  // namespace svdmlp
