// C ABI of libsvdmlp.so (declared in include/svdmlp.h).
//
// Kernel choice per call (svdmlp_svd_mlp and its variants):
//   1 token (padded V rows), 1-3 (dense factors whose shape the MFMA
//   layer's one-branch phase 2 does not fit), bf16, aligned, or up to 4
//   on request (SVDMLP_CONTRACT):    the contracted decode layer
//                                    (decode_layer.hpp): h kept in LDS, two
//                                    grid barriers
//   1-2 tokens, dense bf16 factors neither that layer nor the one-branch
//   phase 2 takes:                   one streaming-GEMV layer launch
//                                    (decode_gemv.hpp)
//   1-128 tokens, bf16, aligned:     one persistent MFMA decode-layer launch
//                                    (decode_layer.hpp): four phases, three
//                                    grid barriers, split-K tiles combined by
//                                    the last-arriving unit in split order
//   more tokens, bf16/fp8, aligned:  the large-tile MFMA GEMM (gemm_big.hpp)
//                                    X.[Ug|Uu] -> g pass -> u pass with the
//                                    SwiGLU epilogue -> h.Ud -> XUd.Vd; stages
//                                    with too few output tiles split K into
//                                    fp32 slices summed in split order
//   anything else (fp32, Linear-layout or transposed operands, odd sizes):
//                                    the general 128x128 GEMM (gemm.hpp) and
//                                    the per-stage decode kernels (decode.hpp),
//                                    whose split-K sums use fp32 atomics
// Every buffer, including the workspace that holds the rank-r intermediates,
// h and the split-K slices, is owned by the caller.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <array>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include <cstdlib>

#include "dispatch.hpp"
#include "decode_gemv.hpp"
#include "decode_layer.hpp"
#include "gemm_big.hpp"
#include "gemm_f8f8.hpp"
#include "svdmlp.h"

using namespace svdmlp;

namespace {

constexpr int64_t kDecodeMaxT = 64;
// Largest T of the persistent MFMA decode layer (token tiles up to 128 rows):
// at the 8B shape it takes 164 us at T=128 against 221 us for the
// large-tile path, whose XU.V stages have only T/256 x ff/224 blocks there.
constexpr int64_t kDlMaxT = 128;
constexpr int kTargetBlocks = 384;  // ~1.5 blocks per CU on 256 CUs

thread_local std::string g_err;
// Set while svdmlp_svd_mlp_noalloc runs on this thread: the stage profiler
// then records no events (creating one may allocate).
thread_local bool t_no_events = false;

int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return SVDMLP_EINVAL;
}

int check(hipError_t e, const char* what, const char* why = nullptr) {
  if (e == hipSuccess) return SVDMLP_OK;
  if (e == hipErrorInvalidValue && why) return fail("%s: %s", what, why);
  g_err = std::string(what) + ": " + hipGetErrorString(e);
  return SVDMLP_EHIP;
}

// ---------------------------------------------------------------------------
// Optional per-stage GPU timing: hipEvents recorded on the caller's stream
// around each stage launch while enabled (svdmlp_profile_enable).
// ---------------------------------------------------------------------------
enum Stage : int {
  ST_ZERO = 0,
  ST_GU_XU,
  ST_GU_XUV,
  ST_D_XU,
  ST_D_XUV,
  ST_DEC_GU_XU,
  ST_DEC_GU_XUV,
  ST_DEC_D_XU,
  ST_DEC_D_XUV,
  ST_FINALIZE,
  ST_GU_XUV_G,
  ST_DEC_LAYER,
  ST_DEC_GEMV,
  ST_DEC_CONTRACT,
  ST_QUANT,
  ST_D_XU_F8,
  ST_GU_XUV_DUAL,
  ST_COUNT
};
const char* const kStageNames[ST_COUNT] = {
    "zero_fill",        "gate_up_xu",       "gate_up_xuv_swiglu", "down_xu",           "down_xuv",
    "decode_gate_up_xu", "decode_gate_up_xuv", "decode_down_xu",   "decode_down_xuv", "finalize",
    "gate_up_xuv_g",    "decode_layer",       "decode_gemv_layer",  "decode_layer_contracted", "quant_h_e4m3", "down_xu_fp8",
    "gate_up_xuv_dual"
};

struct Profiler {
  std::mutex mu;
  bool on = false;
  struct Rec {
    int stage;
    hipEvent_t a, b;
  };
  std::vector<Rec> pending;
  std::vector<hipEvent_t> pool;
  double total_ms[ST_COUNT] = {};
  int64_t count[ST_COUNT] = {};

  hipEvent_t get() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};
Profiler g_prof;

// Brackets one stage launch with events when profiling is enabled.
struct StageScope {
  int stage;
  hipStream_t st;
  hipEvent_t a = nullptr, b = nullptr;
  StageScope(int s, hipStream_t stream) : stage(s), st(stream) {
    if (t_no_events) return;
    std::lock_guard<std::mutex> g(g_prof.mu);
    if (!g_prof.on) return;
    a = g_prof.get();
    b = g_prof.get();
    if (!a || !b || hipEventRecord(a, st) != hipSuccess) {
      if (a) g_prof.pool.push_back(a);
      if (b) g_prof.pool.push_back(b);
      a = b = nullptr;
    }
  }
  ~StageScope() {
    if (!a) return;
    const bool ok = hipEventRecord(b, st) == hipSuccess;
    std::lock_guard<std::mutex> g(g_prof.mu);
    if (ok) {
      g_prof.pending.push_back({stage, a, b});
    } else {
      g_prof.pool.push_back(a);
      g_prof.pool.push_back(b);
    }
  }
};

size_t a256(int64_t x) { return ((size_t)x + 255) & ~(size_t)255; }

// Token counts the contracted decode layer (SVDMLP_CONTRACT) takes: its
// partial XU_d slices grow with T (8B layer: 2.5 MB per token).  It is the
// default where it is the fastest layer, measured on the 8B layer (one box,
// the better of two 200-step groups each): with padded V rows up to two
// tokens (four-phase layer against contracted: T=1 63.76 vs 63.75 us, T=2
// 66.54 vs 65.47, T=3 66.69 vs 67.44, T=4 67.02 vs 69.10), with dense factors
// up to three (the four-phase layer with one-branch phase-2 units against
// contracted: T=1 72.47 vs 71.05, T=2 71.77 vs 71.04, T=3 73.32 vs 72.82, T=4
// 73.40 vs 74.78; before this round's decode changes the four-phase layer
// was the faster one with dense factors).
constexpr int64_t kDlContractMaxT = 4;
constexpr int64_t kDlContractAutoPadded = 2;
constexpr int64_t kDlContractAutoDense = 3;

struct Ws {
  size_t sync;     // 4 KB of grid-barrier words (zero before first use)
  size_t xu_bf16;  // [2][T][r] bf16 (gate, up) rank-r intermediate
  size_t xu32;     // [3][T][r] fp32 (gate, up, down) split-K accumulators
  size_t gu32;     // [2][T][big] fp32 gate/up sums (decode)
  size_t h;        // [T][big] h of the fused layer (4 bytes/elem worst case)
  size_t y32;      // [T][big] fp32 output accumulator (decode)
  size_t part;     // [splits][batch][T][N] fp32 split-K partial slices (prefill)
  size_t norm;     // [T][d] RMSNorm output of the MLP block (4 bytes/elem worst case)
  size_t g;        // bf16 gate values of the large-tile g pass, fragment order over padded tiles
  size_t slices;   // split-K partial sums of the MFMA decode layer (decode only)
  size_t need;     // bytes every call needs (the regions above)
  size_t cslices;  // partial XU_d tiles of the contracted decode layer (T <= kDlContractMaxT), last: a
                   // workspace without them runs the other decode layers
  size_t total;
};

int plan_splits(int64_t T, int64_t K, int64_t N, int fn, int batch, int kg = 1);
// Tile (columns / 32) and K splits of the split gate/up XU.V passes at one or
// two row tiles of tokens; *splits = 0 where the passes are not split.
void gu_split_plan(int64_t T, int64_t ff, int* fn, int* splits);

// Bytes of split-K partial slices for any call with ranks <= r: the
// large-tile stages X.U (gate/up, batch 2), h.Ud and XU.V (both output
// widths), planned as the launches plan them.  The slice size is not
// monotone in the rank (the split count changes with the tile count), so the
// maximum over every rank up to r (multiples of 8, the large-tile path's
// alignment) is taken; the result is cached per shape.
int64_t part_bytes(int64_t T, int64_t d, int64_t ff, int64_t r) {
  static std::mutex mu;
  static std::map<std::array<int64_t, 4>, int64_t> memo;
  const std::array<int64_t, 4> key{T, d, ff, r};
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = memo.find(key);
    if (it != memo.end()) return it->second;
  }
  int64_t part = 0;
  for (int64_t rr = std::min<int64_t>(r, 8); rr <= r; rr += (rr + 8 <= r ? 8 : std::max<int64_t>(1, r - rr))) {
    // {K, N, batch, fn}: the rank is N of the X.U stages and K of the XU.V stages
    const int64_t stages[][4] = {{d, rr, 2, 8}, {ff, rr, 1, 8}, {rr, d, 1, 8}, {rr, ff, 1, 8}, {rr, d, 1, 4},
                                 {rr, ff, 1, 4}, {d, rr, 2, 4}, {ff, rr, 1, 4}, {d, rr, 2, 6}, {d, rr, 2, 7},
                                 {ff, rr, 1, 6}, {ff, rr, 1, 7}};
    for (const auto& st : stages) {
      const int sp = plan_splits(T, st[0], st[1], (int)st[3], (int)st[2]);
      // slices hold whole 256 x 32*fn tiles (fragment order)
      const int64_t bn = 32 * st[3], tp = (T + 255) / 256 * 256, np = (st[1] + bn - 1) / bn * bn;
      if (sp > 1) part = std::max(part, (int64_t)sp * st[2] * tp * np * 4);
      // the K-group tiles of 128 x 128 and 128 x 192 (whole 128-row tiles)
      if (st[3] == 4 || st[3] == 6) {
        const int sp2 = plan_splits(T, st[0], st[1], (int)st[3], (int)st[2], 2);
        const int64_t tp2 = (T + 127) / 128 * 128;
        if (sp2 > 1) part = std::max(part, (int64_t)sp2 * st[2] * tp2 * np * 4);
      }
    }
    if (rr == r) break;
  }
  // split gate/up XU.V passes at one or two row tiles (big_swiglu)
  int gfn = 0, gsp = 0;
  gu_split_plan(T, ff, &gfn, &gsp);
  // (both passes' slices, side by side)
  if (gsp >= 2)
    part = std::max(part, (int64_t)2 * gsp * ((T + 255) / 256 * 256) * ((ff + 32 * gfn - 1) / (32 * gfn) * (32 * gfn)) * 4);
  // the gate/up X.U split tail (split_tail_plan): its compact slices hold at
  // most one round of 256 x 256 tiles, wherever both branches' tiles at the
  // largest rank exceed a round
  if ((T + 255) / 256 * 2 * ((r + 255) / 256) > 256) part = std::max(part, (int64_t)256 * 256 * 256 * 4);
  std::lock_guard<std::mutex> lk(mu);
  if (memo.size() > 4096) memo.clear();
  memo[key] = part;
  return part;
}

Ws ws_layout(int64_t T, int64_t d, int64_t ff, int64_t r) {
  const int64_t big = std::max(d, ff);
  const bool dec = T <= kDecodeMaxT;
  Ws w;
  size_t off = 0;
  w.sync = off;
  off += 4096;
  static_assert(kDlSyncBytes <= 4096, "barrier words fit the sync area");
  w.xu_bf16 = off;
  off += a256(2 * T * r * 2);
  w.xu32 = off;
  off += a256(3 * T * r * 4);
  w.gu32 = off;
  off += T <= kDlMaxT ? a256(2 * T * big * 4) : 0;
  w.h = off;
  off += a256(T * big * 4);
  w.y32 = off;
  off += a256(T * big * 4);
  // split-K slices serve the large-tile path only, which takes T > kDecodeMaxT
  // (they hold whole 256-row tiles, so sizing them at decode T would also
  // make smaller T ask for more than larger T)
  const int64_t part = dec ? 0 : part_bytes(T, d, ff, r);
  w.part = off;
  off += a256(part);
  w.norm = off;
  off += a256(T * d * 4);
  // the large-tile path serves T > kDecodeMaxT only; its g tiles are 256 rows
  // by 224 or 256 columns
  w.g = off;
  off += dec ? 0 : a256(((T + 255) / 256 * 256) * std::max((big + 223) / 224 * 224, (big + 255) / 256 * 256) * 2);
  w.slices = off;
  off += T <= kDlMaxT ? a256((int64_t)dl_slice_banks(decode_layer_mt((int)T)) * kDlMaxGrid * decode_layer_mt((int)T) * 2048 * 4) : 0;
  w.need = off;
  // the contracted layer's slices: one per (XU_d tile, h strip), T rows each
  w.cslices = off;
  off += (T <= kDlContractMaxT && ff % 64 == 0 && ff / 64 + r / 128 <= kDlMaxGrid)
             ? a256(dl_contract_bytes(r / 128, ff / 64, T))
             : 0;
  w.total = off;
  return w;
}

bool aligned16(const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

// The MLP block around a layer call (svdmlp_svd_mlp_block*): the kernels
// that can take them apply the RMSNorm of x on the fly and the residual add
// in their output stage, and record that they did.
struct Block {
  const void* x;  // block input: RMSNorm input and residual
  const float* gain;
  float eps;
  bool norm_done = false;   // the layer's input is the normalised x
  bool resid_done = false;  // y already holds x + MLP
};

struct Common {
  int act, wt;
  bool f32;
  hipStream_t st;
  Block* blk = nullptr;
};

int check_types(int32_t act, int32_t wt) {
  if (act == SVDMLP_BF16 && (wt == SVDMLP_BF16 || wt == SVDMLP_FP8_E4M3)) return SVDMLP_OK;
  if (act == SVDMLP_F32 && wt == SVDMLP_F32) return SVDMLP_OK;
  return fail("unsupported dtype combination: activations %d, weights %d (supported: bf16/bf16, "
              "bf16/fp8_e4m3, f32/f32)", act, wt);
}

int srcb_of(int wt) { return wt == SVDMLP_FP8_E4M3 ? SRC_FP8 : (wt == SVDMLP_F32 ? SRC_F32 : SRC_BF16); }

int choose_splits(int blocks, int K, int BK, int* k_split) {
  int splits = 1;
  if (blocks < kTargetBlocks) splits = std::min((kTargetBlocks + blocks - 1) / blocks, std::max(1, K / 512));
  int ks = (K + splits - 1) / splits;
  ks = (ks + BK - 1) / BK * BK;
  *k_split = ks;
  return (K + ks - 1) / ks;
}

// ---------------------------------------------------------------------------
// Prefill stages
// ---------------------------------------------------------------------------

// out_b = A . U_b for b < batch (gate/up share A).  Writes bf16 rank-r
// intermediates (xu_bf16) when there are enough tiles, otherwise zeroes and
// accumulates fp32 split-K partials (xu32).  *a_src reports what the next
// stage reads.
int prefill_xu(const Common& c, const Operand& a, bool a_kc, const void* const* u, const float* const* su, bool u_lin,
               int T, int K, int r, int batch, bool vec, char* ws, const Ws& L, int32_t xu_slot, int* a_src,
               const void** xu_out, int64_t* xu_bstride) {
  const int BK = c.f32 ? 32 : 64;
  GemmParams p{};
  for (int b = 0; b < batch; ++b) {
    p.a[b] = a;
    p.b[b] = Operand{u[b], nullptr, u_lin ? K : r};
    p.scale[b] = su ? su[b] : nullptr;
  }
  p.M = T;
  p.N = r;
  p.K = K;
  p.mtiles = (T + kGemmBM - 1) / kGemmBM;
  p.ntiles = (r + kGemmBN - 1) / kGemmBN;
  p.ldo = r;
  p.out_bstride = (int64_t)T * r;
  int k_split = 0;
  const int splits = choose_splits(p.mtiles * p.ntiles * batch, K, BK, &k_split);
  p.k_split = k_split;
  GemmDesc d{c.f32, c.f32 ? SRC_F32 : SRC_BF16, srcb_of(c.wt), a_kc, u_lin, 1, EPI_STORE, false, c.f32, vec};
  float* xu32 = reinterpret_cast<float*>(ws + L.xu32) + (int64_t)xu_slot * T * r;
  if (splits > 1) {
    StageScope z(ST_ZERO, c.st);
    int rc = check(launch_fill_zero(xu32, (int64_t)batch * T * r, c.st), "zero rank-r accumulator");
    if (rc) return rc;
    d.epi = EPI_ATOMIC;
    p.out = xu32;
    *a_src = SRC_F32;
    *xu_out = xu32;
  } else if (c.f32) {
    p.out = xu32;
    *a_src = SRC_F32;
    *xu_out = xu32;
  } else {
    p.out = ws + L.xu_bf16;
    *a_src = SRC_BF16;
    *xu_out = ws + L.xu_bf16;
  }
  *xu_bstride = p.out_bstride;
  const char* why = nullptr;
  StageScope ss(batch == 2 ? ST_GU_XU : ST_D_XU, c.st);
  return check(gemm_launch(d, p, splits, batch, c.st, &why), "XU stage", why);
}

// out = SiLU(XUg . Vg) * (XUu . Vu)
int prefill_swiglu(const Common& c, int a_src, const void* xu, int64_t xu_bstride, const void* vg, const void* vu,
                   const float* svg, const float* svu, bool v_lin, int T, int r, int ff, bool vec, bool out_t,
                   void* out) {
  GemmParams p{};
  const size_t esz = (a_src == SRC_F32) ? 4 : 2;
  p.a[0] = Operand{xu, nullptr, r};
  p.a[1] = Operand{static_cast<const char*>(xu) + xu_bstride * esz, nullptr, r};
  p.b[0] = Operand{vg, nullptr, v_lin ? r : ff};
  p.b[1] = Operand{vu, nullptr, v_lin ? r : ff};
  p.scale[0] = svg;
  p.scale[1] = svu;
  p.out = out;
  p.ldo = out_t ? T : ff;
  p.M = T;
  p.N = ff;
  p.K = r;
  p.mtiles = (T + kGemmBM - 1) / kGemmBM;
  p.ntiles = (ff + kGemmBN - 1) / kGemmBN;
  p.k_split = r;
  GemmDesc d{c.f32, a_src, srcb_of(c.wt), true, v_lin, 2, EPI_SWIGLU, out_t, c.f32, vec};
  const char* why = nullptr;
  StageScope ss(ST_GU_XUV, c.st);
  return check(gemm_launch(d, p, 1, 1, c.st, &why), "gate/up XUV stage", why);
}

// y = XU . V
int prefill_v(const Common& c, int a_src, const void* xu, const void* v, const float* sv, bool v_lin, int T, int r,
              int dout, bool vec, void* y) {
  GemmParams p{};
  p.a[0] = Operand{xu, nullptr, r};
  p.b[0] = Operand{v, nullptr, v_lin ? r : dout};
  p.scale[0] = sv;
  p.out = y;
  p.ldo = dout;
  p.M = T;
  p.N = dout;
  p.K = r;
  p.mtiles = (T + kGemmBM - 1) / kGemmBM;
  p.ntiles = (dout + kGemmBN - 1) / kGemmBN;
  p.k_split = r;
  GemmDesc d{c.f32, a_src, srcb_of(c.wt), true, v_lin, 1, EPI_STORE, false, c.f32, vec};
  const char* why = nullptr;
  StageScope ss(ST_D_XUV, c.st);
  return check(gemm_launch(d, p, 1, 1, c.st, &why), "XUV stage", why);
}

// ---------------------------------------------------------------------------
// Large-tile prefill path (bf16 activations and factors, aligned shapes)
// ---------------------------------------------------------------------------

// Tile choices; SVDMLP_TUNE="s1=44,s4=88,split=256" overrides them (read once).
struct Tune {
  int s1 = 8;         // X.U stages: block tile 256 x 32*s1
  int s1g = 0;        // the gate/up X.U stage alone (0: s1)
  int s4 = 8;         // XU.V of the down half: 256 x 32*s4 (8: split-K over r)
  int s2fn = 0;       // gate/up XU.V tile columns/32 (0 = auto: 4 for T <= 512, else 7 when ff % 224 == 0)
  int split = 256;    // CUs assumed by the split-K planner
  bool big = true;    // large-tile path enabled
  bool dlayer = true; // persistent decode layer enabled
  bool gusplit = true; // split-K gate/up XU.V passes at one row tile
  bool dfn6 = true;    // h.Ud on 256 x 192 tiles where they need no K split and the model rates them cheaper
  bool hblk = true;    // the fused layer's h in 16 x 16 block-major order between the u pass and h.Ud
  bool qblk = true;    // e4m3 h (SVDMLP_FP8_ACT) in 16 x 128 blocks between the quantisation and h.Ud
  bool f8tail = true;  // fp8 x fp8 h.Ud: whole rounds of tiles without a split, K splits for the rest only
  bool xutail = true;  // gate/up X.U with 1-2 rounds of tiles: one round without a split, the rest split
  bool gufuse = true;  // split gate/up XU.V passes: one reduction from both passes' slices
  bool gudual = true;  // gate/up XU.V passes in one launch (each block its g tile or split, then its u one)
  bool gukg = true;    // ... split and at most 128 token rows: 128 x 128 K-group tiles
  int gukgu = 2;       // ... unsplit on 128 x 128 K-group tiles: 1 at 129-256 token rows, 2 while they fit one round
  int dlmin = 1 << 30; // lowest T for the persistent decode layer (min with kDlMinT)
  int gvmax = kGvMaxT; // highest T for the streaming-GEMV decode layer (0: off)
  int gvrw = 1;        // GEMV layer: rows per wave load (1: 1 KB rows, 2: 512-byte rows)
  int nw = 8;          // waves per block of the fn-8 X.U and XU.V stages (8, or 4: faster in isolation, not in the layer)
  bool contract = true; // contracted decode layer by default where it is the fastest (kDlContractAuto*)
  int gusfn = 0;       // split gate/up XU.V passes at one row tile: tile columns / 32 (0: 4)
  int gusp = 0;        // ... and their K splits (0: CUs / tiles, at most 4)
  int f8nw = 4;        // waves per block of the fp8 x fp8 GEMM (4: 70B h.Ud 309 -> 293 us against 8)
  int p2split = 1;     // decode layer phase 2 with one branch per unit: 0 never, 1 where it pays (below), 2 always
  int kg = 1;          // K-group 128-row tiles for the rank stages: 0 never, 1 where the planner rates them cheaper, 2 always
  int kgw = 125;       // planner: cycles of a K-group 64-k step, percent of a 256-row tile's 32-k step
  int kgs = 7;         // stages that may take K-group tiles: 1 gate/up X.U, 2 h.Ud, 4 XU_d.Vd
  // decode layer: most K splits of phases 1, 3, 4 (0: grid / tiles; -1: the
  // defaults, dls3 8 at two token tiles, dls4 4 at four, else grid / tiles)
  int dls1 = 0, dls3 = -1, dls4 = -1;
  bool dlpff = true;   // decode layer: the weight prefetch at a grid barrier fills the whole ring
  bool dlready = true;  // decode layer: phase 4 waits for its XU_d tiles' ready flags, not a grid barrier
  bool dlready3 = true; // ... also from two token tiles up (XU_d tiles written by all their splits)
  // decode layer: a split that waits for the tile's other splits issues the
  // next phase's first weights before its share (bit 0: phase 1, bit 1:
  // phase 3).  Phase 1's share first: its XU flags, which phase 2 waits for,
  // are not queued behind 48 KB of DMAs per CU (8B layer, two alternating
  // runs, 3 -> 2: T=64 82.2-82.3 -> 81.8-81.9, T=128 113.6-113.7 -> 112.9 us;
  // phase 3's share first as well (0): no better)
  int dlpre = 2;
  int dlh = 1;          // decode layer: phase 3 waits for its K split's h flag (1: eight token tiles, 2: from two)
  bool dlxu = true;     // decode layer: phase 2 waits for its XU tiles' ready flags, not a grid barrier
  bool dlxu1 = true;    // decode layer at one token tile: phase 2 waits for one "XU complete" flag
  bool dlp4n = true;    // decode layer at one token tile: phase 4 as 16-column units without a K split
  bool dldist = true;  // decode layer, 32+ token rows: split-K tiles and phase-2 pairs finished by all their units
};

const Tune& tune();

// One row tile of 256 x 128 tiles: each block streams its whole V column
// panel, so the passes run at the panel's stream rate per block (8B layer,
// T=256: 62 us for the g pass); K splits put more blocks on the V stream, as
// many as fill the CUs, 2 to 4 (8B, 112 column tiles: 2 splits, the layer
// 230 -> 194 us at T=256; 3B shape, ff=8192, 64 tiles: 4 splits, 141.2 ->
// 134.4 us; 256 x 256 tiles in 8 splits there 151.7 us, and for the 8B
// shape in 4 splits 194.8 -> 192.6 at T=256, no gain at T=160).  Two nearly
// full row tiles (448 < T <= 512): 256 x 256 tiles (whole 512-byte V rows
// per DMA instruction) in two splits (8B: T=512 261 -> 249 us; 3B: 167.3 us,
// against 175.0 with four splits that fill the CUs); with a mostly padded
// second row tile the split costs more than it gains (T=320: 208 -> 224,
// T=384: 221 -> 233 us).  The fp32 slices are summed into g (fragment order)
// and, with SiLU(g) applied, into h.
void gu_split_plan(int64_t T, int64_t ff, int* fn, int* splits) {
  const bool one = T <= 256, two = T > 448 && T <= 512 && ff % 256 == 0;
  *fn = one ? (tune().gusfn ? tune().gusfn : 4) : 8;
  *splits = 0;
  if (!(one || two) || !tune().gusplit || ff % 128) return;
  const int64_t tiles = (one ? 1 : 2) * ((ff + 32 * *fn - 1) / (32 * *fn));
  const int64_t s = tune().gusp ? tune().gusp : (one ? std::min<int64_t>(4, tune().split / std::max<int64_t>(1, tiles)) : 2);
  *splits = s >= 2 ? (int)s : 0;
}

const Tune& tune() {
  static const Tune t = [] {
    Tune r;
    const char* e = getenv("SVDMLP_TUNE");
    if (!e) return r;
    std::string str(e);
    size_t pos = 0;
    while (pos < str.size()) {
      size_t end = str.find(',', pos);
      if (end == std::string::npos) end = str.size();
      const std::string kv = str.substr(pos, end - pos);
      const size_t eq = kv.find('=');
      if (eq != std::string::npos) {
        const std::string k = kv.substr(0, eq);
        const int v = atoi(kv.c_str() + eq + 1);
        if (k == "s1") r.s1 = v;
        if (k == "s1g") r.s1g = v;
        if (k == "s4") r.s4 = v;
        if (k == "s2fn") r.s2fn = v;
        if (k == "split") r.split = v;
        if (k == "big") r.big = v != 0;
        if (k == "dlayer") r.dlayer = v != 0;
        if (k == "contract") r.contract = v != 0;
        if (k == "gusfn") r.gusfn = v;
        if (k == "gusp") r.gusp = v;
        if (k == "gusplit") r.gusplit = v != 0;
        if (k == "dfn6") r.dfn6 = v != 0;
        if (k == "hblk") r.hblk = v != 0;
        if (k == "qblk") r.qblk = v != 0;
        if (k == "f8tail") r.f8tail = v != 0;
        if (k == "xutail") r.xutail = v != 0;
        if (k == "gufuse") r.gufuse = v != 0;
        if (k == "gudual") r.gudual = v != 0;
        if (k == "gukg") r.gukg = v != 0;
        if (k == "gukgu") r.gukgu = v;
        if (k == "dlmin") r.dlmin = v;
        if (k == "gvmax") r.gvmax = v;
        if (k == "gvrw") r.gvrw = v;
        if (k == "nw") r.nw = v;
        if (k == "f8nw") r.f8nw = v == 4 ? 4 : 8;
        if (k == "p2split") r.p2split = v;
        if (k == "kg") r.kg = v;
        if (k == "kgw") r.kgw = v;
        if (k == "kgs") r.kgs = v;
        if (k == "dls1") r.dls1 = v;
        if (k == "dls3") r.dls3 = v;
        if (k == "dls4") r.dls4 = v;
        if (k == "dldist") r.dldist = v != 0;
        if (k == "dlp4n") r.dlp4n = v != 0;
        if (k == "dlxu1") r.dlxu1 = v != 0;
        if (k == "dlxu") r.dlxu = v != 0;
        if (k == "dlready") r.dlready = v != 0;
        if (k == "dlready3") r.dlready3 = v != 0;
        if (k == "dlh") r.dlh = v;
        if (k == "dlpre") r.dlpre = v;
        if (k == "dlpff") r.dlpff = v != 0;
      }
      pos = end + 1;
    }
    return r;
  }();
  return t;
}

// The large-tile kernel takes bf16 operands below 2 GB each (32-bit buffer
// offsets) and contraction lengths that are whole 32-k stages.
int wbytes(const Common& c) { return c.wt == SVDMLP_FP8_E4M3 ? 1 : 2; }

bool big_ok(const Common& c, bool vec, std::initializer_list<int64_t> bytes, std::initializer_list<int64_t> ks) {
  if (c.f32 || !vec || !tune().big) return false;
  if (c.wt != SVDMLP_BF16 && c.wt != SVDMLP_FP8_E4M3) return false;
  for (int64_t b : bytes)
    if (b >= ((int64_t)1 << 31)) return false;
  for (int64_t k : ks)
    if (k % 32 != 0) return false;
  return true;
}

// Waves per block of a large-tile launch: 4 only for the fn-8 natural-layout
// store stages under SVDMLP_TUNE=nw=4.
int big_nw(int fn, int epi, bool b_kc) { return (fn == 8 && epi == BEPI_STORE && !b_kc && tune().nw == 4) ? 4 : 8; }

// Tile shapes whose fragment-order split-K slices the reduction kernel takes.
bool big_frag_reduce_ok(int fn, int nw) { return (nw == 8 && fn >= 4 && fn <= 8 && fn != 5) || (nw == 4 && fn == 8); }

// Batch entry 1 of a large-tile launch whose two entries differ in width
// (gate and up ranks): its output columns, B row pitch, output row pitch
// and B bytes.  Its column tiles follow entry 0's in one grid.
struct Entry1 {
  int N;
  int64_t ldb, ldo, b_bytes;
};

// The second pass of a dual launch (entry 1: XU_u . Vu): its A pitch and
// bytes, K, B pitch and bytes, and (BEPI_DUAL_F32) K per split.
struct DualEntry {
  int64_t lda, a_bytes;
  int K;
  int64_t ldb, b_bytes;
  int k_split = 0;
};

int big_gemm(const Common& c, int stage, const void* a0, const void* a1, int64_t lda, int64_t a_bytes,
             const void* b0, const void* b1, int64_t ldb, int64_t b_bytes, bool b_kc, int M, int N, int K, int batch,
             int fn, int epi, int k_split, void* out, int64_t ldo, int64_t out_bstride, const uint16_t* gmem,
             bool out_f32 = false, int64_t out_sstride = 0, const float* s0 = nullptr, const float* s1 = nullptr,
             int gfrag = 0, int out_frag = 0, const Entry1* e1 = nullptr, const uint16_t* resid = nullptr,
             int kg = 1, int out_blk = 0, int a_blk = 0, int tile0 = 0, int tiles = 0,
             const DualEntry* du = nullptr) {
  BigParams p{};
  p.tile0 = tile0;
  p.tiles = tiles;
  p.out_blk = out_blk;
  p.a_blk = a_blk;
  p.resid = resid;
  p.gfrag = gfrag;
  p.out_frag = out_frag;
  const bool fp8 = c.wt == SVDMLP_FP8_E4M3;
  if (fp8 && (!s0 || b_kc)) return fail("fp8 large-tile GEMM needs natural-layout weights and scales");
  p.scale[0] = s0;
  p.scale[1] = s1 ? s1 : s0;
  p.a[0] = a0;
  p.a[1] = a1 ? a1 : a0;
  p.b[0] = b0;
  p.b[1] = b1 ? b1 : b0;
  p.a_bytes[0] = p.a_bytes[1] = (uint32_t)a_bytes;
  p.b_bytes[0] = (uint32_t)b_bytes;
  p.b_bytes[1] = (uint32_t)(e1 ? e1->b_bytes : b_bytes);
  p.lda = lda;
  p.ldb[0] = ldb;
  p.ldb[1] = e1 ? e1->ldb : ldb;
  p.out = out;
  p.ldo[0] = ldo;
  p.ldo[1] = e1 ? e1->ldo : ldo;
  p.out_bstride = out_bstride;
  p.out_sstride = out_sstride;
  p.gmem = gmem;
  p.M = M;
  p.N[0] = N;
  p.N[1] = e1 ? e1->N : N;
  p.K = K;
  const int bm = kg == 2 ? 128 : 256;  // K-group tiles are 128 rows
  p.mtiles = (M + bm - 1) / bm;
  p.ntiles = (N + 32 * fn - 1) / (32 * fn);
  if (e1) {  // both entries' column tiles in one grid of z = 1
    if (batch != 2) return fail("large-tile GEMM: a second entry of its own width needs a batch of two");
    p.nt0 = p.ntiles;
    p.ntiles += (e1->N + 32 * fn - 1) / (32 * fn);
    batch = 1;
  }
  if (du) {  // dual launches: entry 1 is the second pass of every block
    const bool f32 = epi == BEPI_DUAL_F32;
    if ((epi != BEPI_GU_DUAL && !f32) || batch != 1 || e1 || tiles)
      return fail("large-tile GEMM: a dual gate/up launch takes one batch entry and no tile range");
    if (f32 ? (du->k_split <= 0 || (K + k_split - 1) / k_split != (du->K + du->k_split - 1) / du->k_split)
            : k_split < std::max(K, du->K))
      return fail("large-tile GEMM: a dual launch's passes take the same K splits (none with the SwiGLU epilogue)");
    p.k_split1 = du->k_split;
    p.lda1 = du->lda;
    p.a_bytes[1] = (uint32_t)du->a_bytes;
    p.K1 = du->K;
    p.ldb[1] = du->ldb;
    p.b_bytes[1] = (uint32_t)du->b_bytes;
    p.ldo[1] = ldo;
    p.N[1] = N;
    if (!f32) p.out_bstride = 0;
  } else if (epi == BEPI_GU_DUAL || epi == BEPI_DUAL_F32) {
    return fail("large-tile GEMM: a dual gate/up launch needs its second entry");
  }
  p.k_split = k_split;
  const int splits = (K + k_split - 1) / k_split;
  const BigDesc d{fn, b_kc, epi, out_f32, fp8, kg == 2 ? 8 : big_nw(fn, epi, b_kc), kg};
  const char* why = nullptr;
  StageScope ss(stage, c.st);
  return check(launch_big(d, p, splits, batch, c.st, &why), "large-tile GEMM", why);
}

}  // namespace

namespace {

// K elements per split for the large-tile stages (a multiple of the 32-k
// stage); the number of splits launched is ceil(K / k_split), and the same
// count sizes the workspace and the reduction.  The split count minimises a
// cost model in shader cycles, with one 512-thread block per CU and the
// MI355X's 256 CUs (a fixed count, so that the workspace size does not
// depend on the device queried):
//   rounds * (k-steps per split * cycles per step + fixed cost per block)
//   + per fp32 slice: writing it and reading it back in the reduction.
// The constants are measured on MI355X: a 32-k step of a 256 x 256 tile
// costs ~1312 cycles (41 per MFMA of the 64 x 128 wave tile), of which ~60%
// does not shrink with the tile width (the 256-row A tile, the barrier): a
// 256 x 192 step took ~0.9 of a 256 x 256 one in the X.U stages, hence
// 787 + 65.6 * fn; prologue + epilogue ~20k cycles, and a slice byte
// ~0.00045 cycles each way (~4 TB/s at ~1.8 GHz).
// N1 >= 0: a second batch entry N1 columns wide (its own column tiles);
// otherwise `batch` entries of N columns.  *cost_out (if given) receives the
// model's cost of the chosen split.
//
// kg = 2 plans the K-group tiles (128 rows, 8 waves in two groups that take
// the two 32-k halves of a 64-k step): each wave does the same MFMAs and
// fragment reads per step as in the 256-row tile of the same width, and the
// block fetches twice the B rows per step, which makes the step ~25% dearer
// (tune().kgw percent): 8B layer, T=1024, h.Ud as 240 blocks of 128 x 192
// in two splits took 92.9 us against 78.6 us for 220 blocks of 256 x 256 in
// five (~0.72 against ~0.61 us per MFMA step of a wave), which the slices
// saved (23.6 against 57.7 MB, 8.5 against 12.4 us of reduction) did not
// repay, while X.[Ug|Uu] (240 tiles of 128 x 192, no split) and XU_d.Vd
// (256 of 128 x 128, no split) each saved their reduction: the layer
// 343.3 -> 328.4 us (same box, alternating runs).
int plan_ksplit(int64_t T, int64_t K, int64_t N, int fn, int batch, int64_t N1 = -1, double* cost_out = nullptr,
                int kg = 1) {
  const int64_t cus = tune().split;
  const int64_t bn = 32 * fn, bm = kg == 2 ? 128 : 256, sk = 32 * kg;
  const int64_t ntl = N1 >= 0 ? (N + bn - 1) / bn + (N1 + bn - 1) / bn : ((N + bn - 1) / bn) * batch;
  const int64_t tiles = ((T + bm - 1) / bm) * ntl;
  const double c_step = (787.0 + 65.6 * fn) * (kg == 2 ? tune().kgw / 100.0 : 1.0), c_block = 20000.0;
  const double c_slice = 0.0009 * (double)T * (double)(N1 >= 0 ? N + N1 : batch * N) * 4.0;
  int64_t best_ks = K;
  double best = -1.0;
  const int64_t max_s = std::max<int64_t>(1, std::min<int64_t>(64, K / 128));
  for (int64_t s = 1; s <= max_s; ++s) {
    const int64_t ks = ((K + s - 1) / s + sk - 1) / sk * sk;
    const int64_t splits = (K + ks - 1) / ks;
    const int64_t rounds = (tiles * splits + cus - 1) / cus;
    const double cost = (double)rounds * ((double)(ks / sk) * c_step + c_block) +
                        (splits > 1 ? (double)splits * c_slice : 0.0);
    if (best < 0 || cost < best) {
      best = cost;
      best_ks = ks;
    }
  }
  if (cost_out) *cost_out = best;
  return (int)std::min<int64_t>(best_ks, K);
}

// Tile width (columns / 32) of the gate/up X.U stage: SVDMLP_TUNE s1g, else
// the split planner's cheaper of 256 x 256 and 256 x 192 tiles up to 2048
// tokens.  256 x 192 tiles fill the last round of blocks better where
// 256 x 256 leave it part-empty (70B fp8 layer, T=2048: 352 blocks of
// 256 x 256 in 1.4 rounds against 480 of 256 x 192 in 1.9; the stage 360-371
// -> 310-316 us, the layer 2236-2243 -> 2208-2210 us, 1884-1892 -> 1838-1856
// with e4m3 h; 8B layer, us per layer: T=160 178.7 -> 177.7, T=256 191.9 ->
// 191.1, T=512 249.6 -> 247.5, T=1024 343.7-344.5 -> 341.1-341.6; same box,
// alternating runs).  The model keeps 256 x 256 at T=768 (3 splits of 66
// tiles against 2 of 90: 256 x 192 measured 303.9 -> 308.5 us there).  At
// 4096 tokens (the 32-layer stack) 256 x 256 measured 0.5% faster per stack
// in the same runs, so it stays there.
int gate_xu_fn(int64_t T, int64_t K, int64_t r, int batch, int64_t r1 = -1) {
  if (tune().s1g) return tune().s1g;
  const int fn = tune().s1;
  if (fn != 8 || T > 2048) return fn;
  double c8 = 0.0, c6 = 0.0;
  plan_ksplit(T, K, r, 8, batch, r1, &c8);
  plan_ksplit(T, K, r, 6, batch, r1, &c6);
  return c6 < c8 ? 6 : 8;
}

// Tile width (columns / 32) of the h.Ud stage: 256 x 256, or 256 x 192 where
// those fill the CUs in one round without a K split and the model rates
// them cheaper (tune().dfn6).  With splits the model misjudges the narrower
// tile (8B layer, T=1024: 85.1 against 75.7-76.0 us measured for 256 x 256),
// without them it saves the slices and their reduction: 70B fp8 layer,
// T=2048, 240 blocks of 256 x 192 against 176 tiles of 256 x 256 in four
// splits (704 blocks), h.Ud 521.5-525.7 + 39.5 us (reduction) against
// 523.8-541.4 us.
int down_xu_fn(int64_t T, int64_t K, int64_t N) {
  const int fn = tune().s1;
  if (fn != 8 || !tune().dfn6) return fn;
  double c8 = 0.0, c6 = 0.0;
  plan_ksplit(T, K, N, 8, 1, -1, &c8);
  const int64_t ks6 = plan_ksplit(T, K, N, 6, 1, -1, &c6);
  return (ks6 >= K && c6 < c8) ? 6 : 8;
}

int plan_splits(int64_t T, int64_t K, int64_t N, int fn, int batch, int kg) {
  const int64_t ks = plan_ksplit(T, K, N, fn, batch, -1, nullptr, kg);
  return (int)((K + ks - 1) / ks);
}

// Tile plan of a rank stage (the X.U products and XU_d.Vd): 256-row tiles
// fn1 * 32 wide, or K-group tiles of 128 x 128 or 128 x 192 where they apply
// (kg_ok: natural-layout bf16 B, K a multiple of 64) and the cost model rates
// them cheaper (tune().kg 1; 2 takes them wherever they apply).  At the 8B
// layer's 1024 tokens they run X.[Ug|Uu] (240 tiles of 128 x 192) and
// XU_d.Vd (256 of 128 x 128) without K splits and h.Ud (120 tiles) in two
// instead of five.
struct RankPlan {
  int kg, fn, ks, splits;
};

RankPlan plan_rank(int64_t T, int64_t K, int64_t N, int fn1, int batch, int64_t N1, bool kg_ok, int stage) {
  double c1 = 0.0;
  const int ks1 = plan_ksplit(T, K, N, fn1, batch, N1, &c1, 1);
  RankPlan best{1, fn1, ks1, (int)((K + ks1 - 1) / ks1)};
  const int bit = stage == ST_GU_XU ? 1 : (stage == ST_D_XU ? 2 : 4);
  if (!kg_ok || tune().kg == 0 || !(tune().kgs & bit) || K % 64) return best;
  // the K-group tiles must undercut the 256-row plan by 5% (the model's
  // margin: at 2048 tokens it rates h.Ud within 1% either way)
  double bestc = tune().kg == 2 ? 1e300 : 0.95 * c1;
  for (int fn : {4, 6}) {
    double c = 0.0;
    const int ks = plan_ksplit(T, K, N, fn, batch, N1, &c, 2);
    if (c < bestc) {
      bestc = c;
      best = RankPlan{2, fn, ks, (int)((K + ks - 1) / ks)};
    }
  }
  return best;
}

// The split tail runs on the tile-range instance of the large-tile kernel:
// 256 x 256 tiles of natural-layout bf16 B with 8 waves.
bool xu_tail_ok(const Common& c, int fn, bool u_lin) {
  return fn == 8 && c.wt == SVDMLP_BF16 && !u_lin && big_nw(fn, BEPI_STORE, u_lin) == 8;
}

// Split tail of the two-entry X.U stage (256-row tiles, fn * 32 wide): with
// more tiles than one round of blocks and fewer than two, the first whole
// round of tiles (whole column tiles) runs without a K split and the rest
// in s splits, one round at most, their fp32 slices (compact, at most one
// round of tiles) summed by the reduction.  The head tile count, or 0 when
// the plain plan (`plain_cost`, the planner's model) is as cheap or the
// slices do not fit `cap` bytes; *tail_ks: K per split of the tail.  The
// model's terms are plan_ksplit's.  8B shape, 4096 tokens, ranks
// (2816, 3072): 368 tiles, 256 unsplit and 112 in two splits, against two
// rounds of 256 and 112 blocks.
int split_tail_plan(int64_t T, int64_t K, int64_t N, int64_t N1, int fn, double plain_cost, int64_t cap, int* tail_ks) {
  if (!tune().xutail) return 0;
  const int64_t cus = tune().split, bn = 32 * fn, mt = (T + 255) / 256;
  const int64_t tiles = mt * ((N + bn - 1) / bn + (N1 + bn - 1) / bn);
  const int64_t head = tiles / cus * cus / mt * mt, rem = tiles - head;
  if (head <= 0 || rem <= 0 || head > cus) return 0;
  const double c_step = 787.0 + 65.6 * fn, c_block = 20000.0;
  const double c_slice = 0.0009 * (double)(256 * bn) * 4.0;  // per tile and split
  const double head_cost = (double)(K / 32) * c_step + c_block;
  double best = plain_cost;
  int64_t got = 0;
  for (int64_t s = 2; s <= 8; ++s) {
    const int64_t ks = ((K + s - 1) / s + 31) / 32 * 32, sp = (K + ks - 1) / ks;
    if (rem * sp > cus || sp * rem * 256 * bn * 4 > cap) break;
    const double cost = head_cost + (double)(ks / 32) * c_step + c_block + (double)(sp * rem) * c_slice;
    if (cost < best) {
      best = cost;
      got = head;
      *tail_ks = (int)ks;
    }
  }
  return (int)got;
}

// Row pitch (elements) of the factors as stored, natural layout: ug and uu
// share one, vg and vu one, then ud and vd.  Dense factors have the row
// length as pitch.
struct FactorLd {
  int64_t u, v, ud, vd;
  bool dense;
  int64_t uu = 0, vu = 0;  // up-branch pitches when they differ from u, v (distinct gate and up ranks)
};

FactorLd dense_ld(int64_t d, int64_t ff, int64_t r_gu, int64_t r_d) { return FactorLd{r_gu, ff, r_d, d, true}; }

// XU_g, XU_u = A . Ug, A . Uu of ranks r and r1 != r (one launch, the two
// entries' column tiles side by side) into bf16 ws.xu_bf16: (T, r) then
// (T, r1).  Split-K as in big_xu when the fragment-order slices fit the
// workspace's slice area, else one split.
// The split-tail form of big_xu2 (split_tail_plan): tiles [0, head) in one
// launch without a split, bf16 out; tiles [head, end) in splits of tail_ks
// into compact fp32 slices; then each entry's split column tiles summed.
int big_xu2_tail(const Common& c, int stage, const void* a, int64_t lda, int64_t a_bytes, const void* const* u,
                 bool u_lin, int T, int K, int r, int r1, char* ws, const Ws& L, const float* s0, const float* s1,
                 int64_t ldb0, int64_t ldb1, int64_t b0, int64_t b1, int fn, int head, int tail_ks) {
  uint16_t* xu = reinterpret_cast<uint16_t*>(ws + L.xu_bf16);
  const Entry1 e1{r1, ldb1, r1, b1};
  const int bn = 32 * fn, mt = (T + 255) / 256;
  const int nt0 = (r + bn - 1) / bn, nt1 = (r1 + bn - 1) / bn, tiles = mt * (nt0 + nt1), rem = tiles - head;
  int rc = big_gemm(c, stage, a, a, lda, a_bytes, u[0], u[1], ldb0, b0, u_lin, T, r, K, 2, fn, BEPI_STORE, K, xu, r,
                    (int64_t)T * r, nullptr, false, 0, s0, s1, 0, 0, &e1, nullptr, 1, 0, 0, 0, head);
  if (rc) return rc;
  float* part = reinterpret_cast<float*>(ws + L.part);
  const int64_t tile_elems = (int64_t)256 * bn;
  const int64_t sstride = (int64_t)rem * tile_elems;  // compact slices: the tail's tiles, per split
  if ((rc = big_gemm(c, stage, a, a, lda, a_bytes, u[0], u[1], ldb0, b0, u_lin, T, r, K, 2, fn, BEPI_STORE, tail_ks,
                     part, r, 0, nullptr, true, sstride, s0, s1, 0, 1, &e1, nullptr, 1, 0, 0, head, rem)))
    return rc;
  const int splits = (K + tail_ks - 1) / tail_ks;
  const int nw = big_nw(fn, BEPI_STORE, u_lin);
  StageScope fin(ST_FINALIZE, c.st);
  const int c0 = head / mt;  // first split column tile (both entries' tiles counted)
  if (c0 < nt0) {             // entry 0's split column tiles
    rc = check(launch_reduce_frag_bf16(part, splits, sstride, 0, xu + (int64_t)c0 * bn, r, 0, T, r - c0 * bn, mt,
                                       nt0 - c0, fn, nw, 1, c.st),
               "split-K reduce");
    if (rc) return rc;
  }
  const int c1 = std::max(0, c0 - nt0);  // entry 1's first split column tile
  const int64_t off1 = (int64_t)std::max(0, nt0 - c0) * mt * tile_elems;
  return check(launch_reduce_frag_bf16(part + off1, splits, sstride, 0, xu + (int64_t)T * r + (int64_t)c1 * bn, r1, 0,
                                       T, r1 - c1 * bn, mt, nt1 - c1, fn, nw, 1, c.st),
               "split-K reduce");
}

int big_xu2(const Common& c, int stage, const void* a, int64_t lda, int64_t a_bytes, const void* const* u, bool u_lin,
            int T, int K, int r, int r1, char* ws, const Ws& L, const float* const* su, int64_t ldu, int64_t ldu1) {
  const RankPlan pl = plan_rank(T, K, r, gate_xu_fn(T, K, r, 2, r1), 2, r1, !u_lin && c.wt == SVDMLP_BF16, stage);
  const int fn = pl.fn, kg = pl.kg;
  const int nw = kg == 2 ? 8 : big_nw(fn, BEPI_STORE, u_lin);
  uint16_t* xu = reinterpret_cast<uint16_t*>(ws + L.xu_bf16);
  const int64_t ldb0 = u_lin ? K : (ldu ? ldu : r), ldb1 = u_lin ? K : (ldu1 ? ldu1 : r1);
  const int64_t b0 = (int64_t)(u_lin ? r : K) * ldb0 * wbytes(c), b1 = (int64_t)(u_lin ? r1 : K) * ldb1 * wbytes(c);
  const float* s0 = su ? su[0] : nullptr;
  const float* s1 = su ? su[1] : nullptr;
  const int64_t bn = 32 * fn, bm = kg == 2 ? 128 : 256, tp = (T + bm - 1) / bm * bm;
  const int64_t per0 = tp * ((r + bn - 1) / bn * bn), per1 = tp * ((r1 + bn - 1) / bn * bn);
  int ks = pl.ks;
  int splits = pl.splits;
  if (splits > 1 && ((kg == 1 && !big_frag_reduce_ok(fn, nw)) ||
                     (int64_t)splits * (per0 + per1) * 4 > (int64_t)(L.norm - L.part))) {
    ks = K;
    splits = 1;
  }
  const Entry1 e1{r1, ldb1, r1, b1};
  {  // split tail: a whole round of tiles without a K split, the rest split
    const int fn1 = gate_xu_fn(T, K, r, 2, r1);
    double plain = 0.0;
    plan_ksplit(T, K, r, fn, 2, r1, &plain, kg);
    int tail_ks = K;
    const int head = xu_tail_ok(c, fn1, u_lin)
                         ? split_tail_plan(T, K, r, r1, fn1, plain, (int64_t)(L.norm - L.part), &tail_ks)
                         : 0;
    if (head > 0) return big_xu2_tail(c, stage, a, lda, a_bytes, u, u_lin, T, K, r, r1, ws, L, s0, s1, ldb0, ldb1, b0,
                                      b1, fn1, head, tail_ks);
  }
  if (splits == 1)
    return big_gemm(c, stage, a, a, lda, a_bytes, u[0], u[1], ldb0, b0, u_lin, T, r, K, 2, fn, BEPI_STORE, K, xu, r,
                    (int64_t)T * r, nullptr, false, 0, s0, s1, 0, 0, &e1, nullptr, kg);
  float* part = reinterpret_cast<float*>(ws + L.part);
  int rc = big_gemm(c, stage, a, a, lda, a_bytes, u[0], u[1], ldb0, b0, u_lin, T, r, K, 2, fn, BEPI_STORE, ks, part, r,
                    per0, nullptr, true, per0 + per1, s0, s1, 0, 1, &e1, nullptr, kg);
  if (rc) return rc;
  StageScope fin(ST_FINALIZE, c.st);
  const int mt = (int)(tp / bm);
  rc = check(launch_reduce_frag_bf16(part, splits, per0 + per1, 0, xu, r, 0, T, r, mt, (int)(per0 / tp / bn), fn, nw,
                                     1, c.st, nullptr, nullptr, kg),
             "split-K reduce");
  if (rc) return rc;
  return check(launch_reduce_frag_bf16(part + per0, splits, per0 + per1, 0, xu + (int64_t)T * r, r1, 0, T, r1, mt,
                                       (int)(per1 / tp / bn), fn, nw, 1, c.st, nullptr, nullptr, kg),
               "split-K reduce");
}

// XU_b = A . U_b (b < batch) into bf16 ws.xu_bf16, batch stride T*r.  With
// too few output tiles for the chip, K is split: each split writes an fp32
// slice (plain stores) and one pass sums the slices in order into bf16.
// a_blk: A (h of the fused layer) is 16 x 16 block-major (BigParams::a_blk).
int big_xu(const Common& c, int stage, const void* a, int64_t lda, int64_t a_bytes, const void* const* u, bool u_lin,
           int T, int K, int r, int batch, char* ws, const Ws& L, const float* const* su = nullptr,
           int64_t ldu = 0, bool a_blk = false) {
  if (a_blk) a_bytes = (int64_t)((T + 15) / 16 * 16) * K * 2;  // whole 16-row blocks
  const int fn1 = stage == ST_GU_XU ? gate_xu_fn(T, K, r, batch) : down_xu_fn(T, K, r);
  const RankPlan pl = plan_rank(T, K, r, fn1, batch, -1, !u_lin && c.wt == SVDMLP_BF16, stage);
  if (stage == ST_GU_XU && batch == 2 && !a_blk) {  // the split tail runs in the two-entry form
    double plain = 0.0;
    plan_ksplit(T, K, r, pl.fn, 2, -1, &plain, pl.kg);
    int tail_ks = K;
    if (xu_tail_ok(c, fn1, u_lin) && split_tail_plan(T, K, r, r, fn1, plain, (int64_t)(L.norm - L.part), &tail_ks) > 0)
      return big_xu2(c, stage, a, lda, a_bytes, u, u_lin, T, K, r, r, ws, L, su, ldu, ldu);
  }
  const int fn = pl.fn, kg = pl.kg;
  const int64_t bm = kg == 2 ? 128 : 256;
  int ks = pl.ks;
  int splits = pl.splits;
  {  // the slices must fit the workspace's slice area (sized for the planned tiles)
    const int64_t tp = (T + bm - 1) / bm * bm, np = ((int64_t)r + 32 * fn - 1) / (32 * fn) * (32 * fn);
    if (splits > 1 && (int64_t)splits * batch * std::max(tp * np, (int64_t)T * r) * 4 > (int64_t)(L.norm - L.part)) {
      ks = K;
      splits = 1;
    }
  }
  uint16_t* xu = reinterpret_cast<uint16_t*>(ws + L.xu_bf16);
  const int64_t ldb = u_lin ? K : (ldu ? ldu : r);  // natural U may carry padded rows
  const int64_t u_bytes = (int64_t)(u_lin ? r : K) * ldb * wbytes(c);
  const void* u1 = batch > 1 ? u[1] : u[0];
  const float* s0 = su ? su[0] : nullptr;
  const float* s1 = su && batch > 1 ? su[1] : s0;
  if (splits == 1)
    return big_gemm(c, stage, a, a, lda, a_bytes, u[0], u1, ldb, u_bytes, u_lin, T, r, K, batch, fn,
                    BEPI_STORE, K, xu, r, (int64_t)T * r, nullptr, false, 0, s0, s1, 0, 0, nullptr, nullptr, kg, 0,
                    a_blk);
  float* part = reinterpret_cast<float*>(ws + L.part);
  const int nw = kg == 2 ? 8 : big_nw(fn, BEPI_STORE, u_lin);
  if (kg == 2 || big_frag_reduce_ok(fn, nw)) {
    // slices in fragment order: per split, `batch` blocks of whole tiles
    const int64_t tp = (T + bm - 1) / bm * bm, np = ((int64_t)r + 32 * fn - 1) / (32 * fn) * (32 * fn), per = tp * np;
    int rc = big_gemm(c, stage, a, a, lda, a_bytes, u[0], u1, ldb, u_bytes, u_lin, T, r, K, batch, fn, BEPI_STORE, ks,
                      part, r, per, nullptr, true, batch * per, s0, s1, 0, 1, nullptr, nullptr, kg, 0, a_blk);
    if (rc) return rc;
    StageScope fin(ST_FINALIZE, c.st);
    return check(launch_reduce_frag_bf16(part, splits, batch * per, per, xu, r, (int64_t)T * r, T, r, (int)(tp / bm),
                                         (int)(np / (32 * fn)), fn, nw, batch, c.st, nullptr, nullptr, kg),
                 "split-K reduce");
  }
  const int64_t slice = (int64_t)batch * T * r;
  int rc = big_gemm(c, stage, a, a, lda, a_bytes, u[0], u1, ldb, u_bytes, u_lin, T, r, K, batch, fn,
                    BEPI_STORE, ks, part, r, (int64_t)T * r, nullptr, true, slice, s0, s1, 0, 0, nullptr, nullptr, 1, 0,
                    a_blk);
  if (rc) return rc;
  StageScope fin(ST_FINALIZE, c.st);
  return check(launch_reduce_bf16(part, splits, slice, xu, slice, c.st), "split-K reduce");
}

// out = SiLU(XUg . Vg) * (XUu . Vu): a g pass (bf16 g to the workspace) and a
// u pass whose epilogue applies SiLU(g) * u.
// The up branch's rank r_u may differ from the gate branch's r (0: the same).
// h_blk (optional): asks for h in 16 x 16 block-major order (the fused
// layer's h.Ud stage reads it so: BigParams::a_blk) and reports whether the
// pass wrote it so (the split passes at one or two row tiles write
// row-major h).
int big_swiglu(const Common& c, const uint16_t* xu_g, const uint16_t* xu_u, const void* vg, const void* vu,
               bool v_lin, int T, int r, int ff, uint16_t* gbuf, void* out, float* part, int64_t part_cap,
               const float* s_vg = nullptr, const float* s_vu = nullptr, int64_t ldv = 0, int r_u = 0,
               int64_t ldv_u = 0, bool* h_blk = nullptr) {
  const bool want_blk = h_blk && *h_blk && ff % 16 == 0;
  if (h_blk) *h_blk = false;
  if (r_u <= 0) r_u = r;
  int fn = tune().s2fn;
  // 256 x 224 tiles (fn 7) leave most CUs idle at one or two 256-row tiles
  // of tokens; 256 x 128 tiles (fn 4) double the block count there (8B
  // layer: T=256 268 -> 245 us, T=512 298 -> 288 us; from three row tiles on
  // fn 7 is faster: T=768 349 vs 428 us).
  if (fn == 0) fn = (T <= 512 && ff % 128 == 0) ? 4 : ((ff % 224 == 0) ? 7 : 8);
  const int64_t ldb = v_lin ? r : (ldv ? ldv : ff), ldb_u = v_lin ? r_u : (ldv_u ? ldv_u : ldb);
  const int64_t xu_bytes = (int64_t)T * r * 2, v_bytes = (int64_t)(v_lin ? ff : r) * ldb * wbytes(c);
  const int64_t xuu_bytes = (int64_t)T * r_u * 2, vu_bytes = (int64_t)(v_lin ? ff : r_u) * ldb_u * wbytes(c);
  // 129-256 token rows on 128 x 128 K-group tiles: twice the tiles of the
  // 256-row ones, so the one-launch SwiGLU passes run without a K split (no
  // fp32 slices, no reduction), and the rows past T of a 256-row tile no
  // longer cost MFMAs.  Faster on every shape measured, also where the tiles
  // fill half the CUs (layer, two alternating runs, 256-row split passes ->
  // these: 8B T=160 / 200 / 256 154.2 / 161.9 / 169.7 -> 135.5 / 143.1 /
  // 155.6 us; 3B (3072, 8192, 1792) T=160 / 256 104.6 / 109.2 -> 98.5 / 108.0;
  // (1024, 4096, 512) 66.5 / 62.8 -> 58.8 / 55.5).  Up to 512 rows while the
  // tiles fit one round of the CUs (3B T=384 / 512: 128.1 / 145.0 -> 116.1 /
  // 124.7 us; the 8B shape's 336 tiles at T=384 would take two rounds).
  const int64_t kg_tiles = (int64_t)(T + 127) / 128 * ((ff + 127) / 128);
  if (tune().gukgu && T > 128 && (tune().gukgu >= 2 ? kg_tiles <= tune().split : T <= 256) && fn == 4 &&
      c.wt == SVDMLP_BF16 && !v_lin && tune().gudual && r % 64 == 0 && r_u % 64 == 0 && ff % 128 == 0) {
    const DualEntry du{r_u, xuu_bytes, r_u, ldb_u, vu_bytes};
    if (want_blk) *h_blk = true;
    return big_gemm(c, ST_GU_XUV_DUAL, xu_g, xu_u, r, xu_bytes, vg, vu, ldb, v_bytes, v_lin, T, ff, r, 1, fn,
                    BEPI_GU_DUAL, std::max(r, r_u), out, ff, 0, gbuf, false, 0, s_vg, s_vu, 1, 0, nullptr, nullptr, 2,
                    want_blk ? 1 : 0, 0, 0, 0, &du);
  }
  // At one or two row tiles of tokens the passes split K (gu_split_plan).
  int sfn = 0, nsp = 0;
  gu_split_plan(T, ff, &sfn, &nsp);
  // Up to 128 token rows the one-launch split passes run 128 x 128 K-group
  // tiles: a 256-row tile there spends half its MFMAs and A stages on rows of
  // zeros (8B factors, T=128: 50.5 us in 256-row tiles).  The same tiles and
  // splits otherwise; K splits in whole 64-k stages.
  bool kg2 = tune().gukg && T <= 128 && sfn == 4 && c.wt == SVDMLP_BF16 && !v_lin && tune().gufuse &&
             tune().gudual && r % 64 == 0 && r_u % 64 == 0;
  const int kq = kg2 ? 64 : 32;
  int ks = nsp >= 2 ? (r / nsp + kq - 1) / kq * kq : r, ks_u = nsp >= 2 ? (r_u / nsp + kq - 1) / kq * kq : r_u;
  int splits = (r + ks - 1) / ks, splits_u = (r_u + ks_u - 1) / ks_u;
  const int64_t np = (ff + 32 * sfn - 1) / (32 * sfn) * (32 * sfn);
  int64_t per = (int64_t)((T + 127) / 128 * 128) * np;
  if (kg2 && (splits != splits_u || (int64_t)(splits + splits_u) * per * 4 > part_cap)) {
    kg2 = false;  // the K-group tiles run the one-launch passes only
    ks = nsp >= 2 ? (r / nsp + 31) / 32 * 32 : r;
    ks_u = nsp >= 2 ? (r_u / nsp + 31) / 32 * 32 : r_u;
    splits = (r + ks - 1) / ks;
    splits_u = (r_u + ks_u - 1) / ks_u;
  }
  if (!kg2) per = (int64_t)((T + 255) / 256 * 256) * np;
  const int bm = kg2 ? 128 : 256;
  if (nsp >= 2 && fn == 4 && r >= 32 * nsp && r_u >= 32 * nsp && nsp * per * 4 <= part_cap) {
    fn = sfn;
    // Both passes' slices side by side when the area holds them: one
    // reduction then rounds g from its slices and applies SiLU(g) to the u
    // sum (bitwise the two-reduction result, one launch and the bf16 g round
    // trip fewer); else g is reduced to bf16 before the u pass reuses the area.
    const bool fused = tune().gufuse && (int64_t)(splits + splits_u) * per * 4 <= part_cap;
    float* upart = fused ? part + (int64_t)splits * per : part;
    int rc;
    if (fused && tune().gudual && splits == splits_u && !v_lin) {
      // both passes' slices from one launch: every block its g split, then
      // its u split of the same tile
      const DualEntry du{r_u, xuu_bytes, r_u, ldb_u, vu_bytes, ks_u};
      rc = big_gemm(c, ST_GU_XUV_DUAL, xu_g, xu_u, r, xu_bytes, vg, vu, ldb, v_bytes, v_lin, T, ff, r, 1, fn,
                    BEPI_DUAL_F32, ks, part, ff, (int64_t)splits * per, nullptr, true, per, s_vg, s_vu, 0, 1, nullptr,
                    nullptr, kg2 ? 2 : 1, 0, 0, 0, 0, &du);
      if (rc) return rc;
    } else {
      rc = big_gemm(c, ST_GU_XUV_G, xu_g, nullptr, r, xu_bytes, vg, nullptr, ldb, v_bytes, v_lin, T, ff, r, 1, fn,
                    BEPI_STORE, ks, part, ff, per, nullptr, true, per, s_vg, nullptr, 0, 1);
      if (rc) return rc;
      if (!fused) {
        StageScope fin(ST_FINALIZE, c.st);
        if ((rc = check(launch_reduce_bf16(part, splits, per, gbuf, per, c.st), "split-K reduce"))) return rc;
      }
      rc = big_gemm(c, ST_GU_XUV, xu_u, nullptr, r_u, xuu_bytes, vu, nullptr, ldb_u, vu_bytes, v_lin, T, ff, r_u, 1,
                    fn, BEPI_STORE, ks_u, upart, ff, per, nullptr, true, per, s_vu, nullptr, 0, 1);
      if (rc) return rc;
    }
    StageScope fin(ST_FINALIZE, c.st);
    const int mt = (T + bm - 1) / bm;
    return check(launch_reduce_frag_bf16(upart, splits_u, per, per, static_cast<uint16_t*>(out), ff, (int64_t)T * ff,
                                         T, ff, mt, (int)(per / ((int64_t)bm * mt) / (32 * fn)), fn,
                                         kg2 ? 8 : big_nw(fn, BEPI_STORE, v_lin), 1, c.st, fused ? nullptr : gbuf,
                                         nullptr, kg2 ? 2 : 1, fused ? part : nullptr, fused ? splits : 0),
                 "split-K SwiGLU reduce");
  }
  if (tune().gudual && (fn == 4 || fn == 7 || fn == 8) && !v_lin) {
    // both passes in one launch: each block its g tile, then its u tile
    const DualEntry du{r_u, xuu_bytes, r_u, ldb_u, vu_bytes};
    if (want_blk) *h_blk = true;
    return big_gemm(c, ST_GU_XUV_DUAL, xu_g, xu_u, r, xu_bytes, vg, vu, ldb, v_bytes, v_lin, T, ff, r, 1, fn,
                    BEPI_GU_DUAL, std::max(r, r_u), out, ff, 0, gbuf, false, 0, s_vg, s_vu, 1, 0, nullptr, nullptr, 1,
                    want_blk ? 1 : 0, 0, 0, 0, &du);
  }
  int rc = big_gemm(c, ST_GU_XUV_G, xu_g, nullptr, r, xu_bytes, vg, nullptr, ldb, v_bytes, v_lin, T, ff, r,
                    1, fn, BEPI_STORE_FRAG, r, gbuf, ff, 0, nullptr, false, 0, s_vg);
  if (rc) return rc;
  if (want_blk) *h_blk = true;
  return big_gemm(c, ST_GU_XUV, xu_u, nullptr, r_u, xuu_bytes, vu, nullptr, ldb_u, vu_bytes, v_lin, T, ff, r_u, 1,
                  fn, BEPI_SWIGLU_MEM, r_u, out, ff, 0, gbuf, false, 0, s_vu, nullptr, 1, 0, nullptr, nullptr, 1,
                  want_blk ? 1 : 0);
}

// fp8 activations for h . Ud (SVDMLP_FP8_ACT): h quantised to e4m3 per
// token row, then the fp8 x fp8 GEMM (gemm_f8f8.hpp) into bf16 XU_d.  The
// e4m3 h goes to the g region (dead once the u pass has read it), the row
// scales to xu32 (unused on the large-tile path).
bool f8_down_ok(int64_t T, int64_t ff, int64_t r_d, int64_t ldud) {
  const int64_t lim = (int64_t)1 << 31;  // 32-bit buffer offsets of e4m3 h and Ud
  return T > kDecodeMaxT && ff % 128 == 0 && r_d % 16 == 0 && ldud % 16 == 0 && ff <= 32768 &&
         (T + 15) / 16 * 16 * ff < lim && ff * ldud < lim;
}

int f8_down_xu(const Common& c, const uint16_t* h, const void* ud, const float* sud, int64_t ldud, int T, int ff,
               int r, char* ws, const Ws& L) {
  uint8_t* hq = reinterpret_cast<uint8_t*>(ws + L.g);
  float* hs = reinterpret_cast<float*>(ws + L.xu32);
  uint16_t* xu = reinterpret_cast<uint16_t*>(ws + L.xu_bf16);
  const char* why = nullptr;
  int rc;
  // e4m3 h in 16 x 128 blocks: each 128-k stage of 16 rows is one 2 KB run
  // (the g region holds whole 256-row tiles, so the last block's rows fit)
  const bool blk = tune().qblk;
  {
    StageScope ss(ST_QUANT, c.st);
    rc = check(launch_quant_rows_e4m3(h, ff, hq, ff, hs, T, ff, c.st, &why, blk), "e4m3 row quantisation", why);
  }
  if (rc) return rc;
  F8Params p{};
  p.a = hq;
  p.a_blk = blk ? 1 : 0;
  p.b = static_cast<const uint8_t*>(ud);
  p.a_bytes = (uint32_t)((int64_t)(blk ? (T + 15) / 16 * 16 : T) * ff);
  p.b_bytes = (uint32_t)((int64_t)ff * ldud);
  p.lda = ff;
  p.ldb = ldud;
  p.sa = hs;
  p.sb = sud;
  p.M = T;
  p.N = r;
  p.K = ff;
  p.mtiles = (T + kF8BM - 1) / kF8BM;
  p.ntiles = (r + kF8BN - 1) / kF8BN;
  // K splits: rounds of 256 blocks x (128-k steps x ~1100 cycles + ~20K per
  // block) + the fp32 slices written and read back (~2800 bytes per cycle),
  // within the workspace's slice area.  Either every tile in s splits, or
  // (split tail) the first whole rounds of tiles (whole n-tile columns)
  // without a split and only the remaining tiles in s splits, in a second
  // launch: at the 70B shape (2048 tokens, 352 tiles) 256 tiles in one round
  // and 96 in two splits (192 blocks), against 704 blocks in 2.75 rounds,
  // with a quarter of the slices to sum.
  const int64_t tile_elems = (int64_t)kF8BM * kF8BN;
  const int64_t per = (int64_t)p.mtiles * p.ntiles * tile_elems;
  const int blocks = p.mtiles * p.ntiles, ksteps = ff / kF8BK;
  const int64_t slice_cap = (int64_t)(L.norm - L.part);
  auto round_cost = [&](int nblocks, int s) {
    return (double)((nblocks + 255) / 256) * (((ksteps + s - 1) / s) * 1100.0 + 20000.0);
  };
  int splits = 1, head = 0;  // head: tiles run without a split ahead of the split launch (0: none)
  double best = 0;
  for (int s = 1; s <= 4; ++s) {
    if (s > 1 && (int64_t)s * per * 4 > slice_cap) break;
    const double cost = round_cost(blocks * s, s) + (s > 1 ? (double)s * per * 8 / 2800.0 : 0.0);
    if (s == 1 || cost < best) {
      best = cost;
      splits = s;
    }
  }
  const int full = blocks / 256 * 256 / p.mtiles * p.mtiles;  // whole rounds of whole n-tile columns
  if (tune().f8tail && full > 0 && full < blocks) {
    const int rem = blocks - full;
    for (int s = 2; s <= 4; ++s) {
      if ((int64_t)s * per * 4 > slice_cap) break;
      const double cost = round_cost(full, 1) + round_cost(rem * s, s) + (double)s * rem * tile_elems * 8 / 2800.0;
      if (cost < best) {
        best = cost;
        splits = s;
        head = full;
      }
    }
  }
  const int nw = tune().f8nw;
  if (head > 0) {  // the head tiles: one split, bf16 out
    F8Params q = p;
    q.tile0 = 0;
    q.tiles = head;
    q.k_split = ff;
    q.out = xu;
    q.ldo = r;
    StageScope ss(ST_D_XU_F8, c.st);
    if ((rc = check(launch_f8_gemm(q, 1, nw, c.st, &why), "fp8 x fp8 GEMM", why))) return rc;
  }
  p.tile0 = head;
  p.tiles = blocks - head;
  p.k_split = ((ksteps + splits - 1) / splits) * kF8BK;
  splits = (ff + p.k_split - 1) / p.k_split;
  if (splits == 1) {
    p.out = xu;
    p.ldo = r;
    StageScope ss(ST_D_XU_F8, c.st);
    return check(launch_f8_gemm(p, 1, nw, c.st, &why), "fp8 x fp8 GEMM", why);
  }
  float* part = reinterpret_cast<float*>(ws + L.part);
  p.out = part;
  p.out_sstride = per;
  {
    StageScope ss(ST_D_XU_F8, c.st);
    if ((rc = check(launch_f8_gemm(p, splits, nw, c.st, &why), "fp8 x fp8 GEMM", why))) return rc;
  }
  // the split tiles are whole n-tile columns from column n_base: their slices
  // (indexed by the global tile) from tile `head` on, their output columns
  // from n_base on
  const int n_base = head / p.mtiles * kF8BN;
  StageScope fin(ST_FINALIZE, c.st);
  return check(launch_reduce_frag_bf16(part + head * tile_elems, splits, per, per, xu + n_base, r, (int64_t)T * r, T,
                                       r - n_base, p.mtiles, p.ntiles - head / p.mtiles, 4, nw, 1, c.st),
               "split-K reduce");
}

// y = XU . V with bf16 XU (T x r); bf16 y (T x dout).
int big_v(const Common& c, const uint16_t* xu, const void* v, bool v_lin, int T, int r, int dout, char* ws,
          const Ws& L, void* y, const float* sv = nullptr, int64_t ldv = 0) {
  const int fn1 = tune().s4 > 0 ? tune().s4 : 8;
  const int64_t ldb = v_lin ? r : (ldv ? ldv : dout);
  const int64_t xu_bytes = (int64_t)T * r * 2, v_bytes = (int64_t)(v_lin ? dout : r) * ldb * wbytes(c);
  RankPlan pl = plan_rank(T, r, dout, fn1, 1, -1, !v_lin && c.wt == SVDMLP_BF16, ST_D_XUV);
  if (pl.kg == 1 && tune().s4 > 0 && tune().s4 != 8) pl = RankPlan{1, fn1, r, 1};
  const int fn = pl.fn, kg = pl.kg;
  const int64_t bm = kg == 2 ? 128 : 256;
  const int ks = pl.ks;
  const int splits = pl.splits;
  // the MLP block's residual add rides on the output store or the fragment-order reduction
  const uint16_t* resid = c.blk ? static_cast<const uint16_t*>(c.blk->x) : nullptr;
  if (splits == 1) {
    if (c.blk) c.blk->resid_done = true;
    return big_gemm(c, ST_D_XUV, xu, nullptr, r, xu_bytes, v, nullptr, ldb, v_bytes, v_lin, T, dout, r, 1,
                    fn, BEPI_STORE, r, y, dout, 0, nullptr, false, 0, sv, nullptr, 0, 0, nullptr, resid, kg);
  }
  float* part = reinterpret_cast<float*>(ws + L.part);
  const int nw = kg == 2 ? 8 : big_nw(fn, BEPI_STORE, v_lin);
  if (kg == 2 || big_frag_reduce_ok(fn, nw)) {
    if (c.blk) c.blk->resid_done = true;
    const int64_t tp = (T + bm - 1) / bm * bm, np = ((int64_t)dout + 32 * fn - 1) / (32 * fn) * (32 * fn), per = tp * np;
    int rc = big_gemm(c, ST_D_XUV, xu, nullptr, r, xu_bytes, v, nullptr, ldb, v_bytes, v_lin, T, dout, r, 1, fn,
                      BEPI_STORE, ks, part, dout, per, nullptr, true, per, sv, nullptr, 0, 1, nullptr, nullptr, kg);
    if (rc) return rc;
    StageScope fin(ST_FINALIZE, c.st);
    return check(launch_reduce_frag_bf16(part, splits, per, per, static_cast<uint16_t*>(y), dout, (int64_t)T * dout,
                                         T, dout, (int)(tp / bm), (int)(np / (32 * fn)), fn, nw, 1, c.st, nullptr,
                                         resid, kg),
                 "split-K reduce");
  }
  const int64_t slice = (int64_t)T * dout;
  int rc = big_gemm(c, ST_D_XUV, xu, nullptr, r, xu_bytes, v, nullptr, ldb, v_bytes, v_lin, T, dout, r,
                    1, fn, BEPI_STORE, ks, part, dout, 0, nullptr, true, slice, sv);
  if (rc) return rc;
  StageScope fin(ST_FINALIZE, c.st);
  return check(launch_reduce_bf16(part, splits, slice, static_cast<uint16_t*>(y), slice, c.st), "split-K reduce");
}

// ---------------------------------------------------------------------------
// Decode stages
// ---------------------------------------------------------------------------

int decode_mt(int64_t T) { return T <= 16 ? 1 : (T <= 32 ? 2 : 4); }

int decode_stage(const Common& c, int stage, int T, int K, int nseg, const Operand* a, int srca,
                 const void* const* w, const float* const* sw, bool w_lin, const int* N, float* const* out,
                 const char* what) {
  DecodeParams p{};
  p.nseg = nseg;
  p.T = T;
  p.K = K;
  int tiles = 0;
  for (int s = 0; s < nseg; ++s) {
    p.a[s] = a[s];
    p.seg[s].w = w[s];
    p.seg[s].scale = sw ? sw[s] : nullptr;
    p.seg[s].out = out[s];
    p.seg[s].ldw = w_lin ? K : N[s];
    p.seg[s].ldo = N[s];
    p.seg[s].N = N[s];
    p.seg[s].ntiles = (N[s] + kDecTileN - 1) / kDecTileN;
    tiles += p.seg[s].ntiles;
  }
  // K slice per block: enough blocks to cover the chip ~2x, slices of >= 128.
  int64_t ks = ((int64_t)K * tiles + 511) / 512;
  ks = std::max<int64_t>(128, (ks + 127) / 128 * 128);
  ks = std::min<int64_t>(ks, ((int64_t)K + 31) / 32 * 32);
  p.k_split = (int)ks;
  const int splits = (int)(((int64_t)K + ks - 1) / ks);
  DecodeDesc d{decode_mt(T), srca, srcb_of(c.wt), w_lin};
  const char* why = nullptr;
  StageScope ss(stage, c.st);
  return check(launch_decode(d, p, tiles * splits, c.st, &why), what, why);
}

bool decode_ok(const Common& c, int64_t T, std::initializer_list<int64_t> dims, bool vec) {
  if (c.f32 || T > kDecodeMaxT || !vec) return false;
  for (int64_t v : dims)
    if (v % 8) return false;
  return true;
}

// The persistent decode layer takes bf16 activations and factors in natural
// layout, T <= kDlMaxT, ranks and d multiples of 128 and ff a multiple of 64
// (its tiles), every operand below 2 GB (32-bit buffer offsets).
// It beats the per-stage decode kernels at every T (measured on MI355X, 8B
// shape: T=1 83 us vs 88 us; T=8 82 vs 95; T=64 118 vs 250); the
// streaming-GEMV layer, tried first, takes 1 <= T <= kGvMaxT.
constexpr int64_t kDlMinT = 1;

// r_u: the up branch's rank (r_gu the gate's); with distinct ranks phase 2
// must run one-branch units (p2split_fits).
bool decode_layer_ok(const Common& c, int64_t T, int64_t d, int64_t ff, int64_t r_gu, int64_t r_d, uint32_t flags,
                     bool vec, const FactorLd& ld, int64_t r_u = -1) {
  if (r_u < 0) r_u = r_gu;
  if (c.f32 || c.wt != SVDMLP_BF16 || !vec || flags || T > kDlMaxT || !tune().dlayer) return false;
  if (T < std::min<int64_t>(kDlMinT, tune().dlmin)) return false;
  if (d % 128 || r_gu % 128 || r_u % 128 || r_d % 128 || ff % 64) return false;
  // one counter per split-K tile of phases 1, 3 and 4; the bf16 XU_d
  // lives in the decode-only gu32 region (2 T max(d, ff) fp32)
  if ((r_gu + r_u) / 128 + r_d / 128 + d / 128 > kDlMaxTiles || r_d > 4 * std::max(d, ff)) return false;
  const int64_t lim = (int64_t)1 << 31;
  const int64_t uu = ld.uu ? ld.uu : ld.u, vu = ld.vu ? ld.vu : ld.v;
  for (int64_t bytes : {T * d * 2, d * ld.u * 2, d * uu * 2, r_gu * ld.v * 2, r_u * vu * 2, ff * ld.ud * 2,
                        r_d * ld.vd * 2, T * ff * 2, 2 * T * std::max(r_gu, r_u) * 4})
    if (bytes >= lim) return false;
  return decode_layer_grid(decode_layer_mt((int)T)) > 0;
}

// Split-K plan of one decode-layer phase: `tiles` 128-column tiles over K;
// as many splits as keep tiles * splits within the grid, K per split a
// multiple of 32.  Returns the K per split; *units = tiles * splits.
int dl_plan(int64_t K, int64_t tiles, int grid, int* units, int max_s = 0) {
  int64_t s = std::max<int64_t>(1, grid / std::max<int64_t>(1, tiles));
  if (max_s > 0) s = std::min<int64_t>(s, max_s);
  int64_t ks = ((K + s - 1) / s + 31) / 32 * 32;
  ks = std::min(ks, K);
  *units = (int)(tiles * ((K + ks - 1) / ks));
  return (int)ks;
}

// The contracted instance takes the layer when asked for (SVDMLP_CONTRACT) at
// T <= kDlContractMaxT with a block for every h strip and XU_d tile.
bool decode_contract_ok(int64_t T, int64_t ff, int64_t r_gu, int64_t r_d, const Ws& L, size_t ws_bytes) {
  // the gate/up run-out prefetches the down half's first 5 ring stages of 64 k
  if (T > kDlContractMaxT || L.total == L.cslices || ws_bytes < L.total || r_gu < 320) return false;
  const int grid = decode_layer_contract_grid();
  return grid > 0 && ff / 64 + r_d / 128 <= grid;
}

// Phase 2 with one branch per unit fits the shape: ff in whole 128-column
// tiles, a block per unit and one more tile counter per column tile.
bool p2split_fits(int64_t d, int64_t ff, int64_t r_gu, int64_t r_d, int grid, int64_t r_u = -1) {
  if (r_u < 0) r_u = r_gu;
  const int64_t nt2 = ff / 128;
  return ff % 128 == 0 && 2 * nt2 <= grid && (r_gu + r_u) / 128 + r_d / 128 + d / 128 + nt2 <= kDlMaxTiles;
}

// r_u >= 0 and != r_gu: distinct gate and up ranks (the caller checked
// decode_layer_ok and p2split_fits with both; phase 2 runs one-branch units).
int decode_layer(const Common& c, const void* x, const void* ug, const void* vg, const void* uu, const void* vu,
                 const void* ud, const void* vd, void* y, int64_t T, int64_t d, int64_t ff, int64_t r_gu, int64_t r_d,
                 char* ws, const Ws& L, const FactorLd& ld, bool contract = false, int64_t r_u = -1) {
  if (r_u < 0) r_u = r_gu;
  const bool two = r_u != r_gu;
  const int mt = decode_layer_mt((int)T);
  const int grid = contract ? decode_layer_contract_grid() : decode_layer_grid(mt);
  DecLayerParams p{};
  p.x = x;
  p.ug = ug;
  p.vg = vg;
  p.uu = uu;
  p.vu = vu;
  p.ud = ud;
  p.vd = vd;
  p.y = y;
  p.xu16 = reinterpret_cast<uint16_t*>(ws + L.xu_bf16);
  p.xd16 = reinterpret_cast<uint16_t*>(ws + L.gu32);
  p.h = reinterpret_cast<uint16_t*>(ws + L.h);
  p.slices = reinterpret_cast<float*>(ws + L.slices);
  p.cslices = contract ? reinterpret_cast<float*>(ws + L.cslices) : nullptr;
  p.sync = reinterpret_cast<uint64_t*>(ws + L.sync);
  p.a_cached = ((uintptr_t)ws & 127u) == 0;
  p.T = (int)T;
  p.d = (int)d;
  p.ff = (int)ff;
  p.r_gu = (int)r_gu;
  p.r_up = (int)r_u;
  p.r_d = (int)r_d;
  p.ks1 = dl_plan(d, (r_gu + r_u) / 128, grid, &p.units1, tune().dls1);
  p.units2 = (int)(ff / 64);
  // Phase 2 with one branch per unit over 128 columns (units 2t, 2t+1: g
  // and u of tile t) instead of both over 64; the pair meets through a tile
  // counter after phases 1, 3 and 4's.  From two 16-row token tiles up each
  // unit then streams half the activation bytes per weight byte (8B layer,
  // T=32 / 64 / 128: 77.7 / 94.8 / 140.9 -> 76.0 / 91.7 / 130.2 us).  At one
  // tile it pays with dense factors only: their 4 KB-multiple V row pitch
  // maps the two-branch units' 128-byte column pieces onto a subset of the
  // HBM channels, and 256-byte pieces spread them (T=4 / 8 / 16: 75.8 / 76.4
  // / 78.2 -> 73.2 / 73.5 / 75.0 us); with padded rows the pair's extra
  // slice round trip costs ~1 us there (T=8 69.3 -> 70.4 us).
  const bool p2_pays = mt >= 2 || ld.dense;
  p.p2split = !contract && p2split_fits(d, ff, r_gu, r_d, grid, r_u) &&
              (two || tune().p2split >= 2 || (tune().p2split == 1 && p2_pays));
  // Phase 3 at two token tiles (17-32 tokens) in at most 8 K splits (176
  // units instead of 242 at the 8B shape): T=32 75.4-75.5 -> 74.8-74.9 us
  // padded, 79.7-79.8 -> 79.4-79.5 dense, T=17-24 0-0.6 us less; at four
  // tiles 8 splits cost 0.8 us.
  const int cap3 = tune().dls3 >= 0 ? tune().dls3 : (mt == 2 ? 8 : 0);
  p.ks3 = dl_plan(ff, r_d / 128, grid, &p.units3, cap3);
  // Phase 4 at four token tiles (33-64 tokens) in at most 4 K splits when one
  // block sums each tile: it then sums 4 slices of 64 rows instead of 8, for
  // a stream that is HBM-bound either way (8B layer, T=64: 90.5 -> 89.2 us;
  // at 1-32 tokens 4 splits cost 0.5-1 us, their slices being small).  With
  // the tiles summed by all their splits (dldist) 8 splits pay: T=48 81.6 ->
  // 80.5 us, T=64 unchanged.
  const int cap4 = tune().dls4 >= 0 ? tune().dls4 : (mt == 4 && !tune().dldist ? 4 : 0);
  p.ks4 = dl_plan(r_d, d / 128, grid, &p.units4, cap4);
  p.splits1 = p.units1 / (int)((r_gu + r_u) / 128);
  p.splits3 = p.units3 / (int)(r_d / 128);
  p.splits4 = p.units4 / (int)(d / 128);
  p.dist = mt >= 2 && tune().dldist;
  // (the shared split-K combinations count a second round of arrivals on
  // counters after every other tile counter of the layer: phase 1's XU
  // tiles, then phase 3's XU_d tiles)
  p.cnt2 = (int)((r_gu + r_u) / 128 + r_d / 128 + d / 128 + (p.p2split ? ff / 128 : 0));
  // From two token tiles up the XU_d tiles are written by all their splits,
  // whose second arrivals set the flag (8B layer, padded V rows, two
  // alternating runs: T=17 / 32 / 64 / 128 72.5 / 74.0 / 85.1 / 118.9 ->
  // 71.4 / 72.7 / 83.1 / 115.8 us; the 8-tile instance +5 VGPRs).
  p.xd_ready = (contract || mt == 1 || (p.dist && tune().dlready3 && p.cnt2 + (r_gu + r_u) / 128 + r_d / 128 <= kDlMaxTiles)) &&
               tune().dlready && r_d / 128 <= kDlRowFlag0;
  // Phase 4 at one token tile as 16-column units over the whole rank (T=1
  // 66.3 -> 63.7 us, T=2 -1.1 us); from two tiles up each unit would load
  // all of the (T, r_d) XU_d into registers: T=32 / 64 / 128 +4.5 / +5 / +11 us.
  p.p4narrow = mt == 1 && p.xd_ready && tune().dlp4n && d / 16 == grid && r_d % 32 == 0 &&
               r_d / 32 <= kDlNarrowMaxChunks && r_d * 32 <= 96 * 1024;
  // XU tiles' flags after the XU_d tiles'; the contracted layer needs the XU_d
  // flags as well (it then waits on no grid barrier and arrives at its end)
  p.xu_flag0 = (int)(r_d / 128);
  // From two token tiles up only: with ready flags instead of the barrier
  // 8B T=32 / 64 / 128 -0.35 / -0.7 / -0.3 us, but the contracted layer at T=1
  // +1.5 us and the one-tile layer +0.3 us (224 blocks polling all 44 tiles'
  // flags while the last phase-1 tiles are still combined).
  p.xu_ready = mt >= 2 && tune().dlxu && (r_gu + r_u) / 128 <= 128 &&
               r_d / 128 + (r_gu + r_u) / 128 <= kDlRowFlag0 && (!contract || p.xd_ready) &&
               (!p.dist || p.cnt2 + (r_gu + r_u) / 128 <= kDlMaxTiles);
  // One token tile (four-phase layer): one flag for all of XU (mode 2),
  // stored by the last of the phase-1 tiles' writers to count down on one
  // counter (T=2-16 -0.7 us, the MLP block -0.8 to -1.2 us).  Not in the
  // contracted layer, which then waits on no grid barrier and needs an
  // arrival-only one for the flags' epoch: T=1 +0.85 us with it at the
  // launch's end (the last blocks wait for its atomics), +0.35 us after phase 1.
  if (mt == 1 && !contract && tune().dlxu1 && p.xd_ready && r_d / 128 < kDlRowFlag0 && p.cnt2 < kDlMaxTiles)
    p.xu_ready = 2;
  // Phase 3 on its K splits' h flags instead of a grid barrier, at eight
  // token tiles (65-128 tokens): flags after the XU tiles', counters after
  // the second-round ones of phases 1 and 3.  8B layer, padded V rows, two
  // alternating runs: T=100 / 128 107.2 / 115.1 -> 106.4 / 113.6 us; at two
  // and four tiles, where a split's K range spans 14 (8 splits) or 10 pairs
  // of phase-2 units, T=17 / 32 / 48 / 64 +1.0 / +1.0 / +0.4 / -0.2 us
  // (SVDMLP_TUNE=dlh=2 takes them there too).
  p.hf0 = p.xu_flag0 + (int)((r_gu + r_u) / 128);
  p.hc0 = p.cnt2 + (int)((r_gu + r_u) / 128 + r_d / 128);
  p.h_ready = (mt >= 8 ? tune().dlh >= 1 : mt >= 2 && tune().dlh >= 2) && p.dist && p.p2split && p.xu_ready == 1 &&
              p.hf0 + p.splits3 <= kDlRowFlag0 && p.hc0 + p.splits3 <= kDlMaxTiles;
  p.pf_full = tune().dlpff;
  p.pre_wait = tune().dlpre;
  p.ld_u = (int)ld.u;
  p.ld_v = (int)ld.v;
  p.ld_uu = (int)(ld.uu ? ld.uu : ld.u);
  p.ld_vu = (int)(ld.vu ? ld.vu : ld.v);
  p.ld_ud = (int)ld.ud;
  p.ld_vd = (int)ld.vd;
  if (c.blk) {
    // The MLP block: the residual add in phase 4; the RMSNorm in the
    // kernel's phase 0 (a block per token row, d <= 16384, 16-byte aligned
    // gains), else as its own pass.
    p.resid = c.blk->x;
    c.blk->resid_done = true;
    if (!c.blk->norm_done && d <= 8 * kDlThreads * kDlNormPieces && T <= grid && aligned16(c.blk->gain)) {
      p.gain = c.blk->gain;
      p.eps = c.blk->eps;
      p.xn = reinterpret_cast<uint16_t*>(ws + L.norm);
      c.blk->norm_done = true;
    } else if (!c.blk->norm_done) {
      void* hn = ws + L.norm;
      const int rc = check(launch_rmsnorm(c.blk->x, c.blk->gain, hn, T, d, c.blk->eps, true, c.st), "RMSNorm");
      if (rc) return rc;
      p.x = hn;
      c.blk->norm_done = true;
    }
  }
  const char* why = nullptr;
  StageScope ss(contract ? ST_DEC_CONTRACT : ST_DEC_LAYER, c.st);
  return check(launch_decode_layer(p, mt, grid, c.st, &why, contract), "decode layer", why);
}

// Streaming-GEMV layer (1 <= T <= min(kGvMaxT, gvmax)): bf16, natural
// layout, every K a multiple of the 16-row group, each factor below 2 GB and
// each block's activation rows within the kernel's LDS slice.
bool gemv_layer_ok(const Common& c, int64_t T, int64_t d, int64_t ff, int64_t r_gu, int64_t r_d, uint32_t flags,
                   bool vec, const FactorLd& ld) {
  const int rw = tune().gvrw == 1 ? 1 : 2;
  if (c.f32 || c.wt != SVDMLP_BF16 || !vec || flags || T < 1 || T > std::min(kGvMaxT, tune().gvmax)) return false;
  if (d % 16 || ff % 16 || r_gu % 16 || r_d % 16) return false;
  const int64_t lim = (int64_t)1 << 31;
  for (int64_t bytes : {d * ld.u * 2, r_gu * ld.v * 2, ff * ld.ud * 2, r_d * ld.vd * 2})
    if (bytes >= lim) return false;
  const int grid = gemv_layer_grid(rw);
  if (grid <= 0) return false;
  const int64_t strip = 512 / rw, group = 8 * rw;
  auto rows = [&](int64_t nm, int64_t K, int64_t N) {
    const int64_t groups = nm * ((N + strip - 1) / strip) * (K / group);
    return group * ((groups + grid - 1) / grid);
  };
  const int64_t most = std::max(std::max(rows(2, d, r_gu), rows(2, r_gu, ff)), std::max(rows(1, ff, r_d), rows(1, r_d, d)));
  return most * T <= gemv_layer_a_floats();
}

int gemv_layer(const Common& c, const void* x, const void* ug, const void* vg, const void* uu, const void* vu,
               const void* ud, const void* vd, void* y, int64_t T, int64_t d, int64_t ff, int64_t r_gu, int64_t r_d,
               char* ws, const Ws& L, const FactorLd& ld) {
  const int rw = tune().gvrw == 1 ? 1 : 2;
  GvParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.ug = static_cast<const uint16_t*>(ug);
  p.vg = static_cast<const uint16_t*>(vg);
  p.uu = static_cast<const uint16_t*>(uu);
  p.vu = static_cast<const uint16_t*>(vu);
  p.ud = static_cast<const uint16_t*>(ud);
  p.vd = static_cast<const uint16_t*>(vd);
  p.y = static_cast<uint16_t*>(y);
  if (c.blk) {  // the MLP block (x already normalised): residual add in the output write
    p.resid = static_cast<const uint16_t*>(c.blk->x);
    c.blk->resid_done = true;
  }
  p.xu32 = reinterpret_cast<float*>(ws + L.xu32);
  p.xd32 = p.xu32 + 2 * T * r_gu;
  p.gu32 = reinterpret_cast<float*>(ws + L.gu32);
  p.y32 = reinterpret_cast<float*>(ws + L.y32);
  p.sync = reinterpret_cast<uint64_t*>(ws + L.sync);
  p.T = (int)T;
  p.d = (int)d;
  p.ff = (int)ff;
  p.r_gu = (int)r_gu;
  p.r_d = (int)r_d;
  p.ld_u = (int)ld.u;
  p.ld_v = (int)ld.v;
  p.ld_ud = (int)ld.ud;
  p.ld_vd = (int)ld.vd;
  const char* why = nullptr;
  StageScope ss(ST_DEC_GEMV, c.st);
  return check(launch_gemv_layer(p, rw, gemv_layer_grid(rw), c.st, &why), "decode GEMV layer", why);
}

int validate_dims(int64_t T, int64_t a, int64_t b, int64_t r) {
  if (T <= 0 || a <= 0 || b <= 0 || r <= 0)
    return fail("dimensions must be positive, got T=%lld, %lld, %lld, r=%lld", (long long)T, (long long)a,
                (long long)b, (long long)r);
  const int64_t lim = (int64_t)1 << 30;
  if (T >= lim || a >= lim || b >= lim || r >= lim || T * std::max(a, b) >= ((int64_t)1 << 40))
    return fail("dimensions too large");
  return SVDMLP_OK;
}

// ---------------------------------------------------------------------------
// Fixed scratch of svdmlp_svd_mlp_noalloc: the workspace of calls that may not
// allocate.  One copy per device, at its own address, held until the process
// ends; host code uses only the address hipGetSymbolAddress returns for the
// current device (the array's name is a host-side stand-in).
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};

// Device address of the current device's scratch.  The first call on a
// device looks it up and zeroes its 4096-byte sync area on `st` (the grid
// barrier and tile counters of the persistent decode kernels start at zero;
// every later call leaves them valid for the next).
int scratch_of_current_device(hipStream_t st, char** out) {
  int dev = 0;
  int rc = check(hipGetDevice(&dev), "current device");
  if (rc) return rc;
  if (dev < 0 || dev >= kScratchDevices) return fail("device index %d beyond the scratch table", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if ((rc = check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "scratch symbol address"))) return rc;
    if (!ptr) return fail("scratch symbol address: null");
    if ((rc = check(launch_fill_zero(static_cast<float*>(ptr), 4096 / 4, st), "scratch sync area clear"))) return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = static_cast<char*>(g_scratch_ptr[dev]);
  return SVDMLP_OK;
}

int svd_mlp_run(const void* x, const void* ug, const void* vg, const void* uu, const void* vu, const void* ud,
                const void* vd, const float* const* scales, const int64_t* ld_in, void* y, int64_t T, int64_t d,
                int64_t ff, int64_t r_g, int64_t r_u, int64_t r_d, int32_t act_dtype, int32_t w_dtype, uint32_t flags,
                void* workspace, size_t ws_bytes, void* stream, Block* blk);

}  // namespace

extern "C" {

int svdmlp_svd_mlp_noalloc(const void* x, const void* ug, const void* vg, const void* uu, const void* vu,
                           const void* ud, const void* vd, const float* const* scales, const int64_t* ld, void* y,
                           int64_t T, int64_t d, int64_t ff, int64_t r_gu, int64_t r_d, int32_t act_dtype,
                           int32_t w_dtype, uint32_t flags, void* stream) {
  g_err.clear();
  int rc = validate_dims(T, d, ff, std::min(r_gu, r_d));
  if (rc) return rc;
  const size_t need = ws_layout(T, d, ff, std::max(r_gu, r_d)).need;
  if (need > kScratchBytes)
    return fail("svdmlp_svd_mlp_noalloc: this shape needs %zu bytes of workspace, more than the fixed scratch of "
                "%zu bytes (T=%lld, d=%lld, ff=%lld, r=%lld); use svdmlp_svd_mlp_ld with a workspace",
                need, kScratchBytes, (long long)T, (long long)d, (long long)ff, (long long)std::max(r_gu, r_d));
  char* ws = nullptr;
  if ((rc = scratch_of_current_device((hipStream_t)stream, &ws))) return rc;
  struct NoEvents {
    NoEvents() { t_no_events = true; }
    ~NoEvents() { t_no_events = false; }
  } guard;
  return svdmlp_svd_mlp_ld(x, ug, vg, uu, vu, ud, vd, scales, ld, y, T, d, ff, r_gu, r_d, act_dtype, w_dtype, flags,
                           ws, kScratchBytes, stream);
}

int svdmlp_noalloc_status(int32_t reset, int64_t wait_bound, void* stream) {
  g_err.clear();
  hipStream_t st = (hipStream_t)stream;
  char* ws = nullptr;
  int rc = scratch_of_current_device(st, &ws);
  if (rc) return rc;
  uint64_t flag = 0;
  rc = check(hipMemcpyAsync(&flag, ws + kDlFlag * 8, 8, hipMemcpyDeviceToHost, st), "scratch status read");
  if (!rc) rc = check(hipStreamSynchronize(st), "scratch status read");
  if (!rc && reset) rc = check(launch_fill_zero(reinterpret_cast<float*>(ws), 4096 / 4, st), "scratch sync area reset");
  if (!rc && wait_bound >= 0) {
    const uint64_t bound = (uint64_t)wait_bound;
    rc = check(hipMemcpyAsync(ws + kDlSpin * 8, &bound, 8, hipMemcpyHostToDevice, st), "scratch wait bound");
    if (!rc) rc = check(hipStreamSynchronize(st), "scratch wait bound");
  }
  if (rc) return rc;
  return flag ? 1 : 0;
}

int svdmlp_version(void) { return SVDMLP_VERSION; }

const char* svdmlp_last_error(void) { return g_err.c_str(); }

int svdmlp_svd_mlp_block(const void* x, const float* norm_w, float eps, const void* ug, const void* vg,
                         const void* uu, const void* vu, const void* ud, const void* vd, const float* const* scales,
                         void* y, int64_t T, int64_t d, int64_t ff, int64_t r_gu, int64_t r_d, int32_t act_dtype,
                         int32_t w_dtype, uint32_t flags, void* workspace, size_t ws_bytes, void* stream) {
  return svdmlp_svd_mlp_block_ld(x, norm_w, eps, ug, vg, uu, vu, ud, vd, scales, nullptr, y, T, d, ff, r_gu, r_d,
                                 act_dtype, w_dtype, flags, workspace, ws_bytes, stream);
}

int svdmlp_svd_mlp_block_ld(const void* x, const float* norm_w, float eps, const void* ug, const void* vg,
                            const void* uu, const void* vu, const void* ud, const void* vd,
                            const float* const* scales, const int64_t* ld, void* y, int64_t T, int64_t d, int64_t ff,
                            int64_t r_gu, int64_t r_d, int32_t act_dtype, int32_t w_dtype, uint32_t flags,
                            void* workspace, size_t ws_bytes, void* stream) {
  return svdmlp_svd_mlp_block_ranks(x, norm_w, eps, ug, vg, uu, vu, ud, vd, scales, ld, y, T, d, ff, r_gu, r_gu, r_d,
                                    act_dtype, w_dtype, flags, workspace, ws_bytes, stream);
}

int svdmlp_svd_mlp_block_ranks(const void* x, const float* norm_w, float eps, const void* ug, const void* vg,
                               const void* uu, const void* vu, const void* ud, const void* vd,
                               const float* const* scales, const int64_t* ld, void* y, int64_t T, int64_t d,
                               int64_t ff, int64_t r_g, int64_t r_u, int64_t r_d, int32_t act_dtype, int32_t w_dtype,
                               uint32_t flags, void* workspace, size_t ws_bytes, void* stream) {
  g_err.clear();
  int rc = validate_dims(T, d, ff, std::min(std::min(r_g, r_u), r_d));
  if (rc) return rc;
  if ((rc = check_types(act_dtype, w_dtype))) return rc;
  if (!x || !norm_w || !y || !workspace) return fail("null pointer argument");
  if (x == y) return fail("x and y must not alias (y receives the MLP output before the residual add)");
  if (!(eps > 0.0f)) return fail("eps must be positive, got %g", (double)eps);
  const int64_t r = std::max(std::max(r_g, r_u), r_d);
  const Ws L = ws_layout(T, d, ff, r);
  if (ws_bytes < L.need) return fail("workspace too small: need %zu bytes, got %zu", L.need, ws_bytes);
  const bool bf16 = act_dtype == SVDMLP_BF16;
  hipStream_t st = (hipStream_t)stream;
  Block blk{x, norm_w, eps};
  if ((rc = svd_mlp_run(x, ug, vg, uu, vu, ud, vd, scales, ld, y, T, d, ff, r_g, r_u, r_d, act_dtype, w_dtype, flags,
                        workspace, ws_bytes, stream, &blk)))
    return rc;
  if (blk.resid_done) return SVDMLP_OK;
  return check(launch_residual_add(x, y, T * d, bf16, st), "residual add");
}

int svdmlp_profile_enable(int enable) {
  std::lock_guard<std::mutex> g(g_prof.mu);
  g_prof.on = enable != 0;
  return ST_COUNT;
}

const char* svdmlp_stage_name(int stage) {
  return (stage >= 0 && stage < ST_COUNT) ? kStageNames[stage] : "";
}

int svdmlp_profile_read(double* total_ms, int64_t* launches, int n) {
  std::lock_guard<std::mutex> g(g_prof.mu);
  int rc = SVDMLP_OK;
  for (auto& r : g_prof.pending) {
    float ms = 0.f;
    hipError_t e = hipEventSynchronize(r.b);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.a, r.b);
    if (e != hipSuccess) {
      rc = check(e, "profile read");
    } else {
      g_prof.total_ms[r.stage] += ms;
      g_prof.count[r.stage] += 1;
    }
    g_prof.pool.push_back(r.a);
    g_prof.pool.push_back(r.b);
  }
  g_prof.pending.clear();
  for (int i = 0; i < n && i < ST_COUNT; ++i) {
    if (total_ms) total_ms[i] = g_prof.total_ms[i];
    if (launches) launches[i] = g_prof.count[i];
  }
  for (int i = 0; i < ST_COUNT; ++i) {
    g_prof.total_ms[i] = 0.0;
    g_prof.count[i] = 0;
  }
  return rc == SVDMLP_OK ? ST_COUNT : rc;
}

int svdmlp_workspace_status(void* workspace, size_t ws_bytes, int32_t reset, void* stream) {
  g_err.clear();
  if (!workspace) return fail("null pointer argument");
  if (ws_bytes < 4096) return fail("workspace too small: the sync area alone is 4096 bytes, got %zu", ws_bytes);
  hipStream_t st = (hipStream_t)stream;
  uint64_t flag = 0;
  int rc = check(hipMemcpyAsync(&flag, static_cast<char*>(workspace) + kDlFlag * 8, 8, hipMemcpyDeviceToHost, st),
                 "workspace status read");
  if (!rc) rc = check(hipStreamSynchronize(st), "workspace status read");
  if (!rc && reset) rc = check(launch_fill_zero(static_cast<float*>(workspace), 4096 / 4, st), "sync area reset");
  if (rc) return rc;
  return flag ? 1 : 0;
}

size_t svdmlp_workspace_bytes(int64_t T, int64_t d, int64_t ff, int64_t r, int32_t w_dtype) {
  (void)w_dtype;
  if (T <= 0 || d <= 0 || ff <= 0 || r <= 0) return 0;
  return ws_layout(T, d, ff, r).total;
}

int svdmlp_gate_up(const void* x, const void* ug, const void* vg, const void* uu, const void* vu,
                   const float* s_ug, const float* s_vg, const float* s_uu, const float* s_vu, void* h,
                   int64_t T, int64_t d, int64_t ff, int64_t r, int32_t act_dtype, int32_t w_dtype,
                   uint32_t flags, void* workspace, size_t ws_bytes, void* stream) {
  g_err.clear();
  int rc = validate_dims(T, d, ff, r);
  if (rc) return rc;
  if ((rc = check_types(act_dtype, w_dtype))) return rc;
  if (!x || !ug || !vg || !uu || !vu || !h || !workspace) return fail("null pointer argument");
  const bool fp8 = w_dtype == SVDMLP_FP8_E4M3;
  if (fp8 && (!s_ug || !s_vg || !s_uu || !s_vu)) return fail("fp8 weights need per-column scales");
  if (flags & ~(SVDMLP_U_LINEAR | SVDMLP_V_LINEAR | SVDMLP_OUT_T)) return fail("unsupported flags 0x%x", flags);
  if (fp8 && (flags & (SVDMLP_U_LINEAR | SVDMLP_V_LINEAR))) return fail("fp8 weights must use the natural layout");
  const Ws L = ws_layout(T, d, ff, r);
  if (ws_bytes < L.need) return fail("workspace too small: need %zu bytes, got %zu", L.need, ws_bytes);
  const Common c{act_dtype, w_dtype, act_dtype == SVDMLP_F32, (hipStream_t)stream};
  const bool u_lin = flags & SVDMLP_U_LINEAR, v_lin = flags & SVDMLP_V_LINEAR, out_t = flags & SVDMLP_OUT_T;
  bool vec = d % 8 == 0 && ff % 8 == 0 && r % 8 == 0 && (!out_t || T % 8 == 0);
  for (const void* q : {x, ug, vg, uu, vu, (const void*)h, (const void*)workspace}) vec = vec && aligned16(q);
  if (fp8 && !vec) return fail("fp8 weights need d, ff and r to be multiples of 8 and 16-byte aligned buffers");
  char* ws = static_cast<char*>(workspace);

  if (decode_ok(c, T, {d, ff, r}, vec)) {
    float* xu32 = reinterpret_cast<float*>(ws + L.xu32);
    float* g32 = reinterpret_cast<float*>(ws + L.gu32);
    float* u32 = g32 + T * ff;
    {
      StageScope z(ST_ZERO, c.st);
      rc = check(launch_fill_zero(xu32, (int64_t)(L.h - L.xu32) / 4, c.st), "zero accumulators");
    }
    if (rc) return rc;
    const Operand ax{x, nullptr, d};
    const Operand a1[2] = {ax, ax};
    const void* w1[2] = {ug, uu};
    const float* s1[2] = {s_ug, s_uu};
    const int n1[2] = {(int)r, (int)r};
    float* o1[2] = {xu32, xu32 + T * r};
    rc = decode_stage(c, ST_DEC_GU_XU, T, d, 2, a1, SRC_BF16, w1, fp8 ? s1 : nullptr, u_lin, n1, o1, "decode X.U");
    if (rc) return rc;
    const Operand a2[2] = {Operand{xu32, nullptr, r}, Operand{xu32 + T * r, nullptr, r}};
    const void* w2[2] = {vg, vu};
    const float* s2[2] = {s_vg, s_vu};
    const int n2[2] = {(int)ff, (int)ff};
    float* o2[2] = {g32, u32};
    rc = decode_stage(c, ST_DEC_GU_XUV, T, r, 2, a2, SRC_F32, w2, fp8 ? s2 : nullptr, v_lin, n2, o2, "decode XU.V");
    if (rc) return rc;
    StageScope fin(ST_FINALIZE, c.st);
    return check(launch_finalize(g32, u32, ff, static_cast<uint16_t*>(h), out_t ? T : ff, T, ff, true, out_t, c.st),
                 "SwiGLU finalize");
  }

  if (big_ok(c, vec, {T * d * 2, d * r * 2, r * ff * 2, T * ff * 2}, {d, r})) {
    const void* us[2] = {ug, uu};
    const float* sus[2] = {s_ug, s_uu};
    if ((rc = big_xu(c, ST_GU_XU, x, d, T * d * 2, us, u_lin, T, d, r, 2, ws, L, fp8 ? sus : nullptr))) return rc;
    const uint16_t* xu = reinterpret_cast<const uint16_t*>(ws + L.xu_bf16);
    uint16_t* gbuf = reinterpret_cast<uint16_t*>(ws + L.g);
    // (I, S) output (the reference's TPU launcher fused_mlp_up_T,
    // test_speedup.py:522-544): h in the natural layout into the workspace's
    // h region, then one transpose pass into the caller's buffer
    uint16_t* hn = out_t ? reinterpret_cast<uint16_t*>(ws + L.h) : static_cast<uint16_t*>(h);
    if ((rc = big_swiglu(c, xu, xu + T * r, vg, vu, v_lin, T, r, ff, gbuf, hn, reinterpret_cast<float*>(ws + L.part),
                         (int64_t)(L.norm - L.part), fp8 ? s_vg : nullptr, fp8 ? s_vu : nullptr)) ||
        !out_t)
      return rc;
    StageScope fin(ST_FINALIZE, c.st);
    return check(launch_transpose_bf16(hn, ff, static_cast<uint16_t*>(h), T, (int)T, (int)ff, c.st), "h transpose");
  }

  const Operand ax{x, nullptr, d};
  const void* us[2] = {ug, uu};
  const float* sus[2] = {s_ug, s_uu};
  int a_src = 0;
  const void* xu = nullptr;
  int64_t xu_bs = 0;
  rc = prefill_xu(c, ax, true, us, fp8 ? sus : nullptr, u_lin, T, d, r, 2, vec, ws, L, 0, &a_src, &xu, &xu_bs);
  if (rc) return rc;
  return prefill_swiglu(c, a_src, xu, xu_bs, vg, vu, fp8 ? s_vg : nullptr, fp8 ? s_vu : nullptr, v_lin, T, r, ff,
                        vec, out_t, h);
}

int svdmlp_xuv(const void* x, const void* u, const void* v, const float* s_u, const float* s_v, void* y,
               int64_t T, int64_t din, int64_t dout, int64_t r, int32_t act_dtype, int32_t w_dtype, uint32_t flags,
               void* workspace, size_t ws_bytes, void* stream) {
  g_err.clear();
  int rc = validate_dims(T, din, dout, r);
  if (rc) return rc;
  if ((rc = check_types(act_dtype, w_dtype))) return rc;
  if (!x || !u || !v || !y || !workspace) return fail("null pointer argument");
  const bool fp8 = w_dtype == SVDMLP_FP8_E4M3;
  if (fp8 && (!s_u || !s_v)) return fail("fp8 weights need per-column scales");
  if (flags & ~(SVDMLP_U_LINEAR | SVDMLP_V_LINEAR | SVDMLP_X_T)) return fail("unsupported flags 0x%x", flags);
  if (fp8 && (flags & (SVDMLP_U_LINEAR | SVDMLP_V_LINEAR))) return fail("fp8 weights must use the natural layout");
  const Ws L = ws_layout(T, din, dout, r);
  if (ws_bytes < L.need) return fail("workspace too small: need %zu bytes, got %zu", L.need, ws_bytes);
  const Common c{act_dtype, w_dtype, act_dtype == SVDMLP_F32, (hipStream_t)stream};
  const bool u_lin = flags & SVDMLP_U_LINEAR, v_lin = flags & SVDMLP_V_LINEAR;
  bool x_t = flags & SVDMLP_X_T;
  bool vec = din % 8 == 0 && dout % 8 == 0 && r % 8 == 0 && (!x_t || T % 8 == 0);
  for (const void* q : {x, u, v, (const void*)y, (const void*)workspace}) vec = vec && aligned16(q);
  if (fp8 && !vec) return fail("fp8 weights need d_in, d_out and r to be multiples of 8 and 16-byte aligned buffers");
  char* ws = static_cast<char*>(workspace);
  // x given as (I, S) (the reference's TPU launcher fused_three_mm_XTUV,
  // test_speedup.py:500-519): bf16 x is transposed once into the workspace's
  // h region (unused by this entry point) and the layer runs as for (S, I)
  if (x_t && !c.f32 && vec) {
    uint16_t* xs = reinterpret_cast<uint16_t*>(ws + L.h);
    {
      StageScope ss(ST_FINALIZE, c.st);
      if ((rc = check(launch_transpose_bf16(static_cast<const uint16_t*>(x), T, xs, din, (int)din, (int)T, c.st),
                      "x transpose")))
        return rc;
    }
    x = xs;
    x_t = false;
  }

  if (!x_t && decode_ok(c, T, {din, dout, r}, vec)) {
    float* xd32 = reinterpret_cast<float*>(ws + L.xu32) + 2 * T * r;
    float* y32 = reinterpret_cast<float*>(ws + L.y32);
    {
      StageScope z(ST_ZERO, c.st);
      rc = check(launch_fill_zero(xd32, T * r, c.st), "zero accumulators");
      if (!rc) rc = check(launch_fill_zero(y32, T * dout, c.st), "zero accumulators");
    }
    if (rc) return rc;
    const Operand a1[1] = {Operand{x, nullptr, din}};
    const void* w1[1] = {u};
    const float* s1[1] = {s_u};
    const int n1[1] = {(int)r};
    float* o1[1] = {xd32};
    rc = decode_stage(c, ST_DEC_D_XU, T, din, 1, a1, SRC_BF16, w1, fp8 ? s1 : nullptr, u_lin, n1, o1, "decode X.U");
    if (rc) return rc;
    const Operand a2[1] = {Operand{xd32, nullptr, r}};
    const void* w2[1] = {v};
    const float* s2[1] = {s_v};
    const int n2[1] = {(int)dout};
    float* o2[1] = {y32};
    rc = decode_stage(c, ST_DEC_D_XUV, T, r, 1, a2, SRC_F32, w2, fp8 ? s2 : nullptr, v_lin, n2, o2, "decode XU.V");
    if (rc) return rc;
    StageScope fin(ST_FINALIZE, c.st);
    return check(launch_finalize(y32, nullptr, dout, static_cast<uint16_t*>(y), dout, T, dout, false, false, c.st),
                 "output finalize");
  }

  if (!x_t && big_ok(c, vec, {T * din * 2, din * r * 2, r * dout * 2, T * dout * 2}, {din, r})) {
    const void* us[1] = {u};
    const float* sus[1] = {s_u};
    if ((rc = big_xu(c, ST_D_XU, x, din, T * din * 2, us, u_lin, T, din, r, 1, ws, L, fp8 ? sus : nullptr)))
      return rc;
    return big_v(c, reinterpret_cast<const uint16_t*>(ws + L.xu_bf16), v, v_lin, T, r, dout, ws, L, y,
                 fp8 ? s_v : nullptr);
  }

  const Operand ax{x, nullptr, x_t ? T : din};
  const void* us[1] = {u};
  const float* sus[1] = {s_u};
  int a_src = 0;
  const void* xu = nullptr;
  int64_t xu_bs = 0;
  rc = prefill_xu(c, ax, !x_t, us, fp8 ? sus : nullptr, u_lin, T, din, r, 1, vec, ws, L, 2, &a_src, &xu, &xu_bs);
  if (rc) return rc;
  return prefill_v(c, a_src, xu, v, fp8 ? s_v : nullptr, v_lin, T, r, dout, vec, y);
}

int svdmlp_svd_mlp(const void* x, const void* ug, const void* vg, const void* uu, const void* vu, const void* ud,
                   const void* vd, const float* const* scales, void* y, int64_t T, int64_t d, int64_t ff,
                   int64_t r_gu, int64_t r_d, int32_t act_dtype, int32_t w_dtype, uint32_t flags, void* workspace,
                   size_t ws_bytes, void* stream) {
  return svdmlp_svd_mlp_ld(x, ug, vg, uu, vu, ud, vd, scales, nullptr, y, T, d, ff, r_gu, r_d, act_dtype, w_dtype, flags,
                           workspace, ws_bytes, stream);
}

int svdmlp_svd_mlp_ld(const void* x, const void* ug, const void* vg, const void* uu, const void* vu, const void* ud,
                      const void* vd, const float* const* scales, const int64_t* ld_in, void* y, int64_t T, int64_t d,
                      int64_t ff, int64_t r_gu, int64_t r_d, int32_t act_dtype, int32_t w_dtype, uint32_t flags,
                      void* workspace, size_t ws_bytes, void* stream) {
  return svdmlp_svd_mlp_ranks(x, ug, vg, uu, vu, ud, vd, scales, ld_in, y, T, d, ff, r_gu, r_gu, r_d, act_dtype,
                              w_dtype, flags, workspace, ws_bytes, stream);
}

}  // extern "C"

namespace {

// The layer (svdmlp_svd_mlp_ranks), or with `blk` the MLP block around it:
// the kernel chosen for the shape applies the block's RMSNorm and residual
// add where it can (the decode layers: both; the streaming-GEMV layer and
// the large-tile path: the residual add), the rest run as their own passes.
int svd_mlp_run(const void* x, const void* ug, const void* vg, const void* uu, const void* vu, const void* ud,
                const void* vd, const float* const* scales, const int64_t* ld_in, void* y, int64_t T, int64_t d,
                int64_t ff, int64_t r_g, int64_t r_u, int64_t r_d, int32_t act_dtype, int32_t w_dtype, uint32_t flags,
                void* workspace, size_t ws_bytes, void* stream, Block* blk) {
  g_err.clear();
  int rc = validate_dims(T, d, ff, std::min(std::min(r_g, r_u), r_d));
  if (rc) return rc;
  if ((rc = check_types(act_dtype, w_dtype))) return rc;
  if (!x || !ug || !vg || !uu || !vu || !ud || !vd || !y || !workspace) return fail("null pointer argument");
  const bool fp8 = w_dtype == SVDMLP_FP8_E4M3;
  if (fp8) {
    if (!scales) return fail("fp8 weights need per-column scales");
    for (int i = 0; i < 6; ++i)
      if (!scales[i]) return fail("fp8 weights need per-column scales");
  }
  if (flags & ~(SVDMLP_U_LINEAR | SVDMLP_V_LINEAR | SVDMLP_CONTRACT | SVDMLP_FP8_ACT))
    return fail("unsupported flags 0x%x", flags);
  const bool contract_asked = flags & SVDMLP_CONTRACT;
  const bool fp8_act = flags & SVDMLP_FP8_ACT;
  flags &= ~(SVDMLP_CONTRACT | SVDMLP_FP8_ACT);
  if (fp8_act && !fp8) return fail("SVDMLP_FP8_ACT needs fp8 factors");
  if (fp8 && flags) return fail("fp8 weights must use the natural layout");
  // one rank for both branches below; two ranks only on the large-tile path
  const bool two = r_g != r_u;
  const int64_t r_gu = r_g;
  const int64_t r = std::max(std::max(r_g, r_u), r_d);
  const Ws L = ws_layout(T, d, ff, r);
  if (ws_bytes < L.need) return fail("workspace too small: need %zu bytes, got %zu", L.need, ws_bytes);
  const Common c{act_dtype, w_dtype, act_dtype == SVDMLP_F32, (hipStream_t)stream, blk};
  const bool u_lin = flags & SVDMLP_U_LINEAR, v_lin = flags & SVDMLP_V_LINEAR;
  bool vec = d % 8 == 0 && ff % 8 == 0 && r_g % 8 == 0 && r_u % 8 == 0 && r_d % 8 == 0;
  for (const void* q : {x, ug, vg, uu, vu, ud, vd, (const void*)y, (const void*)workspace}) vec = vec && aligned16(q);
  if (fp8 && !vec) return fail("fp8 weights need d, ff and ranks to be multiples of 8 and 16-byte aligned buffers");
  FactorLd ld = dense_ld(d, ff, r_gu, r_d);
  ld.uu = r_u;
  ld.vu = ff;
  if (ld_in) {
    const int64_t rows[6] = {r_g, ff, r_u, ff, r_d, d};  // row length of ug, vg, uu, vu, ud, vd
    int64_t got[6];
    for (int i = 0; i < 6; ++i) {
      got[i] = ld_in[i] ? ld_in[i] : rows[i];
      if (got[i] < rows[i])
        return fail("leading dimension %lld of factor %d is below its row length %lld", (long long)got[i], i,
                    (long long)rows[i]);
      if (got[i] != rows[i]) ld.dense = false;
    }
    if (!ld.dense) {
      if (fp8 || c.f32 || flags || !vec)
        return fail("factors with padded rows need bf16 natural-layout factors, 16-byte aligned");
      for (int i = 0; i < 6; ++i)
        if (got[i] % 8) return fail("leading dimensions must be multiples of 8 elements (16-byte rows)");
      if (!two && (got[0] != got[2] || got[1] != got[3]))
        return fail("gate and up factors must share their leading dimensions");
      ld = FactorLd{got[0], got[1], got[4], got[5], false, got[2], got[3]};
    }
  }
  char* ws = static_cast<char*>(workspace);
  // The MLP block on a path that does not fuse its RMSNorm: the RMSNorm pass
  // into the workspace's norm region becomes the layer input.
  auto normed = [&]() -> int {
    if (!blk || blk->norm_done) return SVDMLP_OK;
    void* hn = ws + L.norm;
    blk->norm_done = true;
    x = hn;
    return check(launch_rmsnorm(blk->x, blk->gain, hn, T, d, blk->eps, act_dtype == SVDMLP_BF16, c.st), "RMSNorm");
  };
  const float* S[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  if (fp8)
    for (int i = 0; i < 6; ++i) S[i] = scales[i];

  if (two) {
    // The persistent decode layer (up to 128 tokens) runs each branch at its
    // own rank in phases 1 and 2 (one-branch phase-2 units); the large-tile
    // path does too: X.Ug and X.Uu in one launch (their column tiles side by
    // side), then the g pass over r_g and the u pass over r_u.
    if (decode_layer_ok(c, T, d, ff, r_g, r_d, flags, vec, ld, r_u) &&
        p2split_fits(d, ff, r_g, r_d, decode_layer_grid(decode_layer_mt((int)T)), r_u))
      return decode_layer(c, x, ug, vg, uu, vu, ud, vd, y, T, d, ff, r_g, r_d, ws, L, ld, false, r_u);
    const bool big2 = T > kDecodeMaxT &&
                      big_ok(c, vec, {T * d * 2, d * ld.u * 2, d * ld.uu * 2, r_g * ld.v * 2, r_u * ld.vu * 2,
                                      T * ff * 2, ff * ld.ud * 2, r_d * ld.vd * 2},
                             {d, r_g, r_u, ff, r_d});
    if (!big2) {
      fail("distinct gate and up ranks (%lld, %lld) run on the persistent decode layer (bf16 natural-layout "
           "factors, up to %lld tokens, d and ranks multiples of 128, ff of 128) and the large-tile path (bf16 "
           "activations, bf16 or fp8 weights, more than %lld tokens, 16-byte aligned, d, ff and ranks multiples "
           "of 32); pad the smaller branch with zero U columns and V rows for this shape",
           (long long)r_g, (long long)r_u, (long long)kDlMaxT, (long long)kDecodeMaxT);
      return SVDMLP_EUNSUP;
    }
    if ((rc = normed())) return rc;
    const void* us[2] = {ug, uu};
    const float* sus[2] = {S[0], S[2]};
    if ((rc = big_xu2(c, ST_GU_XU, x, d, T * d * 2, us, u_lin, (int)T, (int)d, (int)r_g, (int)r_u, ws, L, sus,
                      ld.u, ld.uu)))
      return rc;
    const uint16_t* xu = reinterpret_cast<const uint16_t*>(ws + L.xu_bf16);
    uint16_t* hbuf = reinterpret_cast<uint16_t*>(ws + L.h);
    uint16_t* gbuf = reinterpret_cast<uint16_t*>(ws + L.g);
    // h in 16 x 16 block-major order between the u pass and h.Ud (the fp8
    // activation path quantises row-major h)
    const bool f8a = fp8_act && f8_down_ok(T, ff, r_d, ld.ud);
    bool hblk = !f8a && tune().hblk;
    if ((rc = big_swiglu(c, xu, xu + T * r_g, vg, vu, v_lin, (int)T, (int)r_g, (int)ff, gbuf, hbuf,
                         reinterpret_cast<float*>(ws + L.part), (int64_t)(L.norm - L.part), S[1], S[3], ld.v,
                         (int)r_u, ld.vu, &hblk)))
      return rc;
    const void* ud1[1] = {ud};
    const float* sud[1] = {S[4]};
    if (f8a) {
      if ((rc = f8_down_xu(c, hbuf, ud, S[4], ld.ud, (int)T, (int)ff, (int)r_d, ws, L))) return rc;
    } else if ((rc = big_xu(c, ST_D_XU, hbuf, ff, T * ff * 2, ud1, u_lin, T, ff, r_d, 1, ws, L, sud, ld.ud, hblk))) {
      return rc;
    }
    return big_v(c, reinterpret_cast<const uint16_t*>(ws + L.xu_bf16), vd, v_lin, T, r_d, d, ws, L, y, S[5], ld.vd);
  }

  // With padded V rows the MFMA decode layers are the faster ones at every T
  // (8B layer at T=1: 75.5 us against 78 us): the streaming-GEMV layer reads
  // whole 1 KB row pieces, which the padding does not spread over channels.
  // With dense factors the four-phase MFMA layer runs one-branch phase-2
  // units at every T where they fit (decode_layer) and beats the
  // streaming-GEMV layer (8B layer, dense V, T=1 / 2: 72.6 / 71.7 us against
  // 78.0 / 81.3).  The contracted instance first wherever it applies (asked
  // for, or where it is the fastest: kDlContractAuto*), then the
  // streaming-GEMV layer where the MFMA layers cannot run one-branch units,
  // then the four-phase MFMA layer.
  const bool mfma_layer = decode_layer_ok(c, T, d, ff, r_gu, r_d, flags, vec, ld);
  const bool dense_p2 = mfma_layer && ld.dense && tune().p2split > 0 &&
                        p2split_fits(d, ff, r_gu, r_d, decode_layer_grid(decode_layer_mt((int)T)));
  const bool contract =
      contract_asked ||
      (tune().contract && T <= (ld.dense ? kDlContractAutoDense : kDlContractAutoPadded));
  if (mfma_layer && contract && decode_contract_ok(T, ff, r_gu, r_d, L, ws_bytes))
    return decode_layer(c, x, ug, vg, uu, vu, ud, vd, y, T, d, ff, r_gu, r_d, ws, L, ld, true);
  if (!(mfma_layer && (!ld.dense || dense_p2)) && gemv_layer_ok(c, T, d, ff, r_gu, r_d, flags, vec, ld)) {
    if ((rc = normed())) return rc;
    return gemv_layer(c, x, ug, vg, uu, vu, ud, vd, y, T, d, ff, r_gu, r_d, ws, L, ld);
  }
  if (mfma_layer)
    return decode_layer(c, x, ug, vg, uu, vu, ud, vd, y, T, d, ff, r_gu, r_d, ws, L, ld);
  const bool big = big_ok(c, vec, {T * d * 2, d * ld.u * 2, r_gu * ld.v * 2, T * ff * 2, ff * ld.ud * 2, r_d * ld.vd * 2},
                          {d, r_gu, ff, r_d});
  if (!ld.dense && (T <= kDecodeMaxT || !big))
    return fail("factors with padded rows: no kernel takes this shape (the decode layers need d, ranks and ff in "
                "multiples of 128, 128 and 64, the large-tile path more than %lld tokens)", (long long)kDecodeMaxT);
  if ((rc = normed())) return rc;

  if (decode_ok(c, T, {d, ff, r_gu, r_d}, vec)) {
    float* xu32 = reinterpret_cast<float*>(ws + L.xu32);
    float* xg = xu32;
    float* xuu = xu32 + T * r;
    float* xd = xu32 + 2 * T * r;
    float* g32 = reinterpret_cast<float*>(ws + L.gu32);
    float* u32 = g32 + T * ff;
    float* y32 = reinterpret_cast<float*>(ws + L.y32);
    {
      StageScope z(ST_ZERO, c.st);
      rc = check(launch_fill_zero(xu32, (int64_t)(L.part - L.xu32) / 4, c.st), "zero accumulators");
    }
    if (rc) return rc;
    const Operand ax{x, nullptr, d};
    {
      const Operand a[2] = {ax, ax};
      const void* w[2] = {ug, uu};
      const float* s[2] = {S[0], S[2]};
      const int n[2] = {(int)r_gu, (int)r_gu};
      float* o[2] = {xg, xuu};
      if ((rc = decode_stage(c, ST_DEC_GU_XU, T, d, 2, a, SRC_BF16, w, s, u_lin, n, o, "decode X.U"))) return rc;
    }
    {
      const Operand a[2] = {Operand{xg, nullptr, r_gu}, Operand{xuu, nullptr, r_gu}};
      const void* w[2] = {vg, vu};
      const float* s[2] = {S[1], S[3]};
      const int n[2] = {(int)ff, (int)ff};
      float* o[2] = {g32, u32};
      if ((rc = decode_stage(c, ST_DEC_GU_XUV, T, r_gu, 2, a, SRC_F32, w, s, v_lin, n, o, "decode XU.V"))) return rc;
    }
    {
      const Operand a[1] = {Operand{g32, u32, ff}};
      const void* w[1] = {ud};
      const float* s[1] = {S[4]};
      const int n[1] = {(int)r_d};
      float* o[1] = {xd};
      if ((rc = decode_stage(c, ST_DEC_D_XU, T, ff, 1, a, SRC_SWIGLU, w, s, u_lin, n, o, "decode h.Ud"))) return rc;
    }
    {
      const Operand a[1] = {Operand{xd, nullptr, r_d}};
      const void* w[1] = {vd};
      const float* s[1] = {S[5]};
      const int n[1] = {(int)d};
      float* o[1] = {y32};
      if ((rc = decode_stage(c, ST_DEC_D_XUV, T, r_d, 1, a, SRC_F32, w, s, v_lin, n, o, "decode XUd.Vd"))) return rc;
    }
    StageScope fin(ST_FINALIZE, c.st);
    return check(launch_finalize(y32, nullptr, d, static_cast<uint16_t*>(y), d, T, d, false, false, c.st),
                 "output finalize");
  }

  // Prefill: h stays in the workspace between the two halves.
  if (big) {
    const void* us[2] = {ug, uu};
    const float* sus[2] = {S[0], S[2]};
    if ((rc = big_xu(c, ST_GU_XU, x, d, T * d * 2, us, u_lin, T, d, r_gu, 2, ws, L, sus, ld.u))) return rc;
    const uint16_t* xu = reinterpret_cast<const uint16_t*>(ws + L.xu_bf16);
    uint16_t* hbuf = reinterpret_cast<uint16_t*>(ws + L.h);
    uint16_t* gbuf = reinterpret_cast<uint16_t*>(ws + L.g);
    const bool f8a = fp8_act && f8_down_ok(T, ff, r_d, ld.ud);
    bool hblk = !f8a && tune().hblk;
    if ((rc = big_swiglu(c, xu, xu + T * r_gu, vg, vu, v_lin, T, r_gu, ff, gbuf, hbuf,
                         reinterpret_cast<float*>(ws + L.part), (int64_t)(L.norm - L.part), S[1], S[3], ld.v, 0, 0,
                         &hblk)))
      return rc;
    const void* ud1[1] = {ud};
    const float* sud[1] = {S[4]};
    if (f8a) {
      if ((rc = f8_down_xu(c, hbuf, ud, S[4], ld.ud, (int)T, (int)ff, (int)r_d, ws, L))) return rc;
    } else if ((rc = big_xu(c, ST_D_XU, hbuf, ff, T * ff * 2, ud1, u_lin, T, ff, r_d, 1, ws, L, sud, ld.ud, hblk))) {
      return rc;
    }
    return big_v(c, reinterpret_cast<const uint16_t*>(ws + L.xu_bf16), vd, v_lin, T, r_d, d, ws, L, y, S[5], ld.vd);
  }

  const Operand ax{x, nullptr, d};
  const void* us[2] = {ug, uu};
  const float* sus[2] = {S[0], S[2]};
  int a_src = 0;
  const void* xu = nullptr;
  int64_t xu_bs = 0;
  rc = prefill_xu(c, ax, true, us, fp8 ? sus : nullptr, u_lin, T, d, r_gu, 2, vec, ws, L, 0, &a_src, &xu, &xu_bs);
  if (rc) return rc;
  void* hbuf = ws + L.h;
  rc = prefill_swiglu(c, a_src, xu, xu_bs, vg, vu, S[1], S[3], v_lin, T, r_gu, ff, vec, false, hbuf);
  if (rc) return rc;
  const Operand ah{hbuf, nullptr, ff};
  const void* ud1[1] = {ud};
  const float* sud[1] = {S[4]};
  rc = prefill_xu(c, ah, true, ud1, fp8 ? sud : nullptr, u_lin, T, ff, r_d, 1, vec, ws, L, 2, &a_src, &xu, &xu_bs);
  if (rc) return rc;
  return prefill_v(c, a_src, xu, vd, S[5], v_lin, T, r_d, d, vec, y);
}

}  // namespace

extern "C" {

int svdmlp_svd_mlp_ranks(const void* x, const void* ug, const void* vg, const void* uu, const void* vu,
                         const void* ud, const void* vd, const float* const* scales, const int64_t* ld_in, void* y,
                         int64_t T, int64_t d, int64_t ff, int64_t r_g, int64_t r_u, int64_t r_d, int32_t act_dtype,
                         int32_t w_dtype, uint32_t flags, void* workspace, size_t ws_bytes, void* stream) {
  return svd_mlp_run(x, ug, vg, uu, vu, ud, vd, scales, ld_in, y, T, d, ff, r_g, r_u, r_d, act_dtype, w_dtype, flags,
                     workspace, ws_bytes, stream, nullptr);
}

}  // extern "C"
