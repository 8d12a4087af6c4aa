/*
 * svdmlp.h - C ABI of libsvdmlp.so, the MI355X (gfx950) implementation of the
 * SVD-compressed LLaMA MLP hot path:
 *
 *     h = SiLU(x . Ug . Vg) * (x . Uu . Vu)          (fused Gate/Up)
 *     y = h . Ud . Vd                                 (low-rank XUV Down)
 *
 * Conventions (every entry point):
 *   - All pointers are device pointers owned by the caller (including the
 *     outputs and the workspace); the library never allocates.  Matrices are
 *     dense and row-major with the leading dimension equal to the row length
 *     (the factors of the _ld entry points excepted).
 *   - Factor layouts follow kernels/reference.py: U is (d_in, r), V is
 *     (r, d_out) ("natural" layout).  Setting SVDMLP_U_LINEAR / SVDMLP_V_LINEAR
 *     declares the PyTorch Linear layout instead: U given as (r, d_in) and V as
 *     (d_out, r) (the checkpoint's *_v_proj / *_u_proj tensors, as consumed by
 *     the reference's nki_mm, test_speedup.py:658-666).
 *   - act_dtype is SVDMLP_BF16 or SVDMLP_F32.  w_dtype is the factor dtype:
 *     equal to act_dtype, or SVDMLP_FP8_E4M3 with bf16 activations, in which
 *     case every factor carries one fp32 scale per output column (U: r scales,
 *     V: d_out scales) and the scale pointers must be non-NULL.
 *   - Arithmetic: fp32 accumulation; with bf16 activations the rank-r
 *     intermediate and h are rounded to bf16 (round-to-nearest-even) at each
 *     GEMM boundary and the output is rounded once, as the reference does.
 *   - Work is enqueued on `stream` (a hipStream_t) and is asynchronous.
 *   - Return value: 0 on success; SVDMLP_EINVAL for an invalid argument (the
 *     message is available from svdmlp_last_error(), thread-local); SVDMLP_EHIP
 *     for a HIP runtime error.
 *   - Decode shapes (1 to 128 tokens, bf16) run as one persistent launch of
 *     one block per CU whose phases meet at grid barriers; it needs the whole
 *     device.  Do not run it concurrently with other work on the device
 *     (another stream, another process): blocks that cannot become resident
 *     stall the barriers, whose bounded waits then give up.  A call whose
 *     wait gave up writes NaN into y wherever the result could be incomplete
 *     and records the timeout in the workspace (svdmlp_workspace_status).
 *     Calls on one stream, or on streams ordered by events, are safe.
 */
#ifndef SVDMLP_H
#define SVDMLP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SVDMLP_VERSION 100 /* 1.0.0 */

/* element types */
#define SVDMLP_F32 0
#define SVDMLP_BF16 1
#define SVDMLP_FP8_E4M3 2

/* layout flags */
#define SVDMLP_U_LINEAR 0x1u /* U stored (r, d_in) instead of (d_in, r) */
#define SVDMLP_V_LINEAR 0x2u /* V stored (d_out, r) instead of (r, d_out) */
#define SVDMLP_OUT_T 0x4u    /* gate_up: write h transposed, (ff, T) */
#define SVDMLP_X_T 0x8u      /* xuv: input given transposed, (d_in, T) */
/* svd_mlp entry points: the contracted layer (models/modeling_llama.py:865-886,
 * _contracted_mlp: Gate/Up/SwiGLU fused through Down-U, so that h never leaves
 * the kernel and only (T, r_d) partials of XU_d cross blocks).  Taken by the
 * persistent decode layer at 1-4 tokens (bf16, natural layout, ff a multiple
 * of 64, gate/up rank >= 320, a block for each 64-column strip of h and each
 * 128-column tile of XU_d: ff/64 + r_d/128 <= CU count); other shapes run as
 * without the flag (same result: at prefill a (rows x r_d) partial per h
 * strip would move far more bytes than h itself).  Without the flag it is
 * taken where it is the fastest layer (LLaMA3-8B): at one token, and with
 * dense factors (no padded rows) up to three. */
#define SVDMLP_CONTRACT 0x10u

/* svd_mlp entry points with fp8 factors: fp8 activations for the h . Ud
 * stage.  No counterpart in the reference, which has no fp8 path; BASELINE
 * configuration 5 asks for the layer on the CDNA4 fp8 MFMA.  h is quantised
 * to e4m3fn per token row (scale amax / 448) and the stage runs fp8 x fp8
 * MFMAs (v_mfma_scale_f32_16x16x128_f8f6f4, twice the bf16 rate) with fp32
 * accumulation.  Only this stage: rounding an activation to e4m3 costs ~2.6%
 * relative error in the GEMM it feeds, so quantising a second GEMM's input
 * would exceed the 3e-2 fp8 tolerance (LLaMA3-70B shape: the layer with the
 * flag is ~2.7% from the math on dequantised factors, against 0.5% without).
 * Taken on the large-tile path (more than 64 tokens) where ff is a multiple
 * of 128 and r_d of 16; other shapes run as without it.  bf16 factors:
 * SVDMLP_EINVAL. */
#define SVDMLP_FP8_ACT 0x20u

/* status codes */
#define SVDMLP_OK 0
#define SVDMLP_EINVAL (-1)
#define SVDMLP_EHIP (-2)
#define SVDMLP_EUNSUP (-3) /* valid arguments that no kernel of this build takes (see svdmlp_svd_mlp_ranks) */

/* Library version (SVDMLP_VERSION of the build). */
int svdmlp_version(void);

/* Message describing the last failed call on this thread ("" if none). */
const char* svdmlp_last_error(void);

/*
 * Workspace bytes needed by svdmlp_gate_up, svdmlp_xuv and svdmlp_svd_mlp for
 * T tokens, hidden size d, intermediate size ff and (maximum) rank r.  The
 * same workspace may be reused by consecutive calls on one stream of one
 * device.  Its first 4096 bytes must be zero before its first use: they hold
 * the grid-barrier and block-done counters of the persistent decode kernels
 * (the streaming-GEMV layer at 1-2 tokens and the MFMA layer up to 128),
 * which only ever grow, and the MFMA layer's split-K tile counters (from byte
 * 2560), which every call leaves at zero.  The 64-bit word at byte 2304 is
 * the timeout flag (see svdmlp_workspace_status); a nonzero 32-bit value at
 * byte 2312 replaces the default bound of the barrier waits (in polls of
 * about a microsecond; failure tests set a tiny one).
 * Replaces the VMEM planning of test_speedup.py:208-258 (the TPU kernels keep
 * XU in VMEM scratch; here the rank-r intermediate lives in this buffer).
 */
size_t svdmlp_workspace_bytes(int64_t T, int64_t d, int64_t ff, int64_t r, int32_t w_dtype);

/*
 * Timeout status of a workspace's persistent decode kernels (no counterpart
 * in the reference, whose kernels have no cross-block waits).  Returns 1 if a
 * grid-barrier wait of an earlier call on this workspace gave up (those calls
 * wrote NaN into y wherever their result could be incomplete; the flag stays
 * set, and later decode calls write NaN too, until reset), 0 if none did, or a
 * negative status.  Waits for `stream` (a hipStream_t) first.  With reset
 * nonzero it then zeroes the 4096-byte sync area (stream-ordered), which makes
 * the workspace usable again; no call may be in flight on the workspace then.
 * The reference rejects non-finite layer outputs (test_speedup.py:852-853,
 * bench/checkpoint_speedup.py:24-25); this names the cause.
 */
int svdmlp_workspace_status(void* workspace, size_t ws_bytes, int32_t reset, void* stream);

/*
 * Fused Gate/Up with the SwiGLU epilogue:
 *   h = SiLU((x . ug) . vg) * ((x . uu) . vu),  x (T, d), h (T, ff)
 * (or h^T (ff, T) with SVDMLP_OUT_T).  Gate and up must have equal shapes.
 * Replaces kernels/reference.py:54-72 (fused_gate_up_ref) and the Pallas
 * launcher fused_mlp_up_T, test_speedup.py:522-544 (which returns (I, S)).
 */
int svdmlp_gate_up(const void* x, const void* ug, const void* vg, const void* uu, const void* vu,
                   const float* s_ug, const float* s_vg, const float* s_uu, const float* s_vu, void* h,
                   int64_t T, int64_t d, int64_t ff, int64_t r, int32_t act_dtype, int32_t w_dtype,
                   uint32_t flags, void* workspace, size_t ws_bytes, void* stream);

/*
 * Low-rank projection y = (x . u) . v, x (T, d_in) (or x^T (d_in, T) with
 * SVDMLP_X_T), u (d_in, r), v (r, d_out), y (T, d_out).
 * Replaces kernels/reference.py:75-82 (fused_xuv_ref) and the Pallas launcher
 * fused_three_mm_XTUV, test_speedup.py:500-519 (which takes x as (I, S)).
 */
int svdmlp_xuv(const void* x, const void* u, const void* v, const float* s_u, const float* s_v, void* y,
               int64_t T, int64_t din, int64_t dout, int64_t r, int32_t act_dtype, int32_t w_dtype,
               uint32_t flags, void* workspace, size_t ws_bytes, void* stream);

/*
 * The whole SVD-MLP layer, y = xuv(gate_up(x)), with h rounded to the
 * activation dtype between the two halves (kernels/reference.py:85-93,
 * svd_mlp_ref; test_speedup.py:631-655, svd_mlp_with_fused_kernel).  Gate/up
 * rank r_gu and down rank r_d may differ.  h does not leave the workspace; at
 * decode shapes it is never materialised at all.
 */
int svdmlp_svd_mlp(const void* x, const void* ug, const void* vg, const void* uu, const void* vu,
                   const void* ud, const void* vd, const float* const* scales /* 6 or NULL */, void* y,
                   int64_t T, int64_t d, int64_t ff, int64_t r_gu, int64_t r_d, int32_t act_dtype,
                   int32_t w_dtype, uint32_t flags, void* workspace, size_t ws_bytes, void* stream);

/*
 * One MLP block of the model: y = x + svd_mlp(RMSNorm(x) * norm_w), with
 * RMSNorm in fp32 (x * rsqrt(mean(x^2) + eps), times the fp32 gain, rounded
 * to the activation dtype) and the residual add rounded to the activation
 * dtype.  norm_w holds d fp32 gains; y must not alias x.  Replaces the MLP
 * half of bench/e2e_block.py:268-278 (_fused_svd_block) with LlamaRMSNorm,
 * models/modeling_llama.py:253-262.  The persistent decode layers run the
 * whole block in their one launch (a phase 0 writes RMSNorm(x), one block
 * per token row, before the layer's first grid barrier; the last phase adds
 * the residual as it writes y); the streaming-GEMV layer and the large-tile
 * path add the residual in their output stage after a separate RMSNorm pass;
 * the other paths run both as passes of their own.
 */
int svdmlp_svd_mlp_block(const void* x, const float* norm_w, float eps, const void* ug, const void* vg,
                         const void* uu, const void* vu, const void* ud, const void* vd,
                         const float* const* scales /* 6 or NULL */, void* y, int64_t T, int64_t d, int64_t ff,
                         int64_t r_gu, int64_t r_d, int32_t act_dtype, int32_t w_dtype, uint32_t flags,
                         void* workspace, size_t ws_bytes, void* stream);

/*
 * svdmlp_svd_mlp and svdmlp_svd_mlp_block for factors whose rows are padded
 * (no counterpart in the reference, whose operators take dense arrays; the
 * math is that of kernels/reference.py:85-93).  ld holds the leading
 * dimension (elements between consecutive rows as stored) of ug, vg, uu, vu,
 * ud, vd in that order; 0 or a NULL ld means the row length.  Padded factors
 * must be bf16, natural layout, 16-byte aligned, with leading dimensions
 * that are multiples of 8 and equal for gate and up.  With row pitches that
 * are multiples of 4 KB (V rows of 4096 or 14336 bf16 elements), each column
 * stripe of a factor maps onto a fixed subset of HBM channels, and at
 * decode shapes the slowest such subset bounds the weight stream; padding
 * V rows by 64 elements spreads every stripe over all channels (8B layer at
 * 8 tokens: 82 -> 75 us; with padded factors the MFMA decode layer also
 * takes 1-2 tokens, 74.5 us against 77.6 us at one token).  Shapes that only other kernels take (fp32, fp8,
 * Linear layout, odd sizes) return SVDMLP_EINVAL with padded factors.
 */
int svdmlp_svd_mlp_ld(const void* x, const void* ug, const void* vg, const void* uu, const void* vu,
                      const void* ud, const void* vd, const float* const* scales /* 6 or NULL */,
                      const int64_t* ld /* 6 or NULL */, void* y, int64_t T, int64_t d, int64_t ff, int64_t r_gu,
                      int64_t r_d, int32_t act_dtype, int32_t w_dtype, uint32_t flags, void* workspace,
                      size_t ws_bytes, void* stream);
int svdmlp_svd_mlp_block_ld(const void* x, const float* norm_w, float eps, const void* ug, const void* vg,
                            const void* uu, const void* vu, const void* ud, const void* vd,
                            const float* const* scales /* 6 or NULL */, const int64_t* ld /* 6 or NULL */, void* y,
                            int64_t T, int64_t d, int64_t ff, int64_t r_gu, int64_t r_d, int32_t act_dtype,
                            int32_t w_dtype, uint32_t flags, void* workspace, size_t ws_bytes, void* stream);

/*
 * svdmlp_svd_mlp_ld and svdmlp_svd_mlp_block_ld with a gate rank r_g and an
 * up rank r_u of their own: ug (d, r_g), vg (r_g, ff), uu (d, r_u),
 * vu (r_u, ff).  kernels/reference.py:54-72 (fused_gate_up_ref) places no
 * constraint between the two ranks; the reference's TPU launcher rejects
 * them ("gate/up factors must have matching shapes", test_speedup.py:
 * 532-533), so its non-uniform models zero-pad the smaller branch.  Here
 * each branch runs at its own rank on the large-tile path (more than 128
 * tokens, bf16 activations, bf16 or fp8 weights, 16-byte aligned, d, ff
 * and ranks multiples of 32); with padded rows, gate and up may have pitches
 * of their own.  Other shapes with r_g != r_u return SVDMLP_EUNSUP (pad the
 * smaller branch with zero U columns and V rows, which changes nothing in
 * the result, and call with one rank).  The workspace is sized with
 * r = max(r_g, r_u, r_d).  r_g == r_u is svdmlp_svd_mlp_ld.
 */
int svdmlp_svd_mlp_ranks(const void* x, const void* ug, const void* vg, const void* uu, const void* vu,
                         const void* ud, const void* vd, const float* const* scales /* 6 or NULL */,
                         const int64_t* ld /* 6 or NULL */, void* y, int64_t T, int64_t d, int64_t ff, int64_t r_g,
                         int64_t r_u, int64_t r_d, int32_t act_dtype, int32_t w_dtype, uint32_t flags,
                         void* workspace, size_t ws_bytes, void* stream);
int svdmlp_svd_mlp_block_ranks(const void* x, const float* norm_w, float eps, const void* ug, const void* vg,
                               const void* uu, const void* vu, const void* ud, const void* vd,
                               const float* const* scales /* 6 or NULL */, const int64_t* ld /* 6 or NULL */,
                               void* y, int64_t T, int64_t d, int64_t ff, int64_t r_g, int64_t r_u, int64_t r_d,
                               int32_t act_dtype, int32_t w_dtype, uint32_t flags, void* workspace,
                               size_t ws_bytes, void* stream);

/*
 * svdmlp_svd_mlp_ld without a workspace argument: the layer runs in a fixed
 * scratch area that the library holds in device memory (64 MiB per device
 * that the library runs on, until the process ends), so the call allocates
 * nothing.  No counterpart in the reference; it is for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  Shapes whose workspace
 * (svdmlp_workspace_bytes) exceeds 64 MiB are rejected with SVDMLP_EINVAL
 * (LLaMA3-8B: up to 64 tokens; prefill shapes need a workspace).  The first
 * call on a device looks the scratch up and clears its sync area on `stream`
 * (the current device's).  Every call on a device shares that device's
 * scratch and leaves its contents behind: calls that overlap on one device
 * (different streams, threads) race; serialise them.  A call whose
 * grid-barrier waits give up writes NaN into y and sets the scratch's sticky
 * timeout flag, after which every later call on that device writes NaN too
 * until svdmlp_noalloc_status resets the scratch.
 */
int svdmlp_svd_mlp_noalloc(const void* x, const void* ug, const void* vg, const void* uu, const void* vu,
                           const void* ud, const void* vd, const float* const* scales /* 6 or NULL */,
                           const int64_t* ld /* 6 or NULL */, void* y, int64_t T, int64_t d, int64_t ff,
                           int64_t r_gu, int64_t r_d, int32_t act_dtype, int32_t w_dtype, uint32_t flags,
                           void* stream);

/*
 * svdmlp_workspace_status for the fixed scratch of svdmlp_svd_mlp_noalloc on
 * the current device (no counterpart in the reference; for the same callers).
 * Waits for `stream`, then returns 1 if a grid-barrier wait of an earlier
 * noalloc call gave up (its y and those of the calls after it hold NaN), 0 if
 * not, or a negative status.  reset != 0 then zeroes the scratch's 4096-byte
 * sync area (a fill kernel on `stream`), after which calls compute again.
 * wait_bound >= 0 afterwards sets the bound of the barrier waits in polls
 * (0: the default of 2^22 polls, seconds; failure tests set 1 so that every
 * wait gives up at once and every kernel still runs to its end); a negative
 * wait_bound leaves it.  Allocates no device memory; it synchronises, so it
 * does not belong inside graph capture.
 */
int svdmlp_noalloc_status(int32_t reset, int64_t wait_bound, void* stream);

/*
 * Per-stage GPU timing (no counterpart in the reference, whose timing is host
 * wall clock around block_until_ready, test_speedup.py:739-749).  While
 * enabled, every stage launch of the calls above is bracketed by hipEvents
 * on the caller's stream.  svdmlp_profile_read waits for the recorded events,
 * writes per-stage total milliseconds and launch counts for the first n
 * stages, clears the totals and returns the number of stages (or a negative
 * status).  svdmlp_stage_name names stage i ("" when out of range).
 * svdmlp_profile_enable returns the number of stages.
 */
int svdmlp_profile_enable(int enable);
int svdmlp_profile_read(double* total_ms, int64_t* launches, int n);
const char* svdmlp_stage_name(int stage);

#ifdef __cplusplus
}
#endif

#endif /* SVDMLP_H */
