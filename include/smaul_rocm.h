/*
 * smaul_rocm.h -- C ABI of the MI355X (gfx950) tiled-FP8 MoE forward library
 * (libsmaul_rocm.so).
 *
 * Storage format (unchanged from the reference, kernel/fp8_tile.py:199-215):
 *   codes  uint8 [out_f, in_f]            E4M3 with 0x7F/0xFF decoding to +-448
 *   scales fp32  [out_f, ceil(in_f/tile)] one scale per (output row, K tile)
 *   decoded weight W[o, k] = lut[codes[o, k]] * scales[o, k / tile]
 *
 * Conventions of every entry point:
 *   - all pointers are device pointers unless stated otherwise;
 *   - work is enqueued on `stream`, asynchronously; nothing synchronises;
 *   - nothing allocates: callers pass outputs and, where needed, a workspace
 *     whose size comes from the matching *_workspace_size query;
 *   - the return value is SMAUL_OK or an error code; smaul_last_error() gives
 *     a message for the calling thread's most recent failure.
 *
 * Activation dtypes: SMAUL_DTYPE_BF16 or SMAUL_DTYPE_F32.  bf16 activations are
 * fed to bf16 MFMA directly; fp32 activations are split into two bf16 terms
 * (hi + lo) so the product keeps ~16 more bits than a single bf16 rounding.
 */
#ifndef SMAUL_ROCM_H
#define SMAUL_ROCM_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  SMAUL_OK = 0,
  SMAUL_ERR_INVALID = 1,      /* bad argument (size, pointer, dtype)          */
  SMAUL_ERR_UNSUPPORTED = 2,  /* valid for the reference, not supported here  */
  SMAUL_ERR_HIP = 3           /* a HIP runtime call or launch failed          */
};

enum { SMAUL_DTYPE_F32 = 0, SMAUL_DTYPE_BF16 = 1 };

/* flags: SMAUL_FLAG_CANONICAL_CODES promises that the code buffers contain no
 * 0x7F/0xFF bytes (see smaul_fp8_canonicalize), which lets the GEMMs skip
 * rewriting them on the fly.  SMAUL_FLAG_ALIGNED_CODES promises that every
 * expert code buffer starts on a 16-byte boundary, which lets the grouped
 * GEMMs stage code rows with 16-byte LDS-DMA loads.  Results are identical
 * with or without either flag.  SMAUL_FLAG_TILED_LAYOUT says that the expert
 * code and scale buffers are in the tiled layout of smaul_fp8_tile_layout
 * instead of FP8Linear's [out_f][in_f] / [out_f][in_f / tile]; it needs tile
 * 64 and d, h multiples of 64, is accepted by smaul_moe_forward*,
 * smaul_moe_gate_up, smaul_moe_down and smaul_swiffn_forward (rejected by
 * smaul_fp8_linear), and gives the same results as the reference layout. */
enum { SMAUL_FLAG_CANONICAL_CODES = 1, SMAUL_FLAG_ALIGNED_CODES = 2, SMAUL_FLAG_TILED_LAYOUT = 4 };

/* Library version as an integer (major*10000 + minor*100 + patch). */
int smaul_version(void);

/* Message of the calling thread's last failure ("" if none). */
const char* smaul_last_error(void);

/*
 * Dense tiled-FP8 linear: y[rows, out_f] = x[rows, in_f] . decode(w, s)^T.
 * Replaces the reference backend entry fp8_forward
 *   kernel/compute.py:125-135 (CpuBackend.fp8_forward) and
 *   kernel/fp8_cpu.cpp:100-141 (native fp8_forward).
 * x: x_dtype [rows, in_f] row-major; w: uint8 [out_f, in_f]; s: fp32
 * [out_f, ceil(in_f/tile)]; y: y_dtype [rows, out_f].  tile must be 32 or a
 * multiple of 64 (SMAUL_ERR_UNSUPPORTED otherwise).  rows may be 0.
 */
int smaul_fp8_linear(const void* x, int x_dtype, const uint8_t* w, const float* s,
                     void* y, int y_dtype, int64_t rows, int64_t in_f, int64_t out_f,
                     int64_t tile, int flags, hipStream_t stream);

/*
 * smaul_fp8_linear with a caller workspace, for fp32 x (what the reference's
 * FP8Linear passes, kernel/fp8_tile.py:168; same reference entry as
 * smaul_fp8_linear: kernel/compute.py:125-135, kernel/fp8_cpu.cpp:100-141).
 * fp32 x is computed as x = hi + lo, two bf16 terms (within 2^-18 |x|), with
 * fp32 sums of exact bf16 x E4M3 products.  smaul_fp8_linear splits the terms
 * in LDS inside the GEMM (tile 64, in_f a multiple of 64, out_f a multiple of
 * 128, more than 64 rows, 16-byte aligned x and w); for more than 1024 rows
 * this entry instead writes the two planes into the workspace in a separate
 * pass and runs the GEMM over both (faster for long calls).  With fewer rows,
 * other shapes, or a workspace smaller than smaul_fp8_linear_workspace_size
 * (0 below 1025 rows or for bf16 x), it is smaul_fp8_linear.  Same arguments,
 * results and errors as smaul_fp8_linear within fp32 summation order.
 */
int64_t smaul_fp8_linear_workspace_size(int64_t rows, int64_t in_f, int x_dtype);
int smaul_fp8_linear_ws(const void* x, int x_dtype, const uint8_t* w, const float* s,
                        void* y, int y_dtype, int64_t rows, int64_t in_f, int64_t out_f,
                        int64_t tile, int flags, void* workspace, int64_t workspace_bytes,
                        hipStream_t stream);

/*
 * Device repack cache of the codes: out = codes with 0x7F -> 0x7E and
 * 0xFF -> 0xFE (the same values, +-448, in the reference codebook
 * kernel/fp8_tile.py:43-44; 0x7F/0xFF are NaN in the OCP E4M3FN encoding the
 * gfx950 converters implement).  No reference counterpart: the stored w8
 * buffers are never modified, this writes a separate cached copy.  Both
 * buffers 16-byte aligned.
 */
int smaul_fp8_canonicalize(const uint8_t* codes, uint8_t* out, int64_t n, hipStream_t stream);

/*
 * One FP8Linear weight (codes uint8 [N][K], fp32 scales [N][K / 64], tile 64)
 * rewritten for SMAUL_FLAG_TILED_LAYOUT: codes_out [K / 64][N][64] holds the
 * canonical codes (as smaul_fp8_canonicalize writes them) of each 64-wide K
 * block of every column, scales_out [K / 64][N] the scales.  A stage of the
 * GEMMs (64 K of a run of columns) then reads whole cache lines of codes and
 * of scales instead of one line per column.  No counterpart in the
 * reference: it is the device repack step of a caller that keeps expert
 * weights resident (RocmBackend's expert cache).  K % 64 == 0; code buffers
 * 16-byte aligned; the outputs must not overlap the inputs.
 */
int smaul_fp8_tile_layout(const uint8_t* codes, const float* scales, uint8_t* codes_out, float* scales_out,
                          int64_t N, int64_t K, hipStream_t stream);

/*
 * MoE router: logits = x . gate_w^T (+ gate_b), prob = softmax(logits),
 * (topv, topi) = top-k of prob with torch's CPU selection order, topw =
 * topv / sum(topv) (uniform 1/k when the sum is below 1e-6).
 * Replaces model.py:558-570 (SwiFFN_MoE.forward router, softmax, topk, renorm).
 * x: x_dtype [T, d]; gate_w fp32 [E, d]; gate_b fp32 [E] or NULL.
 * Outputs: prob fp32 [T, E]; topi int64 [T, k]; topw fp32 [T, k].
 * 1 <= k <= min(E, 8), E <= 64, d a multiple of 8.
 */
int smaul_moe_router(const void* x, int x_dtype, const float* gate_w, const float* gate_b,
                     float* prob, int64_t* topi, float* topw,
                     int64_t T, int64_t d, int64_t E, int64_t k, hipStream_t stream);

/*
 * Deterministic dispatch: for each expert e, the tokens t with a positive
 * routing weight for e, in ascending t (the boolean-mask gather order of
 * model.py:574-581).  Replaces the per-expert mask/gather loop there.
 * Inputs: topi int64 [T, k] (distinct experts per row), topw fp32 [T, k].
 * Outputs (int32 unless noted):
 *   counts  [E]       tokens per expert (model.py:577 `n`)
 *   seg_off [E+1]     first logical row of each expert's segment
 *   tile_off[E+1]     first m-tile of each expert for row tiles of `block_m`
 *   perm_row[T*k]     logical row -> token index (first seg_off[E] valid)
 *   perm_w  fp32 [T*k] logical row -> routing weight
 *   inv     [T*k]     token slot (t*k + j) -> logical row, -1 if not dispatched
 * block_m must be 16, 32, 64, 128 or 256.  `workspace` holds
 * smaul_moe_dispatch_workspace_size(T, E) bytes (per-block counts/offsets).
 */
int64_t smaul_moe_dispatch_workspace_size(int64_t T, int64_t E);

int smaul_moe_dispatch(const int64_t* topi, const float* topw, int32_t* counts,
                       int32_t* seg_off, int32_t* tile_off, int32_t* perm_row, float* perm_w,
                       int32_t* inv, int64_t T, int64_t E, int64_t k, int64_t block_m,
                       void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Grouped expert GEMMs over the dispatched segments (SwiFFN, model.py:289-290).
 * Expert weights are addressed through device arrays of device pointers, one
 * entry per expert, so each expert's FP8Linear buffers are used in place.
 *
 * smaul_moe_gate_up: hdn[r, :] = cast(silu(cast(x[perm_row[r]] . Wg^T)) *
 *   cast(x[perm_row[r]] . Wu^T)) where cast is to act_dtype (a no-op for fp32)
 *   -- the rounding points of SwiFFN.forward with FP8Linear outputs in x.dtype.
 *   x: act_dtype [T, d]; hdn: act_dtype [T*k, h].
 * smaul_moe_down: yperm[r, :] = cast(hdn[r] . Wd^T); yperm: act_dtype [T*k, d].
 * seg_off/tile_off come from smaul_moe_dispatch with block_m = smaul_moe_block_m().
 * max_tiles is an upper bound on tile_off[E] (ceil(T*k/block_m) + E).
 * block_m 16 (chosen for T <= 64, bf16, tile 64, d and h multiples of 128)
 * selects the decode-regime kernels, which stream each expert's weights once
 * for all of its rows.  block_m 128 with bf16 activations, tile 64,
 * SMAUL_FLAG_ALIGNED_CODES and 16-byte aligned activations selects the
 * LDS-DMA kernels (the register-staged ones otherwise, on the same tiles).
 * block_m 64 (never returned by smaul_moe_block_m; smaul_moe_forward picks it
 * for small bf16 layers) runs the LDS-DMA kernels on 64-row tiles and needs
 * their conditions (SMAUL_ERR_UNSUPPORTED otherwise); the outputs equal those
 * of block_m 128 bit for bit.
 */
int smaul_moe_block_m(int64_t T, int64_t d, int64_t h, int64_t E, int64_t k, int64_t tile,
                      int act_dtype);

int smaul_moe_gate_up(const void* x, int act_dtype, const int32_t* perm_row,
                      const uint8_t* const* gate_w, const float* const* gate_s,
                      const uint8_t* const* up_w, const float* const* up_s,
                      void* hdn, const int32_t* seg_off, const int32_t* tile_off,
                      int64_t max_tiles, int64_t E, int64_t d, int64_t h, int64_t tile,
                      int64_t block_m, int flags, hipStream_t stream);

int smaul_moe_down(const void* hdn, int act_dtype, const uint8_t* const* down_w,
                   const float* const* down_s, void* yperm, const int32_t* seg_off,
                   const int32_t* tile_off, int64_t max_tiles, int64_t E, int64_t d,
                   int64_t h, int64_t tile, int64_t block_m, int flags, hipStream_t stream);

/*
 * Combine: out[t] = cast( sum over t's dispatched experts in ascending expert
 * id of float(yperm[inv[t,j]]) * topw[t,j] ), accumulated in fp32 from +0 with
 * no fused multiply-add -- model.py:571,582,585.
 * yperm: act_dtype [T*k, d]; out: act_dtype [T, d].
 */
int smaul_moe_combine(const void* yperm, int act_dtype, const int64_t* topi,
                      const float* topw, const int32_t* inv, void* out, int64_t T,
                      int64_t d, int64_t k, hipStream_t stream);

/*
 * Dense SwiGLU FFN over every row: out = cast(cast(silu(cast(x . Wg^T)) *
 * cast(x . Wu^T)) . Wd^T), cast to act_dtype at each point (a no-op for
 * fp32) -- SwiFFN.forward, model.py:289-290, with its three FP8Linear
 * forwards (kernel/fp8_tile.py:237-239, 163-170).  One launch computes gate
 * and up together with the SwiGLU epilogue into the workspace (hdn [rows, h]),
 * a second the down projection into out.  x: act_dtype [rows, d]; gate/up
 * codes uint8 [h, d] with fp32 scales [h, ceil(d/tile)]; down codes [d, h],
 * scales [d, ceil(h/tile)]; out: act_dtype [rows, d].  x, codes, out and the
 * workspace 16-byte aligned; d and h multiples of 16.  `workspace` holds
 * smaul_swiffn_workspace_size(rows, h, act_dtype) bytes.  With fp32 x the
 * size includes room for bf16 hi / lo planes of x and of hdn: when tile is 64,
 * d and h are multiples of 128, d <= h and rows > 64, both GEMMs run on the
 * LDS-DMA kernels over the two planes (products within 2^-18 relative of
 * fp32); a workspace of only the first align256(rows * h * 4) bytes, or any
 * other shape, runs the register-staged kernels.
 */
int64_t smaul_swiffn_workspace_size(int64_t rows, int64_t h, int act_dtype);

int smaul_swiffn_forward(const void* x, int act_dtype, const uint8_t* gate_w8, const float* gate_s,
                         const uint8_t* up_w8, const float* up_s, const uint8_t* down_w8, const float* down_s,
                         void* out, void* workspace, int64_t workspace_bytes, int64_t rows, int64_t d, int64_t h,
                         int64_t tile, int flags, hipStream_t stream);

/*
 * RMSNorm over the rows of x [T, d]: out = cast((x * rsqrt(mean(x^2) + eps)) *
 * weight) computed in fp32, out in act_dtype (the formula of RMSNorm.forward,
 * model.py:124-139).  weight: fp32 [d], or
 * NULL for a weight of ones (the unit-RMS normalisation).  eps must be positive
 * and finite (model.py:127-128).  The row sum of squares is reduced in a
 * different order than torch's, so results agree to fp32 rounding, not bitwise.
 */
int smaul_rms_norm(const void* x, int act_dtype, const float* weight, void* out, int64_t T,
                   int64_t d, float eps, hipStream_t stream);

/*
 * The whole MoE layer (router -> dispatch -> gate_up -> down -> combine) in
 * one call; SwiFFN_MoE.forward of model.py:557-585.  `workspace` must hold
 * smaul_moe_workspace_size(...) bytes (256-byte aligned).  prob/topi/topw are
 * the router outputs (kept by the module as last_prob / last_topi); counts is
 * int32 [E] (expert_token_counts; last_executed is counts > 0).  In the
 * decode regime (T <= 64, bf16, d % 16 == 0, d <= 1024, canonical codes, an
 * 8-wave down instance) the combine runs in the tail of the down-projection
 * kernel, with the same results: the first workgroups to finish their units
 * wait for the rest through a counter in the workspace (cleared by the
 * gate/up kernel of the same call), so two calls must not share one
 * workspace concurrently.  With fp32 x (tile 64, d and h multiples of 128,
 * SMAUL_FLAG_ALIGNED_CODES) both grouped GEMMs run on the LDS-DMA kernels over
 * bf16 hi / lo planes of x and of the hidden rows (products within 2^-18
 * relative of fp32); the fp32 workspace size includes the planes of x.
 */
int64_t smaul_moe_workspace_size(int64_t T, int64_t d, int64_t h, int64_t E, int64_t k,
                                 int act_dtype);

int smaul_moe_forward(const void* x, int act_dtype, const float* gate_w, const float* gate_b,
                      const uint8_t* const* gate_w8, const float* const* gate_s,
                      const uint8_t* const* up_w8, const float* const* up_s,
                      const uint8_t* const* down_w8, const float* const* down_s,
                      void* out, float* prob, int64_t* topi, float* topw, int32_t* counts,
                      void* workspace, int64_t workspace_bytes,
                      int64_t T, int64_t d, int64_t h, int64_t E, int64_t k, int64_t tile,
                      int flags, hipStream_t stream);

/*
 * smaul_moe_forward without a workspace argument: the layer's workspace is a
 * static device array inside the library (SMAUL_NOALLOC_SCRATCH_BYTES, one per
 * GPU, held until the process ends), so the call allocates nothing -- no
 * hipMalloc, no hipFree, no allocating library routine.  No counterpart in
 * the reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  Results
 * are bit-identical to smaul_moe_forward.  Layers whose
 * smaul_moe_workspace_size exceeds SMAUL_NOALLOC_SCRATCH_BYTES are rejected
 * with SMAUL_ERR_UNSUPPORTED (64 MiB: e.g. up to ~4600 tokens at d=1024,
 * h=2560, top-2, bf16; the 64-token decode step needs ~1 MB).  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (two streams,
 * two threads) race and must be serialised by the caller.
 */
#define SMAUL_NOALLOC_SCRATCH_BYTES (64ll << 20)

int smaul_moe_forward_noalloc(const void* x, int act_dtype, const float* gate_w, const float* gate_b,
                              const uint8_t* const* gate_w8, const float* const* gate_s,
                              const uint8_t* const* up_w8, const float* const* up_s,
                              const uint8_t* const* down_w8, const float* const* down_s, void* out,
                              float* prob, int64_t* topi, float* topw, int32_t* counts, int64_t T, int64_t d,
                              int64_t h, int64_t E, int64_t k, int64_t tile, int flags, hipStream_t stream);

/*
 * smaul_moe_forward followed by RMSNorm of its output rows (the formula of
 * RMSNorm.forward, model.py:124-139): out as smaul_moe_forward writes it, and
 * norm_out [T, d] (act_dtype) = smaul_rms_norm(out, norm_w, eps), bit for bit.
 * With d % 16 == 0 and d <= 4096 the norm is fused into the combine kernel
 * (one wave per token), which in the decode regime of smaul_moe_forward runs
 * in the tail of the down-projection kernel; otherwise the two kernels run
 * one after the other.
 * No counterpart in the reference: its Block norms the FFN output in fp32
 * (n4 on fx.float(), model.py:640-641), so norm_out is not that norm; it is
 * for stacks whose next MoE layer reads the normalised rows in act_dtype
 * (the config-4 decode harness).
 */
int smaul_moe_forward_norm(const void* x, int act_dtype, const float* gate_w, const float* gate_b,
                           const uint8_t* const* gate_w8, const float* const* gate_s,
                           const uint8_t* const* up_w8, const float* const* up_s,
                           const uint8_t* const* down_w8, const float* const* down_s,
                           void* out, float* prob, int64_t* topi, float* topw, int32_t* counts,
                           void* workspace, int64_t workspace_bytes,
                           int64_t T, int64_t d, int64_t h, int64_t E, int64_t k, int64_t tile,
                           int flags, const float* norm_w, float eps, void* norm_out,
                           hipStream_t stream);

/*
 * One layer of a chain of MoE layers in which each layer's normalised output
 * is the next layer's input (the config-4 decode harness; a reference Block
 * routes n5(x + f) instead, so it cannot use this fusion):
 * smaul_moe_forward_norm, plus two ways to move routing across the boundary.
 *   routed != 0: prob/topi/topw are INPUTS holding this layer's routing of x
 *     (as smaul_moe_router writes it, e.g. the previous call's next_*); the
 *     layer runs no router of its own.
 *   next_gate_w != NULL: after the norm, norm_out is routed with
 *     next_gate_w [next_E, d] / next_gate_b (may be NULL) and top next_k
 *     into next_prob [T, next_E], next_topi / next_topw [T, next_k], equal
 *     bit for bit to smaul_moe_router(norm_out, ...).  For bf16, next_E <= 16
 *     and d <= 2048 (d % 16 == 0) the router runs inside the combine + norm
 *     kernel; otherwise it is launched after it.  In the decode regime
 *     (T <= 64, bf16, d <= 1024, 4 < next_E <= 16, canonical codes, an 8-wave
 *     down instance) that combine + norm + router runs in the tail of the
 *     down-projection kernel instead, with the same results: the first
 *     workgroups to finish their units wait for the rest through a counter
 *     in the workspace (cleared by the gate/up kernel of the same call), so
 *     two calls must not share one workspace concurrently.
 * out, norm_out, counts and (when not routed) prob/topi/topw are written as
 * by smaul_moe_forward_norm.  No counterpart entry in the reference: its
 * layers run the norm and the next router as separate calls.
 */
int smaul_moe_forward_chain(const void* x, int act_dtype, const float* gate_w, const float* gate_b,
                            const uint8_t* const* gate_w8, const float* const* gate_s,
                            const uint8_t* const* up_w8, const float* const* up_s,
                            const uint8_t* const* down_w8, const float* const* down_s,
                            void* out, float* prob, int64_t* topi, float* topw, int32_t* counts,
                            void* workspace, int64_t workspace_bytes,
                            int64_t T, int64_t d, int64_t h, int64_t E, int64_t k, int64_t tile,
                            int flags, const float* norm_w, float eps, void* norm_out, int routed,
                            const float* next_gate_w, const float* next_gate_b, int64_t next_E,
                            int64_t next_k, float* next_prob, int64_t* next_topi, float* next_topw,
                            hipStream_t stream);

/*
 * Give-ups of the fused decode combine's bounded wait.  In the decode regime
 * the first workgroups of the down-projection kernel to finish wait (a
 * bounded poll) for the others before they combine.  If that wait gives up
 * (another process holding the compute units for tens of milliseconds), the
 * call still returns SMAUL_OK, but every token the waiting workgroup owns is
 * poisoned instead of combined: out (and norm_out) rows NaN, and for a next
 * router next_prob / next_topw NaN and next_topi -1.  Each give-up also adds
 * one to a per-device counter, which this entry reads: it enqueues on
 * `stream` a copy of the current device's count into *out (device int32)
 * and, with reset != 0, subtracts what it copied.  No sync.  No counterpart
 * in the reference (its combine, model.py:582-585, has no wait); callers
 * that need to know a decode call completed check *out == 0.
 */
int smaul_wait_timeouts(int32_t* out, int reset, hipStream_t stream);

/*
 * Test hook for the wait above (no counterpart in the reference): later
 * decode-regime calls from any thread wait for `extra_arrivals` more
 * workgroups than the grid holds and poll at most `spin_limit` times, so a
 * test can make every wait give up while every kernel still exits normally.
 * (0, 1 << 20) restores the defaults.  Not for use beside other work.
 */
int smaul_debug_tail_wait(int extra_arrivals, int spin_limit);

/*
 * Linear-attention recurrence of SmaulLinear, per (batch, head):
 *   kn_t = k_t / max(||k_t||, 1e-6),  S_t = S_{t-1} + kn_t (x) v_t,
 *   z_t = z_{t-1} + kn_t,  y_t = (q_t @ S_t) / max(q_t . z_t, eps).
 * Replaces the reference's native kernels kernel/attn_cpu.cpp attn_forward
 * (:144-212) and attn_step (:421-492), reached through the backend entries
 * of kernel/compute.py:265-309; results are bit-identical to them (the same
 * per-element operation order, correctly rounded division and square root).
 * Q/K/V/Y fp32 [B,T,H,D] contiguous (K raw: the normalisation is inside);
 * DEN fp32 [B,T,H] or NULL; S_out fp32 [B,H,D,D] and z_out [B,H,D] (the final
 * state, both or neither; zeros when T == 0).  0 < D <= 2048, eps positive
 * and finite.  For D > 128 without S_out the state lives in `workspace`
 * (smaul_attn_workspace_size bytes; 0 otherwise).
 */
int64_t smaul_attn_workspace_size(int64_t B, int64_t H, int64_t D, int need_state);

int smaul_attn_forward(const float* Q, const float* K, const float* V, float* Y, float* DEN, float* S_out,
                       float* z_out, int64_t B, int64_t T, int64_t H, int64_t D, float eps, void* workspace,
                       int64_t workspace_bytes, hipStream_t stream);

/*
 * One decode step from the carried state: S [B,H,D,D] and z [B,H,D] are
 * advanced in place, y [B,H,D] = the step's output (q/k/v [B,H,D]).
 */
int smaul_attn_step(float* S, float* z, const float* q, const float* k, const float* v, float* y, int64_t B,
                    int64_t H, int64_t D, float eps, hipStream_t stream);

/*
 * Backward of the linear-attention recurrence: dQ, dK, dV [B,T,H,D] (K raw,
 * so dK includes the key normalisation's backward) from the upstream
 * gradient dY and the forward's Q, K, V, Y and DEN.  Replaces the reference's
 * native two-pass kernel kernel/attn_cpu.cpp attn_backward (:227-368),
 * reached through the backend entry kernel/compute.py:314-322 from
 * model.py:249,262; results are bit-identical to it.  All fp32 contiguous;
 * 0 < D <= 2048, eps positive and finite (the forward's).  For D > 128 the
 * per-task state lives in `workspace` (smaul_attn_workspace_size(B, H, D, 0)
 * bytes; 0 otherwise).
 */
int smaul_attn_backward(const float* dY, const float* Q, const float* K, const float* V, const float* Y,
                        const float* DEN, float* dQ, float* dK, float* dV, int64_t B, int64_t T, int64_t H, int64_t D,
                        float eps, void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Tiled E4M3 quantizer: per (row, tile) scale = max(max(finite |w|, 1e-12) /
 * 448, 1e-12) and code = order[first i with bounds[i] >= n] for n =
 * clamp(nan_to_num(w / scale), -448, 448), code 0 where n == 0.  Replaces the
 * reference's native quantizer kernel/quant_cpu.cpp:64-137 (the backend entry
 * fp8_quantize_tiles, kernel/compute.py:246-263) with bit-identical codes and
 * scales.  w fp32 [out_f, in_f]; order uint8 [256] / bounds fp32 [255]: the
 * sorted-codebook permutation and its midpoints (torch.argsort's tie order,
 * as the reference passes them); codes uint8 [out_f, ldc], ldc >= nt*tile,
 * the last tile's padding written as 0; scales fp32 [out_f, nt]; *nonfinite
 * (device) = the number of non-finite entries of w.  Any tile > 0.
 */
int smaul_fp8_quantize_tiles(const float* w, int64_t out_f, int64_t in_f, int64_t tile, const uint8_t* order,
                             const float* bounds, uint8_t* codes, int64_t ldc, float* scales,
                             unsigned long long* nonfinite, hipStream_t stream);

/*
 * Input gradient of the tiled-FP8 linear: dx[rows, in_f] = g[rows, out_f] .
 * decode(w, s), fp32.  Replaces the reference's native fp8_backward_input
 * (kernel/fp8_cpu.cpp:167-259; backend entry kernel/compute.py:145-153).
 * g fp32 [rows, out_f] row-major; w uint8 [out_f, in_f]; s fp32
 * [out_f, ceil(in_f/tile)]; any tile > 0; in_f, out_f >= 0 (out_f == 0
 * writes zeros).  The sum runs in another fp32 order than the reference's, so
 * results agree to fp32 rounding, not bitwise.
 */
int smaul_fp8_backward_input(const float* g, const uint8_t* w, const float* s, float* dx, int64_t rows,
                             int64_t in_f, int64_t out_f, int64_t tile, hipStream_t stream);

/*
 * Measured ceilings for the roofline figures (bench.py --peaks); no
 * counterpart in the reference and not on the MoE path.
 * smaul_peak_mfma: `workgroups` x 4 waves, each issuing `iters` rounds of 8
 *   independent v_mfma_f32_32x32x16_bf16 (32768 flop each); out holds one
 *   float per wave.
 * smaul_peak_stream: reads `bytes` (a multiple of 16) from src with 16-byte
 *   loads, grid-stride over `workgroups` x 256 threads; out (one uint32) is
 *   written only in a case that does not occur.
 * smaul_peak_lds_dma: `workgroups` x 4 waves, each copying `iters` rounds of
 *   8 x 1 KB into LDS with global_load_lds_dwordx4 (the prefill GEMM's
 *   staging) from its workgroup's 64 KB of src (bytes >= workgroups * 64 KB);
 *   out holds one uint32 per workgroup.
 */
int smaul_peak_mfma(float* out, int workgroups, int iters, hipStream_t stream);
int smaul_peak_stream(const void* src, int64_t bytes, uint32_t* out, int workgroups, hipStream_t stream);
int smaul_peak_lds_dma(const void* src, int64_t bytes, uint32_t* out, int workgroups, int iters,
                       hipStream_t stream);

/*
 * Host-side self-test of the top-k selection order used by the router (no GPU
 * involved): writes the k indices the router would select for `vals` [n].
 * Exposed only so the CPU test suite can check the order against torch.topk.
 */
int smaul_selftest_topk(const float* vals, int64_t n, int64_t k, int64_t* out_idx);

#ifdef __cplusplus
}
#endif
#endif /* SMAUL_ROCM_H */
