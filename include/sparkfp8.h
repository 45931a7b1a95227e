/*
 * libsparkfp8 -- C ABI of the MI355X (gfx950) SwiGLU MLP kernels.
 *
 * Drop-in boundary for the MLP paths of N8python/spark-gpt: the FP8 MLP
 * sub-block (``_FP8MLPBlock``, train.py:1193-1252), the FP8 MoE experts
 * (``_FP8Experts``, train.py:1255-1606) and the bf16 fused SwiGLU
 * (``_NormSwiGLU`` / ``_FusedSwiGLU``, train.py:1608-2131).  Each entry point
 * replaces one kernel launch (or torch-op sequence) of the reference, cited
 * per function.
 *
 * Conventions
 *  - All pointers are device pointers (hipMalloc / torch CUDA tensors) except
 *    where noted; sizes are elements unless named *_bytes.
 *  - bf16 tensors are passed as `const void*` (uint16 storage), FP8 tensors as
 *    `void*` (one byte per element: OCP e4m3fn or e5m2, as torch.float8_*).
 *  - `scale` points at the 5 delayed per-tensor scales of one block, `amax`
 *    at its 5 amax slots (slot map: 0 = x, 1 = gu, 2 = h (e4m3); 3 = d_gu,
 *    4 = dy (e5m2); train.py:916-919).  Kernels read `scale` on the device and
 *    max-accumulate into `amax`; nothing is read back to the host.
 *  - `wscale` points at the 2 just-in-time weight scales [q_gu, q_d]
 *    (train.py:1213).
 *  - Every scale is a power of two, as fp8_update_scales and the weight
 *    quantizer produce them (train.py:942-943, 951); the kernels rely on it
 *    to fold scales into exact multiplies and into the converters' scale
 *    operand.
 *  - K-slab layout.  Every FP8 GEMM operand, and the bf16 W_down^T, is stored
 *    as a K-slab of a row-major matrix X [R, L] (L = the GEMM's reduction
 *    dimension K, in bytes): [L / 64][rpad][64] bytes, rpad = R rounded up to
 *    a multiple of 256, element (r, l) at (l / 64) * rpad * 64 + r * 64 + l % 64.
 *    One 64-byte K stage of a 256-row GEMM tile is then one contiguous 16 KiB
 *    block (row-major rows K bytes apart put a stage's rows into few memory
 *    channels).  Padding rows r >= R hold zeros; producers write them.
 *    sfp8_slab_bytes(R, L) gives the buffer size.  Token-major activations
 *    (x8, h8, dgu8: R = T) have rpad = ldt = T rounded up to 256.
 *    The weight gradients read these token-major K-slabs (x8, h8, dgu8 and
 *    the dy8 of sfp8_norm_bwd) directly (sfp8_gemm_wgrad_rows).  The
 *    optional token-contiguous copies (x8t, h8t, dgu8t, dy8t: NULL skips
 *    them) are K-slabs of the transposed activation over ldt tokens
 *    (R = features, L = ldt), for sfp8_gemm_wgrad and the grouped MoE
 *    gradient; producers write zeros for tokens T..ldt-1 in every layout.
 *    The standalone quantizer writes a plain row-major x8 and the same K-slab
 *    x8t.
 *  - `stream` is a hipStream_t; every call is asynchronous on it, never
 *    synchronises the device and never allocates device memory.  Callers
 *    provide every output and workspace buffer.
 *  - Return value: 0 on success; a negative SFP8_ERR_* code for invalid
 *    arguments (nothing is launched); a positive hipError_t from the launch.
 *  - Calls are re-entrant: the library has no mutable global state, except
 *    the per-device address of the fixed scratch that sfp8_norm_bwd_noalloc
 *    looks up once per device (under a lock).
 */
#ifndef SPARKFP8_H
#define SPARKFP8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SFP8_OK 0
#define SFP8_ERR_NULL_POINTER (-1)
#define SFP8_ERR_BAD_SHAPE (-2)
#define SFP8_ERR_BAD_ALIGNMENT (-3)
#define SFP8_ERR_WORKSPACE_TOO_SMALL (-4)
#define SFP8_ERR_SCRATCH_LIMIT (-5) /* beyond sfp8_norm_bwd_noalloc's fixed scratch */

/* Pointer arguments are device pointers and must not be NULL, except that
 * buffers sized by the token (or row) count may be NULL when that count is
 * 0: such a call does no work beyond writing the outputs that are not sized
 * by tokens (d_norm_w and the weight gradients come out zero). */

/* ---- quantizers -------------------------------------------------------- */

/* Standalone quantizer: x8 = e4m3(clamp(x * scale[0], +-448)) row-major
 * [rows, cols], x8t = K-slab of x8^T over ldt tokens ([ldt/64][slab_rows(cols)]
 * [64]: the token-contiguous copy the weight gradient reads; tokens
 * rows..ldt-1 and padding rows cols.. are zeros), amax[0] = max(amax[0],
 * max|x|).  The norm-free core of _fp8_norm_quant_kernel (train.py:966-972),
 * whose X8T store (train.py:970) writes the plain [cols, T] transpose.
 * cols % 128 == 0; ldt >= rows, ldt % 64 == 0; x, x8, x8t 16-byte aligned. */
int sfp8_quant_e4m3_rowcol(const void* x, int64_t rows, int64_t cols, const float* scale, float* amax,
                           void* x8, void* x8t, int64_t ldt, void* stream);

/* Norm-fused quantizer, replaces _fp8_norm_quant_kernel (train.py:955-972,
 * launched at train.py:1208-1210).  h [T, D] bf16, norm_w [D] fp32 ->
 * x8 (K-slab of [T, D]: [D/64][ldt][64]) e4m3, x8t (K-slab of [D, ldt];
 * optional) e4m3, rstd [T] fp32; amax[0] max-accumulated.
 * D in {128, 256, 512, 1024, 2048, 4096}, or a multiple of 4096 from 8192
 * on (a two-pass row-chunked form); ldt = T rounded up to 256. */
int sfp8_norm_quant(const void* h, const float* norm_w, int64_t T, int64_t D, float eps,
                    const float* scale, float* amax, void* x8, void* x8t, int64_t ldt, float* rstd,
                    void* stream);

/* Just-in-time weight quantization, replaces _fp8_quantize_weight
 * (train.py:949-952, called at train.py:1211-1212) and the transposed copies
 * the reference saves for backward (w8.t().contiguous(), train.py:1225) plus a
 * transposed bf16 copy of the master (the down-proj dgrad operand; the
 * reference saves w_down.to(bf16), train.py:1224).
 * w [rows, cols] fp32 -> q_out[0] = exp2(floor(log2(448/max(amax,1e-30)))),
 * w8 = K-slab of e4m3(w * q) [rows, cols] (optional), w8t = K-slab of its
 * transpose [cols, rows] (optional), wbf16t = K-slab of bf16(w)^T
 * [cols, rows] bf16 (bytes: [2*rows/64][cols padded][64]) (optional).
 * partials: device workspace of nparts_cap >= 512 floats.  cols % 64 == 0;
 * rows % 64 == 0 with w8t, rows % 32 == 0 with wbf16t. */
int sfp8_weight_quant(const float* w, int64_t rows, int64_t cols, float* partials, int64_t nparts_cap,
                      float* q_out, void* w8, void* w8t, void* wbf16t, void* stream);

/* Delayed-scale roll, replaces fp8_update_scales' tensor ops
 * (train.py:937-946): for each of nsets contiguous 5-slot sets, every slot
 * with amax > 0 gets scale = exp2(floor(log2(fmax/amax)) - 1); amax = 0. */
int sfp8_update_scales(float* scale, float* amax, int64_t nsets, void* stream);

/* The post-step hook of one dense block (fp8_update_scales followed by the
 * two just-in-time weight quantizations, train.py:937-952, 1211-1212) in two
 * launches instead of five: sfp8_update_scales of the block's 5 slots (skipped
 * when scale and amax are both null), then
 *   sfp8_weight_quant(w_gu, gu_rows, gu_cols, .., q_out + 0, w8, w8t, null) and
 *   sfp8_weight_quant(w_down, d_rows, d_cols, .., q_out + 1, wd8, null, wdt),
 * with the same outputs byte for byte.  partials: nparts_cap >= 1024 floats.
 * gu_rows, gu_cols, d_cols % 64 == 0, d_rows % 32 == 0; every output given. */
int sfp8_block_weight_quant(const float* w_gu, int64_t gu_rows, int64_t gu_cols, const float* w_down, int64_t d_rows,
                            int64_t d_cols, float* partials, int64_t nparts_cap, float* q_out, void* w8, void* w8t,
                            void* wd8, void* wdt, float* scale, float* amax, void* stream);

/* ---- GEMMs -------------------------------------------------------------- */

/* gate/up forward + SwiGLU epilogue, replaces _fp8_swiglu_fwd_kernel
 * (train.py:975-1016, launched at train.py:1216-1218).
 * x8 (K-slab of [T, D]) e4m3, w8 (K-slab of [2I, D], gate rows first) e4m3
 * -> gu8 (K-slab of [T, 2I], gate columns first, rpad = ldt) e4m3, h8
 * (K-slab of [T, I]) e4m3, h8t (K-slab of [I, ldt]: optional
 * token-contiguous copy of h8) e4m3; rows T..ldt of gu8 and h8 are zeros;
 * amax[1], amax[2] max-accumulated.  D % 128 == 0, I % 128 == 0, and
 * ldt == T rounded up to 256 (the outputs' padding tokens are written then;
 * any other ldt is SFP8_ERR_BAD_SHAPE). */
int sfp8_gemm_gateup_swiglu_fwd(const void* x8, const void* w8, int64_t T, int64_t D, int64_t I,
                                const float* scale, const float* wscale, float* amax, void* gu8, void* h8,
                                void* h8t, int64_t ldt, void* stream);

/* down forward + residual, replaces _fp8_down_fwd_kernel (train.py:1019-1046,
 * launched at train.py:1220-1222).  h8 (K-slab of [T, I], rpad = ldt) e4m3,
 * wd8 (K-slab of [D, I]) e4m3, res [T, D] bf16 -> y [T, D] bf16.
 * I % 128 == 0, D % 16 == 0. */
int sfp8_gemm_down_fwd(const void* h8, const void* wd8, const void* res, int64_t T, int64_t D, int64_t I,
                       const float* scale, const float* wscale, void* y, int64_t ldt, void* stream);

/* bf16 down dgrad + SwiGLU backward, replaces _fp8_down_dgrad_swiglu_kernel
 * (train.py:1049-1094, launched at train.py:1236-1238).  dy [T, D] bf16
 * row-major, wdt (K-slab of w_down^T [I, D], bf16), gu8 (K-slab of [T, 2I],
 * rpad = ldt, as the forward wrote it) e4m3 -> dgu8 (K-slab of [T, 2I]) e5m2,
 * dgu8t (K-slab of [2I, ldt]; optional) e5m2; amax[3] max-accumulated.  (amax[4] = max|dy| is recorded by
 * sfp8_norm_bwd.)  D % 64 == 0, I % 128 == 0, ldt == T rounded up to 256
 * (as for sfp8_gemm_gateup_swiglu_fwd: every padding token is written). */
int sfp8_gemm_down_dgrad_swiglu(const void* dy, const void* wdt, const void* gu8, int64_t T, int64_t D,
                                int64_t I, const float* scale, float* amax, void* dgu8, void* dgu8t,
                                int64_t ldt, void* stream);

/* gate/up dgrad, replaces torch._scaled_mm (train.py:1239-1241):
 * dxn = bf16((dgu8 @ w8) / (scale[3] * wscale[0])), dgu8 (K-slab of
 * [T, 2I], rpad = ldt) e5m2, w8t (K-slab of W8^T [D, 2I]) e4m3 ->
 * dxn [T, D] bf16.  I % 64 == 0, D % 16 == 0. */
int sfp8_gemm_gateup_dgrad(const void* dgu8, const void* w8t, int64_t T, int64_t D, int64_t I,
                           const float* scale, const float* wscale, void* dxn, int64_t ldt, void* stream);

/* Weight gradient reduced over tokens, replaces _fp8_wgrad / _fp8_wgrad_kernel
 * (train.py:1150-1187, call at train.py:1247) and _fp8_mm_kernel with A read
 * transposed (train.py:1097-1127, call at train.py:1249-1251):
 * out[m, n] = sum_t at[m, t] * bt[n, t] / (sa[0] * sb[0]), fp32 [M, N].
 * at: K-slab copy of M rows over ldt tokens, e5m2 (fmt_a = 1); bt: K-slab
 * copy of N rows, e4m3 (fmt_b = 0).
 * M > 0, N > 0, N % 4 == 0, ldt % 256 == 0.
 * ws: fp32 workspace of sfp8_wgrad_workspace_floats(M, N, ldt) floats (may be
 * NULL when that is 0).  Deterministic: split-K partials are summed in split
 * order by a second kernel on the same stream. */
int sfp8_gemm_wgrad(const void* at, int fmt_a, const void* bt, int fmt_b, int64_t M, int64_t N, int64_t ldt,
                    const float* sa, const float* sb, float* out, float* ws, int64_t ws_floats, void* stream);
/* K splits sfp8_gemm_wgrad / _rows use for (M, N, ldt): the count from 1 to
 * 64 (each split a multiple of 128 tokens and at least 2048, the last one
 * taking the rest) that minimises rounds of work-groups on 256 CUs x the
 * longest split's K stages + the partials' traffic; 5 for both gradients of
 * the T=65536, D=1024, I=3072 block.  A size query: needs no GPU. */
int64_t sfp8_wgrad_splits(int64_t M, int64_t N, int64_t ldt);
/* Bytes of a K-slab of a [rows, k] matrix (k bytes per row; -1 if k is not
 * a multiple of 64). */
int64_t sfp8_slab_bytes(int64_t rows, int64_t k);
int64_t sfp8_wgrad_workspace_floats(int64_t M, int64_t N, int64_t ldt);


/* The same weight gradient (the block's replacement for _fp8_wgrad,
 * train.py:1247, and for _fp8_mm_kernel on d_gu, train.py:1249-1251) with
 * either operand (or both) read from the row K-slab of the token-major
 * activation instead of the token-contiguous copy (a_rows / b_rows != 0:
 * a = [M/64][ldt][64], b = [N/64][ldt][64] bytes: x8, h8, d_gu8 and the
 * dy8 of sfp8_norm_bwd as their producers write them), through transposing
 * LDS reads: bytes equal to sfp8_gemm_wgrad on the copies, which the
 * producers then need not write.  M % 64 == 0 with
 * a_rows, N % 64 == 0 with b_rows, at least one set; ws: fp32 workspace of
 * sfp8_wgrad_rows_workspace_floats(M, N, ldt) floats. */
int64_t sfp8_wgrad_rows_workspace_floats(int64_t M, int64_t N, int64_t ldt);
int sfp8_gemm_wgrad_rows(const void* a, int fmt_a, int a_rows, const void* b, int fmt_b, int b_rows, int64_t M,
                         int64_t N, int64_t ldt, const float* sa, const float* sb, float* out, float* ws,
                         int64_t ws_floats, void* stream);

/* ---- norm backward ------------------------------------------------------ */

/* RMSNorm backward + residual, replaces _fp8_norm_bwd_kernel
 * (train.py:1130-1147, launched at train.py:1243-1246) and the dnw sum
 * (train.py:1252).  h, dxn, dy [T, D] bf16, rstd [T] -> dh [T, D] bf16,
 * dnw [D] fp32; also e5m2(dy * scale[4]) (the down wgrad operand quantized
 * in registers at train.py:1171-1172) as dy8 (K-slab of [T, D]:
 * [D/64][ldt][64]) and/or dy8t (K-slab of [D, ldt]), each optional, and
 * amax[4] = max|dy| (train.py:1074-1081).  partials: fp32 workspace of
 * sfp8_norm_bwd_partials(D, ldt) * D floats. */
int sfp8_norm_bwd(const void* h, const float* rstd, const void* dxn, const void* dy, const float* norm_w,
                  int64_t T, int64_t D, const float* scale, float* amax, void* dh, float* dnw,
                  float* partials, int64_t partials_cap, void* dy8, void* dy8t, int64_t ldt, void* stream);
int64_t sfp8_norm_bwd_partials(int64_t D, int64_t ldt);

/* Allocation-free RMSNorm backward.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as sfp8_norm_bwd without the partials workspace:
 * the dnw partials live in a fixed file-scope device array of
 * SFP8_NOALLOC_SCRATCH_FLOATS floats (32 MiB), one per GPU.  The array is
 * part of the library's code object: every process that loads the library
 * holds 32 MiB of device memory on each GPU it uses, until it exits,
 * whether or not it ever calls this entry point.  Shapes whose
 * sfp8_norm_bwd_partials(D, ldt) * D exceeds it return
 * SFP8_ERR_SCRATCH_LIMIT before anything is launched (ldt up to 522240
 * tokens at D=1024, 130048 at D=2048, 32256 at D=4096).  The call allocates
 * nothing; the first call on a device looks up that device's address of the
 * array (hipGetSymbolAddress), so make that first call outside graph
 * capture; later calls may be captured (they launch kernels only, no
 * memset).  Every call on one GPU shares its array: calls that overlap on
 * one GPU (concurrent streams, threads) race and must be serialised by the
 * caller; nothing in it needs to start at zero. */
#define SFP8_NOALLOC_SCRATCH_FLOATS (8LL << 20)
int sfp8_norm_bwd_noalloc(const void* h, const float* rstd, const void* dxn, const void* dy, const float* norm_w,
                          int64_t T, int64_t D, const float* scale, float* amax, void* dh, float* dnw, void* dy8,
                          void* dy8t, int64_t ldt, void* stream);

/* ---- FP8 MoE experts (grouped) ----------------------------------------- */
/* The grouped twin of the block (_FP8Experts, train.py:1543-1605).  The R
 * expert-order rows (token/expert pairs sorted by expert; expert e owns rows
 * offsets[e-1] .. offsets[e]-1, offsets = inclusive prefix sums of the
 * per-expert counts, int32 [E]) are laid out in "padded expert order":
 * every expert's rows start on a 256-row boundary, so a GEMM tile never
 * straddles two experts, and padding rows are zeros.  ldp =
 * sfp8_moe_padded_rows(R, E) rows hold the worst case.  The plan (int32,
 * sfp8_moe_plan_ints(R, E) entries) maps 256-row tiles to (expert, first
 * expert-order row, valid rows); it is built on the device, so nothing is
 * read back to the host.  Expert weights: E stacked K-slabs (each as the
 * dense entry point's), per-expert scales q[E]. */
int64_t sfp8_moe_plan_ints(int64_t R, int64_t E);
int64_t sfp8_moe_padded_rows(int64_t R, int64_t E);

/* Builds the plan from offsets (replaces _expert_tile's per-program scan,
 * train.py:1266-1297, with one table per layer).  1 <= E <= 1024. */
int sfp8_moe_plan(const int* offsets, int64_t E, int64_t R, int* plan, int64_t plan_ints, void* stream);

/* Gathered rows -> fp8 in padded expert order.  Padded row p of tile t takes
 * source row map[u] (map != NULL: the token index of expert-order row u) or u
 * (map == NULL), u = first row of t + p % 256, while p % 256 < the tile's
 * valid rows; else zeros (and out-of-range indices read as zeros).
 *   fmt = e4m3 (0): replaces _fp8_moe_gather_quant_kernel (train.py:1300-1314):
 *     xs = K-slab of e4m3(clamp(x * scale[sslot])) over [ldp, D] (the gate/up
 *     GEMM's A), xt = its token-contiguous K-slab [D, ldp]; either may be
 *     NULL, not both;
 *   fmt = e5m2 (1), xs = NULL: the e5m2 dout copy the down weight gradient
 *     quantizes in registers (train.py:1525-1526), token-contiguous.
 * amax[aslot] = max |src| over the gathered rows.  D % 128 == 0. */
int sfp8_moe_rows_quant(const void* src, int64_t nsrc, int64_t D, const int64_t* map, int64_t nmap,
                        const int* plan, int64_t ldp, const float* scale, int sslot, float* amax, int aslot,
                        int fmt, void* xs, void* xt, void* stream);

/* Per-expert weight quantization, replaces _fp8_quantize_experts
 * (train.py:1536-1540): E matrices [rows, cols] fp32 -> q_out[e], and
 * optionally per expert w8 / w8t / bf16 W^T K-slabs as sfp8_weight_quant
 * (stacked, one whole K-slab per expert).  partials: 512 * E floats. */
int sfp8_weight_quant_experts(const float* w, int64_t E, int64_t rows, int64_t cols, float* partials,
                              int64_t nparts_cap, float* q_out, void* w8, void* w8t, void* wbf16t, void* stream);

/* Grouped gate/up forward + SwiGLU, replaces _fp8_moe_swiglu_fwd_kernel
 * (train.py:1316-1353): as sfp8_gemm_gateup_swiglu_fwd over padded expert
 * order, expert e's W8 at w8 + e * D * slab_rows(2I) and q_gu[e]; h8t
 * optional. */
int sfp8_moe_gemm_gateup_swiglu_fwd(const void* x8, const void* w8, int64_t E, int64_t D, int64_t I, const int* plan,
                                    int64_t ldp, const float* scale, const float* q_gu, float* amax, void* gu8,
                                    void* h8, void* h8t, void* stream);

/* Grouped down forward, replaces _fp8_moe_down_fwd_kernel
 * (train.py:1356-1378): out [R, D] bf16 expert-order rows (no residual). */
int sfp8_moe_gemm_down_fwd(const void* h8, const void* wd8, int64_t E, int64_t D, int64_t I, const int* plan,
                           int64_t ldp, const float* scale, const float* q_d, void* out, int64_t R, void* stream);

/* Grouped bf16 down dgrad + SwiGLU backward, replaces
 * _fp8_moe_down_dgrad_swiglu_kernel (train.py:1381-1423): dout [R, D] bf16
 * expert-order rows, wdt per expert (bf16 K-slab of W_down[e]^T) ->
 * dgu8 / dgu8t (optional) over padded expert order; amax[3].  (amax[4] = max|dout| is
 * recorded by the e5m2 dout copy, sfp8_moe_rows_quant.) */
int sfp8_moe_gemm_down_dgrad_swiglu(const void* dout, const void* wdt, const void* gu8, int64_t E, int64_t D,
                                    int64_t I, int64_t R, const int* plan, int64_t ldp, const float* scale,
                                    float* amax, void* dgu8, void* dgu8t, void* stream);

/* Grouped gate/up dgrad, replaces _fp8_moe_dgrad_kernel (train.py:1425-1448):
 * dx [R, D] bf16 expert-order rows. */
int sfp8_moe_gemm_gateup_dgrad(const void* dgu8, const void* w8t, int64_t E, int64_t D, int64_t I, const int* plan,
                               int64_t ldp, const float* scale, const float* q_gu, void* dx, int64_t R, void* stream);

/* Grouped weight gradient, replaces _fp8_moe_wgrad_kernel (train.py:1450-1478)
 * and _fp8_moe_wgrad_rows_kernel (train.py:1503-1533, whose fp32 atomics are
 * replaced by split partials summed in order: deterministic):
 * out[e] = sum over expert e's rows of at[:, t] bt[:, t]^T / (sa * sb),
 * fp32 [E, M, N]; experts without rows get zeros.  ws: fp32 workspace of
 * sfp8_moe_wgrad_workspace_floats(M, N, E) floats (may be NULL when 0). */
int64_t sfp8_moe_wgrad_splits(int64_t M, int64_t N, int64_t E);
int64_t sfp8_moe_wgrad_workspace_floats(int64_t M, int64_t N, int64_t E);
int sfp8_moe_gemm_wgrad(const void* at, int fmt_a, const void* bt, int fmt_b, int64_t M, int64_t N, int64_t E,
                        const int* plan, int64_t ldp, const float* sa, const float* sb, float* out, float* ws,
                        int64_t ws_floats, void* stream);

/* The grouped weight gradient with either operand (or both) read from the
 * row K-slab of the expert-order activation over padded rows (a_rows /
 * b_rows != 0: a = [M/64][ldp][64], b = [N/64][ldp][64] bytes: xs, h8 and
 * dgu8 as their producers write them) through transposing LDS reads, as
 * sfp8_gemm_wgrad_rows is to sfp8_gemm_wgrad: bytes equal to
 * sfp8_moe_gemm_wgrad on the token-contiguous copies.  M % 64 == 0 with
 * a_rows, N % 64 == 0 with b_rows, at least one set; ws: fp32 workspace of
 * sfp8_moe_wgrad_rows_workspace_floats(M, N, E) floats. */
int64_t sfp8_moe_wgrad_rows_workspace_floats(int64_t M, int64_t N, int64_t E);
int sfp8_moe_gemm_wgrad_rows(const void* a, int fmt_a, int a_rows, const void* b, int fmt_b, int b_rows, int64_t M,
                             int64_t N, int64_t E, const int* plan, int64_t ldp, const float* sa, const float* sb,
                             float* out, float* ws, int64_t ws_floats, void* stream);

/* out[t] = bf16(sum over slots j < k of dx[inv[t*k + j]]), fp32 sum in slot
 * order: replaces _sum_topk_rows (train.py:2213-2217) in the experts'
 * backward (train.py:1604).  inv int64 [T*k]; out-of-range entries add 0. */
int sfp8_moe_topk_sum(const void* dx, int64_t R, int64_t D, const int64_t* inv, int64_t T, int64_t k, void* out,
                      void* stream);

/* ---------------------------------------------------------------------------
 * bf16 SwiGLU path (spark-gpt's default, non-FP8 MLP path): _NormSwiGLU
 * (train.py:2101-2131) and _FusedSwiGLU (train.py:2067-2090), dense or
 * grouped over MoE experts (rows in padded expert order, a plan from
 * sfp8_moe_plan).  bf16 K-slab of a row-major X [R, C]: element (r, c) at
 * byte ((c / 32) * roundup(R, 256) + r) * 64 + (c % 32) * 2.  D % 64 == 0,
 * I % 64 == 0.
 * ------------------------------------------------------------------------- */

/* Bytes of the bf16 K-slab of [rows, cols] (cols % 32 == 0), else -1. */
int64_t sfp8_bf16_slab_bytes(int64_t rows, int64_t cols);

/* W [E][R][C] (fp32, times nw[c] when nw != NULL; or bf16 when src_bf16)
 * -> ws = bf16 K-slabs of W[e] (when ws != NULL) and wt = of W[e]^T (when
 * wt != NULL), stacked per expert; padding rows zero.  Replaces the weight
 * casts of train.py:2112 (W' = bf16(w_gu * norm_w)), 259 and 2306, whose
 * results the reference's kernels read through strides.  R % 64 == 0,
 * C % 64 == 0. */
int sfp8_bf16_weight_slabs(const void* w, int src_bf16, const float* nw, int64_t E, int64_t R, int64_t C, void* ws,
                           void* wt, void* stream);

/* x [nsrc, D] bf16 rows in padded order (plan, or rows 0..nsrc-1 when plan
 * is NULL) -> xt (optional), the token-contiguous bf16 K-slab of x^T over ldp
 * rows (a weight gradient's plain operand; zeros past the rows); xs
 * (optional), the row K-slab of x over ldp rows ([2D/64][ldp][64] bytes,
 * zeros past the rows: the gate/up forward's A operand with x_slab); and
 * with rstd (plan NULL only) rstd[t] = 1 / sqrt(sum x^2 / D + eps): the row
 * statistic _swiglu_gemm_kernel accumulates in its NORM mode
 * (train.py:1689-1700).  At least one of xt, xs, rstd. */
int sfp8_bf16_rows_prep(const void* x, int64_t nsrc, int64_t D, const int* plan, int64_t ldp, float eps, float* rstd,
                        void* xt, void* xs, void* stream);

/* Gate/up GEMM with the SwiGLU epilogue, replaces _swiglu_gemm_kernel
 * (train.py:1625-1716, launch 1719-1743): x [T, D] bf16 (x_slab 0), or its
 * row K-slab over T rounded up to 256 rows (x_slab 1: the xs of
 * sfp8_bf16_rows_prep, the faster read), w = bf16 K-slab of W [2I, D] (gate
 * rows first), rstd [T] or NULL (the folded-norm row scale):
 * gu = [bf16(acc_g * rs) | bf16(acc_u * rs)] [T, 2I], h = bf16(g sigmoid(g) u)
 * [T, I].  Both layouts give the same bytes. */
int sfp8_bf16_gemm_swiglu_fwd(const void* x, int x_slab, const void* w, int64_t T, int64_t D, int64_t I,
                              const float* rstd, void* gu, void* h, void* stream);

/* The same grouped (E experts, _FusedSwiGLU with several groups): x, gu, h
 * in expert order, w the stacked per-expert K-slabs. */
int sfp8_bf16_moe_gemm_swiglu_fwd(const void* x, const void* w, int64_t E, int64_t D, int64_t I, const int* plan,
                                  int64_t ldp, void* gu, void* h, void* stream);

/* The SwiGLU gradient of the rows, replaces _swiglu_tiles in the prologues of
 * _swiglu_dgrad_kernel and _swiglu_wgrad_kernel (train.py:1899-2026), once
 * for both: G' = [bf16(dh u sig (1 + g (1 - sig))) | bf16(dh g sig)] with
 * dh = dout * rstd (rstd NULL: 1), written as gs = its bf16 K-slab over ldp
 * padded rows and (optionally) gt = the token-contiguous K-slab of G'^T;
 * padding zero. */
int sfp8_bf16_swiglu_bwd(const void* gu, const void* dout, int64_t nsrc, int64_t I, const float* rstd,
                         const int* plan, int64_t ldp, void* gs, void* gt, void* stream);

/* out [T, N] = bf16(A B^T): A the bf16 K-slab of [lda rows, K], B of [N, K];
 * the dgrad of _swiglu_dgrad_kernel (train.py:1907-1980, its d_gu operand
 * precomputed by sfp8_bf16_swiglu_bwd).  N % 8 == 0, K % 32 == 0. */
int sfp8_bf16_gemm(const void* a, const void* b, int64_t T, int64_t N, int64_t K, int64_t lda, void* out,
                   void* stream);

/* The same grouped: A over ldp padded rows, out in expert order. */
int sfp8_bf16_moe_gemm(const void* a, const void* b, int64_t E, int64_t N, int64_t K, const int* plan, int64_t ldp,
                       void* out, void* stream);

/* _NormSwiGLU's RMSNorm backward (train.py:2125-2128): dh = bf16(p - rstd^2
 * sum(h p) / D h) per row, p [T, D] bf16 the dgrad output. */
int sfp8_bf16_norm_dh(const void* p, const void* h, const float* rstd, int64_t T, int64_t D, void* dh, void* stream);

/* Weight gradient, replaces _swiglu_wgrad_kernel (train.py:1983-2026):
 * out [M, N] = bf16(sum over ldt tokens of at[:, t] bt[:, t]^T), at / bt the
 * token-contiguous bf16 K-slabs of [M, ldt] / [N, ldt]; split partials summed
 * in order (deterministic).  ws: fp32 workspace of
 * sfp8_bf16_wgrad_workspace_floats(M, N, ldt) floats.  M N % 8 == 0. */
int64_t sfp8_bf16_wgrad_splits(int64_t M, int64_t N, int64_t ldt);
int64_t sfp8_bf16_wgrad_workspace_floats(int64_t M, int64_t N, int64_t ldt);
int sfp8_bf16_gemm_wgrad(const void* at, const void* bt, int64_t M, int64_t N, int64_t ldt, void* out, float* ws,
                         int64_t ws_floats, void* stream);

/* The same per expert over its padded rows: out [E, M, N] bf16, zeros for
 * experts without rows (train.py:2047-2063 with several groups). */
int64_t sfp8_bf16_moe_wgrad_workspace_floats(int64_t M, int64_t N, int64_t E);
int sfp8_bf16_moe_gemm_wgrad(const void* at, const void* bt, int64_t M, int64_t N, int64_t E, const int* plan,
                             int64_t ldp, void* out, float* ws, int64_t ws_floats, void* stream);

/* The bf16 weight gradients with A read from gs, the bf16 K-slab of G'
 * over the padded rows (the dgrad's A operand, [M/32][ldt][64] bytes),
 * through transposing LDS reads (ds_read_b64_tr_b16), so that no
 * token-contiguous copy of G' is written; bytes equal to
 * sfp8_bf16_gemm_wgrad / sfp8_bf16_moe_gemm_wgrad on the copies.
 * Dense: B is x itself with x_rows != 0, row-major [T, N] bf16 (rows
 * T..ldt-1 read as zero), also transposed on read (N % 32 == 0), or with
 * x_rows == 0 the token-contiguous K-slab of x^T over ldt tokens
 * (sfp8_bf16_rows_prep); M % 32 == 0, T * N * 2 < 2^31; ws as for
 * sfp8_bf16_gemm_wgrad.  Grouped: B is the token-contiguous K-slab of x^T
 * over the padded rows; ws as for sfp8_bf16_moe_gemm_wgrad. */
int sfp8_bf16_gemm_wgrad_rows(const void* gs, const void* x, int x_rows, int64_t M, int64_t N, int64_t T, int64_t ldt,
                              void* out, float* ws, int64_t ws_floats, void* stream);
int sfp8_bf16_moe_gemm_wgrad_rows(const void* gs, const void* bt, int64_t M, int64_t N, int64_t E, const int* plan,
                                  int64_t ldp, void* out, float* ws, int64_t ws_floats, void* stream);

/* _NormSwiGLU's fold of the weight gradient (train.py:2129-2131): dw =
 * f32(dwp) * nw (fp32 [M, N]) and dnw[n] = sum over m of f32(dwp[m, n]) *
 * w[m, n] (fp32: 16-row blocks in order, groups of 16 block sums in order,
 * then the groups in order); part:
 * sfp8_bf16_fold_partials(M, N) floats.  N % 4 == 0. */
int64_t sfp8_bf16_fold_partials(int64_t M, int64_t N);
int sfp8_bf16_fold_grads(const void* dwp, const float* w, const float* nw, int64_t M, int64_t N, float* dw,
                         float* dnw, float* part, int64_t part_floats, void* stream);

/* ---------------------------------------------------------------------------
 * The consumer of the fp32 weight gradients: the Muon optimizer's momentum
 * stage (train.py:2805-2839), alone and fused into the weight gradient.
 * ------------------------------------------------------------------------- */

/* Replaces _momentum_stage_kernel (train.py:2805-2820, launched by
 * _momentum_stage 2829-2839): v <- lerp(v, g, w_v) in place (fp32), u =
 * bf16(lerp(g, v_new, w_u)) (the Newton-Schulz staging matrix), each lerp in
 * torch.lerp's form for its weight (w_v < 0.5 <= w_u): the reference's
 * two-pass torch update bit for bit.  w_v = 1 - momentum, w_u = momentum,
 * each rounded to fp32 from the caller's double.  n % 4 == 0; g, v 16-byte
 * and u 8-byte aligned. */
int sfp8_momentum_stage(const float* g, float* v, void* u, int64_t n, float w_v, float w_u, void* stream);

/* sfp8_gemm_wgrad_rows (e5m2 a, e4m3 b; a_rows = b_rows = 0: the
 * token-contiguous copies of sfp8_gemm_wgrad) with the momentum stage
 * applied as the split sum leaves the registers: d = dW, then v <- lerp(v, d, w_v), u =
 * bf16(lerp(d, v_new, w_u)) ([M, N] bf16: the parameter's layout in the
 * Newton-Schulz staging stack, train.py:2982-2999), grad = d when grad !=
 * NULL.  No counterpart in the reference (its backward writes dW and the
 * optimizer reads it back); valid when nothing reduces or accumulates the
 * gradient between the backward and the optimizer step (one process, no
 * gradient accumulation).  ws: fp32 workspace of
 * sfp8_wgrad_momentum_workspace_floats(M, N, ldt) floats (NULL when ldt = 0:
 * then d = 0). */
int64_t sfp8_wgrad_momentum_workspace_floats(int64_t M, int64_t N, int64_t ldt);
int sfp8_gemm_wgrad_momentum(const void* a, int fmt_a, int a_rows, const void* b, int fmt_b, int b_rows, int64_t M,
                             int64_t N, int64_t ldt, const float* sa, const float* sb, float* grad, float* v, void* u,
                             float w_v, float w_u, float* ws, int64_t ws_floats, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPARKFP8_H */
