/*
 * intcrush.h - C ABI of libintcrush_gfx950.so, the MI355X (gfx950) kernels of
 * the INT-Crush quantized-linear forward.
 *
 * Conventions
 *   - Every pointer argument is a device pointer owned by the caller (the host
 *     side allocates every output; no entry point allocates device memory).
 *   - Matrices are row-major; ld* arguments are row strides in elements
 *     (in bytes for packed INT4 weights).
 *   - Work is enqueued on `stream` (a hipStream_t, NULL = the legacy default
 *     stream) with no host synchronisation, so every entry point may be
 *     recorded into a hipGraph.
 *   - Return value: IC_OK (0) or an IC_ERR_* code; ic_last_error() returns a
 *     thread-local message describing the last failure.
 *   - dtype codes: IC_DTYPE_F16, IC_DTYPE_BF16, IC_DTYPE_F32.
 *
 * Reference citations are file:line in ThunderFun/ComfyUI-INT-Crush.
 */
#ifndef INTCRUSH_H
#define INTCRUSH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { IC_DTYPE_F16 = 0, IC_DTYPE_BF16 = 1, IC_DTYPE_F32 = 2 };
enum { IC_OK = 0, IC_ERR_INVALID_ARG = 1, IC_ERR_UNSUPPORTED = 2, IC_ERR_LAUNCH = 3 };

/* Library identification and diagnostics. */
const char* ic_version(void);
const char* ic_last_error(void);
/* Largest K_w the single-pass ic_rotate_quantize / ic_prepare_activation handle
 * for 16-bit activations (f32 rows are limited to half of it). */
int64_t ic_max_fused_row(void);

/*
 * SmoothRot / SmoothQuant factor preparation (once per layer and activation
 * dtype): fdt[k] = RN_dtype(factors[k]) held as f32, rcp[k] = RN32(1/fdt[k]).
 * Replaces the per-call `factors.to(x.dtype)` of _ops.py:350 and :533.
 */
int ic_smoothrot_prepare(const float* factors, int64_t K, int dtype, float* fdt_out,
                         float* rcp_out, void* stream);

/*
 * Fused activation prep + per-token dynamic INT8 quantization, one HBM pass.
 * Replaces _ops.py:337-365 (_prep_activation: SmoothRot divide, rotate_activations
 * of _quant_utils.py:117-147, pad to w_in, PermuQuant gather), the old
 * SmoothQuant divide of _ops.py:529-533, and dynamic_quantize_activation of
 * kernels/triton_quantize.py:151-198.
 *   x        [M, K_in] activations (dtype), row stride ldx
 *   sr_rcp/sr_f  SmoothRot factors prepared by ic_smoothrot_prepare, or both NULL
 *   rot_size 0 (no rotation) or 16, 64, 256, 1024, 4096
 *   K_w      prepared width (weight K); >= K_in rounded up to rot_size
 *   perm     [K_w] int32 gather indices, or NULL
 *   sm_rcp/sm_f  old-SmoothQuant factors applied after the gather, or both NULL
 *   q_out    [M, K_w] int8 codes, row stride ldq; s_out [M] f32 scales
 */
int ic_rotate_quantize(const void* x, int dtype, int64_t M, int64_t K_in, int64_t ldx,
                       const float* sr_rcp, const float* sr_f, int rot_size, int64_t K_w,
                       const int32_t* perm, const float* sm_rcp, const float* sm_f, int8_t* q_out,
                       int64_t ldq, float* s_out, void* stream);

/* Same preparation without quantization: y_out [M, K_w] in dtype.  Replaces
 * _prep_activation (_ops.py:337-365) for the W4A16 path. */
int ic_prepare_activation(const void* x, int dtype, int64_t M, int64_t K_in, int64_t ldx,
                          const float* sr_rcp, const float* sr_f, int rot_size, int64_t K_w,
                          const int32_t* perm, const float* sm_rcp, const float* sm_f,
                          void* y_out, int64_t ldy, void* stream);

/*
 * Second pass of the preparation for rows wider than ic_max_fused_row() (or
 * half of it for f32): the caller first runs ic_prepare_activation without
 * perm / old-SmoothQuant factors over column chunks of the row that are whole
 * Hadamard blocks (the rotation is block-diagonal), into y [M, K_y] (K_y the
 * rotated width); this pass pads with zeros to K_w, gathers by perm, divides
 * by the old-SmoothQuant factors, and either quantizes per token (q_out
 * [M, K_w] int8, s_out [M] f32) or writes out [M, K_w] in dtype (pass q_out =
 * s_out = NULL).  Together they replace _prep_activation (_ops.py:337-365),
 * the old SmoothQuant divide (_ops.py:529-533) and dynamic_quantize_activation
 * (kernels/triton_quantize.py:151-198) for any row width.
 */
int ic_permute_quantize(const void* y, int dtype, int64_t M, int64_t K_y, int64_t ldy, int64_t K_w,
                        const int32_t* perm, const float* sm_rcp, const float* sm_f, int8_t* q_out, int64_t ldq,
                        float* s_out, void* out, int64_t ldo, void* stream);

/* Per-token dynamic INT8 quantization of any width.
 * Replaces dynamic_quantize_activation, kernels/triton_quantize.py:151-198. */
int ic_dynamic_quantize(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, int8_t* q_out,
                        int64_t ldq, float* s_out, void* stream);

/*
 * Row normalisation + per-token dynamic INT8 quantization, one kernel:
 *   kind IC_NORM_LAYER  y = LayerNorm(x) * gamma (+ beta)   replaces fused_layernorm_quantize,
 *                       kernels/triton_quantize.py:277-345 (kernel :209-274)
 *   kind IC_NORM_RMS    y = x / sqrt(mean(x^2) + eps) * gamma   replaces fused_rmsnorm_quantize,
 *                       kernels/triton_quantize.py:397-459 (kernel :348-394)
 *   kind IC_SOFTMAX     y = softmax(x)   replaces fused_softmax_quantize,
 *                       kernels/triton_quantize.py:518-567 (kernel :462-515)
 * then s_out[m] = max(max|y|, 1e-8) / 127 and q_out = trunc(y / s +- 0.5) clamped
 * to [-128, 127] (the reference GPU rule).  Row statistics are summed in fp64 and
 * y is formed in f32; gamma / beta are f32 [K] (gamma required for LayerNorm and
 * RMSNorm, beta only for LayerNorm and optional, both NULL for softmax).
 *   x [M, K] (dtype), row stride ldx; q_out [M, K] int8, row stride ldq; s_out [M] f32
 */
enum { IC_NORM_LAYER = 1, IC_NORM_RMS = 2, IC_SOFTMAX = 3 };
int ic_norm_quantize(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, int kind,
                     const float* gamma, const float* beta, float eps, int8_t* q_out, int64_t ldq,
                     float* s_out, void* stream);

/*
 * LayerNorm / RMSNorm of each row fused in front of ic_rotate_quantize, for the
 * pre-projection activations of a transformer block (the block-input fusion the
 * reference's fused norm quantizers, kernels/triton_quantize.py:201-459, stop
 * short of: they quantize without the SmoothRot / Hadamard / PermuQuant prep,
 * so a rotated INT4 layer cannot use them).  No reference entry point fuses the
 * two; callers that build y = norm(x) * (1 + scale) + shift and then call
 * rotate_quantize (_ops.py:337-365 on y) use this instead:
 *   y = RN_dtype(norm(x) * weight + bias)   weight / bias optional f32 [K_in]
 *       (adaptive LayerNorm: weight = 1 + scale, bias = shift); statistics over
 *       the K_in values in fp64, y formed in f32 and rounded once;
 *   then exactly ic_rotate_quantize on y (SmoothRot divide, Hadamard, pad, perm,
 *   per-token INT8).
 * f16/bf16 rows only, with K_in and K_w multiples of 16, K_w <= ic_max_fused_row(),
 * 16-byte aligned rows, factors, perm, weight and bias; other shapes return
 * IC_ERR_UNSUPPORTED.
 */
int ic_norm_rotate_quantize(const void* x, int dtype, int64_t M, int64_t K_in, int64_t ldx, int norm_kind,
                            const float* weight, const float* bias, float eps, const float* sr_rcp,
                            const float* sr_f, int rot_size, int64_t K_w, const int32_t* perm, int8_t* q_out,
                            int64_t ldq, float* s_out, void* stream);

/*
 * W8A8: out[M,N] = f32(xq . w^T) * (s_a[m] * s_w[n]) + bias[n].
 * Replaces fused_int8_gemm_dequant, kernels/triton_int8_gemm.py:135-205.
 *   xq [M,K] int8, w [N,K] int8, s_a [M] f32, s_w [N] f32, bias [N] (bias_dtype) or NULL.
 */
int ic_gemm_w8a8(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N,
                 int64_t ldw, const float* s_a, const float* s_w, const void* bias, int bias_dtype,
                 void* out, int out_dtype, int64_t ldo, void* stream);

/*
 * W4A8 with packed INT4 weights (two's complement nibbles, low nibble = even k)
 * unpacked inside the GEMM.  Replaces unpack_int4_to_int8
 * (kernels/triton_int4_to_int8_unpack.py:55-81) + fused_w4a8_gemm_dequant
 * (kernels/triton_w4a8_gemm.py:111-169) as called by _ops.py:443-464.
 *   w_packed [N, K/2] uint8 (row stride ldw bytes); s_w [N, num_groups] f32.
 *   num_groups == 1: out = f32(acc) * (s_a[m] * s_w[n]) + bias[n]
 *   num_groups  > 1: out = (sum_g f32(acc_g) * s_w[n,g]) * s_a[m] + bias[n],
 *                    the sum an fma chain in g order, groups of K/num_groups.
 *                    Every kernel folds once per block of gcd(group, 128)
 *                    columns in K order (acc_g of each block with its group's
 *                    scale), so the result does not depend on the kernel:
 *                    - multiples of 128: MFMA kernels, per 128 columns;
 *                    - odd multiples of 64 or of 32 with a 16-bit output
 *                      whose rows are 16-byte aligned: the 288 x 192 MFMA
 *                      kernel, per 64 or per 32;
 *                    - anything else (other group sizes, K not a multiple of
 *                      128, f32 or unaligned outputs with such groups,
 *                      unaligned operands): a scalar kernel, one thread per
 *                      output, about 100x slower.
 */
int ic_gemm_w4a8(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                 int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a,
                 const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo,
                 void* stream);

/*
 * Split-K forms of ic_gemm_w8a8 / ic_gemm_w4a8 (same kernels as the two entry
 * points above, which the reference functions named there map to).  When the
 * output has too few tiles to occupy the GPU (small M), K is cut into S slices
 * computed in parallel; each slice writes 4-byte partials (exact int32 sums,
 * or the fp32 group fold when num_groups > 1) to the caller's workspace and a
 * second kernel adds them in slice order and applies the epilogue.  Per-row
 * scale outputs are bit-identical to the unsplit GEMM; grouped outputs differ
 * only in the order of the fp32 additions.  ic_gemm_splitk_bytes returns the
 * workspace the launch will use (0: no split; then workspace may be null);
 * a smaller workspace than that runs the unsplit GEMM.  The library itself
 * never allocates.
 */
int64_t ic_gemm_splitk_bytes(int64_t M, int64_t N, int64_t K, int64_t num_groups, int int4);
int ic_gemm_w8a8_ws(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N,
                    int64_t ldw, const float* s_a, const float* s_w, const void* bias, int bias_dtype,
                    void* out, int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes,
                    void* stream);
int ic_gemm_w4a8_ws(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                    int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a,
                    const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo,
                    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * ic_gemm_w4a8_ws without the workspace argument: the split-K partials go to a
 * static scratch array of IC_NOALLOC_SCRATCH_BYTES per device, inside the
 * library's code object, so the call allocates nothing (no hipMalloc, no
 * workspace from the caller).  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under hipGraph capture,
 * tight serving loops, harnesses that forbid allocation).  Shapes whose
 * split-K plan needs more partials than the scratch holds return
 * IC_ERR_UNSUPPORTED (ic_gemm_splitk_bytes tells in advance).  The scratch is
 * shared by every call on a device: calls that overlap in time on one device
 * (different streams, different threads) race; calls on one stream do not.
 * Nothing in it needs clearing: every partial is written before it is read.
 */
#define IC_NOALLOC_SCRATCH_BYTES (32LL << 20)
/* Per-device set-up for the current device: looks up the device address of
 * the no-alloc scratch (a code-object symbol, which the lookup may load).
 * Call it once per device before capturing ic_gemm_w4a8_noalloc into a
 * hipGraph; otherwise the entry point does it on its first call on a device.
 * No reference counterpart. */
int ic_init_device(void);
int ic_gemm_w4a8_noalloc(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                         int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a,
                         const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo,
                         void* stream);

/*
 * The same GEMMs with the epilogue options of fused_int8_gemm_dequant
 * (kernels/triton_int8_gemm.py:119-130, arguments :142-143): after dequant and
 * bias, in f32,
 *   activation 0: none; IC_ACT_SILU: v * sigmoid(v); IC_ACT_GELU:
 *   0.5 v (1 + erf(v / sqrt 2)); IC_ACT_GELU_TANH: 0.5 v (1 + tanh(sqrt(2/pi)
 *   (v + 0.044715 v^3))) (no counterpart in the reference; the MLPs of DiT
 *   models such as Flux use it),
 * then + residual[m, n] (f16/bf16/f32, row stride ldr; NULL for none), then
 * the rounding to out_dtype.  Every M routes as ic_gemm_*_ws does (GEMV for
 * M <= IC_GEMV_MAX_M, split-K with a workspace).  With activation 0 and no
 * residual these are ic_gemm_w8a8_ws / ic_gemm_w4a8_ws.
 */
enum { IC_ACT_NONE = 0, IC_ACT_SILU = 1, IC_ACT_GELU = 2, IC_ACT_GELU_TANH = 3 };
int ic_gemm_w8a8_ex(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N,
                    int64_t ldw, const float* s_a, const float* s_w, const void* bias, int bias_dtype,
                    int activation, const void* residual, int residual_dtype, int64_t ldr, void* out,
                    int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes, void* stream);
int ic_gemm_w4a8_ex(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                    int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a,
                    const void* bias, int bias_dtype, int activation, const void* residual,
                    int residual_dtype, int64_t ldr, void* out, int out_dtype, int64_t ldo, void* workspace,
                    int64_t workspace_bytes, void* stream);

/*
 * K-interleaved INT4 weights.  No reference counterpart: the reference
 * unpacks the checkpoint's nibble order (byte b holds k = 2b low, 2b + 1 high;
 * _quant_utils.py:67-80) inside every GEMM call.  ic_int4_interleave_k
 * rewrites packed rows once, on the device, so that byte 4d + j holds
 * k = 8d + j in its low nibble and k = 8d + 4 + j in its high nibble (a
 * permutation inside each 4-byte word; K a multiple of 8; w_kil may be
 * w_packed itself with ldo == ldw, else the two must not overlap).  The
 * W4A8 kernels then expand 8 weights with 3 instructions instead of 5.
 * ic_gemm_w4a8_kil_ex is ic_gemm_w4a8_ex on such weights: same arguments,
 * routes and results, bit for bit.
 */
int ic_int4_interleave_k(const uint8_t* w_packed, int64_t N, int64_t K, int64_t ldw, uint8_t* w_kil, int64_t ldo,
                         void* stream);
int ic_gemm_w4a8_kil_ex(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_kil, int64_t N,
                        int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a, const void* bias,
                        int bias_dtype, int activation, const void* residual, int residual_dtype, int64_t ldr,
                        void* out, int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes,
                        void* stream);

/*
 * W4A8 on INT4 weights unpacked to one int8 byte each (w [N, K], row stride
 * ldw >= K, as ic_unpack_int4_to_int8 writes them), with the group scales
 * s_w [N, num_groups] of ic_gemm_w4a8_ex: the same arithmetic and results
 * (per 128-column block an exact int32 sum, folded facc = fma(f32(sum), s_w,
 * facc) in K order), without the in-loop INT4 expansion, at twice the weight
 * bytes.  Any int8 weights are accepted.  No reference counterpart: a
 * derived copy of the checkpoint's packed weights (as the K-interleaved one),
 * for the large-M W4A8 launches of callers that can hold N * K bytes more per
 * layer.  M <= 16 runs the tile kernels, not the GEMV.
 */
int ic_gemm_w4a8_unpacked_ex(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N,
                             int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a, const void* bias,
                             int bias_dtype, int activation, const void* residual, int residual_dtype, int64_t ldr,
                             void* out, int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes,
                             void* stream);

/*
 * Chained MLP epilogue: the up-projection GEMM of an MLP, finished as the
 * next linear's prepared activation.  Each output is first what
 * ic_gemm_*_ex computes with this activation and no residual,
 *   h = RN_dt(act(dequant + bias)),
 * and then, per row, the first half of the down-projection's
 * _prep_activation (_ops.py:337-365):
 *   x = RN_dt(h / RN_dt(f[n]))            (SmoothRot divide; sr_rcp = RN32(1/f),
 *                                          sr_f = RN_dt(f) as ic_smoothrot_prepare
 *                                          makes them; both NULL: no divide)
 *   y = RN_dt(H_R x) per block of rot_size columns   (_quant_utils.py:117-147)
 * written to out [M, N] in out_dtype (f16/bf16), bit-identical to
 * ic_gemm_*_ex followed by ic_prepare_activation with the same factors and
 * rot_size and no pad or perm.  The rest of the down-projection's prep -- pad
 * to K_w, PermuQuant gather and the per-row INT8 scale over the whole row --
 * needs every column of a row, so it follows as ic_rotate_quantize(y,
 * rot_size 0, no factors, perm) (the reference's chained-GEMM kernel,
 * int8_gemm_int8out, kernels/triton_int8_gemm.py:392-536, quantizes inside
 * each N-tile with that tile's own abs-max instead).  rot_size is 16, 64 or
 * 256 and divides N; K is a multiple of 128; num_groups is 1 or gives a
 * group size that is a multiple of 128; operands, row strides and out are
 * 16-byte aligned and ldo is a multiple of 8.
 */
int ic_gemm_w8a8_chain(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N,
                       int64_t ldw, const float* s_a, const float* s_w, const void* bias, int bias_dtype,
                       int activation, const float* sr_rcp, const float* sr_f, int rot_size, void* out,
                       int out_dtype, int64_t ldo, void* stream);
int ic_gemm_w4a8_chain(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                       int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a,
                       const void* bias, int bias_dtype, int activation, const float* sr_rcp,
                       const float* sr_f, int rot_size, void* out, int out_dtype, int64_t ldo, void* stream);

/*
 * W4A16: out = x . RN_dt(q * RN_dt(s))^T (+ bias), fp32 accumulation, dtype f16/bf16.
 * Replaces unpack_int4_to_float16 (kernels/triton_int4_unpack.py:62-88) + F.linear
 * of _ops.py:466-481.
 */
int ic_gemm_w4a16(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                  int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const void* bias,
                  int bias_dtype, void* out, int64_t ldo, void* stream);

/*
 * Staged operand layout of the W4A16 big-tile kernel.  ic_w4a16_stage_layout
 * copies packed INT4 weights w_packed [N, K/2] (row stride ldw, 16-byte
 * aligned rows) and scales s_w [N, num_groups] to w_staged [K/64][N][32]
 * (the 32 packed bytes of row n and 64-K stage s at (s * N + n) * 32) and
 * s_staged [num_groups][N] (K a multiple of 64).  ic_gemm_w4a16_staged is
 * ic_gemm_w4a16 on that layout: same arithmetic, results bit for bit, in
 * fewer DMA cache-line requests per stage.  It serves the big-tile shapes
 * only (M > 128, K and the group size multiples of 64, N and ldo multiples
 * of 8, 16-byte aligned x, w_staged and out) and rejects the others, which
 * take ic_gemm_w4a16.  No reference counterpart: a derived copy of the
 * checkpoint's weights (as the K-interleaved W4A8 one), N * K/2 + 4 * N *
 * num_groups bytes per layer, for callers that keep it beside the weights.
 */
int ic_w4a16_stage_layout(const uint8_t* w_packed, int64_t N, int64_t K, int64_t ldw, const float* s_w,
                          int64_t num_groups, uint8_t* w_staged, float* s_staged, void* stream);
int ic_gemm_w4a16_staged(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_staged,
                         int64_t N, const float* s_staged, int64_t num_groups, const void* bias, int bias_dtype,
                         void* out, int64_t ldo, void* stream);

/*
 * Small-batch GEMV forms (1 <= M <= IC_GEMV_MAX_M tokens, K a multiple of 128
 * and <= IC_GEMV_MAX_K, 16-byte aligned operands): same arguments, same
 * arithmetic and same results as ic_gemm_w8a8 / ic_gemm_w4a8 (bit-identical)
 * and ic_gemm_w4a16 (fp32 accumulation, tolerance-equal), reading each packed
 * weight byte once.  The GEMM entry points route such calls here themselves.
 * ic_gemv_w4a8 takes num_groups 1 or groups of a multiple of 32 columns, folded
 * per gcd(group, 128) columns as the GEMM does, while those fold sums of the
 * M rows fit 128 KB (K / gcd * M * 64 bytes); the GEMM entry point runs the
 * tiled kernel otherwise.
 * Replace the M <= 16 use of fused_int8_gemm_dequant / fused_w4a8_gemm_dequant
 * (kernels/triton_int8_gemm.py:135-205, triton_w4a8_gemm.py:111-169) and of
 * F.linear on unpacked weights (_ops.py:466-481), e.g. Flux modulation linears.
 */
#define IC_GEMV_MAX_M 16
#define IC_GEMV_MAX_K 16384
int ic_gemv_w8a8(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N,
                 int64_t ldw, const float* s_a, const float* s_w, const void* bias, int bias_dtype,
                 void* out, int out_dtype, int64_t ldo, void* stream);
int ic_gemv_w4a8(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                 int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a,
                 const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo,
                 void* stream);
int ic_gemv_w4a16(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                  int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const void* bias,
                  int bias_dtype, void* out, int64_t ldo, void* stream);

/*
 * Single-launch small-batch linear on raw activations: the preparation and
 * per-token quantization of ic_rotate_quantize (same x, dtype, M, K_in, ldx,
 * sr_rcp/sr_f, rot_size, perm, sm_rcp/sm_f; K plays K_w) followed by the W4A8
 * / W8A8 GEMV with the epilogue options of ic_gemm_*_ex, in one kernel.  Each
 * workgroup prepares the M rows itself in LDS while its first weight loads are
 * in flight; outputs are bit-identical to ic_rotate_quantize followed by
 * ic_gemm_w4a8_ex / ic_gemm_w8a8_ex (which route M <= IC_GEMV_MAX_M to the
 * GEMV).  Limits: dtype f16/bf16; 1 <= M <= IC_GEMV_MAX_M (M = 0: no-op);
 * K a multiple of 128, K <= IC_PREP_GEMV_MAX_K and M * K <=
 * IC_PREP_GEMV_MAX_CODES; weights 16-byte aligned with a row stride (ldw, in
 * bytes for both formats: INT4 rows hold K/2 bytes) that is a multiple of
 * 16; W4A8 num_groups 1 or K/128.  Outside them IC_ERR_UNSUPPORTED: the two
 * calls cover every shape.  Replace the small-M use of
 * fused_quant_int8_gemm_dequant (kernels/triton_int8_gemm.py:243-389) behind
 * _ops.py:443-464 and :493-579.
 */
#define IC_PREP_GEMV_MAX_K 8192
#define IC_PREP_GEMV_MAX_CODES 16384
int ic_prep_gemv_w4a8(const void* x, int dtype, int64_t M, int64_t K_in, int64_t ldx, const float* sr_rcp,
                      const float* sr_f, int rot_size, const int32_t* perm, const float* sm_rcp, const float* sm_f,
                      const uint8_t* w_packed, int64_t N, int64_t K, int64_t ldw, const float* s_w,
                      int64_t num_groups, const void* bias, int bias_dtype, int activation, const void* residual,
                      int residual_dtype, int64_t ldr, void* out, int out_dtype, int64_t ldo, void* stream);
int ic_prep_gemv_w8a8(const void* x, int dtype, int64_t M, int64_t K_in, int64_t ldx, const float* sr_rcp,
                      const float* sr_f, int rot_size, const int32_t* perm, const float* sm_rcp, const float* sm_f,
                      const int8_t* w, int64_t N, int64_t K, int64_t ldw, const float* s_w, const void* bias,
                      int bias_dtype, int activation, const void* residual, int residual_dtype, int64_t ldr,
                      void* out, int out_dtype, int64_t ldo, void* stream);

/* INT4 -> int8 unpack (no scale).  kernels/triton_int4_to_int8_unpack.py:55-81. */
int ic_unpack_int4_to_int8(const uint8_t* packed, int64_t N, int64_t K, int64_t ldp, int8_t* out,
                           int64_t ldo, void* stream);
/* INT4 -> fp16/bf16 with scale, w = RN_dt(q * RN_dt(s[n, k/gs])).
 * kernels/triton_int4_unpack.py:62-88 (per-row scale there; [N, G] here). */
int ic_unpack_int4_to_float(const uint8_t* packed, const float* s_w, int64_t num_groups, int64_t N,
                            int64_t K, int64_t ldp, void* out, int out_dtype, int64_t ldo, void* stream);

/*
 * Grouped W4A8 on gfx950's f8f6f4 MFMA with 6-bit (e3m2) operands: the same
 * function as ic_gemm_w4a8 with num_groups > 1 (fused_w4a8_gemm_dequant,
 * kernels/triton_w4a8_gemm.py:111-169, with the group layout of
 * _quant_utils.py:237-270), bit-identical outputs, on operands converted once:
 *   ic_f6_split_activations: int8 codes x [M, K] -> a6 (ic_f6_activation_bytes),
 *     each code split as x = 16 h + l with h in [-8, 8], l in [-8, 7];
 *   ic_f6_repack_weights: packed INT4 [N, K/2] -> w6 (ic_f6_weight_bytes).
 * Both buffers are blocked by 16 rows / columns (layout in csrc/gemm_f6.h) and
 * must be 16-byte aligned.  K a multiple of 128, groups of a multiple of 128
 * columns, at least two; N and ldo multiples of 8; f16 / bf16 output.  An
 * alternative path: the library's own routing keeps the int8 kernel, which
 * measured as fast.
 */
int64_t ic_f6_activation_bytes(int64_t M, int64_t K);
int64_t ic_f6_weight_bytes(int64_t N, int64_t K);
int ic_f6_split_activations(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, uint8_t* a6, void* stream);
int ic_f6_repack_weights(const uint8_t* w_packed, int64_t N, int64_t K, int64_t ldw, uint8_t* w6, void* stream);
int ic_gemm_w4a8_f6(const uint8_t* a6, int64_t M, int64_t K, const uint8_t* w6, int64_t N, const float* s_w,
                    int64_t num_groups, const float* s_a, const void* bias, int bias_dtype, void* out,
                    int out_dtype, int64_t ldo, void* stream);

/* Debug: raw int32 accumulators of the production GEMM kernels (generic != 0
 * selects the shape-generic kernel instead).  W8A8: acc [M,N].  W4A8: acc
 * [num_groups, M, N], one slab per group.  Pins the integer stage of
 * triton_int8_gemm.py:96-103 / triton_w4a8_gemm.py:84-91 bit-exactly. */
int ic_gemm_w8a8_acc_i32(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w,
                         int64_t N, int64_t ldw, int32_t* acc, int generic, void* stream);
int ic_gemm_w4a8_acc_i32(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                         int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, int32_t* acc,
                         int generic, void* stream);
/* Shape-generic W8A8 kernel (any K/alignment); same arithmetic as ic_gemm_w8a8. */
int ic_gemm_w8a8_generic(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w,
                         int64_t N, int64_t ldw, const float* s_a, const float* s_w,
                         const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INTCRUSH_H */
