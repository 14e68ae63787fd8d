/*
 * C-ABI of libmi355x_fp8.so: the dynamic block-scaled FP8 linear on AMD MI355X (gfx950).
 *
 * Contract (reference: engine/kernels/sm89_fp8.py): bf16/fp16 activations in, OCP
 * e4m3fn weights [N, K] (K contiguous) with fp32 128x128 block scales
 * [ceil(N/128), ceil(K/128)], bf16/fp16 out.  Activations are quantized per row and
 * 128-wide K group: s = amax/448 (stored raw), q = e4m3fn(x / max(s, 1e-12)).  The GEMM
 * accumulates, per 128-wide K group in increasing order, dot(q, w) * a_s * w_s in fp32.
 *
 * All pointers are device pointers; all sizes, strides and leading dimensions are in
 * elements and are 64-bit.  Calls are asynchronous on `stream` (a hipStream_t, NULL =
 * the null stream), never allocate, never synchronize, and are therefore safe to capture
 * in a HIP graph.  Every entry point returns an MI355X_FP8_* status code.
 */
#ifndef MI355X_FP8_H
#define MI355X_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI355X_FP8_ABI_VERSION 2

/* Element types of activations and outputs. */
#define MI355X_FP8_DTYPE_BF16 0
#define MI355X_FP8_DTYPE_F16 1

/* GEMM kernel selection (the `gemm_config` of the reference's wrapper). */
#define MI355X_FP8_CONFIG_AUTO 0
#define MI355X_FP8_CONFIG_STREAM 1  /* weight-streaming decode kernel (auto: up to 64 rows) */
#define MI355X_FP8_CONFIG_TILE128 2 /* LDS-tiled 128x128 MFMA kernel, any M */
#define MI355X_FP8_CONFIG_TILE256 3 /* 256-row MFMA kernel, width by cost model; needs K % 128
                                       == 0, 16-byte aligned q/w and K-group-major activation
                                       scales */
/* One prefill kernel variant each (same preconditions as TILE256; otherwise the call returns
 * MI355X_FP8_ERR_UNSUPPORTED): the 128-row LDS-DMA kernel at width 64, 128 or 160, the
 * 256-row kernel and its 192-row form at width 128, 160, 192, 224 or 256, and the 64-row form
 * of the LDS-DMA kernel at width 64 or 128.  Every config gives
 * the same bits; these exist for tuning and so that tests can reach each variant. */
#define MI355X_FP8_CONFIG_DMA128_64 4
#define MI355X_FP8_CONFIG_DMA128_128 5
#define MI355X_FP8_CONFIG_DMA128_160 6
#define MI355X_FP8_CONFIG_T256_128 7
#define MI355X_FP8_CONFIG_T256_160 8
#define MI355X_FP8_CONFIG_T256_192 9
#define MI355X_FP8_CONFIG_T256_224 10
#define MI355X_FP8_CONFIG_T256_256 11
#define MI355X_FP8_CONFIG_T192_128 12
#define MI355X_FP8_CONFIG_T192_160 13
#define MI355X_FP8_CONFIG_T192_192 14
#define MI355X_FP8_CONFIG_T192_224 15
#define MI355X_FP8_CONFIG_T192_256 16
#define MI355X_FP8_CONFIG_DMA64_64 17
#define MI355X_FP8_CONFIG_DMA64_128 18

/* Status codes. */
#define MI355X_FP8_OK 0
#define MI355X_FP8_ERR_INVALID 1     /* bad size, stride or dtype (Python: ValueError) */
#define MI355X_FP8_ERR_UNSUPPORTED 2 /* valid but not supported here (RuntimeError) */
#define MI355X_FP8_ERR_WORKSPACE 3   /* workspace missing or too small (ValueError) */
#define MI355X_FP8_ERR_LAUNCH 4      /* HIP launch failure (RuntimeError) */
#define MI355X_FP8_ERR_SCRATCH 5     /* larger than the static scratch of the no-allocation
                                        entry point (ValueError) */

/* Bytes of device scratch each GPU holds for mi355x_fp8_linear_noalloc (24 MiB). */
#define MI355X_FP8_NOALLOC_SCRATCH_BYTES (24u << 20)

/* Version of this ABI; equals MI355X_FP8_ABI_VERSION of the header it was built with. */
int mi355x_fp8_abi_version(void);

/* Static text for a status code. */
const char* mi355x_fp8_status_string(int status);

/*
 * Activation quantizer.  Replaces quantize_sm89_fp8_activation and its
 * _quantize_activation_kernel (engine/kernels/sm89_fp8.py:401-424, :304-332).
 *   x     : M x K activations of x_dtype, element (m, k) at x[m*sxm + k*sxk]
 *   q     : e4m3fn codes, element (m, k) at q[m*ldq + k]; columns [K, kpad) are written
 *           as code 0 (kpad >= K, kpad <= 128*ceil(K/128), ldq >= kpad)
 *   s     : fp32 scales, element (m, g) at s[m*s_sm + g*s_sk], g < ceil(K/128)
 * M == 0 is a no-op; K must be positive.
 */
int mi355x_fp8_act_quant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm,
                         int64_t sxk, uint8_t* q, int64_t ldq, int64_t kpad, float* s,
                         int64_t s_sm, int64_t s_sk, void* stream);

/*
 * Workspace bytes that mi355x_fp8_block_gemm needs for (M, N, K, config); 0 when the
 * chosen kernels need none (the current ones).  A workspace is scratch: its contents need
 * no initialisation, and calls that overlap in time must not share one.
 */
size_t mi355x_fp8_block_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int config);

/*
 * Block-scaled FP8 GEMM on pre-quantized activations.  Replaces _launch_split_gemm and
 * _fp8_split_gemm_kernel (engine/kernels/sm89_fp8.py:427-441, :344-398).
 *   q   : M x K e4m3fn, (m, k) at q[m*ldq + k]
 *   as  : activation scales, (m, kb) at as[m*as_sm + kb*as_sk]
 *   w   : N x K e4m3fn, (n, k) at w[n*ldw + k]
 *   ws  : weight block scales, (nb, kb) at ws[nb*ws_sn + kb*ws_sk]
 *   out : M x N of out_dtype, (m, n) at out[m*ldo + n]
 */
int mi355x_fp8_block_gemm(const uint8_t* q, int64_t ldq, const float* as, int64_t as_sm,
                          int64_t as_sk, const uint8_t* w, int64_t ldw, const float* ws,
                          int64_t ws_sn, int64_t ws_sk, void* out, int out_dtype, int64_t ldo,
                          int64_t M, int64_t N, int64_t K, void* workspace,
                          size_t workspace_bytes, int config, void* stream);

/* Workspace bytes that mi355x_fp8_linear needs: the quantized activations, their scales
 * and the GEMM's workspace.  Same rules as the GEMM workspace. */
size_t mi355x_fp8_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int config);

/*
 * The full linear: quantize x, then the block GEMM.  Replaces the kernel launches of
 * sm89_fp8_linear (engine/kernels/sm89_fp8.py:488-526); the Python wrapper keeps the
 * reference's validation, reshaping and bias handling.  Arguments as above.  At decode
 * sizes with short K (M <= 16, K <= 3072, K % 16 == 0, 16-byte aligned rows) it is one
 * launch that quantizes inside the GEMM, like the reference's fused path; the workspace is
 * then untouched.  Either way the output bits are the same.
 */
int mi355x_fp8_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm,
                      int64_t sxk, const uint8_t* w, int64_t ldw, const float* ws,
                      int64_t ws_sn, int64_t ws_sk, int64_t N, void* out, int out_dtype,
                      int64_t ldo, void* workspace, size_t workspace_bytes, int config,
                      void* stream);

/*
 * mi355x_fp8_linear without a workspace argument: no reference counterpart.  For callers
 * that cannot allocate device memory (code under HIP-graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The quantized activations and their scales go to a
 * static device array of MI355X_FP8_NOALLOC_SCRATCH_BYTES per GPU (held until the process
 * ends); calls whose mi355x_fp8_linear_workspace_bytes exceed it return
 * MI355X_FP8_ERR_SCRATCH before launching anything.  The call allocates nothing and gives
 * the bits of mi355x_fp8_linear.  Every call on one GPU shares that GPU's scratch:
 * calls that overlap in time on one GPU (different streams, or host threads) race.
 * Set-up: call mi355x_fp8_linear_noalloc_scratch_bytes() once per device, with that device
 * current and outside graph capture; it looks up the device's scratch address (a
 * hipGetSymbolAddress), which the first noalloc call on a device would otherwise do.
 */
int mi355x_fp8_linear_noalloc(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm,
                              int64_t sxk, const uint8_t* w, int64_t ldw, const float* ws,
                              int64_t ws_sn, int64_t ws_sk, int64_t N, void* out, int out_dtype,
                              int64_t ldo, int config, void* stream);

/* MI355X_FP8_NOALLOC_SCRATCH_BYTES, as built into the library; also resolves the current
 * device's scratch address (the no-allocation entry point's set-up call). */
size_t mi355x_fp8_linear_noalloc_scratch_bytes(void);

/*
 * Dispatch introspection, no reference counterpart (for tests and tuning): the prefill
 * kernel the automatic dispatch runs for an M x N output (M above the decode range, LDS-DMA
 * preconditions met) on a device with `cus` CUs, from the table of measured wave times:
 * *rows = tile rows (64 or 128: the LDS-DMA kernel; 192 or 256: the 256-row kernel and its
 * 192-row form), *bn = tile width.  Pure host computation: no device is touched.
 */
int mi355x_fp8_prefill_choice(int64_t M, int64_t N, int64_t cus, int* rows, int* bn);

/*
 * Dispatch introspection, no reference counterpart (for benchmarks and tests): the kernel
 * family the automatic dispatch of an M x N x K GEMM picks on a device with `cus` CUs, for
 * 16-byte aligned operands with K % 128 == 0.  *kernel = MI355X_FP8_CONFIG_STREAM (the
 * weight-streaming decode kernel: *rows = weight rows per workgroup, *cols = token rows per
 * slice) or MI355X_FP8_CONFIG_TILE128 (a prefill tile: *rows x *cols as in
 * mi355x_fp8_prefill_choice).  Pure host computation: no device is touched.
 */
int mi355x_fp8_dispatch_choice(int64_t M, int64_t N, int64_t K, int64_t cus, int* kernel, int* rows, int* cols);

/*
 * Measurement helper, no reference counterpart: reads `bytes` of device memory at `src`
 * once (16-byte loads over all CUs) and nothing else, so that a benchmark can time the
 * streaming-read rate one launch reaches over the same bytes as a decode GEMM.  bytes must
 * be a multiple of 16 and src 16-byte aligned; sink is a device buffer of sink_words >=
 * 8 x (number of CUs) 32-bit words (its contents are unspecified afterwards).
 */
int mi355x_fp8_read_probe(const void* src, size_t bytes, void* sink, size_t sink_words, void* stream);

/*
 * Fused SiLU(gate) * up followed by the activation quantizer, for the MLP's down_proj.
 * Replaces silu_mul (engine/kernels/fused.py:127-137, 217-232) plus the quantizer launch of
 * the down projection (engine/kernels/sm89_fp8.py:401-424) in _mlp_forward
 * (fused.py:280-283).
 *   gate, up : M x I bf16, (m, i) at gate[m*ld + i] / up[m*ld + i] (for one merged
 *              gate_up output: up = gate + I, ld = 2 I)
 *   h        : optional (NULL: not written) bf16 bf16(bf16(silu(g)) * u), (m, i) at h[m*ldh + i]
 *   q, s     : quantized h and its raw fp32 scales, as in mi355x_fp8_act_quant
 * x_dtype must be MI355X_FP8_DTYPE_BF16 (fp16 returns MI355X_FP8_ERR_UNSUPPORTED).
 */
int mi355x_fp8_silu_mul_quant(const void* gate, const void* up, int x_dtype, int64_t M, int64_t I,
                              int64_t ld, void* h, int64_t ldh, uint8_t* q, int64_t ldq, int64_t kpad,
                              float* s, int64_t s_sm, int64_t s_sk, void* stream);

/*
 * Fused RMSNorm (optionally after the residual add) followed by the activation quantizer,
 * the input of the q/k/v and gate/up projections.  Replaces rms_norm
 * (engine/kernels/fused.py:89-124, 165-199) plus the quantizer launch of the projection
 * that consumes its output (engine/kernels/sm89_fp8.py:401-424).
 *   x        : M x K bf16, (m, k) at x[m*sxm + k]; K % 4 == 0 and K >= 128 (rows wider
 *              than 16128 return MI355X_FP8_ERR_UNSUPPORTED: a row and the weight are
 *              staged in LDS)
 *   residual : optional (NULL: none) M x K bf16 at residual[m*ldr + k]; then residual_out
 *              (m, k) at residual_out[m*ldro + k] receives bf16(x + residual), the input
 *              of the normalization
 *   weight   : K bf16 (the norm's gain)
 *   y        : optional (NULL: not written) bf16 normalized output at y[m*ldy + k]
 *   q, s     : quantized normalized output and its raw fp32 scales, as in mi355x_fp8_act_quant
 * The row sum follows PyTorch's reduction order for M rows of width K; 1/sqrt is correctly
 * rounded (the reference's libdevice rsqrt is approximate: y can differ in the last bf16
 * place).  x_dtype must be MI355X_FP8_DTYPE_BF16 (fp16 returns MI355X_FP8_ERR_UNSUPPORTED).
 */
int mi355x_fp8_rmsnorm_quant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm,
                             const void* residual, int64_t ldr, void* residual_out, int64_t ldro,
                             const void* weight, float eps, void* y, int64_t ldy, uint8_t* q,
                             int64_t ldq, int64_t kpad, float* s, int64_t s_sm, int64_t s_sk,
                             void* stream);

/* Residual add + RMSNorm + activation quantizer + block GEMM in one launch, at decode sizes:
 * out = fp8_linear(rms_norm(x [+ residual])) for bf16 x and bf16 out.  It replaces the pair
 * the reference runs for the q/k/v and gate/up projections, rms_norm
 * (engine/kernels/fused.py:165-199) followed by sm89_fp8_linear (engine/kernels/
 * sm89_fp8.py:444-528), and gives the bits of this library's two-launch form of that pair
 * (mi355x_fp8_rmsnorm_quant, then mi355x_fp8_block_gemm on its q and scales); residual_out
 * receives bf16(x + residual) as there.  Each workgroup of the weight-streaming kernel
 * recomputes the rows' norms, so this pays only at few rows: it returns
 * MI355X_FP8_ERR_UNSUPPORTED, having launched nothing, when the call does not fit one launch
 * (more than 8 rows, K not a multiple of 256 or above 2560, rows not 16-byte aligned, or a
 * shape the decode kernel does not take), and the caller then runs the two launches.
 * Operands as in mi355x_fp8_rmsnorm_quant (x, residual, norm weight) and mi355x_fp8_linear
 * (w, ws, out).  residual_out must not overlap x or residual (every workgroup reads them
 * while one writes the sum): such a call also returns MI355X_FP8_ERR_UNSUPPORTED. */
int mi355x_fp8_rmsnorm_linear(const void* x, int64_t M, int64_t K, int64_t sxm, const void* residual, int64_t ldr,
                              void* residual_out, int64_t ldro, const void* norm_weight, float eps, const uint8_t* w,
                              int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, int64_t N, void* out,
                              int64_t ldo, void* stream);

/* Residual add + RMSNorm + activation quantizer + merged gate/up block GEMM + SiLU*up in one
 * launch, at decode sizes: h = silu_mul(fp8_linear(rms_norm(x [+ residual]), w)) with w the
 * merged gate/up weight (N = 2 I rows, gate rows first, as merged_projections builds it) and
 * h [M, I] bf16 (row stride ldh >= I).  It replaces the reference's rms_norm
 * (engine/kernels/fused.py:165-199), the merged gate_up sm89_fp8_linear (engine/kernels/
 * sm89_fp8.py:444-528, through merged_projections.project_gate_up) and silu_mul
 * (fused.py:217-232, the _silu_mul_kernel of fused.py:127-137), and gives the bits of this
 * library's separate forms: mi355x_fp8_rmsnorm_linear's gate_up output, then
 * h = bf16(bf16(g / (1 + exp(-g))) * u) on its bf16 gate and up columns (the h of
 * mi355x_fp8_silu_mul_quant).  residual_out receives bf16(x + residual).  Each workgroup owns
 * matching gate and up rows; it returns MI355X_FP8_ERR_UNSUPPORTED, having launched nothing,
 * under the conditions of mi355x_fp8_rmsnorm_linear (more than 8 rows, K not a multiple of
 * 256 or above 2560, unaligned rows, residual_out over an input) or when N is odd, and the
 * caller then runs the separate launches.  Operands as in mi355x_fp8_rmsnorm_linear. */
int mi355x_fp8_rmsnorm_gate_up_silu(const void* x, int64_t M, int64_t K, int64_t sxm, const void* residual,
                                    int64_t ldr, void* residual_out, int64_t ldro, const void* norm_weight, float eps,
                                    const uint8_t* w, int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk,
                                    int64_t N, void* h, int64_t ldh, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI355X_FP8_H */
