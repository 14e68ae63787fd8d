// Internal declarations shared by the kernel translation units and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/mi355x_fp8.h"

namespace mi355x {

int launch_act_quant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm, int64_t sxk,
                     uint8_t* q, int64_t ldq, int64_t kpad, float* s, int64_t ssm, int64_t ssk,
                     hipStream_t stream);

int launch_silu_mul_quant(const void* gate, const void* up, int dtype, int64_t ld, int64_t M, int64_t I,
                          uint16_t* h_out, int64_t ldh, uint8_t* q, int64_t ldq, int64_t kpad, float* s,
                          int64_t ssm, int64_t ssk, hipStream_t stream);

int launch_rmsnorm_quant(const uint16_t* x, int64_t sxm, const uint16_t* res, int64_t ldr, uint16_t* res_out,
                         int64_t ldro, const uint16_t* weight, float eps, int64_t M, int64_t K, uint16_t* y,
                         int64_t ldy, uint8_t* q, int64_t ldq, int64_t kpad, float* s, int64_t ssm, int64_t ssk,
                         hipStream_t stream);
// Virtual threads per row of PyTorch's last-dim reduction (the RMSNorm summation order).
int rmsnorm_block_width(int64_t rows, int64_t K);

// Plan of one block-GEMM launch: which kernel and its tile shape.
struct GemmPlan {
  int kernel;       // MI355X_FP8_CONFIG_STREAM or MI355X_FP8_CONFIG_TILE128
  int token_tiles;  // stream kernel: 16-token MFMA tiles per slice (1 or 2)
  int row_tiles;    // stream kernel: 16-row MFMA tiles of W per workgroup (1 to 5)
  int rows;         // stream kernel: W rows per workgroup (at most 16 row_tiles)
};

int plan_gemm(int64_t M, int64_t N, int64_t K, int config, GemmPlan* plan);
// The same plan for a device with `cus` compute units (plan_gemm: the current device's).
int plan_gemm_on(int64_t M, int64_t N, int64_t K, int config, int64_t cus, GemmPlan* plan);

// Device workspace the GEMM needs (none: every reduction stays inside a workgroup).
size_t gemm_workspace_bytes(const GemmPlan& plan);

int launch_block_gemm(const GemmPlan& plan, const uint8_t* q, int64_t ldq, const float* as,
                      int64_t as_sm, int64_t as_sk, const uint8_t* w, int64_t ldw, const float* ws,
                      int64_t ws_sn, int64_t ws_sk, void* out, int out_dtype, int64_t ldo,
                      int64_t M, int64_t N, int64_t K, void* workspace, hipStream_t stream);

// The whole linear in one stream-kernel launch (quantization inside), for plans of the stream
// kernel with one token tile; MI355X_FP8_ERR_UNSUPPORTED (nothing launched) when the call
// does not fit that form.
int launch_linear_stream(const GemmPlan& plan, const void* x, int x_dtype, int64_t sxm, int64_t sxk,
                         const uint8_t* w, int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, void* out,
                         int out_dtype, int64_t ldo, int64_t M, int64_t N, int64_t K, hipStream_t stream);

// Residual add + RMSNorm + quantizer + GEMM in one stream-kernel launch (bf16 in and out);
// MI355X_FP8_ERR_UNSUPPORTED (nothing launched) when the call does not fit that form.
int launch_norm_linear(const GemmPlan& plan, const uint16_t* x, int64_t sxm, const uint16_t* res, int64_t ldr,
                       uint16_t* res_out, int64_t ldro, const uint16_t* norm_w, float eps, const uint8_t* w,
                       int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, uint16_t* out, int64_t ldo,
                       int64_t M, int64_t N, int64_t K, hipStream_t stream);

// Residual add + RMSNorm + quantizer + merged gate/up GEMM + SiLU*up in one stream-kernel
// launch: h[M, N / 2] = bf16(bf16(silu(gate)) * up); MI355X_FP8_ERR_UNSUPPORTED (nothing
// launched) when the call does not fit that form.
int launch_norm_gate_up_silu(const uint16_t* x, int64_t sxm, const uint16_t* res, int64_t ldr, uint16_t* res_out,
                             int64_t ldro, const uint16_t* norm_w, float eps, const uint8_t* w, int64_t ldw,
                             const float* ws, int64_t ws_sn, int64_t ws_sk, uint16_t* h, int64_t ldh, int64_t M,
                             int64_t N, int64_t K, hipStream_t stream);

// LDS-DMA pipelined prefill kernel (tile_gemm_dma.hip) and its preconditions.
bool tile_dma_supported(const uint8_t* q, int64_t ldq, int64_t as_sm, int64_t as_sk, const uint8_t* w,
                        int64_t ldw, int64_t M, int64_t K);
// bn: tile width, 64, 128 or 160; rows: tile rows, 128, or 64 (widths 64 and 128).
int launch_tile_dma(const uint8_t* q, int64_t ldq, const float* as, int64_t as_sk, const uint8_t* w,
                    int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, void* out, int out_dtype,
                    int64_t ldo, int64_t M, int64_t N, int64_t K, int bn, int rows, hipStream_t stream);

// 256-row-tile prefill kernel (tile_gemm_256.hip), or its 192-row form (rows = 192); same
// preconditions as the DMA kernel.  bn: tile width, 256, 224 or 192 (two-stage LDS ring) or
// 160 or 128 (three-stage ring); tile256_width picks the 256-row width with the lowest
// measured cost on `cus` CUs.
int launch_tile256(const uint8_t* q, int64_t ldq, const float* as, int64_t as_sk, const uint8_t* w,
                   int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, void* out, int out_dtype,
                   int64_t ldo, int64_t M, int64_t N, int64_t K, int bn, int rows, hipStream_t stream);
int tile256_width(int64_t M, int64_t N, int64_t cus);
// The prefill kernel the automatic dispatch picks for an M x N output on `cus` CUs (when the
// LDS-DMA preconditions hold and the offsets fit): tile rows (64, 128, 192 or 256) and width.
void prefill_choice(int64_t M, int64_t N, int64_t cus, int* rows, int* bn);
// Whether the 256-row kernel's 32-bit byte offsets reach every byte of q and W.
bool tile256_offsets_ok(int64_t ldq, int64_t ldw, int64_t M, int64_t N, int64_t K);

// Streaming read of `bytes` (a multiple of 16, 16-byte aligned) for the decode ceiling;
// sink holds sink_words >= 8 x CUs words.
int launch_read_probe(const void* src, size_t bytes, void* sink, size_t sink_words, hipStream_t stream);

// Compute units of the current device (cached per device; 256 if it cannot be queried).
int64_t device_cus();

inline size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

// How a prefill kernel may store its 16-bit output rows: 2 in 16-byte pieces through LDS
// (16-byte aligned rows), 1 in 8-byte pieces, 0 one element at a time.
inline int out_vec_mode(const void* out, int64_t ldo) {
  const uintptr_t p = reinterpret_cast<uintptr_t>(out);
  if (ldo % 8 == 0 && p % 16 == 0) return 2;
  return (ldo % 4 == 0 && p % 8 == 0) ? 1 : 0;
}

}  // namespace mi355x
