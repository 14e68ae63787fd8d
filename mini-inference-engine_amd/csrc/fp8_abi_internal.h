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

// Plan of one block-GEMM launch: which kernel, its grid, and the workspace it needs.
struct GemmPlan {
  int kernel;        // MI355X_FP8_CONFIG_STREAM or MI355X_FP8_CONFIG_TILE128
  int token_tiles;   // stream kernel: 16-token MFMA tiles per wave (1, 2 or 4)
  int64_t strips;    // stream kernel: 64-row strips of W
  int64_t splits;    // stream kernel: K splits (workgroups per strip)
  int64_t kb_per_split;
  size_t partial_bytes;  // fp32 split-K partials
};

// Every workspace starts with a fixed region of per-strip arrival counters.  The caller
// zero-fills it once; the stream kernel's last-arriving workgroup of each strip resets its
// counter, so the region is zero again after every call, whatever shapes share it.
constexpr int64_t kCounterSlots = 65536;
constexpr size_t kCounterRegionBytes = kCounterSlots * sizeof(unsigned);

int plan_gemm(int64_t M, int64_t N, int64_t K, int config, GemmPlan* plan);

// Workspace layout: [counter region | partials], 256-byte aligned.
size_t gemm_workspace_bytes(const GemmPlan& plan);

int launch_block_gemm(const GemmPlan& plan, const uint8_t* q, int64_t ldq, const float* as,
                      int64_t as_sm, int64_t as_sk, const uint8_t* w, int64_t ldw, const float* ws,
                      int64_t ws_sn, int64_t ws_sk, void* out, int out_dtype, int64_t ldo,
                      int64_t M, int64_t N, int64_t K, void* workspace, hipStream_t stream);

inline size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

}  // namespace mi355x
