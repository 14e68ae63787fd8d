// extern "C" entry points of libmi355x_fp8.so (declared in include/mi355x_fp8.h).
// Argument validation lives here; the kernels assume validated shapes.
#include "fp8_abi_internal.h"

#include <mutex>

using namespace mi355x;

// Device-resident scratch of mi355x_fp8_linear_noalloc: the quantized activations and their
// scales.  Every GPU the library runs on holds its own copy until the process ends.  Host
// code must never pass this name to a kernel (on the host it is only a stand-in for the
// symbol): the device address comes from hipGetSymbolAddress, per device, in
// scratch_ptr().
static __device__ __align__(256) uint8_t scratch[MI355X_FP8_NOALLOC_SCRATCH_BYTES];

namespace {

int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool valid_dtype(int d) { return d == MI355X_FP8_DTYPE_BF16 || d == MI355X_FP8_DTYPE_F16; }

// Byte range [p, p + bytes) of rows x cols 2-byte elements at row stride ld (elements).
bool overlaps(const void* a, int64_t rows_a, int64_t cols_a, int64_t ld_a, const void* b, int64_t rows_b,
              int64_t cols_b, int64_t ld_b) {
  if (a == nullptr || b == nullptr || rows_a <= 0 || rows_b <= 0) return false;
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
  const uintptr_t a1 = a0 + 2 * static_cast<uintptr_t>((rows_a - 1) * ld_a + cols_a);
  const uintptr_t b1 = b0 + 2 * static_cast<uintptr_t>((rows_b - 1) * ld_b + cols_b);
  return a0 < b1 && b0 < a1;
}

// Layout of the linear's workspace: [GEMM workspace | q (M x Kpad) | a_s (KB x Mpad)].
struct LinearLayout {
  GemmPlan plan;
  int64_t kpad, mpad, kb;
  size_t gemm_bytes, q_off, s_off, total;
};

int linear_layout(int64_t M, int64_t N, int64_t K, int config, LinearLayout* L) {
  int st = plan_gemm(M, N, K, config, &L->plan);
  if (st != MI355X_FP8_OK) return st;
  L->kb = cdiv64(K, 128);
  L->kpad = L->kb * 128;
  L->mpad = cdiv64(M > 0 ? M : 1, 64) * 64;
  L->gemm_bytes = gemm_workspace_bytes(L->plan);
  L->q_off = align256(L->gemm_bytes);
  L->s_off = L->q_off + align256(static_cast<size_t>(M) * static_cast<size_t>(L->kpad));
  L->total = L->s_off + align256(static_cast<size_t>(L->kb) * static_cast<size_t>(L->mpad) * sizeof(float));
  return MI355X_FP8_OK;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device (with that device
// current, as hipGetSymbolAddress answers for the current device).  nullptr on failure.
void* scratch_ptr() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) return nullptr;
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int mi355x_fp8_abi_version(void) { return MI355X_FP8_ABI_VERSION; }

const char* mi355x_fp8_status_string(int status) {
  switch (status) {
    case MI355X_FP8_OK: return "ok";
    case MI355X_FP8_ERR_INVALID: return "invalid argument";
    case MI355X_FP8_ERR_UNSUPPORTED: return "unsupported call";
    case MI355X_FP8_ERR_WORKSPACE: return "workspace missing or too small";
    case MI355X_FP8_ERR_LAUNCH: return "HIP kernel launch failed";
    case MI355X_FP8_ERR_SCRATCH: return "call needs more than the library's static scratch";
    default: return "unknown status";
  }
}

int mi355x_fp8_act_quant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm,
                         int64_t sxk, uint8_t* q, int64_t ldq, int64_t kpad, float* s,
                         int64_t s_sm, int64_t s_sk, void* stream) {
  if (!valid_dtype(x_dtype) || M < 0 || K <= 0 || kpad < K || kpad > cdiv64(K, 128) * 128 || ldq < kpad)
    return MI355X_FP8_ERR_INVALID;
  if (M == 0) return MI355X_FP8_OK;
  if (!x || !q || !s) return MI355X_FP8_ERR_INVALID;
  return launch_act_quant(x, x_dtype, M, K, sxm, sxk, q, ldq, kpad, s, s_sm, s_sk,
                          static_cast<hipStream_t>(stream));
}

int mi355x_fp8_silu_mul_quant(const void* gate, const void* up, int x_dtype, int64_t M, int64_t I,
                              int64_t ld, void* h, int64_t ldh, uint8_t* q, int64_t ldq, int64_t kpad,
                              float* s, int64_t s_sm, int64_t s_sk, void* stream) {
  if (!valid_dtype(x_dtype) || M < 0 || I <= 0 || ld < I || kpad < I || kpad > cdiv64(I, 128) * 128 ||
      ldq < kpad || (h != nullptr && ldh < I))
    return MI355X_FP8_ERR_INVALID;
  if (M == 0) return MI355X_FP8_OK;
  if (!gate || !up || !q || !s) return MI355X_FP8_ERR_INVALID;
  return launch_silu_mul_quant(gate, up, x_dtype, ld, M, I, static_cast<uint16_t*>(h), ldh, q, ldq, kpad, s, s_sm,
                               s_sk, static_cast<hipStream_t>(stream));
}

int mi355x_fp8_rmsnorm_quant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm,
                             const void* residual, int64_t ldr, void* residual_out, int64_t ldro,
                             const void* weight, float eps, void* y, int64_t ldy, uint8_t* q,
                             int64_t ldq, int64_t kpad, float* s, int64_t s_sm, int64_t s_sk,
                             void* stream) {
  if (!valid_dtype(x_dtype) || M < 0 || K < 128 || K % 4 != 0 || sxm < K || kpad < K ||
      kpad > cdiv64(K, 128) * 128 || ldq < kpad || (y != nullptr && ldy < K) ||
      (residual != nullptr && (ldr < K || residual_out == nullptr || ldro < K)))
    return MI355X_FP8_ERR_INVALID;
  // bf16 only: the reference fuses the norm for bf16 activations (fused.py:265-267).
  if (x_dtype != MI355X_FP8_DTYPE_BF16) return MI355X_FP8_ERR_UNSUPPORTED;
  if (M == 0) return MI355X_FP8_OK;
  if (!x || !weight || !q || !s) return MI355X_FP8_ERR_INVALID;
  return launch_rmsnorm_quant(static_cast<const uint16_t*>(x), sxm, static_cast<const uint16_t*>(residual), ldr,
                              static_cast<uint16_t*>(residual_out), ldro, static_cast<const uint16_t*>(weight), eps, M,
                              K, static_cast<uint16_t*>(y), ldy, q, ldq, kpad, s, s_sm, s_sk,
                              static_cast<hipStream_t>(stream));
}

int mi355x_fp8_rmsnorm_linear(const void* x, int64_t M, int64_t K, int64_t sxm, const void* residual, int64_t ldr,
                              void* residual_out, int64_t ldro, const void* norm_weight, float eps, const uint8_t* w,
                              int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, int64_t N, void* out,
                              int64_t ldo, void* stream) {
  if (M < 0 || N < 0 || K < 128 || K % 4 != 0 || sxm < K || ldw < K || ldo < N ||
      (residual != nullptr && (ldr < K || residual_out == nullptr || ldro < K)))
    return MI355X_FP8_ERR_INVALID;
  if (M == 0 || N == 0) return MI355X_FP8_ERR_UNSUPPORTED;  // nothing to fuse: the caller's two launches handle it
  if (!x || !norm_weight || !w || !ws || !out) return MI355X_FP8_ERR_INVALID;
  // Every workgroup reads x and residual while one of them writes residual_out: the sum may
  // not land on either input (the two-launch form, one workgroup per row, takes that case).
  if (residual != nullptr &&
      (overlaps(residual_out, M, K, ldro, x, M, K, sxm) || overlaps(residual_out, M, K, ldro, residual, M, K, ldr)))
    return MI355X_FP8_ERR_UNSUPPORTED;
  GemmPlan plan;
  const int st = plan_gemm(M, N, K, MI355X_FP8_CONFIG_AUTO, &plan);
  if (st != MI355X_FP8_OK) return st;
  return launch_norm_linear(plan, static_cast<const uint16_t*>(x), sxm, static_cast<const uint16_t*>(residual), ldr,
                            static_cast<uint16_t*>(residual_out), ldro, static_cast<const uint16_t*>(norm_weight), eps,
                            w, ldw, ws, ws_sn, ws_sk, static_cast<uint16_t*>(out), ldo, M, N, K,
                            static_cast<hipStream_t>(stream));
}

int mi355x_fp8_rmsnorm_gate_up_silu(const void* x, int64_t M, int64_t K, int64_t sxm, const void* residual,
                                    int64_t ldr, void* residual_out, int64_t ldro, const void* norm_weight, float eps,
                                    const uint8_t* w, int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk,
                                    int64_t N, void* h, int64_t ldh, void* stream) {
  if (M < 0 || N < 0 || N % 2 != 0 || K < 128 || K % 4 != 0 || sxm < K || ldw < K || ldh < N / 2 ||
      (residual != nullptr && (ldr < K || residual_out == nullptr || ldro < K)))
    return MI355X_FP8_ERR_INVALID;
  if (M == 0 || N == 0) return MI355X_FP8_ERR_UNSUPPORTED;
  if (!x || !norm_weight || !w || !ws || !h) return MI355X_FP8_ERR_INVALID;
  if (residual != nullptr &&
      (overlaps(residual_out, M, K, ldro, x, M, K, sxm) || overlaps(residual_out, M, K, ldro, residual, M, K, ldr)))
    return MI355X_FP8_ERR_UNSUPPORTED;
  return launch_norm_gate_up_silu(static_cast<const uint16_t*>(x), sxm, static_cast<const uint16_t*>(residual), ldr,
                                  static_cast<uint16_t*>(residual_out), ldro,
                                  static_cast<const uint16_t*>(norm_weight), eps, w, ldw, ws, ws_sn, ws_sk,
                                  static_cast<uint16_t*>(h), ldh, M, N, K, static_cast<hipStream_t>(stream));
}

size_t mi355x_fp8_block_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int config) {
  GemmPlan plan;
  if (plan_gemm(M, N, K, config, &plan) != MI355X_FP8_OK) return 0;
  return gemm_workspace_bytes(plan);
}

int mi355x_fp8_block_gemm(const uint8_t* q, int64_t ldq, const float* as, int64_t as_sm,
                          int64_t as_sk, const uint8_t* w, int64_t ldw, const float* ws,
                          int64_t ws_sn, int64_t ws_sk, void* out, int out_dtype, int64_t ldo,
                          int64_t M, int64_t N, int64_t K, void* workspace,
                          size_t workspace_bytes, int config, void* stream) {
  if (!valid_dtype(out_dtype) || M < 0 || N < 0 || K <= 0 || ldq < K || ldw < K || ldo < N)
    return MI355X_FP8_ERR_INVALID;
  GemmPlan plan;
  int st = plan_gemm(M, N, K, config, &plan);
  if (st != MI355X_FP8_OK) return st;
  if (M == 0 || N == 0) return MI355X_FP8_OK;
  if (!q || !as || !w || !ws || !out) return MI355X_FP8_ERR_INVALID;
  const size_t need = gemm_workspace_bytes(plan);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return MI355X_FP8_ERR_WORKSPACE;
  return launch_block_gemm(plan, q, ldq, as, as_sm, as_sk, w, ldw, ws, ws_sn, ws_sk, out, out_dtype,
                           ldo, M, N, K, workspace, static_cast<hipStream_t>(stream));
}

size_t mi355x_fp8_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int config) {
  LinearLayout L;
  if (M < 0 || N < 0 || K <= 0 || linear_layout(M, N, K, config, &L) != MI355X_FP8_OK) return 0;
  return L.total;
}

int mi355x_fp8_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm,
                      int64_t sxk, const uint8_t* w, int64_t ldw, const float* ws,
                      int64_t ws_sn, int64_t ws_sk, int64_t N, void* out, int out_dtype,
                      int64_t ldo, void* workspace, size_t workspace_bytes, int config,
                      void* stream) {
  if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype) || M < 0 || N < 0 || K <= 0 || ldw < K || ldo < N)
    return MI355X_FP8_ERR_INVALID;
  LinearLayout L;
  int st = linear_layout(M, N, K, config, &L);
  if (st != MI355X_FP8_OK) return st;
  if (M == 0 || N == 0) return MI355X_FP8_OK;
  if (!x || !w || !ws || !out) return MI355X_FP8_ERR_INVALID;
  if (workspace == nullptr || workspace_bytes < L.total) return MI355X_FP8_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Decode sizes: one launch, the stream kernel quantizing its own K groups (same codes,
  // scales and output bits as the two launches below).
  st = launch_linear_stream(L.plan, x, x_dtype, sxm, sxk, w, ldw, ws, ws_sn, ws_sk, out, out_dtype, ldo, M, N, K, s);
  if (st != MI355X_FP8_ERR_UNSUPPORTED) return st;
  char* base = static_cast<char*>(workspace);
  uint8_t* q = reinterpret_cast<uint8_t*>(base + L.q_off);
  float* as = reinterpret_cast<float*>(base + L.s_off);
  // Activation scales are stored K-group-major ([KB][Mpad]) so that GEMM lanes that own
  // consecutive rows read consecutive scales.
  st = launch_act_quant(x, x_dtype, M, K, sxm, sxk, q, L.kpad, L.kpad, as, 1, L.mpad, s);
  if (st != MI355X_FP8_OK) return st;
  return launch_block_gemm(L.plan, q, L.kpad, as, 1, L.mpad, w, ldw, ws, ws_sn, ws_sk, out, out_dtype,
                           ldo, M, N, K, workspace, s);
}

int mi355x_fp8_read_probe(const void* src, size_t bytes, void* sink, size_t sink_words, void* stream) {
  return launch_read_probe(src, bytes, sink, sink_words, static_cast<hipStream_t>(stream));
}

size_t mi355x_fp8_linear_noalloc_scratch_bytes(void) {
  // Also the set-up call of the no-allocation entry point: resolves the scratch address of
  // the current device here, outside any graph capture the caller starts later.
  (void)scratch_ptr();
  return MI355X_FP8_NOALLOC_SCRATCH_BYTES;
}

int mi355x_fp8_prefill_choice(int64_t M, int64_t N, int64_t cus, int* rows, int* bn) {
  if (M <= 0 || N <= 0 || cus <= 0 || rows == nullptr || bn == nullptr) return MI355X_FP8_ERR_INVALID;
  prefill_choice(M, N, cus, rows, bn);
  return MI355X_FP8_OK;
}

int mi355x_fp8_dispatch_choice(int64_t M, int64_t N, int64_t K, int64_t cus, int* kernel, int* rows, int* cols) {
  if (M <= 0 || N <= 0 || K <= 0 || cus <= 0 || kernel == nullptr || rows == nullptr || cols == nullptr)
    return MI355X_FP8_ERR_INVALID;
  GemmPlan plan;
  const int st = plan_gemm_on(M, N, K, MI355X_FP8_CONFIG_AUTO, cus, &plan);
  if (st != MI355X_FP8_OK) return st;
  *kernel = plan.kernel;
  if (plan.kernel == MI355X_FP8_CONFIG_STREAM) {
    *rows = plan.rows;
    *cols = 16 * plan.token_tiles;
  } else {
    prefill_choice(M, N, cus, rows, cols);
  }
  return MI355X_FP8_OK;
}

int mi355x_fp8_linear_noalloc(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm, int64_t sxk,
                              const uint8_t* w, int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk,
                              int64_t N, void* out, int out_dtype, int64_t ldo, int config, void* stream) {
  if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype) || M < 0 || N < 0 || K <= 0 || ldw < K || ldo < N)
    return MI355X_FP8_ERR_INVALID;
  LinearLayout L;
  int st = linear_layout(M, N, K, config, &L);
  if (st != MI355X_FP8_OK) return st;
  if (M == 0 || N == 0) return MI355X_FP8_OK;
  if (!x || !w || !ws || !out) return MI355X_FP8_ERR_INVALID;
  if (L.total > MI355X_FP8_NOALLOC_SCRATCH_BYTES) return MI355X_FP8_ERR_SCRATCH;
  void* base = scratch_ptr();
  if (base == nullptr) return MI355X_FP8_ERR_LAUNCH;
  // Same kernels and layout as mi355x_fp8_linear, with the scratch in place of the caller's
  // workspace.  Every byte the GEMM reads is written by the quantizer first in stream order
  // (codes up to Kpad, scales of rows < M), so nothing needs clearing between calls.
  return mi355x_fp8_linear(x, x_dtype, M, K, sxm, sxk, w, ldw, ws, ws_sn, ws_sk, N, out, out_dtype, ldo, base,
                           L.total, config, stream);
}

}  // extern "C"
