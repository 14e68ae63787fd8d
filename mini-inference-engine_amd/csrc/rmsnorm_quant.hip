// Fused RMSNorm (optionally after the residual add) -> per-token 1x128 FP8 quantization,
// the input of the q/k/v and gate/up projections.
//
// Semantics follow the reference's _rms_norm_kernel / rms_norm
// (engine/kernels/fused.py:89-124, 165-199), with its quantizer
// (engine/kernels/sm89_fp8.py:304-332) applied to the result:
//   x    = bf16(x + residual)           residual variant (fp32 add, one rounding; also stored)
//   ss   = sum of rounded squares x*x  in PyTorch's reduction order (below)
//   var  = ss * fl(1 / K)              a separate rounding (no fused multiply-add)
//   inv  = 1 / sqrt(var + eps)         here computed in double and rounded once to fp32
//   y    = bf16(w * bf16(x * inv))
//   q, s = the quantizer of y
// The reference calls libdevice's approximate rsqrt; the correctly rounded value used here
// differs from it by at most a couple of ulp, which moves y by one bf16 ulp when a product
// lands next to a rounding boundary.  Everything else is the reference's arithmetic.
//
// Reduction order (PyTorch's vectorized last-dim mean, ATen/native/cuda/Reduce.cuh, as the
// reference reproduces it): bw virtual threads (rmsnorm_block_width below, from the row
// count M and the width K); thread t sums the rounded squares of the 4 elements of vectors
// v = k bw + t, k = 0, 1, ..., in four sequential accumulators; combines them as
// ((a0 + a1) + a2) + a3; then threads fold pairwise, s_t += s_{t+h} for h = bw/2, ..., 1.
//
// Layout: one wave per row.  Lane l plays virtual threads l, l + 64, ... (bw / 64 of them
// when bw >= 64; lanes >= bw idle when bw < 64), so folds with h >= 64 stay inside a lane
// and the rest are shuffles.  A second pass re-reads the row (an L2 hit), normalizes it and
// quantizes it one 128-wide group per 16-lane slice, 8 elements per lane.  HBM traffic per
// row: 2K bytes in (4K with the residual), K + 4K/128 out (+2K for the residual sum).
#include "fp8_abi_internal.h"
#include "fp8_common.h"

namespace mi355x {
namespace {

constexpr int kRnqThreads = 256;           // 4 waves = 4 rows per workgroup
constexpr int kRnqRows = kRnqThreads / 64;

__device__ __forceinline__ float bf16_at(const uint16_t* p) { return __uint_as_float(static_cast<uint32_t>(*p) << 16); }

template <bool RESIDUAL>
__global__ __launch_bounds__(kRnqThreads) void rmsnorm_quant_kernel(
    const uint16_t* __restrict__ x, int64_t sxm, const uint16_t* __restrict__ res, int64_t ldr,
    uint16_t* __restrict__ res_out, int64_t ldro, const uint16_t* __restrict__ weight, float eps, float inv_k,
    int64_t M, int64_t K, int bw, uint16_t* __restrict__ y_out, int64_t ldy, uint8_t* __restrict__ q, int64_t ldq,
    int64_t kpad, float* __restrict__ s, int64_t ssm, int64_t ssk) {
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * kRnqRows + (threadIdx.x >> 6);
  if (m >= M) return;  // whole waves: the row index is uniform across the wave
  const uint16_t* xr = x + m * sxm;
  const uint16_t* rr = RESIDUAL ? res + m * ldr : nullptr;
  uint16_t* ro = RESIDUAL ? res_out + m * ldro : nullptr;

  // ---- pass 1: sum of squares in the reference's order ----------------------------
  const int64_t nvec = K / 4;
  const int per_lane = bw >= 64 ? bw / 64 : 1;  // virtual threads of this lane
  float part[8];                                // bw <= 512: at most 8 per lane
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    part[j] = 0.0f;
    if (j >= per_lane) continue;
    const int t = lane + 64 * j;
    if (t >= bw) continue;
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t v = t; v < nvec; v += bw) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float xv = bf16_at(xr + 4 * v + e);
        if constexpr (RESIDUAL) {
          const uint16_t sb = f32_to_bf16_bits(xv + bf16_at(rr + 4 * v + e));
          ro[4 * v + e] = sb;
          xv = __uint_as_float(static_cast<uint32_t>(sb) << 16);
        }
        a[e] = __fadd_rn(a[e], __fmul_rn(xv, xv));
      }
    }
    part[j] = __fadd_rn(__fadd_rn(__fadd_rn(a[0], a[1]), a[2]), a[3]);
  }
  // Folds with h >= 64: virtual threads j and j + h/64 of the same lane.
  for (int h = bw / 2; h >= 64; h >>= 1) {
    const int hj = h / 64;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < hj) part[j] = __fadd_rn(part[j], part[j + hj]);
  }
  // Folds with h < 64: lane l adds lane l + h.
  float ssum = part[0];
  for (int h = (bw < 64 ? bw : 64) / 2; h >= 1; h >>= 1) {
    const float other = __shfl_down(ssum, h, 64);
    if (lane < h) ssum = __fadd_rn(ssum, other);
  }
  ssum = __shfl(ssum, 0, 64);
  const float var = __fmul_rn(ssum, inv_k);
  const float inv = static_cast<float>(1.0 / sqrt(static_cast<double>(__fadd_rn(var, eps))));
  // ---- pass 2: normalize and quantize, one group per 16-lane slice -----------------
  // The residual sum is recomputed from the inputs (the same rounding as pass 1) rather
  // than re-read from res_out, which other lanes of this wave have just stored.
  const int lane16 = lane & 15;
  const int64_t G = (K + kGroup - 1) / kGroup;
  for (int64_t g = lane >> 4; g < G; g += 4) {
    const int64_t k0 = g * kGroup + lane16 * 8;
    float t[8];
    uint16_t yb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (k0 + i < K) {
        float xv = bf16_at(xr + k0 + i);
        if constexpr (RESIDUAL) xv = round_bf16(xv + bf16_at(rr + k0 + i));
        const float normed = round_bf16(xv * inv);
        yb[i] = f32_to_bf16_bits(bf16_at(weight + k0 + i) * normed);
      } else {
        yb[i] = 0;
      }
      t[i] = __uint_as_float(static_cast<uint32_t>(yb[i]) << 16);
    }
    uint32_t packed[2];
    const float scale = quant_group16(t, packed);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (k0 + i < kpad) q[m * ldq + k0 + i] = static_cast<uint8_t>(packed[i >> 2] >> (8 * (i & 3)));
      if (y_out != nullptr && k0 + i < K) y_out[m * ldy + k0 + i] = yb[i];
    }
    if (lane16 == 0) s[m * ssm + g * ssk] = scale;
  }
}

}  // namespace

int rmsnorm_block_width(int64_t rows, int64_t K) {
  // PyTorch's setReduceConfig for an fp32 last-dim reduction over 4-wide vectors (the
  // reference's _torch_reduce_block_width, fused.py:205-214).
  constexpr int64_t kMaxThreads = 512, kWarp = 32;
  auto last_pow2 = [](int64_t n) {
    int64_t p = 1;
    while (p * 2 <= n) p *= 2;
    return p;
  };
  const int64_t dim0 = K / 4;
  const int64_t dim0_pow2 = dim0 < kMaxThreads ? last_pow2(dim0) : kMaxThreads;
  const int64_t dim1_pow2 = rows < kMaxThreads ? last_pow2(rows > 0 ? rows : 1) : kMaxThreads;
  const int64_t height = dim1_pow2 < kMaxThreads / (dim0_pow2 < kWarp ? dim0_pow2 : kWarp)
                             ? dim1_pow2
                             : kMaxThreads / (dim0_pow2 < kWarp ? dim0_pow2 : kWarp);
  const int64_t bw = dim0_pow2 < kMaxThreads / height ? dim0_pow2 : kMaxThreads / height;
  return static_cast<int>(bw);
}

int launch_rmsnorm_quant(const uint16_t* x, int64_t sxm, const uint16_t* res, int64_t ldr, uint16_t* res_out,
                         int64_t ldro, const uint16_t* weight, float eps, int64_t M, int64_t K, uint16_t* y,
                         int64_t ldy, uint8_t* q, int64_t ldq, int64_t kpad, float* s, int64_t ssm, int64_t ssk,
                         hipStream_t stream) {
  if (M == 0) return MI355X_FP8_OK;
  const int64_t blocks = (M + kRnqRows - 1) / kRnqRows;
  if (blocks > 0x7fffffffLL) return MI355X_FP8_ERR_UNSUPPORTED;
  const int bw = rmsnorm_block_width(M, K);
  const float inv_k = 1.0f / static_cast<float>(K);
  const dim3 grid(static_cast<unsigned>(blocks));
  if (res != nullptr)
    rmsnorm_quant_kernel<true><<<grid, kRnqThreads, 0, stream>>>(x, sxm, res, ldr, res_out, ldro, weight, eps, inv_k,
                                                                 M, K, bw, y, ldy, q, ldq, kpad, s, ssm, ssk);
  else
    rmsnorm_quant_kernel<false><<<grid, kRnqThreads, 0, stream>>>(x, sxm, res, ldr, res_out, ldro, weight, eps,
                                                                  inv_k, M, K, bw, y, ldy, q, ldq, kpad, s, ssm, ssk);
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

}  // namespace mi355x
