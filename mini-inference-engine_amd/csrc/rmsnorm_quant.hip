// Fused RMSNorm (optionally after the residual add) -> per-token 1x128 FP8 quantization,
// the input of the q/k/v and gate/up projections.
//
// Semantics follow the reference's _rms_norm_kernel / rms_norm
// (engine/kernels/fused.py:89-124, 165-199), with its quantizer
// (engine/kernels/sm89_fp8.py:304-332) applied to the result:
//   x    = bf16(x + residual)           residual variant (fp32 add, one rounding; also stored)
//   ss   = sum of rounded squares x*x  in PyTorch's reduction order (below)
//   var  = ss * fl(1 / K)              a separate rounding (no fused multiply-add: __fmul_rn and
//                                      __fadd_rn are plain operators in HIP, so the library is
//                                      built with -ffp-contract=off; fused, var + eps came out
//                                      one rounding short and moved y by one ulp near ties)
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
// Layout: a workgroup of 4 waves holds 4 / wpr rows, each row spread over wpr waves (4 for
// up to 256 rows, 2 up to 512, else 1; the reduction order does not depend on wpr).  The
// norm weight and the rows are read once into LDS (rows up to 16128 wide).  Virtual thread
// t of the reduction lives in lane t % 64 of the row's wave (t / 64) % wpr, so folds with
// h >= 64 wpr stay inside a lane, folds between 64 and 64 wpr go through LDS, and the rest
// are shuffles.  The second pass normalizes and quantizes one 128-wide group per 16-lane
// slice, 8 elements per lane.
// HBM traffic per row: 2K bytes in (4K with the residual), K + 4K/128 out (+2K for the
// residual sum).
#include "fp8_abi_internal.h"
#include "fp8_common.h"

namespace mi355x {
namespace {

constexpr int kRnqWavesPerBlock = 4;
constexpr int kRnqBatch = 8;                // 16-byte loads in flight per lane
constexpr int64_t kRnqLdsBytes = 64 * 1024;  // weight, row buffers and fold buffer of one workgroup

extern __shared__ uint16_t rnq_lds[];  // [K] norm weight, then [rows per block][K] rows after the residual add

__device__ __forceinline__ float bf16_val(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// The norm weight (once per workgroup) and the row (after the residual add) go global ->
// LDS once, 16-byte loads when aligned; both passes then read LDS: pass 1 in the
// reduction's order, pass 2 one 128-wide group per 16-lane slice.  One workgroup barrier
// separates the loads from both passes.
template <bool RESIDUAL>
__global__ __launch_bounds__(64 * kRnqWavesPerBlock) void rmsnorm_quant_kernel(
    const uint16_t* __restrict__ x, int64_t sxm, const uint16_t* __restrict__ res, int64_t ldr,
    uint16_t* __restrict__ res_out, int64_t ldro, const uint16_t* __restrict__ weight, float eps, float inv_k,
    int64_t M, int64_t K, int bw, int rows_per_block, int wpr, int vec, uint16_t* __restrict__ y_out, int64_t ldy,
    uint8_t* __restrict__ q, int64_t ldq, int64_t kpad, float* __restrict__ s, int64_t ssm, int64_t ssk) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int slot = wave / wpr;  // row of this workgroup
  const int sub = wave % wpr;   // this wave's share of the row
  const int rl = sub * 64 + lane;  // lane index within the row's wpr waves
  const int64_t m = static_cast<int64_t>(blockIdx.x) * rows_per_block + slot;
  uint16_t* wlds = rnq_lds;
  uint16_t* row = rnq_lds + (slot + 1) * K;
  float* red = reinterpret_cast<float*>(rnq_lds + (rows_per_block + 1) * K) + slot * 64 * wpr;
  const bool live = m < M;
  const int64_t mr = live ? m : M - 1;  // waves past the last row load a real row, write nothing
  const uint16_t* xr = x + mr * sxm;

  // ---- load: row = bf16(x + residual) into LDS (and residual_out), the norm weight ---
  // A lane's loads of a batch are all issued before any is waited on, and the weight's
  // loads ride along with the first batch, so a row of up to 8 x 64 x 8 elements costs
  // one memory round trip.
  if (vec) {
    const int64_t chunks = K / 8;
    const int stride = 64 * wpr;
    for (int64_t c0 = 0; c0 < chunks; c0 += static_cast<int64_t>(stride) * kRnqBatch) {
      uint4 xv[kRnqBatch], rv[kRnqBatch];
#pragma unroll
      for (int b = 0; b < kRnqBatch; ++b) {
        // Unconditional (clamped into the row) so the loads issue back to back.
        const int64_t c = c0 + rl + stride * b < chunks ? c0 + rl + stride * b : chunks - 1;
        xv[b] = *reinterpret_cast<const uint4*>(xr + 8 * c);
        if constexpr (RESIDUAL) rv[b] = *reinterpret_cast<const uint4*>(res + mr * ldr + 8 * c);
      }
      if (c0 == 0) {
        for (int64_t c = threadIdx.x; c < K / 8; c += blockDim.x)
          *reinterpret_cast<uint4*>(wlds + 8 * c) = *reinterpret_cast<const uint4*>(weight + 8 * c);
      }
#pragma unroll
      for (int b = 0; b < kRnqBatch; ++b) {
        const int64_t c = c0 + rl + stride * b;
        if (live && c < chunks) {
          uint4 v = xv[b];
          if constexpr (RESIDUAL) {
            const uint32_t xw[4] = {v.x, v.y, v.z, v.w}, rw[4] = {rv[b].x, rv[b].y, rv[b].z, rv[b].w};
            uint32_t sw[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const uint32_t lo = f32_to_bf16_bits(bf16_val(xw[i] & 0xffffu) + bf16_val(rw[i] & 0xffffu));
              const uint32_t hi = f32_to_bf16_bits(bf16_val(xw[i] >> 16) + bf16_val(rw[i] >> 16));
              sw[i] = lo | (hi << 16);
            }
            v = make_uint4(sw[0], sw[1], sw[2], sw[3]);
            // Non-temporal: the next reader of the residual stream is a later layer, and
            // full-line streaming stores leave no dirty lines for the end-of-kernel
            // write-back (measured 12.6 -> 11.2 us at 2048 rows).
            store16_nt(res_out + m * ldro + 8 * c, v);
          }
          *reinterpret_cast<uint4*>(row + 8 * c) = v;
        }
      }
    }
  } else {
    for (int64_t k = threadIdx.x; k < K; k += blockDim.x) wlds[k] = weight[k];
    if (live) {
      for (int64_t k = rl; k < K; k += 64 * wpr) {
        uint16_t b = xr[k];
        if constexpr (RESIDUAL) {
          b = f32_to_bf16_bits(bf16_val(b) + bf16_val(res[m * ldr + k]));
          res_out[m * ldro + k] = b;
        }
        row[k] = b;
      }
    }
  }
  __syncthreads();  // the weight and the rows are in LDS


  // ---- pass 1: sum of squares in the reference's order ----------------------------
  // Virtual thread t lives in lane t % 64 of wave (t / 64) % wpr, as its slot j = t / (64 wpr).
  // Waves past the last row run it on whatever their LDS holds and discard the result: every
  // wave has to reach the barrier below.
  const int64_t nvec = K / 4;
  const int span = 64 * wpr;  // virtual threads per slot
  float part[8];              // bw <= 512: at most 8 slots per lane
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    part[j] = 0.0f;
    const int t = rl + span * j;
    if (t >= bw) continue;
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t v = t; v < nvec; v += bw) {
      const uint2 pair = *reinterpret_cast<const uint2*>(row + 4 * v);
      const float e[4] = {bf16_val(pair.x & 0xffffu), bf16_val(pair.x >> 16), bf16_val(pair.y & 0xffffu),
                          bf16_val(pair.y >> 16)};
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = __fadd_rn(a[i], __fmul_rn(e[i], e[i]));
    }
    part[j] = __fadd_rn(__fadd_rn(__fadd_rn(a[0], a[1]), a[2]), a[3]);
  }
  // Folds with h >= 64 wpr: slots j and j + h / (64 wpr) of the same lane.
  for (int h = bw / 2; h >= span; h >>= 1) {
    const int hj = h / span;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < hj) part[j] = __fadd_rn(part[j], part[j + hj]);
  }
  // Folds with 64 <= h < 64 wpr: the same lane of waves sub and sub + h / 64, through LDS.
  float ssum = part[0];
  if (wpr > 1) {
    red[rl] = ssum;
    __syncthreads();
    const int nsub = bw >= span ? wpr : (bw >= 64 ? bw / 64 : 1);
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = i < nsub ? red[i * 64 + lane] : 0.0f;
    for (int h = nsub / 2; h >= 1; h >>= 1) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (i < h) v[i] = __fadd_rn(v[i], v[i + h]);
    }
    ssum = v[0];
  }
  if (!live) return;  // no barrier follows
  // Folds with h < 64: lane l adds lane l + h (tree_sum64: lane swaps and DPP; a reduction
  // narrower than a wave keeps the shuffles).
  if (bw >= 64) {
    ssum = tree_sum64(ssum);
  } else {
    for (int h = bw / 2; h >= 1; h >>= 1) {
      const float other = __shfl_down(ssum, h, 64);
      if (lane < h) ssum = __fadd_rn(ssum, other);
    }
    ssum = __shfl(ssum, 0, 64);
  }
  const float var = __fmul_rn(ssum, inv_k);
  const float inv = static_cast<float>(1.0 / sqrt(static_cast<double>(__fadd_rn(var, eps))));

  // ---- pass 2: normalize and quantize, one group per 16-lane slice -----------------
  const int lane16 = lane & 15;
  const int64_t G = (K + kGroup - 1) / kGroup;
  for (int64_t g = (rl >> 4); g < G; g += 4 * wpr) {
    const int64_t k0 = g * kGroup + lane16 * 8;
    float t[8];
    uint16_t yb[8];
    if (vec && k0 + 8 <= K) {
      const uint4 rv = *reinterpret_cast<const uint4*>(row + k0), wv = *reinterpret_cast<const uint4*>(wlds + k0);
      const uint32_t rw[4] = {rv.x, rv.y, rv.z, rv.w}, ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint16_t rb = static_cast<uint16_t>(rw[i >> 1] >> (16 * (i & 1)));
        const uint16_t wb = static_cast<uint16_t>(ww[i >> 1] >> (16 * (i & 1)));
        yb[i] = f32_to_bf16_bits(bf16_val(wb) * round_bf16(bf16_val(rb) * inv));
        t[i] = bf16_val(yb[i]);
      }
    } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (k0 + i < K) {
        const float normed = round_bf16(bf16_val(row[k0 + i]) * inv);
        yb[i] = f32_to_bf16_bits(bf16_val(wlds[k0 + i]) * normed);
      } else {
        yb[i] = 0;
      }
      t[i] = bf16_val(yb[i]);
    }
    }
    uint32_t packed[2];
    const float scale = quant_group16(t, packed);
    if (vec && k0 + 8 <= kpad) {
      *reinterpret_cast<uint2*>(q + m * ldq + k0) = make_uint2(packed[0], packed[1]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (k0 + i < kpad) q[m * ldq + k0 + i] = static_cast<uint8_t>(packed[i >> 2] >> (8 * (i & 3)));
    }
    if (y_out != nullptr) {
      if (vec && ldy % 8 == 0 && k0 + 8 <= K) {
        *reinterpret_cast<uint4*>(y_out + m * ldy + k0) =
            make_uint4(yb[0] | (static_cast<uint32_t>(yb[1]) << 16), yb[2] | (static_cast<uint32_t>(yb[3]) << 16),
                       yb[4] | (static_cast<uint32_t>(yb[5]) << 16), yb[6] | (static_cast<uint32_t>(yb[7]) << 16));
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (k0 + i < K) y_out[m * ldy + k0 + i] = yb[i];
      }
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
  const int64_t row_bytes = 2 * K;
  if (2 * row_bytes + 1024 > kRnqLdsBytes) return MI355X_FP8_ERR_UNSUPPORTED;  // K > 16128
  // Waves per row: few rows spread each over several waves (the reduction order does not
  // depend on it), so that more of the chip works on them.
  const int wpr = M <= 256 ? 4 : (M <= 512 ? 2 : 1);
  int rows = static_cast<int>((kRnqLdsBytes - 1024) / row_bytes) - 1;  // the weight and the fold buffer
  rows = rows < kRnqWavesPerBlock / wpr ? rows : kRnqWavesPerBlock / wpr;
  const int64_t blocks = (M + rows - 1) / rows;
  if (blocks > 0x7fffffffLL) return MI355X_FP8_ERR_UNSUPPORTED;
  const auto aligned16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; };
  const int vec = K % 8 == 0 && sxm % 8 == 0 && aligned16(x) && aligned16(weight) && aligned16(y ? y : x) &&
                  (ldq % 8) == 0 && (reinterpret_cast<uintptr_t>(q) % 8) == 0 &&
                  (res == nullptr || (ldr % 8 == 0 && ldro % 8 == 0 && aligned16(res) && aligned16(res_out)));
  const int bw = rmsnorm_block_width(M, K);
  const float inv_k = 1.0f / static_cast<float>(K);
  const dim3 grid(static_cast<unsigned>(blocks));
  const size_t lds = static_cast<size_t>(rows + 1) * row_bytes + static_cast<size_t>(rows) * 64 * wpr * 4;
  if (res != nullptr)
    rmsnorm_quant_kernel<true><<<grid, 64 * rows * wpr, lds, stream>>>(x, sxm, res, ldr, res_out, ldro, weight, eps, inv_k,
                                                                 M, K, bw, rows, wpr, vec, y, ldy, q, ldq, kpad, s, ssm, ssk);
  else
    rmsnorm_quant_kernel<false><<<grid, 64 * rows * wpr, lds, stream>>>(x, sxm, res, ldr, res_out, ldro, weight, eps,
                                                                  inv_k, M, K, bw, rows, wpr, vec, y, ldy, q, ldq, kpad, s,
                                                                  ssm, ssk);
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

}  // namespace mi355x
