// Kernel (a): per-token 1x128 dynamic activation quantizer for gfx950.
//
// Semantics follow the reference's _quantize_activation_kernel
// (engine/kernels/sm89_fp8.py:304-332):
//   t = x[m, 128g : 128g+128] as fp32, K tail read as 0.0
//   s = max(|t|) / 448.0          -- stored raw (0 for an all-zero group)
//   q = e4m3fn(t / max(s, 1e-12)) -- IEEE round-to-nearest division, RNE conversion
//
// Layout: one 16-lane slice of a wave owns one (row, group) unit; each lane holds 8
// consecutive elements (one 16-byte bf16/fp16 load), so a 256-thread block covers 16
// units.  The group amax is a 4-step butterfly inside the 16-lane slice.  The kernel is
// HBM-bound: it moves 2 (x) + 1 (q) bytes per element plus 4 bytes per group.
#include "fp8_abi_internal.h"
#include "fp8_common.h"

namespace mi355x {

constexpr int kQuantThreads = 256;
constexpr int kUnitsPerBlock = kQuantThreads / 16;

template <typename InT>
__global__ __launch_bounds__(kQuantThreads) void act_quant_kernel(
    const InT* __restrict__ x, int64_t M, int64_t K, int64_t sxm, int64_t sxk,
    uint8_t* __restrict__ q, int64_t ldq, int64_t kpad, float* __restrict__ s, int64_t ssm,
    int64_t ssk, int64_t G, int vec_in, int vec_out) {
  const int lane16 = threadIdx.x & 15;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * kUnitsPerBlock + (threadIdx.x >> 4);
  const bool live = unit < M * G;
  const int64_t m = live ? unit / G : 0;
  const int64_t g = live ? unit - m * G : 0;
  const int64_t k0 = g * kGroup + lane16 * 8;

  float t[8];
  if (live && vec_in && k0 + 8 <= K) {
    const uint4 raw = *reinterpret_cast<const uint4*>(x + m * sxm + k0);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      t[2 * i] = to_f32(InT{static_cast<uint16_t>(w[i] & 0xffffu)});
      t[2 * i + 1] = to_f32(InT{static_cast<uint16_t>(w[i] >> 16)});
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = (live && k0 + i < K) ? to_f32(x[m * sxm + (k0 + i) * sxk]) : 0.0f;
  }

  uint32_t packed[2];
  const float scale = quant_group16(t, packed);
  if (!live) return;
  if (vec_out && k0 + 8 <= kpad) {
    *reinterpret_cast<uint2*>(q + m * ldq + k0) = make_uint2(packed[0], packed[1]);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (k0 + i < kpad) q[m * ldq + k0 + i] = static_cast<uint8_t>(packed[i >> 2] >> (8 * (i & 3)));
    }
  }
  if (lane16 == 0) s[m * ssm + g * ssk] = scale;
}

// The same quantizer with 16 elements per lane (two 16-byte loads in flight, one 16-byte code
// store), one (row, group) unit per 8-lane slice, 32 units per block: for contiguous rows
// (16-byte aligned, K % 16 == 0) and 16-byte aligned code rows.  The per-element arithmetic
// is quant_group16's (amax, scale = amax / 448, quant_codes), the amax a maximum over the
// slice (order-free), so the codes and scales are the same bits.
constexpr int kWideE = 16;  // elements per lane (32 measured no faster)

template <typename InT, int E>
__global__ __launch_bounds__(kQuantThreads) void act_quant_wide_kernel(
    const InT* __restrict__ x, int64_t M, int64_t K, int64_t sxm, uint8_t* __restrict__ q, int64_t ldq,
    float* __restrict__ s, int64_t ssm, int64_t ssk, int64_t G) {
  constexpr int L = kGroup / E;  // lanes per unit
  const int lane8 = threadIdx.x & (L - 1);
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * (kQuantThreads / L) + (threadIdx.x / L);
  const bool live = unit < M * G;
  const int64_t m = live ? unit / G : 0;
  const int64_t g = live ? unit - m * G : 0;
  const int64_t k0 = g * kGroup + lane8 * E;

  float t[E];
  if (live && k0 < K) {
    const uint4* p = reinterpret_cast<const uint4*>(x + m * sxm + k0);
    uint4 r[E / 8];
#pragma unroll
    for (int c = 0; c < E / 8; ++c) r[c] = p[c];
#pragma unroll
    for (int c = 0; c < E / 8; ++c) {
      const uint32_t w[4] = {r[c].x, r[c].y, r[c].z, r[c].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        t[8 * c + 2 * i] = to_f32(InT{static_cast<uint16_t>(w[i] & 0xffffu)});
        t[8 * c + 2 * i + 1] = to_f32(InT{static_cast<uint16_t>(w[i] >> 16)});
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) t[i] = 0.0f;
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < E; ++i) amax = fmaxf(amax, fabsf(t[i]));
  amax = group_max<L>(amax);
  const float scale = amax / 448.0f;
  const float den = scale > 1e-12f ? scale : 1e-12f;
  uint32_t packed[E / 4];
  quant_codes<E>(t, den, packed);
  if (!live) return;
#pragma unroll
  for (int c = 0; c < E / 16; ++c)
    *reinterpret_cast<uint4*>(q + m * ldq + k0 + 16 * c) =
        make_uint4(packed[4 * c], packed[4 * c + 1], packed[4 * c + 2], packed[4 * c + 3]);
  if (lane8 == 0) s[m * ssm + g * ssk] = scale;
}

int launch_act_quant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm, int64_t sxk,
                     uint8_t* q, int64_t ldq, int64_t kpad, float* s, int64_t ssm, int64_t ssk,
                     hipStream_t stream) {
  const int64_t G = (K + kGroup - 1) / kGroup;
  const int64_t units = M * G;
  if (units == 0) return MI355X_FP8_OK;
  const int64_t blocks = (units + kUnitsPerBlock - 1) / kUnitsPerBlock;
  if (blocks > 0x7fffffffLL) return MI355X_FP8_ERR_UNSUPPORTED;
  const int vec_in = sxk == 1 && (sxm % 8) == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0;
  const int vec_out = (ldq % 8) == 0 && (reinterpret_cast<uintptr_t>(q) % 8) == 0;
  if (vec_in && K % kWideE == 0 && ldq % 16 == 0 && (reinterpret_cast<uintptr_t>(q) % 16) == 0 && kpad == G * kGroup) {
    constexpr int64_t kUnits = kQuantThreads / (kGroup / kWideE);
    const int64_t wide_blocks = (units + kUnits - 1) / kUnits;
    if (x_dtype == kBF16)
      act_quant_wide_kernel<bf16_t, kWideE><<<dim3(static_cast<unsigned>(wide_blocks)), dim3(kQuantThreads), 0, stream>>>(
          static_cast<const bf16_t*>(x), M, K, sxm, q, ldq, s, ssm, ssk, G);
    else
      act_quant_wide_kernel<f16_t, kWideE><<<dim3(static_cast<unsigned>(wide_blocks)), dim3(kQuantThreads), 0, stream>>>(
          static_cast<const f16_t*>(x), M, K, sxm, q, ldq, s, ssm, ssk, G);
    return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
  }
  if (x_dtype == kBF16) {
    act_quant_kernel<bf16_t><<<dim3(static_cast<unsigned>(blocks)), dim3(kQuantThreads), 0, stream>>>(
        static_cast<const bf16_t*>(x), M, K, sxm, sxk, q, ldq, kpad, s, ssm, ssk, G, vec_in, vec_out);
  } else {
    act_quant_kernel<f16_t><<<dim3(static_cast<unsigned>(blocks)), dim3(kQuantThreads), 0, stream>>>(
        static_cast<const f16_t*>(x), M, K, sxm, sxk, q, ldq, kpad, s, ssm, ssk, G, vec_in, vec_out);
  }
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

}  // namespace mi355x
