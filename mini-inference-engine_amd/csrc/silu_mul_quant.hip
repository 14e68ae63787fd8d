// Fused SiLU(gate) * up  ->  per-token 1x128 FP8 quantization, for the MLP's down_proj.
//
// Elementwise semantics follow the reference's _silu_mul_kernel
// (engine/kernels/fused.py:127-137, PyTorch's bf16 silu-mul):
//   silu = bf16( g / (1 + exp(-g)) )      fp32 math, IEEE division
//   h    = bf16( silu * u )               fp32 product of two bf16 values
// and the quantizer is exactly act_quant.hip's (engine/kernels/sm89_fp8.py:304-332) applied
// to h.  exp() is ROCm's expf (faithfully rounded); the reference's CUDA exp may differ in
// the last place, which can move h by one bf16 ulp: the quantized codes and scales are
// bit-exact with respect to this kernel's own h, which it can also write out.
//
// Layout: like the quantizer, one 16-lane slice per (row, 128-column group), 8 columns per
// lane (16-byte loads of gate and up).  HBM-bound: 4 bytes in (+2 if h is written) and
// 1 byte + scales out per element, instead of a bf16 round trip between two kernels.
#include "fp8_abi_internal.h"
#include "fp8_common.h"

namespace mi355x {
namespace {

constexpr int kSmqThreads = 256;
constexpr int kSmqUnits = kSmqThreads / 16;

template <typename InT>
__global__ __launch_bounds__(kSmqThreads) void silu_mul_quant_kernel(
    const InT* __restrict__ gate, const InT* __restrict__ up, int64_t ld, int64_t M, int64_t I,
    uint16_t* __restrict__ h_out, int64_t ldh, uint8_t* __restrict__ q, int64_t ldq, int64_t kpad,
    float* __restrict__ s, int64_t ssm, int64_t ssk, int64_t G, int vec) {
  const int lane16 = threadIdx.x & 15;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * kSmqUnits + (threadIdx.x >> 4);
  const bool live = unit < M * G;
  const int64_t m = live ? unit / G : 0;
  const int64_t g = live ? unit - m * G : 0;
  const int64_t k0 = g * kGroup + lane16 * 8;

  float gv[8], uv[8];
  if (live && vec && k0 + 8 <= I) {
    const uint4 rg = *reinterpret_cast<const uint4*>(gate + m * ld + k0);
    const uint4 ru = *reinterpret_cast<const uint4*>(up + m * ld + k0);
    const uint32_t wg[4] = {rg.x, rg.y, rg.z, rg.w}, wu[4] = {ru.x, ru.y, ru.z, ru.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      gv[2 * i] = to_f32(InT{static_cast<uint16_t>(wg[i] & 0xffffu)});
      gv[2 * i + 1] = to_f32(InT{static_cast<uint16_t>(wg[i] >> 16)});
      uv[2 * i] = to_f32(InT{static_cast<uint16_t>(wu[i] & 0xffffu)});
      uv[2 * i + 1] = to_f32(InT{static_cast<uint16_t>(wu[i] >> 16)});
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool in = live && k0 + i < I;
      gv[i] = in ? to_f32(gate[m * ld + k0 + i]) : 0.0f;
      uv[i] = in ? to_f32(up[m * ld + k0 + i]) : 0.0f;
    }
  }

  float t[8];
  uint16_t hb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float silu = round_bf16(gv[i] / (1.0f + expf(-gv[i])));
    hb[i] = f32_to_bf16_bits(silu * uv[i]);
    t[i] = __uint_as_float(static_cast<uint32_t>(hb[i]) << 16);
  }
  uint32_t packed[2];
  const float scale = quant_group16(t, packed);
  if (!live) return;
  if (vec && k0 + 8 <= kpad) {
    *reinterpret_cast<uint2*>(q + m * ldq + k0) = make_uint2(packed[0], packed[1]);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (k0 + i < kpad) q[m * ldq + k0 + i] = static_cast<uint8_t>(packed[i >> 2] >> (8 * (i & 3)));
  }
  if (h_out) {
    if (vec && k0 + 8 <= I) {
      *reinterpret_cast<uint4*>(h_out + m * ldh + k0) =
          make_uint4(hb[0] | (static_cast<uint32_t>(hb[1]) << 16), hb[2] | (static_cast<uint32_t>(hb[3]) << 16),
                     hb[4] | (static_cast<uint32_t>(hb[5]) << 16), hb[6] | (static_cast<uint32_t>(hb[7]) << 16));
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (k0 + i < I) h_out[m * ldh + k0 + i] = hb[i];
    }
  }
  if (lane16 == 0) s[m * ssm + g * ssk] = scale;
}

}  // namespace

int launch_silu_mul_quant(const void* gate, const void* up, int dtype, int64_t ld, int64_t M, int64_t I,
                          uint16_t* h_out, int64_t ldh, uint8_t* q, int64_t ldq, int64_t kpad, float* s,
                          int64_t ssm, int64_t ssk, hipStream_t stream) {
  const int64_t G = (I + kGroup - 1) / kGroup;
  const int64_t units = M * G;
  if (units == 0) return MI355X_FP8_OK;
  const int64_t blocks = (units + kSmqUnits - 1) / kSmqUnits;
  if (blocks > 0x7fffffffLL) return MI355X_FP8_ERR_UNSUPPORTED;
  const int vec = (ld % 8) == 0 && (reinterpret_cast<uintptr_t>(gate) % 16) == 0 &&
                  (reinterpret_cast<uintptr_t>(up) % 16) == 0 && (ldq % 8) == 0 &&
                  (reinterpret_cast<uintptr_t>(q) % 8) == 0 &&
                  (h_out == nullptr || ((ldh % 8) == 0 && (reinterpret_cast<uintptr_t>(h_out) % 16) == 0));
  // bf16 only: the reference's fused silu_mul rounds to bf16 (fused.py:135-137).
  if (dtype != kBF16) return MI355X_FP8_ERR_UNSUPPORTED;
  dim3 grid(static_cast<unsigned>(blocks));
  silu_mul_quant_kernel<bf16_t><<<grid, kSmqThreads, 0, stream>>>(
      static_cast<const bf16_t*>(gate), static_cast<const bf16_t*>(up), ld, M, I, h_out, ldh, q, ldq, kpad, s, ssm,
      ssk, G, vec);
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

}  // namespace mi355x
