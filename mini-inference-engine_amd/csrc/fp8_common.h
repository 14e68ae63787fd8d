// Shared device helpers for the gfx950 FP8 block-scaled linear kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi355x {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kGroup = 128;  // K elements per activation/weight scale group
constexpr int kWave = 64;

// Element type tags shared with the C-ABI (include/mi355x_fp8.h: MI355X_FP8_DTYPE_*).
enum DType : int { kBF16 = 0, kF16 = 1 };

struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float to_f32(bf16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h.bits) << 16);
}
__device__ __forceinline__ float to_f32(f16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h.bits, 2);
  return static_cast<float>(v);
}

// fp32 -> bf16 with round-to-nearest-even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  const __bf16 v = static_cast<__bf16>(f);  // v_cvt_pk_bf16_f32: round to nearest even
  uint16_t b;
  __builtin_memcpy(&b, &v, 2);
  return b;
}
// fp32 -> binary16 with the hardware's round-to-nearest-even conversion.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 v = static_cast<_Float16>(f);
  uint16_t b;
  __builtin_memcpy(&b, &v, 2);
  return b;
}

template <typename T> struct OutCvt;
template <> struct OutCvt<bf16_t> {
  __device__ static uint16_t cvt(float f) { return f32_to_bf16_bits(f); }
};
template <> struct OutCvt<f16_t> {
  __device__ static uint16_t cvt(float f) { return f32_to_f16_bits(f); }
};

// Prefill epilogue through LDS.  Each lane first writes its 4-column pieces of the output
// tile into LDS (row-major, a row of BN halfwords at pitch staged_pitch<BN>()), then every
// row goes out in 16-byte pieces with consecutive lanes on consecutive pieces, as
// non-temporal stores.  Full-line streaming stores leave no dirty output lines in L2 for the
// end-of-kernel write-back, which otherwise runs after the last tile's loop; scattered 8-byte
// stores (non-temporal or not) measured slower.
// A row pitch of BN halfwords when BN is a multiple of 128, with the 16-byte pieces of row r
// XOR-swizzled by r & 15, else BN + 8 halfwords: either way the 16 rows a wave writes at once
// and the 16-byte reads land in distinct banks.
template <int BN>
__device__ constexpr int staged_pitch() {
  return BN % 128 == 0 ? BN : BN + 8;
}
// Halfword index of column col (a multiple of 4) of staged row row.
template <int BN>
__device__ __forceinline__ int staged_index(int row, int col) {
  const int piece = BN % 128 == 0 ? ((col >> 3) ^ (row & 15)) : (col >> 3);
  return row * staged_pitch<BN>() + piece * 8 + (col & 7);
}
__device__ __forceinline__ void store16_nt(uint16_t* dst, uint4 v) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(dst));
}

// fp32 rounded to the nearest bf16 (ties to even), returned as fp32.
__device__ __forceinline__ float round_bf16(float f) {
  return __uint_as_float(static_cast<uint32_t>(f32_to_bf16_bits(f)) << 16);
}

// Two fp32 -> two OCP e4m3fn codes (round-to-nearest-even), packed into the low 16 bits.
__device__ __forceinline__ uint32_t cvt_pk_e4m3(float a, float b) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) & 0xffffu;
}

// t / den, correctly rounded, from r = 1 / den (correctly rounded) by one remainder
// correction: q0 = t r, rem = t - q0 den (exact, fused), q = q0 + rem r, with t's sign
// (which fixes the sign of a zero quotient).  This is the classic reciprocal-based
// division with a final correction (Markstein).  For the quantizer's operands (t a
// bf16/fp16 value with |t| <= amax, den = max(amax / 448, 1e-12), den finite) it has been
// checked exhaustively against IEEE division over every (amax, t) pair of both 16-bit
// formats: equal bits wherever |t / den| >= 2^-12, and below that (where every e4m3 code
// is a zero) the same sign.  Four instructions instead of the ten of a full division.
__device__ __forceinline__ float div_by_scale(float t, float den, float r) {
  const float q0 = t * r;
  const float rem = __builtin_fmaf(-q0, den, t);
  return __builtin_copysignf(__builtin_fmaf(rem, r, q0), t);
}

// Codes of 4 consecutive elements t[0..3] scaled by den (r = 1 / den when den is finite).
template <bool FAST>
__device__ __forceinline__ uint32_t quant4(const float* t, float den, float r) {
  if (FAST)
    return cvt_pk_e4m3(div_by_scale(t[0], den, r), div_by_scale(t[1], den, r)) |
           (cvt_pk_e4m3(div_by_scale(t[2], den, r), div_by_scale(t[3], den, r)) << 16);
  return cvt_pk_e4m3(t[0] / den, t[1] / den) | (cvt_pk_e4m3(t[2] / den, t[3] / den) << 16);
}

// Codes of n consecutive elements (n % 4 == 0) into n / 4 words.  An infinite den (an
// infinity in the group) takes plain IEEE division.
template <int N>
__device__ __forceinline__ void quant_codes(const float* t, float den, uint32_t* packed) {
  if (__builtin_isfinite(den)) {
    const float r = 1.0f / den;
#pragma unroll
    for (int i = 0; i < N / 4; ++i) packed[i] = quant4<true>(t + 4 * i, den, r);
  } else {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) packed[i] = quant4<false>(t + 4 * i, den, 0.0f);
  }
}

// Lane t's value from lane t ^ 16 (row_partner16) or t ^ 32 (row_partner32), through the
// gfx950 lane swaps: with both operands the same register, the swap's second result holds the
// odd rows' (upper half's) values in the even rows (lower half), its first result the reverse.
__device__ __forceinline__ float row_partner16(float x) {
  const auto v = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(((__lane_id() >> 4) & 1) ? v[0] : v[1]);
}
__device__ __forceinline__ float row_partner32(float x) {
  const auto v = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(((__lane_id() >> 5) & 1) ? v[0] : v[1]);
}

// The halving tree s[t] += s[t + h], h = 32, 16, ..., 1, over the 64 lanes, with lane-to-lane
// VALU moves instead of LDS shuffles: v_permlane32_swap and v_permlane16_swap bring lanes
// t + 32 and t + 16 to lanes t, DPP row_shl:h brings t + h within each 16-lane row.  Lane t < h
// adds lane t + h's value at every step, so lane 0 ends with the tree's sum, which goes to
// every lane.
__device__ __forceinline__ float tree_sum64(float s) {
  s = s + __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false)[1]);
  s = s + __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false)[1]);
  s = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x108, 0xf, 0xf, true));  // row_shl:8
  s = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x104, 0xf, 0xf, true));  // row_shl:4
  s = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x102, 0xf, 0xf, true));  // row_shl:2
  s = s + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x101, 0xf, 0xf, true));  // row_shl:1
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
}

// The maximum over each aligned group of L consecutive lanes (L a power of two), in every lane
// of the group: quad permutes, then the half-row and row mirrors (each lane meets a lane of the
// other half, already reduced), then the 16- and 32-lane swaps.  A maximum does not depend on
// the pairing, so this equals any other reduction order.
template <int L>
__device__ __forceinline__ float group_max(float x) {
  const auto dpp = [](float v, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  if constexpr (L >= 2) x = fmaxf(x, dpp(x, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
  if constexpr (L >= 4) x = fmaxf(x, dpp(x, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
  if constexpr (L >= 8) x = fmaxf(x, dpp(x, std::integral_constant<int, 0x141>{}));  // row_half_mirror
  if constexpr (L >= 16) x = fmaxf(x, dpp(x, std::integral_constant<int, 0x140>{})); // row_mirror
  if constexpr (L >= 32) x = fmaxf(x, row_partner16(x));
  if constexpr (L >= 64) x = fmaxf(x, row_partner32(x));
  return x;
}

// The maximum over the four lanes r, r + 16, r + 32, r + 48 (each 16-lane row's lane r).
__device__ __forceinline__ float row_max(float x) {
  x = fmaxf(x, row_partner16(x));
  return fmaxf(x, row_partner32(x));
}

// The quantizer of one 128-wide group held by a 16-lane slice, 8 consecutive elements per
// lane (reference engine/kernels/sm89_fp8.py:321-324): scale = amax / 448 (IEEE division,
// stored raw), codes = e4m3fn(t / max(scale, 1e-12)), round-to-nearest-even, saturating.
// Returns the scale (the same in all 16 lanes); packed[0..1] receive this lane's 8 codes.
// The division by the scale goes through div_by_scale (same bits).
__device__ __forceinline__ float quant_group16(const float (&t)[8], uint32_t (&packed)[2]) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(t[i]));
  amax = group_max<16>(amax);
  const float scale = amax / 448.0f;
  const float den = scale > 1e-12f ? scale : 1e-12f;
  quant_codes<8>(t, den, packed);
  return scale;
}

// D(16x16, fp32) = A(16 x 128 e4m3) * B(128 x 16 e4m3), accumulator input zero.
// Lane l supplies row (l % 16) of A and column (l % 16) of B; both operands place the
// same 32 K-bytes in lane group l / 16, so the 128-long dot is complete in one
// instruction.  Lane l receives D[4 * (l / 16) + v][l % 16] in element v.
__device__ __forceinline__ v4f mfma_16x16x128_e4m3(v8i a, v8i b) {
  v4f zero = {0.f, 0.f, 0.f, 0.f};
  // cbsz = blgp = 0 selects e4m3 for both operands; zero scales select the unscaled form.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, zero, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ v8i pack_v8i(uint4 lo, uint4 hi) {
  v8i r;
  r[0] = static_cast<int>(lo.x); r[1] = static_cast<int>(lo.y);
  r[2] = static_cast<int>(lo.z); r[3] = static_cast<int>(lo.w);
  r[4] = static_cast<int>(hi.x); r[5] = static_cast<int>(hi.y);
  r[6] = static_cast<int>(hi.z); r[7] = static_cast<int>(hi.w);
  return r;
}

// Loads 16 bytes of row `row` starting at column `k` of a byte matrix (row stride ld).
// Bytes outside [0, rows) x [0, K) read as zero (e4m3 +0).  ALIGNED means K, ld and the
// base pointer are multiples of 16, so a chunk is either fully inside K or fully outside
// and one 16-byte load serves it; otherwise the chunk is assembled from byte loads.
template <bool ALIGNED>
__device__ __forceinline__ uint4 load_chunk16(const uint8_t* __restrict__ base, int64_t ld,
                                              int64_t row, int64_t rows, int64_t k, int64_t K) {
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (ALIGNED) {
    if (row < rows && k < K) v = *reinterpret_cast<const uint4*>(base + row * ld + k);
    return v;
  }
  if (row >= rows) return v;
  const uint8_t* p = base + row * ld + k;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (k + i < K) w[i >> 2] |= static_cast<uint32_t>(p[i]) << (8 * (i & 3));
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

}  // namespace mi355x
