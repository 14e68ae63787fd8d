// Kernel (b): block-scaled FP8 GEMM on CDNA4 MFMA (v_mfma_f32_16x16x128_f8f6f4, e4m3).
//
// Semantics follow the reference's _fp8_split_gemm_kernel
// (engine/kernels/sm89_fp8.py:344-398): for every 128-wide K group kb,
//   acc += dot(q[m, kb], W[n, kb]) * a_s[m, kb] * w_s[n / 128, kb]   (fp32)
// then out = acc rounded to bf16/fp16.  One 16x16x128 MFMA consumes exactly one K
// group, so each instruction's fp32 result is the per-group partial sum; it is folded into
// the fp32 accumulator as acc = fma(partial, a_s * w_s, acc).  (The reference multiplies
// by the two scales one after the other; the fused form differs only in fp32 rounding and
// is held to the output tolerance stated in the tests.)
//
// Both operands of the MFMA carry the same K permutation: lane group g = lane / 16 holds
// the 16-byte chunks g and g + 4 of the 128-byte K group.  The permutation is the same for
// A and B, so the dot product is unchanged, and every load instruction reads whole 64-byte
// row halves.
//
// Kernels here:
//   stream_gemm_kernel  decode-sized M (16 or 32 tokens per slice).  HBM-bound weight
//   (+ rounds variant)  streaming: each workgroup owns up to 80 W rows over the whole of K
//                       (the same number on every CU where that fits), W goes global ->
//                       registers (read once per slice, one or two K groups in flight per
//                       wave), the small activation matrix is served from L2 (or quantized
//                       in the kernel, for the one-launch linear); the K groups' MFMA
//                       partials meet in LDS and are folded in K order, so the bits equal
//                       the prefill kernels'.  No workspace, no cross-workgroup
//                       synchronisation.
//   tile_gemm_kernel    prefill-sized M.  MFMA-bound: 128x128 output tile per 256-thread
//                       workgroup, 2x2 waves of 64x64, K groups staged global -> registers
//                       -> LDS with double buffering and an XOR-swizzled (conflict-free)
//                       layout; XCD-aware, grouped tile order for L2 reuse.
#include "fp8_abi_internal.h"
#include "fp8_common.h"

#include <type_traits>

namespace mi355x {

constexpr int kThreads = 256;  // tile kernel

// ------------------------------------------------------------------------------------
// Stream kernel (decode M)
// ------------------------------------------------------------------------------------
// One workgroup owns up to 16*AF consecutive W rows and reads them over the whole of K
// exactly once.  Its 16 waves take K groups round-robin (wave w: w, w + 16, ...) with the next one
// or two groups' loads in flight, and compute each group's MFMA partial; the partials then
// meet in LDS, where one thread per output element folds them in K order (below).  16
// waves per workgroup measured best on the Qwen3-4B shapes.
constexpr int kStreamWaves = 16;
// One-round partial buffer limit: two workgroups of 1024 threads share a CU's 160 KiB.
constexpr size_t kStreamFoldLds = 80 * 1024;
// With at most one workgroup per CU (the ragged row counts) the buffer may take most of the LDS.
constexpr size_t kStreamFoldLdsOne = 144 * 1024;
constexpr int64_t kStreamMinRows = 8;

// LDS of the one-round fold: the raw partials [KB][tokens][16 af] and, per K group and token,
// the scale products with the `blocks` (one, two for ragged row counts, four for the paired
// gate/up rows) 128-row weight-scale blocks a workgroup's rows touch.  tokens = tok_slots when
// given (the norm forms keep 8), else the slice's 16 nt.
__host__ __device__ constexpr size_t stream_fold_bytes(int64_t kb, int af, int nt, int blocks = 1, int tok_slots = 0) {
  return static_cast<size_t>(kb) *
         (static_cast<size_t>(af) * 16 * (tok_slots ? tok_slots : 16 * nt) + blocks * (tok_slots ? tok_slots : 16 * nt)) *
         sizeof(float);
}

// The fold: the waves publish each K group's raw MFMA partials and the scale products
// a_s * w_s in LDS, and one thread per output element folds acc = fma(partial, a_s * w_s,
// acc) over the K groups in increasing order -- the fold of every prefill kernel, on
// bit-identical MFMA partials (same operands, same K order within the instruction).  A
// row's bits are then the same for every M and every kernel, so the dispatch may pick any
// kernel for any shape.
//
// stream_rounds_kernel: for when the partials of all K groups do not fit in LDS at once.
// It works in rounds of kStreamWaves consecutive groups (one per wave), each published,
// folded and followed by the next; the next round's loads are issued before the publish
// and fold, so they overlap them.
template <int NT, int AF, bool ALIGNED, typename OutT>
__global__ __launch_bounds__(kStreamWaves * 64) void stream_rounds_kernel(
    const uint8_t* __restrict__ q, int64_t ldq, const float* __restrict__ as, int64_t as_sm,
    int64_t as_sk, const uint8_t* __restrict__ w, int64_t ldw, const float* __restrict__ ws,
    int64_t ws_sn, int64_t ws_sk, uint16_t* __restrict__ out, int64_t ldo, int64_t M, int64_t N,
    int64_t K, int64_t KB) {
  static_assert(8 % AF == 0, "a workgroup's rows lie in one weight-scale block");
  constexpr int kRows = 16 * AF;  // W rows of this workgroup
  constexpr int kTok = 16 * NT;   // token rows of this slice
  constexpr int kBufs = AF * NT >= 4 ? 1 : 2;  // double-buffered publish when it fits
  constexpr int kTiles = AF * NT;
  __shared__ float4 part[kBufs][kStreamWaves][kTiles][64];  // raw partials, lane layout
  __shared__ float scl[kBufs][kStreamWaves][kTok];          // a_s * w_s per token

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kRows;
  const int64_t m_base = static_cast<int64_t>(blockIdx.z) * kTok;
  const int64_t m_rows = (M - m_base) < kTok ? (M - m_base) : kTok;
  const int64_t nb = n0 / kGroup;
  const int64_t wave_u = __builtin_amdgcn_readfirstlane(wave);

  // This thread's output element in the fold (threads past the tile's elements only help
  // compute partials).
  const int e = tid;
  const bool folder = e < kRows * kTok;
  const int ftok = e / kRows, fnl = e - (e / kRows) * kRows;
  const int fi = fnl >> 4, fj = ftok >> 4;
  const int flane = (ftok & 15) + 16 * ((fnl & 15) >> 2), fv = fnl & 3;
  float acc = 0.0f;

  v8i a[AF], b[NT];
  float asv[NT], wsv;
  auto load = [&](int64_t kb) {  // kb < KB (callers skip groups past the end)
    const int64_t kbc = kb;
    const int64_t k_lo = kbc * kGroup + 16 * g;
#pragma unroll
    for (int i = 0; i < AF; ++i) {
      const int64_t row = n0 + 16 * i + r;
      a[i] = pack_v8i(load_chunk16<ALIGNED>(w, ldw, row, N, k_lo, K), load_chunk16<ALIGNED>(w, ldw, row, N, k_lo + 64, K));
    }
    wsv = ws[nb * ws_sn + kbc * ws_sk];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int64_t tok = 16 * j + r;
      const int64_t m = m_base + tok;
      b[j] = pack_v8i(load_chunk16<ALIGNED>(q, ldq, m, M, k_lo, K), load_chunk16<ALIGNED>(q, ldq, m, M, k_lo + 64, K));
      asv[j] = tok < m_rows ? as[m * as_sm + kbc * as_sk] : 0.0f;
    }
  };

  if (wave_u < KB) load(wave_u);
  int buf = 0;
  for (int64_t t0 = 0; t0 < KB; t0 += kStreamWaves) {
    const bool have = t0 + wave_u < KB;  // wave-uniform
    const bool next = t0 + kStreamWaves + wave_u < KB;
    v4f p[AF][NT];
    if (have) {
#pragma unroll
      for (int i = 0; i < AF; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) p[i][j] = mfma_16x16x128_e4m3(a[i], b[j]);
    }
    float sc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) sc[j] = asv[j] * wsv;
    // The next round's group, in flight during the publish and fold (unaligned shapes,
    // whose loads are assembled from bytes, load after the fold to stay within registers).
    if constexpr (ALIGNED) {
      if (next) load(t0 + kStreamWaves + wave_u);
    }
    if constexpr (kBufs == 1) __syncthreads();  // the previous fold has read the buffer
    if (have) {
#pragma unroll
      for (int i = 0; i < AF; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          part[buf][wave][i * NT + j][lane] = make_float4(p[i][j][0], p[i][j][1], p[i][j][2], p[i][j][3]);
      if (g == 0) {
#pragma unroll
        for (int j = 0; j < NT; ++j) scl[buf][wave][16 * j + r] = sc[j];
      }
    }
    __syncthreads();
    if (folder) {
      const int64_t nk = KB - t0 < kStreamWaves ? KB - t0 : kStreamWaves;
      for (int x = 0; x < nk; ++x) {
        const float* pv = reinterpret_cast<const float*>(&part[buf][x][fi * NT + fj][flane]);
        acc = __builtin_fmaf(pv[fv], scl[buf][x][ftok], acc);
      }
    }
    if constexpr (!ALIGNED) {
      if (next) load(t0 + kStreamWaves + wave_u);
    }
    if constexpr (kBufs == 2) buf ^= 1;
  }
  if (folder && ftok < m_rows && n0 + fnl < N) out[(m_base + ftok) * ldo + n0 + fnl] = OutCvt<OutT>::cvt(acc);
}

// stream_gemm_kernel: the same arithmetic in one round, when every K group's partials fit
// in LDS at once (dynamic LDS): each wave walks its K groups (w, w + 16, ...) with the
// next group's loads in flight, publishes every partial, and after a single barrier one
// thread per output element folds the whole K chain in order.
//
// RAGGED: a workgroup owns `rows` consecutive W rows (at most 16 AF; the MFMA tiles' rows
// past them read as zero and are never stored), so the dispatch can give every CU the same
// number of rows (a CU keeps only so many loads in flight, and the rows it streams set the
// time).  The rows may then cross a 128-row weight-scale block: each K group publishes the
// scale products with both blocks the rows touch, and the fold takes its row's.  Otherwise
// a workgroup owns exactly 16 AF rows with 8 % AF == 0, inside one block.
extern __shared__ float4 stream_fold_lds[];

// The RMSNorm in front of a one-launch decode linear (stream_gemm_kernel with NORM): x is
// the norm's input, `res` the residual added to it first (or null), `sum` receives
// bf16(x + res) (or null), `w` is the norm weight; bw is the reduction's block width
// (rmsnorm_block_width).
struct NormArgs {
  const uint16_t* res = nullptr;
  int64_t ldr = 0;
  uint16_t* sum = nullptr;
  int64_t lds = 0;
  const uint16_t* w = nullptr;
  float eps = 0.0f;
  float inv_k = 0.0f;
  int bw = 0;
};
constexpr size_t kNormLds = 160 * 1024;  // a CU's whole LDS (one workgroup per CU)
constexpr int kNormMaxVec = 10;  // vectors of 4 elements per lane: K <= 2560 (the registers it holds)

__device__ __forceinline__ float bf16_bits_val(uint32_t b) { return __uint_as_float((b & 0xffffu) << 16); }
__device__ __forceinline__ uint32_t bf16_add_pair(uint32_t x, uint32_t r) {
  return f32_to_bf16_bits(bf16_bits_val(x) + bf16_bits_val(r)) |
         (static_cast<uint32_t>(f32_to_bf16_bits(bf16_bits_val(x >> 16) + bf16_bits_val(r >> 16))) << 16);
}

// One row's 1 / sqrt(mean(x^2) + eps) in the reference's order (engine/kernels/fused.py:
// 95-116, the tree of fused.py:61-75), the same additions rmsnorm_quant_kernel makes: lane l
// holds vectors v = l + 64 i (i < nv), which are virtual thread t = v mod bw's vectors in
// order; thread t = l + 64 j keeps four accumulators, combined ((a0 + a1) + a2) + a3; the
// partials fold as s[t] += s[t + h] for h = bw/2 .. 64 inside the lane, then .. 1 across lanes.
// xv holds bf16(x + residual) on return.
template <int J>
__device__ __forceinline__ float norm_row_inv(const uint2 (&xv)[kNormMaxVec], int nv, const NormArgs& na) {
  float a[J][4];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) a[j][c] = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormMaxVec; ++i) {
    if (i < nv) {
      const uint32_t w2[2] = {xv[i].x, xv[i].y};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float e = bf16_bits_val(w2[c >> 1] >> (16 * (c & 1)));
        a[i % J][c] = a[i % J][c] + e * e;
      }
    }
  }
  float part[J];
#pragma unroll
  for (int j = 0; j < J; ++j) part[j] = ((a[j][0] + a[j][1]) + a[j][2]) + a[j][3];
#pragma unroll
  for (int hj = J / 2; hj >= 1; hj >>= 1)
#pragma unroll
    for (int j = 0; j < hj; ++j) part[j] = part[j] + part[j + hj];
  const float ss = tree_sum64(part[0]);
  const float var = ss * na.inv_k;
  return static_cast<float>(1.0 / sqrt(static_cast<double>(var + na.eps)));
}

template <int NT, int AF, bool ALIGNED, bool RAGGED, typename OutT, typename XIn = uint8_t, int QT = 16,
          bool NORM = false, bool SILU = false>
__global__ __launch_bounds__(kStreamWaves * 64) void stream_gemm_kernel(
    const uint8_t* __restrict__ q, int64_t ldq, const float* __restrict__ as, int64_t as_sm,
    int64_t as_sk, const uint8_t* __restrict__ w, int64_t ldw, const float* __restrict__ ws,
    int64_t ws_sn, int64_t ws_sk, uint16_t* __restrict__ out, int64_t ldo, int64_t M, int64_t N,
    int64_t K, int64_t KB, int rows_arg, NormArgs na = NormArgs{}) {
  static_assert(RAGGED || 8 % AF == 0, "a workgroup's rows lie in one weight-scale block");
  // XIn = uint8_t: q holds the quantized activations (ldq bytes per row) and as their scales.
  // XIn = bf16_t / f16_t: q holds the unquantized activations (ldq elements per row, 16-byte
  // aligned rows, K % 16 == 0) and each wave quantizes its own K groups in registers, with
  // the quantizer's arithmetic (quant_group16's amax, scale and codes), so the codes and
  // scales, and therefore the output bits, are those of the two-launch path.
  constexpr bool kQuant = !std::is_same<XIn, uint8_t>::value;
  using XT = typename std::conditional<kQuant, XIn, bf16_t>::type;  // element type when quantizing
  static_assert(!kQuant || (ALIGNED && NT == 1), "in-kernel quantization: aligned, one token tile");
  // QT: tokens one quantization pass covers (at least the slice's rows).  16: each lane
  // quantizes 32 elements of its own MFMA operand row (token r = lane % 16), so with fewer
  // tokens the lanes of the missing ones idle.  8, 4 or 2: the 64 lanes share the QT
  // tokens' groups, kLPT consecutive lanes per token and 2 QT consecutive elements each,
  // and the codes and scales then move to the MFMA operand layout by ds_bpermute.  Same
  // amax (a maximum: order-free), scale and per-element division, so the same bits.
  static_assert(QT == 16 || QT == 8 || QT == 4 || QT == 2, "tokens per quantization pass");
  constexpr bool kDense = kQuant && QT < 16;
  constexpr int kLPT = 64 / QT;  // lanes per token (dense pass)
  constexpr int kE = 128 / kLPT; // elements per lane (dense pass)
  // NORM: x is an RMSNorm's input (bf16).  Waves 0 .. rows-1 each hold one row,
  // x = bf16(x + residual), form its 1 / sqrt(mean(x^2) + eps) (norm_row_inv), code
  // y = bf16(w * bf16(x * inv)) group by group and leave the codes and scales in LDS, where
  // the K loop reads its operands: rmsnorm_quant_kernel's arithmetic and the quantizer's, so
  // y, the codes, the scales and the output bits are those of rmsnorm_quant followed by the
  // GEMM.  Each workgroup repeats this for the (at most 8) rows: 8 K-element rows of work
  // against its own 16 AF K-element weight rows.
  static_assert(!NORM || (kDense && std::is_same<XIn, bf16_t>::value), "RMSNorm: bf16 rows, up to 8 tokens");
  // SILU: the merged gate/up weight (N = 2 I rows, gate rows first) times the rows, then
  // h = bf16(bf16(silu(gate)) * up) per column (the reference's silu_mul, engine/kernels/
  // fused.py:127-137): a workgroup owns gate rows [n0, n0 + rows) and the up rows I + n0 ..,
  // its first AF / 2 MFMA tiles the gate rows, the rest the up rows, so that one thread folds
  // a column's gate and up outputs and writes h[.., n0 + j] (ldo, N / 2 columns).
  static_assert(!SILU || (NORM && RAGGED && AF % 2 == 0), "SiLU epilogue: the norm form, paired row tiles");
  constexpr int kRows = 16 * AF;
  constexpr int kTok = 16 * NT;
  // Token slots kept in the fold buffer: the norm form takes at most 8 rows, so only the MFMA
  // tile's first 8 token columns are published.
  constexpr int kTokS = NORM ? 8 : kTok;
  constexpr int kSB = SILU ? 4 : (RAGGED ? 2 : 1);
  constexpr int kHalfT = SILU ? AF / 2 : AF;  // MFMA tiles per row range
  const int rows = RAGGED ? rows_arg : kRows;
  // [KB][kTokS][kRows] partials, element-major (the fold's reads are consecutive), then
  // [KB][kSB][kTokS] scale products (first and last weight-scale block of the rows; with SILU
  // those of the gate rows, then those of the up rows).
  float* part = reinterpret_cast<float*>(stream_fold_lds);
  float* scl = part + KB * kTokS * kRows;
  // NORM: the rows' 1 / rms [16], the norm weight [K] (bf16), then the rows' bf16(x + residual)
  // [M][K + 8] (rows four banks apart).
  [[maybe_unused]] float* ninv = scl + KB * kSB * kTokS;
  [[maybe_unused]] uint16_t* wl = reinterpret_cast<uint16_t*>(ninv + 16);
  [[maybe_unused]] const int64_t xpitch = K + 8;
  [[maybe_unused]] uint16_t* xs = wl + K;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  // SILU: rows index the gate half [0, N / 2); the up rows sit N / 2 further on.
  const int64_t n_rows = SILU ? N / 2 : N;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * rows;
  const int64_t n_end = n0 + rows < n_rows ? n0 + rows : n_rows;
  const int64_t m_base = static_cast<int64_t>(blockIdx.z) * kTok;
  const int64_t m_rows = (M - m_base) < kTok ? (M - m_base) : kTok;
  const int64_t nb0 = n0 / kGroup, nb1 = (n_end - 1) / kGroup;
  [[maybe_unused]] const int64_t nbu0 = (n_rows + n0) / kGroup, nbu1 = (n_rows + n_end - 1) / kGroup;
  const int64_t wave_u = __builtin_amdgcn_readfirstlane(wave);
  // First weight row of MFMA tile i and the end of its row range.
  auto tile_row = [&](int i) -> int64_t { return i < kHalfT ? n0 + 16 * i : n_rows + n0 + 16 * (i - kHalfT); };
  auto tile_end = [&](int i) -> int64_t { return RAGGED ? (i < kHalfT ? n_end : n_rows + n_end) : N; };

  // Operands of one K group in registers.  Waves keep two groups of loads in flight when
  // the workgroup holds up to three 16-row tiles of one token tile (two when quantizing),
  // one otherwise: measured at M = 8, o_proj 6.9 -> 6.3 us (one tile), qkv 6.83 -> 6.44 us
  // (two tiles), an 11008-row weight 12.35 -> 11.65 us (three); with five tiles the
  // registers spill (gate_up 12.8 -> 17.4 us), and unaligned shapes assemble their loads
  // from bytes and need the registers.
  struct Operands {
    v8i a[AF], b[NT];
    float asv[NT], wsv[kSB];
    // Unquantized activations: elements 16 g .. +15 and 64 + 16 g .. +15 of token r (QT = 16),
    // or the kE elements of this lane's share (dense pass), as raw 16-bit pairs.
    uint32_t xr[kQuant && !NORM ? (kDense ? kE / 2 : 16) : 1];  // NORM: the rows come from LDS
  };
  auto load = [&](Operands& o, int64_t kb) {
    const int64_t k_lo = kb * kGroup + 16 * g;
    // Unquantized activations first: loads complete in issue order, so the wait for them
    // (before the group's quantization) then leaves this group's weight loads in flight, and
    // the quantization overlaps them (qkv and gate_up linears 0.2-0.4 us faster at 1-8 rows).
    if constexpr (NORM) {
      // The rows and the norm weight are in LDS (the norm pass put them there).
    } else if constexpr (kDense) {
      // Token lane / kLPT, elements kb * 128 + (lane % kLPT) kE .. + kE - 1 (K % 16 == 0 and
      // kE divides 16, so a share is either whole or past K).
      const int t = lane / kLPT;
      const int64_t k = kb * kGroup + (lane % kLPT) * kE;
      const XT* xp = reinterpret_cast<const XT*>(q) + (m_base + t) * ldq + k;
      const bool ok = t < m_rows && k < K;
      auto fetch = [&](const uint16_t* p, bool live, uint32_t* dst) {
#pragma unroll
        for (int c = 0; c < kE / 8; ++c) {
          const uint4 v = live ? reinterpret_cast<const uint4*>(p)[c] : make_uint4(0u, 0u, 0u, 0u);
          dst[4 * c] = v.x; dst[4 * c + 1] = v.y; dst[4 * c + 2] = v.z; dst[4 * c + 3] = v.w;
        }
        if constexpr (kE == 4) {
          const uint2 v = live ? *reinterpret_cast<const uint2*>(p) : make_uint2(0u, 0u);
          dst[0] = v.x; dst[1] = v.y;
        }
      };
      fetch(reinterpret_cast<const uint16_t*>(xp), ok, o.xr);
    } else if constexpr (kQuant) {
      const int64_t m = m_base + r;
      const XT* xrow = reinterpret_cast<const XT*>(q) + m * ldq;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int64_t k = k_lo + 64 * (c >> 1) + 8 * (c & 1);
        const uint4 v = (r < m_rows && k < K) ? *reinterpret_cast<const uint4*>(xrow + k) : make_uint4(0u, 0u, 0u, 0u);
        o.xr[4 * c] = v.x; o.xr[4 * c + 1] = v.y; o.xr[4 * c + 2] = v.z; o.xr[4 * c + 3] = v.w;
      }
    }
#pragma unroll
    for (int i = 0; i < AF; ++i) {
      const int64_t row = tile_row(i) + r;
      o.a[i] = pack_v8i(load_chunk16<ALIGNED>(w, ldw, row, tile_end(i), k_lo, K),
                        load_chunk16<ALIGNED>(w, ldw, row, tile_end(i), k_lo + 64, K));
    }
    o.wsv[0] = ws[nb0 * ws_sn + kb * ws_sk];
    if constexpr (RAGGED) o.wsv[1] = ws[nb1 * ws_sn + kb * ws_sk];
    if constexpr (SILU) {
      o.wsv[2] = ws[nbu0 * ws_sn + kb * ws_sk];
      o.wsv[3] = ws[nbu1 * ws_sn + kb * ws_sk];
    }
    if constexpr (!kQuant) {
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int64_t tok = 16 * j + r;
        const int64_t m = m_base + tok;
        o.b[j] = pack_v8i(load_chunk16<ALIGNED>(q, ldq, m, M, k_lo, K), load_chunk16<ALIGNED>(q, ldq, m, M, k_lo + 64, K));
        o.asv[j] = tok < m_rows ? as[m * as_sm + kb * as_sk] : 0.0f;
      }
    }
  };
  // The 1x128 quantizer on the lane's 32 elements of its token's K group; the four lanes of a
  // token (g = 0..3) hold the whole group, so the amax takes two cross-lane steps.
  auto quantize = [&](Operands& o, int64_t kb) {
    constexpr int kN = kDense ? kE : 32;  // elements this lane quantizes
    float t[kN];
    if constexpr (NORM) {
      // y = bf16(w * bf16(x * inv)) from the rows the norm pass left in LDS
      // (rmsnorm_quant_kernel's pass 2); the slice's padding tokens quantize zeros.
      const int tok = lane / kLPT;
      const int64_t k = kb * kGroup + (lane % kLPT) * kE;
      const bool live = tok < m_rows;
      const float inv = live ? ninv[tok] : 0.0f;
      uint32_t xw[kE / 2], ww[kE / 2];
#pragma unroll
      for (int c = 0; c < kE / 2; c += (kE >= 8 ? 4 : 2)) {
        if constexpr (kE >= 8) {
          const uint4 xv = live ? *reinterpret_cast<const uint4*>(xs + tok * xpitch + k + 2 * c) : make_uint4(0u, 0u, 0u, 0u);
          const uint4 wv = *reinterpret_cast<const uint4*>(wl + k + 2 * c);
          xw[c] = xv.x; xw[c + 1] = xv.y; xw[c + 2] = xv.z; xw[c + 3] = xv.w;
          ww[c] = wv.x; ww[c + 1] = wv.y; ww[c + 2] = wv.z; ww[c + 3] = wv.w;
        } else {
          const uint2 xv = live ? *reinterpret_cast<const uint2*>(xs + tok * xpitch + k + 2 * c) : make_uint2(0u, 0u);
          const uint2 wv = *reinterpret_cast<const uint2*>(wl + k + 2 * c);
          xw[c] = xv.x; xw[c + 1] = xv.y; ww[c] = wv.x; ww[c + 1] = wv.y;
        }
      }
#pragma unroll
      for (int e = 0; e < kN / 2; ++e)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float normed = round_bf16(bf16_bits_val(xw[e] >> (16 * h)) * inv);
          t[2 * e + h] = round_bf16(bf16_bits_val(ww[e] >> (16 * h)) * normed);
        }
    } else {
#pragma unroll
      for (int e = 0; e < kN / 2; ++e) {
        t[2 * e] = to_f32(XT{static_cast<uint16_t>(o.xr[e] & 0xffffu)});
        t[2 * e + 1] = to_f32(XT{static_cast<uint16_t>(o.xr[e] >> 16)});
      }
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < kN; ++e) amax = fmaxf(amax, fabsf(t[e]));
    if constexpr (kDense) {
      amax = group_max<kLPT>(amax);
    } else {
      // The four lanes of a token (g = 0..3, lanes r + 16 g) hold the whole group.
      amax = row_max(amax);
    }
    const float scale = amax / 448.0f;
    const float den = scale > 1e-12f ? scale : 1e-12f;
    uint32_t packed[kN / 4];
    quant_codes<kN>(t, den, packed);
    if constexpr (kDense) {
      // Operand lane (r, g) takes token r's code words 4 g .. 4 g + 3 and 16 + 4 g .. +3; word d
      // of token r sits in lane r kLPT + d / (kE / 4), slot d % (kE / 4), which is j % (kE / 4)
      // for both ranges (kE / 4 divides 4).
      constexpr int kW = kE / 4;
      const int src0 = r * kLPT;
      v8i b;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        b[j] = __builtin_amdgcn_ds_bpermute(4 * (src0 + (4 * g + j) / kW), static_cast<int>(packed[j % kW]));
        b[4 + j] = __builtin_amdgcn_ds_bpermute(4 * (src0 + (16 + 4 * g + j) / kW), static_cast<int>(packed[j % kW]));
      }
      const float sc = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * src0, __builtin_bit_cast(int, scale)));
      const bool live = r < QT;
#pragma unroll
      for (int j = 0; j < 8; ++j) b[j] = live ? b[j] : 0;
      o.b[0] = b;
      o.asv[0] = live ? sc : 0.0f;
    } else {
      o.b[0] = pack_v8i(make_uint4(packed[0], packed[1], packed[2], packed[3]),
                        make_uint4(packed[4], packed[5], packed[6], packed[7]));
      o.asv[0] = scale;
    }
  };
  // MFMA partials of group kb and their publication; `refill` loads group kb_next into the
  // registers just consumed (issued before the LDS writes, so it overlaps them).
  auto consume = [&](Operands& o, int64_t kb, int64_t kb_next) {
    if constexpr (kQuant) quantize(o, kb);
    v4f p[AF][NT];
#pragma unroll
    for (int i = 0; i < AF; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) p[i][j] = mfma_16x16x128_e4m3(o.a[i], o.b[j]);
    float sc[kSB][NT];
#pragma unroll
    for (int b = 0; b < kSB; ++b)
#pragma unroll
      for (int j = 0; j < NT; ++j) sc[b][j] = o.asv[j] * o.wsv[b];
    if (kb_next < KB) load(o, kb_next);
    // Lane holds D[n = 16 i + 4 g + v][tok = 16 j + r]: four consecutive n of one token.
    if (kTokS == kTok || r < kTokS) {
#pragma unroll
      for (int i = 0; i < AF; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          *reinterpret_cast<float4*>(part + (kb * kTokS + 16 * j + r) * kRows + 16 * i + 4 * g) =
              make_float4(p[i][j][0], p[i][j][1], p[i][j][2], p[i][j][3]);
      if (g == 0) {
#pragma unroll
        for (int b = 0; b < kSB; ++b)
#pragma unroll
          for (int j = 0; j < NT; ++j) scl[(kb * kSB + b) * kTokS + 16 * j + r] = sc[b][j];
      }
    }
  };
  constexpr int kDepth = ALIGNED && NT == 1 && AF <= (kQuant ? 2 : 3) ? 2 : 1;
  constexpr int64_t kStep = static_cast<int64_t>(kStreamWaves) * kDepth;
  Operands ops[kDepth];
  // NORM: each of the first rows waves loads its row (and residual) before the group loads
  // below, so that its wait for them leaves the weight loads in flight (loads complete in
  // issue order).
  [[maybe_unused]] uint2 nxv[NORM ? kNormMaxVec : 1], nrv[NORM ? kNormMaxVec : 1];
  [[maybe_unused]] uint4 nwv = make_uint4(0u, 0u, 0u, 0u);  // norm weight elements 8 tid .. +7
  [[maybe_unused]] const int nv = NORM ? static_cast<int>(K / 256) : 0;
  [[maybe_unused]] const bool nrow = NORM && wave_u < m_rows;
  if constexpr (NORM) {
    if (tid < K / 8) nwv = reinterpret_cast<const uint4*>(na.w)[tid];
    if (nrow) {
      const uint16_t* xrow = reinterpret_cast<const uint16_t*>(q) + (m_base + wave_u) * ldq;
      const uint16_t* rrow = na.res != nullptr ? na.res + (m_base + wave_u) * na.ldr : nullptr;
#pragma unroll
      for (int i = 0; i < kNormMaxVec; ++i) {
        if (i < nv) {
          nxv[i] = *reinterpret_cast<const uint2*>(xrow + 4 * (lane + 64 * i));
          if (rrow != nullptr) nrv[i] = *reinterpret_cast<const uint2*>(rrow + 4 * (lane + 64 * i));
        }
      }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int d = 0; d < kDepth; ++d)
    if (wave_u + d * kStreamWaves < KB) load(ops[d], wave_u + d * kStreamWaves);
  if constexpr (NORM) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    float inv = 0.0f;
    if (nrow) {
      const int64_t m = m_base + wave_u;
      if (na.res != nullptr) {
#pragma unroll
        for (int i = 0; i < kNormMaxVec; ++i) {
          if (i < nv) {
            nxv[i] = make_uint2(bf16_add_pair(nxv[i].x, nrv[i].x), bf16_add_pair(nxv[i].y, nrv[i].y));
            if (na.sum != nullptr && blockIdx.x == 0)
              *reinterpret_cast<uint2*>(na.sum + m * na.lds + 4 * (lane + 64 * i)) = nxv[i];
          }
        }
      }
#pragma unroll
      for (int i = 0; i < kNormMaxVec; ++i)
        if (i < nv) *reinterpret_cast<uint2*>(xs + wave_u * xpitch + 4 * (lane + 64 * i)) = nxv[i];
      switch (na.bw) {
        case 512: inv = norm_row_inv<8>(nxv, nv, na); break;
        case 256: inv = norm_row_inv<4>(nxv, nv, na); break;
        case 128: inv = norm_row_inv<2>(nxv, nv, na); break;
        default: inv = norm_row_inv<1>(nxv, nv, na); break;
      }
    }
    if (lane == 0 && nrow) ninv[wave_u] = inv;
    if (tid < K / 8) reinterpret_cast<uint4*>(wl)[tid] = nwv;
    __syncthreads();
  }
  for (int64_t kb = wave_u; kb < KB; kb += kStep) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      const int64_t k = kb + d * kStreamWaves;
      if (k < KB) consume(ops[d], k, k + kStep);
    }
  }
  __syncthreads();
  // One output element (token, row) per thread, two when rows x tokens exceeds the threads.
  // The chain over the K groups in increasing order; reads in batches of eight ahead of their
  // FMAs, so the chain waits on LDS once per batch.
  auto fold = [&](const float* pf, const float* sf) {
    float acc = 0.0f;
    int64_t kb = 0;
    for (; kb + 8 <= KB; kb += 8) {
      float pv[8], sv[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        pv[x] = pf[(kb + x) * kTokS * kRows];
        sv[x] = sf[(kb + x) * kSB * kTokS];
      }
#pragma unroll
      for (int x = 0; x < 8; ++x) acc = __builtin_fmaf(pv[x], sv[x], acc);
    }
    for (; kb < KB; ++kb) acc = __builtin_fmaf(pf[kb * kTokS * kRows], sf[kb * kSB * kTokS], acc);
    return acc;
  };
  const int live = RAGGED ? static_cast<int>(n_end - n0) : kRows;
  for (int e = tid; e < live * kTok; e += kStreamWaves * 64) {
    const int tok = e / live, nl = e - (e / live) * live;
    if (tok >= m_rows) break;  // padding tokens: nothing to fold (later e only have larger tok)
    const float* pf = part + tok * kRows + nl;
    const float* sf = scl + (RAGGED && (n0 + nl) / kGroup != nb0 ? kTokS : 0) + tok;
    if constexpr (SILU) {
      // gate row n0 + nl and up row N / 2 + n0 + nl of this token, rounded to the GEMM's
      // bf16 output, then silu = bf16(g / (1 + exp(-g))) and h = bf16(silu * u): the
      // arithmetic of silu_mul_quant_kernel on the bf16 gate/up outputs.
      const float* sfu = scl + (2 + ((n_rows + n0 + nl) / kGroup != nbu0 ? 1 : 0)) * kTokS + tok;
      const float g = bf16_bits_val(OutCvt<bf16_t>::cvt(fold(pf, sf)));
      const float u = bf16_bits_val(OutCvt<bf16_t>::cvt(fold(pf + 16 * kHalfT, sfu)));
      const float silu = round_bf16(g / (1.0f + expf(-g)));
      out[(m_base + tok) * ldo + n0 + nl] = f32_to_bf16_bits(silu * u);
    } else {
      const float acc = fold(pf, sf);
      if (RAGGED || n0 + nl < N) out[(m_base + tok) * ldo + n0 + nl] = OutCvt<OutT>::cvt(acc);
    }
  }
}

// ------------------------------------------------------------------------------------
// Tile kernel (prefill M)
// ------------------------------------------------------------------------------------
constexpr int kTileM = 128;
constexpr int kTileN = 128;
constexpr int kGroupTiles = 8;  // tile rows per L2-reuse group

// Logical tile of workgroup `pid`: workgroups are dispatched round-robin over the 8 XCDs,
// so consecutive pids land on different L2s.  Remap so that each XCD owns a contiguous
// range of logical tiles, then walk that range in groups of kGroupTiles tile rows.
__device__ __forceinline__ void tile_of(int64_t pid, int64_t tiles_m, int64_t tiles_n,
                                        int64_t* tm, int64_t* tn) {
  const int64_t total = tiles_m * tiles_n;
  const int64_t per = total / 8, rem = total % 8;
  const int64_t xcd = pid % 8, idx = pid / 8;
  const int64_t logical = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  const int64_t per_group = kGroupTiles * tiles_n;
  const int64_t group = logical / per_group;
  const int64_t first_m = group * kGroupTiles;
  const int64_t gm = (tiles_m - first_m) < kGroupTiles ? (tiles_m - first_m) : kGroupTiles;
  const int64_t within = logical - group * per_group;
  *tm = first_m + within % gm;
  *tn = within / gm;
}

template <bool ALIGNED, typename OutT>
__global__ __launch_bounds__(kThreads, 2) void tile_gemm_kernel(
    const uint8_t* __restrict__ q, int64_t ldq, const float* __restrict__ as, int64_t as_sm,
    int64_t as_sk, const uint8_t* __restrict__ w, int64_t ldw, const float* __restrict__ ws,
    int64_t ws_sn, int64_t ws_sk, uint16_t* __restrict__ out, int64_t ldo, int64_t M, int64_t N,
    int64_t K, int64_t KB, int64_t tiles_m, int64_t tiles_n, int vec_out) {
  // [buffer][0 = W tile, 1 = activation tile][row * 8 + swizzled 16-byte chunk]
  __shared__ uint4 lds[2][2][kTileM * 8];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int wm = wave & 1;   // activation-row half of the tile
  const int wn = wave >> 1;  // weight-row half of the tile
  int64_t tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, &tm, &tn);
  const int64_t m0 = tm * kTileM;
  const int64_t n0 = tn * kTileN;
  const int64_t nb = n0 / kGroup;

  // Global -> LDS copy assignment: thread covers chunk c of rows rr + 32 i.
  const int c = tid & 7;
  const int rr = tid >> 3;
  uint4 gw[4], gx[4];
  auto gload = [&](int64_t kb) {
    const int64_t k = kb * kGroup + 16 * c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      gw[i] = load_chunk16<ALIGNED>(w, ldw, n0 + rr + 32 * i, N, k, K);
      gx[i] = load_chunk16<ALIGNED>(q, ldq, m0 + rr + 32 * i, M, k, K);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = rr + 32 * i;
      const int slot = row * 8 + (c ^ (row & 7));
      lds[buf][0][slot] = gw[i];
      lds[buf][1][slot] = gx[i];
    }
  };

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  gload(0);
  lstore(0);
  __syncthreads();
  for (int64_t kb = 0; kb < KB; ++kb) {
    const int buf = static_cast<int>(kb & 1);
    if (kb + 1 < KB) gload(kb + 1);
    const float wsv = ws[nb * ws_sn + kb * ws_sk];
    float sc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t m = m0 + wm * 64 + 16 * j + r;
      sc[j] = (m < M ? as[m * as_sm + kb * as_sk] : 0.0f) * wsv;
    }
    v8i a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = wn * 64 + 16 * i + r;
      a[i] = pack_v8i(lds[buf][0][row * 8 + (g ^ (row & 7))], lds[buf][0][row * 8 + ((g + 4) ^ (row & 7))]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = wm * 64 + 16 * j + r;
      b[j] = pack_v8i(lds[buf][1][row * 8 + (g ^ (row & 7))], lds[buf][1][row * 8 + ((g + 4) ^ (row & 7))]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4f d = mfma_16x16x128_e4m3(a[i], b[j]);
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(d[v], sc[j], acc[i][j][v]);
      }
    if (kb + 1 < KB) lstore(buf ^ 1);
    __syncthreads();
  }

  // Lane holds out[m = m0 + 64 wm + 16 j + r][n = n0 + 64 wn + 16 i + 4 g + v].
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t m = m0 + wm * 64 + 16 * j + r;
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t n = n0 + wn * 64 + 16 * i + 4 * g;
      uint16_t h[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) h[v] = OutCvt<OutT>::cvt(acc[i][j][v]);
      uint16_t* dst = out + m * ldo + n;
      if (vec_out && n + 4 <= N) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16),
                                                    h[2] | (static_cast<uint32_t>(h[3]) << 16));
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (n + v < N) dst[v] = h[v];
      }
    }
  }
}

// ------------------------------------------------------------------------------------
// Host side: planning and launch
// ------------------------------------------------------------------------------------
static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

int plan_gemm(int64_t M, int64_t N, int64_t K, int config, GemmPlan* plan) {
  return plan_gemm_on(M, N, K, config, device_cus(), plan);
}

int plan_gemm_on(int64_t M, int64_t N, int64_t K, int config, int64_t cus, GemmPlan* plan) {
  if (M < 0 || N < 0 || K <= 0 || cus <= 0) return MI355X_FP8_ERR_INVALID;
  *plan = GemmPlan{};
  if (config == MI355X_FP8_CONFIG_AUTO) {
    // Every kernel gives the same bits, so this is a speed choice only.  The stream kernel
    // re-reads the activations from L2 in every workgroup, so with more rows it keeps the
    // lead only while the weight rows give few workgroups, and its re-reads grow with M x K.
    // Measured on the Qwen3-4B shapes with the weights streamed from HBM (µs, streamed
    // against tiled): o_proj (K = 4096) at 64 rows 10.8 / 12.9; down (K = 9728) at 48 rows
    // 22.6 / 24.8, at 56 and 64 rows 27.4 / 25.6 and 29.8 / 26.3; qkv at 32 rows 9.1 / 9.5,
    // at 40 rows 13.3 / 9.8; gate_up at 17 rows 19.4 / 16.1.
    const bool stream = M <= 16 || (M <= 64 && cdiv(N, 16) <= cus && M * K <= 48 * 9728) ||
                        (M <= 32 && cdiv(N, 16) <= 2 * cus);
    config = stream ? MI355X_FP8_CONFIG_STREAM : MI355X_FP8_CONFIG_TILE128;
  }
  if (config < MI355X_FP8_CONFIG_STREAM || config > MI355X_FP8_CONFIG_DMA64_128) return MI355X_FP8_ERR_INVALID;
  plan->kernel = config;
  if (config != MI355X_FP8_CONFIG_STREAM) return MI355X_FP8_OK;
  // One 16-token tile per workgroup up to 16 rows, else slices of 32 rows (two tiles), one
  // slice per grid z.  Each slice re-reads the weights, mostly from L2 and the MALL while the
  // slices run side by side; 64-row slices re-read the activations 4x per workgroup instead
  // and measured slower (down at 40 rows 24.5 against 19.2 us).
  plan->token_tiles = M <= 16 ? 1 : 2;
  // Two 16-row MFMA tiles per workgroup from N = 6144 up: halves the L2 re-reads of the
  // activations.  Measured on the Qwen3-4B shapes: the merged qkv (N = 6144, 192 workgroups)
  // 7.12 -> 6.78 us at 8 rows and 7.96 -> 7.14 us at 16, unchanged at 1 and 32 rows; o_proj
  // and down (N = 2560) are slower with 80 workgroups and keep one tile.
  plan->row_tiles = (N >= 6144 &&
                     stream_fold_bytes(cdiv(K, kGroup), 2, plan->token_tiles) <= kStreamFoldLds)
                        ? 2
                        : 1;
  plan->rows = 16 * plan->row_tiles;
  // The same number of weight rows on every CU, one workgroup per CU and token slice, when
  // that fits in five MFMA tiles and the LDS, and either a workgroup then holds one MFMA tile
  // or the 16-row-multiple plan needs more workgroups than CUs.  A CU keeps only so many loads
  // in flight, so the rows it streams matter; every workgroup also re-reads all of the
  // activations, which is why spreading a plan that already runs in one round does not pay
  // for two-tile workgroups.
  // Measured at M = 8 (Qwen3-4B): o_proj 16 -> 10 rows per CU 6.25 -> 5.99 us, down 16 -> 10
  // 10.1 -> 9.7 us, gate_up 96 (three 32-row workgroups on some CUs) -> 76 14.7 -> 12.7 us;
  // qkv 32 -> 24 measured 6.84 -> 6.93 us and keeps 32.  At least kStreamMinRows rows per
  // workgroup, so that narrow weights do not spread over workgroups for a few rows each.
  {
    const int64_t slices = M > 0 ? cdiv(M, 16 * plan->token_tiles) : 1;
    const int64_t share = cus / slices > 1 ? cus / slices : 1;
    const int64_t rows = cdiv(N, share) > kStreamMinRows ? cdiv(N, share) : kStreamMinRows;
    const int64_t af = cdiv(rows, 16);
    const int64_t old_wgs = cdiv(N, plan->rows) * slices;
    const int64_t old_rows = plan->rows * cdiv(old_wgs, cus);
    if (af <= 5 && cdiv(N, rows) * slices <= cus && rows < old_rows && (af == 1 || old_wgs > cus) &&
        stream_fold_bytes(cdiv(K, kGroup), static_cast<int>(af), plan->token_tiles, 2) <= kStreamFoldLdsOne) {
      plan->row_tiles = static_cast<int>(af);
      plan->rows = static_cast<int>(rows);
    }
  }
  return MI355X_FP8_OK;
}

size_t gemm_workspace_bytes(const GemmPlan&) { return 0; }

int64_t device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Prefill kernel choice when the LDS-DMA kernels can run, from measured wave times.  Each
// K step waits for its operands (a fifth of the lines miss L2), so a wave of tiles costs
// about the same whatever the tile width, and the deeper rings of the narrower tiles make
// their steps shorter.  Time of one full wave of tiles over K = 2560 on MI355X (µs, every
// CU busy; the DMA kernel's second figure is for two workgroups per CU, the layout it
// takes when the tiles outnumber the CUs):
//   256 x 256 / 224 / 192 (two stages)   46.5  42.4  37.4
//   256 x 160 / 128 (three stages)       33.5  28.0
//   128 x 160 / 128 / 64 (three stages)  21.4  17.5  12.5   (two per CU: 33.5  28.5  20.4)
//   192 x 256 (two stages)               40.7
//   192 x 160 / 128 (three stages)       26.0  24.5
//   64 x 128 / 64 (three / four stages)  13.5   8.1   (two per CU: 22.0  13.5)
// The 192-row tiles serve row counts just past a multiple of 256 or 128 (M = 536: 3 x 192
// rows against 3 x 256), the 64-row ones small M whose 128-row tiles leave CUs idle (o_proj
// and down up to 384 rows, qkv up to 128 and at 257-320).  Their figures are fitted to
// measured cases with the weights streamed from HBM (40 rotating sets, beyond the MALL), set
// so that the model keeps the older variant where the two measured within 4 %, or where the
// 64-row tile re-reads the weights from HBM more than it gains (64 x 128 for o_proj and down
// at 536 and 700 rows, gate_up at 160 and 176); listed last, they lose ties.  (qkv at 1024
// rows takes 192 x 160: 1-3 % either way against 256 x 128.)
// A last, partly filled wave costs 0.7 + 0.3 x its fill of a full one (a half-filled wave
// measured 0.75-0.98).  Every kernel gives the same bits, so the choice may follow M.
namespace {
struct TileVariant {
  int rows, bn;
  double wave_one;  // µs per full wave, one workgroup per CU
  double wave_two;  // µs per full wave of two workgroups per CU (0: not used)
};
constexpr TileVariant kTileVariants[] = {
    {256, 256, 46.5, 0.0}, {256, 224, 42.4, 0.0}, {256, 192, 37.4, 0.0}, {256, 160, 33.5, 0.0},
    {256, 128, 28.0, 0.0}, {128, 160, 21.4, 33.5}, {128, 128, 17.5, 28.5}, {128, 64, 12.5, 20.4},
    {192, 256, 40.7, 0.0}, {192, 160, 26.0, 0.0}, {192, 128, 24.5, 0.0},
    {64, 128, 13.5, 22.0},  {64, 64, 8.1, 13.5},
};

double waves_cost(int64_t tiles, int64_t slots, double wave) {
  const int64_t full = tiles / slots, rem = tiles % slots;
  return wave * (static_cast<double>(full) + (rem ? 0.7 + 0.3 * static_cast<double>(rem) / slots : 0.0));
}

double variant_cost(const TileVariant& v, int64_t M, int64_t N, int64_t cus) {
  const int64_t tiles = cdiv(M, v.rows) * cdiv(N, v.bn);
  if (v.wave_two == 0.0 || tiles <= cus) return waves_cost(tiles, cus, v.wave_one);
  return waves_cost(tiles, 2 * cus, v.wave_two);
}

struct PrefillChoice {
  int rows;  // 64 or 128: tile_gemm_dma; 192 or 256: tile_gemm_256
  int bn;
};

// rows256_ok: the 256-row kernel's 32-bit offsets reach every byte of q and W (its 192-row
// form has the same limits).
PrefillChoice choose_prefill(int64_t M, int64_t N, int64_t cus, bool rows256_ok) {
  PrefillChoice best{128, 128};
  double best_cost = -1.0;
  for (const TileVariant& v : kTileVariants) {
    if (v.rows > 128 && !rows256_ok) continue;
    const double cost = variant_cost(v, M, N, cus);
    if (best_cost < 0.0 || cost < best_cost) {
      best = {v.rows, v.bn};
      best_cost = cost;
    }
  }
  return best;
}
}  // namespace

void prefill_choice(int64_t M, int64_t N, int64_t cus, int* rows, int* bn) {
  const PrefillChoice c = choose_prefill(M, N, cus, true);
  *rows = c.rows;
  *bn = c.bn;
}

int tile256_width(int64_t M, int64_t N, int64_t cus) {
  int best = 256;
  double best_cost = -1.0;
  for (const TileVariant& v : kTileVariants) {
    if (v.rows != 256) continue;
    const double cost = variant_cost(v, M, N, cus);
    if (best_cost < 0.0 || cost < best_cost) {
      best = v.bn;
      best_cost = cost;
    }
  }
  return best;
}

template <int NT, int AF, bool ALIGNED, typename OutT>
static void launch_stream_t(const uint8_t* q, int64_t ldq, const float* as, int64_t as_sm, int64_t as_sk,
                            const uint8_t* w, int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk,
                            uint16_t* out, int64_t ldo, int64_t M, int64_t N, int64_t K, int rows,
                            hipStream_t stream) {
  dim3 grid(static_cast<unsigned>(cdiv(N, rows)), 1, static_cast<unsigned>(cdiv(M, 16 * NT)));
  const int64_t kb = cdiv(K, kGroup);
  // Ragged row counts are planned only where the one-round buffer fits (plan_gemm).
  if constexpr (8 % AF == 0) {
    if (rows == 16 * AF) {
      const size_t one_round = stream_fold_bytes(kb, AF, NT);
      if (one_round <= kStreamFoldLds)
        stream_gemm_kernel<NT, AF, ALIGNED, false, OutT><<<grid, kStreamWaves * 64, one_round, stream>>>(
            q, ldq, as, as_sm, as_sk, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, kb, rows);
      else
        stream_rounds_kernel<NT, AF, ALIGNED, OutT><<<grid, kStreamWaves * 64, 0, stream>>>(
            q, ldq, as, as_sm, as_sk, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, kb);
      return;
    }
  }
  stream_gemm_kernel<NT, AF, ALIGNED, true, OutT><<<grid, kStreamWaves * 64, stream_fold_bytes(kb, AF, NT, 2), stream>>>(
      q, ldq, as, as_sm, as_sk, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, kb, rows);
}

template <bool ALIGNED, typename OutT>
static void launch_stream(const GemmPlan& p, const uint8_t* q, int64_t ldq, const float* as,
                          int64_t as_sm, int64_t as_sk, const uint8_t* w, int64_t ldw,
                          const float* ws, int64_t ws_sn, int64_t ws_sk, uint16_t* out, int64_t ldo,
                          int64_t M, int64_t N, int64_t K, hipStream_t stream) {
#define MI355X_STREAM_ARGS q, ldq, as, as_sm, as_sk, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, p.rows, stream
  if (p.token_tiles == 1) {
    switch (p.row_tiles) {
      case 5: launch_stream_t<1, 5, ALIGNED, OutT>(MI355X_STREAM_ARGS); break;
      case 4: launch_stream_t<1, 4, ALIGNED, OutT>(MI355X_STREAM_ARGS); break;
      case 3: launch_stream_t<1, 3, ALIGNED, OutT>(MI355X_STREAM_ARGS); break;
      case 2: launch_stream_t<1, 2, ALIGNED, OutT>(MI355X_STREAM_ARGS); break;
      default: launch_stream_t<1, 1, ALIGNED, OutT>(MI355X_STREAM_ARGS); break;
    }
  } else {
    switch (p.row_tiles) {
      case 5: launch_stream_t<2, 5, ALIGNED, OutT>(MI355X_STREAM_ARGS); break;
      case 4: launch_stream_t<2, 4, ALIGNED, OutT>(MI355X_STREAM_ARGS); break;
      case 3: launch_stream_t<2, 3, ALIGNED, OutT>(MI355X_STREAM_ARGS); break;
      case 2: launch_stream_t<2, 2, ALIGNED, OutT>(MI355X_STREAM_ARGS); break;
      default: launch_stream_t<2, 1, ALIGNED, OutT>(MI355X_STREAM_ARGS); break;
    }
  }
#undef MI355X_STREAM_ARGS
}

template <bool ALIGNED, typename OutT>
static void launch_tile(const uint8_t* q, int64_t ldq, const float* as, int64_t as_sm, int64_t as_sk,
                        const uint8_t* w, int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk,
                        uint16_t* out, int64_t ldo, int64_t M, int64_t N, int64_t K, int64_t tiles_m,
                        int64_t tiles_n, int vec_out, hipStream_t stream) {
  dim3 grid(static_cast<unsigned>(tiles_m * tiles_n));
  tile_gemm_kernel<ALIGNED, OutT><<<grid, kThreads, 0, stream>>>(q, ldq, as, as_sm, as_sk, w, ldw, ws, ws_sn,
                                                                 ws_sk, out, ldo, M, N, K, cdiv(K, kGroup),
                                                                 tiles_m, tiles_n, vec_out);
}

template <bool ALIGNED, typename OutT>
static int launch_typed(const GemmPlan& plan, const uint8_t* q, int64_t ldq, const float* as,
                        int64_t as_sm, int64_t as_sk, const uint8_t* w, int64_t ldw, const float* ws,
                        int64_t ws_sn, int64_t ws_sk, uint16_t* out, int64_t ldo, int64_t M, int64_t N,
                        int64_t K, void* workspace, hipStream_t stream) {
  if (plan.kernel == MI355X_FP8_CONFIG_STREAM) {
    if (plan.rows < 1 || cdiv(N, plan.rows) > 0x7fffffffLL || cdiv(M, 16 * plan.token_tiles) > 65535)
      return MI355X_FP8_ERR_UNSUPPORTED;
    launch_stream<ALIGNED, OutT>(plan, q, ldq, as, as_sm, as_sk, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K,
                                 stream);
  } else {
    const int64_t tiles_m = cdiv(M, kTileM), tiles_n = cdiv(N, kTileN);
    if (tiles_m * tiles_n > 0x7fffffffLL) return MI355X_FP8_ERR_UNSUPPORTED;
    const int vec_out = (ldo % 4) == 0 && (reinterpret_cast<uintptr_t>(out) % 8) == 0;
    launch_tile<ALIGNED, OutT>(q, ldq, as, as_sm, as_sk, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, tiles_m,
                               tiles_n, vec_out, stream);
  }
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

int launch_block_gemm(const GemmPlan& plan, const uint8_t* q, int64_t ldq, const float* as,
                      int64_t as_sm, int64_t as_sk, const uint8_t* w, int64_t ldw, const float* ws,
                      int64_t ws_sn, int64_t ws_sk, void* out, int out_dtype, int64_t ldo,
                      int64_t M, int64_t N, int64_t K, void* workspace, hipStream_t stream) {
  if (M == 0 || N == 0) return MI355X_FP8_OK;
  const bool dma_ok = tile_dma_supported(q, ldq, as_sm, as_sk, w, ldw, M, K);
  if (plan.kernel >= MI355X_FP8_CONFIG_DMA128_64) {
    // A forced variant: the LDS-DMA preconditions, and for 256- and 192-row tiles their 32-bit
    // offsets.
    static constexpr int kWidth[] = {64, 128, 160, 128, 160, 192, 224, 256, 128, 160, 192, 224, 256, 64, 128};
    const int bn = kWidth[plan.kernel - MI355X_FP8_CONFIG_DMA128_64];
    if (!dma_ok) return MI355X_FP8_ERR_UNSUPPORTED;
    if (plan.kernel <= MI355X_FP8_CONFIG_DMA128_160)
      return launch_tile_dma(q, ldq, as, as_sk, w, ldw, ws, ws_sn, ws_sk, out, out_dtype, ldo, M, N, K, bn, 128, stream);
    if (plan.kernel >= MI355X_FP8_CONFIG_DMA64_64)
      return launch_tile_dma(q, ldq, as, as_sk, w, ldw, ws, ws_sn, ws_sk, out, out_dtype, ldo, M, N, K, bn, 64, stream);
    const int rows = plan.kernel >= MI355X_FP8_CONFIG_T192_128 ? 192 : 256;
    return launch_tile256(q, ldq, as, as_sk, w, ldw, ws, ws_sn, ws_sk, out, out_dtype, ldo, M, N, K, bn, rows,
                          stream);
  }
  if (plan.kernel == MI355X_FP8_CONFIG_TILE256) {
    if (!dma_ok) return MI355X_FP8_ERR_UNSUPPORTED;
    return launch_tile256(q, ldq, as, as_sk, w, ldw, ws, ws_sn, ws_sk, out, out_dtype, ldo, M, N, K,
                          tile256_width(M, N, device_cus()), 256, stream);
  }
  if (plan.kernel == MI355X_FP8_CONFIG_TILE128 && dma_ok) {
    const PrefillChoice c = choose_prefill(M, N, device_cus(), tile256_offsets_ok(ldq, ldw, M, N, K));
    if (c.rows > 128)
      return launch_tile256(q, ldq, as, as_sk, w, ldw, ws, ws_sn, ws_sk, out, out_dtype, ldo, M, N, K, c.bn, c.rows,
                            stream);
    return launch_tile_dma(q, ldq, as, as_sk, w, ldw, ws, ws_sn, ws_sk, out, out_dtype, ldo, M, N, K, c.bn, c.rows,
                           stream);
  }
  const bool aligned = (K % 16) == 0 && (ldq % 16) == 0 && (ldw % 16) == 0 &&
                       (reinterpret_cast<uintptr_t>(q) % 16) == 0 &&
                       (reinterpret_cast<uintptr_t>(w) % 16) == 0;
  uint16_t* o = static_cast<uint16_t*>(out);
#define MI355X_GEMM_ARGS plan, q, ldq, as, as_sm, as_sk, w, ldw, ws, ws_sn, ws_sk, o, ldo, M, N, K, workspace, stream
  if (aligned)
    return out_dtype == kBF16 ? launch_typed<true, bf16_t>(MI355X_GEMM_ARGS) : launch_typed<true, f16_t>(MI355X_GEMM_ARGS);
  return out_dtype == kBF16 ? launch_typed<false, bf16_t>(MI355X_GEMM_ARGS) : launch_typed<false, f16_t>(MI355X_GEMM_ARGS);
#undef MI355X_GEMM_ARGS
}

// The whole linear in one launch at decode sizes: the stream kernel quantizing its own K
// groups (XIn = bf16_t / f16_t).  Returns MI355X_FP8_ERR_UNSUPPORTED, having launched
// nothing, when the call does not fit that form (then the caller quantizes first).
template <int AF, typename OutT, typename XIn, int QT>
static int launch_linear_stream_q(const GemmPlan& p, const XIn* x, int64_t sxm, const uint8_t* w, int64_t ldw,
                                  const float* ws, int64_t ws_sn, int64_t ws_sk, uint16_t* out, int64_t ldo,
                                  int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  const int64_t kb = cdiv(K, kGroup);
  const bool ragged = p.rows != 16 * AF || 8 % AF != 0;
  const size_t bytes = stream_fold_bytes(kb, AF, 1, ragged ? 2 : 1);
  if (bytes > (ragged ? kStreamFoldLdsOne : kStreamFoldLds)) return MI355X_FP8_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(cdiv(N, p.rows)), 1, 1);
  const uint8_t* xq = reinterpret_cast<const uint8_t*>(x);
  if (ragged)
    stream_gemm_kernel<1, AF, true, true, OutT, XIn, QT><<<grid, kStreamWaves * 64, bytes, stream>>>(
        xq, sxm, nullptr, 0, 0, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, kb, p.rows);
  else if constexpr (8 % AF == 0)
    stream_gemm_kernel<1, AF, true, false, OutT, XIn, QT><<<grid, kStreamWaves * 64, bytes, stream>>>(
        xq, sxm, nullptr, 0, 0, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, kb, p.rows);
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

// Tokens per quantization pass: the fewest of 2, 4, 8 and 16 that hold the rows.
template <int AF, typename OutT, typename XIn>
static int launch_linear_stream_t(const GemmPlan& p, const XIn* x, int64_t sxm, const uint8_t* w, int64_t ldw,
                                  const float* ws, int64_t ws_sn, int64_t ws_sk, uint16_t* out, int64_t ldo,
                                  int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  if (M <= 2) return launch_linear_stream_q<AF, OutT, XIn, 2>(p, x, sxm, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, stream);
  if (M <= 4) return launch_linear_stream_q<AF, OutT, XIn, 4>(p, x, sxm, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, stream);
  if (M <= 8) return launch_linear_stream_q<AF, OutT, XIn, 8>(p, x, sxm, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, stream);
  return launch_linear_stream_q<AF, OutT, XIn, 16>(p, x, sxm, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, stream);
}

template <typename OutT, typename XIn>
static int launch_linear_stream_x(const GemmPlan& p, const XIn* x, int64_t sxm, const uint8_t* w, int64_t ldw,
                                  const float* ws, int64_t ws_sn, int64_t ws_sk, uint16_t* out, int64_t ldo,
                                  int64_t M, int64_t N, int64_t K, hipStream_t stream) {
#define MI355X_LIN_ARGS p, x, sxm, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, stream
  switch (p.row_tiles) {
    case 5: return launch_linear_stream_t<5, OutT, XIn>(MI355X_LIN_ARGS);
    case 4: return launch_linear_stream_t<4, OutT, XIn>(MI355X_LIN_ARGS);
    case 3: return launch_linear_stream_t<3, OutT, XIn>(MI355X_LIN_ARGS);
    case 2: return launch_linear_stream_t<2, OutT, XIn>(MI355X_LIN_ARGS);
    default: return launch_linear_stream_t<1, OutT, XIn>(MI355X_LIN_ARGS);
  }
#undef MI355X_LIN_ARGS
}

// RMSNorm + linear in one launch (stream_gemm_kernel with NORM), bf16 in and out.
template <int AF, int QT>
static int launch_norm_linear_q(const GemmPlan& p, const bf16_t* x, int64_t sxm, const NormArgs& na,
                                const uint8_t* w, int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk,
                                uint16_t* out, int64_t ldo, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  const int64_t kb = cdiv(K, kGroup);
  const bool ragged = p.rows != 16 * AF || 8 % AF != 0;
  // The fold buffer (8 token slots), the rows' 1 / rms, the norm weight and the M rows at
  // pitch K + 8.
  const size_t bytes = stream_fold_bytes(kb, AF, 1, ragged ? 2 : 1, 8) + 16 * sizeof(float) +
                       static_cast<size_t>(K + M * (K + 8)) * sizeof(uint16_t);
  // The rows staged in LDS take the buffer past the two-per-CU budget: one workgroup per CU
  // (a decode projection's stream grid holds about one per CU anyway) with all its LDS.
  if (bytes > kNormLds) return MI355X_FP8_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(cdiv(N, p.rows)), 1, 1);
  const uint8_t* xq = reinterpret_cast<const uint8_t*>(x);
  if (ragged)
    stream_gemm_kernel<1, AF, true, true, bf16_t, bf16_t, QT, true><<<grid, kStreamWaves * 64, bytes, stream>>>(
        xq, sxm, nullptr, 0, 0, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, kb, p.rows, na);
  else if constexpr (8 % AF == 0)
    stream_gemm_kernel<1, AF, true, false, bf16_t, bf16_t, QT, true><<<grid, kStreamWaves * 64, bytes, stream>>>(
        xq, sxm, nullptr, 0, 0, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, kb, p.rows, na);
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

template <int QT>
static int launch_norm_linear_af(const GemmPlan& p, const bf16_t* x, int64_t sxm, const NormArgs& na,
                                 const uint8_t* w, int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk,
                                 uint16_t* out, int64_t ldo, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
#define MI355X_NL_ARGS p, x, sxm, na, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, stream
  switch (p.row_tiles) {
    case 5: return launch_norm_linear_q<5, QT>(MI355X_NL_ARGS);
    case 4: return launch_norm_linear_q<4, QT>(MI355X_NL_ARGS);
    case 3: return launch_norm_linear_q<3, QT>(MI355X_NL_ARGS);
    case 2: return launch_norm_linear_q<2, QT>(MI355X_NL_ARGS);
    default: return launch_norm_linear_q<1, QT>(MI355X_NL_ARGS);
  }
#undef MI355X_NL_ARGS
}

int launch_norm_linear(const GemmPlan& plan, const uint16_t* x, int64_t sxm, const uint16_t* res, int64_t ldr,
                       uint16_t* res_out, int64_t ldro, const uint16_t* norm_w, float eps, const uint8_t* w,
                       int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, uint16_t* out, int64_t ldo,
                       int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  // One launch up to 8 rows (one lane-dense quantization pass), a row of at most 10 vectors
  // of 4 elements per lane (K % 256 == 0, K <= 2560), a reduction of at least 64 virtual
  // threads, 16-byte aligned rows throughout.
  const auto a16 = [](const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
  if (plan.kernel != MI355X_FP8_CONFIG_STREAM || plan.token_tiles != 1 || plan.rows < 1 || M < 1 || M > 8 ||
      N <= 0 || K % 256 != 0 || K / 256 > kNormMaxVec || sxm % 8 != 0 || ldw % 16 != 0 || !a16(x) || !a16(w) ||
      !a16(norm_w) || (res != nullptr && (ldr % 8 != 0 || !a16(res) || res_out == nullptr || ldro % 8 != 0 ||
                                           !a16(res_out))))
    return MI355X_FP8_ERR_UNSUPPORTED;
  const int bw = rmsnorm_block_width(M, K);
  if (bw < 64 || bw > 512 || bw % 64 != 0) return MI355X_FP8_ERR_UNSUPPORTED;
  NormArgs na;
  na.res = res;
  na.ldr = ldr;
  na.sum = res_out;
  na.lds = ldro;
  na.w = norm_w;
  na.eps = eps;
  na.inv_k = 1.0f / static_cast<float>(K);
  na.bw = bw;
  const bf16_t* xb = reinterpret_cast<const bf16_t*>(x);
  if (M <= 2) return launch_norm_linear_af<2>(plan, xb, sxm, na, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, stream);
  if (M <= 4) return launch_norm_linear_af<4>(plan, xb, sxm, na, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, stream);
  return launch_norm_linear_af<8>(plan, xb, sxm, na, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, stream);
}

// RMSNorm + gate/up GEMM + SiLU*up in one launch (stream_gemm_kernel with NORM and SILU):
// `rows` gate rows and as many up rows per workgroup, AF / 2 MFMA tiles each.
template <int AF, int QT>
static int launch_norm_silu_q(int rows, const bf16_t* x, int64_t sxm, const NormArgs& na, const uint8_t* w,
                              int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, uint16_t* h, int64_t ldh,
                              int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  const int64_t kb = cdiv(K, kGroup);
  const size_t bytes = stream_fold_bytes(kb, AF, 1, 4, 8) + 16 * sizeof(float) +
                       static_cast<size_t>(K + M * (K + 8)) * sizeof(uint16_t);
  if (bytes > kNormLds) return MI355X_FP8_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(cdiv(N / 2, rows)), 1, 1);
  stream_gemm_kernel<1, AF, true, true, bf16_t, bf16_t, QT, true, true><<<grid, kStreamWaves * 64, bytes, stream>>>(
      reinterpret_cast<const uint8_t*>(x), sxm, nullptr, 0, 0, w, ldw, ws, ws_sn, ws_sk, h, ldh, M, N, K, kb, rows,
      na);
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

template <int QT>
static int launch_norm_silu_af(int rows, const bf16_t* x, int64_t sxm, const NormArgs& na, const uint8_t* w,
                               int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, uint16_t* h, int64_t ldh,
                               int64_t M, int64_t N, int64_t K, hipStream_t stream) {
#define MI355X_NS_ARGS rows, x, sxm, na, w, ldw, ws, ws_sn, ws_sk, h, ldh, M, N, K, stream
  switch (cdiv(rows, 16)) {
    case 1: return launch_norm_silu_q<2, QT>(MI355X_NS_ARGS);
    case 2: return launch_norm_silu_q<4, QT>(MI355X_NS_ARGS);
    case 3: return launch_norm_silu_q<6, QT>(MI355X_NS_ARGS);
    default: return MI355X_FP8_ERR_UNSUPPORTED;
  }
#undef MI355X_NS_ARGS
}

int launch_norm_gate_up_silu(const uint16_t* x, int64_t sxm, const uint16_t* res, int64_t ldr, uint16_t* res_out,
                             int64_t ldro, const uint16_t* norm_w, float eps, const uint8_t* w, int64_t ldw,
                             const float* ws, int64_t ws_sn, int64_t ws_sk, uint16_t* h, int64_t ldh, int64_t M,
                             int64_t N, int64_t K, hipStream_t stream) {
  // The one-launch norm-linear's conditions (launch_norm_linear), an even N whose halves start
  // on a 16-byte row boundary, and h rows 4-byte aligned.
  const auto a16 = [](const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
  if (M < 1 || M > 8 || N <= 0 || N % 2 != 0 || K % 256 != 0 || K / 256 > kNormMaxVec || sxm % 8 != 0 ||
      ldw % 16 != 0 || !a16(x) || !a16(w) || !a16(norm_w) ||
      (res != nullptr && (ldr % 8 != 0 || !a16(res) || res_out == nullptr || ldro % 8 != 0 || !a16(res_out))))
    return MI355X_FP8_ERR_UNSUPPORTED;
  const int bw = rmsnorm_block_width(M, K);
  if (bw < 64 || bw > 512 || bw % 64 != 0) return MI355X_FP8_ERR_UNSUPPORTED;
  // One workgroup per CU: the same number of gate rows (and up rows) on every CU, at least
  // kStreamMinRows, at most three MFMA tiles of each.
  const int64_t cus = device_cus();
  const int64_t half = N / 2;
  const int64_t rows = cdiv(half, cus) > kStreamMinRows ? cdiv(half, cus) : kStreamMinRows;
  if (rows > 48 || cdiv(half, rows) > 0x7fffffffLL) return MI355X_FP8_ERR_UNSUPPORTED;
  NormArgs na;
  na.res = res;
  na.ldr = ldr;
  na.sum = res_out;
  na.lds = ldro;
  na.w = norm_w;
  na.eps = eps;
  na.inv_k = 1.0f / static_cast<float>(K);
  na.bw = bw;
  const bf16_t* xb = reinterpret_cast<const bf16_t*>(x);
  const int r = static_cast<int>(rows);
  if (M <= 2) return launch_norm_silu_af<2>(r, xb, sxm, na, w, ldw, ws, ws_sn, ws_sk, h, ldh, M, N, K, stream);
  if (M <= 4) return launch_norm_silu_af<4>(r, xb, sxm, na, w, ldw, ws, ws_sn, ws_sk, h, ldh, M, N, K, stream);
  return launch_norm_silu_af<8>(r, xb, sxm, na, w, ldw, ws, ws_sn, ws_sk, h, ldh, M, N, K, stream);
}

int launch_linear_stream(const GemmPlan& plan, const void* x, int x_dtype, int64_t sxm, int64_t sxk,
                         const uint8_t* w, int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, void* out,
                         int out_dtype, int64_t ldo, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  // One 16-token tile, and every load a whole aligned 16-byte piece: K % 16 == 0, unit
  // column stride, 16-byte aligned rows of x and W.
  if (plan.kernel != MI355X_FP8_CONFIG_STREAM || plan.token_tiles != 1 || M > 16 || M <= 0 || N <= 0 ||
      plan.rows < 1 || sxk != 1 || sxm % 8 != 0 || K % 16 != 0 || ldw % 16 != 0 ||
      reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(w) % 16 != 0)
    return MI355X_FP8_ERR_UNSUPPORTED;
  // Every workgroup reads and quantizes all of x, about 7 VALU instructions per element of
  // x: the quantization pays only while it hides behind the workgroup's own weight loads.
  // Up to 8 rows (the lane-dense quantization passes) that holds for every Qwen3-4B
  // projection, K = 9728 included.  Measured, one launch against quantizer + GEMM: at 8 rows
  // o_proj 8.77 -> 7.14 us, down 12.6 -> 11.8 us; at 1 row o_proj 7.95 -> 6.49 us, down
  // 11.0 -> 10.0 us.  At 9-16 rows the 16-token pass quantizes twice the elements per lane
  // and one launch pays only while x is the smaller read and a wave quantizes at most about
  // one and a half groups (qkv and gate_up, K = 2560: 1.3-1.9 us faster; down at 16 rows
  // 14.6 -> 18.5 us, o_proj 9.4 -> 9.9 us).
  const int64_t kgroups = cdiv(K, kGroup);
  if (M <= 8 ? kgroups > 80 : (2 * M > plan.rows || kgroups > 24)) return MI355X_FP8_ERR_UNSUPPORTED;
  uint16_t* o = static_cast<uint16_t*>(out);
  if (x_dtype == kBF16)
    return out_dtype == kBF16
               ? launch_linear_stream_x<bf16_t>(plan, static_cast<const bf16_t*>(x), sxm, w, ldw, ws, ws_sn, ws_sk, o,
                                                ldo, M, N, K, stream)
               : launch_linear_stream_x<f16_t>(plan, static_cast<const bf16_t*>(x), sxm, w, ldw, ws, ws_sn, ws_sk, o,
                                               ldo, M, N, K, stream);
  return out_dtype == kBF16
             ? launch_linear_stream_x<bf16_t>(plan, static_cast<const f16_t*>(x), sxm, w, ldw, ws, ws_sn, ws_sk, o,
                                              ldo, M, N, K, stream)
             : launch_linear_stream_x<f16_t>(plan, static_cast<const f16_t*>(x), sxm, w, ldw, ws, ws_sn, ws_sk, o,
                                             ldo, M, N, K, stream);
}

}  // namespace mi355x
