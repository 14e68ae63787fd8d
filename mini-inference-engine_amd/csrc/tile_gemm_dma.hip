// Prefill block-scaled FP8 GEMM, LDS-DMA pipelined variant (gfx950).
//
// Same arithmetic and lane layout as tile_gemm_kernel (block_gemm.hip): one
// v_mfma_f32_16x16x128_f8f6f4 per 128-wide K group and 16x16 output tile, folded into the
// fp32 accumulator as acc = fma(partial, a_s * w_s, acc); 128 x BN output tile per
// 256-thread workgroup (BN = 64, 128 or 160), 2x2 waves of 64 x BN/2.  BN = 160 gives the
// Qwen3-4B o_proj and down projections at M = 2048 exactly 256 tiles (16 x 16) instead
// of 320; a wave's columns may then straddle two 128-column weight-scale blocks, so each
// 16-column MFMA tile uses its own block's scale.
//
// What differs is the feed: global memory goes straight into LDS with
// global_load_lds_dwordx4 (no register staging, no ds_write), through a ring of STAGES
// stages (2 as launched, two workgroups per CU; 3 is kept as a template option), so the
// loads of K group kb+STAGES-1 are in flight while kb is multiplied.  Each stage
// holds the W tile (BN rows x 128 B), the activation tile (128 x 128 B) and the 128
// activation scales of its K group.  A 64-lane DMA instruction fills 1 KiB of LDS
// linearly (lane i -> byte 16 i), i.e. 8 rows of 8 16-byte chunks; the XOR swizzle
// (physical chunk p of row r holds logical chunk p ^ (r & 7)) is applied by choosing each
// lane's source address, so the MFMA fragment reads (ds_read_b128) are bank-conflict free.
//
// The stages are distinct LDS objects and the K loop is unrolled by STAGES, so the
// compiler can tell the stages apart and does not wait for in-flight DMA before reading
// the current stage; the waits are explicit (vmcnt) before each workgroup barrier.
//
// Preconditions (checked by the launcher): K % 128 == 0, W/q base pointers and leading
// dimensions 16-byte aligned, activation scales K-group-major (as_sm == 1) with row
// length as_sk >= M.  Out-of-range tile rows read the last valid row (finite data whose
// outputs are never stored).
#include "fp8_abi_internal.h"
#include "fp8_common.h"

namespace mi355x {
namespace {

constexpr int kDmaThreads = 256;
#ifndef MI355X_DMA_STAGES_FEW
#define MI355X_DMA_STAGES_FEW 3  // ring depth when the tiles do not exceed the CUs
#endif
#ifndef MI355X_DMA_STAGES_MANY
#define MI355X_DMA_STAGES_MANY 2  // ring depth otherwise (two workgroups per CU)
#endif
constexpr int kTileRows = 128;                          // activation rows per tile
constexpr int kMaxBN = 160;                             // widest W tile (columns of the output tile)
constexpr int kStageChunks = (kMaxBN + kTileRows) * 8 + 64;  // W tile, X tile, 4 x 64 scales (uint4 units)

// Tile geometry for width BN (128 or 160): stage layout [W tile | X tile | scales].
template <int BN>
struct DmaGeo {
  static_assert(BN == 64 || BN == 128 || BN == 160, "tile width");
  static constexpr int kNI = BN / 32;                  // 16-column MFMA tiles per wave (2 x 2 waves)
  static constexpr int kXOff = BN * 8;                 // uint4 offset of the activation tile
  static constexpr int kScaleOff = (BN + kTileRows) * 8;
  static constexpr int kDmaPerStage = BN / 32 + 4 + 1;  // DMA instructions per wave per stage
};

__shared__ uint4 stage0[kStageChunks];
__shared__ uint4 stage1[kStageChunks];
__shared__ uint4 stage2[kStageChunks];
__shared__ uint4 stage3[kStageChunks];

typedef __attribute__((address_space(3))) void lds_void_t;
typedef const __attribute__((address_space(1))) void global_void_t;

__device__ __forceinline__ void dma16(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds((global_void_t*)(src),
                                   (lds_void_t*)(lds_dst), 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds((global_void_t*)(src),
                                   (lds_void_t*)(lds_dst), 4, 0, 0);
}

// s_waitcnt with vmcnt = N (6 bits: 3:0 and 15:14) and lgkmcnt = 0, expcnt left at its maximum.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}

__device__ __forceinline__ void tile_of_dma(int64_t pid, int64_t tiles_m, int64_t tiles_n, int64_t* tm,
                                            int64_t* tn) {
  constexpr int64_t kGroupTiles = 8;
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

struct DmaSources {
  const uint8_t* w[5];
  const uint8_t* x[4];
  const float* as;
  const float* ws_a;  // weight scales of the (at most two) 128-column blocks the wave's columns touch
  const float* ws_b;
  uint32_t use_b;     // bit i: the wave's column tile i lies in block ws_b
};

template <int S>
__device__ __forceinline__ uint4* stage_ptr() {
  if constexpr (S == 0) return stage0;
  else if constexpr (S == 1) return stage1;
  else if constexpr (S == 2) return stage2;
  else return stage3;
}

template <int BN, int S>
__device__ __forceinline__ void issue_stage(const DmaSources& src, int64_t kb, int64_t as_sk, int wave, int lane) {
  using G = DmaGeo<BN>;
  uint4* st = stage_ptr<S>();
  const int64_t koff = kb * kGroup;
#pragma unroll
  for (int i = 0; i < G::kNI; ++i) dma16(src.w[i] + koff, st + (i * 4 + wave) * 64);
#pragma unroll
  for (int i = 0; i < 4; ++i) dma16(src.x[i] + koff, st + G::kXOff + (i * 4 + wave) * 64);
  dma4(src.as + kb * as_sk, reinterpret_cast<float*>(st + G::kScaleOff) + wave * 64);
}

template <int BN, int S>
__device__ __forceinline__ void compute_stage(v4f (&acc)[DmaGeo<BN>::kNI][4], float wa, float wb, uint32_t use_b,
                                              int wm, int wn, int r, int g) {
  using G = DmaGeo<BN>;
  constexpr int NI = G::kNI;
  const uint4* st = stage_ptr<S>();
  const float* sc_lds = reinterpret_cast<const float*>(st + G::kScaleOff);
  float as_v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) as_v[j] = sc_lds[wm * 64 + 16 * j + r];  // region wm: rows 64 wm ..
  v8i a[NI], b[4];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int row = wn * (BN / 2) + 16 * i + r;
    a[i] = pack_v8i(st[row * 8 + (g ^ (row & 7))], st[row * 8 + ((g + 4) ^ (row & 7))]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = wm * 64 + 16 * j + r;
    b[j] = pack_v8i(st[G::kXOff + row * 8 + (g ^ (row & 7))], st[G::kXOff + row * 8 + ((g + 4) ^ (row & 7))]);
  }
  // 4 NI independent MFMAs into as many partial tiles, each folded into the accumulator
  // once it is done; the scheduling groups interleave the folds of earlier tiles with the
  // issue of later MFMAs so that the matrix core never waits on the VALU.
  v4f p[NI * 4];
#pragma unroll
  for (int t = 0; t < NI * 4; ++t) p[t] = mfma_16x16x128_e4m3(a[t >> 2], b[t & 3]);
#pragma unroll
  for (int t = 0; t < NI * 4; ++t) {
    const float sc = as_v[t & 3] * ((use_b >> (t >> 2)) & 1 ? wb : wa);
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[t >> 2][t & 3][v] = __builtin_fmaf(p[t][v], sc, acc[t >> 2][t & 3][v]);
  }
#pragma unroll
  for (int t = 0; t < NI * 4; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // four VALU
  }
}

// One K group: wait for its stage, barrier, refill the stage two groups ahead, multiply.
// The refill is unconditional (past the end it reloads the last K group into a stage that
// is no longer read), so every wave always has exactly kDmaPerStage DMA instructions per
// stage in flight and the waits are static.
template <int BN, int STAGES, int CUR>
__device__ __forceinline__ void k_step(v4f (&acc)[DmaGeo<BN>::kNI][4], const DmaSources& src, int64_t kb, int64_t KB,
                                       int64_t as_sk, int64_t ws_sk, int wave, int lane, int wm, int wn, int r,
                                       int g) {
  constexpr int NXT = (CUR + STAGES - 1) % STAGES;
  wait_vm_lgkm0<DmaGeo<BN>::kDmaPerStage * (STAGES - 2)>();
  __builtin_amdgcn_s_barrier();
  const int64_t ahead = kb + STAGES - 1;
  issue_stage<BN, NXT>(src, ahead < KB ? ahead : KB - 1, as_sk, wave, lane);
  if (kb < KB) compute_stage<BN, CUR>(acc, src.ws_a[kb * ws_sk], src.ws_b[kb * ws_sk], src.use_b, wm, wn, r, g);
  // Keep this step's MFMAs ahead of the next step's wait and barrier, so the matrix core
  // works through them while the wave waits (measured 6 % faster on o_proj and down).
  __builtin_amdgcn_sched_barrier(0);
}

template <int STAGES, int BN, typename OutT>
__global__ __launch_bounds__(kDmaThreads, STAGES == 2 ? 2 : 1) void tile_gemm_dma_kernel(
    const uint8_t* __restrict__ q, int64_t ldq, const float* __restrict__ as, int64_t as_sk,
    const uint8_t* __restrict__ w, int64_t ldw, const float* __restrict__ ws, int64_t ws_sn,
    int64_t ws_sk, uint16_t* __restrict__ out, int64_t ldo, int64_t M, int64_t N, int64_t KB,
    int64_t tiles_m, int64_t tiles_n, int vec_out) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int wm = wave & 1;
  const int wn = wave >> 1;
  int64_t tm, tn;
  tile_of_dma(blockIdx.x, tiles_m, tiles_n, &tm, &tn);
  using G = DmaGeo<BN>;
  constexpr int NI = G::kNI;
  const int64_t m0 = tm * kTileRows;
  const int64_t n0 = tn * BN;

  DmaSources src;
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int rr = (i * 4 + wave) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ (rr & 7);
    const int64_t wrow = (n0 + rr) < N ? (n0 + rr) : (N - 1);
    src.w[i] = i < NI ? w + wrow * ldw + 16 * c : w;
    if (i < 4) {
      const int64_t xrow = (m0 + rr) < M ? (m0 + rr) : (M - 1);
      src.x[i] = q + xrow * ldq + 16 * c;
    }
  }
  {
    // Wave w stages the scales of tile rows 64 (w & 1) .. +63 (waves 2, 3 duplicate 0, 1).
    const int64_t srow = m0 + (wave & 1) * 64 + lane;
    src.as = as + (srow < M ? srow : M - 1);
  }
  {
    // The wave's columns [nw, nw + BN/2) touch at most two 128-column weight-scale blocks.
    const int64_t nw = n0 + wn * (BN / 2);
    const int64_t last_blk = (N - 1) / kGroup;
    const int64_t blk_a = nw / kGroup < last_blk ? nw / kGroup : last_blk;
    const int64_t blk_b = blk_a + 1 < last_blk ? blk_a + 1 : last_blk;
    src.ws_a = ws + blk_a * ws_sn;
    src.ws_b = ws + blk_b * ws_sn;
    uint32_t use_b = 0;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      if ((nw + 16 * i) / kGroup != nw / kGroup) use_b |= 1u << i;
    src.use_b = use_b;
  }

  v4f acc[NI][4];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  static_assert(STAGES >= 2 && STAGES <= 4, "stages");
  issue_stage<BN, 0>(src, 0, as_sk, wave, lane);
  if constexpr (STAGES >= 3) issue_stage<BN, 1>(src, KB > 1 ? 1 : KB - 1, as_sk, wave, lane);
  if constexpr (STAGES >= 4) issue_stage<BN, 2>(src, KB > 2 ? 2 : KB - 1, as_sk, wave, lane);
  for (int64_t kb = 0; kb < KB; kb += STAGES) {
    k_step<BN, STAGES, 0>(acc, src, kb, KB, as_sk, ws_sk, wave, lane, wm, wn, r, g);
    k_step<BN, STAGES, 1>(acc, src, kb + 1, KB, as_sk, ws_sk, wave, lane, wm, wn, r, g);
    if constexpr (STAGES >= 3) k_step<BN, STAGES, 2>(acc, src, kb + 2, KB, as_sk, ws_sk, wave, lane, wm, wn, r, g);
    if constexpr (STAGES >= 4) k_step<BN, STAGES, 3>(acc, src, kb + 3, KB, as_sk, ws_sk, wave, lane, wm, wn, r, g);
  }
  wait_vm_lgkm0<0>();  // no DMA may still target LDS when the workgroup ends

  // Lane holds out[m = m0 + 64 wm + 16 j + r][n = n0 + BN/2 wn + 16 i + 4 g + v].
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t m = m0 + wm * 64 + 16 * j + r;
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int64_t n = n0 + wn * (BN / 2) + 16 * i + 4 * g;
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

}  // namespace

bool tile_dma_supported(const uint8_t* q, int64_t ldq, int64_t as_sm, int64_t as_sk, const uint8_t* w,
                        int64_t ldw, int64_t M, int64_t K) {
  return K % kGroup == 0 && ldq % 16 == 0 && ldw % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(w) % 16 == 0 && as_sm == 1 && as_sk >= M;
}

int launch_tile_dma(const uint8_t* q, int64_t ldq, const float* as, int64_t as_sk, const uint8_t* w,
                    int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, void* out, int out_dtype,
                    int64_t ldo, int64_t M, int64_t N, int64_t K, int bn, hipStream_t stream) {
  if (bn != 64 && bn != 128 && bn != 160) return MI355X_FP8_ERR_INVALID;
  const int64_t tiles_m = (M + kTileRows - 1) / kTileRows;
  const int64_t tiles_n = (N + bn - 1) / bn;
  if (tiles_m * tiles_n > 0x7fffffffLL) return MI355X_FP8_ERR_UNSUPPORTED;
  const int vec_out = (ldo % 4) == 0 && (reinterpret_cast<uintptr_t>(out) % 8) == 0;
  dim3 grid(static_cast<unsigned>(tiles_m * tiles_n));
  uint16_t* o = static_cast<uint16_t*>(out);
  // Two stages (76 KiB, room for the 160-wide W tile) let two workgroups share a CU.
  // When the tiles do not fill the CUs anyway, each K step waits on its DMA round trip,
  // so a deeper ring (one workgroup per CU) keeps more K groups in flight.
  const int stages = tiles_m * tiles_n <= device_cus() ? MI355X_DMA_STAGES_FEW : MI355X_DMA_STAGES_MANY;
#define MI355X_DMA_ARGS q, ldq, as, as_sk, w, ldw, ws, ws_sn, ws_sk, o, ldo, M, N, K / kGroup, tiles_m, tiles_n, vec_out
#define MI355X_DMA_LAUNCH(ST, BN)                                                                                  \
  (out_dtype == kBF16 ? tile_gemm_dma_kernel<ST, BN, bf16_t><<<grid, kDmaThreads, 0, stream>>>(MI355X_DMA_ARGS) \
                      : tile_gemm_dma_kernel<ST, BN, f16_t><<<grid, kDmaThreads, 0, stream>>>(MI355X_DMA_ARGS))
#define MI355X_DMA_BY_BN(ST)                \
  do {                                      \
    if (bn == 160) MI355X_DMA_LAUNCH(ST, 160); \
    else if (bn == 64) MI355X_DMA_LAUNCH(ST, 64); \
    else MI355X_DMA_LAUNCH(ST, 128);        \
  } while (0)
  if (stages == MI355X_DMA_STAGES_MANY) MI355X_DMA_BY_BN(MI355X_DMA_STAGES_MANY);
  else MI355X_DMA_BY_BN(MI355X_DMA_STAGES_FEW);
#undef MI355X_DMA_BY_BN
#undef MI355X_DMA_LAUNCH
#undef MI355X_DMA_ARGS
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

}  // namespace mi355x
