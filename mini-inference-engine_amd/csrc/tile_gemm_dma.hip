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
// stages (2 when two workgroups share a CU; when the tiles do not fill the CUs, 3, or 4 for
// BN = 64).  Each stage holds the W tile (BN rows x 128 B), the activation tile
// (128 x 128 B) and the 128 activation scales of its K group.  A 64-lane DMA instruction fills 1 KiB of LDS
// linearly (lane i -> byte 16 i), i.e. 8 rows of 8 16-byte chunks; the XOR swizzle
// (physical chunk p of row r holds logical chunk p ^ (r & 7)) is applied by choosing each
// lane's source address, so the MFMA fragment reads (ds_read_b128) are bank-conflict free.
//
// With one wave per SIMD nothing else hides a wave's LDS reads, so each K step is
// software-pipelined (k_step): the fragments its first MFMAs need are read during the
// previous step, each later weight fragment is read while the MFMAs of the one before run,
// and the workgroup barrier sits between the two parts of a step rather than in front of
// it.  The K loop is unrolled by STAGES so that every stage index is a compile-time
// constant.
//
// The output tile leaves through LDS as full-row 16-byte non-temporal stores when the output
// rows are 16-byte aligned (staged_index, fp8_common.h), else straight from the registers.
//
// Preconditions (checked by the launcher): K % 128 == 0, W/q base pointers and leading
// dimensions 16-byte aligned, activation scales K-group-major (as_sm == 1) with row
// length as_sk >= M, row strides below 2^32 / 159 bytes (W) and 2^32 / 127 bytes (q), so that
// the 32-bit per-lane offsets within a tile reach every row.  Out-of-range tile rows read the
// last valid row (finite data whose outputs are never stored).
#include "fp8_abi_internal.h"
#include "fp8_common.h"

namespace mi355x {
namespace {

constexpr int kDmaThreads = 256;
#ifndef MI355X_DMA_STAGES_FEW
#define MI355X_DMA_STAGES_FEW 3  // ring depth when the tiles do not exceed the CUs
#endif
#ifndef MI355X_DMA_STAGES_FEW_NARROW
#define MI355X_DMA_STAGES_FEW_NARROW 4  // the same for the 64-wide tiles
#endif
#ifndef MI355X_DMA_STAGES_MANY
#define MI355X_DMA_STAGES_MANY 2  // ring depth otherwise (two workgroups per CU)
#endif
constexpr int kTileRows = 128;                          // activation rows per tile
constexpr int kMaxBN = 160;                             // widest W tile (columns of the output tile)

// Tile geometry for width BN (64, 128 or 160) and J 16-row activation fragments per wave
// (tile rows 32 J: 128 for J = 4, 64 for J = 2): stage layout [W tile | X tile | scales].
template <int BN, int J = 4>
struct DmaGeo {
  static_assert(BN == 64 || BN == 128 || BN == 160, "tile width");
  static_assert(J == 4 || J == 2, "tile rows");
  static constexpr int kNI = BN / 32;                  // 16-column MFMA tiles per wave (2 x 2 waves)
  static constexpr int kRows = 32 * J;                 // activation rows of the tile
  static constexpr int kXOff = BN * 8;                 // uint4 offset of the activation tile
  static constexpr int kScaleOff = (BN + kRows) * 8;
  static constexpr int kDmaPerStage = BN / 32 + J + 1;  // DMA instructions per wave per stage
  static constexpr int kStageU4 = (BN + kRows) * 8 + 64;  // one stage, in uint4
};


typedef __attribute__((address_space(3))) void lds_void_t;

// The DMA instructions are issued through inline assembly.  The compiler then does not
// track them, so it adds no waits of its own before LDS reads; its alias tracking of LDS
// DMA is not precise enough for this ring and put vmcnt(0) (every load in flight) in front
// of fragment reads of a stage whose data had long arrived, and lgkmcnt(0) in front of
// every MFMA.  All waits for the DMA are the explicit vmcnt waits before the workgroup
// barriers.  M0 is written without being declared clobbered (it is a reserved register):
// nothing else in this kernel uses M0, as every LDS DMA of it goes through these helpers.
// SALU writes of M0 need one wait state before an LDS DMA reads it (the s_nop).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)(p)));
}
// 16 (dma16) or 4 (dma4) bytes per lane from base + off: a 64-bit uniform base in SGPRs and
// a 32-bit per-lane offset, so the K loop spends no VALU on addresses.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, void* lds_dst) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base),
               "s"(lds_addr(lds_dst))
               : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, void* lds_dst) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base),
               "s"(lds_addr(lds_dst))
               : "memory");
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
  const uint8_t* w;   // W row n0 of the tile
  const uint8_t* x;   // activation row m0 of the tile
  const float* as;    // activation scale of row m0, K group 0
  uint32_t woff[5];   // per-lane byte offsets from w of the W rows each DMA instruction fills
  uint32_t xoff[4];   // the same for the activation rows, from x (J of them)
  uint32_t soff;      // per-lane byte offset from as of the scale this lane stages
  const float* ws_a;  // weight scales of the (at most two) 128-column blocks the wave's columns touch
  const float* ws_b;
  uint32_t use_b;     // bit i: the wave's column tile i lies in block ws_b
};

// The ring: STAGES stages of DmaGeo<BN>::kStageU4 each, in the kernel's own LDS array (sized
// per instantiation, so the two-stage form still fits two workgroups per CU).
template <int BN, int S, int J = 4>
__device__ __forceinline__ uint4* stage_ptr(uint4* ring) {
  return ring + S * DmaGeo<BN, J>::kStageU4;
}

// DMA instruction d (0 .. kDmaPerStage-1) of a stage: W rows, then X rows, then scales.
template <int BN, int S, int J = 4>
__device__ __forceinline__ void issue_one(uint4* ring, const DmaSources& src, int64_t kb, int64_t as_sk, int wave,
                                          int d) {
  using G = DmaGeo<BN, J>;
  uint4* st = stage_ptr<BN, S, J>(ring);
  const int64_t koff = kb * kGroup;
  if (d < G::kNI) dma16(src.w + koff, src.woff[d], st + (d * 4 + wave) * 64);
  else if (d < G::kNI + J) dma16(src.x + koff, src.xoff[d - G::kNI], st + G::kXOff + ((d - G::kNI) * 4 + wave) * 64);
  else dma4(src.as + kb * as_sk, src.soff, reinterpret_cast<float*>(st + G::kScaleOff) + wave * 64);
}

template <int BN, int S, int J = 4>
__device__ __forceinline__ void issue_stage(uint4* ring, const DmaSources& src, int64_t kb, int64_t as_sk, int wave) {
#pragma unroll
  for (int d = 0; d < DmaGeo<BN, J>::kDmaPerStage; ++d) issue_one<BN, S, J>(ring, src, kb, as_sk, wave, d);
}

// What the first MFMAs of a K step need, read from its stage one step early: the four
// activation fragments, the first weight fragment, the activation scales and the weight
// scales of the K group.
template <int BN, int J = 4>
struct StepHead {
  v8i b[J];
  v8i a0;
  float as_v[J];
  float wa, wb;
};

template <int BN, int S, int J = 4>
__device__ __forceinline__ v8i read_a(const uint4* ring, int i, int wn, int r, int g) {
  const uint4* st = ring + S * DmaGeo<BN, J>::kStageU4;
  const int row = wn * (BN / 2) + 16 * i + r;
  return pack_v8i(st[row * 8 + (g ^ (row & 7))], st[row * 8 + ((g + 4) ^ (row & 7))]);
}

template <int BN, int S, int J = 4>
__device__ __forceinline__ void read_head(const uint4* ring, StepHead<BN, J>& h, const DmaSources& src, int64_t kb,
                                          int64_t ws_sk, int wm, int wn, int r, int g) {
  using G = DmaGeo<BN, J>;
  const uint4* st = ring + S * G::kStageU4;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int row = wm * 16 * J + 16 * j + r;
    h.b[j] = pack_v8i(st[G::kXOff + row * 8 + (g ^ (row & 7))], st[G::kXOff + row * 8 + ((g + 4) ^ (row & 7))]);
  }
  h.a0 = read_a<BN, S, J>(ring, 0, wn, r, g);
  const float* sc_lds = reinterpret_cast<const float*>(st + G::kScaleOff);
#pragma unroll
  for (int j = 0; j < J; ++j) h.as_v[j] = sc_lds[wm * 16 * J + 16 * j + r];
  h.wa = src.ws_a[kb * ws_sk];
  h.wb = src.ws_b[kb * ws_sk];
}

// Folds column tile i's partials into the accumulator: acc = fma(p, as * ws, acc), ws being
// the scale of the 128-column weight block the tile lies in.  Only BN = 160 lets a wave's
// tiles straddle two blocks; the step forms both blocks' four products once (sa, sb), and each
// tile picks its block's set on the scalar unit.
template <int BN, int J = 4>
__device__ __forceinline__ void fold_tile(v4f (&acc)[BN / 32][J], const v4f (&p)[J], const float (&sa)[J],
                                          const float (&sb)[J], uint32_t use_b, int i) {
  const bool ub = BN == 160 && ((use_b >> i) & 1);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const float sc = ub ? sb[j] : sa[j];
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(p[j][v], sc, acc[i][j][v]);
  }
}

// One K group kb from stage CUR, whose head h was read during the previous step.
//   A: weight fragments 0 .. NA-1 are multiplied while fragment i+1 is read;
//   then the rest of the stage's fragments are read, and the wave waits for them and for
//   the DMA of the next stage, and passes the workgroup barrier;
//   B: the next step's head is read from stage CUR+1, stage CUR (now read by every wave)
//   is refilled with K group kb+STAGES, and the last weight fragments are multiplied.
// The LDS reads of each part so run behind MFMAs that do not depend on them.  Every
// output element is still folded once per K group, in K order.
template <int BN, int STAGES, int CUR, int J = 4>
__device__ __forceinline__ void k_step(uint4* ring, v4f (&acc)[BN / 32][J], StepHead<BN, J>& h, const DmaSources& src,
                                       int64_t kb, int64_t KB, int64_t as_sk, int64_t ws_sk, int wave, int wm,
                                       int wn, int r, int g) {
  using G = DmaGeo<BN, J>;
  constexpr int NI = G::kNI;
  constexpr int NB = NI >= 4 ? 2 : 1;  // weight fragments multiplied after the barrier
  constexpr int NA = NI - NB;
  constexpr int NXT = (CUR + 1) % STAGES;
  float sa[J], sb[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    sa[j] = h.as_v[j] * h.wa;
    sb[j] = BN == 160 ? h.as_v[j] * h.wb : sa[j];
  }
  v8i a[NI];
  a[0] = h.a0;
  v4f p[NI][J];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
#pragma unroll
    for (int j = 0; j < J; ++j) p[i][j] = mfma_16x16x128_e4m3(a[i], h.b[j]);
    a[i + 1] = read_a<BN, CUR, J>(ring, i + 1, wn, r, g);
    if (i > 0) fold_tile<BN, J>(acc, p[i - 1], sa, sb, src.use_b, i - 1);
  }
#pragma unroll
  for (int i = NA + 1; i < NI; ++i) a[i] = read_a<BN, CUR, J>(ring, i, wn, r, g);
  // Per weight fragment of part A: its first MFMA, the two reads of the next fragment
  // (so that the wait before this MFMA covers only the fragment it needs), then the other
  // three MFMAs, each followed by folds of the fragment before.
#pragma unroll
  for (int i = 0; i < (J == 4 ? NA : 0); ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  wait_vm_lgkm0<G::kDmaPerStage * (STAGES - 2)>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  StepHead<BN, J> nh;
  read_head<BN, NXT, J>(ring, nh, src, kb + 1 < KB ? kb + 1 : KB - 1, ws_sk, wm, wn, r, g);
  const int64_t ahead = kb + STAGES < KB ? kb + STAGES : KB - 1;
  // The refill's DMA instructions are spread over the MFMAs of part B.
  constexpr int ND = G::kDmaPerStage, NM = J * NB;
#pragma unroll
  for (int t = 0; t < NM; ++t) {
    const int i = NA + t / J, j = t % J;
    p[i][j] = mfma_16x16x128_e4m3(a[i], h.b[j]);
#pragma unroll
    for (int d = t * ND / NM; d < (t + 1) * ND / NM; ++d) issue_one<BN, CUR, J>(ring, src, ahead, as_sk, wave, d);
    if (j == J - 1 && i > 0) fold_tile<BN, J>(acc, p[i - 1], sa, sb, src.use_b, i - 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  fold_tile<BN, J>(acc, p[NI - 1], sa, sb, src.use_b, NI - 1);
  __builtin_amdgcn_sched_barrier(0);
  h = nh;
}

template <int STAGES, int BN, typename OutT, int J = 4>
__global__ __launch_bounds__(kDmaThreads, STAGES == 2 ? 2 : 1) void tile_gemm_dma_kernel(
    const uint8_t* __restrict__ q, int64_t ldq, const float* __restrict__ as, int64_t as_sk,
    const uint8_t* __restrict__ w, int64_t ldw, const float* __restrict__ ws, int64_t ws_sn,
    int64_t ws_sk, uint16_t* __restrict__ out, int64_t ldo, int64_t M, int64_t N, int64_t KB,
    int64_t tiles_m, int64_t tiles_n, int vec_out) {
  __shared__ uint4 ring[STAGES * DmaGeo<BN, J>::kStageU4];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int wm = wave & 1;
  const int wn = wave >> 1;
  int64_t tm, tn;
  tile_of_dma(blockIdx.x, tiles_m, tiles_n, &tm, &tn);
  using G = DmaGeo<BN, J>;
  constexpr int NI = G::kNI;
  const int64_t m0 = tm * G::kRows;
  const int64_t n0 = tn * BN;

  DmaSources src;
  src.w = w + n0 * ldw;
  src.x = q + m0 * ldq;
  src.as = as + m0;
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int rr = (i * 4 + wave) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ (rr & 7);
    const int64_t wrow = (n0 + rr) < N ? rr : (N - 1 - n0);
    src.woff[i] = static_cast<uint32_t>(wrow * ldw + 16 * c);
    if (i < J) {
      const int64_t xrow = (m0 + rr) < M ? rr : (M - 1 - m0);
      src.xoff[i] = static_cast<uint32_t>(xrow * ldq + 16 * c);
    }
  }
  {
    // Wave w stages the scales of tile rows 64 (w & 1) .. +63 (waves 2, 3 duplicate 0, 1); a
    // 64-row tile's are staged by every wave alike.
    const int64_t srow = (J == 4 ? (wave & 1) * 64 : 0) + lane;
    src.soff = static_cast<uint32_t>(4 * (m0 + srow < M ? srow : M - 1 - m0));
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

  v4f acc[NI][J];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  static_assert(STAGES >= 2 && STAGES <= 6, "stages");
  issue_stage<BN, 0, J>(ring, src, 0, as_sk, wave);
  issue_stage<BN, 1, J>(ring, src, KB > 1 ? 1 : KB - 1, as_sk, wave);
  if constexpr (STAGES >= 3) issue_stage<BN, 2, J>(ring, src, KB > 2 ? 2 : KB - 1, as_sk, wave);
  if constexpr (STAGES >= 4) issue_stage<BN, 3, J>(ring, src, KB > 3 ? 3 : KB - 1, as_sk, wave);
  if constexpr (STAGES >= 5) issue_stage<BN, 4, J>(ring, src, KB > 4 ? 4 : KB - 1, as_sk, wave);
  if constexpr (STAGES >= 6) issue_stage<BN, 5, J>(ring, src, KB > 5 ? 5 : KB - 1, as_sk, wave);
  wait_vm_lgkm0<G::kDmaPerStage * (STAGES - 1)>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  StepHead<BN, J> h;
  read_head<BN, 0, J>(ring, h, src, 0, ws_sk, wm, wn, r, g);
  int64_t kb = 0;
#define MI355X_KSTEP(S, KBV) k_step<BN, STAGES, S, J>(ring, acc, h, src, KBV, KB, as_sk, ws_sk, wave, wm, wn, r, g)
  for (; kb + STAGES <= KB; kb += STAGES) {
    MI355X_KSTEP(0, kb);
    MI355X_KSTEP(1, kb + 1);
    if constexpr (STAGES >= 3) MI355X_KSTEP(2, kb + 2);
    if constexpr (STAGES >= 4) MI355X_KSTEP(3, kb + 3);
    if constexpr (STAGES >= 5) MI355X_KSTEP(4, kb + 4);
    if constexpr (STAGES >= 6) MI355X_KSTEP(5, kb + 5);
  }
  // The last KB % STAGES groups.
  if (kb < KB) MI355X_KSTEP(0, kb);
  if constexpr (STAGES >= 3)
    if (kb + 1 < KB) MI355X_KSTEP(1, kb + 1);
  if constexpr (STAGES >= 4)
    if (kb + 2 < KB) MI355X_KSTEP(2, kb + 2);
  if constexpr (STAGES >= 5)
    if (kb + 3 < KB) MI355X_KSTEP(3, kb + 3);
  if constexpr (STAGES >= 6)
    if (kb + 4 < KB) MI355X_KSTEP(4, kb + 4);
#undef MI355X_KSTEP
  wait_vm_lgkm0<0>();  // no DMA may still target LDS when the workgroup ends

  if (vec_out == 2) {
    // Through LDS (staged_index, fp8_common.h): the tile's first 16 J rows in stage0, the
    // others in stage1.
    constexpr int kHalf = 16 * J;
    static_assert(kHalf * staged_pitch<BN>() * 2 <= G::kStageU4 * 16, "staged rows fit a stage");
    __syncthreads();  // every wave is done with the ring
    uint4* const stage0 = stage_ptr<BN, 0, J>(ring);
    uint4* const stage1 = stage_ptr<BN, 1, J>(ring);
    uint16_t* reg = reinterpret_cast<uint16_t*>(wm == 0 ? stage0 : stage1);
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        uint16_t h[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) h[v] = OutCvt<OutT>::cvt(acc[i][j][v]);
        *reinterpret_cast<uint2*>(reg + staged_index<BN>(16 * j + r, wn * (BN / 2) + 16 * i + 4 * g)) =
            make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16));
      }
    }
    __syncthreads();
    constexpr int C = BN / 8;  // 16-byte pieces per row
    static_assert((G::kRows * C) % kDmaThreads == 0, "whole passes");
#pragma unroll
    for (int it = 0; it < G::kRows * C / kDmaThreads; ++it) {
      const int idx = tid + it * kDmaThreads;
      const int row = idx / C, c = idx - (idx / C) * C;
      const int64_t m = m0 + row, n = n0 + 8 * c;
      const uint16_t* reg_r = reinterpret_cast<const uint16_t*>(row < kHalf ? stage0 : stage1);
      const uint4 val = *reinterpret_cast<const uint4*>(reg_r + staged_index<BN>(row % kHalf, 8 * c));
      if (m >= M) continue;
      uint16_t* dst = out + m * ldo + n;
      if (n + 8 <= N) {
        store16_nt(dst, val);
      } else {
        const uint16_t* hv = reinterpret_cast<const uint16_t*>(&val);
        for (int v = 0; v < 8; ++v)
          if (n + v < N) dst[v] = hv[v];
      }
    }
    return;
  }

  // Lane holds out[m = m0 + 16 J wm + 16 j + r][n = n0 + BN/2 wn + 16 i + 4 g + v].
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int64_t m = m0 + wm * 16 * J + 16 * j + r;
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
  // The per-lane DMA offsets within a tile are 32-bit (the row bases are 64-bit).
  constexpr int64_t kMaxOff = 0xffffffffLL - kGroup;
  if (ldq > kMaxOff / (kTileRows - 1) || ldw > kMaxOff / (kMaxBN - 1)) return false;
  return K % kGroup == 0 && ldq % 16 == 0 && ldw % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(w) % 16 == 0 && as_sm == 1 && as_sk >= M;
}

int launch_tile_dma(const uint8_t* q, int64_t ldq, const float* as, int64_t as_sk, const uint8_t* w,
                    int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, void* out, int out_dtype,
                    int64_t ldo, int64_t M, int64_t N, int64_t K, int bn, int rows, hipStream_t stream) {
  if (bn != 64 && bn != 128 && bn != 160) return MI355X_FP8_ERR_INVALID;
  if (rows != 128 && (rows != 64 || bn == 160)) return MI355X_FP8_ERR_INVALID;
  const int64_t tiles_m = (M + rows - 1) / rows;
  const int64_t tiles_n = (N + bn - 1) / bn;
  if (tiles_m * tiles_n > 0x7fffffffLL) return MI355X_FP8_ERR_UNSUPPORTED;
  const int vec_out = out_vec_mode(out, ldo);
  dim3 grid(static_cast<unsigned>(tiles_m * tiles_n));
  uint16_t* o = static_cast<uint16_t*>(out);
  // Two stages (76 KiB, room for the 160-wide W tile) let two workgroups share a CU.
  // When the tiles do not fill the CUs anyway, each K step waits on its DMA round trip,
  // so a deeper ring (one workgroup per CU) keeps more K groups in flight: three stages,
  // four for the 64-wide tiles, whose short steps wait longest (measured on o_proj and down
  // at 256 and 536 rows; four stages for the wider tiles measured slower).
  const bool few = tiles_m * tiles_n <= device_cus();
#define MI355X_DMA_ARGS q, ldq, as, as_sk, w, ldw, ws, ws_sn, ws_sk, o, ldo, M, N, K / kGroup, tiles_m, tiles_n, vec_out
#define MI355X_DMA_LAUNCH(ST, BN)                                                                                  \
  (out_dtype == kBF16 ? tile_gemm_dma_kernel<ST, BN, bf16_t><<<grid, kDmaThreads, 0, stream>>>(MI355X_DMA_ARGS) \
                      : tile_gemm_dma_kernel<ST, BN, f16_t><<<grid, kDmaThreads, 0, stream>>>(MI355X_DMA_ARGS))
#define MI355X_DMA_LAUNCH64(ST, BN)                                                                                   \
  (out_dtype == kBF16 ? tile_gemm_dma_kernel<ST, BN, bf16_t, 2><<<grid, kDmaThreads, 0, stream>>>(MI355X_DMA_ARGS) \
                      : tile_gemm_dma_kernel<ST, BN, f16_t, 2><<<grid, kDmaThreads, 0, stream>>>(MI355X_DMA_ARGS))
  if (rows == 64) {
    // 64-row tiles (half the activation rows of a tile, J = 2): for row counts just past a
    // multiple of 64 whose 128-row tiles leave CUs idle.  Two workgroups per CU share it when
    // the tiles outnumber the CUs.
    if (!few) {
      if (bn == 64) MI355X_DMA_LAUNCH64(MI355X_DMA_STAGES_MANY, 64);
      else MI355X_DMA_LAUNCH64(MI355X_DMA_STAGES_MANY, 128);
    } else {
      if (bn == 64) MI355X_DMA_LAUNCH64(MI355X_DMA_STAGES_FEW_NARROW, 64);
      else MI355X_DMA_LAUNCH64(MI355X_DMA_STAGES_FEW, 128);
    }
  } else if (!few) {
    if (bn == 160) MI355X_DMA_LAUNCH(MI355X_DMA_STAGES_MANY, 160);
    else if (bn == 64) MI355X_DMA_LAUNCH(MI355X_DMA_STAGES_MANY, 64);
    else MI355X_DMA_LAUNCH(MI355X_DMA_STAGES_MANY, 128);
  } else {
    if (bn == 160) MI355X_DMA_LAUNCH(MI355X_DMA_STAGES_FEW, 160);
    else if (bn == 64) MI355X_DMA_LAUNCH(MI355X_DMA_STAGES_FEW_NARROW, 64);
    else MI355X_DMA_LAUNCH(MI355X_DMA_STAGES_FEW, 128);
  }
#undef MI355X_DMA_LAUNCH64
#undef MI355X_DMA_LAUNCH
#undef MI355X_DMA_ARGS
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

}  // namespace mi355x
