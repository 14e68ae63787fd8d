// Prefill block-scaled FP8 GEMM for gfx950: 256-row output tiles, one workgroup per CU.
//
// Arithmetic (same as every GEMM kernel of this library): one
// v_mfma_f32_16x16x128_f8f6f4 per 128-wide K group and 16x16 output tile gives the
// group's fp32 partial sum, folded into the fp32 accumulator as
// acc = fma(partial, a_s * w_s, acc), K groups in increasing order.  The tile shape does
// not enter the arithmetic, so every tile width gives the same bits as the other kernels.
//
// Why 256 rows: a CU sustains about 40 B/clk from L2 (its LDS reads about 256 B/clk).  A per-CU
// output tile of BM x BN needs (BM + BN) * 128 bytes of operands per K group for
// 2 * BM * BN * 128 flops; at 256x256 that is 22 B/clk at 70 % of the fp8 MFMA peak,
// where 128x128 would need 44 B/clk, more than L2 delivers.
//
// Tile width BN: 256, 224 or 192 with a two-stage LDS ring, or 160 or 128 with a
// three-stage ring (3 x 52 KiB), which keeps two K groups in flight: the steps wait on their
// operands' L2 misses, so the narrower tiles with the deeper ring finish a wave sooner.
// The width is chosen per launch from measured wave times (the Qwen3-4B qkv projection at
// M = 2048 gets exactly 256 tiles of 256x192; at M = 1024, 192 tiles of 256x128).
//
// Layout: 512 threads = 8 waves (2 per SIMD), wave w owns output rows 64 (w & 3) .. +63
// and columns BN/2 (w >> 2) .. +BN/2-1, i.e. 4 x BN/32 MFMA tiles.
//
// Feed: global -> LDS with global_load_lds_dwordx4 (no register staging), two stages, the
// K group kb+1 in flight while kb is multiplied.  Each stage holds the W tile (BN rows x
// 128 B) and the activation tile (256 x 128 B); the activation and weight scales of the
// next K group go to registers.  A 64-lane DMA instruction writes 1 KiB of LDS linearly
// (8 rows x 8 chunks); the XOR swizzle (physical chunk p of row r holds logical chunk
// p ^ (r & 7)) is applied through each lane's source address, so fragment reads
// (ds_read_b128) are bank-conflict free.  The stages are distinct LDS objects and the K
// loop is unrolled by two, so the compiler never waits for in-flight DMA before reading
// the current stage; the waits are explicit.  (BN = 160 and 128 use a three-stage ring.)
//
// The output tile leaves through LDS as full-row 16-byte non-temporal stores when the output
// rows are 16-byte aligned (store_tile_lds), else straight from the registers (store_tile).
//
// Preconditions (checked by the launcher): K % 128 == 0, q/W 16-byte aligned with
// leading dimensions multiple of 16, scales K-group-major (as_sm == 1, as_sk >= M), byte
// offsets into q and W below 2^32.  Out-of-range tile rows read the last valid row
// (finite data, outputs never stored).
#include "fp8_abi_internal.h"
#include "fp8_common.h"

namespace mi355x {
namespace {

constexpr int kT256Threads = 512;
constexpr int kRowsT = 256;
constexpr int kXTileChunks = kRowsT * 8;  // the 256 x 128 B activation tile, in uint4
constexpr int kStageU4 = 2 * kXTileChunks;  // room for the widest W tile (256 rows) + activations

__shared__ uint4 t256_stage0[kStageU4];
__shared__ uint4 t256_stage1[kStageU4];
// Three-stage ring for tiles up to 160 wide: 3 x (160 + 256) x 128 B = 156 KiB.
constexpr int kMaxBN3 = 160;
constexpr int kStage3U4 = (kMaxBN3 + kRowsT) * 8;
__shared__ uint4 t256_ring0[kStage3U4];
__shared__ uint4 t256_ring1[kStage3U4];
__shared__ uint4 t256_ring2[kStage3U4];

typedef __attribute__((address_space(3))) void lds_void_t;

// The DMA instructions are issued through inline assembly.  The compiler then does not
// track them, so it adds no waits of its own before LDS reads of the *other* stage (its
// alias tracking of LDS DMA is not precise enough for this kernel and would serialise every
// step on the DMA latency).  Every wait for them is explicit: the vmcnt waits before the
// workgroup barriers.  (Untracked loads can only make the compiler's own vmcnt waits for
// ordinary loads stricter, never looser.)  M0 is written without being declared clobbered
// (it is a reserved register): nothing else in this kernel uses M0, as every LDS DMA of it
// goes through this helper.  SALU writes of M0 need one wait state before an LDS DMA
// reads it (the s_nop).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)(p)));
}
// 16 bytes per lane from base + off (32-bit per-lane offset, 64-bit uniform base).
__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t off, void* lds_dst) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base),
               "s"(lds_addr(lds_dst))
               : "memory");
}

template <int NS, int S>
__device__ __forceinline__ uint4* stage256() {
  if constexpr (NS == 2) {
    if constexpr (S == 0) return t256_stage0;
    else return t256_stage1;
  } else {
    if constexpr (S == 0) return t256_ring0;
    else if constexpr (S == 1) return t256_ring1;
    else return t256_ring2;
  }
}

// Tile geometry for width BN and J 16-row activation fragments per wave (tile rows 64 J:
// 256 for J = 4, 192 for J = 3).
template <int BN, int J>
struct Geo {
  static_assert(BN % 32 == 0 && BN <= 256 && BN >= 128, "tile width");
  static_assert(J == 3 || J == 4, "tile rows");
  static constexpr int kNI = BN / 32;             // 16-column MFMA tiles per wave
  static constexpr int kJ = J;
  static constexpr int kRows = 64 * J;            // tile rows
  static constexpr int kWBlocks = BN / 8;         // 1 KiB DMA blocks of the W tile
  static constexpr int kWPerWave = (kWBlocks + 7) / 8;
  static constexpr int kXOff = BN * 8;            // activation tile offset in the stage (uint4)
  static constexpr int kNDma = kWPerWave + J;     // DMA instructions per wave per stage (X: 8 J blocks)
};

// Per-tile feed state of one lane.
struct Src256 {
  uint32_t w[4];         // byte offset in W of this lane's 16-byte chunk of its rows of block 8 i + wave
  uint32_t x[4];         // same in the activations (rows of block 8 i + wave, i < J)
  const float* as;       // activation scales (K-group-major), K group 0
  const float* ws_a;     // weight scales of the 128-column blocks the wave's columns touch, K group 0
  const float* ws_b;
  int as_row[4];         // this lane's rows 16 J wm + 16 j + r (j < J), clamped to M - 1
  uint32_t use_b;        // bit i: column tile i lies in block ws_b
  int vzero;             // 0 held in a VGPR, so that loads indexed by it are per-lane loads
};

// Fills stage S with K group kb.  W blocks past the tile (BN/8 not a multiple of 8) repeat
// the last block: the two waves write identical bytes.
template <int BN, int J, int NS, int S>
__device__ __forceinline__ void issue256(const Src256& src, const uint8_t* w, const uint8_t* q, int64_t kb, int wave) {
  using G = Geo<BN, J>;
  uint4* st = stage256<NS, S>();
  const uint8_t* wk = w + kb * kGroup;
  const uint8_t* qk = q + kb * kGroup;
#pragma unroll
  for (int i = 0; i < G::kWPerWave; ++i) {
    const int blk = (i * 8 + wave) < G::kWBlocks ? (i * 8 + wave) : (G::kWBlocks - 1);
    dma16(wk, src.w[i], st + blk * 64);
  }
#pragma unroll
  for (int i = 0; i < J; ++i) dma16(qk, src.x[i], st + G::kXOff + (i * 8 + wave) * 64);
}

// One of the step's DMA instructions: t < kWPerWave loads W block 8 t + wave, the rest the
// activation blocks.
template <int BN, int J, int NS, int S>
__device__ __forceinline__ void issue_one(const Src256& src, const uint8_t* w, const uint8_t* q, int64_t kb, int wave,
                                          int t) {
  using G = Geo<BN, J>;
  uint4* st = stage256<NS, S>();
  if (t < G::kWPerWave) {
    const int blk = (t * 8 + wave) < G::kWBlocks ? (t * 8 + wave) : (G::kWBlocks - 1);
    dma16(w + kb * kGroup, src.w[t], st + blk * 64);
  } else {
    const int i = t - G::kWPerWave;
    dma16(q + kb * kGroup, src.x[i], st + G::kXOff + (i * 8 + wave) * 64);
  }
}

template <int S>
__device__ __forceinline__ v8i frag(const uint4* tile, int row, int g) {
  const uint4* p = tile + row * 8;
  return pack_v8i(p[g ^ (row & 7)], p[(g + 4) ^ (row & 7)]);
}

// Scales of one K group in registers: J activation scales (this lane's rows) and the two
// weight scales the wave may need.
struct Scales {
  float a[4];
  float wa, wb;
};

// The wave's four activation fragments stay in registers for the whole K group; the W
// fragments stream through two ahead, each feeding four independent MFMAs.  Read order:
// the first W fragment, then the four activation fragments, then the second W fragment,
// so the first MFMA waits for two fragments, not for all of them.  The DMA loads of the
// next K group (into the other stage, kn) go out in two halves, before the first and
// before the middle MFMA group: a wave then never sits behind its whole DMA batch while
// its partner wave on the SIMD does the same (measured 2-5 % faster than one batch).
//
// The fold is software-pipelined: column tile i's four MFMAs are issued, then tile i-1's
// sixteen partials are folded while they run (one MFMA per four FMAs), so no fold waits on
// the MFMA it follows.  The eight scale products a_s[j] * w_s (two weight-scale blocks at
// most) are formed once per step; each is the same single fp32 product as before, so the
// folded values are unchanged bit for bit.
template <int BN, int J, int NS, int S, int NXT>
__device__ __forceinline__ void compute256(v4f (&acc)[BN / 32][J], const Scales& sc_in, uint32_t use_b, int wm,
                                           int wn, int r, int g, const Src256& src, const uint8_t* w,
                                           const uint8_t* q, int64_t kn, int wave) {
  using G = Geo<BN, J>;
  constexpr int NI = G::kNI;
  constexpr int NDMA = G::kNDma;
  const uint4* st = stage256<NS, S>();
  const int wrow0 = wn * (BN / 2) + r;
  float sa[J], sb[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    sa[j] = sc_in.a[j] * sc_in.wa;
    sb[j] = sc_in.a[j] * sc_in.wb;
  }
  v8i a0 = frag<S>(st, wrow0, g);
  v8i b[J];
#pragma unroll
  for (int j = 0; j < J; ++j) b[j] = frag<S>(st + G::kXOff, wm * 16 * J + 16 * j + r, g);
  v8i a1 = frag<S>(st, wrow0 + 16, g);
  v4f p[2][J];
#pragma unroll
  for (int i = 0; i <= NI; ++i) {
    v8i a2;
    if (i < NI) {
#pragma unroll
      for (int t = 0; t < NDMA; ++t)
        if ((t < NDMA / 2 ? 0 : NI / 2) == i) issue_one<BN, J, NS, NXT>(src, w, q, kn, wave, t);
      if (i + 2 < NI) a2 = frag<S>(st, wrow0 + 16 * (i + 2), g);
    }
    // MFMA (i, j), then the fold of (i - 1, j), whose MFMA went out four MFMAs earlier; the
    // scheduling barriers keep that order, so no fold waits on the MFMA just issued.
    const bool ub = i > 0 && ((use_b >> (i - 1)) & 1);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (i < NI) p[i & 1][j] = mfma_16x16x128_e4m3(a0, b[j]);
      if (i > 0) {
        const float sc = ub ? sb[j] : sa[j];
#pragma unroll
        for (int v = 0; v < 4; ++v)
          acc[i - 1][j][v] = __builtin_fmaf(p[(i - 1) & 1][j][v], sc, acc[i - 1][j][v]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (i < NI) {
      a0 = a1;
      if (i + 2 < NI) a1 = a2;
    }
  }
}

// The unpipelined fold, for the 256-row, 256-wide tiles: their accumulators leave no registers
// for a second set of partials (the pipelined form spills there; the 192-row form has room).
template <int BN, int J, int NS, int S, int NXT>
__device__ __forceinline__ void compute256_plain(v4f (&acc)[BN / 32][J], const Scales& sc_in, uint32_t use_b,
                                                 int wm, int wn, int r, int g, const Src256& src, const uint8_t* w,
                                                 const uint8_t* q, int64_t kn, int wave) {
  using G = Geo<BN, J>;
  constexpr int NI = G::kNI;
  constexpr int NDMA = G::kNDma;
  const uint4* st = stage256<NS, S>();
  const int wrow0 = wn * (BN / 2) + r;
  v8i a0 = frag<S>(st, wrow0, g);
  v8i b[J];
#pragma unroll
  for (int j = 0; j < J; ++j) b[j] = frag<S>(st + G::kXOff, wm * 16 * J + 16 * j + r, g);
  v8i a1 = frag<S>(st, wrow0 + 16, g);
#pragma unroll
  for (int i = 0; i < NI; ++i) {
#pragma unroll
    for (int t = 0; t < NDMA; ++t)
      if ((t < NDMA / 2 ? 0 : NI / 2) == i) issue_one<BN, J, NS, NXT>(src, w, q, kn, wave, t);
    v8i a2;
    if (i + 2 < NI) a2 = frag<S>(st, wrow0 + 16 * (i + 2), g);
    const float wsv = (use_b >> i) & 1 ? sc_in.wb : sc_in.wa;
    v4f p[J];
#pragma unroll
    for (int j = 0; j < J; ++j) p[j] = mfma_16x16x128_e4m3(a0, b[j]);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const float sc = sc_in.a[j] * wsv;
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(p[j][v], sc, acc[i][j][v]);
    }
    a0 = a1;
    if (i + 2 < NI) a1 = a2;
  }
}

// Wait until this wave's DMA of the next stage has landed and its LDS reads are done, then
// the workgroup barrier: after it every wave's DMA has landed and nobody reads the current
// stage any more.  The wait sits at the end of a step, not the start, so that the loop's
// back edge follows it directly (the compiler then needs no wait of its own before the reads).
template <int N = 0>
__device__ __forceinline__ void sync_stage() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));  // vmcnt(N) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
}

template <int J>
__device__ __forceinline__ void load_scales(Scales& s, const Src256& src, int64_t kb, int64_t as_sk, int64_t ws_sk) {
#pragma unroll
  for (int j = 0; j < J; ++j) s.a[j] = src.as[kb * as_sk + src.as_row[j]];
  // Per-lane loads (vzero keeps them off the scalar unit: scalar loads share the LDS
  // counter, and waiting for one would wait for every fragment read).
  s.wa = src.ws_a[kb * ws_sk + src.vzero];
  s.wb = src.ws_b[kb * ws_sk + src.vzero];
}

// One K group kb of the range [.., khi), multiplied from ring stage CUR of NS.  The scales
// of K group kb + 1 go to registers (per-lane loads, L2 hits), issued before the DMA loads
// so that the end-of-step wait also covers them.  The DMA refills the stage NS - 1 groups
// ahead (the one read in the previous step); the end-of-step wait leaves only that newest
// batch in flight (loads complete in issue order).  Past the end of the range the loads
// repeat its last group (the stage they fill is not read again).
template <int BN, int J, int NS, int CUR>
__device__ __forceinline__ void step256(v4f (&acc)[BN / 32][J], const Scales& cur, Scales& next,
                                        const Src256& src, const uint8_t* w, const uint8_t* q, int64_t kb,
                                        int64_t khi, int64_t as_sk, int64_t ws_sk, int wave, int wm, int wn, int r,
                                        int g) {
  constexpr int NDMA = Geo<BN, J>::kNDma;
  const int64_t kn = kb + 1 < khi ? kb + 1 : khi - 1;
  const int64_t kd = kb + NS - 1 < khi ? kb + NS - 1 : khi - 1;
  load_scales<J>(next, src, kn, as_sk, ws_sk);
  // Keep the scale loads ahead of the DMA loads (compiler and scheduler barriers).
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (BN == 256 && J == 4)
    compute256_plain<BN, J, NS, CUR, (CUR + NS - 1) % NS>(acc, cur, src.use_b, wm, wn, r, g, src, w, q, kd, wave);
  else
    compute256<BN, J, NS, CUR, (CUR + NS - 1) % NS>(acc, cur, src.use_b, wm, wn, r, g, src, w, q, kd, wave);
  // Every MFMA of the step is issued before the wait: the matrix core then works through
  // them while the wave waits for its DMA and the other waves (without this barrier the
  // scheduler moves the last MFMA groups behind s_barrier; measured 7 % slower on qkv).
  __builtin_amdgcn_sched_barrier(0);
  sync_stage<NDMA * (NS - 2)>();
}

__device__ __forceinline__ void tile_order(int64_t pid, int64_t tiles_m, int64_t tiles_n, int64_t* tm, int64_t* tn) {
  // Workgroups go round-robin over the 8 XCDs; give each XCD a contiguous range of
  // logical tiles, walked in groups of 4 tile rows so concurrent tiles share operands in L2.
  constexpr int64_t kGroupRows = 4;
  const int64_t total = tiles_m * tiles_n;
  const int64_t per = total / 8, rem = total % 8;
  const int64_t xcd = pid % 8, idx = pid / 8;
  const int64_t logical = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  const int64_t per_group = kGroupRows * tiles_n;
  const int64_t group = logical / per_group;
  const int64_t first_m = group * kGroupRows;
  const int64_t gm = (tiles_m - first_m) < kGroupRows ? (tiles_m - first_m) : kGroupRows;
  const int64_t within = logical - group * per_group;
  *tm = first_m + within % gm;
  *tn = within / gm;
}

struct Dims256 {
  const uint8_t* q;
  const float* as;
  const uint8_t* w;
  const float* ws;
  uint16_t* out;
  int64_t ldq, as_sk, ldw, ws_sn, ws_sk, ldo, M, N, KB;
  int vec_out;  // out_vec_mode(out, ldo)
};

template <int BN, int J>
__device__ __forceinline__ void setup_tile(Src256& src, const Dims256& d, int64_t m0, int64_t n0, int wave,
                                           int lane, int wm, int wn, int r) {
  using G = Geo<BN, J>;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i < G::kWPerWave) {
      const int blk = (i * 8 + wave) < G::kWBlocks ? (i * 8 + wave) : (G::kWBlocks - 1);
      const int rr = blk * 8 + (lane >> 3);
      const int c = (lane & 7) ^ (rr & 7);
      const int64_t wrow = (n0 + rr) < d.N ? (n0 + rr) : (d.N - 1);
      src.w[i] = static_cast<uint32_t>(wrow * d.ldw + 16 * c);  // < 2^32: checked by the launcher
    } else {
      src.w[i] = 0;
    }
    const int rx = (i * 8 + wave) * 8 + (lane >> 3);
    const int cx = (lane & 7) ^ (rx & 7);
    const int64_t xrow = (m0 + rx) < d.M ? (m0 + rx) : (d.M - 1);
    src.x[i] = static_cast<uint32_t>(xrow * d.ldq + 16 * cx);
  }
  src.as = d.as;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t row = m0 + wm * 16 * J + 16 * j + r;
    src.as_row[j] = static_cast<int>(row < d.M ? row : d.M - 1);  // j >= J: unused
  }
  // The wave's columns [nw, nw + BN/2) touch at most two 128-column weight-scale blocks.
  const int64_t nw = n0 + wn * (BN / 2);
  const int64_t last_blk = (d.N - 1) / kGroup;
  const int64_t blk_a = nw / kGroup < last_blk ? nw / kGroup : last_blk;
  const int64_t blk_b = blk_a + 1 < last_blk ? blk_a + 1 : last_blk;
  src.ws_a = d.ws + blk_a * d.ws_sn;
  src.ws_b = d.ws + blk_b * d.ws_sn;
  uint32_t use_b = 0;
#pragma unroll
  for (int i = 0; i < G::kNI; ++i)
    if ((nw + 16 * i) / kGroup != nw / kGroup) use_b |= 1u << i;
  src.use_b = use_b;
}

// acc = the tile's products over K groups [klo, khi), in increasing order, through a ring
// of NS (2 or 3) LDS stages.
template <int BN, int J, int NS>
__device__ __forceinline__ void run_k(v4f (&acc)[BN / 32][J], const Src256& src, const Dims256& d, int64_t klo,
                                      int64_t khi, int wave, int wm, int wn, int r, int g) {
  static_assert(NS == 2 || (NS == 3 && BN <= kMaxBN3), "ring depth");
  constexpr int NDMA = Geo<BN, J>::kNDma;
#pragma unroll
  for (int i = 0; i < Geo<BN, J>::kNI; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
#define MI355X_STEP(CUR, SC, SN, KB) \
  step256<BN, J, NS, CUR>(acc, SC, SN, src, d.w, d.q, KB, khi, d.as_sk, d.ws_sk, wave, wm, wn, r, g)
  if constexpr (NS == 2) {
    Scales s_even, s_odd;
    load_scales<J>(s_even, src, klo, d.as_sk, d.ws_sk);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    issue256<BN, J, 2, 0>(src, d.w, d.q, klo, wave);
    __builtin_amdgcn_sched_barrier(0);
    sync_stage();
    int64_t kb = klo;
    for (; kb + 1 < khi; kb += 2) {
      MI355X_STEP(0, s_even, s_odd, kb);
      MI355X_STEP(1, s_odd, s_even, kb + 1);
    }
    if (kb < khi) MI355X_STEP(0, s_even, s_odd, kb);
  } else {
    Scales s0, s1, s2;
    load_scales<J>(s0, src, klo, d.as_sk, d.ws_sk);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    issue256<BN, J, 3, 0>(src, d.w, d.q, klo, wave);
    issue256<BN, J, 3, 1>(src, d.w, d.q, klo + 1 < khi ? klo + 1 : khi - 1, wave);
    __builtin_amdgcn_sched_barrier(0);
    sync_stage<NDMA>();  // stage 0 and the scales landed; stage 1 may still be in flight
    int64_t kb = klo;
    for (; kb + 2 < khi; kb += 3) {
      MI355X_STEP(0, s0, s1, kb);
      MI355X_STEP(1, s1, s2, kb + 1);
      MI355X_STEP(2, s2, s0, kb + 2);
    }
    if (kb < khi) MI355X_STEP(0, s0, s1, kb);
    if (kb + 1 < khi) MI355X_STEP(1, s1, s2, kb + 1);
  }
#undef MI355X_STEP
}

// Lane holds out[m = m0 + 16 J wm + 16 j + r][n = n0 + BN/2 wn + 16 i + 4 g + v].
template <int BN, int J, typename OutT>
__device__ __forceinline__ void store_tile(const v4f (&acc)[BN / 32][J], const Dims256& d, int64_t m0,
                                           int64_t n0, int wm, int wn, int r, int g) {
  const int64_t nw = n0 + wn * (BN / 2);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int64_t m = m0 + wm * 16 * J + 16 * j + r;
    if (m >= d.M) continue;
#pragma unroll
    for (int i = 0; i < Geo<BN, J>::kNI; ++i) {
      const int64_t n = nw + 16 * i + 4 * g;
      uint16_t h[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) h[v] = OutCvt<OutT>::cvt(acc[i][j][v]);
      uint16_t* dst = d.out + m * d.ldo + n;
      if (d.vec_out && n + 4 <= d.N) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16),
                                                    h[2] | (static_cast<uint32_t>(h[3]) << 16));
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (n + v < d.N) dst[v] = h[v];
      }
    }
  }
}

// The epilogue through LDS (staged_index, fp8_common.h): the tile's first half of rows (32 J)
// in ring stage 0, the second in stage 1.  Needs 16-byte aligned output rows (vec_out == 2).
template <int BN, int J, int NS, typename OutT>
__device__ __forceinline__ void store_tile_lds(const v4f (&acc)[BN / 32][J], const Dims256& d, int64_t m0,
                                               int64_t n0, int wm, int wn, int r, int g, int tid) {
  constexpr int kHalf = 32 * J;
  uint16_t* r0 = reinterpret_cast<uint16_t*>(stage256<NS, 0>());
  uint16_t* r1 = reinterpret_cast<uint16_t*>(stage256<NS, 1>());
  static_assert(kHalf * staged_pitch<BN>() * 2 <= (NS == 2 ? kStageU4 : kStage3U4) * 16, "staged rows fit a stage");
  __syncthreads();  // every wave is done with the ring
  uint16_t* reg = wm < 2 ? r0 : r1;
#pragma unroll
  for (int j = 0; j < J; ++j) {
#pragma unroll
    for (int i = 0; i < Geo<BN, J>::kNI; ++i) {
      uint16_t h[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) h[v] = OutCvt<OutT>::cvt(acc[i][j][v]);
      *reinterpret_cast<uint2*>(reg + staged_index<BN>((wm & 1) * 16 * J + 16 * j + r, wn * (BN / 2) + 16 * i + 4 * g)) =
          make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16));
    }
  }
  __syncthreads();
  constexpr int C = BN / 8;  // 16-byte pieces per row
#pragma unroll 4
  for (int idx = tid; idx < 2 * kHalf * C; idx += kT256Threads) {
    const int row = idx / C, c = idx - (idx / C) * C;
    const int64_t m = m0 + row, n = n0 + 8 * c;
    const uint4 val = *reinterpret_cast<const uint4*>(row < kHalf ? r0 + staged_index<BN>(row, 8 * c)
                                                                   : r1 + staged_index<BN>(row - kHalf, 8 * c));
    if (m >= d.M) continue;
    uint16_t* dst = d.out + m * d.ldo + n;
    if (n + 8 <= d.N) {
      store16_nt(dst, val);
    } else {
      const uint16_t* hv = reinterpret_cast<const uint16_t*>(&val);
      for (int v = 0; v < 8; ++v)
        if (n + v < d.N) dst[v] = hv[v];
    }
  }
}

template <int BN, int J, int NS, typename OutT>
__global__ __launch_bounds__(kT256Threads, 2) void tile256_gemm_kernel(Dims256 d, int64_t tiles_m, int64_t tiles_n) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int wm = wave & 3;
  const int wn = wave >> 2;
  int64_t tm, tn;
  tile_order(blockIdx.x, tiles_m, tiles_n, &tm, &tn);
  Src256 src;
  asm volatile("v_mov_b32 %0, 0" : "=v"(src.vzero));
  constexpr int RT = Geo<BN, J>::kRows;
  setup_tile<BN, J>(src, d, tm * RT, tn * BN, wave, lane, wm, wn, r);
  v4f acc[Geo<BN, J>::kNI][J];
  run_k<BN, J, NS>(acc, src, d, 0, d.KB, wave, wm, wn, r, g);
  __builtin_amdgcn_s_waitcnt(0x70);  // no DMA may still target LDS when the workgroup ends
  if (d.vec_out == 2) store_tile_lds<BN, J, NS, OutT>(acc, d, tm * RT, tn * BN, wm, wn, r, g, tid);
  else store_tile<BN, J, OutT>(acc, d, tm * RT, tn * BN, wm, wn, r, g);
}

template <int BN, int J, int NS>
int launch_bn(const Dims256& d, int out_dtype, hipStream_t stream) {
  constexpr int RT = Geo<BN, J>::kRows;
  const int64_t tiles_m = (d.M + RT - 1) / RT;
  const int64_t tiles_n = (d.N + BN - 1) / BN;
  if (tiles_m * tiles_n > 0x7fffffffLL) return MI355X_FP8_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(tiles_m * tiles_n));
  if (out_dtype == kBF16)
    tile256_gemm_kernel<BN, J, NS, bf16_t><<<grid, kT256Threads, 0, stream>>>(d, tiles_m, tiles_n);
  else
    tile256_gemm_kernel<BN, J, NS, f16_t><<<grid, kT256Threads, 0, stream>>>(d, tiles_m, tiles_n);
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

}  // namespace

bool tile256_offsets_ok(int64_t ldq, int64_t ldw, int64_t M, int64_t N, int64_t K) {
  // Tile rows are tracked in 32-bit registers, and byte offsets into q and W in 32-bit lanes.
  return M <= 0x7fff0000LL && N <= 0x7fff0000LL && (M - 1) * ldq + K <= 0xffffffffLL &&
         (N - 1) * ldw + K <= 0xffffffffLL;
}

int launch_tile256(const uint8_t* q, int64_t ldq, const float* as, int64_t as_sk, const uint8_t* w,
                   int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, void* out, int out_dtype,
                   int64_t ldo, int64_t M, int64_t N, int64_t K, int bn, int rows, hipStream_t stream) {
  if (!tile256_offsets_ok(ldq, ldw, M, N, K)) return MI355X_FP8_ERR_UNSUPPORTED;
  const Dims256 d{q, as, w, ws, static_cast<uint16_t*>(out), ldq, as_sk, ldw, ws_sn, ws_sk, ldo, M, N, K / kGroup,
                  out_vec_mode(out, ldo)};
  if (rows == 192) {
    switch (bn) {
      case 256: return launch_bn<256, 3, 2>(d, out_dtype, stream);
      case 224: return launch_bn<224, 3, 2>(d, out_dtype, stream);
      case 192: return launch_bn<192, 3, 2>(d, out_dtype, stream);
      case 160: return launch_bn<160, 3, 3>(d, out_dtype, stream);
      case 128: return launch_bn<128, 3, 3>(d, out_dtype, stream);
      default: return MI355X_FP8_ERR_INVALID;
    }
  }
  if (rows != 256) return MI355X_FP8_ERR_INVALID;
  switch (bn) {
    case 256: return launch_bn<256, 4, 2>(d, out_dtype, stream);
    case 224: return launch_bn<224, 4, 2>(d, out_dtype, stream);
    case 192: return launch_bn<192, 4, 2>(d, out_dtype, stream);
    case 160: return launch_bn<160, 4, 3>(d, out_dtype, stream);  // three-stage ring
    case 128: return launch_bn<128, 4, 3>(d, out_dtype, stream);
    default: return MI355X_FP8_ERR_INVALID;
  }
}

}  // namespace mi355x
