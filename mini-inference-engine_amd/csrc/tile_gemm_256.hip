// Prefill block-scaled FP8 GEMM for gfx950: 256x256 output tile per CU.
//
// Arithmetic (same as every GEMM kernel of this library): one
// v_mfma_f32_16x16x128_f8f6f4 per 128-wide K group and 16x16 output tile gives the
// group's fp32 partial sum, folded into the fp32 accumulator as
// acc = fma(partial, a_s * w_s, acc), K groups in increasing order.
//
// Why 256x256: a CU sustains about 40 B/clk from L2 and 128 B/clk from LDS.  A per-CU
// output tile of BM x BN needs (BM + BN) * 128 bytes of operands per K group for
// 2 * BM * BN * 128 flops; at 256x256 that is 22 B/clk at 70 % of the fp8 MFMA peak,
// where 128x128 would need 44 B/clk, more than L2 delivers.
//
// Layout: 512 threads = 8 waves (2 per SIMD), wave w owns output rows 64 (w & 3) .. +63
// and columns 128 (w >> 2) .. +127, i.e. 4 x 8 MFMA tiles; its LDS reads are
// (64 + 128) * 128 B per K group, 8 waves -> 192 KiB per 2 * 256^2 * 128 flops, about
// 70 % of the LDS bandwidth at 70 % of peak.
//
// Feed: global -> LDS with global_load_lds_dwordx4 (no register staging), two stages
// (2 x 66 KiB), the K group kb+1 in flight while kb is multiplied.  Each stage holds the W
// tile (256 rows x 128 B), the activation tile (256 x 128 B) and 4 x 64 activation scales.
// A 64-lane DMA instruction writes 1 KiB of LDS linearly (8 rows x 8 chunks); the XOR
// swizzle (physical chunk p of row r holds logical chunk p ^ (r & 7)) is applied through
// each lane's source address, so fragment reads (ds_read_b128) are bank-conflict free.
// The stages are distinct LDS objects and the K loop is unrolled by two, so the compiler
// never waits for in-flight DMA before reading the current stage; the waits are explicit.
//
// Preconditions (checked by the launcher): K % 128 == 0, q/W 16-byte aligned with
// leading dimensions multiple of 16, scales K-group-major (as_sm == 1, as_sk >= M).
// Out-of-range tile rows read the last valid row (finite data, outputs never stored).
#include "fp8_abi_internal.h"
#include "fp8_common.h"

namespace mi355x {
namespace {

constexpr int kT256Threads = 512;
constexpr int kRowsT = 256;
constexpr int kTileChunks = kRowsT * 8;                 // one 256 x 128 B tile, in uint4
constexpr int kSinkOff = 2 * kTileChunks;              // 8 waves x 256 B written by the L2 prefetch, never read
constexpr int kStageU4 = kSinkOff + 128;


__shared__ uint4 t256_stage0[kStageU4];
__shared__ uint4 t256_stage1[kStageU4];

// K groups ahead of the one being multiplied that each step pulls into L2 (0: none).
// Off by default: on the Qwen3-4B shapes every distance tried (2, 4, 8) was slower than
// none (the extra 4-byte DMA per lane costs more than the L2 hits it buys).
#ifndef MI355X_T256_PREFETCH
#define MI355X_T256_PREFETCH 0
#endif
constexpr int kPrefetchAhead = MI355X_T256_PREFETCH;

typedef __attribute__((address_space(3))) void lds_void_t;

// The DMA instructions are issued through inline assembly.  The compiler then does not
// track them, so it adds no waits of its own before LDS reads of the *other* stage (its
// alias tracking of LDS DMA is not precise enough for this kernel and would serialise every
// step on the DMA latency).  Every wait for them is explicit: the vmcnt waits before the
// workgroup barriers.  (Untracked loads can only make the compiler's own vmcnt waits for
// ordinary loads stricter, never looser.)  M0 is written without being declared clobbered
// (it is a reserved register): nothing else in this kernel uses M0, as every LDS DMA of it
// goes through these two helpers.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)(p)));
}
__device__ __forceinline__ void dma16(const void* src, void* lds_dst) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr(lds_dst)) : "memory");
}
__device__ __forceinline__ void dma4(const void* src, void* lds_dst) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds_addr(lds_dst)) : "memory");
}

template <int S>
__device__ __forceinline__ uint4* stage256() {
  if constexpr (S == 0) return t256_stage0;
  else return t256_stage1;
}

struct Src256 {
  const uint8_t* w[4];
  const uint8_t* x[4];
  const float* as;   // activation scales of K group 0
  int as_row[4];     // this lane's rows 64 wm + 16 j + r, clamped to M - 1
  const uint8_t* pf;  // this thread's 128-byte line of the tile (W rows, then X rows)
};

// Fills stage S with K group kb and pulls K group kp's tile lines into L2 (the 4-byte
// prefetch lands in the stage's sink, so every DMA of a step targets one LDS object).
template <int S>
__device__ __forceinline__ void issue256(const Src256& src, int64_t kb, int64_t kp, int64_t as_sk, int wave) {
  uint4* st = stage256<S>();
  const int64_t koff = kb * kGroup;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    dma16(src.w[i] + koff, st + (i * 8 + wave) * 64);
    dma16(src.x[i] + koff, st + kTileChunks + (i * 8 + wave) * 64);
  }
  if constexpr (kPrefetchAhead > 0) dma4(src.pf + kp * kGroup, reinterpret_cast<float*>(st + kSinkOff) + wave * 64);
}

template <int S>
__device__ __forceinline__ v8i frag(const uint4* tile, int row, int g) {
  const uint4* p = tile + row * 8;
  return pack_v8i(p[g ^ (row & 7)], p[(g + 4) ^ (row & 7)]);
}

// The wave's four activation fragments stay in registers for the whole K group; the
// eight W fragments stream through two ahead, each feeding four independent MFMAs, so the
// LDS latency of a fragment hides behind 8 x 32 MFMA cycles and the registers left over
// (accumulators take 128) let several MFMA results be in flight before they are folded.
template <int S>
__device__ __forceinline__ void compute256(v4f (&acc)[8][4], const float (&asv)[4], float wsv, int wm, int wn,
                                           int r, int g) {
  const uint4* st = stage256<S>();
  v8i b[4];
  float sc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    b[j] = frag<S>(st + kTileChunks, wm * 64 + 16 * j + r, g);
    sc[j] = asv[j] * wsv;
  }
  v8i a0 = frag<S>(st, wn * 128 + r, g);
  v8i a1 = frag<S>(st, wn * 128 + 16 + r, g);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v8i a2;
    if (i + 2 < 8) a2 = frag<S>(st, wn * 128 + 16 * (i + 2) + r, g);
    v4f p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = mfma_16x16x128_e4m3(a0, b[j]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(p[j][v], sc[j], acc[i][j][v]);
    a0 = a1;
    if (i + 2 < 8) a1 = a2;
  }
}

// One K group.  Per wave and step the memory instructions are, in order: the 9 DMA loads
// of the next K group into the other stage, then one 4-byte DMA per lane that touches
// the K group kPrefetchAhead steps ahead (one 128-byte line per thread, 512 lines = the
// whole W and activation tile), so that its later DMA finds the data in L2 instead of
// paying the HBM latency with only one stage of lookahead.  Waiting for the current
// stage therefore leaves exactly the newest prefetch outstanding: vmcnt(1).
// Wait until this wave's DMA of the next stage has landed (everything but the newest
// prefetch: vmcnt(1)) and every wave has done the same and finished reading the current
// stage.  The wait sits at the end of a step, not the start, so that the loop's back edge
// follows it directly (the compiler then needs no wait of its own before the reads).
__device__ __forceinline__ void sync_stage() {
  __builtin_amdgcn_s_waitcnt(0x70 | (kPrefetchAhead > 0 ? 1 : 0));  // vmcnt(1 or 0), lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
}

template <int CUR>
__device__ __forceinline__ void step256(v4f (&acc)[8][4], const float (&asv)[4], float (&next)[4], const Src256& src,
                                        int64_t kb, int64_t KB,
                                        int64_t as_sk, const float* ws_row, int64_t ws_sk, int wave, int wm, int wn,
                                        int r, int g) {
  // The activation scales of K group kb + 1 go to registers (plain loads, L2 hits), issued
  // before the DMA batch so that the end-of-step vmcnt(1) also covers them; the two
  // unrolled steps alternate between two register sets, so no copy waits for a load.
  const int64_t kn = kb + 1 < KB ? kb + 1 : KB - 1;
#pragma unroll
  for (int j = 0; j < 4; ++j) next[j] = src.as[kn * as_sk + src.as_row[j]];
  // Keep the issue order scales, DMA batch, prefetch (compiler and scheduler barriers).
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  issue256<CUR ^ 1>(src, kn, kb + kPrefetchAhead < KB ? kb + kPrefetchAhead : KB - 1, as_sk, wave);
  __builtin_amdgcn_sched_barrier(0);
  compute256<CUR>(acc, asv, ws_row[kb * ws_sk], wm, wn, r, g);
  sync_stage();
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

#ifdef MI355X_T256_TIMING
// Development instrumentation only (never compiled into the library): per-workgroup
// start/end timestamps (s_memrealtime, 100 MHz) and the hardware id of the CU.
__device__ unsigned long long t256_timing[1 << 16][3];
#endif

template <typename OutT>
__global__ __launch_bounds__(kT256Threads, 2) void tile256_gemm_kernel(
    const uint8_t* __restrict__ q, int64_t ldq, const float* __restrict__ as, int64_t as_sk,
    const uint8_t* __restrict__ w, int64_t ldw, const float* __restrict__ ws, int64_t ws_sn,
    int64_t ws_sk, uint16_t* __restrict__ out, int64_t ldo, int64_t M, int64_t N, int64_t KB,
    int64_t tiles_m, int64_t tiles_n, int vec_out) {
  const int tid = threadIdx.x;
#ifdef MI355X_T256_TIMING
  const unsigned long long t_start = __builtin_amdgcn_s_memrealtime();
#endif
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int wm = wave & 3;
  const int wn = wave >> 2;
  int64_t tm, tn;
  tile_order(blockIdx.x, tiles_m, tiles_n, &tm, &tn);
  const int64_t m0 = tm * kRowsT;
  const int64_t n0 = tn * kRowsT;

  Src256 src;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rr = (i * 8 + wave) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ (rr & 7);
    const int64_t wrow = (n0 + rr) < N ? (n0 + rr) : (N - 1);
    const int64_t xrow = (m0 + rr) < M ? (m0 + rr) : (M - 1);
    src.w[i] = w + wrow * ldw + 16 * c;
    src.x[i] = q + xrow * ldq + 16 * c;
  }
  {
    src.as = as;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t row = m0 + wm * 64 + 16 * j + r;
      src.as_row[j] = static_cast<int>(row < M ? row : M - 1);
    }
    const int64_t prow = tid < kRowsT ? n0 + tid : m0 + tid - kRowsT;
    src.pf = tid < kRowsT ? w + (prow < N ? prow : N - 1) * ldw : q + (prow < M ? prow : M - 1) * ldq;
  }
  const int64_t nw = n0 + wn * 128;
  const float* ws_row = ws + ((nw < N ? nw : N - 1) / kGroup) * ws_sn;

  v4f acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  float as_even[4], as_odd[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) as_even[j] = src.as[src.as_row[j]];
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  issue256<0>(src, 0, KB > kPrefetchAhead - 1 ? kPrefetchAhead - 1 : KB - 1, as_sk, wave);
  __builtin_amdgcn_sched_barrier(0);
  sync_stage();
  int64_t kb = 0;
  for (; kb + 1 < KB; kb += 2) {
    step256<0>(acc, as_even, as_odd, src, kb, KB, as_sk, ws_row, ws_sk, wave, wm, wn, r, g);
    step256<1>(acc, as_odd, as_even, src, kb + 1, KB, as_sk, ws_row, ws_sk, wave, wm, wn, r, g);
  }
  if (kb < KB) step256<0>(acc, as_even, as_odd, src, kb, KB, as_sk, ws_row, ws_sk, wave, wm, wn, r, g);
  __builtin_amdgcn_s_waitcnt(0x70);  // no DMA may still target LDS when the workgroup ends

  // Lane holds out[m = m0 + 64 wm + 16 j + r][n = n0 + 128 wn + 16 i + 4 g + v].
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t m = m0 + wm * 64 + 16 * j + r;
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t n = nw + 16 * i + 4 * g;
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
#ifdef MI355X_T256_TIMING
  __syncthreads();
  if (tid == 0 && blockIdx.x < (1u << 16)) {
    t256_timing[blockIdx.x][0] = t_start;
    t256_timing[blockIdx.x][1] = __builtin_amdgcn_s_memrealtime();
    t256_timing[blockIdx.x][2] = __builtin_amdgcn_s_getreg((4 << 0) | (0 << 6) | (31 << 11));  // HW_ID
  }
#endif
}

}  // namespace

int launch_tile256(const uint8_t* q, int64_t ldq, const float* as, int64_t as_sk, const uint8_t* w,
                   int64_t ldw, const float* ws, int64_t ws_sn, int64_t ws_sk, void* out, int out_dtype,
                   int64_t ldo, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  const int64_t tiles_m = (M + kRowsT - 1) / kRowsT;
  const int64_t tiles_n = (N + kRowsT - 1) / kRowsT;
  if (tiles_m * tiles_n > 0x7fffffffLL) return MI355X_FP8_ERR_UNSUPPORTED;
  const int vec_out = (ldo % 4) == 0 && (reinterpret_cast<uintptr_t>(out) % 8) == 0;
  dim3 grid(static_cast<unsigned>(tiles_m * tiles_n));
  uint16_t* o = static_cast<uint16_t*>(out);
  if (out_dtype == kBF16)
    tile256_gemm_kernel<bf16_t><<<grid, kT256Threads, 0, stream>>>(q, ldq, as, as_sk, w, ldw, ws, ws_sn, ws_sk, o,
                                                                   ldo, M, N, K / kGroup, tiles_m, tiles_n, vec_out);
  else
    tile256_gemm_kernel<f16_t><<<grid, kT256Threads, 0, stream>>>(q, ldq, as, as_sk, w, ldw, ws, ws_sn, ws_sk, o,
                                                                  ldo, M, N, K / kGroup, tiles_m, tiles_n, vec_out);
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

}  // namespace mi355x
