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
// Two kernels:
//   stream_gemm_kernel  decode-sized M (<= 64 rows per launch slice).  HBM-bound weight
//                       streaming: W goes global -> registers (each byte read once), the
//                       small activation matrix is served from L2.  Grid = 64-row W strips x
//                       K splits; the 4 waves of a workgroup take interleaved K groups and
//                       reduce through LDS; K splits reduce through an fp32 workspace, the
//                       last-arriving workgroup of a strip summing the partials in split
//                       order (deterministic) and resetting the strip's counter.
//   tile_gemm_kernel    prefill-sized M.  MFMA-bound: 128x128 output tile per 256-thread
//                       workgroup, 2x2 waves of 64x64, K groups staged global -> registers
//                       -> LDS with double buffering and an XOR-swizzled (conflict-free)
//                       layout; XCD-aware, grouped tile order for L2 reuse.
#include "fp8_abi_internal.h"
#include "fp8_common.h"

namespace mi355x {

constexpr int kThreads = 256;
constexpr int kStripRows = 64;           // W rows per stream-kernel workgroup
constexpr int kRedStride = kStripRows + 4;

// ------------------------------------------------------------------------------------
// Stream kernel (decode M)
// ------------------------------------------------------------------------------------
template <int NT, bool ALIGNED, typename OutT>
__global__ __launch_bounds__(kThreads) void stream_gemm_kernel(
    const uint8_t* __restrict__ q, int64_t ldq, const float* __restrict__ as, int64_t as_sm,
    int64_t as_sk, const uint8_t* __restrict__ w, int64_t ldw, const float* __restrict__ ws,
    int64_t ws_sn, int64_t ws_sk, uint16_t* __restrict__ out, int64_t ldo, int64_t M, int64_t N,
    int64_t K, int64_t KB, int64_t kb_per_split, int64_t splits, float* __restrict__ partials,
    unsigned* __restrict__ counters) {
  constexpr int kTok = 16 * NT;                      // token rows of this slice
  constexpr int kElems = kTok * kStripRows;          // outputs per workgroup
  __shared__ float red[2 * kTok * kRedStride];
  __shared__ int is_last;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int64_t strip = blockIdx.x;
  const int64_t split = blockIdx.y;
  const int64_t tslice = blockIdx.z;
  const int64_t n0 = strip * kStripRows;
  const int64_t m_base = tslice * 64;
  const int64_t m_rows = (M - m_base) < kTok ? (M - m_base) : kTok;
  const int64_t kb_begin = split * kb_per_split;
  const int64_t kb_end = (kb_begin + kb_per_split) < KB ? (kb_begin + kb_per_split) : KB;
  const int64_t nb = n0 / kGroup;

  v4f acc[4][NT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int64_t kb = kb_begin + wave; kb < kb_end; kb += 4) {
    const int64_t k_lo = kb * kGroup + 16 * g;
    const int64_t k_hi = k_lo + 64;
    v8i a[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = n0 + 16 * i + r;
      a[i] = pack_v8i(load_chunk16<ALIGNED>(w, ldw, row, N, k_lo, K),
                      load_chunk16<ALIGNED>(w, ldw, row, N, k_hi, K));
    }
    v8i b[NT];
    float sc[NT];
    const float wsv = ws[nb * ws_sn + kb * ws_sk];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int64_t tok = 16 * j + r;
      const int64_t m = m_base + tok;
      b[j] = pack_v8i(load_chunk16<ALIGNED>(q, ldq, m, M, k_lo, K),
                      load_chunk16<ALIGNED>(q, ldq, m, M, k_hi, K));
      sc[j] = (tok < m_rows ? as[m * as_sm + kb * as_sk] : 0.0f) * wsv;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const v4f d = mfma_16x16x128_e4m3(a[i], b[j]);
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(d[v], sc[j], acc[i][j][v]);
      }
  }

  // Lane holds D[n = 16 i + 4 g + v][token = 16 j + r].  Combine the four waves as
  // (w0 + w1) + (w2 + w3) through two LDS slots laid out [token][n] (fixed order, so the
  // result does not depend on wave timing), leaving the sum in slot A.
  float* slot_a = red;
  float* slot_b = red + kTok * kRedStride;
  auto put = [&](float* slot) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j)
        *reinterpret_cast<float4*>(slot + (16 * j + r) * kRedStride + 16 * i + 4 * g) =
            make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
  };
  auto add = [&](const float* slot) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const float4 t = *reinterpret_cast<const float4*>(slot + (16 * j + r) * kRedStride + 16 * i + 4 * g);
        acc[i][j][0] += t.x; acc[i][j][1] += t.y; acc[i][j][2] += t.z; acc[i][j][3] += t.w;
      }
  };
  if (wave == 1) put(slot_a);
  if (wave == 3) put(slot_b);
  __syncthreads();
  if (wave == 0) add(slot_a);
  if (wave == 2) add(slot_b);
  __syncthreads();
  if (wave == 2) put(slot_a);
  __syncthreads();
  if (wave == 0) {
    add(slot_a);
    put(slot_a);
  }
  __syncthreads();

  const int64_t region = ((tslice * gridDim.x + strip) * splits) * kElems;
  for (int e = tid; e < kElems; e += kThreads) {
    const int tok = e / kStripRows;
    const int nl = e - tok * kStripRows;
    const float val = slot_a[tok * kRedStride + nl];
    const int64_t n = n0 + nl;
    if (tok >= m_rows || n >= N) continue;
    if (splits == 1) {
      out[(m_base + tok) * ldo + n] = OutCvt<OutT>::cvt(val);
    } else {
      // Agent-scope relaxed atomic stores write through to the device coherence point, so
      // no L2 write-back fence is needed before the arrival counter is bumped.
      __hip_atomic_store(&partials[region + split * kElems + e], val, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (splits == 1) return;

  // Split-K: every partial store of this workgroup has completed (the barrier waits for
  // outstanding memory operations) before one thread bumps the strip's counter; the
  // workgroup that brings the count to `splits` sums the partials in split order.
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(&counters[tslice * gridDim.x + strip], 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == static_cast<unsigned>(splits - 1);
  }
  __syncthreads();
  if (!is_last) return;
  for (int e = tid; e < kElems; e += kThreads) {
    const int tok = e / kStripRows;
    const int nl = e - tok * kStripRows;
    const int64_t n = n0 + nl;
    if (tok >= m_rows || n >= N) continue;
    float val = 0.0f;
    for (int64_t s = 0; s < splits; ++s)
      val += __hip_atomic_load(&partials[region + s * kElems + e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    out[(m_base + tok) * ldo + n] = OutCvt<OutT>::cvt(val);
  }
  if (tid == 0)
    __hip_atomic_store(&counters[tslice * gridDim.x + strip], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
  if (M < 0 || N < 0 || K <= 0) return MI355X_FP8_ERR_INVALID;
  *plan = GemmPlan{};
  if (config == MI355X_FP8_CONFIG_AUTO) config = M <= 64 ? MI355X_FP8_CONFIG_STREAM : MI355X_FP8_CONFIG_TILE128;
  if (config != MI355X_FP8_CONFIG_STREAM && config != MI355X_FP8_CONFIG_TILE128) return MI355X_FP8_ERR_INVALID;
  plan->kernel = config;
  if (config == MI355X_FP8_CONFIG_TILE128) return MI355X_FP8_OK;
  const int64_t KB = cdiv(K, kGroup);
  const int64_t slice_rows = M < 64 ? M : 64;
  plan->token_tiles = slice_rows <= 16 ? 1 : (slice_rows <= 32 ? 2 : 4);
  plan->strips = cdiv(N, kStripRows);
  const int64_t slices = M > 0 ? cdiv(M, 64) : 0;
  // The K split depends on K alone, never on M or N: a row's (or a column's) result is then
  // the same whichever other rows or N-concatenated projections share the launch.
  const int64_t kbps = KB <= 48 ? 4 : 8;  // one or two K groups per wave
  plan->kb_per_split = kbps;
  plan->splits = cdiv(KB, kbps);
  if (plan->splits > 1) {
    plan->partial_bytes = static_cast<size_t>(slices * plan->strips * plan->splits) *
                          static_cast<size_t>(16 * plan->token_tiles * kStripRows) * sizeof(float);
    if (slices * plan->strips > kCounterSlots) return MI355X_FP8_ERR_UNSUPPORTED;
  }
  return MI355X_FP8_OK;
}

size_t gemm_workspace_bytes(const GemmPlan& plan) {
  // The counter region is reserved whatever the plan, so that it stays zero whichever
  // sequence of shapes shares the workspace.
  return kCounterRegionBytes + align256(plan.partial_bytes);
}

template <bool ALIGNED, typename OutT>
static void launch_stream(const GemmPlan& p, const uint8_t* q, int64_t ldq, const float* as,
                          int64_t as_sm, int64_t as_sk, const uint8_t* w, int64_t ldw,
                          const float* ws, int64_t ws_sn, int64_t ws_sk, uint16_t* out, int64_t ldo,
                          int64_t M, int64_t N, int64_t K, float* partials, unsigned* counters,
                          hipStream_t stream) {
  const int64_t KB = cdiv(K, kGroup);
  dim3 grid(static_cast<unsigned>(p.strips), static_cast<unsigned>(p.splits),
            static_cast<unsigned>(cdiv(M, 64)));
#define MI355X_STREAM_ARGS                                                                        \
  q, ldq, as, as_sm, as_sk, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K, KB, p.kb_per_split,     \
      p.splits, partials, counters
  switch (p.token_tiles) {
    case 1: stream_gemm_kernel<1, ALIGNED, OutT><<<grid, kThreads, 0, stream>>>(MI355X_STREAM_ARGS); break;
    case 2: stream_gemm_kernel<2, ALIGNED, OutT><<<grid, kThreads, 0, stream>>>(MI355X_STREAM_ARGS); break;
    default: stream_gemm_kernel<4, ALIGNED, OutT><<<grid, kThreads, 0, stream>>>(MI355X_STREAM_ARGS); break;
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
    if (plan.strips > 0x7fffffffLL || plan.splits > 65535 || cdiv(M, 64) > 65535) return MI355X_FP8_ERR_UNSUPPORTED;
    unsigned* counters = static_cast<unsigned*>(workspace);
    float* partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterRegionBytes);
    launch_stream<ALIGNED, OutT>(plan, q, ldq, as, as_sm, as_sk, w, ldw, ws, ws_sn, ws_sk, out, ldo, M, N, K,
                                 partials, counters, stream);
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

}  // namespace mi355x
