// Microbenchmarks behind the prefill kernels' design numbers (gfx950, one GPU).
//
//   1. LDS read bandwidth: ds_read_b128 from a conflict-free pattern, per CU, as a function of
//      the waves per CU and the reads each wave keeps in flight.
//   2. LDS-DMA feed: global_load_lds_dwordx4 into a two-stage LDS ring, 60 KiB per step per
//      CU in rows of 128 bytes at a 2560-byte row stride (the 256 x 224 tile's operands), one
//      step in flight, from a footprint that stays in the XCD's L2 (4 row blocks per XCD) and
//      from one that does not (64 row blocks per XCD).
//
// Build and run: make -C mini-inference-engine_amd/microbench && mini-inference-engine_amd/microbench/_build/lds_feed
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#define CHECK(x)                                                                   \
  do {                                                                             \
    hipError_t e_ = (x);                                                           \
    if (e_ != hipSuccess) {                                                        \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));               \
      return 1;                                                                    \
    }                                                                              \
  } while (0)

typedef __attribute__((address_space(3))) void lds_void_t;

// N reads of 16 bytes per lane in flight, then a wait; lanes read consecutive 16-byte words.
template <int N>
__global__ void __launch_bounds__(1024) lds_read(uint32_t* sink, int iters) {
  __shared__ uint4 buf[8192];
  const int tid = threadIdx.x;
  for (int i = tid; i < 8192; i += blockDim.x) buf[i] = make_uint4(i, 3 * i, 5 * i, 7 * i);
  __syncthreads();
  const uint32_t addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)buf)) + (tid & 511) * 16;
  uint32_t x = 0;
  for (int it = 0; it < iters; ++it) {
    uint4 v[N];
#pragma unroll
    for (int u = 0; u < N; ++u) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v[u]) : "v"(addr), "i"(u * 1024));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int u = 0; u < N; ++u) x ^= v[u].x;
  }
  if (x == 0x12345678u) sink[blockIdx.x * blockDim.x + tid] = x;  // keeps the reads
}

__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
               : "memory");
}

__shared__ uint4 ring[2 * 480 * 8];

// 480 rows x 128 B per step (60 DMA instructions over 8 waves), K group `kb` of a [rows x 2560]
// matrix; workgroup b reads row block (b / 8) % regions, so the 32 CUs of an XCD share `regions`
// blocks.  The step's batch is waited for before the next is issued (one step in flight).
__global__ void __launch_bounds__(512) dma_feed(const uint8_t* src, int kgroups, int reps, int regions, uint32_t* sink) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t region = (blockIdx.x / 8) % regions;
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)ring));
  uint32_t off[8];
  for (int i = 0; i < 8; ++i) {
    const int blk = i * 8 + wave < 60 ? i * 8 + wave : 59;
    off[i] = static_cast<uint32_t>((region * 480 + blk * 8 + (lane >> 3)) * 2560 + (lane & 7) * 16);
  }
  int step = 0;
  for (int rep = 0; rep < reps; ++rep)
    for (int kb = 0; kb < kgroups; ++kb, ++step) {
      const uint8_t* base = src + kb * 128;
      const uint32_t st = lds0 + (step & 1) * 480 * 128;
#pragma unroll
      for (int i = 0; i < 8; ++i) dma16(base, off[i], __builtin_amdgcn_readfirstlane(st + (i * 8 + wave < 60 ? i * 8 + wave : 59) * 1024));
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
    }
  __syncthreads();
  if (ring[tid].x == 0xdeadbeefu) sink[tid] = 1;
}

template <int N>
static int run_lds(uint32_t* sink, int threads, int cus) {
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  const int iters = 4 * 32768 / N;
  lds_read<N><<<cus, threads>>>(sink, iters);
  CHECK(hipEventRecord(e0));
  lds_read<N><<<cus, threads>>>(sink, iters);
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  const double bytes = static_cast<double>(threads) * iters * N * 16;
  std::printf("lds_read   waves/CU %2d  reads in flight/wave %2d  %6.1f GB/s per CU\n", threads / 64, N,
              bytes / (ms * 1e-3) / 1e9);
  return 0;
}

int main() {
  int cus = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  uint32_t* sink = nullptr;
  CHECK(hipMalloc(&sink, 1 << 24));
  for (int threads : {256, 512, 1024})
    if (run_lds<2>(sink, threads, cus) || run_lds<4>(sink, threads, cus) || run_lds<8>(sink, threads, cus)) return 1;

  const size_t rows = 480 * 64 + 480;
  uint8_t* src = nullptr;
  CHECK(hipMalloc(&src, rows * 2560));
  CHECK(hipMemset(src, 0x38, rows * 2560));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  for (int regions : {4, 64}) {
    const int kg = 20, reps = 20;
    dma_feed<<<cus, 512>>>(src, kg, reps, regions, sink);
    CHECK(hipEventRecord(e0));
    dma_feed<<<cus, 512>>>(src, kg, reps, regions, sink);
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    const double bytes = static_cast<double>(cus) * reps * kg * 480 * 128;
    std::printf("dma_feed   row blocks/XCD %2d (%s)  %.3f us per 60 KiB step  %6.1f GB/s per CU\n", regions,
                regions == 4 ? "L2-resident" : "beyond L2  ", ms * 1000 / (reps * kg), bytes / (ms * 1e-3) / cus / 1e9);
  }
  return 0;
}
