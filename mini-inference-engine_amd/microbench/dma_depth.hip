// Per-CU operand feed rate of one K step of the 128 x 64 prefill tile (gfx950, one GPU):
// 192 rows x 128 B (the 128 activation rows and 64 weight rows of a K group) per step, 256
// threads, one workgroup per CU (100 KiB of dynamic LDS), D steps in flight:
//   dma_feed:  global_load_lds_dwordx4 into a D-stage LDS ring, explicit vmcnt waits, with or
//              without a workgroup barrier per step;
//   vgpr_feed: plain 16-byte global loads into registers (folded into a checksum).
// The footprint is one row block per XCD (L2-resident) or four (spilling past L2).
//
// Build and run: make -C mini-inference-engine_amd/microbench && mini-inference-engine_amd/microbench/_build/dma_depth
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#define CHECK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_)); return 1; } } while (0)
typedef __attribute__((address_space(3))) void lds_void_t;
constexpr int kRows = 192, kPer = 6, kLd = 9728;

__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds) : "memory");
}
template <int N> __device__ __forceinline__ void vmwait() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

extern __shared__ uint4 dyn[];

template <int D, bool BAR>
__global__ void __launch_bounds__(256) dma_feed(const uint8_t* src, int kgroups, int reps, int regions, uint32_t* sink) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t region = (blockIdx.x / 8) % regions;
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)dyn));
  uint32_t off[kPer];
  for (int i = 0; i < kPer; ++i) off[i] = static_cast<uint32_t>((region * kRows + (i * 4 + wave) * 8 + (lane >> 3)) * kLd + (lane & 7) * 16);
  const int total = kgroups * reps;
  auto issue = [&](int s) {
    const uint8_t* base = src + (s % kgroups) * 128;
    const uint32_t st = lds0 + (s % D) * kRows * 128;
#pragma unroll
    for (int i = 0; i < kPer; ++i) dma16(base, off[i], __builtin_amdgcn_readfirstlane(st + (i * 4 + wave) * 1024));
  };
  for (int s = 0; s < D - 1; ++s) issue(s);
  for (int s = 0; s < total; ++s) {
    if (s + D - 1 < total) issue(s + D - 1);
    vmwait<kPer * (D - 1)>();
    if (BAR) __builtin_amdgcn_s_barrier();
  }
  vmwait<0>();
  __syncthreads();
  if (dyn[tid].x == 0xdeadbeefu) sink[tid] = 1;
}

template <int D>
__global__ void __launch_bounds__(256) vgpr_feed(const uint8_t* src, int kgroups, int reps, int regions, uint32_t* sink) {
  const int tid = threadIdx.x;
  const int64_t region = (blockIdx.x / 8) % regions;
  int64_t off[kPer];
  for (int i = 0; i < kPer; ++i) off[i] = (region * kRows + i * 32 + (tid >> 3)) * kLd + (tid & 7) * 16;
  uint4 buf[D][kPer];
  uint32_t x = 0;
  const int total = kgroups * reps;
  auto issue = [&](int s, uint4 (&b)[kPer]) {
    const uint8_t* base = src + (s % kgroups) * 128;
#pragma unroll
    for (int i = 0; i < kPer; ++i) b[i] = *reinterpret_cast<const uint4*>(base + off[i]);
  };
#pragma unroll
  for (int d = 0; d < D - 1; ++d) issue(d, buf[d]);
  for (int s0 = 0; s0 < total; s0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      issue(s0 + d + D - 1, buf[(d + D - 1) % D]);
#pragma unroll
      for (int i = 0; i < kPer; ++i) x ^= buf[d][i].x ^ buf[d][i].y ^ buf[d][i].z ^ buf[d][i].w;
    }
  }
  if (x == 0x12345678u) sink[blockIdx.x * 256 + tid] = x;
}

template <typename F>
static int timeit(const char* name, F launch, int cus, int total) {
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0)); CHECK(hipEventCreate(&e1));
  launch();
  CHECK(hipEventRecord(e0));
  launch();
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0; CHECK(hipEventElapsedTime(&ms, e0, e1));
  const double bytes = static_cast<double>(cus) * total * kRows * 128;
  std::printf("%-28s %.3f us/step  %6.1f GB/s per CU\n", name, ms * 1000 / total, bytes / (ms * 1e-3) / cus / 1e9);
  return 0;
}

int main() {
  int cus = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  uint32_t* sink; CHECK(hipMalloc(&sink, 1 << 24));
  const size_t rows = kRows * 64 + kRows;
  uint8_t* src; CHECK(hipMalloc(&src, rows * kLd)); CHECK(hipMemset(src, 0x38, rows * kLd));
  const int kg = 76, reps = 10, total = kg * reps;
  for (int regions : {1, 4}) {
    std::printf("row blocks per XCD: %d\n", regions);
    // dynamic LDS of 100 KiB: one workgroup per CU, as in the kernel
    const size_t lds = 100 * 1024;
#define DMA(D, B) timeit("dma D=" #D " bar=" #B, [&] { dma_feed<D, B><<<cus, 256, lds>>>(src, kg, reps, regions, sink); }, cus, total)
#define VG(D) timeit("vgpr D=" #D, [&] { vgpr_feed<D><<<cus, 256, lds>>>(src, kg, reps, regions, sink); }, cus, total)
    if (DMA(1, true) || DMA(2, true) || DMA(3, true) || DMA(4, true) || DMA(4, false)) return 1;
    if (VG(1) || VG(2) || VG(3) || VG(4)) return 1;
  }
  return 0;
}
