// A model of the 256-row prefill kernel's K step (tile_gemm_256.hip at 256 x 224: 8 waves,
// each 64 x 112 = 4 x 7 MFMA tiles), with its parts switched on one at a time:
//   MFMA      v_mfma_f32_16x16x128_f8f6f4, operands in registers
//   FOLD      the per-K-group fold acc = fma(partial, scale, acc), software-pipelined by one
//             column tile as in the kernel
//   LDS       the operand fragments read from LDS every step (ds_read_b128, the kernel's
//             swizzled layout), W fragments streamed two ahead
//   BARRIER   a workgroup barrier per step
//   DMA       the next stage's operands (60 KiB per CU: 480 rows x 128 B at a 2560-byte row
//             stride) fetched by global_load_lds_dwordx4 at the start of the step and waited
//             for at its end, from a footprint that stays in L2 (1) or one that does not (2)
// on random e4m3 codes (the MFMA's power draw, and with it the clock, depends on the data) and
// on a structured pattern.  Reports us per step and the MFMA rate (2 * 256 * 224 * 128 flops
// per CU per step).
//
// Build and run: make -C mini-inference-engine_amd/microbench && mini-inference-engine_amd/microbench/_build/prefill_step
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

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ v4f mfma(v8i a, v8i b, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
__device__ __forceinline__ v8i frag(const uint4* t, int row, int g) {
  const uint4* p = t + row * 8;
  const uint4 lo = p[g ^ (row & 7)], hi = p[(g + 4) ^ (row & 7)];
  v8i r;
  r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w; r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
  return r;
}
__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
               : "memory");
}
// A hash of i as four e4m3 codes, none of them NaN (0x7f / 0xff).
__device__ __forceinline__ uint32_t codes(uint32_t i) {
  uint32_t x = i * 2654435761u + 12345u;
  x ^= x >> 15; x *= 2246822519u; x ^= x >> 13; x *= 3266489917u; x ^= x >> 16;
  for (int b = 0; b < 4; ++b)
    if (((x >> (8 * b)) & 0x7fu) == 0x7fu) x ^= 1u << (8 * b);
  return x;
}

template <bool LDS, bool FOLD, bool BAR, int DMA>
__global__ void __launch_bounds__(512, 2) step_model(float* out, int steps, int random, const uint8_t* src) {
  __shared__ uint4 st[480 * 8];   // the operand stage the fragments are read from
  __shared__ uint4 st2[480 * 8];  // the stage the DMA fills
  const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  for (int i = tid; i < 480 * 8; i += 512)
    st[i] = random ? make_uint4(codes(4 * i), codes(4 * i + 1), codes(4 * i + 2), codes(4 * i + 3))
                   : make_uint4(0x38383838u ^ i, 0x30303030u, 0x28282828u + i, 0x34343434u);
  __syncthreads();
  v4f acc[7][4];
  for (int i = 0; i < 7; ++i)
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  v8i breg[4], areg[7];
  for (int j = 0; j < 4; ++j) breg[j] = frag(st + 224 * 8, wm * 64 + 16 * j + r, g);
  for (int i = 0; i < 7; ++i) areg[i] = frag(st, wn * 112 + 16 * i + r, g);
  float sc[4];
  for (int j = 0; j < 4; ++j) sc[j] = 1.0f + 0.25f * j;
  const int64_t region = ((blockIdx.x / 8) % (DMA == 2 ? 64 : 4)) * 480;
  uint32_t off[8];
  for (int i = 0; i < 8; ++i) {
    const int blk = i * 8 + wave < 60 ? i * 8 + wave : 59;
    off[i] = static_cast<uint32_t>((region + blk * 8 + (lane >> 3)) * 2560 + (lane & 7) * 16);
  }
  const uint32_t lds2 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)st2));
  for (int it = 0; it < steps; ++it) {
    if (DMA) {
      const uint8_t* base = src + (it % 20) * 128;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        dma16(base, off[i], __builtin_amdgcn_readfirstlane(lds2 + (i * 8 + wave < 60 ? i * 8 + wave : 59) * 1024));
    }
    v8i b[4];
    for (int j = 0; j < 4; ++j) b[j] = LDS ? frag(st + 224 * 8, wm * 64 + 16 * j + r, g) : breg[j];
    v8i a0 = LDS ? frag(st, wn * 112 + r, g) : areg[0];
    v8i a1 = LDS ? frag(st, wn * 112 + 16 + r, g) : areg[1];
    v4f p[2][4];
#pragma unroll
    for (int i = 0; i <= 7; ++i) {
      v8i a2;
      if (i + 2 < 7) a2 = LDS ? frag(st, wn * 112 + 16 * (i + 2) + r, g) : areg[i + 2];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (i < 7) {
          if (FOLD) p[i & 1][j] = mfma(a0, b[j], v4f{0.f, 0.f, 0.f, 0.f});
          else acc[i][j] = mfma(a0, b[j], acc[i][j]);
        }
        if (FOLD && i > 0)
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[i - 1][j][v] = __builtin_fmaf(p[(i - 1) & 1][j][v], sc[j], acc[i - 1][j][v]);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (i < 7) {
        a0 = a1;
        if (i + 2 < 7) a1 = a2;
      }
    }
    if (DMA) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (BAR) {
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
    }
  }
  float sum = 0.f;
  for (int i = 0; i < 7; ++i)
    for (int j = 0; j < 4; ++j) sum += acc[i][j][0] + acc[i][j][3];
  out[blockIdx.x * 512 + tid] = sum;
}

template <bool L, bool F, bool B, int D>
static int run(const char* name, float* out, int random, const uint8_t* src, int cus) {
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  const int steps = 2000;
  for (int warm = 0; warm < 2; ++warm) step_model<L, F, B, D><<<cus, 512>>>(out, steps, random, src);
  CHECK(hipEventRecord(e0));
  step_model<L, F, B, D><<<cus, 512>>>(out, steps, random, src);
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  const double flops = static_cast<double>(cus) * steps * 256 * 224 * 128 * 2;
  std::printf("%-8s %-44s %.3f us/step  %.2f PFLOP/s\n", random ? "random" : "pattern", name, ms * 1000 / steps,
              flops / (ms * 1e-3) / 1e15);
  return 0;
}

int main() {
  int cus = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  float* out = nullptr;
  CHECK(hipMalloc(&out, static_cast<size_t>(cus) * 512 * 4));
  const size_t bytes = static_cast<size_t>(480 * 64 + 480) * 2560;
  uint8_t* src = nullptr;
  CHECK(hipMalloc(&src, bytes));
  CHECK(hipMemset(src, 0x38, bytes));
  for (int random : {0, 1}) {
    if (run<false, false, false, 0>("MFMA", out, random, src, cus) ||
        run<false, true, false, 0>("MFMA + fold", out, random, src, cus) ||
        run<true, true, true, 0>("MFMA + fold + LDS + barrier", out, random, src, cus) ||
        run<true, true, true, 1>("... + DMA from L2", out, random, src, cus) ||
        run<true, true, true, 2>("... + DMA from beyond L2", out, random, src, cus) ||
        run<false, false, true, 1>("MFMA + barrier + DMA from L2", out, random, src, cus) ||
        run<false, false, true, 2>("MFMA + barrier + DMA from beyond L2", out, random, src, cus))
      return 1;
  }
  return 0;
}
