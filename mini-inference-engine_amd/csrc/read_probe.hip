// Measurement helper for the decode roofline: one streaming read of a device buffer.
//
// The decode GEMM is bound by reading its weights once from HBM.  What a single launch of
// any kernel can reach over the same bytes (launch, ramp-up and drain included) is the
// ceiling its rate is compared with; this kernel is that reference: every byte read once
// with 16-byte loads, spread over all CUs, nothing else.  It has no counterpart in the
// reference engine.
#include "fp8_abi_internal.h"

namespace mi355x {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 4;

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const uint4* __restrict__ src, int64_t n16,
                                                                   uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kProbeThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
  for (; i + (kProbeUnroll - 1) * stride < n16; i += kProbeUnroll * stride) {
    uint4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = src[i + u * stride];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const uint4 v = src[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  // One word per workgroup, written only when the XOR is a fixed, practically impossible
  // value, so the loads cannot be removed and the sink costs no traffic.
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

}  // namespace

int launch_read_probe(const void* src, size_t bytes, void* sink, size_t sink_words, hipStream_t stream) {
  if (src == nullptr || sink == nullptr || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0)
    return MI355X_FP8_ERR_INVALID;
  const int64_t n16 = static_cast<int64_t>(bytes / 16);
  if (n16 == 0) return MI355X_FP8_OK;
  // Four loads in flight per lane, eight workgroups per CU at most.
  int64_t blocks = (n16 + kProbeThreads * kProbeUnroll - 1) / (kProbeThreads * kProbeUnroll);
  const int64_t cap = 8 * device_cus();
  if (blocks > cap) blocks = cap;
  if (static_cast<size_t>(blocks) > sink_words) return MI355X_FP8_ERR_WORKSPACE;
  read_probe_kernel<<<dim3(static_cast<unsigned>(blocks)), kProbeThreads, 0, stream>>>(
      static_cast<const uint4*>(src), n16, static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? MI355X_FP8_OK : MI355X_FP8_ERR_LAUNCH;
}

}  // namespace mi355x
