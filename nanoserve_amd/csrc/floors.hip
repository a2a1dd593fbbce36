// Measurement floors for the benchmark: what an empty launch and a plain
// streaming read of N bytes cost on this device, so the attention kernels'
// times can be put next to the best any kernel reading the same bytes does.
// Built into a library of its own (libnanoserve_floors.so) that only the
// benchmark loads; the product library and its header do not carry it.
//
// ns_stream_read reads `bytes` (a multiple of 16) from `src` with 16-byte
// loads, each workgroup folding what it read into one 32-bit value written to
// out[blockIdx.x] (so the loads cannot be dropped).  bytes == 0 launches
// `grid` workgroups that only write their zero: the launch floor.
#include "ns_common.h"

extern "C" int ns_stream_read(const void* src, int64_t bytes, uint32_t* out, int grid, void* stream);

namespace ns {
namespace {

constexpr int kReadThreads = 256;
constexpr int kReadUnroll = 8;  // 16-byte loads in flight per lane per trip

__global__ __launch_bounds__(kReadThreads) void stream_read_kernel(const u32x4* src, int64_t n16,
                                                                   uint32_t* out) {
  uint32_t acc = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kReadThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kReadThreads + threadIdx.x;
  for (; i + (kReadUnroll - 1) * stride < n16; i += kReadUnroll * stride) {
    u32x4 v[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  // Wave-level fold, then one store per wave into the workgroup's word.
  for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off);
  __shared__ uint32_t s_acc[kReadThreads / 64];
  if ((threadIdx.x & 63) == 0) s_acc[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t a = 0;
    for (int w = 0; w < kReadThreads / 64; ++w) a ^= s_acc[w];
    out[blockIdx.x] = a;
  }
}

}  // namespace
}  // namespace ns

extern "C" int ns_stream_read(const void* src, int64_t bytes, uint32_t* out, int grid, void* stream) {
  if (bytes < 0 || bytes % 16 != 0 || grid <= 0 || grid > 65535 || !out) return NS_ERR_INVALID_ARG;
  if (bytes > 0 && (!src || reinterpret_cast<uintptr_t>(src) % 16 != 0)) return NS_ERR_INVALID_ARG;
  const ns::u32x4* s = static_cast<const ns::u32x4*>(src);
  int64_t n16 = bytes / 16;
  void* args[] = {&s, &n16, &out};
  const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&ns::stream_read_kernel), dim3(grid),
                                       dim3(ns::kReadThreads), args, 0, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NS_OK : NS_ERR_HIP;
}
