// argmax_rows: greedy token selection over the logits.
//
// Replaces logits.argmax(dim=-1) in the reference's greedy sampler
// (nanoserve/sampler.py:24-27).  A row of Qwen2.5-0.5B logits is 151936
// elements; one workgroup per row is VALU-bound on its single CU, so each row
// is cut into slices of 4096 elements scanned by separate workgroups (38 per
// row, over 1200 for a batch of 32) and a second small launch combines the
// slices.
//
// torch's rules -- the first index among equal maxima, the first NaN if the
// row holds one -- are folded into one 64-bit key per candidate:
//     key = order(value) << 32 | (2^32 - 1 - index)
// where order() maps floats to unsigned integers in value order (+0 and -0
// equal, every NaN above +inf), so the largest key is the answer.
#include "ns_convert.h"

namespace ns {
namespace {

constexpr int kSliceThreads = 256;
constexpr int kSliceElems = 4096;  // elements per workgroup slice

__device__ __forceinline__ uint64_t key_of(float v, uint32_t idx) {
  uint32_t u = __float_as_uint(v);
  uint32_t ord;
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) {
    ord = 0xFFFFFFFFu;                   // NaN
  } else {
    if (u == 0x80000000u) u = 0u;        // -0 == +0
    ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
  return (static_cast<uint64_t>(ord) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max(uint64_t k) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) k = max_u64(k, __shfl_xor(k, off));
  return k;
}

template <int DT>
__device__ __forceinline__ float elem_f32(const char* row, int64_t i) {
  if constexpr (DT == NS_DTYPE_F32) return reinterpret_cast<const float*>(row)[i];
  const uint16_t h = reinterpret_cast<const uint16_t*>(row)[i];
  if constexpr (DT == NS_DTYPE_F16) return static_cast<float>(__builtin_bit_cast(_Float16, h));
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Stage 1: grid (slices, rows).  Writes each slice's best key to keys[row * slices + slice].
template <int DT>
__global__ __launch_bounds__(kSliceThreads) void argmax_slices_kernel(uint64_t* keys, const char* x,
                                                                       int64_t row_bytes, int64_t n) {
  constexpr int ESZ = DT == NS_DTYPE_F32 ? 4 : 2;
  constexpr int VEC = 16 / ESZ;
  const char* row = x + static_cast<int64_t>(blockIdx.y) * row_bytes;
  const int64_t s0 = static_cast<int64_t>(blockIdx.x) * kSliceElems;
  const int64_t s1 = s0 + kSliceElems < n ? s0 + kSliceElems : n;
  uint64_t best = 0;
  // Whole 16-byte vectors of the slice (slice starts are multiples of 4096
  // elements and rows are 16-byte aligned), then the row's ragged tail.
  const int64_t v1 = s1 / VEC;
  for (int64_t j = s0 / VEC + threadIdx.x; j < v1; j += kSliceThreads) {
    const u32x4 w = reinterpret_cast<const u32x4*>(row)[j];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float v;
      if constexpr (DT == NS_DTYPE_F32) {
        v = __uint_as_float(w[e]);
      } else {
        const uint16_t h = static_cast<uint16_t>((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
        v = DT == NS_DTYPE_F16 ? static_cast<float>(__builtin_bit_cast(_Float16, h))
                               : __uint_as_float(static_cast<uint32_t>(h) << 16);
      }
      best = max_u64(best, key_of(v, static_cast<uint32_t>(VEC * j + e)));
    }
  }
  for (int64_t i = VEC * v1 + threadIdx.x; i < s1; i += kSliceThreads)
    best = max_u64(best, key_of(elem_f32<DT>(row, i), static_cast<uint32_t>(i)));
  best = wave_max(best);
  __shared__ uint64_t wk[kSliceThreads / 64];
  if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kSliceThreads / 64; ++w) best = max_u64(best, wk[w]);
    keys[static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x] = best;
  }
}

// Stage 2: one wave per row combines its slices.
__global__ __launch_bounds__(64) void argmax_combine_kernel(int64_t* out, const uint64_t* keys, int slices) {
  const uint64_t* k = keys + static_cast<int64_t>(blockIdx.x) * slices;
  uint64_t best = 0;
  for (int i = threadIdx.x; i < slices; i += 64) best = max_u64(best, k[i]);
  best = wave_max(best);
  if (threadIdx.x == 0) out[blockIdx.x] = static_cast<int64_t>(0xFFFFFFFFu - static_cast<uint32_t>(best));
}

int64_t slices_for(int64_t n) { return (n + kSliceElems - 1) / kSliceElems; }

}  // namespace
}  // namespace ns

extern "C" size_t ns_argmax_rows_workspace_size(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return 0;
  return static_cast<size_t>(M * ns::slices_for(N)) * sizeof(uint64_t);
}

extern "C" int ns_argmax_rows(int64_t* out, const void* x, int64_t x_stride_row, int64_t M, int64_t N,
                              int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace ns;
  const int esz = dtype_size(dtype);
  if (esz == 0) return NS_ERR_UNSUPPORTED;
  if (M < 0 || N <= 0 || x_stride_row < N || N > 0xFFFFFFFFll) return NS_ERR_INVALID_ARG;
  if (M == 0) return NS_OK;
  if (!out || !x || M > 65535) return NS_ERR_INVALID_ARG;
  const int64_t row_bytes = x_stride_row * esz;
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || row_bytes % 16 != 0) return NS_ERR_INVALID_ARG;
  const int64_t slices = slices_for(N);
  if (!workspace || workspace_bytes < static_cast<size_t>(M * slices) * sizeof(uint64_t) ||
      reinterpret_cast<uintptr_t>(workspace) % 8 != 0)
    return NS_ERR_WORKSPACE;
  const void* fn = dtype == NS_DTYPE_F32 ? reinterpret_cast<const void*>(&argmax_slices_kernel<NS_DTYPE_F32>)
                 : dtype == NS_DTYPE_F16 ? reinterpret_cast<const void*>(&argmax_slices_kernel<NS_DTYPE_F16>)
                                         : reinterpret_cast<const void*>(&argmax_slices_kernel<NS_DTYPE_BF16>);
  uint64_t* keys = static_cast<uint64_t*>(workspace);
  const char* xp = static_cast<const char*>(x);
  int64_t rb = row_bytes, n = N;
  void* args1[] = {&keys, &xp, &rb, &n};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipLaunchKernel(fn, dim3(static_cast<unsigned>(slices), static_cast<unsigned>(M)),
                                 dim3(kSliceThreads), args1, 0, s);
  if (e != hipSuccess) return NS_ERR_HIP;
  int nslices = static_cast<int>(slices);
  const uint64_t* ck = keys;
  void* args2[] = {&out, &ck, &nslices};
  e = hipLaunchKernel(reinterpret_cast<const void*>(&argmax_combine_kernel), dim3(static_cast<unsigned>(M)),
                      dim3(64), args2, 0, s);
  return e == hipSuccess ? NS_OK : NS_ERR_HIP;
}
