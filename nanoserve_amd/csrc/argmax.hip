// argmax_rows: greedy token selection over the logits, one workgroup per row.
//
// Replaces logits.argmax(dim=-1) in the reference's greedy sampler
// (nanoserve/sampler.py:24-27).  A row of Qwen2.5-0.5B logits is 151936
// elements; 1024 threads each scan a strided slice with 16-byte loads, keep
// (value, index) with torch's rules -- the first index among equal maxima,
// and the first NaN if there is one -- and the workgroup reduces the 1024
// candidates with wave shuffles and LDS.
#include "ns_convert.h"

namespace ns {
namespace {

constexpr int kArgmaxThreads = 1024;

// Candidate order: NaN beats every number; among equal values (or two NaNs)
// the lower index wins.
__device__ __forceinline__ bool better(float v, int64_t i, float bv, int64_t bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

template <int DT>
__device__ __forceinline__ float elem_f32(const char* row, int64_t i);

template <>
__device__ __forceinline__ float elem_f32<NS_DTYPE_F32>(const char* row, int64_t i) {
  return reinterpret_cast<const float*>(row)[i];
}
template <>
__device__ __forceinline__ float elem_f32<NS_DTYPE_F16>(const char* row, int64_t i) {
  return static_cast<float>(reinterpret_cast<const _Float16*>(row)[i]);
}
template <>
__device__ __forceinline__ float elem_f32<NS_DTYPE_BF16>(const char* row, int64_t i) {
  return __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(row)[i]) << 16);
}

template <int DT>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(int64_t* out, const char* x,
                                                                      int64_t row_bytes, int64_t n) {
  constexpr int ESZ = DT == NS_DTYPE_F32 ? 4 : 2;
  constexpr int VEC = 16 / ESZ;
  const char* row = x + static_cast<int64_t>(blockIdx.x) * row_bytes;
  float bv = -INFINITY;
  int64_t bi = INT64_MAX;
  // Vector part: element ranges [VEC*j, VEC*j + VEC) for j = tid, tid + 1024, ...
  // (the row start is 16-byte aligned; the host checks it).
  const int64_t nvec = n / VEC;
  for (int64_t j = threadIdx.x; j < nvec; j += kArgmaxThreads) {
    const u32x4 w = reinterpret_cast<const u32x4*>(row)[j];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float v;
      if constexpr (DT == NS_DTYPE_F32) {
        v = __uint_as_float(w[e]);
      } else {
        const uint32_t h = (w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
        v = DT == NS_DTYPE_F16 ? static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)))
                               : __uint_as_float(h << 16);
      }
      const int64_t i = VEC * j + e;
      if (better(v, i, bv, bi)) {
        bv = v;
        bi = i;
      }
    }
  }
  for (int64_t i = VEC * nvec + threadIdx.x; i < n; i += kArgmaxThreads) {
    const float v = elem_f32<DT>(row, i);
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  // Wave reduction, then across the 16 waves through LDS.
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off);
    const int64_t oi = __shfl_xor(bi, off);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ int64_t si[kArgmaxThreads / 64];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; ++w) {
      if (better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    }
    out[blockIdx.x] = bi;
  }
}

}  // namespace
}  // namespace ns

extern "C" int ns_argmax_rows(int64_t* out, const void* x, int64_t x_stride_row, int64_t M, int64_t N,
                              int dtype, void* stream) {
  using namespace ns;
  const int esz = dtype_size(dtype);
  if (esz == 0) return NS_ERR_UNSUPPORTED;
  if (M < 0 || N <= 0 || x_stride_row < N) return NS_ERR_INVALID_ARG;
  if (M == 0) return NS_OK;
  if (!out || !x || M > 0x7FFFFFFF) return NS_ERR_INVALID_ARG;
  const int64_t row_bytes = x_stride_row * esz;
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || row_bytes % 16 != 0) return NS_ERR_INVALID_ARG;
  const void* fn = dtype == NS_DTYPE_F32 ? reinterpret_cast<const void*>(&argmax_rows_kernel<NS_DTYPE_F32>)
                 : dtype == NS_DTYPE_F16 ? reinterpret_cast<const void*>(&argmax_rows_kernel<NS_DTYPE_F16>)
                                         : reinterpret_cast<const void*>(&argmax_rows_kernel<NS_DTYPE_BF16>);
  const char* xp = static_cast<const char*>(x);
  void* args[] = {&out, const_cast<char**>(&xp), const_cast<int64_t*>(&row_bytes), &N};
  const hipError_t e = hipLaunchKernel(fn, dim3(static_cast<unsigned>(M)), dim3(kArgmaxThreads), args, 0,
                                       static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NS_OK : NS_ERR_HIP;
}
