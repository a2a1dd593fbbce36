// int4_linear: y = x · dequant(W)^T + bias with W stored as group-wise
// asymmetric INT4 (the reference's QuantLinear "int4" format), dequantised in
// registers on its way into the MFMA.
//
// Replaces QuantLinear.forward (reference nanoserve/quant.py:157-158), which
// expands the whole weight to the model dtype on every call
// (dequantize_int4, quant.py:83-95) and then runs F.linear: per call it writes
// and re-reads N·K·2 bytes beside the GEMM.  Here each weight byte is read once
// per output tile and never expanded in memory.
//
// Format (quant.py:53-80): qweight [N, K/2] uint8, two 4-bit codes per byte,
// even k in the low nibble and odd k in the high nibble; scales [N, K/gs]
// float32; zeros [N, K/gs] uint8.  Weight (n, k) is
//     w = (q - zero) * scale          (float32)
// rounded to the model dtype, exactly as dequantize_int4 computes it, so the
// MFMA sees the reference's own dequantised weights.
//
// Tiling (gfx950, wave64): a workgroup owns 16 output features (one MFMA row
// tile of W) and MT tokens (MT/16 MFMA column tiles of x^T).  Its four waves
// split K into four contiguous ranges and reduce through LDS.  Per 32-wide K
// step a lane loads 4 bytes of packed weights (row n0 + lane%16, codes
// 8·(lane/16) .. +7 of the step: exactly its MFMA A operand) and one 16-byte
// row piece of x per column tile (its B operand).  The result D[n][m] lands as
// four consecutive features of one token per lane: one 8-byte store.
#include "ns_common.h"

namespace ns {
namespace {

struct Int4LinearParams {
  void* out;              // [M, N] contiguous, model dtype
  const char* x;          // [M, K] rows of x_stride elements
  int64_t x_stride;
  const uint8_t* qweight; // [N, K/2]
  const float* scales;    // [N, G]
  const uint8_t* zeros;   // [N, G]
  const void* bias;       // [N] model dtype, or null
  int M, N, K, group_size, groups;
};

template <class DT>
__device__ __forceinline__ typename DT::T to_model(float x) {
  return static_cast<typename DT::T>(x);
}

template <class DT>
__device__ __forceinline__ float from_model(typename DT::T x) {
  return static_cast<float>(x);
}

template <class DT, int MT>
__global__ __launch_bounds__(256) void int4_linear_kernel(Int4LinearParams p) {
  constexpr int NT = MT / 16;  // MFMA column tiles
  using V8 = typename DT::vec8;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * MT;
  const int row = lane & 15;      // A row (feature) / B column (token) of this lane
  const int kq = 8 * (lane >> 4); // this lane's 8 k-slots within a K step

  const int steps = p.K / 32;
  const int s_begin = (steps * wave) / 4;
  const int s_end = (steps * (wave + 1)) / 4;

  const int n = n0 + row;
  const uint8_t* wrow = p.qweight + static_cast<int64_t>(n) * (p.K / 2);
  const float* srow = p.scales + static_cast<int64_t>(n) * p.groups;
  const uint8_t* zrow = p.zeros + static_cast<int64_t>(n) * p.groups;
  const char* xrow[NT];
  bool xok[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int m = m0 + 16 * t + row;
    xok[t] = m < p.M;
    xrow[t] = p.x + static_cast<int64_t>(xok[t] ? m : 0) * p.x_stride * sizeof(typename DT::T);
  }

  floatx4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int s = s_begin; s < s_end; ++s) {
    const int k = 32 * s + kq;
    const uint32_t codes = *reinterpret_cast<const uint32_t*>(wrow + k / 2);
    const int g = k / p.group_size;
    const float scale = srow[g];
    const float zero = static_cast<float>(zrow[g]);
    V8 a;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float q = static_cast<float>((codes >> (4 * e)) & 0xFu);
      a[e] = to_model<DT>((q - zero) * scale);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const V8 b = xok[t] ? load16<DT>(xrow[t] + k * sizeof(typename DT::T)) : zero8<DT>();
      acc[t] = mfma16x16x32(DT{}, a, b, acc[t]);
    }
  }

  // Waves 1-3 hand their partial sums to wave 0.
  __shared__ floatx4 red[3][NT][64];
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t) red[wave - 1][t][lane] = acc[t];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int w = 0; w < 3; ++w) acc[t] += red[w][t][lane];
  }

  // D[4·(lane/16) + r][lane%16]: features nf .. nf+3 of token m.
  const int nf = n0 + 4 * (lane >> 4);
  float bias[4] = {0.f, 0.f, 0.f, 0.f};
  if (p.bias) {
    const typename DT::T* b = static_cast<const typename DT::T*>(p.bias) + nf;
#pragma unroll
    for (int r = 0; r < 4; ++r) bias[r] = from_model<DT>(b[r]);
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int m = m0 + 16 * t + row;
    if (m >= p.M) continue;
    typename DT::vec4 o;
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = to_model<DT>(acc[t][r] + bias[r]);
    *reinterpret_cast<typename DT::vec4*>(static_cast<typename DT::T*>(p.out) +
                                          static_cast<int64_t>(m) * p.N + nf) = o;
  }
}

template <class DT>
hipError_t launch_int4_linear(const Int4LinearParams& p, hipStream_t stream) {
  void* args[] = {const_cast<Int4LinearParams*>(&p)};
  const void* fn;
  int mt;
  if (p.M <= 16) {
    fn = reinterpret_cast<const void*>(&int4_linear_kernel<DT, 16>);
    mt = 16;
  } else if (p.M <= 32) {
    fn = reinterpret_cast<const void*>(&int4_linear_kernel<DT, 32>);
    mt = 32;
  } else {
    fn = reinterpret_cast<const void*>(&int4_linear_kernel<DT, 64>);
    mt = 64;
  }
  const dim3 grid(static_cast<unsigned>(p.N / 16), static_cast<unsigned>((p.M + mt - 1) / mt));
  return hipLaunchKernel(fn, grid, dim3(256), args, 0, stream);
}

bool aligned(const void* q, uintptr_t a) { return reinterpret_cast<uintptr_t>(q) % a == 0; }

}  // namespace
}  // namespace ns

extern "C" int ns_int4_linear(void* out, const void* x, int64_t x_stride_row,
                              const void* qweight, const void* scales, const void* zeros, const void* bias,
                              int64_t M, int N, int K, int group_size, int dtype, void* stream) {
  using namespace ns;
  if (dtype != NS_DTYPE_F16 && dtype != NS_DTYPE_BF16) return NS_ERR_UNSUPPORTED;
  if (M < 0 || N <= 0 || K <= 0 || group_size <= 0) return NS_ERR_INVALID_ARG;
  if (M == 0) return NS_OK;
  if (!out || !x || !qweight || !scales || !zeros) return NS_ERR_INVALID_ARG;
  // One MFMA row tile per 16 features; a K step of 32 lies inside one group.
  if (N % 16 != 0 || K % 32 != 0 || group_size % 32 != 0 || K % group_size != 0) return NS_ERR_UNSUPPORTED;
  if ((M + 15) / 16 > 65535) return NS_ERR_INVALID_ARG;  // grid.y bound of the smallest tile
  if (x_stride_row < K || x_stride_row % 8 != 0 || !aligned(x, 16) || !aligned(out, 8) ||
      !aligned(qweight, 4) || !aligned(scales, 4) || (bias && !aligned(bias, 2)))
    return NS_ERR_INVALID_ARG;

  Int4LinearParams p;
  p.out = out;
  p.x = static_cast<const char*>(x);
  p.x_stride = x_stride_row;
  p.qweight = static_cast<const uint8_t*>(qweight);
  p.scales = static_cast<const float*>(scales);
  p.zeros = static_cast<const uint8_t*>(zeros);
  p.bias = bias;
  p.M = static_cast<int>(M);
  p.N = N;
  p.K = K;
  p.group_size = group_size;
  p.groups = K / group_size;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t e = dtype == NS_DTYPE_F16 ? launch_int4_linear<F16>(p, s) : launch_int4_linear<BF16>(p, s);
  return e == hipSuccess ? NS_OK : NS_ERR_HIP;
}
