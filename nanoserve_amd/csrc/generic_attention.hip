// Generic paged attention: one wave per (token row, query head), float32
// arithmetic, any float dtype, head size up to 256 and any block size.
//
// The reference computes every row as gather + masked SDPA
// (nanoserve/attention.py:118-150 for variable-length rows, :154-190 for
// decode-only batches): the row of sequence s at query offset j sees keys
// 0 .. seq_len - query_len + j.  Here the wave walks those keys 64 at a time,
// one key per lane: the lane's dot product with the query (held in LDS as
// float32), scaled, joins the wave's running maximum and sum (online
// softmax); then every lane adds the chunk's keys' weighted values into the
// output dims it owns (lane, lane + 64, ...), one key at a time with the
// weight and row offset broadcast across the wave.  Only keys below the row's
// limit are read; a block id outside the cache makes the row NaN and is never
// dereferenced; a row without keys is zero.
//
// These shapes are outside the serving configurations, so the kernel is
// plain: no LDS staging of K/V, no MFMA.  The MFMA kernels in
// paged_attention.hip take float16/bfloat16 at head sizes 64 and 128.
#include "generic_attention.h"
#include "ns_common.h"

namespace ns {
namespace {

template <class T>
__device__ __forceinline__ float as_f32(T x) {
  return static_cast<float>(x);
}

// DL: output dims per lane (head_dim <= 64 * DL).
template <class T, int DL>
__global__ __launch_bounds__(64) void paged_attention_generic_kernel(GenericAttnParams p) {
  __shared__ float q_lds[64 * DL];
  const int lane = threadIdx.x;
  const int64_t t = blockIdx.x;
  const int h = blockIdx.y;
  const int D = p.head_dim, bs = p.block_size;
  const int kvh = h / (p.num_heads / p.num_kv_heads);

  // The row's sequence: the last s with query_start_loc[s] <= t.
  int s;
  int64_t row0, ql;
  if (p.decode_only) {
    s = static_cast<int>(t);
    row0 = t;
    ql = 1;
  } else {
    int lo = 0, hi = p.num_seqs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (load_index(p.qsl, mid, p.qsl64) <= t) lo = mid;
      else hi = mid - 1;
    }
    s = lo;
    row0 = load_index(p.qsl, s, p.qsl64);
    ql = load_index(p.qsl, s + 1, p.qsl64) - row0;
  }
  int64_t L = load_index(p.seq_lens, s, p.sl64);
  L = L < 0 ? 0 : (L < p.max_ctx ? L : p.max_ctx);
  const bool covered = t >= row0 && t < row0 + ql;  // offsets that leave a row to no sequence: zero
  const int64_t limit = L - ql + (t - row0);        // the row's last key
  const int64_t nkeys = !covered || limit < 0 ? 0 : (limit + 1 < L ? limit + 1 : L);

  const T* qrow = static_cast<const T*>(p.query) + (t * p.num_heads + h) * D;
  for (int d = lane; d < 64 * DL; d += 64) q_lds[d] = d < D ? as_f32(qrow[d]) : 0.f;
  __syncthreads();

  const T* kc = static_cast<const T*>(p.k_cache);
  const T* vc = static_cast<const T*>(p.v_cache);
  const int64_t bt_row = static_cast<int64_t>(s) * p.bt_stride;
  float m = -INFINITY, l = 0.f, o[DL];
#pragma unroll
  for (int j = 0; j < DL; ++j) o[j] = 0.f;
  int bad = 0;
  for (int64_t c0 = 0; c0 < nkeys; c0 += 64) {
    const int64_t key = c0 + lane;
    int64_t row = 0;  // element offset of this lane's key (its K and V rows)
    bool ok = false;
    if (key < nkeys) {
      const int64_t blk = load_index(p.bt, bt_row + key / bs, p.bt64);
      if (blk < 0 || blk >= p.num_blocks) {
        bad = 1;
      } else {
        ok = true;
        row = ((blk * bs + key % bs) * p.num_kv_heads + kvh) * D;
      }
    }
    float sc = -INFINITY;
    if (ok) {
      float acc = 0.f;
      for (int d = 0; d < D; ++d) acc = __builtin_fmaf(q_lds[d], as_f32(kc[row + d]), acc);
      sc = acc * p.scale;
    }
    float cm = sc;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) cm = fmaxf(cm, __shfl_xor(cm, off));
    const float m_new = fmaxf(m, cm);
    if (m_new == -INFINITY) continue;  // nothing valid so far
    const float alpha = expf(m - m_new);
    const float pk = ok ? expf(sc - m_new) : 0.f;
    float ps = pk;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ps += __shfl_xor(ps, off);
    l = l * alpha + ps;
    m = m_new;
#pragma unroll
    for (int j = 0; j < DL; ++j) o[j] *= alpha;
    const int nk = nkeys - c0 < 64 ? static_cast<int>(nkeys - c0) : 64;
    const uint32_t row_lo = static_cast<uint32_t>(row), row_hi = static_cast<uint32_t>(row >> 32);
    for (int kk = 0; kk < nk; ++kk) {
      const float w = __shfl(pk, kk);
      if (w == 0.f) continue;  // uniform: the weight is broadcast
      const int64_t r = static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(__shfl(row_hi, kk))) << 32) |
                                             static_cast<uint32_t>(__shfl(row_lo, kk)));
#pragma unroll
      for (int j = 0; j < DL; ++j) {
        const int d = lane + 64 * j;
        if (d < D) o[j] = __builtin_fmaf(w, as_f32(vc[r + d]), o[j]);
      }
    }
  }
  bad = __builtin_amdgcn_ballot_w64(bad != 0) != 0;

  T* orow = static_cast<T*>(p.out) + (t * p.num_heads + h) * D;
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int j = 0; j < DL; ++j) {
    const int d = lane + 64 * j;
    if (d < D) orow[d] = static_cast<T>(bad ? NAN : o[j] * inv);
  }
}

template <class T>
hipError_t launch_typed(const GenericAttnParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.num_tokens), static_cast<unsigned>(p.num_heads));
  void* args[] = {const_cast<GenericAttnParams*>(&p)};
  const void* fn = p.head_dim <= 64    ? reinterpret_cast<const void*>(&paged_attention_generic_kernel<T, 1>)
                   : p.head_dim <= 128 ? reinterpret_cast<const void*>(&paged_attention_generic_kernel<T, 2>)
                                       : reinterpret_cast<const void*>(&paged_attention_generic_kernel<T, 4>);
  return hipLaunchKernel(fn, grid, dim3(64), args, 0, stream);
}

}  // namespace

hipError_t launch_generic_attention(const GenericAttnParams& p, int dtype, hipStream_t stream) {
  if (p.head_dim <= 0 || p.head_dim > kGenericMaxHeadDim || p.num_tokens <= 0 || p.num_tokens > 0x7FFFFFFF ||
      p.num_heads <= 0 || p.num_heads > 65535)
    return hipErrorInvalidValue;
  switch (dtype) {
    case NS_DTYPE_F32: return launch_typed<float>(p, stream);
    case NS_DTYPE_F16: return launch_typed<_Float16>(p, stream);
    case NS_DTYPE_BF16: return launch_typed<__bf16>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ns
