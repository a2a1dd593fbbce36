// rope_reshape_and_cache: the rotary embedding of this step's Q and K fused
// with the paged-cache write of K and V.
//
// Replaces, at the attention call site (reference nanoserve/qwen2.py:53-57),
// RotaryEmbedding.apply (reference nanoserve/layers.py:84-88)
//     q = q * cos + rotate_half(q) * sin,   k likewise,
//     rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2])
// followed by PagedKVCache.write (reference nanoserve/kv_cache.py:73-81) of
// the rotated K and of V.  The reference runs these as separate elementwise
// kernels (two products, a negation, a concatenation and a sum per tensor)
// plus two index_copy_ launches; here one launch reads every Q/K/V row once,
// writes rotated Q back and rotated K and V into their cache slots.
//
// Results are bit-exact with the reference's tensor arithmetic: each torch
// op on f16/bf16 tensors computes in f32 and rounds its result to the
// tensor dtype, so
//     out[i]       = R(R(x[i] * cos[i])       - R(x[i+h] * sin[i]))
//     out[i+h]     = R(R(x[i+h] * cos[i+h])   + R(x[i] * sin[i+h]))
// with R = round to nearest even in the model dtype (the identity after each
// f32 op for f32 tensors), evaluated here with explicit roundings and no
// contraction into fused multiply-adds.
//
// Work split: one thread per (row, chunk) where a row is one head of one token
// of Q, K or V and a thread owns the 16-byte chunk c of the row's first half
// together with the matching chunk of its second half (the pair rotate_half
// couples).  Threads are numbered query rows first, then key rows, then value
// rows, each as (token, head, chunk) with the chunk fastest, so a wave works
// on one kind of row and neighbouring lanes touch neighbouring bytes.
#include "ns_convert.h"

namespace ns {
namespace {

struct RopeCacheParams {
  char* q_out;             // [T, Hq, D] contiguous, model dtype (may alias q)
  const char* q;
  const char* key;
  const char* value;
  const char* cos;
  const char* sin;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, cs_st;  // element strides
  char* k_cache;
  char* v_cache;
  const void* slots;
  int slots64;
  int num_heads, num_kv_heads, head_dim;
  int64_t num_slots;
  uint32_t cph;            // chunk pairs per row
  uint32_t nq, nk;         // query / key threads (value threads = nk)
};

// Element access and exact conversions for one storage dtype.
template <int DT>
struct Elem;

template <>
struct Elem<NS_DTYPE_F32> {
  static constexpr int size = 4;
  static __device__ __forceinline__ uint32_t get(const u32x4& w, int e) { return w[e]; }
  static __device__ __forceinline__ float to_f32(uint32_t b) { return __uint_as_float(b); }
  static __device__ __forceinline__ uint32_t from_f32(float x) { return __float_as_uint(x); }
};

// f16 and bf16 use the hardware conversions: the kernels run with round to
// nearest even and denormals kept for f32 and f16 (the default float mode of
// HIP kernels), which is exactly what torch's per-op rounding does.
template <>
struct Elem<NS_DTYPE_F16> {
  static constexpr int size = 2;
  static __device__ __forceinline__ uint32_t get(const u32x4& w, int e) {
    return (w[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
  }
  static __device__ __forceinline__ float to_f32(uint32_t b) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
  }
  static __device__ __forceinline__ uint32_t from_f32(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
  }
};

template <>
struct Elem<NS_DTYPE_BF16> {
  static constexpr int size = 2;
  static __device__ __forceinline__ uint32_t get(const u32x4& w, int e) {
    return (w[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
  }
  static __device__ __forceinline__ float to_f32(uint32_t b) { return __uint_as_float(b << 16); }
  static __device__ __forceinline__ uint32_t from_f32(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
  }
};

// Round an f32 value to dtype DT and back (the identity for f32).
template <int DT>
__device__ __forceinline__ float round_to(float x) {
  return Elem<DT>::to_f32(Elem<DT>::from_f32(x));
}

// Store N values, given as bit patterns of dtype DT, at dst (16-byte aligned
// when N * size is 16 or 32, 8-byte aligned when it is 8).
template <int DT, int N>
__device__ __forceinline__ void store_elems(char* dst, const uint32_t (&bits)[N]) {
  constexpr int bytes = N * Elem<DT>::size;
  uint32_t w[bytes / 4];
  if constexpr (Elem<DT>::size == 4) {
#pragma unroll
    for (int e = 0; e < N; ++e) w[e] = bits[e];
  } else {
#pragma unroll
    for (int i = 0; i < bytes / 4; ++i) w[i] = (bits[2 * i] & 0xFFFFu) | (bits[2 * i + 1] << 16);
  }
  if constexpr (bytes == 8) {
    *reinterpret_cast<u32x2*>(dst) = u32x2{w[0], w[1]};
  } else {
#pragma unroll
    for (int i = 0; i < bytes / 16; ++i)
      *reinterpret_cast<u32x4*>(dst + 16 * i) = u32x4{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
  }
}

template <int DT, int CT>
__global__ __launch_bounds__(256) void rope_reshape_and_cache_kernel(RopeCacheParams p) {
#pragma clang fp contract(off)
  using M = Elem<DT>;
  constexpr int EPT = 16 / M::size;  // model elements per 16-byte chunk
  const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
  int kind;
  uint32_t rel;
  if (idx < p.nq) {
    kind = 0;
    rel = idx;
  } else if (idx < p.nq + p.nk) {
    kind = 1;
    rel = idx - p.nq;
  } else if (idx < p.nq + 2 * p.nk) {
    kind = 2;
    rel = idx - p.nq - p.nk;
  } else {
    return;
  }
  const uint32_t heads = kind == 0 ? p.num_heads : p.num_kv_heads;
  const uint32_t c = rel % p.cph;
  const uint32_t r = rel / p.cph;
  const uint32_t h = r % heads;
  const int64_t t = r / heads;
  const int half = p.head_dim / 2;

  int64_t slot = 0;
  if (kind != 0) {
    slot = load_index(p.slots, t, p.slots64);
    if (slot < 0 || slot >= p.num_slots) return;  // padding / invalid slot: never written
  }
  const char* src = kind == 0 ? p.q + (t * p.q_st + h * p.q_sh) * M::size
                  : kind == 1 ? p.key + (t * p.k_st + h * p.k_sh) * M::size
                              : p.value + (t * p.v_st + h * p.v_sh) * M::size;
  const int e0 = static_cast<int>(c) * EPT;
  const u32x4 xlo = *reinterpret_cast<const u32x4*>(src + e0 * M::size);
  const u32x4 xhi = *reinterpret_cast<const u32x4*>(src + (half + e0) * M::size);

  if (kind == 2) {
    // V: the cache write alone, converted to the cache dtype.
    uint32_t lo[EPT], hi[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      lo[e] = Elem<CT>::from_f32(M::to_f32(M::get(xlo, e)));
      hi[e] = Elem<CT>::from_f32(M::to_f32(M::get(xhi, e)));
    }
    char* d = p.v_cache + ((slot * p.num_kv_heads + h) * p.head_dim) * Elem<CT>::size;
    store_elems<CT>(d + e0 * Elem<CT>::size, lo);
    store_elems<CT>(d + (half + e0) * Elem<CT>::size, hi);
    return;
  }

  const char* cs = p.cos + t * p.cs_st * M::size;
  const char* sn = p.sin + t * p.cs_st * M::size;
  const u32x4 clo = *reinterpret_cast<const u32x4*>(cs + e0 * M::size);
  const u32x4 chi = *reinterpret_cast<const u32x4*>(cs + (half + e0) * M::size);
  const u32x4 slo = *reinterpret_cast<const u32x4*>(sn + e0 * M::size);
  const u32x4 shi = *reinterpret_cast<const u32x4*>(sn + (half + e0) * M::size);
  float o1[EPT], o2[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const float x1 = M::to_f32(M::get(xlo, e)), x2 = M::to_f32(M::get(xhi, e));
    const float c1 = M::to_f32(M::get(clo, e)), c2 = M::to_f32(M::get(chi, e));
    const float s1 = M::to_f32(M::get(slo, e)), s2 = M::to_f32(M::get(shi, e));
    // One rounding per tensor op, no fused multiply-adds (contraction is off).
    const float a1 = round_to<DT>(x1 * c1), b1 = round_to<DT>(x2 * s1);
    const float a2 = round_to<DT>(x2 * c2), b2 = round_to<DT>(x1 * s2);
    o1[e] = round_to<DT>(a1 - b1);
    o2[e] = round_to<DT>(a2 + b2);
  }
  if (kind == 0) {
    uint32_t lo[EPT], hi[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      lo[e] = M::from_f32(o1[e]);
      hi[e] = M::from_f32(o2[e]);
    }
    char* d = p.q_out + ((t * p.num_heads + h) * p.head_dim) * M::size;
    store_elems<DT>(d + e0 * M::size, lo);
    store_elems<DT>(d + (half + e0) * M::size, hi);
    return;
  }
  // o1/o2 are exact in the model dtype; converting them to the cache dtype is
  // the `.to(cache dtype)` of the write.
  uint32_t lo[EPT], hi[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    lo[e] = Elem<CT>::from_f32(o1[e]);
    hi[e] = Elem<CT>::from_f32(o2[e]);
  }
  char* d = p.k_cache + ((slot * p.num_kv_heads + h) * p.head_dim) * Elem<CT>::size;
  store_elems<CT>(d + e0 * Elem<CT>::size, lo);
  store_elems<CT>(d + (half + e0) * Elem<CT>::size, hi);
}

using RopeKernel = void (*)(RopeCacheParams);

template <int DT>
RopeKernel rope_kernel_for_cache(int cache_dtype) {
  switch (cache_dtype) {
    case NS_DTYPE_F32: return &rope_reshape_and_cache_kernel<DT, NS_DTYPE_F32>;
    case NS_DTYPE_F16: return &rope_reshape_and_cache_kernel<DT, NS_DTYPE_F16>;
    case NS_DTYPE_BF16: return &rope_reshape_and_cache_kernel<DT, NS_DTYPE_BF16>;
    default: return nullptr;
  }
}

RopeKernel rope_kernel_for(int dtype, int cache_dtype) {
  switch (dtype) {
    case NS_DTYPE_F32: return rope_kernel_for_cache<NS_DTYPE_F32>(cache_dtype);
    case NS_DTYPE_F16: return rope_kernel_for_cache<NS_DTYPE_F16>(cache_dtype);
    case NS_DTYPE_BF16: return rope_kernel_for_cache<NS_DTYPE_BF16>(cache_dtype);
    default: return nullptr;
  }
}

bool aligned16(const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; }

}  // namespace
}  // namespace ns

extern "C" int ns_rope_reshape_and_cache(void* q_out, const void* query,
                                         int64_t q_stride_token, int64_t q_stride_head,
                                         const void* key, int64_t key_stride_token, int64_t key_stride_head,
                                         const void* value, int64_t value_stride_token, int64_t value_stride_head,
                                         const void* cos, const void* sin, int64_t cos_sin_stride_token,
                                         void* k_cache, void* v_cache,
                                         const void* slot_mapping, int slot_mapping_is_int64,
                                         int64_t num_tokens, int num_heads, int num_kv_heads, int head_dim,
                                         int block_size, int64_t num_blocks,
                                         int dtype, int cache_dtype, void* stream) {
  using namespace ns;
  const int isz = dtype_size(dtype), cisz = dtype_size(cache_dtype);
  if (isz == 0 || cisz == 0) return NS_ERR_UNSUPPORTED;
  if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      num_blocks <= 0)
    return NS_ERR_INVALID_ARG;
  if (num_tokens == 0) return NS_OK;
  if (!q_out || !query || !key || !value || !cos || !sin || !k_cache || !v_cache || !slot_mapping)
    return NS_ERR_INVALID_ARG;
  const int ept = 16 / isz;
  if (head_dim % (2 * ept) != 0 || head_dim > 1024) return NS_ERR_UNSUPPORTED;
  // Every row chunk is read and written as an aligned 16-byte vector (the
  // cache side as 8, 16 or 2x16 bytes for the cache dtype).
  const int64_t a = ept;
  const bool strides_ok = q_stride_token % a == 0 && q_stride_head % a == 0 && key_stride_token % a == 0 &&
                          key_stride_head % a == 0 && value_stride_token % a == 0 &&
                          value_stride_head % a == 0 && cos_sin_stride_token % a == 0;
  if (!strides_ok || !aligned16(q_out) || !aligned16(query) || !aligned16(key) || !aligned16(value) ||
      !aligned16(cos) || !aligned16(sin) || !aligned16(k_cache) || !aligned16(v_cache))
    return NS_ERR_INVALID_ARG;

  const int64_t cph = head_dim / 2 / ept;
  const int64_t nq = num_tokens * num_heads * cph;
  const int64_t nk = num_tokens * num_kv_heads * cph;
  if (nq + 2 * nk > INT32_MAX) return NS_ERR_INVALID_ARG;  // thread indices are 32-bit
  RopeKernel kernel = rope_kernel_for(dtype, cache_dtype);
  if (!kernel) return NS_ERR_UNSUPPORTED;

  RopeCacheParams p;
  p.q_out = static_cast<char*>(q_out);
  p.q = static_cast<const char*>(query);
  p.key = static_cast<const char*>(key);
  p.value = static_cast<const char*>(value);
  p.cos = static_cast<const char*>(cos);
  p.sin = static_cast<const char*>(sin);
  p.q_st = q_stride_token;
  p.q_sh = q_stride_head;
  p.k_st = key_stride_token;
  p.k_sh = key_stride_head;
  p.v_st = value_stride_token;
  p.v_sh = value_stride_head;
  p.cs_st = cos_sin_stride_token;
  p.k_cache = static_cast<char*>(k_cache);
  p.v_cache = static_cast<char*>(v_cache);
  p.slots = slot_mapping;
  p.slots64 = slot_mapping_is_int64 ? 1 : 0;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.head_dim = head_dim;
  p.num_slots = num_blocks * static_cast<int64_t>(block_size);
  p.cph = static_cast<uint32_t>(cph);
  p.nq = static_cast<uint32_t>(nq);
  p.nk = static_cast<uint32_t>(nk);

  const int64_t blocks = (nq + 2 * nk + 255) / 256;
  void* args[] = {&p};
  hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(kernel),
                                 dim3(static_cast<unsigned>(blocks)), dim3(256), args, 0,
                                 static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NS_OK : NS_ERR_HIP;
}
