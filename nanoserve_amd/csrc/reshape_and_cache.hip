// reshape_and_cache: scatter this step's K/V rows into the paged cache.
//
// Replaces PagedKVCache.write (reference nanoserve/kv_cache.py:73-81), which
// issues two index_copy_ launches over the [NB*BS, Hkv, D] view after a
// `.to(cache dtype)` cast.  Here one launch covers K and V: each thread owns
// one 16-byte chunk of a destination row (8 f16/bf16 or 4 f32 elements), so a
// wave writes 1 KiB of contiguous cache per instruction.  The op is pure data
// movement and HBM/latency bound; conversions are done in integer arithmetic so
// the result does not depend on the wave's denormal mode.
#include "ns_common.h"

namespace ns {
namespace {

struct CacheWriteParams {
  const char* key;
  const char* value;
  int64_t key_st, key_sh, val_st, val_sh;  // element strides
  char* k_cache;
  char* v_cache;
  const void* slots;
  int slots64;
  int64_t num_tokens;
  int num_kv_heads, head_dim;
  int64_t num_slots;  // num_blocks * block_size
  int src_dtype, dst_dtype;
  int src_isz, dst_isz;
  int ept;            // destination elements per 16-byte chunk
  int vec_src;        // source chunk is a 16-byte aligned copy of the destination type
};

__device__ __forceinline__ uint32_t f16_bits_to_f32_bits(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  const uint32_t m = h & 0x3FFu;
  if (e == 0) {
    if (m == 0) return sign;
    // Subnormal: m * 2^-24 is exactly representable as a normal f32.
    return sign | __float_as_uint(static_cast<float>(m) * 5.9604644775390625e-08f);
  }
  if (e == 31) return sign | 0x7F800000u | (m << 13);
  return sign | ((e + 112u) << 23) | (m << 13);
}

// IEEE binary32 -> binary16, round to nearest even, subnormals kept, NaN -> quiet NaN.
__device__ __forceinline__ uint32_t f32_bits_to_f16_bits(uint32_t u) {
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7E00u;            // NaN
  if (a >= 0x477FF000u) return sign | 0x7C00u;           // >= 65520 rounds to inf
  if (a >= 0x38800000u) {                                // normal f16 range (>= 2^-14)
    const uint32_t mant = a - 0x38000000u;               // rebias exponent 127 -> 15
    return sign | ((mant + 0xFFFu + ((mant >> 13) & 1u)) >> 13);
  }
  if (a <= 0x33000000u) return sign;                     // <= 2^-25 rounds to zero
  // f16 subnormal: value = q * 2^-24 with q = round(full_mantissa >> shift).
  const uint32_t e = a >> 23;                            // 102..112
  const uint32_t fm = (a & 0x7FFFFFu) | 0x800000u;
  const uint32_t rs = 126u - e;                          // 14..24
  uint32_t q = fm >> rs;
  const uint32_t rem = fm & ((1u << rs) - 1u);
  const uint32_t half = 1u << (rs - 1u);
  if (rem > half || (rem == half && (q & 1u))) ++q;
  return sign | q;
}

// IEEE binary32 -> bfloat16, round to nearest even, NaN -> 0x7FC0.
__device__ __forceinline__ uint32_t f32_bits_to_bf16_bits(uint32_t u) {
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ uint32_t load_as_f32_bits(const char* p, int dtype) {
  if (dtype == NS_DTYPE_F32) return *reinterpret_cast<const uint32_t*>(p);
  const uint32_t h = *reinterpret_cast<const uint16_t*>(p);
  return dtype == NS_DTYPE_F16 ? f16_bits_to_f32_bits(h) : (h << 16);
}

__device__ __forceinline__ uint32_t f32_bits_to(uint32_t f, int dtype) {
  if (dtype == NS_DTYPE_F32) return f;
  return dtype == NS_DTYPE_F16 ? f32_bits_to_f16_bits(f) : f32_bits_to_bf16_bits(f);
}

__global__ __launch_bounds__(256) void reshape_and_cache_kernel(CacheWriteParams p) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int chunks_per_row = p.head_dim / p.ept;
  const int64_t per_tensor = p.num_tokens * p.num_kv_heads * chunks_per_row;
  if (idx >= 2 * per_tensor) return;
  const int which = idx >= per_tensor;  // 0 = key, 1 = value
  int64_t rem = idx - which * per_tensor;
  const int chunk = static_cast<int>(rem % chunks_per_row);
  rem /= chunks_per_row;
  const int h = static_cast<int>(rem % p.num_kv_heads);
  const int64_t t = rem / p.num_kv_heads;

  const int64_t slot = load_index(p.slots, t, p.slots64);
  if (slot < 0 || slot >= p.num_slots) return;  // padding / invalid slot: never written

  const char* src = which ? p.value : p.key;
  const int64_t st = which ? p.val_st : p.key_st;
  const int64_t sh = which ? p.val_sh : p.key_sh;
  char* dst_base = which ? p.v_cache : p.k_cache;

  const int e0 = chunk * p.ept;
  const char* s = src + (t * st + h * sh + e0) * p.src_isz;
  char* d = dst_base + ((slot * p.num_kv_heads + h) * p.head_dim + e0) * p.dst_isz;

  if (p.vec_src) {
    *reinterpret_cast<u32x4*>(d) = *reinterpret_cast<const u32x4*>(s);
    return;
  }
  uint32_t words[4] = {0u, 0u, 0u, 0u};
  if (p.src_dtype == p.dst_dtype) {
    // Unaligned same-type copy: move raw bits element by element.
    for (int e = 0; e < p.ept; ++e) {
      const uint32_t bits = p.dst_isz == 4 ? *reinterpret_cast<const uint32_t*>(s + e * 4)
                                           : *reinterpret_cast<const uint16_t*>(s + e * 2);
      if (p.dst_isz == 4) words[e] = bits;
      else words[e >> 1] |= bits << ((e & 1) * 16);
    }
  } else {
    for (int e = 0; e < p.ept; ++e) {
      const uint32_t f = load_as_f32_bits(s + e * p.src_isz, p.src_dtype);
      const uint32_t bits = f32_bits_to(f, p.dst_dtype);
      if (p.dst_isz == 4) words[e] = bits;
      else words[e >> 1] |= bits << ((e & 1) * 16);
    }
  }
  *reinterpret_cast<u32x4*>(d) = u32x4{words[0], words[1], words[2], words[3]};
}

int dtype_size(int dtype) {
  switch (dtype) {
    case NS_DTYPE_F32: return 4;
    case NS_DTYPE_F16: return 2;
    case NS_DTYPE_BF16: return 2;
    default: return 0;
  }
}

}  // namespace
}  // namespace ns

extern "C" int ns_reshape_and_cache(const void* key, const void* value,
                                    int64_t key_stride_token, int64_t key_stride_head,
                                    int64_t value_stride_token, int64_t value_stride_head,
                                    void* k_cache, void* v_cache,
                                    const void* slot_mapping, int slot_mapping_is_int64,
                                    int64_t num_tokens, int num_kv_heads, int head_dim,
                                    int block_size, int64_t num_blocks,
                                    int src_dtype, int cache_dtype, void* stream) {
  using namespace ns;
  const int src_isz = dtype_size(src_dtype);
  const int dst_isz = dtype_size(cache_dtype);
  if (src_isz == 0 || dst_isz == 0) return NS_ERR_UNSUPPORTED;
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks <= 0)
    return NS_ERR_INVALID_ARG;
  if (num_tokens == 0) return NS_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return NS_ERR_INVALID_ARG;
  const int ept = 16 / dst_isz;
  if (head_dim % ept != 0) return NS_ERR_UNSUPPORTED;
  if (reinterpret_cast<uintptr_t>(k_cache) % 16 || reinterpret_cast<uintptr_t>(v_cache) % 16)
    return NS_ERR_INVALID_ARG;

  CacheWriteParams p;
  p.key = static_cast<const char*>(key);
  p.value = static_cast<const char*>(value);
  p.key_st = key_stride_token;
  p.key_sh = key_stride_head;
  p.val_st = value_stride_token;
  p.val_sh = value_stride_head;
  p.k_cache = static_cast<char*>(k_cache);
  p.v_cache = static_cast<char*>(v_cache);
  p.slots = slot_mapping;
  p.slots64 = slot_mapping_is_int64 ? 1 : 0;
  p.num_tokens = num_tokens;
  p.num_kv_heads = num_kv_heads;
  p.head_dim = head_dim;
  p.num_slots = num_blocks * static_cast<int64_t>(block_size);
  p.src_dtype = src_dtype;
  p.dst_dtype = cache_dtype;
  p.src_isz = src_isz;
  p.dst_isz = dst_isz;
  p.ept = ept;
  // A 16-byte vector copy is legal when the types match and every source chunk
  // starts on a 16-byte boundary.
  const int64_t a = 16 / src_isz;
  p.vec_src = src_dtype == cache_dtype &&
              reinterpret_cast<uintptr_t>(key) % 16 == 0 &&
              reinterpret_cast<uintptr_t>(value) % 16 == 0 &&
              key_stride_token % a == 0 && key_stride_head % a == 0 &&
              value_stride_token % a == 0 && value_stride_head % a == 0;

  const int64_t threads = 2 * num_tokens * num_kv_heads * (head_dim / ept);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7FFFFFFF) return NS_ERR_INVALID_ARG;
  void* args[] = {&p};
  hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&reshape_and_cache_kernel),
                                 dim3(static_cast<unsigned>(blocks)), dim3(256), args, 0,
                                 static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NS_OK : NS_ERR_HIP;
}
