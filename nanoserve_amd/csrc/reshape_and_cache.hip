// reshape_and_cache: scatter this step's K/V rows into the paged cache.
//
// Replaces PagedKVCache.write (reference nanoserve/kv_cache.py:73-81), which
// issues two index_copy_ launches over the [NB*BS, Hkv, D] view after a
// `.to(cache dtype)` cast.  Here one launch covers K and V: each thread owns
// one 16-byte chunk of a destination row (8 f16/bf16 or 4 f32 elements), so a
// wave writes 1 KiB of contiguous cache per instruction.  The op is pure data
// movement and HBM/latency bound; conversions are done in integer arithmetic so
// the result does not depend on the wave's denormal mode.
#include "ns_convert.h"

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

}  // namespace

int dtype_size(int dtype) {
  switch (dtype) {
    case NS_DTYPE_F32: return 4;
    case NS_DTYPE_F16: return 2;
    case NS_DTYPE_BF16: return 2;
    default: return 0;
  }
}

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
