// Paged attention for the shapes the MFMA kernels do not take (see
// generic_attention_takes): float32 caches, head sizes other than 64 and 128,
// block sizes that are not powers of two, and more than 16 query heads per
// KV head.  The reference's op accepts every float dtype and head size
// (nanoserve/attention.py:99-151; its own tests run float32 at head size 8,
// tests/test_paged_attention.py:97-134), so these calls run here instead of
// being refused.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ns {

struct GenericAttnParams {
  void* out;              // [num_tokens, num_heads, head_dim], the cache dtype
  const void* query;      // [num_tokens, num_heads, head_dim]
  const void* k_cache;    // [num_blocks, block_size, num_kv_heads, head_dim]
  const void* v_cache;
  const void* bt;         // block tables, rows of bt_stride entries
  int64_t bt_stride;
  const void* seq_lens;   // [num_seqs]
  const void* qsl;        // [num_seqs + 1] query offsets (not read for decode-only batches)
  int bt64, sl64, qsl64, decode_only;
  int num_seqs, num_heads, num_kv_heads, head_dim, block_size;
  int64_t num_tokens, num_blocks;
  int64_t max_ctx;        // keys a row may have: max_seq_len rounded to blocks, within the table
  float scale;
};

// Whether a call of this shape runs the generic kernel.
inline bool generic_attention_takes(int dtype_code_is_f32, int head_dim, int block_size, int group) {
  const bool pow2 = block_size > 0 && (block_size & (block_size - 1)) == 0;
  return dtype_code_is_f32 || (head_dim != 64 && head_dim != 128) || !pow2 || group > 16;
}

// Head sizes the generic kernel takes.
constexpr int kGenericMaxHeadDim = 256;

// Launch over every (token row, query head); dtype is an NS_DTYPE_* code.
hipError_t launch_generic_attention(const GenericAttnParams& p, int dtype, hipStream_t stream);

}  // namespace ns
