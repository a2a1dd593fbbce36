/*
 * nanoserve_paged.h -- C ABI of the MI355X (gfx950) paged-attention library.
 *
 * The library replaces the GPU side of nanoserve's attention op and KV-cache
 * write.  Every entry point takes plain device pointers, element strides and
 * sizes, and a HIP stream (passed as void*, e.g. the value of
 * torch.cuda.current_stream().cuda_stream).  Nothing here allocates device
 * memory, synchronises the device or keeps state between calls, except the
 * split-K counters inside the caller-owned workspace (see
 * ns_paged_attention_workspace_size).
 *
 * Layouts (unchanged from the reference):
 *   query / out          [num_tokens, num_heads, head_dim], contiguous
 *   k_cache / v_cache    [num_blocks, block_size, num_kv_heads, head_dim], contiguous
 *   block_tables         [num_seqs, >= ceil(max_seq_len / block_size)], row stride given
 *   seq_lens             [num_seqs]      context length including this step
 *   query_start_loc      [num_seqs + 1]  prefix sums of the per-sequence query lengths
 *   slot_mapping         [num_tokens]    slot = block_table[pos / bs] * bs + pos % bs
 *
 * Integer index tensors may be int32 or int64 (the engine ships int64, the
 * reference tests int32); each pointer carries its own width flag so no cast
 * kernel is ever needed.
 *
 * Every function returns NS_OK (0) or a negative NS_ERR_* code and never
 * aborts the process.  Argument checks run on the host before any HIP call.
 * The library creates no streams, events or device allocations of its own:
 * a mixed batch that should overlap its decode and prefill launches gets a
 * second stream and two events from the caller (ns_paged_attention).
 */
#ifndef NANOSERVE_PAGED_H
#define NANOSERVE_PAGED_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define NS_OK 0
#define NS_ERR_INVALID_ARG (-1)  /* null pointer, bad size, bad stride      */
#define NS_ERR_UNSUPPORTED (-2)  /* shape/dtype combination not compiled   */
#define NS_ERR_WORKSPACE (-3)    /* workspace missing or too small         */
#define NS_ERR_HIP (-4)          /* the HIP launch itself reported an error */

/* Element types. */
#define NS_DTYPE_F32 0
#define NS_DTYPE_F16 1
#define NS_DTYPE_BF16 2

/* Epilogues of ns_int4_linear. */
#define NS_EPILOGUE_NONE 0
#define NS_EPILOGUE_RESIDUAL 1
#define NS_EPILOGUE_SILU_MUL 2

/* Human-readable text for a status code (static storage, never NULL). */
const char* ns_error_string(int code);

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int ns_version(void);

/*
 * ns_reshape_and_cache -- scatter this step's K and V rows into the paged cache.
 *
 * Replaces PagedKVCache.write (reference nanoserve/kv_cache.py:73-81):
 *     k_cache.view(NB*BS, Hkv, D).index_copy_(0, slot_mapping, key.to(cache dtype))
 *     v_cache.view(NB*BS, Hkv, D).index_copy_(0, slot_mapping, value.to(cache dtype))
 * in one launch for both caches.  Same-dtype rows are copied bit for bit;
 * f32 -> f16/bf16 and f16 <-> bf16 conversions round to nearest even like
 * torch's Tensor.to (NaN becomes a canonical quiet NaN).  Slots outside
 * [0, num_blocks*block_size) -- e.g. -1 for padding tokens -- are skipped and
 * never dereferenced.
 *
 * key/value strides are in elements; the head_dim stride must be 1.
 */
int ns_reshape_and_cache(const void* key, const void* value,
                         int64_t key_stride_token, int64_t key_stride_head,
                         int64_t value_stride_token, int64_t value_stride_head,
                         void* k_cache, void* v_cache,
                         const void* slot_mapping, int slot_mapping_is_int64,
                         int64_t num_tokens, int num_kv_heads, int head_dim,
                         int block_size, int64_t num_blocks,
                         int src_dtype, int cache_dtype, void* stream);

/*
 * ns_rope_reshape_and_cache -- rotary embedding of Q and K fused with the
 * paged-cache write of K and V (the two steps before attention at the
 * reference call site, nanoserve/qwen2.py:53-57).
 *
 * Replaces RotaryEmbedding.apply (reference nanoserve/layers.py:84-88):
 *     q' = q * cos + rotate_half(q) * sin,  k' likewise,
 *     rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2]),
 * followed by PagedKVCache.write (reference nanoserve/kv_cache.py:73-81) of
 * k' and v through slot_mapping, in one launch.  q' is written to q_out
 * ([num_tokens, num_heads, head_dim] contiguous; q_out may equal query when
 * query is contiguous); k' is only written to the cache, as in the
 * reference, where the rotated k has no other use.
 *
 * cos and sin are the per-forward lookups of the reference
 * (RotaryEmbedding.cos_sin, layers.py:75-79): [num_tokens, head_dim] rows in
 * the model dtype `dtype` with token stride cos_sin_stride_token.  The result
 * is bit-exact with the reference's tensor arithmetic (each product and the
 * sum rounded to `dtype`, then `.to(cache_dtype)`).  Slots outside
 * [0, num_blocks*block_size) are skipped.  All pointers must be 16-byte
 * aligned and all strides (in elements) multiples of 16 bytes' worth of
 * elements; head_dim must be a multiple of 2 * (16 / dtype size).
 */
int ns_rope_reshape_and_cache(void* q_out, const void* query,
                              int64_t q_stride_token, int64_t q_stride_head,
                              const void* key, int64_t key_stride_token, int64_t key_stride_head,
                              const void* value, int64_t value_stride_token, int64_t value_stride_head,
                              const void* cos, const void* sin, int64_t cos_sin_stride_token,
                              void* k_cache, void* v_cache,
                              const void* slot_mapping, int slot_mapping_is_int64,
                              int64_t num_tokens, int num_heads, int num_kv_heads, int head_dim,
                              int block_size, int64_t num_blocks,
                              int dtype, int cache_dtype, void* stream);

/*
 * ns_int4_linear -- out = x · W^T + bias with W held as group-wise asymmetric
 * INT4, dequantised in registers inside the GEMM.
 *
 * Replaces QuantLinear.forward in "int4" mode (reference
 * nanoserve/quant.py:157-158: F.linear(x, dequantize_int4(...), bias),
 * dequantize_int4 at quant.py:83-95), with the weight format of
 * quantize_int4_groupwise (quant.py:53-80):
 *   qweight [N, K/2] uint8, code of (n, k) in the low nibble of byte k/2 for
 *           even k and in the high nibble for odd k;
 *   scales  [N, K/group_size] float32;  zeros [N, K/group_size] uint8;
 *   w(n, k) = (code - zero) * scale in float32, rounded to `dtype`.
 * x is [M, K] with row stride x_stride_row (elements, a multiple of 8, rows
 * 16-byte aligned); bias is [N] in `dtype` or NULL.  Accumulation is fp32
 * (MFMA); y = round(acc + bias) is what F.linear returns.  The epilogue then
 * continues the reference's next elementwise op in the same launch, rounding
 * where the reference's separate tensor ops round:
 *   NS_EPILOGUE_NONE      out [M, N] = y;
 *   NS_EPILOGUE_RESIDUAL  out [M, N] = round(y + residual), residual [M, N]
 *                         contiguous (may be out itself): the residual add
 *                         after o_proj / down_proj (reference qwen2.py:78-84);
 *   NS_EPILOGUE_SILU_MUL  W's rows are interleaved (gate_j, up_j) pairs and
 *                         out [M, N/2] = round(round(silu(gate)) * up): the
 *                         SwiGLU of reference layers.py:108-109.
 * With norm_weight (a [K] `dtype` vector, 16-byte aligned) the rows of x are
 * RMS-normalised in the same launch, the reference's RMSNorm (layers.py:25-47)
 * before q/k/v and gate/up: out = rsqrt(mean(x^2) + eps) * (round(x *
 * norm_weight) · W^T) per row, then the bias and the epilogue.  The
 * operands round at the precision of torch's F.rms_norm (round(x * rsqrt(..)
 * * norm_weight) before the product); this needs K a multiple of 128 and at
 * most 1024.
 * dtype is NS_DTYPE_F16 or NS_DTYPE_BF16.  N must be a multiple of 16, K and
 * group_size multiples of 32 with K a multiple of group_size; qweight 16-byte
 * aligned, out 8-byte aligned.  Up to 128 rows one kernel dequantises each
 * weight tile per 16 or 64 tokens; above, a tiled GEMM (K a multiple of 64,
 * no norm_weight, bias 8-byte and zeros 4-byte aligned; otherwise the first
 * kernel) dequantises it once per 128 or 256 tokens.
 */
int ns_int4_linear(void* out, const void* x, int64_t x_stride_row,
                   const void* qweight, const void* scales, const void* zeros, const void* bias,
                   const void* residual, int epilogue, const void* norm_weight, float norm_eps,
                   int64_t M, int N, int K, int group_size, int dtype, void* stream);

/*
 * ns_int4_linear_splitk -- ns_int4_linear with the K loop of long-K layers
 * split over several workgroups per output tile (down_proj of
 * Qwen2.5-0.5B: N = 896 is 56 tiles of 16 features, or 14 of 64, too few for
 * the device, each walking K = 4864).  Same operands, epilogues and RMSNorm
 * as ns_int4_linear; the fp32 partial sums of each split go to `workspace`
 * and the last split of a tile adds them in split order (deterministic) and
 * runs the epilogue.  The split count (up to 4) keeps tiles x splits within
 * 256 workgroups up to 128 tokens (register-dequant kernel); above (tiled
 * GEMM), the tiles of the last dispatch round split (all tiles when one round
 * holds them) when they fill at most half of the device's slots, within
 * those slots and with at least 8 K steps of 64 a split, so it depends on N,
 * K and the number of token tiles, and the partials never exceed one round
 * of fp32 tiles (32 MiB).
 * Same replacement as ns_int4_linear (reference
 * nanoserve/quant.py:157-158).  workspace: 256-byte aligned,
 * ns_int4_linear_splitk_workspace_size(M, N, K) bytes, zeroed once before
 * first use; every call leaves its arrival counters at zero.  Calls that
 * overlap in time must not share a workspace.  Shapes that do not split
 * (size 0) ignore it.
 */
size_t ns_int4_linear_splitk_workspace_size(int64_t M, int N, int K);
int ns_int4_linear_splitk(void* out, const void* x, int64_t x_stride_row,
                          const void* qweight, const void* scales, const void* zeros, const void* bias,
                          const void* residual, int epilogue, const void* norm_weight, float norm_eps,
                          int64_t M, int N, int K, int group_size, int dtype,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * ns_int4_linear_rope_cache -- the q|k|v projection of one attention layer
 * with the rotary embedding and the paged-cache write in its epilogue: one
 * launch for what the reference runs as QuantLinear.forward of q, k and v
 * (nanoserve/quant.py:157-158), RotaryEmbedding.apply (layers.py:84-88) and
 * PagedKVCache.write (kv_cache.py:73-81), the steps between the layer's input
 * and attention at reference qwen2.py:46-57.
 *
 * W holds the (num_heads + 2 * num_kv_heads) * head_dim rows of q, k and v
 * in that order, in the format of ns_int4_linear, with the rows of every
 * head in rotary-pair order: 16-row tile i of a head holds dims
 * [8i, 8i+8) then [head_dim/2 + 8i, +8).  With y = round(x · W^T + bias)
 * (and the RMSNorm of ns_int4_linear when norm_weight is given),
 * q and k are rotated exactly as ns_rope_reshape_and_cache rotates them;
 * q' goes to q_out ([M, num_heads, head_dim] contiguous, original dim
 * order), k' and v to slot_mapping's slots of k_cache / v_cache
 * ([num_blocks, block_size, num_kv_heads, head_dim], model dtype; slots
 * outside the cache are skipped).  Every value is bit-identical to
 * ns_int4_linear followed by ns_rope_reshape_and_cache on the rows in
 * original order.  cos/sin: [M, head_dim] rows, token stride
 * cos_sin_stride_token (a multiple of 4).  K a multiple of 128 and at most
 * 1024, head_dim a multiple of 16; q_out, the caches, cos and sin 8-byte
 * aligned.
 */
int ns_int4_linear_rope_cache(void* q_out, const void* x, int64_t x_stride_row,
                              const void* qweight, const void* scales, const void* zeros,
                              const void* bias, const void* norm_weight, float norm_eps,
                              const void* cos, const void* sin, int64_t cos_sin_stride_token,
                              void* k_cache, void* v_cache,
                              const void* slot_mapping, int slot_mapping_is_int64,
                              int64_t M, int K, int group_size,
                              int num_heads, int num_kv_heads, int head_dim,
                              int block_size, int64_t num_blocks, int dtype, void* stream);

/*
 * ns_int4_dequantize -- out [N, K] (`dtype`, contiguous, 16-byte aligned) =
 * the model-dtype weights of an INT4 layer: dequantize_int4 (reference
 * nanoserve/quant.py:83-95), bit for bit, in one pass.  For large token
 * counts a library GEMM on this weight is faster than ns_int4_linear, which
 * dequantises each weight tile once per 64-token tile.  K and group_size
 * multiples of 8, K a multiple of group_size.
 */
int ns_int4_dequantize(void* out, const void* qweight, const void* scales, const void* zeros,
                       int N, int K, int group_size, int dtype, void* stream);

/*
 * ns_argmax_rows -- out[m] = index of the largest element of row m of x
 * ([M, N] with row stride x_stride_row elements), the first such index on
 * ties and the first NaN if the row holds one: torch.argmax(dim=-1), which
 * the reference's greedy sampler calls (nanoserve/sampler.py:24-27).  out is
 * int64 [M]; x 16-byte aligned with 16-byte-multiple rows; M <= 65535 and
 * N < 2^32.  dtype is NS_DTYPE_F32, NS_DTYPE_F16 or NS_DTYPE_BF16.  Each row
 * is scanned in slices by separate workgroups whose results meet in
 * `workspace` (ns_argmax_rows_workspace_size bytes, 8-byte aligned, no
 * initialisation needed); calls that overlap in time need separate
 * workspaces.  Returns NS_ERR_WORKSPACE when it is missing or too small.
 */
size_t ns_argmax_rows_workspace_size(int64_t M, int64_t N);
int ns_argmax_rows(int64_t* out, const void* x, int64_t x_stride_row, int64_t M, int64_t N,
                   int dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * ns_paged_attention_workspace_size -- bytes of device workspace that
 * ns_paged_attention needs for these sizes: arrival counters, a region for
 * the call's own decode plan, the decode split-K slots and, without
 * is_decode_only, the prefill split state (512 slots of 40 KiB at head_dim
 * 64, 72 KiB at 128).  No counterpart in the reference, which allocates per
 * call.
 *
 * Layout: an 8 MiB head (arrival counters, a zero page, the plan region),
 * then the prefill split state (36 MiB, present in every workspace so the
 * offsets after it never move), then the decode split-K slots.
 *
 * The workspace must be zero-filled once when it is first allocated.  Every
 * call leaves the counters and the prefill split state as it found them
 * (back at zero: the workgroup that consumes a prefill slot clears it), so
 * the same buffer serves later calls of any shape on the same stream
 * without clearing; the decode slots keep the last call's partials, which no
 * later call reads before writing.  Calls that overlap in time (different
 * streams) must use different workspaces.
 */
size_t ns_paged_attention_workspace_size(int num_seqs, int num_heads, int num_kv_heads,
                                         int head_dim, int block_size,
                                         int max_seq_len, int max_query_len,
                                         int64_t num_tokens, int is_decode_only);

/*
 * ns_paged_decode_plan_size, ns_paged_decode_plan -- the decode work plan of
 * one step's metadata, built on the device.  No counterpart in the
 * reference; it is the device-side form of the launch schedule that the
 * reference's Triton wrapper derives from the device seq_lens on every call
 * (nanoserve/triton_attention.py:144-160).
 *
 * The plan cuts the decode rows (every sequence of a decode-only batch; the
 * one-query-row sequences of a mixed batch, found from query_start_loc)
 * into items of context tokens of one (sequence, kv head) pair, sized so
 * the items about fill the device once for light batches and in several
 * rounds, longest sequences first, for heavy ones; at head_dim 64 a
 * one-round plan keeps items of 512 tokens while that still gives half of
 * the CUs an item or every context fits one item.  Each item also carries
 * the block ids of its waves' first K/V loads (block size >= 16), so those
 * loads need no table round trip.  It reads only device memory (seq_lens,
 * query_start_loc, block_tables), so a captured HIP graph rebuilds it from
 * the step's lengths and tables on every replay.
 *
 * ns_paged_attention builds the plan itself (one extra launch into its
 * workspace) when it is given none.  The engine's metadata is shared by all
 * layers of a step, so the shim builds it once per step with
 * ns_paged_decode_plan and passes it to every layer's call.  A plan is valid
 * for calls with the same metadata and sizes (num_seqs, num_kv_heads,
 * head_dim, block_size, max_seq_len, block_table_width, decode-only or not,
 * and the same device lengths, query offsets and block tables); plan must be
 * 16-byte aligned with at least ns_paged_decode_plan_size bytes.
 */
size_t ns_paged_decode_plan_size(int num_seqs, int num_kv_heads, int head_dim, int block_size,
                                 int max_seq_len);
int ns_paged_decode_plan(void* plan, size_t plan_bytes,
                         const void* block_tables, int64_t block_table_stride,
                         int64_t block_table_width, int block_tables_is_int64,
                         const void* seq_lens, int seq_lens_is_int64,
                         const void* query_start_loc, int query_start_loc_is_int64,
                         int num_seqs, int is_decode_only, int num_kv_heads, int head_dim,
                         int block_size, int max_seq_len, void* stream);

/*
 * ns_paged_attention -- unified paged attention (prefill, decode, chunked
 * prefill and mixed batches in one entry point).
 *
 * Replaces the attn_fn contract shared by paged_attention_torch
 * (reference nanoserve/attention.py:99-151, decode fast path 154-190) and
 * paged_attention_triton (reference nanoserve/triton_attention.py:117-161):
 * query token j of sequence i sits at absolute position
 * seq_lens[i] - query_len_i + j and attends to keys [0, that position] of
 * that sequence, with kv head h / (num_heads / num_kv_heads), scores scaled
 * by `scale`, softmax accumulated in fp32, output written in `dtype`.
 *
 * When is_decode_only is set every sequence has exactly one query token and
 * token i belongs to sequence i (query_start_loc is not read), as in the
 * reference decode fast path.  Otherwise query_start_loc delimits each
 * sequence's query rows; sequences with an empty query range are skipped.
 *
 * Decode rows run as one workgroup per plan item (see
 * ns_paged_decode_plan): decode_plan, when not NULL, is a plan built for
 * this call's metadata (decode_plan_bytes its size); NULL makes the call
 * build one in its workspace first.  A pair cut into several items is merged
 * inside the launch by the pair's last workgroup to start, in item order,
 * so results do not depend on timing.
 *
 * seq_lens_host and query_start_loc_host (optional, may be NULL; read only
 * together and without is_decode_only) are HOST copies of seq_lens and
 * query_start_loc -- the reference's AttentionMetadata.seq_lens_cpu and
 * query_start_loc_cpu (attention.py:52-54), which its non-decode path
 * already treats as authoritative (attention.py:124).  With them the prefill
 * rows are scheduled exactly: heaviest column blocks first, long key ranges
 * split across workgroups and merged in-launch (the workspace holds the split
 * state), and the decode launch is skipped when no sequence has a single
 * query row.  They must equal the device copies; a sequence whose device
 * query length differs has its reached outputs written as NaN (nothing is
 * read or written out of bounds).
 *
 * dtype is NS_DTYPE_F32, NS_DTYPE_F16 or NS_DTYPE_BF16 for query, caches
 * and out.  The MFMA kernels take float16/bfloat16 with head_dim 64 or 128, a
 * power-of-two block_size and num_heads / num_kv_heads <= 16 (all pointers
 * 16-byte aligned); every other shape with head_dim <= 256 runs a generic
 * float32-arithmetic kernel (pointers aligned to the element size) that
 * reads no plan, workspace or aux stream.  Loops are bounded by each sequence's
 * length (never by the block-table width), so zero-padded table rows are
 * safe.  A block id outside [0, num_blocks) is never dereferenced; the
 * affected (sequence, head) outputs are written as NaN.
 *
 * aux_stream, fork_event, join_event (optional: all three or none, owned by
 * the caller; aux_stream must differ from stream).  With them, a batch that
 * has both decode rows and prefill rows forks the decode launch onto
 * aux_stream (fork_event recorded on stream, waited on by aux_stream) and
 * joins it back (join_event recorded on aux_stream, waited on by stream), so
 * the two launches overlap; graph capture records both dependencies.  Without
 * them both launches run in order on stream.  Decode-only and prefill-only
 * batches never touch them.  Calls that overlap in time need their own set.
 */
int ns_paged_attention(void* out, const void* query,
                       const void* k_cache, const void* v_cache,
                       const void* block_tables, int64_t block_table_stride,
                       int64_t block_table_width, int block_tables_is_int64,
                       const void* seq_lens, int seq_lens_is_int64,
                       const void* query_start_loc, int query_start_loc_is_int64,
                       const void* seq_lens_host, int seq_lens_host_is_int64,
                       const void* query_start_loc_host, int query_start_loc_host_is_int64,
                       int num_seqs, int64_t num_tokens, int max_query_len, int max_seq_len,
                       int is_decode_only,
                       int num_heads, int num_kv_heads, int head_dim,
                       int block_size, int64_t num_blocks,
                       float scale, int dtype,
                       const void* decode_plan, size_t decode_plan_bytes,
                       void* workspace, size_t workspace_bytes, void* stream,
                       void* aux_stream, void* fork_event, void* join_event);

/*
 * ns_paged_attention_noalloc -- ns_paged_attention without a workspace
 * argument and without any allocation.  No counterpart in the reference: it
 * is for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, results
 * and errors as ns_paged_attention, whose kernels it runs, but the split-K
 * workspace is a 128 MiB array inside the library, one per device, held from
 * module load until the process ends.  A call whose
 * ns_paged_attention_workspace_size exceeds 128 MiB returns NS_ERR_WORKSPACE.
 * The first call on a device looks the array up (and, outside graph
 * capture, clears it with one fill launch on `stream`); every call leaves it
 * ready for the next.  All calls on one device share the array, so calls
 * that overlap in time on one device (different streams) race and must not
 * be issued.
 */
int ns_paged_attention_noalloc(void* out, const void* query,
                               const void* k_cache, const void* v_cache,
                               const void* block_tables, int64_t block_table_stride,
                               int64_t block_table_width, int block_tables_is_int64,
                               const void* seq_lens, int seq_lens_is_int64,
                               const void* query_start_loc, int query_start_loc_is_int64,
                               const void* seq_lens_host, int seq_lens_host_is_int64,
                               const void* query_start_loc_host, int query_start_loc_host_is_int64,
                               int num_seqs, int64_t num_tokens, int max_query_len, int max_seq_len,
                               int is_decode_only,
                               int num_heads, int num_kv_heads, int head_dim,
                               int block_size, int64_t num_blocks,
                               float scale, int dtype,
                               const void* decode_plan, size_t decode_plan_bytes, void* stream,
                               void* aux_stream, void* fork_event, void* join_event);

#ifdef __cplusplus
}
#endif

#endif /* NANOSERVE_PAGED_H */
