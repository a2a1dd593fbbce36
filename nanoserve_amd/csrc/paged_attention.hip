// Paged attention for gfx950 (MI355X): decode with in-launch split-K merge,
// and a variable-length (prefill / chunked prefill / mixed) kernel.
//
// Semantics follow the reference's unified op (nanoserve/attention.py:99-190):
// query row j of a sequence with context length L and query length ql sits at
// absolute position L - ql + j and attends to keys [0, L - ql + j]; kv head of
// query head h is h / (Hq / Hkv); scores are scaled by `scale`; the softmax is
// accumulated in fp32; the output is written in the query dtype.
//
// Both kernels compute S^T = K * Q^T with v_mfma_f32_16x16x32_{f16,bf16}:
// the 16 MFMA rows are KV tokens and the 16 MFMA columns are query heads of
// one GQA group (decode) or flattened (query row, head) pairs (prefill).  With
// K as the A operand, a lane's 8 k-slots are 8 consecutive head dims of one
// token, i.e. one 16-byte load straight out of the [NB, BS, Hkv, D] cache.
// The result puts tokens 4*g + r (g = lane / 16) of column lane % 16 in lane
// registers, which is exactly the B operand P^T of the O^T = V^T * P^T MFMA
// once the k-slots of two 16-token tiles are interleaved, so P never moves
// between lanes.  V^T is staged through LDS.
#include <math.h>

#include <algorithm>
#include <mutex>
#include <utility>
#include <vector>

#include "decode_plan.h"
#include "generic_attention.h"
#include "ns_common.h"

namespace ns {
namespace {

// Plan entries carried in the kernel arguments (keeps them under 4 KiB).
constexpr int kPlanMax = 768;

struct AttnParams {
  char* out;
  const char* query;
  const char* k_cache;
  const char* v_cache;
  const void* bt;
  int64_t bt_stride;
  const void* seq_lens;
  const void* qsl;
  int bt64, sl64, qsl64;
  int decode_only;
  int num_seqs;
  int64_t num_tokens;     // rows of query/out; query rows outside are never touched
  int num_heads, num_kv_heads, group;
  int bs_shift;
  int64_t num_blocks;
  int64_t max_ctx;        // tokens addressable through a table row
  float scale_log2;       // scale * log2(e): softmax runs in base 2
  int skip_decode_rows;   // varlen: one-row sequences belong to the decode kernel
  // Decode: the plan (decode_plan.h) and the split-K state.  Partial slot i
  // (of plan item i) is slot_words 32-bit words of `part` (part_bytes in all).
  const DecodePlanHeader* plan_hdr;
  const DecodeItem* items;
  int64_t item_cap;
  int inline_blocks;      // items carry their waves' first-steps block ids (block size >= 16)
  const void* zeros;      // kZeroPageBytes of the workspace head that are never written
  uint32_t* part;
  int part_bytes;
  int slot_words;
  unsigned* counters;     // [S, Hkv] arrivals per (sequence, kv head); left at zero
  // Prefill split-K: partial slots of one workgroup's columns each, and one
  // arrival counter per split (sequence, kv head, column block); left at zero.
  float* pf_part;
  int pf_part_bytes;
  unsigned* pf_counters;
  int plan_n;             // prefill: sequences listed (0: no plan)
};

// The prefill kernel's arguments add its host-built schedule: two entries per
// listed sequence y, s | (nsplit - 1) << 16 | split_macro << 22 and
// slot_base | pair_base << 16, then its query length.  The decode kernel takes
// the 200-byte base alone, so its launches do not carry the 3 KB schedule.
struct PrefillParams : AttnParams {
  uint32_t plan[kPlanMax];
};

typedef short short4_t __attribute__((ext_vector_type(4)));

// Address-space views for global_load_lds (global source, LDS destination).
typedef __attribute__((address_space(1))) void* gbl_void_ptr;
typedef __attribute__((address_space(3))) void* lds_void_ptr;

// LDS swizzles of K and V tiles ([keys][D] rows of 16-byte units): unit c of
// key k is stored at unit c ^ k_swz(k) (K) or c ^ v_swz(k) (V) of its row, so
// the 16-byte K operand reads and the 8-byte transposing V reads of a wave
// spread over all banks.  A DMA lane picks the global unit that belongs at
// its LDS slot, so the swizzle costs nothing on the write side.
__device__ __forceinline__ int k_swz(int key) { return key & 7; }
__device__ __forceinline__ int v_swz(int key) { return (key & 3) << 1; }

// --------------------------------------------------------------------------
// Decode: one workgroup of W waves per plan item (a token range of one
// (sequence, kv head) pair); the grid loops over the plan's items.
// --------------------------------------------------------------------------
// A wave walks its tokens in chunks of 32 (two 16-token MFMA tiles).  Chunks
// go from HBM into a ring of R slots in the wave's own LDS with
// global_load_lds, so loads in flight hold no registers and every wait for
// them is an explicit vmcnt the wave chooses; the query tile and the block
// ids past the item's carried ones arrive the same way, ahead of the first
// chunk.
template <int D, int W, int R_>
struct DecodeCfg {
  static constexpr int kThreads = W * 64;
  static constexpr int CHUNK = 32;               // tokens per chunk
  static constexpr int NC = D / 32;              // k-chunks of the QK^T contraction
  static constexpr int NN = D / 16;              // 16-dim tiles of the output
  static constexpr int CPR = D / 8;              // 16-byte units per token row
  static constexpr int TILE_B = CHUNK * D * 2;   // bytes of a chunk's K (or V)
  static constexpr int DMA = TILE_B / 1024;      // global_load_lds per K (or V) of a chunk
  static constexpr int PER_CHUNK = 2 * DMA;      // vector-memory operations per chunk
  static constexpr int R = R_;                   // ring slots per wave
  static constexpr int SLOT_B = 2 * TILE_B;
  static constexpr int QD = 16 * D * 2 / 1024;   // global_load_lds of the 16-row query tile
  static constexpr int Q_B = QD * 1024;
  static constexpr int CARRIED = kItemBlocks / W;  // tiles per wave whose block ids come with the item
  static constexpr int IDS_B = 512;              // later block-table entries: 64 low words, 64 high words
  static constexpr int WAVE_B = R * SLOT_B + Q_B + IDS_B;
  static constexpr int RED_LD = D + 4;           // padded row of a wave's block in the cross-wave reduce
  static constexpr int LDS = W * WAVE_B;
  static_assert((R - 1) * PER_CHUNK + 2 <= 63, "waits (with two later table loads) fit vmcnt");
  static_assert(2 * R <= CARRIED && CARRIED % 2 == 0 && CARRIED <= 8, "the first R chunks' tiles are carried by the item");
};

// Wait until at most k chunks (k * PC vector-memory operations) of this wave,
// plus X operations issued after them, are in flight; k is wave-uniform and
// below R.
template <int PC, int R, int X = 0>
__device__ __forceinline__ void wait_chunks(int k) {
  if constexpr (R > 3) {
    if (k >= 3) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * PC + X) : "memory");
      return;
    }
  }
  if constexpr (R > 2) {
    if (k >= 2) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * PC + X) : "memory");
      return;
    }
  }
  if constexpr (R > 1) {
    if (k >= 1) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PC + X) : "memory");
      return;
    }
  }
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(X) : "memory");
}

// Split-K state crosses workgroups (and XCDs, whose L2s are not coherent
// with each other) through device-scope accesses: stores with the SC1 cache
// policy write through to the device coherence point, and agent-scope atomic
// loads read from it.  No L2 writeback or invalidate is issued.
constexpr int kSc1 = 16;                      // cache-policy bit SC1 of gfx94x/gfx950 buffer ops
constexpr int kBufferWord3 = 0x00020000;      // raw 32-bit buffer descriptor, word 3

// 32-bit device-scope buffer load.  Wider partial loads are written as runs
// of these, which the backend merges into dwordx2/x4: with ROCm 7.2's clang,
// taking elements of a raw_buffer_load_b64/b128 result was miscompiled into a
// single dword load at the base offset (both halves of a b64 read the same
// dword), while b32 loads merge and narrow correctly.
__device__ __forceinline__ float ld_sc1(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kSc1));
}

__device__ __forceinline__ void merge_into(float& m, float& l, floatx4& o, float m2, float l2, floatx4 o2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;  // both empty
  const float a = fast_exp2(m - mn), b = fast_exp2(m2 - mn);
  l = l * a + l2 * b;
  o = o * a + o2 * b;
  m = mn;
}

template <class IDX>
__device__ __forceinline__ int64_t ld_idx(const void* p, int64_t i) {
  return static_cast<int64_t>(reinterpret_cast<const IDX*>(p)[i]);
}

// Split-K partials.  Plan item i of a pair that has several items owns slot i
// of `part`: slot_words 32-bit words holding, for each query head col of the
// group, its unnormalised output at word col * D + d and its running (max in
// log2 units, sum) at words G * D + 2 * col + {0, 1}.
//
// Merge protocol: the pair's last workgroup to FINISH merges.  Every item
// stores its partial at device scope (sc1), waits until the stores are
// acknowledged, and only then adds one to the pair's arrival count; the item
// whose add returns nsplit - 1 has every partial visible, reads them back
// (sc1) and folds them in split order, so the result does not depend on
// which workgroup merges, then sets the count back to zero for the next
// call.  Nobody waits for another workgroup, so the merge never stalls on a
// straggler: it happens when the last one arrives.
//
// The merger's reads: each float4 column (head, 4 dims) of the output is
// owned by tpi consecutive lanes that walk disjoint split subsets with up to
// 8 loads in flight each, then combine by butterfly; the order of operations
// is fixed by tpi and nsplit alone.
template <class DT, int D, int THREADS>
__device__ void merge_partials(const AttnParams& p, __amdgpu_buffer_rsrc_t pr, uint32_t first, int nsplit,
                               typename DT::T* out_row) {
  using T = typename DT::T;
  const int G = p.group;
  const int items = G * (D / 4);
  const int slot_words = p.slot_words;
  int tpi = THREADS / items;
  tpi = tpi >= 8 ? 8 : tpi >= 4 ? 4 : tpi >= 2 ? 2 : 1;
  const int tid = threadIdx.x, sub = tid % tpi;
  for (int it = tid / tpi; it < items; it += THREADS / tpi) {
    // The lanes of a tpi group share `it`, so they run the same trip count
    // and are all active at the butterfly below.
    const int col = it / (D / 4), d4 = it % (D / 4);
    const int o_word = col * D + 4 * d4, ml_word = G * D + 2 * col;
    float m = -INFINITY, l = 0.f;
    floatx4 o = {0.f, 0.f, 0.f, 0.f};
    int poison = 0;
    for (int sp0 = sub; sp0 < nsplit; sp0 += 8 * tpi) {
      float mb[8], lb[8];
      floatx4 ob[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        // Slots past nsplit read the pair's first slot again (in bounds) and are dropped below.
        const int sp = sp0 + k * tpi < nsplit ? sp0 + k * tpi : 0;
        const int base = (static_cast<int>(first) + sp) * slot_words;
        mb[k] = ld_sc1(pr, 4 * (base + ml_word));
        lb[k] = ld_sc1(pr, 4 * (base + ml_word + 1));
        const int ob4 = 4 * (base + o_word);
        ob[k] = floatx4{ld_sc1(pr, ob4), ld_sc1(pr, ob4 + 4), ld_sc1(pr, ob4 + 8), ld_sc1(pr, ob4 + 12)};
      }
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (sp0 + k * tpi < nsplit) {
          poison |= lb[k] != lb[k];
          merge_into(m, l, o, mb[k], lb[k], ob[k]);
        }
    }
    for (int off = 1; off < tpi; off <<= 1) {
      const float m2 = __shfl_xor(m, off), l2 = __shfl_xor(l, off);
      const floatx4 o2 = {__shfl_xor(o[0], off), __shfl_xor(o[1], off), __shfl_xor(o[2], off), __shfl_xor(o[3], off)};
      poison |= __shfl_xor(poison, off);
      merge_into(m, l, o, m2, l2, o2);
    }
    if (sub == 0) {
      // A split that met an invalid block id carries NaN, which propagates.
      if (poison) l = NAN;
      const float inv = l > 0.f || l != l ? 1.f / l : 0.f;
      typename DT::vec4 v4;
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = static_cast<T>(o[r] * inv);
      *reinterpret_cast<u32x2*>(out_row + col * D + 4 * d4) = __builtin_bit_cast(u32x2, v4);
    }
  }
}

// One plan item: context tokens [t0, t1) of (sequence s, kv head), read once
// and used by all G query heads of the group.  The item's 16-token tiles are
// dealt out evenly, each wave a contiguous run.  The item carries the block
// ids of each wave's first eight tiles.
struct WaveBlocks {
  int32_t id[8];
};

// The item rows and this wave's carried block ids of plan item idx (uniform
// per wave, so they come through the scalar cache, outside the vector-memory
// order the K/V loads keep).
__device__ __forceinline__ void load_item(const AttnParams& p, uint32_t idx, u32x4& r0, u32x4& r1,
                                          WaveBlocks& wb) {
  const u32x4* rows = reinterpret_cast<const u32x4*>(p.items + idx);
  r0 = rows[0];
  r1 = rows[1];
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const u32x4* ib = rows + 2 + wave * 2;
  const u32x4 a = ib[0], b = ib[1];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    wb.id[e] = static_cast<int32_t>(a[e]);
    wb.id[4 + e] = static_cast<int32_t>(b[e]);
  }
}

template <class DT, int D, int W, int R, class BTI, bool BIG>
__device__ __forceinline__ void decode_item(const AttnParams& p, uint32_t idx, u32x4 r0, u32x4 r1,
                                            const WaveBlocks& ib, char* smem, int& s_merger) {
  using Cfg = DecodeCfg<D, W, R>;
  using T = typename DT::T;
  using V8 = typename DT::vec8;
  constexpr int THREADS = Cfg::kThreads;
  constexpr int NC = Cfg::NC, NN = Cfg::NN, CPR = Cfg::CPR, DMA = Cfg::DMA, PC = Cfg::PER_CHUNK;
  constexpr int TILE_B = Cfg::TILE_B, SLOT_B = Cfg::SLOT_B;

  const int s = static_cast<int>(r0[0]);
  const int64_t qtok = r0[1], t0 = r0[2], t1 = r0[3];
  const uint32_t first = r1[0];
  const int nsplit = static_cast<int>(r1[1]), kvh = static_cast<int>(r1[2]), split = static_cast<int>(r1[3]);
  const int G = p.group, Hkv = p.num_kv_heads;
  // A plan that does not belong to this call is skipped, never followed out of bounds.
  if (static_cast<uint32_t>(s) >= static_cast<uint32_t>(p.num_seqs) || kvh >= Hkv || qtok >= p.num_tokens ||
      t1 < t0 || t1 > p.max_ctx || nsplit < 1 || split >= nsplit || first + static_cast<uint32_t>(split) != idx ||
      static_cast<int64_t>(first) + nsplit > p.item_cap)
    return;

  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps the chunk logic scalar
  const int64_t pair = static_cast<int64_t>(s) * Hkv + kvh;

  const int bs_shift = p.bs_shift;
  const int64_t bs_mask = (int64_t{1} << bs_shift) - 1;
  const int64_t bt_row = static_cast<int64_t>(s) * p.bt_stride;
  const int64_t tiles = (t1 - t0 + 15) >> 4;
  const int64_t per_wave = (tiles + W - 1) / W * 16;
  const int64_t wb = t0 + w * per_wave;
  const int64_t we = t1 < wb + per_wave ? t1 : wb + per_wave;  // wave w's tokens: [wb, we)
  const int nch = wb < we ? static_cast<int>((we - wb + 31) >> 5) : 0;
  const int wtiles = wb < we ? static_cast<int>((we - wb + 15) >> 4) : 0;

  T* out_row = reinterpret_cast<T*>(p.out) + (qtok * p.num_heads + static_cast<int64_t>(kvh) * G) * D;
  const int64_t slot_stride = static_cast<int64_t>(Hkv) * D;  // elements between token rows
  const T* kbase = reinterpret_cast<const T*>(p.k_cache) + static_cast<int64_t>(kvh) * D;
  const T* vbase = reinterpret_cast<const T*>(p.v_cache) + static_cast<int64_t>(kvh) * D;

  // This wave's LDS: the chunk ring, the query tile, the block ids past the carried ones.
  char* ring = smem + w * Cfg::WAVE_B;
  char* qlds = ring + R * SLOT_B;
  char* ids = qlds + Cfg::Q_B;

  int bad = 0;
  float m_run = -INFINITY, l_run = 0.f;
  floatx4 acc[NN];
#pragma unroll
  for (int n = 0; n < NN; ++n) acc[n] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Block id of the wave's tile `tile` >= CARRIED (BIG), from the table
  // entries the wave loaded into `ids`.  Uniform, so the DMA addresses stay
  // scalar.  The first CARRIED tiles' ids come with the item and stay in
  // scalar registers (ib): reading them back from LDS would put an LDS read
  // and its wait in front of those chunks' loads.
  const int64_t e_first = (wb + 16 * Cfg::CARRIED) >> bs_shift;  // table entry of the first tile not carried
  auto carried_block = [&](int tile) -> int64_t {
    int32_t v = ib.id[0];
#pragma unroll
    for (int j = 1; j < Cfg::CARRIED; ++j) v = tile == j ? ib.id[j] : v;
    return v;
  };
  auto tile_block = [&](int tile) -> int64_t {
    uint32_t lo, hi = 0;
    const int64_t e = ((wb + 16 * static_cast<int64_t>(tile)) >> bs_shift) - e_first;
    lo = ds_read_b32(ids + 4 * e);
    if constexpr (sizeof(BTI) == 8) hi = ds_read_b32(ids + 256 + 4 * e);
    lds_wait_all();
    lds_ready(lo);
    lds_ready(hi);
    if constexpr (sizeof(BTI) == 4) hi = static_cast<uint32_t>(static_cast<int32_t>(lo) >> 31);
    lo = __builtin_amdgcn_readfirstlane(lo);
    hi = __builtin_amdgcn_readfirstlane(hi);
    return static_cast<int64_t>(static_cast<uint64_t>(hi) << 32 | lo);
  };

  // Start chunk ci's K and V loads into ring slot `slot`.  LDS unit u * 64 +
  // lane of a tile holds token k = unit / CPR of the chunk, unit position
  // unit % CPR; a token past the wave's range loads token we - 1 again (the
  // same addresses as a lane that needs it, so no extra traffic) and is
  // masked when read.  BIG: one load covers tokens of one 16-token tile,
  // whose block id (blk_a for the first tile, blk_b for the second) is
  // uniform.  Otherwise every lane reads its token's table entry.
  auto issue_chunk = [&](int ci, int slot, int64_t blk_a, int64_t blk_b) {
    const int64_t tb = wb + 32 * static_cast<int64_t>(ci);
    char* kd = ring + slot * SLOT_B;
    char* vd = kd + TILE_B;
#pragma unroll
    for (int u = 0; u < DMA; ++u) {
      const int unit = u * 64 + lane;
      const int k = unit / CPR, pc = unit % CPR;
      int64_t t = tb + k;
      t = t < we ? t : we - 1;
      int64_t blk;
      if constexpr (BIG) {
        blk = (u * 64) / CPR < 16 ? blk_a : blk_b;
      } else {
        blk = ld_idx<BTI>(p.bt, bt_row + (t >> bs_shift));
      }
      if (blk < 0 || blk >= p.num_blocks) {
        bad = 1;
        blk = 0;
      }
      const int64_t row = ((blk << bs_shift) + (t & bs_mask)) * slot_stride;
      dma_lds16(kbase + row + ((pc ^ k_swz(k)) << 3), kd + u * 1024);
      dma_lds16(vbase + row + ((pc ^ v_swz(k)) << 3), vd + u * 1024);
    }
  };

  V8 qop[NC];
  // One chunk from ring slot `slot`: S^T = K Q^T (sacc[h][r]: token 16h + 4g
  // + r of the chunk, head c16), the online softmax, O^T += V^T P^T.
  auto compute_chunk = [&](int ci, int slot) {
    const int64_t tb = wb + 32 * static_cast<int64_t>(ci);
    const char* kt = ring + slot * SLOT_B;
    const char* vt = kt + TILE_B;
    // Every LDS read of the chunk goes out before one wait: K rows (key
    // 16h + c16, dims 32c + 8g ..) and the transposing V^T reads
    // (ds_read_b64_tr_b16 gives lane c16 of group g V^T row 16n + c16 at keys
    // 16h + 4g + 0..3 when it points at dims 16n + 4 (c16 & 3) .. +3 of key
    // 16h + 4g + (c16 >> 2)).
    u32x4 kraw[2][NC];
    u32x2 hop[NN][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int key = 16 * h + c16;
#pragma unroll
      for (int c = 0; c < NC; ++c) kraw[h][c] = ds_read_b128(kt + key * D * 2 + (((4 * c + g) ^ k_swz(key)) << 4));
    }
    const int d0 = 4 * (c16 & 3);
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int key = 16 * h + 4 * g + (c16 >> 2);
        const int d = 16 * n + d0;
        hop[n][h] = ds_read_tr16_b64(vt + key * D * 2 + (((d >> 3) ^ v_swz(key)) << 4) + ((d & 7) << 1));
      }
    lds_wait_all();
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int c = 0; c < NC; ++c) lds_ready(kraw[h][c]);
#pragma unroll
    for (int n = 0; n < NN; ++n) {
      lds_ready(hop[n][0]);
      lds_ready(hop[n][1]);
    }
    floatx4 sacc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sacc[h] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) sacc[h] = mfma16x16x32(DT{}, __builtin_bit_cast(V8, kraw[h][c]), qop[c], sacc[h]);
    }
    float sv[2][4];
    float mloc = -INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = tb + 16 * h + 4 * g + r < we ? sacc[h][r] * p.scale_log2 : -INFINITY;
        sv[h][r] = x;
        mloc = fmaxf(mloc, x);
      }
    mloc = group4_max_swap(mloc);
    const float m_new = fmaxf(m_run, mloc);
    const bool none = m_new == -INFINITY;
    const float alpha = none ? 1.f : fast_exp2(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pr = none ? 0.f : fast_exp2(sv[h][r] - m_new);
        sv[h][r] = pr;
        psum += pr;
      }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int n = 0; n < NN; ++n) acc[n] *= alpha;
    m_run = m_new;
    // P^T operand: k-slot e of group g is token 4g + e of tile 0 (e < 4) or
    // of tile 1 (e >= 4), matching the V^T reads above.
    V8 pt;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pt[e] = static_cast<T>(sv[0][e]);
      pt[4 + e] = static_cast<T>(sv[1][e]);
    }
    // Tokens past the wave's range hold a copy of token we - 1: their V
    // elements are zeroed (their P is zero, but V may hold inf or NaN).
    const bool vfull = tb + 32 <= we;
#pragma unroll
    for (int n = 0; n < NN; ++n) {
      V8 va = __builtin_bit_cast(V8, u32x4{hop[n][0][0], hop[n][0][1], hop[n][1][0], hop[n][1][1]});
      if (!vfull) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = 16 * (e >> 2) + 4 * g + (e & 3);
          va[e] = tb + key < we ? va[e] : static_cast<T>(0.f);
        }
      }
      acc[n] = mfma16x16x32(DT{}, va, pt, acc[n]);
    }
  };

  // All nch (<= R) chunks of the wave from ring slots 0 .. nch-1 at once.
  auto compute_all = [&](int n_ch) {
    floatx4 sacc[R][2];
#pragma unroll
    for (int ci = 0; ci < R; ++ci) {
      if (ci < n_ch) {
        const char* kt = ring + ci * SLOT_B;
        u32x4 kraw[2][NC];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int key = 16 * h + c16;
#pragma unroll
          for (int c = 0; c < NC; ++c)
            kraw[h][c] = ds_read_b128(kt + key * D * 2 + (((4 * c + g) ^ k_swz(key)) << 4));
        }
        lds_wait_all();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          sacc[ci][h] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            lds_ready(kraw[h][c]);
            sacc[ci][h] = mfma16x16x32(DT{}, __builtin_bit_cast(V8, kraw[h][c]), qop[c], sacc[ci][h]);
          }
        }
      }
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int ci = 0; ci < R; ++ci)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t t = wb + 32 * ci + 16 * h + 4 * g + r;
          const float x = ci < n_ch && t < we ? sacc[ci][h][r] * p.scale_log2 : -INFINITY;
          sacc[ci][h][r] = x;
          mloc = fmaxf(mloc, x);
        }
    const float m = group4_max_swap(mloc);
    const bool none = m == -INFINITY;
    float psum = 0.f;
    const int d0 = 4 * (c16 & 3);
#pragma unroll
    for (int ci = 0; ci < R; ++ci) {
      if (ci < n_ch) {
        V8 pt;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float pr = none ? 0.f : fast_exp2(sacc[ci][h][r] - m);
            psum += pr;
            pt[4 * h + r] = static_cast<T>(pr);
          }
        const char* vt = ring + ci * SLOT_B + TILE_B;
        u32x2 hop[NN][2];
#pragma unroll
        for (int n = 0; n < NN; ++n)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int key = 16 * h + 4 * g + (c16 >> 2);
            const int d = 16 * n + d0;
            hop[n][h] = ds_read_tr16_b64(vt + key * D * 2 + (((d >> 3) ^ v_swz(key)) << 4) + ((d & 7) << 1));
          }
        lds_wait_all();
        const int64_t tb = wb + 32 * ci;
        const bool vfull = tb + 32 <= we;
#pragma unroll
        for (int n = 0; n < NN; ++n) {
          lds_ready(hop[n][0]);
          lds_ready(hop[n][1]);
          V8 va = __builtin_bit_cast(V8, u32x4{hop[n][0][0], hop[n][0][1], hop[n][1][0], hop[n][1][1]});
          if (!vfull) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int key = 16 * (e >> 2) + 4 * g + (e & 3);
              va[e] = tb + key < we ? va[e] : static_cast<T>(0.f);
            }
          }
          acc[n] = mfma16x16x32(DT{}, va, pt, acc[n]);
        }
      }
    }
    m_run = none ? -INFINITY : m;
    l_run = psum;
  };

  if (nch > 0) {
    // The query tile (rows: the group's heads; rows past G repeat the last
    // head and are zeroed when read), then, for waves with more tiles than
    // the item carries, the table entries from the first tile not carried
    // on: both land before chunk 0.  Waves with only carried tiles skip the
    // table load: issued by every wave, it delayed every wave's first data
    // (c1 8.10 -> 7.84 us, c2 12.16 -> 12.01 us per call on MI355X without
    // it).
    {
      const T* qg = reinterpret_cast<const T*>(p.query) + (qtok * p.num_heads + static_cast<int64_t>(kvh) * G) * D;
#pragma unroll
      for (int u = 0; u < Cfg::QD; ++u) {
        const int unit = u * 64 + lane;
        int row = unit / CPR;
        row = row < G ? row : G - 1;
        dma_lds16(qg + row * D + (unit % CPR) * 8, qlds + u * 1024);
      }
    }
    if constexpr (BIG) {
      if (wtiles > Cfg::CARRIED) {
        // Lane l: entry e_first + l (at most the wave's last), low words at
        // ids[l], high words (int64 tables) at ids[64 + l].
        const int64_t e_last = (we - 1) >> bs_shift;
        int64_t e = e_first + lane;
        e = e <= e_last ? e : e_last;
        const char* src = reinterpret_cast<const char*>(reinterpret_cast<const BTI*>(p.bt) + bt_row + e);
        dma_lds4(src, ids);
        if constexpr (sizeof(BTI) == 8) dma_lds4(src + 4, ids + 256);
      }
    }
    // Chunks 0 .. R-1 (their tiles' block ids come with the item).
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (r < nch) {
        if constexpr (BIG) {
          const int64_t a = ib.id[2 * r];
          issue_chunk(r, r, a, 2 * r + 1 < wtiles ? static_cast<int64_t>(ib.id[2 * r + 1]) : a);
        } else {
          issue_chunk(r, r, 0, 0);
        }
      }
    if (nch <= R) {
      // Every chunk of the wave is in flight: they land at about the same
      // time, so they are processed together (one maximum, one pass of
      // exponentials) instead of one dependent online-softmax step each.
      wait_chunks<PC, R>(0);
      u32x4 qraw[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) qraw[c] = ds_read_b128(qlds + c16 * D * 2 + (4 * c + g) * 16);
      lds_wait_all();
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        lds_ready(qraw[c]);
        qop[c] = c16 < G ? __builtin_bit_cast(V8, qraw[c]) : zero8<DT>();
      }
      compute_all(nch);
    } else
    for (int ci = 0; ci < nch; ++ci) {
      const int slot = ci % R;
      const int ahead = nch - 1 - ci;
      wait_chunks<PC, R>(ahead < R - 1 ? ahead : R - 1);
      if (ci == 0) {
        u32x4 qraw[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) qraw[c] = ds_read_b128(qlds + c16 * D * 2 + (4 * c + g) * 16);
        lds_wait_all();
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          lds_ready(qraw[c]);
          qop[c] = c16 < G ? __builtin_bit_cast(V8, qraw[c]) : zero8<DT>();
        }
      }
      compute_chunk(ci, slot);
      const int nx = ci + R;
      if (nx < nch) {
        // The slot's LDS reads are done (their results were used above).
        if constexpr (BIG) {
          int64_t a, b;
          if (2 * nx + 1 < Cfg::CARRIED) {
            a = carried_block(2 * nx);
            b = carried_block(2 * nx + 1);
          } else {
            a = tile_block(2 * nx);
            b = 2 * nx + 1 < wtiles ? tile_block(2 * nx + 1) : a;
          }
          issue_chunk(nx, slot, a, 2 * nx + 1 < wtiles ? b : a);
        } else {
          issue_chunk(nx, slot, 0, 0);
        }
      }
    }
  }
  l_run = group4_sum_swap(l_run);

  // Merge the waves' (max, sum, O) through LDS.  Each wave writes its block
  // into the first slot of its own ring (no other wave touches that memory,
  // so no barrier is needed before the writes): rows (head) padded to RED_LD
  // floats and written a float4 at a time, so the 16 head lanes of a store
  // start on 16 different 4-bank groups; then the maxima, the sums and the
  // wave's invalid-block flag.  One barrier hands the blocks over.
  constexpr int RED_LD = Cfg::RED_LD;
  static_assert(16 * RED_LD * 4 + 33 * 4 <= Cfg::SLOT_B, "a wave's reduce block fits its first ring slot");
  auto red_o = [&](int ww) { return reinterpret_cast<float*>(smem + ww * Cfg::WAVE_B); };
  auto red_m = [&](int ww) { return red_o(ww) + 16 * RED_LD; };
  auto red_l = [&](int ww) { return red_o(ww) + 16 * RED_LD + 16; };
  auto red_bad = [&](int ww) { return reinterpret_cast<int*>(red_o(ww) + 16 * RED_LD + 32); };
  {
    float* ro = red_o(w);
#pragma unroll
    for (int n = 0; n < NN; ++n) *reinterpret_cast<floatx4*>(ro + c16 * RED_LD + 16 * n + 4 * g) = acc[n];
    if (g == 0) {
      red_m(w)[c16] = m_run;
      red_l(w)[c16] = l_run;
    }
    const int wave_bad = __builtin_amdgcn_ballot_w64(bad != 0) != 0;
    if (lane == 0) *red_bad(w) = wave_bad;
  }
  __syncthreads();
  bad = 0;
#pragma unroll
  for (int ww = 0; ww < W; ++ww) bad |= *red_bad(ww);

  const int slot_words = p.slot_words;
  const __amdgpu_buffer_rsrc_t pr =
      __builtin_amdgcn_make_buffer_rsrc(p.part, static_cast<short>(0), p.part_bytes, kBufferWord3);
  // One float4 of the workgroup's output per thread and round: (head col, dims 4*d4..+3).
  for (int it = tid; it < G * (D / 4); it += THREADS) {
    const int col = it / (D / 4), d4 = it % (D / 4);
    // Every read first, then branch-free arithmetic: a wave without tokens
    // (max -inf) contributes nothing.
    float mw[W], lw[W];
    floatx4 ow[W];
#pragma unroll
    for (int ww = 0; ww < W; ++ww) {
      mw[ww] = red_m(ww)[col];
      lw[ww] = red_l(ww)[col];
      ow[ww] = *reinterpret_cast<const floatx4*>(red_o(ww) + col * RED_LD + 4 * d4);
    }
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < W; ++ww) M = fmaxf(M, mw[ww]);
    float lsum = 0.f;
    floatx4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ww = 0; ww < W; ++ww) {
      const bool on = mw[ww] != -INFINITY;
      const float sc = on ? fast_exp2(mw[ww] - M) : 0.f;
      lsum += on ? lw[ww] * sc : 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] += on ? ow[ww][r] * sc : 0.f;
    }
    if (bad) {
      lsum = NAN;
      o = floatx4{NAN, NAN, NAN, NAN};
    }
    if (nsplit == 1) {
      const float inv = lsum > 0.f || lsum != lsum ? 1.f / lsum : 0.f;
      typename DT::vec4 v4;
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = static_cast<T>(o[r] * inv);
      *reinterpret_cast<u32x2*>(out_row + col * D + 4 * d4) = __builtin_bit_cast(u32x2, v4);
    } else {
      const int base = static_cast<int>(idx) * slot_words;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), pr, 4 * (base + col * D + 4 * d4), 0,
                                             kSc1);
      if (d4 == 0)
        __builtin_amdgcn_raw_buffer_store_b64(
            u32x2{__builtin_bit_cast(uint32_t, M), __builtin_bit_cast(uint32_t, lsum)}, pr,
            4 * (base + G * D + 2 * col), 0, kSc1);
    }
  }
  if (nsplit == 1) return;

  // Arrive only once this workgroup's partial is acknowledged (device scope).
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(&p.counters[pair], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_merger = prev == static_cast<unsigned>(nsplit - 1);
  }
  __syncthreads();
  if (!s_merger) return;
  merge_partials<DT, D, THREADS>(p, pr, first, nsplit, out_row);
  if (tid == 0) __hip_atomic_store(&p.counters[pair], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <class DT, int D, int W, int R, class BTI, bool BIG>
__global__ __launch_bounds__(W * 64) void paged_decode_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) char smem[DecodeCfg<D, W, R>::LDS];
  __shared__ int s_merger;
  // The first item loads together with the plan's item count: the grid
  // never exceeds the plan's capacity, so the read is in bounds either way.
  uint32_t idx = blockIdx.x;
  u32x4 r0, r1;
  WaveBlocks ib;
  load_item(p, idx, r0, r1, ib);
  const uint32_t n_hdr = p.plan_hdr->n_items;
  // Both scalar loads are in flight before either is waited for (the
  // compiler would otherwise sink the item's load below the count check:
  // two round trips before the first K/V load instead of one).
  asm volatile("" ::"s"(n_hdr), "s"(r0), "s"(r1), "s"(ib.id[0]), "s"(ib.id[1]), "s"(ib.id[2]), "s"(ib.id[3]),
               "s"(ib.id[4]), "s"(ib.id[5]), "s"(ib.id[6]), "s"(ib.id[7]));
  const uint32_t n_items = n_hdr < p.item_cap ? n_hdr : static_cast<uint32_t>(p.item_cap);
  while (idx < n_items) {
    decode_item<DT, D, W, R, BTI, BIG>(p, idx, r0, r1, ib, smem, s_merger);
    // Everything the item issued has completed, and the compiler's wait-count
    // pass sees that through this builtin: it then carries no pending loads
    // around the loop, so it puts no wait of its own into the next item,
    // where any vmcnt wait would also drain that item's K/V loads.
    __builtin_amdgcn_s_waitcnt(0);
    idx += gridDim.x;
    if (idx < n_items) load_item(p, idx, r0, r1, ib);
    __syncthreads();  // the next item reuses the LDS
  }
  // The next call of a step (every layer uses the step's plan) starts this
  // workgroup index on the same XCD (blockIdx mod 8) and reads the same
  // first item and the header: read them once more now, with vector loads,
  // so they wait in this XCD's L2.  Measured on MI355X as paired library
  // swaps on one box (four runs each, spread 0.02 us): c2 12.25 -> 12.19 us
  // per call, c1 8.19 -> 8.11.  Read-only and inside the plan buffer (the
  // grid never exceeds its capacity); a call whose neighbour has another
  // grid only loses the warm lines.
  if (threadIdx.x < 11) {
    const u32x4* rows = reinterpret_cast<const u32x4*>(p.items + blockIdx.x);
    const void* ptr = threadIdx.x < 10 ? static_cast<const void*>(rows + threadIdx.x)
                                       : static_cast<const void*>(p.plan_hdr);
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(ptr) : "memory");
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

// --------------------------------------------------------------------------
// Variable-length rows (prefill, chunked prefill, the prefill rows of a mixed
// batch): flash-attention forward over the paged cache.  The columns of a
// (sequence, kv head) are its flattened (query row, head of the group) pairs,
// ql * G of them; a workgroup owns COLS of them and walks the pair's keys
// from position 0 to the causal limit of its last column, KT keys per step.
//
// The workgroup is KG key groups of WC waves.  Wave i of every group owns the
// same CT 16-column tiles; group k takes steps k, k + KG, k + 2KG, ... with
// its own running (max, sum, O) and the groups are merged through LDS at the
// end, so the dependent chain of steps is KG times shorter and each SIMD
// holds KG waves.  Each step's K and V tiles go from HBM straight into LDS
// with global_load_lds (16 bytes per lane, no registers), two macro-steps
// (KG steps each) ahead of the one being computed, through a ring of three
// macro-slots; every byte is read once per workgroup and one barrier per
// macro-step hands a slot over.  The block-table entries of the keys come
// first into LDS (a window of TBL entries), so the loads need no table round
// trip of their own.
//
// LDS layout of a stage: K tile then V tile, both [KT][D] rows of 16-byte
// chunks, chunk c of key k stored at chunk c ^ k_swz(k) (K) or c ^ v_swz(k)
// (V) of its row.  A DMA lane picks the global chunk that belongs at its LDS
// slot, so the swizzle costs nothing on the write side and spreads the MFMA
// operand reads (16-byte K rows; 8-byte transposing V reads) over all banks.
// --------------------------------------------------------------------------
template <int D, int CT_>
struct PrefillCfg {
  // Four key groups of two column waves (32 keys a step, 64 columns per
  // workgroup) measured slower at c3 than two groups of four (51.0 against
  // 45.2 us per call): twice the workgroups, still one per CU.
  static constexpr int KG = 2;                  // key groups
  static constexpr int WC = 4;                  // column waves per group
  static constexpr int W = KG * WC;             // waves per workgroup
  static constexpr int THREADS = W * 64;
  static constexpr int CT = CT_;                // 16-column tiles per wave
  static constexpr int KT = D == 64 ? 64 : 32;  // keys per step (8 KiB per tile)
  static constexpr int NT = KT / 16, NC = D / 32, NN = D / 16;
  static constexpr int CPR = D / 8;             // 16-byte chunks per key row
  static constexpr int TILE = KT * D * 2;       // bytes of one K or V tile
  static constexpr int DMA = KG * TILE / (THREADS * 16);  // 16-byte loads per thread per K (or V) of a macro-step
  static constexpr int NSLOT = 3;               // macro-slots in the ring
  static constexpr int RING = NSLOT * KG * 2 * TILE;
  static constexpr int TBL = 4096;              // table entries per window
  static constexpr int LDS = RING + TBL * 4 + 16;
  static constexpr int COLS = WC * CT * 16;     // columns per workgroup
  static constexpr int NF = CT * (NN * 4 + 2);  // floats per lane a group hands over in the merge
  static constexpr int PU = CT * (NN + 1);      // 16-byte units per lane of a split's partial
  static constexpr int SLOT_BYTES = WC * PU * 64 * 16;
  static_assert(DMA >= 1 && DMA * THREADS * 16 == KG * TILE && TILE % 1024 == 0, "loads must tile a macro-step");
  static_assert(NT % 2 == 0, "P^T operand pairs two 16-key tiles");
  static_assert(WC * NF * 64 * 4 <= RING, "merge buffer fits the ring");
};


// Wait until at most N of this wave's vector-memory operations are pending,
// drain its LDS operations, then barrier.  Written as one asm statement so the
// compiler adds no wait of its own for the LDS loads still in flight.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

constexpr int kPrefillThreads = 512;

template <class DT, int D, int CT, class BTI>
__global__ __launch_bounds__(kPrefillThreads) void paged_prefill_kernel(PrefillParams p) {
  using Cfg = PrefillCfg<D, CT>;
  static_assert(Cfg::THREADS == kPrefillThreads, "launch bounds match the workgroup");
  using T = typename DT::T;
  using V8 = typename DT::vec8;
  constexpr int KT = Cfg::KT, NT = Cfg::NT, NC = Cfg::NC, NN = Cfg::NN, KG = Cfg::KG;
  constexpr int CPR = Cfg::CPR, TILE = Cfg::TILE, DMA = Cfg::DMA, W = Cfg::W;
  __shared__ __attribute__((aligned(16))) char smem[Cfg::LDS];
  int* tbl = reinterpret_cast<int*>(smem + Cfg::RING);
  int* bad_first = tbl + Cfg::TBL;

  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps step logic scalar
  const int kg = w / Cfg::WC, wc = w % Cfg::WC;            // key group, column wave
  const int G = p.group, Hkv = p.num_kv_heads;

  // Work item: (sequence, kv head, column block) and, with a plan, the split
  // of its key range.  Planned items run the heaviest column blocks first.
  int s, kvh, split = 0, nsplit = 1, split_mk = 0, slot_base = 0, pair_base = 0;
  int64_t ql_host = -1;
  if (p.plan_n > 0) {
    const uint32_t e0w = p.plan[3 * blockIdx.y], e1w = p.plan[3 * blockIdx.y + 1];
    ql_host = p.plan[3 * blockIdx.y + 2];
    s = static_cast<int>(e0w & 0xFFFFu);
    nsplit = static_cast<int>((e0w >> 16) & 0x3Fu) + 1;
    split_mk = static_cast<int>(e0w >> 22);
    slot_base = static_cast<int>(e1w & 0xFFFFu);
    pair_base = static_cast<int>(e1w >> 16);
    kvh = static_cast<int>(blockIdx.x % Hkv);
    split = static_cast<int>((blockIdx.x / Hkv) % nsplit);
  } else {
    kvh = blockIdx.y;
    s = blockIdx.z;
  }

  // Positions are int32 (the host caps max_ctx below 2^31).
  const int64_t q0 = load_index(p.qsl, s, p.qsl64);
  const int64_t ql64 = load_index(p.qsl, s + 1, p.qsl64) - q0;
  // Loaded with the query range (one round trip instead of two: c3 44.64 ->
  // 44.49 us); s + 1 indexes query_start_loc, so s indexes seq_lens.
  int64_t L64 = load_index(p.seq_lens, s, p.sl64);
  if (ql64 <= 0 || (p.skip_decode_rows && ql64 == 1)) return;
  if (q0 < 0 || q0 + ql64 > p.num_tokens) return;
  const int64_t ncols = ql64 * G;
  const int64_t ncb = (ncols + Cfg::COLS - 1) / Cfg::COLS;
  int64_t cb = blockIdx.x;
  bool plan_broken = false;
  if (p.plan_n > 0) {
    const int64_t rcb = blockIdx.x / Hkv / nsplit;
    if (rcb >= ncb) return;
    cb = ncb - 1 - rcb;
    // A device query length the host plan did not describe is a broken
    // contract: the blocks it reaches are written as NaN and no split state
    // (slots, counters) is touched.
    if (ql64 != ql_host) {
      if (split != 0) return;
      plan_broken = true;
      nsplit = 1;
    }
  }
  const int64_t c_wg = cb * Cfg::COLS;
  if (c_wg >= ncols) return;
  L64 = L64 < p.max_ctx ? L64 : p.max_ctx;
  const int L = static_cast<int>(L64 > 0 ? L64 : 0);
  const int64_t ctx0 = L - ql64;  // absolute position of query row 0 (may be negative)
  const int bs_shift = p.bs_shift;
  const int bs_mask = (1 << bs_shift) - 1;

  // Keys the workgroup needs: up to the causal limit of its last column.
  const int64_t c_last_wg = (ncols < c_wg + Cfg::COLS ? ncols : c_wg + Cfg::COLS) - 1;
  int64_t kv_end64 = ctx0 + c_last_wg / G + 1;
  kv_end64 = kv_end64 < L ? kv_end64 : L;
  const int kv_end = static_cast<int>(kv_end64 > 0 ? kv_end64 : 0);

  // This wave's columns: Q^T operands, causal limits, output rows.
  const int64_t c_wave = c_wg + wc * CT * 16;
  const bool wave_on = c_wave < ncols;
  int kv_end_w = 0;
  int64_t qmin_w = -1;
  if (wave_on) {
    const int64_t c_last = (ncols < c_wave + CT * 16 ? ncols : c_wave + CT * 16) - 1;
    const int64_t e = ctx0 + c_last / G + 1;
    kv_end_w = static_cast<int>(e < 0 ? 0 : (e < L ? e : L));
    qmin_w = ctx0 + c_wave / G;
  }
  V8 qop[CT][NC];
  int lim[CT];  // last key position a column may see (-1: none)
  int64_t orow[CT];
  bool cval[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int64_t c = c_wave + ct * 16 + c16;
    cval[ct] = c < ncols;
    const int64_t qi = cval[ct] ? c / G : 0;
    const int64_t h = cval[ct] ? c - qi * G : 0;
    const int64_t qpos = ctx0 + qi;
    lim[ct] = cval[ct] ? static_cast<int>(qpos < kv_end_w - 1 ? qpos : kv_end_w - 1) : -1;
    orow[ct] = ((q0 + qi) * p.num_heads + static_cast<int64_t>(kvh) * G + h) * D;
    const T* qrow = reinterpret_cast<const T*>(p.query) + orow[ct];
#pragma unroll
    for (int c2 = 0; c2 < NC; ++c2) {
      qop[ct][c2] = cval[ct] ? load16<DT>(qrow + 32 * c2 + 8 * g) : zero8<DT>();
      // A negative scale moves into Q (exact sign flips), so the softmax can
      // take maxima over raw scores and fold the scale into one FMA.
      if (p.scale_log2 < 0.f)
        qop[ct][c2] = __builtin_bit_cast(V8, __builtin_bit_cast(u32x4, qop[ct][c2]) ^ 0x80008000u);
    }
  }
  const float sc = fabsf(p.scale_log2);

  // Running softmax state per column: maximum, the row sum of P, and O^T.
  // The row sum runs on the matrix cores: one more PV product whose V^T
  // operand is a row of ones (row 0 of the tile, every key) puts sum_k P[k]
  // of column c16 in element 0 of lane (g = 0, c16) and zero everywhere else,
  // which is this lane's share of the column's sum as group4_sum_swap adds
  // them up at the end.  It sums the same half-precision P that the PV
  // product weighs V with, and takes 16 VALU adds per column tile and step
  // off the softmax.
  float m_run[CT], l_run[CT];
  floatx4 acc[CT][NN], lacc[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    m_run[ct] = -INFINITY;
    l_run[ct] = 0.f;
    lacc[ct] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < NN; ++n) acc[ct][n] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  V8 ones_row;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones_row[e] = static_cast<T>(c16 == 0 ? 1.f : 0.f);

  const int64_t slot_stride = static_cast<int64_t>(Hkv) * D;
  const int64_t bt_row = static_cast<int64_t>(s) * p.bt_stride;
  const T* kbase = reinterpret_cast<const T*>(p.k_cache) + static_cast<int64_t>(kvh) * D;
  const T* vbase = reinterpret_cast<const T*>(p.v_cache) + static_cast<int64_t>(kvh) * D;
  int e0 = 0;      // first table entry of the current window
  int kv_win = 0;  // keys covered by the window's entries (and below kv_end)

  // Start the K/V loads of macro-step M into macro-slot `slot` (stages
  // slot * KG + k, k < KG, one per step).  Load u of wave w covers the 1 KiB
  // piece b = u * W + w of the macro-step's K (and of its V): piece b % PT of
  // step M * KG + b / PT, lane `lane` filling its 16-byte slot b % PT * 64 +
  // lane.  Keys past the window or kv_end read an in-bounds slot; their
  // scores are masked and their V values replaced by zero when read.
  auto dma_macro = [&](int M, int slot) {
    constexpr int PT = TILE / 1024;  // 1 KiB pieces per tile
#pragma unroll
    for (int u = 0; u < DMA; ++u) {
      const int b = u * W + w;
      const int k = b / PT, piece = b % PT;
      char* st = smem + (slot * KG + k) * 2 * TILE;
      const int pos = piece * 64 + lane;
      const int key = pos / CPR, pc = pos % CPR;
      const int t = (M * KG + k) * KT + key;
      const bool in = t < kv_win;
      const int blk = tbl[in ? (t >> bs_shift) - e0 : 0];
      const bool valid = in && blk >= 0;
      const int64_t off = valid ? ((static_cast<int64_t>(blk) << bs_shift) + (t & bs_mask)) * slot_stride : 0;
      const T* gk = kbase + off + ((pc ^ k_swz(key)) << 3);
      const T* gv = vbase + off + ((pc ^ v_swz(key)) << 3);
      __builtin_amdgcn_global_load_lds((gbl_void_ptr)(gk), (lds_void_ptr)(st + piece * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((gbl_void_ptr)(gv), (lds_void_ptr)(st + TILE + piece * 1024), 16, 0, 0);
    }
  };

  // One step of this wave's columns from `stage`.
  auto compute = [&](int stage, int step) {
    const int tb = step * KT;
    if (tb >= kv_end_w) return;
    const char* kt = smem + stage * 2 * TILE;
    const char* vt = kt + TILE;
    floatx4 sacc[CT][NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int key = 16 * j + c16;
      V8 kop[NC];
#pragma unroll
      for (int c2 = 0; c2 < NC; ++c2)
        kop[c2] = *reinterpret_cast<const V8*>(kt + key * D * 2 + (((4 * c2 + g) ^ k_swz(key)) << 4));
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        sacc[ct][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c2 = 0; c2 < NC; ++c2) sacc[ct][j] = mfma16x16x32(DT{}, kop[c2], qop[ct][c2], sacc[ct][j]);
      }
    }
    // The V^T operands of the whole step (see the PV product below), issued
    // now as asm so their LDS latency hides behind the softmax.  Through the
    // builtin, the compiler's wait-count pass would put an s_waitcnt vmcnt(0)
    // in front of the first one (it cannot tell them from the K/V loads in
    // flight into the ring), draining the prefetch of the next macro-steps.
    const int d0 = 4 * (c16 & 3);
    u32x2 vraw[NT / 2][NN][2];
#pragma unroll
    for (int pb = 0; pb < NT / 2; ++pb)
#pragma unroll
      for (int n = 0; n < NN; ++n)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int key = 32 * pb + 16 * h + 4 * g + (c16 >> 2);
          const int d = 16 * n + d0;
          vraw[pb][n][h] = ds_read_tr16_b64(vt + key * D * 2 + (((d >> 3) ^ v_swz(key)) << 4) + ((d & 7) << 1));
        }
    // Online softmax in base 2 (sc = |scale| * log2 e).  When every key of the
    // step precedes every column of the wave, the maximum is taken over raw
    // scores and p = exp2(s * sc - m) is one FMA; otherwise key
    // tb + 16j + 4g + r of a column is masked by the column's limit.
    const bool full = tb + KT - 1 <= qmin_w;
    const bool vfull = tb + KT <= kv_end;
    V8 pt[CT][NT / 2], va[NT / 2][NN];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      float sv[NT][4];
      float m_new, alpha;
      if (full) {
        float mloc = sacc[ct][0][0];
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) mloc = fmaxf(mloc, sacc[ct][j][r]);
        m_new = fmaxf(m_run[ct], group4_max_swap(mloc) * sc);
        alpha = fast_exp2(m_run[ct] - m_new);
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) sv[j][r] = fast_exp2(__builtin_fmaf(sacc[ct][j][r], sc, -m_new));
      } else {
        const int room = lim[ct] - tb - 4 * g;
        float mloc = -INFINITY;
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            sv[j][r] = 16 * j + r <= room ? sacc[ct][j][r] * sc : -INFINITY;
            mloc = fmaxf(mloc, sv[j][r]);
          }
        m_new = fmaxf(m_run[ct], group4_max_swap(mloc));
        const bool none = m_new == -INFINITY;
        alpha = none ? 1.f : fast_exp2(m_run[ct] - m_new);
        const float msub = none ? 0.f : m_new;  // exp2(-inf - 0) = 0 for fully masked columns
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) sv[j][r] = fast_exp2(sv[j][r] - msub);
      }
      // Rescale only when some column's maximum moved (alpha == 1 is exact);
      // the row sum's other elements stay zero.
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
        for (int n = 0; n < NN; ++n) acc[ct][n] *= alpha;
        lacc[ct][0] *= alpha;
      }
      m_run[ct] = m_new;
#pragma unroll
      for (int pb = 0; pb < NT / 2; ++pb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pt[ct][pb][e] = static_cast<T>(sv[2 * pb][e]);
          pt[ct][pb][4 + e] = static_cast<T>(sv[2 * pb + 1][e]);
        }
      // O^T += V^T P^T for this column tile, right after its softmax: the
      // MFMAs run while the next tile's softmax issues.  k-slot 4h + e of lane
      // group g is key 32pb + 16h + 4g + e, matching P^T.  ds_read_b64_tr_b16
      // gives lane i of a 16-lane group element e = element i & 3 of the 8
      // bytes lane (i >> 2) + 4e of the group addressed, so lane c16 of group
      // g points at head dims 16n + 4 (c16 & 3) .. +3 of key 32pb + 16h + 4g +
      // (c16 >> 2) and receives V^T row 16n + c16 at keys 32pb + 16h + 4g +
      // 0..3.  Keys at or past kv_end (only in the last step) contribute zero.
      if (ct == 0) {
        lds_wait_all();
#pragma unroll
        for (int pb = 0; pb < NT / 2; ++pb)
#pragma unroll
          for (int n = 0; n < NN; ++n) {
            lds_ready(vraw[pb][n][0]);
            lds_ready(vraw[pb][n][1]);
            va[pb][n] = __builtin_bit_cast(
                V8, u32x4{vraw[pb][n][0][0], vraw[pb][n][0][1], vraw[pb][n][1][0], vraw[pb][n][1][1]});
            if (!vfull) {
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const int key = 32 * pb + 16 * (e >> 2) + 4 * g + (e & 3);
                va[pb][n][e] = tb + key < kv_end ? va[pb][n][e] : static_cast<T>(0.f);
              }
            }
          }
      }
#pragma unroll
      for (int pb = 0; pb < NT / 2; ++pb) {
#pragma unroll
        for (int n = 0; n < NN; ++n) acc[ct][n] = mfma16x16x32(DT{}, va[pb][n], pt[ct][pb], acc[ct][n]);
        lacc[ct] = mfma16x16x32(DT{}, ones_row, pt[ct][pb], lacc[ct]);
      }
    }
  };

  if (tid == 0) *bad_first = 0x7FFFFFFF;
  // Macro-step M covers steps M * KG + k, k < KG (step M * KG + k by group k).
  // A split runs macro-steps [M_begin, M_end) of the column block's range.
  constexpr int MKEYS = KG * KT;
  const int nmacro = (kv_end + MKEYS - 1) / MKEYS;
  int nsplit_eff = 1, M_begin = 0, M_end = nmacro;
  if (nsplit > 1) {
    nsplit_eff = nmacro > split_mk ? (nmacro + split_mk - 1) / split_mk : 1;
    if (split >= nsplit_eff) return;  // no keys for this split: it does not arrive
    M_begin = split * split_mk;
    M_end = M_begin + split_mk < nmacro ? M_begin + split_mk : nmacro;
  }
  const int win_macro = (Cfg::TBL << bs_shift) / MKEYS;
  for (int M0 = M_begin; M0 < M_end; M0 += win_macro) {
    const int M1 = M0 + win_macro < M_end ? M0 + win_macro : M_end;
    e0 = (M0 * MKEYS) >> bs_shift;
    kv_win = M1 * MKEYS < kv_end ? M1 * MKEYS : kv_end;
    const int ne_all = ((kv_win + bs_mask) >> bs_shift) - e0;
    const int ne = ne_all < Cfg::TBL ? ne_all : Cfg::TBL;
    __syncthreads();  // the previous window's loads and table readers are done
    for (int base = 0; base < ne; base += 4 * Cfg::THREADS) {
      int64_t v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        int i = base + u * Cfg::THREADS + tid;
        i = i < ne ? i : ne - 1;
        v[u] = ld_idx<BTI>(p.bt, bt_row + e0 + i);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = base + u * Cfg::THREADS + tid;
        if (i < ne) {
          const bool ok = v[u] >= 0 && v[u] < p.num_blocks;
          tbl[i] = ok ? static_cast<int>(v[u]) : -1;
          if (!ok) atomicMin(bad_first, e0 + i);
        }
      }
    }
    __syncthreads();

    // Macro-steps M0 .. M1-1 through the three slots: at the top of macro-step
    // M the loads of M+1 may still be in flight (2 * DMA per thread), M's
    // have landed once every wave has waited for its own and passed the
    // barrier; then M+2's loads go into the slot M-1 used.  Macro-steps past
    // M1 still load (nothing valid) so the pending count stays exact.
    dma_macro(M0, 0);
    dma_macro(M0 + 1, 1);
    int slot = 0;
    for (int M = M0; M < M1; ++M) {
      stage_barrier<2 * DMA>();
      dma_macro(M + 2, slot == 0 ? 2 : slot - 1);
      compute(slot * KG + kg, M * KG + kg);
      slot = slot == 2 ? 0 : slot + 1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  __syncthreads();  // every group's steps are done; the ring is free
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) l_run[ct] = lacc[ct][0];
  const int need_w = (kv_end_w + bs_mask) >> bs_shift;
  const bool bad_w = *bad_first < need_w;

  // Merge the key groups into group 0 through LDS, [wave][float][lane].
  float* mbuf = reinterpret_cast<float*>(smem) + wc * Cfg::NF * 64 + lane;
#pragma unroll
  for (int k = 1; k < KG; ++k) {
    if (kg == k && wave_on) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        mbuf[(ct * (NN * 4 + 2)) * 64] = m_run[ct];
        mbuf[(ct * (NN * 4 + 2) + 1) * 64] = l_run[ct];
#pragma unroll
        for (int n = 0; n < NN; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) mbuf[(ct * (NN * 4 + 2) + 2 + 4 * n + r) * 64] = acc[ct][n][r];
      }
    }
    __syncthreads();
    if (kg == 0 && wave_on) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const float mo = mbuf[(ct * (NN * 4 + 2)) * 64];
        const float lo = mbuf[(ct * (NN * 4 + 2) + 1) * 64];
        const float m = fmaxf(m_run[ct], mo);
        const bool none = m == -INFINITY;
        const float a0 = none ? 0.f : fast_exp2(m_run[ct] - m);
        const float a1 = none ? 0.f : fast_exp2(mo - m);
        l_run[ct] = l_run[ct] * a0 + lo * a1;
        m_run[ct] = m;
#pragma unroll
        for (int n = 0; n < NN; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[ct][n][r] = acc[ct][n][r] * a0 + mbuf[(ct * (NN * 4 + 2) + 2 + 4 * n + r) * 64] * a1;
      }
    }
    __syncthreads();
  }

  bool bad_out = bad_w || plan_broken;
  if (nsplit_eff > 1) {
    // Split-K: park this split's state in its slot ([wave][float][lane], a
    // bad table entry as l = NaN), count the arrival, and let the last split
    // of the column block merge all slots in split order.
    const int pair = pair_base + static_cast<int>(kvh * ncb + cb);
    const int slot0 = slot_base + (kvh * static_cast<int>(ncb) + static_cast<int>(cb)) * nsplit;
    const __amdgpu_buffer_rsrc_t pr =
        __builtin_amdgcn_make_buffer_rsrc(p.pf_part, static_cast<short>(0), p.pf_part_bytes, kBufferWord3);
    // Slot layout [wave][ct][unit][lane] of 16-byte units: unit 0 is
    // (m, l, 0, 0), unit 1 + n is O^T tile n.  Units are stored whole (b128)
    // and read as runs of b32 loads, which the backend merges: storing single
    // vector elements with buffer stores miscompiles with ROCm 7.2's clang.
    auto uofs = [&](int sl, int ct, int u) {
      return sl * Cfg::SLOT_BYTES + (((wc * CT + ct) * (NN + 1) + u) * 64 + lane) * 16;
    };
    if (kg == 0 && wave_on) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const float lw = bad_out ? NAN : l_run[ct];
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{__builtin_bit_cast(uint32_t, m_run[ct]), __builtin_bit_cast(uint32_t, lw), 0u, 0u}, pr,
            uofs(slot0 + split, ct, 0), 0, kSc1);
#pragma unroll
        for (int n = 0; n < NN; ++n)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[ct][n]), pr,
                                                 uofs(slot0 + split, ct, 1 + n), 0, kSc1);
      }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial stores are acknowledged
    __syncthreads();
    int* s_last = bad_first;  // the table window is done with it
    if (tid == 0) {
      const unsigned prev = __hip_atomic_fetch_add(&p.pf_counters[pair], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *s_last = prev == static_cast<unsigned>(nsplit_eff - 1);
    }
    __syncthreads();
    if (!*s_last) return;
    if (kg == 0 && wave_on) {
      // Two passes over the slots, each with its loads independent of one
      // another: the common maximum, then the rescaled sums in split order.
      bad_out = false;
      float mx[CT];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) mx[ct] = -INFINITY;
#pragma unroll 8
      for (int k = 0; k < nsplit_eff; ++k)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) mx[ct] = fmaxf(mx[ct], ld_sc1(pr, uofs(slot0 + k, ct, 0)));
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        m_run[ct] = mx[ct];
        l_run[ct] = 0.f;
#pragma unroll
        for (int n = 0; n < NN; ++n) acc[ct][n] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll 2
      for (int k = 0; k < nsplit_eff; ++k) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const int o0 = uofs(slot0 + k, ct, 0);
          const float mk = ld_sc1(pr, o0);
          const float lk = ld_sc1(pr, o0 + 4);
          floatx4 ak[NN];
#pragma unroll
          for (int n = 0; n < NN; ++n) {
            const int on = uofs(slot0 + k, ct, 1 + n);
            ak[n] = floatx4{ld_sc1(pr, on), ld_sc1(pr, on + 4), ld_sc1(pr, on + 8), ld_sc1(pr, on + 12)};
          }
          // The slot units this lane read are its own (every split stored
          // them at the same wave, tile and lane): clear them for the next
          // call, whose workspace tail must be zero.
          __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, pr, o0, 0, kSc1);
#pragma unroll
          for (int n = 0; n < NN; ++n)
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, pr, uofs(slot0 + k, ct, 1 + n), 0, kSc1);
          bad_out |= lk != lk;
          const float a = mx[ct] == -INFINITY ? 0.f : fast_exp2(mk - mx[ct]);
          l_run[ct] += lk * a;
#pragma unroll
          for (int n = 0; n < NN; ++n) acc[ct][n] += ak[n] * a;
        }
      }
    }
    if (tid == 0) __hip_atomic_store(&p.pf_counters[pair], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if (kg != 0 || !wave_on) return;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const float lsum = group4_sum_swap(l_run[ct]);
    if (!cval[ct]) continue;
    const float inv = bad_out ? NAN : (lsum > 0.f ? 1.f / lsum : 0.f);
    T* orow_p = reinterpret_cast<T*>(p.out) + orow[ct];
#pragma unroll
    for (int n = 0; n < NN; ++n) {
      typename DT::vec4 v4;
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = static_cast<T>(acc[ct][n][r] * inv);
      *reinterpret_cast<u32x2*>(orow_p + 16 * n + 4 * g) = __builtin_bit_cast(u32x2, v4);
    }
  }
}

// --------------------------------------------------------------------------
// Host side.
// --------------------------------------------------------------------------
// 16-column tiles per prefill wave (columns per workgroup = 64 * kPrefillTiles).
constexpr int kPrefillTiles = 2;

// Decode launch shape: kDecodeWaves waves per workgroup, each with a ring of
// decode_ring<D> chunk slots (16 KiB of LDS per wave at head_dim 64, 32 KiB
// at 128).  Two chunks in flight per wave measured faster than three or
// four (c2 12.43 / 12.64 / 12.80 us per call): the fewer bytes each wave
// has queued, the sooner its first chunk lands and its compute overlaps
// the rest of the stream.
constexpr int kDecodeWaves = 4;
template <int D>
constexpr int decode_ring() { return 2; }

// Words of one decode split-K slot: G rows of D outputs, then G (max, sum)
// pairs, padded to 16 bytes.
int slot_words(int group, int head_dim) { return (group * head_dim + 2 * group + 3) / 4 * 4; }

struct WorkspaceLayout {
  size_t counters_off, pf_counters_off;  // arrival counters (zero between calls)
  size_t zero_off;                       // a page no call writes (zero since the workspace was cleared)
  size_t plan_off, plan_cap;             // the call's own decode plan, when the caller passes none
  size_t pf_part_off, pf_part_bytes;     // prefill split-K slots (zero between calls; 0 bytes: none)
  size_t part_off, part_bytes;           // decode split-K slots (hold the last call's partials)
  size_t total;
};

// Prefill split-K slots a workspace provides (one per split of a column
// block), and the bytes of one slot: a workgroup's per-lane softmax state.
constexpr int kPrefillSlots = 512;
size_t prefill_slot_bytes(int head_dim) {
  return head_dim == 64 ? PrefillCfg<64, kPrefillTiles>::SLOT_BYTES : PrefillCfg<128, kPrefillTiles>::SLOT_BYTES;
}
constexpr size_t kPrefillRegion =
    size_t{kPrefillSlots} * (PrefillCfg<64, kPrefillTiles>::SLOT_BYTES > PrefillCfg<128, kPrefillTiles>::SLOT_BYTES
                                 ? PrefillCfg<64, kPrefillTiles>::SLOT_BYTES
                                 : PrefillCfg<128, kPrefillTiles>::SLOT_BYTES);

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Everything but the decode split-K slots sits at the same offsets for every
// call: the arrival counters (decode pairs from 0, prefill pairs after
// kMaxDecodePairs), a zero page, the region the call's own decode plan is
// built in and, for calls with prefill rows, the prefill split-K slots
// (sized for the largest head_dim).  The counters and the prefill slots are
// zero between calls -- their protocols need that, and the workgroup that
// consumes a prefill slot clears it -- so a workspace reused by calls of
// other shapes never shows one call's data to another.  Decode slots come
// last and need no clearing: a merger reads only slots its own call's
// producers wrote and acknowledged before they arrived.
constexpr size_t kMaxDecodePairs = (size_t{1} << 20) - kPrefillSlots;
constexpr size_t kCounterBytes = (kMaxDecodePairs + kPrefillSlots) * sizeof(unsigned);
constexpr size_t kZeroPageBytes = 4096;  // read by decode lanes that have no token to load
constexpr size_t kPlanRegion = (size_t{4} << 20) - kZeroPageBytes;

WorkspaceLayout workspace_layout(int group, int head_dim, int64_t item_cap, bool with_prefill) {
  WorkspaceLayout l;
  l.counters_off = 0;
  l.pf_counters_off = kMaxDecodePairs * sizeof(unsigned);
  l.zero_off = kCounterBytes;
  l.plan_off = l.zero_off + kZeroPageBytes;
  l.plan_cap = kPlanRegion;
  l.pf_part_off = l.plan_off + l.plan_cap;
  l.pf_part_bytes = with_prefill ? kPrefillSlots * prefill_slot_bytes(head_dim) : 0;
  l.part_off = l.pf_part_off + kPrefillRegion;
  l.part_bytes = align_up(static_cast<size_t>(item_cap) * slot_words(group, head_dim) * 4, 256);
  l.total = align_up(l.part_off + l.part_bytes, 256);
  return l;
}

// Decode grid and plan capacity of a call: CUs x rounds workgroups loop over
// the plan's items, which never exceed kPlanCUs x rounds + num_seqs x Hkv.
struct DecodeShape {
  int rounds;
  int64_t item_cap;
  int cus, grid;
};

DecodeShape decode_shape(int num_seqs, int num_kv_heads, int64_t max_ctx, int head_dim, int device_cus) {
  DecodeShape d;
  d.rounds = plan_max_rounds(num_seqs, num_kv_heads, max_ctx, head_dim);
  d.item_cap = plan_item_cap(num_seqs, num_kv_heads, max_ctx, d.rounds);
  d.cus = device_cus < 1 ? 1 : (device_cus > kPlanCUs ? kPlanCUs : device_cus);
  d.grid = d.cus * d.rounds;
  return d;
}

size_t plan_bytes_needed(int64_t num_seqs, int64_t item_cap) { return plan_bytes(num_seqs, item_cap); }

int current_device_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess)
    return kPlanCUs;
  return n;
}

// CUs a decode plan is sized for.  The decode rows of a mixed batch run
// beside the prefill kernel (on the caller's aux stream), and a workgroup of
// either holds most of a CU's LDS, so their plan takes a quarter of the CUs
// and leaves the rest to the prefill column blocks.
int plan_cus(bool decode_only) {
  const int n = current_device_cus();
  if (decode_only) return n;
  const int q = n / 4;
  return q < 1 ? 1 : q;
}

DecodePlanArgs plan_args(void* plan, int64_t item_cap, const void* block_tables, int64_t bt_stride, int bt64,
                         int bs_shift, const void* seq_lens, int sl64, const void* qsl, int qsl64,
                         int is_decode_only, int num_seqs, int num_kv_heads, int64_t max_ctx, int head_dim,
                         const DecodeShape& d) {
  DecodePlanArgs a;
  a.plan = plan;
  a.item_cap = static_cast<uint32_t>(item_cap);
  a.block_tables = block_tables;
  a.bt_stride = bt_stride;
  a.bt64 = bt64 ? 1 : 0;
  a.bs_shift = bs_shift;
  a.tiles_per_step = 2;  // a 32-token chunk; the carried ids are wave w's tiles 0..7 either way
  a.seq_lens = seq_lens;
  a.sl64 = sl64 ? 1 : 0;
  a.qsl = qsl;
  a.qsl64 = qsl64 ? 1 : 0;
  a.decode_only = is_decode_only ? 1 : 0;
  a.num_seqs = num_seqs;
  a.num_kv_heads = num_kv_heads;
  a.max_ctx = max_ctx;
  a.cus = d.cus;
  a.rounds = d.rounds;
  a.min_tokens = plan_min_tokens(head_dim);
  a.round_tokens = plan_round_tokens(head_dim);
  a.long_tokens = plan_long_tokens(head_dim);
  return a;
}

int ilog2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((1 << s) < v) ++s;
  return s;
}

int64_t round_up_ctx(int max_seq_len, int block_size) {
  return (static_cast<int64_t>(max_seq_len) + block_size - 1) / block_size * block_size;
}


// The caller's secondary stream and fork/join events of a mixed batch
// (all three, or none).  The library owns none of them.
struct AuxStream {
  hipStream_t stream;
  hipEvent_t fork, join;
};

// Launch the decode kernel with `p` and, unless the batch is decode-only,
// the prefill kernel with `pp` (its own plan); `launch_decode` is false when
// the host query offsets show no one-row sequence.  A mixed batch with an aux
// stream runs its decode rows there, forked from and joined back to `stream`
// with the caller's events, so the memory-bound decode kernel overlaps the
// compute-bound prefill kernel; graph capture records the fork and join as
// ordinary cross-stream dependencies.  Without one the two launches run in
// order on `stream`.
// The decode rows: the plan kernel first when the call builds its own plan
// (`build` non-null), then the decode kernel over `grid` workgroups.
template <class DT, int D>
hipError_t launch_decode_rows(AttnParams& p, const DecodePlanArgs* build, int grid, hipStream_t stream) {
  if (build) {
    const hipError_t e = launch_decode_plan(*build, stream);
    if (e != hipSuccess) return e;
  }
  void* args[] = {&p};
  constexpr int W = kDecodeWaves, R = decode_ring<D>();
  // The block-table width is a template argument so table loads need no
  // per-lane branch.
  // Block size >= 16 (the item carries block ids) and the table's index
  // width select the kernel at compile time.
  const void* dk =
      p.inline_blocks
          ? (p.bt64 ? reinterpret_cast<const void*>(&paged_decode_kernel<DT, D, W, R, int64_t, true>)
                    : reinterpret_cast<const void*>(&paged_decode_kernel<DT, D, W, R, int32_t, true>))
          : (p.bt64 ? reinterpret_cast<const void*>(&paged_decode_kernel<DT, D, W, R, int64_t, false>)
                    : reinterpret_cast<const void*>(&paged_decode_kernel<DT, D, W, R, int32_t, false>));
  return hipLaunchKernel(dk, dim3(grid), dim3(W * 64), args, 0, stream);
}

// Launch the decode rows with `p` and, unless the batch is decode-only, the
// prefill kernel with `pp` (its own plan); `launch_decode` is false when the
// host query offsets show no one-row sequence.  A mixed batch with an aux
// stream runs its decode rows there, forked from and joined back to `stream`
// with the caller's events, so the memory-bound decode kernel overlaps the
// compute-bound prefill kernel; graph capture records the fork and join as
// ordinary cross-stream dependencies.  Without one the launches run in order
// on `stream`.
template <class DT, int D>
hipError_t launch_attention(AttnParams& p, PrefillParams& pp, const DecodePlanArgs* build, int decode_grid,
                            int pf_grid_x, bool launch_decode, int num_seqs, int max_query_len, hipStream_t stream,
                            const AuxStream* aux) {
  if (p.decode_only) return launch_decode_rows<DT, D>(p, build, decode_grid, stream);

  void* pargs[] = {&pp};
  using PCfg = PrefillCfg<D, kPrefillTiles>;
  const void* vk = pp.bt64 ? reinterpret_cast<const void*>(&paged_prefill_kernel<DT, D, kPrefillTiles, int64_t>)
                           : reinterpret_cast<const void*>(&paged_prefill_kernel<DT, D, kPrefillTiles, int32_t>);
  dim3 vgrid;
  if (pp.plan_n > 0) {
    vgrid = dim3(static_cast<unsigned>(pf_grid_x), static_cast<unsigned>(pp.plan_n), 1);
  } else {
    const int64_t cols = static_cast<int64_t>(max_query_len) * pp.group;
    const int64_t nblk = (cols + PCfg::COLS - 1) / PCfg::COLS;
    if (nblk > 0x7FFFFFFF) return hipErrorInvalidValue;
    vgrid = dim3(static_cast<unsigned>(nblk), pp.num_kv_heads, num_seqs);
  }
  if (!launch_decode) return hipLaunchKernel(vk, vgrid, dim3(PCfg::THREADS), pargs, 0, stream);

  if (!aux) {
    hipError_t e = launch_decode_rows<DT, D>(p, build, decode_grid, stream);
    if (e != hipSuccess) return e;
    return hipLaunchKernel(vk, vgrid, dim3(PCfg::THREADS), pargs, 0, stream);
  }
  hipError_t e = hipEventRecord(aux->fork, stream);
  if (e == hipSuccess) e = hipStreamWaitEvent(aux->stream, aux->fork, 0);
  if (e != hipSuccess) return e;
  // Once the aux stream depends on the caller's, it is joined back whatever
  // else fails (an unjoined fork would also break a graph capture).
  const hipError_t ed = launch_decode_rows<DT, D>(p, build, decode_grid, aux->stream);
  const hipError_t er = hipEventRecord(aux->join, aux->stream);
  const hipError_t ev = hipLaunchKernel(vk, vgrid, dim3(PCfg::THREADS), pargs, 0, stream);
  const hipError_t ej = er == hipSuccess ? hipStreamWaitEvent(stream, aux->join, 0) : er;
  return ed != hipSuccess ? ed : (ev != hipSuccess ? ev : ej);
}

bool aligned16(const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; }

int64_t host_index(const void* a, int is64, int64_t i) {
  return is64 ? static_cast<const int64_t*>(a)[i] : static_cast<const int32_t*>(a)[i];
}

// Fill pp.plan with the prefill schedule from host query offsets and lengths:
// every sequence with more than one query row, heaviest first, three entries
// each (s | (nsplit - 1) << 16 | split_macro << 22; slot_base | pair_base << 16;
// ql).  A column block's key range is cut into splits of split_macro
// macro-steps so that no workgroup carries more than about twice an even
// share of the batch's work over the 256 CUs (a long context behind a short
// chunk); splits need partial slots, so the share doubles until the slots
// fit.  Returns the sequences listed (0: no plan, the launch then uses the
// full grid without splits) and the grid width.
int build_prefill_plan(PrefillParams& pp, const void* lens, int lens64, const void* qsl, int qsl64, int num_seqs,
                       int cols_per_wg, int macro_keys, int& grid_x) {
  constexpr int kCUs = 256, kMinSplitMacro = 4, kMaxListed = kPlanMax / 3;
  struct Seq {
    int s, ncb;
    int64_t ql, nm_max, work;
  };
  std::vector<Seq> seqs;
  int64_t total = 0;
  for (int i = 0; i < num_seqs; ++i) {
    const int64_t ql = host_index(qsl, qsl64, i + 1) - host_index(qsl, qsl64, i);
    if (ql <= 1) continue;
    int64_t L = host_index(lens, lens64, i);
    L = L < 0 ? 0 : (L < pp.max_ctx ? L : pp.max_ctx);
    const int64_t ncols = ql * pp.group;
    const int64_t ncb = (ncols + cols_per_wg - 1) / cols_per_wg;
    if (ncb > 0x7FFF) return 0;
    Seq q{i, static_cast<int>(ncb), ql, 0, 0};
    for (int64_t cb = 0; cb < ncb; ++cb) {
      const int64_t c_last = (ncols < (cb + 1) * cols_per_wg ? ncols : (cb + 1) * cols_per_wg) - 1;
      int64_t kv_end = L - ql + c_last / pp.group + 1;
      kv_end = kv_end < 0 ? 0 : (kv_end < L ? kv_end : L);
      const int64_t nm = (kv_end + macro_keys - 1) / macro_keys;
      q.work += nm * pp.num_kv_heads;
      q.nm_max = nm > q.nm_max ? nm : q.nm_max;
    }
    total += q.work;
    seqs.push_back(q);
  }
  if (seqs.empty() || static_cast<int>(seqs.size()) > kMaxListed) return 0;
  std::stable_sort(seqs.begin(), seqs.end(), [](const Seq& a, const Seq& b) { return a.nm_max > b.nm_max; });
  // A workgroup holds a whole CU, so once the column blocks alone fill the
  // CUs, splits only add merges: split what is longer than twice the even
  // share.
  int64_t share = 2 * ((total + kCUs - 1) / kCUs);
  share = share < kMinSplitMacro ? kMinSplitMacro : share;
  for (;; share *= 2) {
    int64_t slots = 0, pairs = 0, gx = 0;
    bool fits = true;
    for (size_t k = 0; k < seqs.size(); ++k) {
      const Seq& q = seqs[k];
      int64_t nsplit = (q.nm_max + share - 1) / share;
      nsplit = nsplit < 1 ? 1 : (nsplit > 64 ? 64 : nsplit);
      int64_t split_mk = (q.nm_max + nsplit - 1) / nsplit;
      if (split_mk > 1023) {
        nsplit = 1;
        split_mk = 0;
      }
      const int64_t items = static_cast<int64_t>(pp.num_kv_heads) * q.ncb * nsplit;
      if (nsplit > 1) {
        if (slots + items > kPrefillSlots || slots > 0xFFFF || pairs > 0xFFFF) {
          fits = false;
          break;
        }
      }
      pp.plan[3 * k] = static_cast<uint32_t>(q.s) | static_cast<uint32_t>(nsplit - 1) << 16 |
                       static_cast<uint32_t>(split_mk) << 22;
      pp.plan[3 * k + 1] = static_cast<uint32_t>(slots) | static_cast<uint32_t>(pairs) << 16;
      pp.plan[3 * k + 2] = static_cast<uint32_t>(q.ql);
      if (nsplit > 1) {
        slots += items;
        pairs += static_cast<int64_t>(pp.num_kv_heads) * q.ncb;
      }
      gx = items > gx ? items : gx;
    }
    if (fits) {
      if (gx > 0x7FFFFFFF) return 0;
      grid_x = static_cast<int>(gx);
      return static_cast<int>(seqs.size());
    }
  }
}

}  // namespace
}  // namespace ns

extern "C" const char* ns_error_string(int code) {
  switch (code) {
    case NS_OK: return "ok";
    case NS_ERR_INVALID_ARG: return "invalid argument";
    case NS_ERR_UNSUPPORTED: return "unsupported shape or dtype";
    case NS_ERR_WORKSPACE: return "workspace missing or too small";
    case NS_ERR_HIP: return "HIP launch failed";
    default: return "unknown status";
  }
}

extern "C" int ns_version(void) { return 200; }

extern "C" size_t ns_paged_attention_workspace_size(int num_seqs, int num_heads, int num_kv_heads,
                                                    int head_dim, int block_size,
                                                    int max_seq_len, int max_query_len,
                                                    int64_t num_tokens, int is_decode_only) {
  (void)max_query_len;
  (void)num_tokens;
  if (num_seqs <= 0 || num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads ||
      block_size <= 0 || max_seq_len < 0 || head_dim <= 0)
    return 0;
  // The generic kernel (float32, other head sizes or block sizes, wide
  // groups) uses no workspace; a token size keeps the buffer non-empty.
  if (ns::generic_attention_takes(0, head_dim, block_size, num_heads / num_kv_heads))
    return head_dim <= ns::kGenericMaxHeadDim ? 256 : 0;
  const ns::DecodeShape d =
      ns::decode_shape(num_seqs, num_kv_heads, ns::round_up_ctx(max_seq_len, block_size), head_dim, ns::kPlanCUs);
  return ns::workspace_layout(num_heads / num_kv_heads, head_dim, d.item_cap, !is_decode_only).total;
}

extern "C" size_t ns_paged_decode_plan_size(int num_seqs, int num_kv_heads, int head_dim, int block_size,
                                            int max_seq_len) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || block_size <= 0 || max_seq_len < 0 ||
      (head_dim != 64 && head_dim != 128))
    return 0;
  const ns::DecodeShape d =
      ns::decode_shape(num_seqs, num_kv_heads, ns::round_up_ctx(max_seq_len, block_size), head_dim, ns::kPlanCUs);
  return ns::align_up(ns::plan_bytes(num_seqs, d.item_cap), 256);
}

extern "C" int ns_paged_decode_plan(void* plan, size_t plan_bytes, const void* block_tables,
                                    int64_t block_table_stride, int64_t block_table_width, int block_tables_is_int64,
                                    const void* seq_lens, int seq_lens_is_int64, const void* query_start_loc,
                                    int query_start_loc_is_int64, int num_seqs, int is_decode_only,
                                    int num_kv_heads, int head_dim, int block_size, int max_seq_len, void* stream) {
  using namespace ns;
  if (num_seqs < 0) return NS_ERR_INVALID_ARG;
  if (num_seqs == 0) return NS_OK;
  if (!plan || !block_tables || !seq_lens || (!is_decode_only && !query_start_loc)) return NS_ERR_INVALID_ARG;
  if (num_kv_heads <= 0 || max_seq_len < 0 || block_table_width <= 0 || block_table_stride < block_table_width)
    return NS_ERR_INVALID_ARG;
  if (head_dim != 64 && head_dim != 128) return NS_ERR_UNSUPPORTED;
  const int bs_shift = ilog2_exact(block_size);
  if (bs_shift < 0) return NS_ERR_UNSUPPORTED;
  if (num_seqs > 65535 || num_kv_heads > 65535) return NS_ERR_UNSUPPORTED;
  if (reinterpret_cast<uintptr_t>(plan) % 16 != 0) return NS_ERR_INVALID_ARG;
  const int64_t ctx_plan = round_up_ctx(max_seq_len, block_size);
  const int64_t table_tokens = block_table_width * static_cast<int64_t>(block_size);
  const int64_t max_ctx = ctx_plan < table_tokens ? ctx_plan : table_tokens;
  DecodeShape d = decode_shape(num_seqs, num_kv_heads, max_ctx, head_dim, kPlanCUs);
  if (plan_bytes < plan_bytes_needed(num_seqs, d.item_cap)) return NS_ERR_WORKSPACE;
  d = decode_shape(num_seqs, num_kv_heads, max_ctx, head_dim, plan_cus(is_decode_only != 0));
  const DecodePlanArgs a = plan_args(plan, d.item_cap, block_tables, block_table_stride, block_tables_is_int64,
                                     bs_shift, seq_lens, seq_lens_is_int64, query_start_loc,
                                     query_start_loc_is_int64, is_decode_only, num_seqs, num_kv_heads, max_ctx,
                                     head_dim, d);
  return launch_decode_plan(a, static_cast<hipStream_t>(stream)) == hipSuccess ? NS_OK : NS_ERR_HIP;
}

namespace ns {
namespace {

// Scratch of ns_paged_attention_noalloc: the workspace of calls whose caller
// cannot allocate one.  A file-scope device array, so each device the library
// runs on holds its own copy from module load (zero-filled by the loader)
// until the process ends.  In host code `g_noalloc_scratch` names a host-side
// stand-in, never the device memory: kernels and fills get the address that
// hipGetSymbolAddress returns for the current device, kept per device.
constexpr size_t kNoallocScratchBytes = size_t{128} << 20;
__device__ __align__(256) unsigned char g_noalloc_scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kMaxDevices];

__global__ __launch_bounds__(256) void zero_fill_kernel(u32x4* dst, size_t n16) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n16;
       i += static_cast<size_t>(gridDim.x) * 256)
    dst[i] = u32x4{0u, 0u, 0u, 0u};
}

// The scratch address on the current device, looked up (and, outside graph
// capture, cleared with a fill kernel on `stream`) on the device's first call.
// Returns nullptr if the lookup fails.
void* noalloc_scratch(hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (g_noalloc_ptr[dev]) return g_noalloc_ptr[dev];
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_noalloc_scratch)) != hipSuccess || !ptr) return nullptr;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) {
    // The loader already zero-fills the array; clearing it once more in
    // stream order costs one launch and makes no assumption about that.
    u32x4* dst = static_cast<u32x4*>(ptr);
    size_t n16 = kNoallocScratchBytes / 16;
    void* args[] = {&dst, &n16};
    if (hipLaunchKernel(reinterpret_cast<const void*>(&zero_fill_kernel), dim3(1024), dim3(256), args, 0,
                        stream) != hipSuccess)
      return nullptr;
  }
  g_noalloc_ptr[dev] = ptr;
  return ptr;
}

int paged_attention_entry(void* out, const void* query, const void* k_cache, const void* v_cache,
                          const void* block_tables, int64_t block_table_stride, int64_t block_table_width,
                          int block_tables_is_int64, const void* seq_lens, int seq_lens_is_int64,
                          const void* query_start_loc, int query_start_loc_is_int64,
                          const void* seq_lens_host, int seq_lens_host_is_int64,
                          const void* query_start_loc_host, int query_start_loc_host_is_int64,
                          int num_seqs, int64_t num_tokens, int max_query_len, int max_seq_len,
                          int is_decode_only, int num_heads, int num_kv_heads, int head_dim,
                          int block_size, int64_t num_blocks, float scale, int dtype,
                          const void* decode_plan, size_t decode_plan_bytes,
                          void* workspace, size_t workspace_bytes, bool noalloc, void* stream,
                          void* aux_stream, void* fork_event, void* join_event) {
  if (num_seqs < 0 || num_tokens < 0) return NS_ERR_INVALID_ARG;
  if (num_seqs == 0 || num_tokens == 0) return NS_OK;
  if (!out || !query || !k_cache || !v_cache || !block_tables || !seq_lens) return NS_ERR_INVALID_ARG;
  if (!is_decode_only && !query_start_loc) return NS_ERR_INVALID_ARG;
  if (is_decode_only && num_tokens != num_seqs) return NS_ERR_INVALID_ARG;
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads) return NS_ERR_INVALID_ARG;
  if (num_blocks <= 0 || block_table_width <= 0 || block_table_stride < block_table_width)
    return NS_ERR_INVALID_ARG;
  // The prefill kernel keeps block ids and key positions as 32-bit values.
  if (!is_decode_only && num_blocks > 0x7FFFFFFF) return NS_ERR_UNSUPPORTED;
  if (!is_decode_only && static_cast<int64_t>(max_seq_len) + block_size > 0x7FFFFFFF) return NS_ERR_UNSUPPORTED;
  if (max_seq_len < 0 || max_query_len < 0) return NS_ERR_INVALID_ARG;
  if (!(scale == scale)) return NS_ERR_INVALID_ARG;
  if (block_size <= 0 || head_dim <= 0) return NS_ERR_INVALID_ARG;
  if (dtype != NS_DTYPE_F32 && dtype != NS_DTYPE_F16 && dtype != NS_DTYPE_BF16) return NS_ERR_UNSUPPORTED;
  const int group = num_heads / num_kv_heads;
  if (generic_attention_takes(dtype == NS_DTYPE_F32, head_dim, block_size, group)) {
    // Shapes outside the MFMA kernels: the generic kernel, which needs no
    // workspace, plan or second stream (those arguments are not read).
    if (head_dim > kGenericMaxHeadDim || num_heads > 65535 || num_tokens > 0x7FFFFFFF) return NS_ERR_UNSUPPORTED;
    const size_t esz = dtype == NS_DTYPE_F32 ? 4 : 2;
    for (const void* a : {static_cast<const void*>(out), query, k_cache, v_cache})
      if (reinterpret_cast<uintptr_t>(a) % esz != 0) return NS_ERR_INVALID_ARG;
    GenericAttnParams g{};
    g.out = out;
    g.query = query;
    g.k_cache = k_cache;
    g.v_cache = v_cache;
    g.bt = block_tables;
    g.bt_stride = block_table_stride;
    g.seq_lens = seq_lens;
    g.qsl = query_start_loc;
    g.bt64 = block_tables_is_int64 ? 1 : 0;
    g.sl64 = seq_lens_is_int64 ? 1 : 0;
    g.qsl64 = query_start_loc_is_int64 ? 1 : 0;
    g.decode_only = is_decode_only ? 1 : 0;
    g.num_seqs = num_seqs;
    g.num_heads = num_heads;
    g.num_kv_heads = num_kv_heads;
    g.head_dim = head_dim;
    g.block_size = block_size;
    g.num_tokens = num_tokens;
    g.num_blocks = num_blocks;
    const int64_t ctx = round_up_ctx(max_seq_len, block_size), table = block_table_width * block_size;
    g.max_ctx = ctx < table ? ctx : table;
    g.scale = scale;
    return launch_generic_attention(g, dtype, static_cast<hipStream_t>(stream)) == hipSuccess ? NS_OK
                                                                                             : NS_ERR_HIP;
  }
  const int bs_shift = ilog2_exact(block_size);
  if (num_seqs > 65535 || num_kv_heads > 65535) return NS_ERR_UNSUPPORTED;
  if (!aligned16(out) || !aligned16(query) || !aligned16(k_cache) || !aligned16(v_cache))
    return NS_ERR_INVALID_ARG;
  // The aux stream comes with both events or not at all.
  const int aux_given = (aux_stream != nullptr) + (fork_event != nullptr) + (join_event != nullptr);
  if (aux_given != 0 && aux_given != 3) return NS_ERR_INVALID_ARG;
  if (aux_given && aux_stream == stream) return NS_ERR_INVALID_ARG;
  const AuxStream aux{static_cast<hipStream_t>(aux_stream), static_cast<hipEvent_t>(fork_event),
                      static_cast<hipEvent_t>(join_event)};

  const int64_t ctx_plan = round_up_ctx(max_seq_len, block_size);
  const int64_t table_tokens = block_table_width * static_cast<int64_t>(block_size);
  const int64_t max_ctx = ctx_plan < table_tokens ? ctx_plan : table_tokens;
  // Sizes first (they do not depend on the device); the device's CU count,
  // which only shapes the grid, is queried once every check has passed.
  DecodeShape dshape = decode_shape(num_seqs, num_kv_heads, max_ctx, head_dim, kPlanCUs);
  const WorkspaceLayout wl = workspace_layout(group, head_dim, dshape.item_cap, !is_decode_only);
  if (static_cast<size_t>(num_seqs) * num_kv_heads > kMaxDecodePairs) return NS_ERR_UNSUPPORTED;
  // Partials are addressed through buffer descriptors with 32-bit offsets.
  if (wl.part_bytes > 0x7FFFFFFFu || wl.pf_part_bytes > 0x7FFFFFFFu) return NS_ERR_UNSUPPORTED;
  if (decode_plan) {
    if (reinterpret_cast<uintptr_t>(decode_plan) % 16 != 0) return NS_ERR_INVALID_ARG;
    if (decode_plan_bytes < plan_bytes_needed(num_seqs, dshape.item_cap)) return NS_ERR_INVALID_ARG;
  } else if (plan_bytes_needed(num_seqs, dshape.item_cap) > wl.plan_cap) {
    return NS_ERR_UNSUPPORTED;  // too many pairs for the workspace's plan region: pass a plan
  }
  if (noalloc) {
    // Shapes whose workspace exceeds the scratch are refused before any HIP call.
    if (wl.total > kNoallocScratchBytes) return NS_ERR_WORKSPACE;
    workspace = noalloc_scratch(static_cast<hipStream_t>(stream));
    if (!workspace) return NS_ERR_HIP;
    workspace_bytes = kNoallocScratchBytes;
  }
  if (!workspace || workspace_bytes < wl.total) return NS_ERR_WORKSPACE;
  dshape = decode_shape(num_seqs, num_kv_heads, max_ctx, head_dim, plan_cus(is_decode_only != 0));

  AttnParams p;
  p.out = static_cast<char*>(out);
  p.query = static_cast<const char*>(query);
  p.k_cache = static_cast<const char*>(k_cache);
  p.v_cache = static_cast<const char*>(v_cache);
  p.bt = block_tables;
  p.bt_stride = block_table_stride;
  p.seq_lens = seq_lens;
  p.qsl = query_start_loc;
  p.bt64 = block_tables_is_int64 ? 1 : 0;
  p.sl64 = seq_lens_is_int64 ? 1 : 0;
  p.qsl64 = query_start_loc_is_int64 ? 1 : 0;
  p.decode_only = is_decode_only ? 1 : 0;
  p.num_seqs = num_seqs;
  p.num_tokens = num_tokens;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.group = group;
  p.bs_shift = bs_shift;
  p.num_blocks = num_blocks;
  p.max_ctx = max_ctx;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.skip_decode_rows = 1;
  char* ws = static_cast<char*>(workspace);
  char* plan_base = decode_plan ? static_cast<char*>(const_cast<void*>(decode_plan)) : ws + wl.plan_off;
  p.plan_hdr = reinterpret_cast<const DecodePlanHeader*>(plan_base);
  p.items = reinterpret_cast<const DecodeItem*>(plan_base + sizeof(DecodePlanHeader));
  p.item_cap = dshape.item_cap;
  p.inline_blocks = bs_shift >= 4 ? 1 : 0;
  p.zeros = static_cast<char*>(workspace) + wl.zero_off;
  p.part = reinterpret_cast<uint32_t*>(ws + wl.part_off);
  p.part_bytes = static_cast<int>(wl.part_bytes);
  p.slot_words = slot_words(group, head_dim);
  p.counters = reinterpret_cast<unsigned*>(ws + wl.counters_off);
  p.pf_counters = reinterpret_cast<unsigned*>(ws + wl.pf_counters_off);
  p.pf_part = reinterpret_cast<float*>(ws + wl.pf_part_off);
  p.pf_part_bytes = static_cast<int>(wl.pf_part_bytes);
  p.plan_n = 0;
  // The decode plan is built on the device (in the workspace's plan region)
  // unless the caller passes one built for this metadata.
  DecodePlanArgs build_args;
  const DecodePlanArgs* build = nullptr;
  if (!decode_plan) {
    build_args = plan_args(plan_base, dshape.item_cap, block_tables, block_table_stride, block_tables_is_int64,
                           bs_shift, seq_lens, seq_lens_is_int64, query_start_loc, query_start_loc_is_int64,
                           is_decode_only, num_seqs, num_kv_heads, max_ctx, head_dim, dshape);
    build = &build_args;
  }
  // With host query offsets, a batch without one-row sequences launches no decode rows.
  const void* qsl_host = is_decode_only ? nullptr : query_start_loc_host;
  bool launch_decode = true;
  if (qsl_host && seq_lens_host) {
    launch_decode = false;
    for (int i = 0; i < num_seqs && !launch_decode; ++i)
      launch_decode = host_index(qsl_host, query_start_loc_host_is_int64, i + 1) -
                          host_index(qsl_host, query_start_loc_host_is_int64, i) == 1;
  }
  // Prefill plan (split-K over the CUs) from host offsets and lengths.
  PrefillParams pp;
  int pf_grid_x = 0;
  if (!is_decode_only) {
    static_cast<AttnParams&>(pp) = p;
    pp.plan_n = 0;
    if (seq_lens_host && qsl_host) {
      const int mkeys = head_dim == 64 ? PrefillCfg<64, kPrefillTiles>::KG * PrefillCfg<64, kPrefillTiles>::KT
                                       : PrefillCfg<128, kPrefillTiles>::KG * PrefillCfg<128, kPrefillTiles>::KT;
      pp.plan_n = build_prefill_plan(pp, seq_lens_host, seq_lens_host_is_int64, qsl_host,
                                     query_start_loc_host_is_int64, num_seqs, PrefillCfg<64, kPrefillTiles>::COLS,
                                     mkeys, pf_grid_x);
    }
  }

  hipStream_t st = static_cast<hipStream_t>(stream);
  const AuxStream* ax = aux_given ? &aux : nullptr;
  const int dg = dshape.grid;
  hipError_t e;
  if (dtype == NS_DTYPE_F16)
    e = head_dim == 64
            ? launch_attention<F16, 64>(p, pp, build, dg, pf_grid_x, launch_decode, num_seqs, max_query_len, st, ax)
            : launch_attention<F16, 128>(p, pp, build, dg, pf_grid_x, launch_decode, num_seqs, max_query_len, st, ax);
  else
    e = head_dim == 64
            ? launch_attention<BF16, 64>(p, pp, build, dg, pf_grid_x, launch_decode, num_seqs, max_query_len, st, ax)
            : launch_attention<BF16, 128>(p, pp, build, dg, pf_grid_x, launch_decode, num_seqs, max_query_len, st,
                                          ax);
  return e == hipSuccess ? NS_OK : NS_ERR_HIP;
}

}  // namespace
}  // namespace ns

extern "C" int ns_paged_attention(void* out, const void* query,
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
                                  void* aux_stream, void* fork_event, void* join_event) {
  return ns::paged_attention_entry(out, query, k_cache, v_cache, block_tables, block_table_stride,
                                   block_table_width, block_tables_is_int64, seq_lens, seq_lens_is_int64,
                                   query_start_loc, query_start_loc_is_int64, seq_lens_host,
                                   seq_lens_host_is_int64, query_start_loc_host, query_start_loc_host_is_int64,
                                   num_seqs, num_tokens, max_query_len, max_seq_len, is_decode_only, num_heads,
                                   num_kv_heads, head_dim, block_size, num_blocks, scale, dtype, decode_plan,
                                   decode_plan_bytes, workspace, workspace_bytes, false, stream, aux_stream,
                                   fork_event, join_event);
}

extern "C" int ns_paged_attention_noalloc(void* out, const void* query,
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
                                          void* aux_stream, void* fork_event, void* join_event) {
  return ns::paged_attention_entry(out, query, k_cache, v_cache, block_tables, block_table_stride,
                                   block_table_width, block_tables_is_int64, seq_lens, seq_lens_is_int64,
                                   query_start_loc, query_start_loc_is_int64, seq_lens_host,
                                   seq_lens_host_is_int64, query_start_loc_host, query_start_loc_host_is_int64,
                                   num_seqs, num_tokens, max_query_len, max_seq_len, is_decode_only, num_heads,
                                   num_kv_heads, head_dim, block_size, num_blocks, scale, dtype, decode_plan,
                                   decode_plan_bytes, nullptr, 0, true, stream, aux_stream, fork_event,
                                   join_event);
}
