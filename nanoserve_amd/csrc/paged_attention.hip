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

// --------------------------------------------------------------------------
// Decode: one workgroup of W waves per plan item (a token range of one
// (sequence, kv head) pair); the grid loops over the plan's items.
// --------------------------------------------------------------------------
template <int D, int W, int CH_>
struct DecodeCfg {
  static constexpr int kThreads = W * 64;
  static constexpr int CH = CH_;                // tokens per wave per step
  static constexpr int NT = CH / 16;            // 16-token MFMA tiles per step
  static constexpr int NC = D / 32;             // k-chunks of the QK^T contraction
  static constexpr int NN = D / 16;             // 16-dim tiles of the output
  static constexpr int VT_LD = CH + 4;          // padded row of the transposed V tile
  static constexpr int LDS_V = W * D * VT_LD * 2;
  static constexpr int RED_LD = D + 4;             // padded row of the cross-wave reduce
  static constexpr int LDS_RED = (W * 16 * RED_LD + 2 * W * 16) * 4;
  static constexpr int LDS = LDS_V > LDS_RED ? LDS_V : LDS_RED;
  static_assert(NT % 2 == 0, "P^T operand pairs two 16-token tiles");
};

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
// dealt out evenly, each wave a contiguous run walked CH tokens per step with
// the next step's K/V loads (and the step after's table entries) in flight.
// A wave's share of an item's carried block ids: steps IS of NT tiles.
template <int W, int CH>
struct WaveBlocks {
  static constexpr int NT = CH / 16;
  static constexpr int IS = kItemBlocks / (W * NT);
  static constexpr int N = IS * NT;
  static_assert(N == 8, "two 16-byte rows per wave");
  int32_t id[N];
};

// The item rows and this wave's carried block ids of plan item idx (uniform
// per wave, so they come through the scalar cache, outside the vector-memory
// order the K/V loads keep).
template <int W, int CH>
__device__ __forceinline__ void load_item(const AttnParams& p, uint32_t idx, u32x4& r0, u32x4& r1,
                                          WaveBlocks<W, CH>& wb) {
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

template <class DT, int D, int W, int CH, class BTI, bool BIG>
__device__ __forceinline__ void decode_item(const AttnParams& p, uint32_t idx, u32x4 r0, u32x4 r1,
                                            const WaveBlocks<W, CH>& ib, char* smem, int64_t* later_lds,
                                            int& s_merger) {
  using Cfg = DecodeCfg<D, W, CH>;
  using T = typename DT::T;
  using V8 = typename DT::vec8;
  constexpr int THREADS = Cfg::kThreads;
  constexpr int NT = Cfg::NT, NC = Cfg::NC, NN = Cfg::NN, VT_LD = Cfg::VT_LD;
  constexpr int IS = WaveBlocks<W, CH>::IS;
  static_assert(W == kItemWaves, "items carry the block ids of kItemWaves waves");

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

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
  const int64_t pair = static_cast<int64_t>(s) * Hkv + kvh;

  const int bs_mask = (1 << p.bs_shift) - 1;
  const int64_t bt_row = static_cast<int64_t>(s) * p.bt_stride;
  const int64_t tiles = (t1 - t0 + 15) >> 4;
  const int64_t per_wave = (tiles + W - 1) / W * 16;
  const int64_t wb = t0 + w * per_wave;
  const int64_t we = t1 < wb + per_wave ? t1 : wb + per_wave;  // wave w's tokens: [wb, we)

  V8 qop[NC];
  {
    const int hq = c16 < G ? c16 : G - 1;  // in-row address for the padding columns
    const T* qrow = reinterpret_cast<const T*>(p.query) +
                    (qtok * p.num_heads + static_cast<int64_t>(kvh) * G + hq) * D;
#pragma unroll
    for (int c = 0; c < NC; ++c) qop[c] = load16<DT>(qrow + 32 * c + 8 * g);
    if (c16 >= G)
#pragma unroll
      for (int c = 0; c < NC; ++c) qop[c] = zero8<DT>();
  }
  T* out_row = reinterpret_cast<T*>(p.out) + (qtok * p.num_heads + static_cast<int64_t>(kvh) * G) * D;

  T* vt = reinterpret_cast<T*>(smem) + w * D * VT_LD;  // this wave's V^T tile [D][VT_LD]
  int bad = 0;
  float m_run = -INFINITY, l_run = 0.f;
  floatx4 acc[NN];
#pragma unroll
  for (int n = 0; n < NN; ++n) acc[n] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int64_t slot_stride = static_cast<int64_t>(Hkv) * D;  // elements between slots
  const T* kbase = reinterpret_cast<const T*>(p.k_cache) + static_cast<int64_t>(kvh) * D + 8 * g;
  const T* vbase = reinterpret_cast<const T*>(p.v_cache) + static_cast<int64_t>(kvh) * D + 8 * g;
  const T* zbase = reinterpret_cast<const T*>(p.zeros) + 8 * g;  // a never-written zero page

  // Issue the K/V loads of the step starting at token tb.  Lanes past the
  // wave's range or with an invalid block id read the zero page, so their V
  // contributes nothing (their scores are masked) and nothing here or later
  // waits on the data to fix it up.
  auto issue_step = [&](int64_t tb, const int64_t (&bk)[NT], V8 (&kx)[NT][NC], V8 (&vx)[NT][NC]) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int64_t t = tb + 16 * j + c16;
      bool valid = t < we;
      if (valid && (bk[j] < 0 || bk[j] >= p.num_blocks)) {
        bad = 1;
        valid = false;
      }
      const int64_t off = ((bk[j] << p.bs_shift) + (t & bs_mask)) * slot_stride;
      const T* kp = valid ? kbase + off : zbase;
      const T* vp = valid ? vbase + off : zbase;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        kx[j][c] = load16<DT>(kp + 32 * c);
        vx[j][c] = load16<DT>(vp + 32 * c);
      }
    }
  };

  // Where the block ids of every step come from.  BIG (block size >= 16: a
  // tile lies in one block): the item carries those of the wave's first IS
  // steps, and the ids of its later tiles come in one vector load (lane l:
  // tile IS * NT + l) issued before any K/V load and staged in LDS, so the
  // step loop reads them with LDS loads.  Vector-memory loads return in
  // order, and this way no K/V load waits for another step's data.  (The
  // plan caps an item at 4096 tokens, which keeps a wave within IS * NT + 64
  // tiles.)  Smaller blocks: per-lane block-table entries per step, clamped
  // into the wave's range.
  const int64_t nsteps = wb < we ? (we - wb + CH - 1) / CH : 0;
  // Loads in the BIG kernel are unconditional (clamped addresses, or the
  // zero page), so the compiler can count them exactly: a wait for one step's
  // data never turns into a wait for everything in flight.
  int64_t later_ids = 0;
  if constexpr (BIG) {
    int64_t t = wb + 16 * (IS * NT + lane);
    t = t < we ? t : we - 1;
    t = t > 0 ? t : 0;
    later_ids = ld_idx<BTI>(p.bt, bt_row + (t >> p.bs_shift));
  }
  int64_t* my_later = later_lds + w * 64;
  auto step_blocks = [&](int64_t st, int64_t (&bk)[NT]) {
    if constexpr (BIG) {
      if (st < IS) {
#pragma unroll
        for (int q = 0; q < IS; ++q)
          if (q == st)
#pragma unroll
            for (int j = 0; j < NT; ++j) bk[j] = ib.id[q * NT + j];
      } else {
        const int64_t* src = my_later + (st - IS) * NT;
#pragma unroll
        for (int j = 0; j < NT; ++j) bk[j] = src[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        int64_t t = wb + st * CH + 16 * j + c16;
        t = t < we ? t : we - 1;
        t = t > 0 ? t : 0;
        bk[j] = ld_idx<BTI>(p.bt, bt_row + (t >> p.bs_shift));
      }
    }
  };

  // Software pipeline over the wave's steps: step st + 1's K/V loads are in
  // flight while step st computes.
  V8 kr[NT][NC], vr[NT][NC];
  if (BIG || nsteps > 0) {
    int64_t bk[NT];
    step_blocks(0, bk);
    issue_step(wb, bk, kr, vr);
  }
  if constexpr (BIG) {
    my_later[lane] = later_ids;  // waits for the id load only: it went out before the K/V loads
    wave_lds_sync();
  }
  for (int64_t st = 0; st < nsteps; ++st) {
    const int64_t tb = wb + st * CH;
    const bool has_next = st + 1 < nsteps;
    V8 kn[NT][NC], vn[NT][NC];
    if (BIG || has_next) {
      // (BIG: past the wave's last step every lane reads the zero page.)
      int64_t bk[NT];
      step_blocks(has_next ? st + 1 : st, bk);
      issue_step(tb + CH, bk, kn, vn);
    }
    // Scheduling boundary: the next step's loads are issued before anything
    // below uses (and so waits for) this step's K/V registers.  The empty asm
    // takes them as in/out operands, so nothing that reads them can be
    // hoisted above it, and its memory clobber keeps the loads above it.
    asm volatile("" ::: "memory");
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int c = 0; c < NC; ++c) asm volatile("" : "+v"(kr[j][c]), "+v"(vr[j][c]));
    // Stage V transposed (vt[dim][token]) for the PV operand.
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) vt[(32 * c + 8 * g + e) * VT_LD + 16 * j + c16] = vr[j][c][e];

    // S^T = K Q^T: sacc[j][r] = score of token tb + 16j + 4g + r, head c16.
    floatx4 sacc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      sacc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) sacc[j] = mfma16x16x32(DT{}, kr[j][c], qop[c], sacc[j]);
    }
    float sv[NT][4];
    float mloc = -INFINITY;
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t t = tb + 16 * j + 4 * g + r;
        const float x = t < we ? sacc[j][r] * p.scale_log2 : -INFINITY;
        sv[j][r] = x;
        mloc = fmaxf(mloc, x);
      }
    mloc = group4_max(mloc);
    const float m_new = fmaxf(m_run, mloc);
    const bool none = m_new == -INFINITY;
    const float alpha = none ? 1.f : fast_exp2(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pr = none ? 0.f : fast_exp2(sv[j][r] - m_new);
        sv[j][r] = pr;
        psum += pr;
      }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int n = 0; n < NN; ++n) acc[n] *= alpha;
    m_run = m_new;

    wave_lds_sync();
    // O^T += V^T P^T over 32-token pairs: k-slot e of group g is token 4g+e of
    // the even tile (e < 4) or of the odd tile (e >= 4).
#pragma unroll
    for (int pb = 0; pb < NT / 2; ++pb) {
      V8 pt;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pt[e] = static_cast<T>(sv[2 * pb][e]);
        pt[4 + e] = static_cast<T>(sv[2 * pb + 1][e]);
      }
#pragma unroll
      for (int n = 0; n < NN; ++n) {
        const T* r0p = vt + (16 * n + c16) * VT_LD + 32 * pb + 4 * g;
        const u32x2 lo = *reinterpret_cast<const u32x2*>(r0p);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(r0p + 16);
        const V8 va = __builtin_bit_cast(V8, u32x4{lo[0], lo[1], hi[0], hi[1]});
        acc[n] = mfma16x16x32(DT{}, va, pt, acc[n]);
      }
    }
    wave_lds_sync();
    if (has_next) {
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          kr[j][c] = kn[j][c];
          vr[j][c] = vn[j][c];
        }
    }
  }
  l_run = group4_sum(l_run);

  // Merge the waves' (max, sum, O) through LDS.
  bad = __syncthreads_or(bad);
  // Rows (wave, head) padded to RED_LD floats and written a float4 at a
  // time: the 16 head lanes of one store then start on 16 different 4-bank
  // groups instead of one bank (a 16-way conflict: ~0.4 us of a 13 us call).
  constexpr int RED_LD = Cfg::RED_LD;
  float* red_o = reinterpret_cast<float*>(smem);
  float* red_m = red_o + W * 16 * RED_LD;
  float* red_l = red_m + W * 16;
#pragma unroll
  for (int n = 0; n < NN; ++n)
    *reinterpret_cast<floatx4*>(red_o + (w * 16 + c16) * RED_LD + 16 * n + 4 * g) = acc[n];
  if (g == 0) {
    red_m[w * 16 + c16] = m_run;
    red_l[w * 16 + c16] = l_run;
  }
  __syncthreads();

  const int slot_words = p.slot_words;
  const __amdgpu_buffer_rsrc_t pr =
      __builtin_amdgcn_make_buffer_rsrc(p.part, static_cast<short>(0), p.part_bytes, kBufferWord3);
  // One float4 of the workgroup's output per thread and round: (head col, dims 4*d4..+3).
  for (int it = tid; it < G * (D / 4); it += THREADS) {
    const int col = it / (D / 4), d4 = it % (D / 4);
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < W; ++ww) M = fmaxf(M, red_m[ww * 16 + col]);
    float lsum = 0.f;
    floatx4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ww = 0; ww < W; ++ww) {
      const float mw = red_m[ww * 16 + col];
      if (mw != -INFINITY) {
        const float sc = fast_exp2(mw - M);
        lsum += red_l[ww * 16 + col] * sc;
        o += *reinterpret_cast<const floatx4*>(red_o + (ww * 16 + col) * RED_LD + 4 * d4) * sc;
      }
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

template <class DT, int D, int W, int CH, class BTI, bool BIG>
__global__ __launch_bounds__(W * 64) void paged_decode_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) char smem[DecodeCfg<D, W, CH>::LDS];
  __shared__ int64_t later_lds[BIG ? W * 64 : 1];
  __shared__ int s_merger;
  // The first item loads together with the plan's item count: the grid
  // never exceeds the plan's capacity, so the read is in bounds either way.
  uint32_t idx = blockIdx.x;
  u32x4 r0, r1;
  WaveBlocks<W, CH> ib;
  load_item<W, CH>(p, idx, r0, r1, ib);
  const uint32_t n_hdr = p.plan_hdr->n_items;
  // Both scalar loads are in flight before either is waited for (the
  // compiler would otherwise sink the item's load below the count check:
  // two round trips before the first K/V load instead of one).
  asm volatile("" ::"s"(n_hdr), "s"(r0), "s"(r1), "s"(ib.id[0]), "s"(ib.id[1]), "s"(ib.id[2]), "s"(ib.id[3]),
               "s"(ib.id[4]), "s"(ib.id[5]), "s"(ib.id[6]), "s"(ib.id[7]));
  const uint32_t n_items = n_hdr < p.item_cap ? n_hdr : static_cast<uint32_t>(p.item_cap);
  while (idx < n_items) {
    decode_item<DT, D, W, CH, BTI, BIG>(p, idx, r0, r1, ib, smem, later_lds, s_merger);
    idx += gridDim.x;
    if (idx < n_items) load_item<W, CH>(p, idx, r0, r1, ib);
    __syncthreads();  // the next item reuses the LDS
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
  static constexpr int KG = 2;                  // key groups
  static constexpr int WC = 4;                  // column waves per group
  static constexpr int W = KG * WC;             // waves per workgroup
  static constexpr int THREADS = W * 64;
  static constexpr int CT = CT_;                // 16-column tiles per wave
  static constexpr int KT = D == 64 ? 64 : 32;  // keys per step (8 KiB per tile)
  static constexpr int NT = KT / 16, NC = D / 32, NN = D / 16;
  static constexpr int CPR = D / 8;             // 16-byte chunks per key row
  static constexpr int TILE = KT * D * 2;       // bytes of one K or V tile
  static constexpr int DMA = TILE / (THREADS * 16);  // 16-byte loads per thread per tile
  static constexpr int NSLOT = 3;               // macro-slots in the ring
  static constexpr int RING = NSLOT * KG * 2 * TILE;
  static constexpr int TBL = 4096;              // table entries per window
  static constexpr int LDS = RING + TBL * 4 + 16;
  static constexpr int COLS = WC * CT * 16;     // columns per workgroup
  static constexpr int NF = CT * (NN * 4 + 2);  // floats per lane a group hands over in the merge
  static constexpr int PU = CT * (NN + 1);      // 16-byte units per lane of a split's partial
  static constexpr int SLOT_BYTES = WC * PU * 64 * 16;
  static_assert(DMA >= 1 && DMA * THREADS * 16 == TILE, "loads must tile a K/V tile");
  static_assert(NT % 2 == 0, "P^T operand pairs two 16-key tiles");
  static_assert(WC * NF * 64 * 4 <= RING, "merge buffer fits the ring");
};

typedef short short4_t __attribute__((ext_vector_type(4)));

// Address-space views for global_load_lds (global source, LDS destination).
typedef __attribute__((address_space(1))) void* gbl_void_ptr;
typedef __attribute__((address_space(3))) void* lds_void_ptr;

__device__ __forceinline__ int k_swz(int key) { return key & 7; }
__device__ __forceinline__ int v_swz(int key) { return (key & 3) << 1; }

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
  int64_t L64 = load_index(p.seq_lens, s, p.sl64);
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

  float m_run[CT], l_run[CT];
  floatx4 acc[CT][NN];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    m_run[ct] = -INFINITY;
    l_run[ct] = 0.f;
#pragma unroll
    for (int n = 0; n < NN; ++n) acc[ct][n] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  const int64_t slot_stride = static_cast<int64_t>(Hkv) * D;
  const int64_t bt_row = static_cast<int64_t>(s) * p.bt_stride;
  const T* kbase = reinterpret_cast<const T*>(p.k_cache) + static_cast<int64_t>(kvh) * D;
  const T* vbase = reinterpret_cast<const T*>(p.v_cache) + static_cast<int64_t>(kvh) * D;
  int e0 = 0;      // first table entry of the current window
  int kv_win = 0;  // keys covered by the window's entries (and below kv_end)

  // Start the K/V loads of `step` into `stage`.  Lane `lane` of load u of
  // wave w fills 16-byte slot (u * W + w) * 64 + lane of each tile.  Keys
  // past the window or kv_end read an in-bounds slot; their scores are
  // masked and their V values replaced by zero when read.
  auto dma = [&](int step, int stage) {
    char* st = smem + stage * 2 * TILE;
#pragma unroll
    for (int u = 0; u < DMA; ++u) {
      const int pos = (u * W + w) * 64 + lane;
      const int key = pos / CPR, pc = pos % CPR;
      const int t = step * KT + key;
      const bool in = t < kv_win;
      const int blk = tbl[in ? (t >> bs_shift) - e0 : 0];
      const bool valid = in && blk >= 0;
      const int64_t off = valid ? ((static_cast<int64_t>(blk) << bs_shift) + (t & bs_mask)) * slot_stride : 0;
      const T* gk = kbase + off + ((pc ^ k_swz(key)) << 3);
      const T* gv = vbase + off + ((pc ^ v_swz(key)) << 3);
      __builtin_amdgcn_global_load_lds((gbl_void_ptr)(gk), (lds_void_ptr)(st + (u * W + w) * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((gbl_void_ptr)(gv), (lds_void_ptr)(st + TILE + (u * W + w) * 1024), 16, 0, 0);
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
    // Online softmax in base 2 (sc = |scale| * log2 e).  When every key of the
    // step precedes every column of the wave, the maximum is taken over raw
    // scores and p = exp2(s * sc - m) is one FMA; otherwise key
    // tb + 16j + 4g + r of a column is masked by the column's limit.
    const bool full = tb + KT - 1 <= qmin_w;
    V8 pt[CT][NT / 2];
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
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) psum += sv[j][r];
      l_run[ct] = l_run[ct] * alpha + psum;
      // Rescale only when some column's maximum moved (alpha == 1 is exact).
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
        for (int n = 0; n < NN; ++n) acc[ct][n] *= alpha;
      }
      m_run[ct] = m_new;
#pragma unroll
      for (int pb = 0; pb < NT / 2; ++pb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pt[ct][pb][e] = static_cast<T>(sv[2 * pb][e]);
          pt[ct][pb][4 + e] = static_cast<T>(sv[2 * pb + 1][e]);
        }
    }
    // O^T += V^T P^T.  k-slot 4h + e of lane group g is key 32pb + 16h + 4g + e,
    // matching P^T.  ds_read_b64_tr_b16 gives lane i of a 16-lane group
    // element e = element i & 3 of the 8 bytes lane (i >> 2) + 4e of the group
    // addressed, so lane c16 of group g points at head dims 16n + 4 (c16 & 3)
    // .. +3 of key 32pb + 16h + 4g + (c16 >> 2) and receives V^T row 16n + c16
    // at keys 32pb + 16h + 4g + 0..3.  Keys at or past kv_end (only in the
    // last step) contribute zero.
    const bool vfull = tb + KT <= kv_end;
    const int d0 = 4 * (c16 & 3);
#pragma unroll
    for (int pb = 0; pb < NT / 2; ++pb)
#pragma unroll
      for (int n = 0; n < NN; ++n) {
        u32x2 half_op[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int key = 32 * pb + 16 * h + 4 * g + (c16 >> 2);
          const int d = 16 * n + d0;
          const char* src = vt + key * D * 2 + (((d >> 3) ^ v_swz(key)) << 4) + ((d & 7) << 1);
          half_op[h] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                      (__attribute__((address_space(3))) short4_t*)(src)));
        }
        V8 va = __builtin_bit_cast(V8, u32x4{half_op[0][0], half_op[0][1], half_op[1][0], half_op[1][1]});
        if (!vfull) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int key = 32 * pb + 16 * (e >> 2) + 4 * g + (e & 3);
            va[e] = tb + key < kv_end ? va[e] : static_cast<T>(0.f);
          }
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[ct][n] = mfma16x16x32(DT{}, va, pt[ct][pb], acc[ct][n]);
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
  auto dma_macro = [&](int M, int slot) {
#pragma unroll
    for (int k = 0; k < KG; ++k) dma(M * KG + k, slot * KG + k);
  };
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
    // M the loads of M+1 may still be in flight (KG * 2 * DMA per thread), M's
    // have landed once every wave has waited for its own and passed the
    // barrier; then M+2's loads go into the slot M-1 used.  Macro-steps past
    // M1 still load (nothing valid) so the pending count stays exact.
    dma_macro(M0, 0);
    dma_macro(M0 + 1, 1);
    int slot = 0;
    for (int M = M0; M < M1; ++M) {
      stage_barrier<KG * 2 * DMA>();
      dma_macro(M + 2, slot == 0 ? 2 : slot - 1);
      compute(slot * KG + kg, M * KG + kg);
      slot = slot == 2 ? 0 : slot + 1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  __syncthreads();  // every group's steps are done; the ring is free
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

// Decode launch shape: kDecodeWaves waves per workgroup, each moving
// decode_chunk<D> tokens (16 KiB of K+V) per step.
constexpr int kDecodeWaves = 4;
template <int D>
constexpr int decode_chunk() { return D == 64 ? 64 : 32; }

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
  a.tiles_per_step = (head_dim == 64 ? decode_chunk<64>() : decode_chunk<128>()) / 16;
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
  constexpr int W = kDecodeWaves, CH = decode_chunk<D>();
  // The block-table width is a template argument so table loads need no
  // per-lane branch.
  // Block size >= 16 (the item carries block ids) and the table's index
  // width select the kernel at compile time.
  const void* dk =
      p.inline_blocks
          ? (p.bt64 ? reinterpret_cast<const void*>(&paged_decode_kernel<DT, D, W, CH, int64_t, true>)
                    : reinterpret_cast<const void*>(&paged_decode_kernel<DT, D, W, CH, int32_t, true>))
          : (p.bt64 ? reinterpret_cast<const void*>(&paged_decode_kernel<DT, D, W, CH, int64_t, false>)
                    : reinterpret_cast<const void*>(&paged_decode_kernel<DT, D, W, CH, int32_t, false>));
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
      block_size <= 0 || max_seq_len < 0 || (head_dim != 64 && head_dim != 128))
    return 0;
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
  d = decode_shape(num_seqs, num_kv_heads, max_ctx, head_dim, current_device_cus());
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
  const int bs_shift = ilog2_exact(block_size);
  if (bs_shift < 0) return NS_ERR_UNSUPPORTED;
  if (head_dim != 64 && head_dim != 128) return NS_ERR_UNSUPPORTED;
  if (dtype != NS_DTYPE_F16 && dtype != NS_DTYPE_BF16) return NS_ERR_UNSUPPORTED;
  const int group = num_heads / num_kv_heads;
  if (group > 16) return NS_ERR_UNSUPPORTED;
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
  dshape = decode_shape(num_seqs, num_kv_heads, max_ctx, head_dim, current_device_cus());

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
