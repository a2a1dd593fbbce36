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

#include "ns_common.h"

namespace ns {
namespace {

// Plan entries carried in the kernel arguments (keeps them under 4 KiB).
constexpr int kPlanMax = 768;
constexpr uint32_t kPlanEmpty = 0xFFFFFFFFu;  // plan slot with no work (sequence ids stay below 0xFFFF)

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
  int64_t num_tokens;     // rows of query/out; query rows outside are never touched
  int num_heads, num_kv_heads, group;
  int bs_shift;
  int64_t num_blocks;
  int64_t max_ctx;        // tokens addressable through a table row
  float scale_log2;       // scale * log2(e): softmax runs in base 2
  int split_tokens;       // decode: context tokens per workgroup (pair plans: the base, shifted per pair)
  int split_tokens_max;   // decode, host side: the longest split any workgroup takes
  int max_splits;         // decode: workgroups per (sequence, kv head)
  int skip_decode_rows;   // varlen: one-row sequences belong to the decode kernel
  float* part_o;          // [S, Hkv, max_splits, G, D]  unnormalised partial outputs
  float* part_ml;         // [S, Hkv, max_splits, G, 2]  (running max, running sum)
  int part_o_bytes, part_ml_bytes;
  unsigned* counters;     // [S, Hkv] arrivals per (sequence, kv head); left at zero
  // Prefill split-K: partial slots of one workgroup's columns each, and one
  // arrival counter per split (sequence, kv head, column block); left at zero.
  float* pf_part;
  int pf_part_bytes;
  unsigned* pf_counters;
  int plan_n;             // decode: workgroups in the planned grid; prefill: sequences listed (0: no plan)
  int plan_pairs;         // decode: 0 = one plan entry per workgroup, else pairs listed
  // Decode schedule from host-side lengths, either one entry per workgroup x,
  // s | kvh << 16 | split << 20 | (nsplit - 1) << 26 or kPlanEmpty, or (long
  // contexts) one entry pair per (sequence, kv head): plan[0..8] are the
  // per-XCD offsets into the pair list, pair k is plan[9 + 2k] = s | kvh << 16 |
  // (nsplit - 1) << 20 and plan[10 + 2k] = its first workgroup index on its XCD.
  // Prefill schedule (its own copy of the parameters): two entries per listed
  // sequence y, s | (nsplit - 1) << 16 | split_macro << 22 and
  // slot_base | pair_base << 16.
  uint32_t plan[kPlanMax];
};

// --------------------------------------------------------------------------
// Decode: one workgroup of W waves per (sequence, kv head, context split).
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

// Split-K partials.  Split sp of pair (sequence, kv head) stores, for each
// query head col of the group, its running (max, sum) at
//   part_ml[2 * ((pair * max_splits + sp) * G + col) + {0, 1}]
// and its unnormalised output at
//   part_o[((pair * max_splits + sp) * G + col) * D + d].
//
// Partials cross workgroups (and XCDs, whose L2s are not coherent with each
// other) through device-scope (sc1) buffer accesses: the stores write through
// to the device coherence point and the loads bypass the non-coherent caches,
// so the only ordering the merge needs is that a workgroup's stores are
// acknowledged (s_waitcnt vmcnt(0)) before its arrival is counted.  No L2
// writeback or invalidate is issued.
constexpr int kSc1 = 16;                      // cache-policy bit SC1 of gfx94x/gfx950 buffer ops
constexpr int kBufferWord3 = 0x00020000;      // raw 32-bit buffer descriptor, word 3

struct PartBuffers {
  __amdgpu_buffer_rsrc_t ml, o;
};

// 32-bit device-scope buffer load.  Wider partial loads are written as runs
// of these, which the backend merges into dwordx2/x4: with ROCm 7.2's clang,
// taking elements of a raw_buffer_load_b64/b128 result was miscompiled into a
// single dword load at the base offset (both halves of a b64 read the same
// dword), while b32 loads merge and narrow correctly.
__device__ __forceinline__ float ld_sc1(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kSc1));
}

__device__ __forceinline__ PartBuffers part_buffers(const AttnParams& p) {
  PartBuffers b;
  b.ml = __builtin_amdgcn_make_buffer_rsrc(p.part_ml, static_cast<short>(0), p.part_ml_bytes, kBufferWord3);
  b.o = __builtin_amdgcn_make_buffer_rsrc(p.part_o, static_cast<short>(0), p.part_o_bytes, kBufferWord3);
  return b;
}

__device__ __forceinline__ void merge_into(float& m, float& l, floatx4& o, float m2, float l2, floatx4 o2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;  // both empty
  const float a = fast_exp2(m - mn), b = fast_exp2(m2 - mn);
  l = l * a + l2 * b;
  o = o * a + o2 * b;
  m = mn;
}

// Combine the nsplit partials of one pair into out_row ([G, D] of this kv
// head's query heads).  Each float4 column (head, 4 dims) is owned by tpi
// consecutive lanes that walk disjoint split subsets with up to 8 loads in
// flight each, then merge by butterfly; the order of operations is fixed, so
// the result does not depend on timing.
template <class DT, int D, int THREADS>
__device__ void merge_splits(const AttnParams& p, const PartBuffers& pb, int64_t pair, int nsplit,
                             typename DT::T* out_row) {
  using T = typename DT::T;
  const int G = p.group;
  const int items = G * (D / 4);
  int tpi = THREADS / items;
  tpi = tpi >= 8 ? 8 : tpi >= 4 ? 4 : tpi >= 2 ? 2 : 1;
  const int tid = threadIdx.x, sub = tid % tpi;
  const int64_t base = pair * p.max_splits;
  for (int it = tid / tpi; it < items; it += THREADS / tpi) {
    // The lanes of a tpi group share `it`, so they run the same trip count
    // and are all active at the butterfly below.
    const int col = it / (D / 4), d4 = it % (D / 4);
    float m = -INFINITY, l = 0.f;
    floatx4 o = {0.f, 0.f, 0.f, 0.f};
    for (int sp0 = sub; sp0 < nsplit; sp0 += 8 * tpi) {
      float mb[8], lb[8];
      floatx4 ob[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        // Slots past nsplit read split 0 again (in bounds) and are dropped below.
        const int sp = sp0 + k * tpi < nsplit ? sp0 + k * tpi : 0;
        const int pi = static_cast<int>((base + sp) * G + col);
        mb[k] = ld_sc1(pb.ml, pi * 8);
        lb[k] = ld_sc1(pb.ml, pi * 8 + 4);
        const int oo = pi * (D * 4) + 16 * d4;
        ob[k] = floatx4{ld_sc1(pb.o, oo), ld_sc1(pb.o, oo + 4), ld_sc1(pb.o, oo + 8), ld_sc1(pb.o, oo + 12)};
      }
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (sp0 + k * tpi < nsplit) merge_into(m, l, o, mb[k], lb[k], ob[k]);
    }
    for (int off = 1; off < tpi; off <<= 1) {
      const float m2 = __shfl_xor(m, off), l2 = __shfl_xor(l, off);
      const floatx4 o2 = {__shfl_xor(o[0], off), __shfl_xor(o[1], off), __shfl_xor(o[2], off), __shfl_xor(o[3], off)};
      merge_into(m, l, o, m2, l2, o2);
    }
    if (sub == 0) {
      // A split that met an invalid block id carries NaN, which propagates.
      const float inv = l > 0.f || l != l ? 1.f / l : 0.f;
      typename DT::vec4 v4;
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = static_cast<T>(o[r] * inv);
      *reinterpret_cast<u32x2*>(out_row + col * D + 4 * d4) = __builtin_bit_cast(u32x2, v4);
    }
  }
}

template <class IDX>
__device__ __forceinline__ int64_t ld_idx(const void* p, int64_t i) {
  return static_cast<int64_t>(reinterpret_cast<const IDX*>(p)[i]);
}

// Decode.  Work unit: (sequence s, kv head, split) = split_tokens consecutive
// context tokens of one kv head, read once and used by all G query heads of
// the group.  With a host plan the grid is (plan_n) and entry x names
// (s, kv head, split, nsplit): all splits of a pair sit on workgroup ids with
// the same x % 8, i.e. on one XCD, so the merging workgroup reads the
// partials from its own L2 (the protocol does not depend on that placement,
// only its speed does).  Otherwise the grid is (max_splits, Hkv, S) and splits
// past a sequence's end exit at once.
template <class DT, int D, int W, int CH, class BTI, bool PIPE>
__global__ __launch_bounds__(W * 64) void paged_decode_kernel(AttnParams p) {
  using Cfg = DecodeCfg<D, W, CH>;
  using T = typename DT::T;
  using V8 = typename DT::vec8;
  constexpr int THREADS = Cfg::kThreads;
  constexpr int NT = Cfg::NT, NC = Cfg::NC, NN = Cfg::NN, VT_LD = Cfg::VT_LD;
  __shared__ __attribute__((aligned(16))) char smem[Cfg::LDS];
  __shared__ int s_last;

  int s, split, kvh, nsplit_plan = 0;
  int split_tok = p.split_tokens;
  if (p.plan_n > 0 && p.plan_pairs == 0) {
    const uint32_t e = p.plan[blockIdx.x];
    if (e == kPlanEmpty) return;
    s = static_cast<int>(e & 0xFFFFu);
    kvh = static_cast<int>((e >> 16) & 0xFu);
    split = static_cast<int>((e >> 20) & 0x3Fu);
    nsplit_plan = static_cast<int>(e >> 26) + 1;
  } else if (p.plan_n > 0) {
    // Pair list: workgroup x is the (x / 8)-th of XCD x % 8; find the pair
    // whose splits cover it (binary search over first-workgroup indices).
    const int x = static_cast<int>(blockIdx.x & 7u), idx = static_cast<int>(blockIdx.x >> 3);
    int lo = static_cast<int>(p.plan[x]), hi = static_cast<int>(p.plan[x + 1]);
    if (lo >= hi) return;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (static_cast<int>(p.plan[10 + 2 * mid] & 0x3FFFFFFu) <= idx) lo = mid;
      else hi = mid;
    }
    const uint32_t e = p.plan[9 + 2 * lo], f = p.plan[10 + 2 * lo];
    nsplit_plan = static_cast<int>(e >> 20) + 1;
    split = idx - static_cast<int>(f & 0x3FFFFFFu);
    split_tok = p.split_tokens << (f >> 26);
    if (split >= nsplit_plan) return;  // past the last pair of this XCD
    s = static_cast<int>(e & 0xFFFFu);
    kvh = static_cast<int>((e >> 16) & 0xFu);
  } else {
    split = blockIdx.x;
    kvh = blockIdx.y;
    s = blockIdx.z;
  }
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
  const int G = p.group, Hkv = p.num_kv_heads;
  const int bs_mask = (1 << p.bs_shift) - 1;
  const int64_t bt_row = static_cast<int64_t>(s) * p.bt_stride;
  const int64_t t_split0 = static_cast<int64_t>(split) * split_tok;
  const int64_t t_cap = p.max_ctx < t_split0 + split_tok ? p.max_ctx : t_split0 + split_tok;

  // Loads that do not depend on the context length go out together: the
  // length, this wave's first block-table entries and (decode-only) Q.
  const int64_t L_raw = load_index(p.seq_lens, s, p.sl64);
  const int64_t tb0 = t_split0 + w * CH;
  int64_t blk[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    // Clamped into the table so the load is unconditional; entries past the
    // split are never used.
    int64_t t = tb0 + 16 * j + c16;
    t = t < t_cap ? t : t_cap - 1;
    t = t > 0 ? t : 0;
    blk[j] = ld_idx<BTI>(p.bt, bt_row + (t >> p.bs_shift));
  }
  int64_t qtok = s;
  if (!p.decode_only) {
    const int64_t q0 = load_index(p.qsl, s, p.qsl64);
    const int64_t q1 = load_index(p.qsl, s + 1, p.qsl64);
    if (q1 - q0 != 1) return;  // not a decode row: the varlen kernel owns it
    qtok = q0;
  }
  if (qtok < 0 || qtok >= p.num_tokens) return;
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

  const int64_t L = L_raw < p.max_ctx ? L_raw : p.max_ctx;
  T* out_row = reinterpret_cast<T*>(p.out) + (qtok * p.num_heads + static_cast<int64_t>(kvh) * G) * D;
  const int nsplit_len = static_cast<int>((L + split_tok - 1) / split_tok);
  // The splits that arrive at this pair's merge.  A plan fixes them from the
  // host lengths, so every launched workgroup arrives even if the device
  // length is shorter; a device length the plan does not cover is a broken
  // contract and poisons the pair with NaN.
  int bad = 0;
  int nsplit = nsplit_len;
  if (p.plan_n > 0) {
    bad = nsplit_len > nsplit_plan;
    nsplit = nsplit_plan;
  } else if (split >= nsplit_len) {
    if (split == 0)  // no key is visible: the reference's masked softmax yields zeros
      for (int i = tid; i < G * D; i += THREADS) out_row[i] = static_cast<T>(0.f);
    return;
  }
  const int64_t t_split1 = L < t_split0 + split_tok ? L : t_split0 + split_tok;

  T* vt = reinterpret_cast<T*>(smem) + w * D * VT_LD;  // this wave's V^T tile [D][VT_LD]
  float m_run = -INFINITY, l_run = 0.f;
  floatx4 acc[NN];
#pragma unroll
  for (int n = 0; n < NN; ++n) acc[n] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int64_t slot_stride = static_cast<int64_t>(Hkv) * D;  // elements between slots
  const T* kbase = reinterpret_cast<const T*>(p.k_cache) + static_cast<int64_t>(kvh) * D + 8 * g;
  const T* vbase = reinterpret_cast<const T*>(p.v_cache) + static_cast<int64_t>(kvh) * D + 8 * g;

  // Issue the K/V loads of the step starting at token tb: returns, per
  // 16-token tile, whether this lane's token is valid (its V is zeroed at
  // use, so nothing here waits for the data).  Invalid lanes read slot 0,
  // which is always in bounds.
  auto issue_step = [&](int64_t tb, const int64_t (&bk)[NT], V8 (&kx)[NT][NC], V8 (&vx)[NT][NC]) {
    int vmask = 0;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int64_t t = tb + 16 * j + c16;
      bool valid = t < t_split1;
      if (valid && (bk[j] < 0 || bk[j] >= p.num_blocks)) {
        bad = 1;
        valid = false;
      }
      const int64_t off = valid ? ((bk[j] << p.bs_shift) + (t & bs_mask)) * slot_stride : 0;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        kx[j][c] = load16<DT>(kbase + off + 32 * c);
        vx[j][c] = load16<DT>(vbase + off + 32 * c);
      }
      vmask |= valid ? 1 << j : 0;
    }
    return vmask;
  };
  // Block-table entries of the step at tb (clamped into this split).
  auto table_step = [&](int64_t tb, int64_t (&bk)[NT]) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      int64_t t = tb + 16 * j + c16;
      t = t < t_split1 ? t : t_split1 - 1;
      bk[j] = ld_idx<BTI>(p.bt, bt_row + (t >> p.bs_shift));
    }
  };

  // Software pipeline over the wave's steps: step i+1's K/V loads and step
  // i+2's table entries are in flight while step i computes.
  V8 kr[NT][NC], vr[NT][NC];
  int vmask = 0;
  if (tb0 < t_split1) {
    vmask = issue_step(tb0, blk, kr, vr);
    table_step(tb0 + W * CH, blk);
  }
  for (int64_t tb = tb0; tb < t_split1; tb += W * CH) {
    if (!PIPE && tb != tb0) {
      // Without the pipeline (one step per wave in the common case) later
      // steps issue their loads at the top of the step.
      vmask = issue_step(tb, blk, kr, vr);
      table_step(tb + W * CH, blk);
    }
    const bool has_next = PIPE && tb + W * CH < t_split1;
    V8 kn[NT][NC], vn[NT][NC];
    int vmask_n = 0;
    if (has_next) {
      vmask_n = issue_step(tb + W * CH, blk, kn, vn);
      table_step(tb + 2 * W * CH, blk);
    }
#pragma unroll
    for (int j = 0; j < NT; ++j)
      if (!(vmask >> j & 1))
#pragma unroll
        for (int c = 0; c < NC; ++c) vr[j][c] = zero8<DT>();
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
        const float x = t < t_split1 ? sacc[j][r] * p.scale_log2 : -INFINITY;
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
        const T* r0 = vt + (16 * n + c16) * VT_LD + 32 * pb + 4 * g;
        const u32x2 lo = *reinterpret_cast<const u32x2*>(r0);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(r0 + 16);
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
      vmask = vmask_n;
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

  // One float4 of the workgroup's output per thread: (head col, dims 4*d4..+3).
  const int64_t pair = static_cast<int64_t>(s) * Hkv + kvh;
  const PartBuffers pbuf = part_buffers(p);
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
      const int pi = static_cast<int>((pair * p.max_splits + split) * G + col);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), pbuf.o, pi * (D * 4) + 16 * d4, 0, kSc1);
      if (d4 == 0)
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{__builtin_bit_cast(uint32_t, M), __builtin_bit_cast(uint32_t, lsum)},
                                              pbuf.ml, pi * 8, 0, kSc1);
    }
  }
  if (nsplit == 1) return;

  // Split-K merge inside the same launch: the last workgroup of this pair to
  // arrive combines every split's partial.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial stores are acknowledged
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(&p.counters[pair], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == static_cast<unsigned>(nsplit - 1);
  }
  __syncthreads();
  if (!s_last) return;
  merge_splits<DT, D, THREADS>(p, pbuf, pair, nsplit, out_row);
  if (tid == 0) __hip_atomic_store(&p.counters[pair], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
__global__ __launch_bounds__(kPrefillThreads) void paged_prefill_kernel(AttnParams p) {
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
struct DecodePlan {
  int split_tokens;
  int max_splits;
};

// 16-column tiles per prefill wave (columns per workgroup = 64 * kPrefillTiles).
constexpr int kPrefillTiles = 2;

// Decode launch shape: kDecodeWaves waves per workgroup, each moving
// decode_chunk<D> tokens (16 KiB of K+V) per step.
constexpr int kDecodeWaves = 4;
template <int D>
constexpr int decode_chunk() { return D == 64 ? 64 : 32; }

// Tokens per decode workgroup: one step of every wave, doubled until a
// sequence needs at most 64 workgroups, which bounds the partial buffers
// while giving short batches enough workgroups to cover 256 CUs.
DecodePlan plan_decode(int head_dim, int64_t ctx_tokens) {
  const int base = kDecodeWaves * (head_dim == 64 ? decode_chunk<64>() : decode_chunk<128>());
  int64_t tok = base;
  while ((ctx_tokens + tok - 1) / tok > 64) tok *= 2;
  DecodePlan plan;
  plan.split_tokens = static_cast<int>(tok);
  plan.max_splits = static_cast<int>(ctx_tokens <= 0 ? 1 : (ctx_tokens + tok - 1) / tok);
  return plan;
}

struct WorkspaceLayout {
  size_t counters_off, ml_off, o_off;
  size_t pf_counters_off, pf_part_off, pf_part_bytes;  // prefill split-K region (0 bytes: none)
  size_t total;
};

// Prefill split-K slots a workspace provides (one per split of a column
// block), and the bytes of one slot: a workgroup's per-lane softmax state.
constexpr int kPrefillSlots = 512;
size_t prefill_slot_bytes(int head_dim) {
  return head_dim == 64 ? PrefillCfg<64, kPrefillTiles>::SLOT_BYTES : PrefillCfg<128, kPrefillTiles>::SLOT_BYTES;
}

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Arrival counters sit at the same offsets for every call (decode pairs from
// 0, prefill pairs after kMaxDecodePairs), ahead of all partials: a workspace
// reused by calls of other shapes never has one call's partials where another
// call's counters are, so the counters stay at zero between calls.
constexpr size_t kMaxDecodePairs = (size_t{1} << 20) - kPrefillSlots;
constexpr size_t kCounterBytes = (kMaxDecodePairs + kPrefillSlots) * sizeof(unsigned);

WorkspaceLayout workspace_layout(int num_seqs, int num_kv_heads, int group, int head_dim,
                                 const DecodePlan& plan, bool with_prefill) {
  const size_t pairs = static_cast<size_t>(num_seqs) * num_kv_heads;
  const size_t parts = pairs * plan.max_splits * group;
  WorkspaceLayout l;
  l.counters_off = 0;
  l.pf_counters_off = kMaxDecodePairs * sizeof(unsigned);
  l.ml_off = kCounterBytes;
  l.o_off = align_up(l.ml_off + parts * 2 * sizeof(float), 256);
  l.pf_part_off = align_up(l.o_off + parts * head_dim * sizeof(float), 256);
  l.pf_part_bytes = with_prefill ? kPrefillSlots * prefill_slot_bytes(head_dim) : 0;
  l.total = align_up(l.pf_part_off + l.pf_part_bytes, 256);
  return l;
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
template <class DT, int D>
hipError_t launch_attention(AttnParams& p, AttnParams& pp, int pf_grid_x, bool launch_decode, int num_seqs,
                            int max_query_len, hipStream_t stream, const AuxStream* aux) {
  void* args[] = {&p};
  void* pargs[] = {&pp};
  constexpr int W = kDecodeWaves, CH = decode_chunk<D>();
  // The block-table width is a template argument so table loads need no
  // per-lane branch.
  // Workgroups whose waves take several steps pipeline their K/V loads
  // (double-buffered registers, fewer resident waves); one-step workgroups
  // keep the lean variant and its occupancy.
  const bool pipe = p.split_tokens_max > W * CH;
  const void* dk =
      p.bt64 ? (pipe ? reinterpret_cast<const void*>(&paged_decode_kernel<DT, D, W, CH, int64_t, true>)
                     : reinterpret_cast<const void*>(&paged_decode_kernel<DT, D, W, CH, int64_t, false>))
             : (pipe ? reinterpret_cast<const void*>(&paged_decode_kernel<DT, D, W, CH, int32_t, true>)
                     : reinterpret_cast<const void*>(&paged_decode_kernel<DT, D, W, CH, int32_t, false>));
  const dim3 grid = p.plan_n > 0 ? dim3(p.plan_n, 1, 1) : dim3(p.max_splits, p.num_kv_heads, num_seqs);
  if (p.decode_only) return hipLaunchKernel(dk, grid, dim3(W * 64), args, 0, stream);

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
    hipError_t e = hipLaunchKernel(dk, grid, dim3(W * 64), args, 0, stream);
    if (e != hipSuccess) return e;
    return hipLaunchKernel(vk, vgrid, dim3(PCfg::THREADS), pargs, 0, stream);
  }
  hipError_t e = hipEventRecord(aux->fork, stream);
  if (e == hipSuccess) e = hipStreamWaitEvent(aux->stream, aux->fork, 0);
  if (e != hipSuccess) return e;
  // Once the aux stream depends on the caller's, it is joined back whatever
  // else fails (an unjoined fork would also break a graph capture).
  const hipError_t ed = hipLaunchKernel(dk, grid, dim3(W * 64), args, 0, aux->stream);
  const hipError_t er = hipEventRecord(aux->join, aux->stream);
  const hipError_t ev = hipLaunchKernel(vk, vgrid, dim3(PCfg::THREADS), pargs, 0, stream);
  const hipError_t ej = er == hipSuccess ? hipStreamWaitEvent(stream, aux->join, 0) : er;
  return ed != hipSuccess ? ed : (ev != hipSuccess ? ev : ej);
}

bool aligned16(const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; }

// Fill p.plan from host-side context lengths: one entry per (sequence, kv
// head, split) of a decode batch.  Workgroup x runs on XCD x % 8 (the
// dispatcher's round-robin over XCDs), so the pairs are bin-packed onto the 8
// XCDs by context length (longest first, each to the least loaded XCD) and a
// pair's splits all get ids of one residue: its partials then meet in one L2.
// Within an XCD the longest pairs come first, so their merges overlap the
// streaming of shorter ones.  Returns the entry count (a multiple of 8,
// unused slots kPlanEmpty), or 0 when the batch does not fit the plan (the
// launch then uses the full (max_splits, Hkv, S) grid).
int build_decode_plan_for(AttnParams& p, const std::vector<std::pair<int64_t, int>>& order, int split) {
  constexpr int kXcds = 8;
  int64_t units = 0;
  for (const auto& pr : order) {
    const int64_t n = (pr.first + split - 1) / split;
    units += (n < 1 ? 1 : n) * p.num_kv_heads;
  }
  if (units > kPlanMax) return 0;
  std::vector<uint32_t> bucket[kXcds];
  int64_t load[kXcds] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (const auto& [L, i] : order) {
    int64_t n = (L + split - 1) / split;
    n = n < 1 ? 1 : n;
    for (int kvh = 0; kvh < p.num_kv_heads; ++kvh) {
      int b = 0;
      for (int x = 1; x < kXcds; ++x)
        if (load[x] < load[b]) b = x;
      load[b] += L + split / 4;  // tokens, plus a per-pair overhead
      for (int64_t sp = 0; sp < n; ++sp)
        bucket[b].push_back(static_cast<uint32_t>(i) | static_cast<uint32_t>(kvh) << 16 |
                            static_cast<uint32_t>(sp) << 20 | static_cast<uint32_t>(n - 1) << 26);
    }
  }
  size_t rows = 0;
  for (int x = 0; x < kXcds; ++x) rows = bucket[x].size() > rows ? bucket[x].size() : rows;
  if (rows * kXcds > static_cast<size_t>(kPlanMax)) return 0;
  for (size_t k = 0; k < rows; ++k)
    for (int x = 0; x < kXcds; ++x)
      p.plan[k * kXcds + x] = k < bucket[x].size() ? bucket[x][k] : kPlanEmpty;
  p.split_tokens = split;
  p.split_tokens_max = split;
  return static_cast<int>(rows * kXcds);
}

// Pair-list plan at a given split: the same XCD bin-packing as above, but
// one kernel-argument entry pair per (sequence, kv head) instead of one entry
// per workgroup, so long contexts keep short splits (the dispatcher then
// balances the tail) without overflowing the kernel arguments.
// A pair's split is the base, doubled until the pair has at most
// kMaxPairSplits splits: the last split to arrive merges them all, and that
// merge's length grows with their number.
constexpr int kPairMax = (kPlanMax - 9) / 2;
constexpr int kMaxPairSplits = 64;

int build_decode_pair_plan(AttnParams& p, const std::vector<std::pair<int64_t, int>>& order, int split) {
  constexpr int kXcds = 8;
  if (static_cast<int64_t>(order.size()) * p.num_kv_heads > kPairMax) return 0;
  struct Item {
    uint32_t e;
    int64_t n;
    int shift;
  };
  std::vector<Item> bucket[kXcds];
  int64_t load[kXcds] = {0, 0, 0, 0, 0, 0, 0, 0};
  int max_shift = 0;
  for (const auto& [L, i] : order) {
    int shift = 0;
    while ((L + (static_cast<int64_t>(split) << shift) - 1) / (static_cast<int64_t>(split) << shift) > kMaxPairSplits)
      ++shift;
    if (shift > 20) return 0;
    const int64_t sp = static_cast<int64_t>(split) << shift;
    int64_t n = (L + sp - 1) / sp;
    n = n < 1 ? 1 : n;
    max_shift = shift > max_shift ? shift : max_shift;
    for (int kvh = 0; kvh < p.num_kv_heads; ++kvh) {
      int b = 0;
      for (int x = 1; x < kXcds; ++x)
        if (load[x] < load[b]) b = x;
      load[b] += L + sp / 4;
      bucket[b].push_back({static_cast<uint32_t>(i) | static_cast<uint32_t>(kvh) << 16 |
                               static_cast<uint32_t>(n - 1) << 20,
                           n, shift});
    }
  }
  int k = 0;
  int64_t rows = 0;
  for (int x = 0; x < kXcds; ++x) {
    p.plan[x] = static_cast<uint32_t>(k);
    int64_t first = 0;
    for (const Item& it : bucket[x]) {
      if (first > 0x3FFFFFF) return 0;
      p.plan[9 + 2 * k] = it.e;
      p.plan[10 + 2 * k] = static_cast<uint32_t>(first) | static_cast<uint32_t>(it.shift) << 26;
      first += it.n;
      ++k;
    }
    rows = first > rows ? first : rows;
  }
  p.plan[kXcds] = static_cast<uint32_t>(k);
  if (rows * kXcds > 0x7FFFFFFF) return 0;
  p.split_tokens = split;
  p.split_tokens_max = split << max_shift;
  p.plan_pairs = k;
  return static_cast<int>(rows * kXcds);
}

// The split starts at the workspace layout's (so at most max_splits per
// sequence).  If one entry per workgroup does not fit, a pair-list plan keeps
// that split; failing that, the split doubles until the batch fits: long
// contexts then get long splits, whose waves pipeline their steps.
int64_t host_index(const void* a, int is64, int64_t i) {
  return is64 ? static_cast<const int64_t*>(a)[i] : static_cast<const int32_t*>(a)[i];
}

// With host query offsets only the one-row sequences are planned (a batch
// without any gets an empty plan, -1, and no decode launch).
int build_decode_plan(AttnParams& p, const void* lens, int lens64, const void* qsl, int qsl64, int num_seqs) {
  if (num_seqs > 0xFFFF || p.num_kv_heads > 16 || p.max_splits > 64) return 0;
  std::vector<std::pair<int64_t, int>> order;
  order.reserve(num_seqs);
  for (int i = 0; i < num_seqs; ++i) {
    if (qsl && host_index(qsl, qsl64, i + 1) - host_index(qsl, qsl64, i) != 1) continue;
    int64_t L = host_index(lens, lens64, i);
    L = L < 0 ? 0 : (L < p.max_ctx ? L : p.max_ctx);
    order.push_back({L, i});
  }
  if (order.empty()) return -1;
  std::stable_sort(order.begin(), order.end(),
                   [](const std::pair<int64_t, int>& a, const std::pair<int64_t, int>& b) { return a.first > b.first; });
  p.plan_pairs = 0;
  {
    const int n = build_decode_plan_for(p, order, p.split_tokens);
    if (n > 0) return n;
    const int np = build_decode_pair_plan(p, order, p.split_tokens);
    if (np > 0) return np;
  }
  for (int64_t split = p.split_tokens;; split *= 2) {
    const int n = build_decode_plan_for(p, order, static_cast<int>(split));
    if (n > 0) return n;
    if (split >= p.max_ctx || split > (1 << 24)) return 0;  // one split per sequence did not fit either
  }
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
int build_prefill_plan(AttnParams& pp, const void* lens, int lens64, const void* qsl, int qsl64, int num_seqs,
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
  const ns::DecodePlan plan = ns::plan_decode(head_dim, ns::round_up_ctx(max_seq_len, block_size));
  return ns::workspace_layout(num_seqs, num_kv_heads, num_heads / num_kv_heads, head_dim, plan, !is_decode_only)
      .total;
}

namespace ns {
namespace {

// Scratch of ns_paged_attention_noalloc: the workspace of calls whose caller
// cannot allocate one.  A file-scope device array, so each device the library
// runs on holds its own copy from module load (zero-filled by the loader)
// until the process ends.  In host code `g_noalloc_scratch` names a host-side
// stand-in, never the device memory: kernels and fills get the address that
// hipGetSymbolAddress returns for the current device, kept per device.
constexpr size_t kNoallocScratchBytes = size_t{64} << 20;
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
  const DecodePlan plan = plan_decode(head_dim, ctx_plan);
  const WorkspaceLayout wl = workspace_layout(num_seqs, num_kv_heads, group, head_dim, plan, !is_decode_only);
  if (noalloc) {
    // Shapes whose workspace exceeds the scratch are refused before any HIP call.
    if (wl.total > kNoallocScratchBytes) return NS_ERR_WORKSPACE;
    workspace = noalloc_scratch(static_cast<hipStream_t>(stream));
    if (!workspace) return NS_ERR_HIP;
    workspace_bytes = kNoallocScratchBytes;
  }
  if (!workspace || workspace_bytes < wl.total) return NS_ERR_WORKSPACE;
  // Partials are addressed through buffer descriptors with 32-bit offsets.
  if (wl.pf_part_off - wl.o_off > 0x7FFFFFFFu || wl.pf_part_bytes > 0x7FFFFFFFu) return NS_ERR_UNSUPPORTED;
  if (static_cast<size_t>(num_seqs) * num_kv_heads > kMaxDecodePairs) return NS_ERR_UNSUPPORTED;

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
  p.num_tokens = num_tokens;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.group = group;
  p.bs_shift = bs_shift;
  p.num_blocks = num_blocks;
  const int64_t table_tokens = block_table_width * static_cast<int64_t>(block_size);
  p.max_ctx = ctx_plan < table_tokens ? ctx_plan : table_tokens;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.split_tokens = plan.split_tokens;
  p.split_tokens_max = plan.split_tokens;
  p.max_splits = plan.max_splits;
  p.skip_decode_rows = 1;
  char* ws = static_cast<char*>(workspace);
  p.counters = reinterpret_cast<unsigned*>(ws + wl.counters_off);
  p.part_ml = reinterpret_cast<float*>(ws + wl.ml_off);
  p.part_o = reinterpret_cast<float*>(ws + wl.o_off);
  p.part_ml_bytes = static_cast<int>(wl.o_off - wl.ml_off);
  p.part_o_bytes = static_cast<int>(wl.pf_part_off - wl.o_off);
  p.pf_counters = reinterpret_cast<unsigned*>(ws + wl.pf_counters_off);
  p.pf_part = reinterpret_cast<float*>(ws + wl.pf_part_off);
  p.pf_part_bytes = static_cast<int>(wl.pf_part_bytes);
  p.plan_n = 0;
  p.plan_pairs = 0;
  // Decode plan from the host lengths.  Without host query offsets a mixed
  // batch's plan covers every sequence and the workgroups of sequences with
  // more than one query row leave at once (the prefill kernel owns them).
  const void* qsl_host = is_decode_only ? nullptr : query_start_loc_host;
  bool launch_decode = true;
  if (seq_lens_host) {
    const int n = build_decode_plan(p, seq_lens_host, seq_lens_host_is_int64, qsl_host,
                                    query_start_loc_host_is_int64, num_seqs);
    launch_decode = n >= 0;
    p.plan_n = n > 0 ? n : 0;
  }
  // Prefill plan (split-K over the CUs) from host offsets and lengths.
  AttnParams pp;
  int pf_grid_x = 0;
  if (!is_decode_only) {
    pp = p;
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
  hipError_t e;
  if (dtype == NS_DTYPE_F16)
    e = head_dim == 64 ? launch_attention<F16, 64>(p, pp, pf_grid_x, launch_decode, num_seqs, max_query_len, st, ax)
                       : launch_attention<F16, 128>(p, pp, pf_grid_x, launch_decode, num_seqs, max_query_len, st, ax);
  else
    e = head_dim == 64 ? launch_attention<BF16, 64>(p, pp, pf_grid_x, launch_decode, num_seqs, max_query_len, st, ax)
                       : launch_attention<BF16, 128>(p, pp, pf_grid_x, launch_decode, num_seqs, max_query_len, st, ax);
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
                                  void* workspace, size_t workspace_bytes, void* stream,
                                  void* aux_stream, void* fork_event, void* join_event) {
  return ns::paged_attention_entry(out, query, k_cache, v_cache, block_tables, block_table_stride,
                                   block_table_width, block_tables_is_int64, seq_lens, seq_lens_is_int64,
                                   query_start_loc, query_start_loc_is_int64, seq_lens_host,
                                   seq_lens_host_is_int64, query_start_loc_host, query_start_loc_host_is_int64,
                                   num_seqs, num_tokens, max_query_len, max_seq_len, is_decode_only, num_heads,
                                   num_kv_heads, head_dim, block_size, num_blocks, scale, dtype, workspace,
                                   workspace_bytes, false, stream, aux_stream, fork_event, join_event);
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
                                          float scale, int dtype, void* stream,
                                          void* aux_stream, void* fork_event, void* join_event) {
  return ns::paged_attention_entry(out, query, k_cache, v_cache, block_tables, block_table_stride,
                                   block_table_width, block_tables_is_int64, seq_lens, seq_lens_is_int64,
                                   query_start_loc, query_start_loc_is_int64, seq_lens_host,
                                   seq_lens_host_is_int64, query_start_loc_host, query_start_loc_host_is_int64,
                                   num_seqs, num_tokens, max_query_len, max_seq_len, is_decode_only, num_heads,
                                   num_kv_heads, head_dim, block_size, num_blocks, scale, dtype, nullptr, 0,
                                   true, stream, aux_stream, fork_event, join_event);
}
