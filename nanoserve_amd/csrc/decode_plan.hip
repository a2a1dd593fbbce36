// Device-side decode plan: turns the batch's device lengths into the decode
// kernel's work items (decode_plan.h).
//
// 1. Each sequence's context length, clamped to the table, and whether it is
//    a decode row (one query row; every row of a decode-only batch).
// 2. Tokens per item, T: the smallest multiple of 16, at least min_tokens,
//    for which Hkv * sum_s max(1, ceil(L_s / T)) items fit the target of
//    `cus` x rounds items (rounds = work / (cus x round_tokens), at most the
//    host's bound); when even the largest T (the longest context, at most
//    kMaxItemTokens) does not fit, T is that largest value.  Sequence s is
//    cut into n_s = max(1, ceil(L_s / T)) ranges of equal 16-aligned size.
//    A one-round plan raises T to long_tokens when the batch still has at
//    least half as many items as CUs at that length, or when every context
//    fits one item of that length.
// 3. Pairs are listed longest sequence first (so the dispatcher starts the
//    long pairs, whose merges finish last, first), the n_s items of each
//    (sequence, kv head) pair next to each other.
// 4. Every item carries the block ids of its waves' first steps.
//
// Batches of up to kLdsSeqs sequences: every workgroup of the grid computes
// steps 1-3 in its own LDS (the same result everywhere: they read the same
// lengths) and writes its own slice of the items, so the block-id reads of
// step 4 are spread over the device.  Larger batches run one workgroup that
// keeps its per-sequence arrays in scratch after the items and lists them in
// batch order.
#include "decode_plan.h"
#include "ns_common.h"

namespace ns {
namespace {

constexpr int kThreads = 256;           // threads of a plan workgroup
constexpr int kWaves = kThreads / 64;
constexpr int kLdsSeqs = 2048;          // batches held in LDS
constexpr int kEntryPasses = 4;         // items of 32 entries per thread pass: kThreads / 32 per pass
constexpr int kItemsPerGroup = kThreads / 32 * kEntryPasses;

// Wavefront reductions and scans of the device library (DPP lane moves, no
// LDS round trips).
extern "C" __device__ uint32_t __ockl_wfred_add_u32(uint32_t);
extern "C" __device__ uint64_t __ockl_wfred_add_u64(uint64_t);
extern "C" __device__ uint32_t __ockl_wfred_max_u32(uint32_t);
extern "C" __device__ uint32_t __ockl_wfred_min_u32(uint32_t);
extern "C" __device__ uint32_t __ockl_wfscan_add_u32(uint32_t, bool inclusive);

// Exclusive prefix sum of v over the workgroup in thread order; `total` gets
// the workgroup's sum.  `red` holds one word per wave.
__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t& total, uint32_t* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t x = __ockl_wfscan_add_u32(v, true);
  if (lane == 63) red[w] = x;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int k = 0; k < kWaves; ++k) {
    const uint32_t t = red[k];
    before += k < w ? t : 0u;
    all += t;
  }
  __syncthreads();
  total = all;
  return before + x - v;
}

// Ranges of a context of L tokens at T tokens per item (an empty context is
// one empty item).
__device__ __forceinline__ uint32_t items_of(uint32_t L, uint32_t T) { return L <= T ? 1u : (L + T - 1) / T; }

struct alignas(16) PlanShared {
  uint64_t red64[kWaves];
  uint32_t red[kWaves], red2[kWaves];
  uint32_t fits[kWaves];
  uint32_t cnt[kThreads];          // item counts of the candidate tokens per item
  int32_t item_r[kItemsPerGroup];  // listed sequence of each of this workgroup's items
  int32_t len[kLdsSeqs], order[kLdsSeqs], qtok[kLdsSeqs];
  int32_t first[kLdsSeqs + 1];
};

__global__ __launch_bounds__(kThreads) void decode_plan_kernel(DecodePlanArgs a, int items_per_group) {
  __shared__ PlanShared sh;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int S = a.num_seqs, Hkv = a.num_kv_heads;
  auto* hdr = static_cast<DecodePlanHeader*>(a.plan);
  auto* items = reinterpret_cast<DecodeItem*>(hdr + 1);
  // Per-sequence arrays: length (-1: not a decode row), query row, sequences
  // in list order, and the first item of the r-th listed sequence.
  const bool in_lds = S <= kLdsSeqs;
  int32_t* g_scratch = reinterpret_cast<int32_t*>(items + a.item_cap);
  int32_t* lens = in_lds ? sh.len : g_scratch;
  int32_t* qtok = in_lds ? sh.qtok : g_scratch + S;
  int32_t* order = in_lds ? sh.order : g_scratch + 2 * S;
  int32_t* firstr = in_lds ? sh.first : g_scratch + 3 * S;  // S + 1 entries: the last is the item count

  // 1. Lengths and query rows.
  uint64_t work = 0;
  uint32_t active = 0, max_len = 0;
  for (int s = tid; s < S; s += kThreads) {
    int64_t L = load_index(a.seq_lens, s, a.sl64);
    L = L < 0 ? 0 : (L < a.max_ctx ? L : a.max_ctx);
    int64_t q = s;
    bool on = true;
    if (!a.decode_only) {
      q = load_index(a.qsl, s, a.qsl64);
      on = load_index(a.qsl, s + 1, a.qsl64) - q == 1;
    }
    lens[s] = on ? static_cast<int32_t>(L) : -1;
    qtok[s] = static_cast<int32_t>(q);
    if (on) {
      work += static_cast<uint64_t>(L);
      active += 1;
      max_len = static_cast<uint32_t>(L) > max_len ? static_cast<uint32_t>(L) : max_len;
    }
  }
  work = __ockl_wfred_add_u64(work);
  active = __ockl_wfred_add_u32(active);
  max_len = __ockl_wfred_max_u32(max_len);
  if (lane == 0) {
    sh.red64[w] = work;
    sh.red[w] = active;
    sh.red2[w] = max_len;
  }
  __syncthreads();  // also publishes lens / qtok
  work = 0;
  active = 0;
  max_len = 0;
#pragma unroll
  for (int k = 0; k < kWaves; ++k) {
    work += sh.red64[k];
    active += sh.red[k];
    max_len = sh.red2[k] > max_len ? sh.red2[k] : max_len;
  }
  const int64_t pair_work = static_cast<int64_t>(work) * Hkv;
  const int64_t pairs = static_cast<int64_t>(active) * Hkv;

  // 2. Tokens per item, in units of 16 tokens.  The item count at T is at
  // least Hkv * work / T and at most Hkv * (work / T + active), so the
  // smallest fitting T lies in [ca, cb]; the waves search it nw points at a
  // time.
  const int64_t per_round = static_cast<int64_t>(a.cus) * a.round_tokens;
  int64_t rounds = (pair_work + per_round - 1) / per_round;
  rounds = rounds < 1 ? 1 : (rounds > a.rounds ? a.rounds : rounds);
  const int64_t target = static_cast<int64_t>(a.cus) * rounds;
  const int64_t lo = (a.min_tokens + 15) / 16;
  int64_t hi = (static_cast<int64_t>(max_len) + 15) / 16;
  hi = hi < lo ? lo : (hi > kMaxItemTokens / 16 ? kMaxItemTokens / 16 : hi);
  auto clamp = [&](int64_t x) { return x < lo ? lo : (x > hi ? hi : x); };
  int64_t ca = clamp((pair_work + 16 * target - 1) / (16 * target));  // 16 * ca >= Hkv * work / target
  int64_t cb = hi;
  if (pairs < target) {
    const int64_t room = target - pairs;
    cb = clamp((pair_work + 16 * room - 1) / (16 * room));  // Hkv * (work / T + active) <= target
  }
  // Smallest fitting point of [ca, cb], or cb when none fits (cb is hi then).
  // When candidates x sequences are few, every point below cb is counted in
  // one pass (one (point, sequence) pair per thread and round, summed with
  // LDS atomics); otherwise the waves narrow the range kWaves points a pass.
  if (ca < cb && cb - ca <= kThreads && (cb - ca) * S <= 16 * kThreads) {
    const int C = static_cast<int>(cb - ca);
    for (int c = tid; c < C; c += kThreads) sh.cnt[c] = 0;
    if (tid == 0) sh.fits[0] = static_cast<uint32_t>(C);
    __syncthreads();
    for (int u = tid; u < C * S; u += kThreads) {
      const int c = u / S, sq = u - c * S;
      const int32_t L = lens[sq];
      if (L >= 0) atomicAdd(&sh.cnt[c], items_of(static_cast<uint32_t>(L), static_cast<uint32_t>((ca + c) * 16)));
    }
    __syncthreads();
    for (int c = tid; c < C; c += kThreads)
      if (static_cast<int64_t>(sh.cnt[c]) * Hkv <= target) atomicMin(&sh.fits[0], static_cast<uint32_t>(c));
    __syncthreads();
    ca += sh.fits[0];  // ca + C == cb when no point below cb fits
    cb = ca;
  }
  while (ca < cb) {
    const int64_t step = (cb - ca + kWaves - 1) / kWaves;
    const int64_t pt = ca + static_cast<int64_t>(w) * step;
    uint32_t n = 0;
    if (pt < cb) {
      const uint32_t T = static_cast<uint32_t>(pt * 16);
      for (int s = lane; s < S; s += 64) {
        const int32_t L = lens[s];
        if (L >= 0) n += items_of(static_cast<uint32_t>(L), T);
      }
      n = __ockl_wfred_add_u32(n);
    }
    if (lane == 0) sh.fits[w] = pt < cb && static_cast<int64_t>(n) * Hkv <= target;
    __syncthreads();
    int k = kWaves;
#pragma unroll
    for (int j = kWaves - 1; j >= 0; --j)
      if (sh.fits[j]) k = j;
    __syncthreads();  // fits is rewritten by the next pass
    if (k == 0) {
      cb = ca;
    } else if (k < kWaves) {  // in (point k - 1, point k]
      cb = ca + static_cast<int64_t>(k) * step;
      ca += static_cast<int64_t>(k - 1) * step + 1;
    } else {  // past the last point evaluated (the points below cb)
      int64_t m = (cb - ca - 1) / step;
      m = m < kWaves - 1 ? m : kWaves - 1;
      ca += m * step + 1;
    }
  }
  uint32_t T = static_cast<uint32_t>(ca * 16);
  // One-round plans: items of long_tokens when they still give half of the
  // CUs an item (fewer, longer items: fewer split-K merges), or when every
  // context fits one such item (no split-K merge at all).
  if (rounds == 1 && T < static_cast<uint32_t>(a.long_tokens)) {
    const uint32_t TL = static_cast<uint32_t>(a.long_tokens);
    uint32_t nl = 0;
    for (int s = tid; s < S; s += kThreads) {
      const int32_t L = lens[s];
      if (L >= 0) nl += items_of(static_cast<uint32_t>(L), TL);
    }
    nl = __ockl_wfred_add_u32(nl);
    if (lane == 0) sh.red[w] = nl;
    __syncthreads();
    nl = 0;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) nl += sh.red[k];
    __syncthreads();  // red is reused below
    if (2 * static_cast<int64_t>(nl) * Hkv >= a.cus || max_len <= TL) T = TL;
  }

  // 3. List order.  When every item runs at once (at most `cus` items) the
  // order does not matter and the batch's own order is kept; otherwise
  // decreasing length (ties by index) for batches held in LDS, so the longest
  // pairs start first, else batch order.  Sequences that are not decode rows
  // drop out.
  uint32_t total = 0;
  for (int s = tid; s < S; s += kThreads) {
    const int32_t L = lens[s];
    if (L >= 0) total += items_of(static_cast<uint32_t>(L), T);
  }
  total = __ockl_wfred_add_u32(total);
  if (lane == 0) sh.red[w] = total;
  __syncthreads();
  total = 0;
#pragma unroll
  for (int k = 0; k < kWaves; ++k) total += sh.red[k];
  __syncthreads();  // red is reused below
  const bool one_round = static_cast<int64_t>(total) * Hkv <= a.cus;
  const bool identity = one_round && static_cast<int>(active) == S;  // every sequence listed in place
  if (identity) {
    // order[r] = r: nothing to write.
  } else if (in_lds && !one_round) {
    for (int s = tid; s < S; s += kThreads) {
      const int32_t L = lens[s];
      if (L < 0) continue;
      int r = 0;
      int j = 0;
      for (; j + 4 <= S; j += 4) {
        const int4 l4 = *reinterpret_cast<const int4*>(lens + j);
        r += (l4.x > L || (l4.x == L && j < s)) + (l4.y > L || (l4.y == L && j + 1 < s)) +
             (l4.z > L || (l4.z == L && j + 2 < s)) + (l4.w > L || (l4.w == L && j + 3 < s));
      }
      for (; j < S; ++j) {
        const int32_t Lj = lens[j];
        r += Lj > L || (Lj == L && j < s);
      }
      order[r] = s;
    }
  } else {
    uint32_t base = 0;
    for (int s0 = 0; s0 < S; s0 += kThreads) {
      const int s = s0 + tid;
      const uint32_t on = s < S && lens[s] >= 0;
      uint32_t tot;
      const uint32_t r = base + block_exclusive_scan(on, tot, sh.red);
      if (on) order[r] = s;
      base += tot;
    }
  }
  __syncthreads();
  auto listed = [&](int r) { return identity ? r : order[r]; };

  // 4. First item of each listed sequence: prefix sums of Hkv * n_s.
  uint32_t base = 0;
  for (int r0 = 0; r0 < static_cast<int>(active); r0 += kThreads) {
    const int r = r0 + tid;
    const uint32_t n = r < static_cast<int>(active) ? items_of(lens[listed(r)], T) * Hkv : 0u;
    uint32_t tot;
    const uint32_t f = base + block_exclusive_scan(n, tot, sh.red);
    if (r < static_cast<int>(active)) firstr[r] = static_cast<int32_t>(f);
    base += tot;
  }
  const uint32_t n_items = base < a.item_cap ? base : a.item_cap;
  if (tid == 0) firstr[active] = static_cast<int32_t>(base);
  __syncthreads();

  // 5. This workgroup's items, 32 threads per item: thread e of an item
  // writes header word e (e < 8) and block-id entry e.  Every pass covers
  // kThreads / 32 items; the passes' block-table loads go out together.
  const int NT = a.tiles_per_step;
  const int IS = kItemBlocks / (kItemWaves * NT);
  const bool inline_blocks = a.bs_shift >= 4;
  const int e = tid & 31;
  const int ew = e / (IS * NT), est = e / NT % IS, ej = e % NT;  // entry e: tile ej of step est of wave ew
  const int64_t g0 = static_cast<int64_t>(blockIdx.x) * items_per_group;
  int64_t g1 = g0 + items_per_group;
  g1 = g1 < n_items ? g1 : n_items;
  // A grid of small slices looks each item's listed sequence up in a table
  // filled from the prefix sums; the single workgroup of a large batch
  // searches them.
  const bool table = items_per_group <= kItemsPerGroup;
  if (table) {
    for (int r = tid; r < static_cast<int>(active); r += kThreads) {
      int64_t f0 = firstr[r], f1 = firstr[r + 1];
      f0 = f0 > g0 ? f0 : g0;
      f1 = f1 < g1 ? f1 : g1;
      for (int64_t i = f0; i < f1; ++i) sh.item_r[i - g0] = r;
    }
    __syncthreads();
  }
  for (int64_t i0 = g0; i0 < g1; i0 += kThreads / 32 * kEntryPasses) {
    uint32_t hw[kEntryPasses];
    int64_t id[kEntryPasses];
    int64_t at[kEntryPasses];
#pragma unroll
    for (int ps = 0; ps < kEntryPasses; ++ps) {
      const int64_t idx = i0 + ps * (kThreads / 32) + (tid >> 5);
      at[ps] = idx < g1 ? idx : -1;
      hw[ps] = 0;
      id[ps] = 0;
      if (idx >= g1) continue;
      int lo_r = 0;
      if (table) {
        lo_r = sh.item_r[idx - g0];
      } else {
        int hi_r = static_cast<int>(active) - 1;
        while (lo_r < hi_r) {
          const int mid = (lo_r + hi_r + 1) >> 1;
          if (firstr[mid] <= idx) lo_r = mid;
          else hi_r = mid - 1;
        }
      }
      const int s = listed(lo_r);
      const uint32_t L = static_cast<uint32_t>(lens[s]);
      const uint32_t n = items_of(L, T);
      const uint32_t rel = static_cast<uint32_t>(idx - firstr[lo_r]);
      const uint32_t h = rel / n, k = rel % n;
      const uint32_t size = n == 1 ? L : ((L + n - 1) / n + 15) / 16 * 16;
      const uint32_t t0 = k * size;
      const uint32_t t1 = k + 1 == n ? L : (t0 + size < L ? t0 + size : L);
      // DecodeItem{s, qtok, t0, t1, first, nsplit, kvh, split}.
      const uint32_t fields[8] = {static_cast<uint32_t>(s), static_cast<uint32_t>(qtok[s]), t0, t1,
                                  static_cast<uint32_t>(idx) - k, n, h, k};
#pragma unroll
      for (int f = 0; f < 8; ++f)
        if (e == f) hw[ps] = fields[f];
      // Wave ew's tokens are [t0 + ew * per_wave, ...) in steps of 16 * NT.
      const uint32_t tiles = (t1 - t0 + 15) >> 4;
      const uint32_t per_wave = (tiles + kItemWaves - 1) / kItemWaves * 16;
      const uint32_t t = t0 + ew * per_wave + 16 * (est * NT + ej);
      if (inline_blocks && t < t1 && t < t0 + (ew + 1) * per_wave) {
        const int64_t row = static_cast<int64_t>(s) * a.bt_stride;
        id[ps] = load_index(a.block_tables, row + (t >> a.bs_shift), a.bt64);
      }
    }
#pragma unroll
    for (int ps = 0; ps < kEntryPasses; ++ps) {
      if (at[ps] < 0) continue;
      uint32_t* dst = reinterpret_cast<uint32_t*>(items + at[ps]);
      const int64_t v = id[ps];
      const int32_t b = v < INT32_MIN ? INT32_MIN : (v > INT32_MAX ? INT32_MAX : static_cast<int32_t>(v));
      if (e < 8) dst[e] = hw[ps];
      dst[8 + e] = static_cast<uint32_t>(b);
    }
  }
  if (blockIdx.x == 0 && tid < 4) {
    // DecodePlanHeader{n_items, num_seqs, num_kv_heads, item_tokens, item_cap, 0...}.
    u32x4* dst = reinterpret_cast<u32x4*>(hdr);
    dst[tid] = tid == 0 ? u32x4{n_items, static_cast<uint32_t>(S), static_cast<uint32_t>(Hkv), T}
                        : (tid == 1 ? u32x4{a.item_cap, 0u, 0u, 0u} : u32x4{0u, 0u, 0u, 0u});
  }
}

}  // namespace

hipError_t launch_decode_plan(const DecodePlanArgs& a, hipStream_t stream) {
  DecodePlanArgs args = a;
  // Batches held in LDS spread the items over a grid; larger ones use one
  // workgroup (their per-sequence scratch is shared).  A workgroup writes
  // kThreads / 32 items per pass and its passes run one after another, while
  // the grid's workgroups run side by side, so the grid takes as few items
  // per workgroup (whole passes, at most kItemsPerGroup) as keep it within
  // one workgroup per CU.  Measured on MI355X (c2, B = 32: 320 items of
  // capacity, 40 workgroups of 8 items against 10 of 32): the plan kernel
  // 8.26 -> 6.52 us, the c2 call 11.98 -> 11.89 us.
  const int pass_items = kThreads / 32;
  int64_t want = (static_cast<int64_t>(a.item_cap) + kPlanCUs - 1) / kPlanCUs;
  want = (want + pass_items - 1) / pass_items * pass_items;
  int per_group = static_cast<int>(want < pass_items ? pass_items : (want > kItemsPerGroup ? kItemsPerGroup : want));
  int grid = static_cast<int>((static_cast<int64_t>(a.item_cap) + per_group - 1) / per_group);
  if (a.num_seqs > kLdsSeqs || grid < 1) {
    grid = 1;
    per_group = static_cast<int>(a.item_cap);
  }
  void* kargs[] = {&args, &per_group};
  return hipLaunchKernel(reinterpret_cast<const void*>(&decode_plan_kernel), dim3(grid), dim3(kThreads), kargs, 0,
                         stream);
}

}  // namespace ns
