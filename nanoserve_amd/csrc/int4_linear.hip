// int4_linear: y = x · dequant(W)^T + bias with W stored as group-wise
// asymmetric INT4 (the reference's QuantLinear "int4" format), dequantised in
// registers on its way into the MFMA.
//
// Replaces QuantLinear.forward (reference nanoserve/quant.py:157-158), which
// expands the whole weight to the model dtype on every call
// (dequantize_int4, quant.py:83-95) and then runs F.linear: per call it writes
// and re-reads N·K·2 bytes beside the GEMM.  Here each weight byte is read once
// per output tile and never expanded in memory.
//
// Format (quant.py:53-80): qweight [N, K/2] uint8, two 4-bit codes per byte,
// even k in the low nibble and odd k in the high nibble; scales [N, K/gs]
// float32; zeros [N, K/gs] uint8.  Weight (n, k) is
//     w = (q - zero) * scale          (float32)
// rounded to the model dtype, exactly as dequantize_int4 computes it, so the
// MFMA sees the reference's own dequantised weights.
//
// Tiling (gfx950, wave64): a workgroup owns FT·16 output features (FT MFMA
// row tiles of W, which share every x load) and MT tokens (MT/16 MFMA column
// tiles of x^T).  K is walked in chunks of 128; the workgroup's WAVES waves
// split the chunks between them and reduce through LDS.  Within a chunk, lane group g = lane/16 owns the 32
// consecutive k values [128c + 32g, +32) of its feature row: one 16-byte load
// brings all 32 codes, which feed four MFMA steps (k order permuted the same
// way for both operands, so the sum is unchanged).  The same lane reads the
// matching 8 x values per step for each column tile.  The result D[n][m]
// lands as four consecutive features of one token per lane: one 8-byte store.
#include <algorithm>

#include "ns_common.h"

namespace ns {
namespace {

// Every float op below rounds to f32 once, as the reference's separate tensor
// ops do: no contraction into fused multiply-adds.
#pragma clang fp contract(off)

struct Int4LinearParams {
  void* out;              // [M, N] contiguous ([M, N/2] for NS_EPILOGUE_SILU_MUL), model dtype
  const char* x;          // [M, K] rows of x_stride elements
  int64_t x_stride;
  const uint8_t* qweight; // [N, K/2]
  const float* scales;    // [N, G]
  const uint8_t* zeros;   // [N, G]
  const void* bias;       // [N] model dtype, or null
  const void* residual;   // [M, N] contiguous, model dtype (NS_EPILOGUE_RESIDUAL)
  const void* norm_weight; // [K] model dtype: RMSNorm the rows of x first (or null)
  float norm_eps;
  int epilogue;
  int M, N, K, group_size, groups;
  // Rotary + cache-write epilogue (ROPE kernels): W's rows are q|k|v heads in
  // rotary-pair order (rope_pair_row), out is q' [M, num_heads, head_dim].
  const void* cos;         // [M, head_dim] rows of cs_stride elements, model dtype
  const void* sin;
  int64_t cs_stride;
  void* k_cache;           // [num_slots, num_kv_heads, head_dim], model dtype
  void* v_cache;
  const void* slots;       // [M] int32 or int64
  int slots64;
  int64_t num_slots;
  int num_heads, num_kv_heads, head_dim;
  // Split-K (multi-chunk kernels, gridDim.z = splits > 1): partial sums of
  // every (tile, split) go to `part`, arrivals are counted in `counters` (one
  // per tile, zero between calls) and the last split of a tile finishes it.
  float* part;
  unsigned* counters;
  int part_bytes;
  // Tiled GEMM (1-D grid): gemm_gx feature tiles per token tile; tiles
  // 0 .. gemm_whole-1 run whole, one workgroup each, and every later tile as
  // gemm_splits K splits (split-K for the tiles of a last, part-filled
  // dispatch round, or for every tile when gemm_whole is 0).
  int gemm_gx, gemm_whole, gemm_splits;
  // Group of a 32-k half n (n = 2 * step + half): n / gemm_gh with
  // gemm_gh = group_size / 32, computed as umulhi(n, gemm_ghinv) (ceil(2^32 /
  // gemm_gh); exact since n * gemm_gh < 2^32) or n itself when gemm_gh is 1.
  uint32_t gemm_gh, gemm_ghinv;
};

// Device-scope (sc1) buffer accesses carry partials between workgroups, which
// may sit on different XCDs whose L2s are not coherent with each other: the
// stores write through to the device coherence point and the loads bypass the
// non-coherent caches, so a split's stores only need to be acknowledged
// (s_waitcnt vmcnt(0)) before its arrival is counted.
constexpr int kSc1 = 16;                  // cache-policy bit SC1 of gfx950 buffer ops
constexpr int kBufferWord3 = 0x00020000;  // raw 32-bit buffer descriptor, word 3

// Row order of a q|k|v weight for the rotary epilogue.  Within each head of
// D rows, 16-row tile i holds dims [8i, 8i+8) then [D/2+8i, D/2+8i+8): lane
// group g of the MFMA result then holds four dims of one half and lane group
// g^2 (lane ^ 32) the four dims rotate_half pairs them with.  Row j of tile i
// is this original dim:
__host__ __device__ inline int rope_pair_dim(int i, int j, int D) {
  return (j < 8 ? 0 : D / 2) + 8 * i + (j & 7);
}

// f32 -> model dtype, from a value already rounded to f32.  The empty asm
// makes that value opaque: otherwise the backend may fold the conversion into
// the instruction that produced it (v_fma_mixlo_f16 / v_fma_mixhi_f16 round
// x·y straight to f16, skipping the f32 rounding in between), even with
// contraction off and only in some instantiations, which changed the last bit
// of dequantised weights and normalised operands between launch shapes.
template <class DT>
__device__ __forceinline__ typename DT::T to_model(float x) {
  asm("" : "+v"(x));
  return static_cast<typename DT::T>(x);
}

template <class DT>
__device__ __forceinline__ float from_model(typename DT::T x) {
  return static_cast<float>(x);
}

// Eight codes (one 32-bit word, even k in the low nibble) -> model-dtype weights.
template <class DT>
__device__ __forceinline__ typename DT::vec8 dequant8(uint32_t word, float zero, float scale) {
  typename DT::vec8 a;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float q = static_cast<float>((word >> (4 * e)) & 0xFu);
    a[e] = to_model<DT>((q - zero) * scale);
  }
  return a;
}

// dequant8 in fewer VALU operations, with the same result.  The codes of
// byte i (k = 2i, 2i+1) become the f16 pair (1024 + q) by one byte permute
// and one and-or (1024 + q is exact in f16 for q < 1024); one packed f16 add
// of `zbias` = the pair (-(1024 + z), -(1024 + z)) leaves q - z, exact (an
// integer in [-255, 15]); v_fma_mix_f32 then forms (q - z) * scale in fp32
// with one rounding (f16 operand times f32 operand, plus 0): the float32
// product of dequantize_int4, which the model-dtype conversion rounds.
__device__ __forceinline__ uint32_t zero_bias_f16x2(uint32_t zero) { return (0xE400u | zero) * 0x00010001u; }

// `magic` holds 0x64006400 in a VGPR (opaque to the compiler, so the mask
// and this constant fit one v_and_or_b32: VOP3 takes no second literal).
__device__ __forceinline__ uint32_t f16_magic_pair() {
  uint32_t m = 0x64006400u;
  asm("" : "+v"(m));
  return m;
}

template <class DT>
__device__ __forceinline__ typename DT::vec8 dequant8_mix(uint32_t word, uint32_t zbias, float scale, uint32_t magic) {
  typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
  const uint32_t hi = word >> 4;
  typename DT::vec8 a;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // bytes [byte i of word, 0, byte i of word >> 4, 0]: the low nibbles are
    // the codes of k = 2i and 2i + 1.
    const uint32_t sel = static_cast<uint32_t>(i) | 0x0C00u | (static_cast<uint32_t>(4 + i) << 16) | 0x0C000000u;
    const uint32_t t = (__builtin_amdgcn_perm(hi, word, sel) & 0x000F000Fu) | magic;
    const uint32_t d = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, t) + __builtin_bit_cast(half2_t, zbias));
    float lo, up;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(lo) : "v"(d), "v"(scale));
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(up) : "v"(d), "v"(scale));
    a[2 * i] = static_cast<typename DT::T>(lo);
    a[2 * i + 1] = static_cast<typename DT::T>(up);
  }
  return a;
}

// SiLU in float32 as torch evaluates it for half tensors: x / (1 + exp(-x)).
// Hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32: about one float32 ulp
// each) instead of the library expf and the IEEE division sequence: 5 VALU
// operations instead of about 40, which made the SwiGLU epilogue of a prefill
// gate|up tile a fifth of its workgroup's lifetime.  The float32 result stays
// within a few ulps of x / (1 + exp(-x)), far below the half-precision
// rounding that follows; -inf -> -0, +inf -> +inf and NaN -> NaN as before.
__device__ __forceinline__ float silu_f32(float x) {
  const float e = __builtin_amdgcn_exp2f(x * -1.44269504088896341f);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

template <class DT, int MT, int WAVES, int BATCH, int FT, bool NORM, bool ROPE>
__global__ __launch_bounds__(WAVES * 64) void int4_linear_kernel(Int4LinearParams p) {
  // BATCH: 128-wide chunks whose weights one wave loads at once (1 when every
  // wave has a single chunk, which keeps the register count low).
  // FT: 16-feature row tiles per workgroup (several only with one chunk per wave).
  // NORM: RMS-normalise the rows of x with p.norm_weight, in its own
  // instantiation so that its registers do not lower every projection's
  // occupancy.
  static_assert(FT == 1 || BATCH == 1, "feature tiles need one chunk per wave");
  static_assert(!NORM || BATCH == 1, "the RMSNorm runs with one chunk per wave");
  // ROPE: the epilogue rotates q and k and writes q' to out, k' and v to their
  // cache slots (the steps between the q|k|v projection and attention).
  static_assert(!ROPE || (BATCH == 1 && FT == 1), "the rotary epilogue runs one tile per workgroup");
  constexpr int NT = MT / 16;  // MFMA column tiles
  constexpr int ESZ = sizeof(typename DT::T);
  using V8 = typename DT::vec8;
  using T = typename DT::T;
  const int lane = threadIdx.x & 63;
  // Uniform per wave: the chunk split below then branches on scalars, and
  // the compiler does not treat the batch paths as divergent (which made it
  // wait for every load in flight where they join).
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int n0 = blockIdx.x * 16 * FT;
  const int m0 = blockIdx.y * MT;
  const int row = lane & 15;  // A row (feature) / B column (token) of this lane
  const int grp = lane >> 4;  // lane group: k-slots 8*grp .. +7 of an MFMA step
  // First of the four output features this lane ends with, in row tile f: n0 + 16f + 4grp.
  const int nf = n0 + 4 * grp;

  // The epilogue's inputs are fetched first so their latency hides behind the
  // K loop.  They stay in the model dtype until the epilogue: converting them
  // here would make the wave wait for them before issuing any weight load.
  T bias_raw[FT][4];
  typename DT::vec4 resid_raw[FT][NT];
#pragma unroll
  for (int f = 0; f < FT; ++f) {
#pragma unroll
    for (int r = 0; r < 4; ++r) bias_raw[f][r] = T(0.f);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) resid_raw[f][t][r] = T(0.f);
  }
  // Rotary epilogue operands (wave 0 runs the epilogue): this lane's four
  // dims (one half of a rotary pair) of the tile's head, their cos/sin
  // entries per token tile, and the tokens' cache slots.
  int head = 0, dim0 = 0;
  typename DT::vec4 cos_raw[NT], sin_raw[NT];
  int64_t slot[NT];
  if constexpr (ROPE) {
    const int tiles_per_head = p.head_dim / 16;
    head = blockIdx.x / tiles_per_head;
    dim0 = rope_pair_dim(blockIdx.x % tiles_per_head, 4 * grp, p.head_dim);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (wave != 0) break;
      const int m = min(m0 + 16 * t + row, p.M - 1);
      const T* cp = static_cast<const T*>(p.cos) + static_cast<int64_t>(m) * p.cs_stride + dim0;
      const T* sp = static_cast<const T*>(p.sin) + static_cast<int64_t>(m) * p.cs_stride + dim0;
      cos_raw[t] = *reinterpret_cast<const typename DT::vec4*>(cp);
      sin_raw[t] = *reinterpret_cast<const typename DT::vec4*>(sp);
      slot[t] = p.slots64 ? static_cast<const int64_t*>(p.slots)[m]
                          : static_cast<int64_t>(static_cast<const int32_t*>(p.slots)[m]);
    }
  }
  if (wave == 0) {
#pragma unroll
    for (int f = 0; f < FT; ++f) {
      if (p.bias) {
        const T* bp = static_cast<const T*>(p.bias) + nf + 16 * f;
#pragma unroll
        for (int r = 0; r < 4; ++r) bias_raw[f][r] = bp[r];
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int m = m0 + 16 * t + row;
        if (p.epilogue == NS_EPILOGUE_RESIDUAL && m < p.M)
          resid_raw[f][t] = *reinterpret_cast<const typename DT::vec4*>(
              static_cast<const T*>(p.residual) + static_cast<int64_t>(m) * p.N + nf + 16 * f);
      }
    }
  }

  const uint8_t* wrow[FT];
  const float* srow[FT];
  const uint8_t* zrow[FT];
#pragma unroll
  for (int f = 0; f < FT; ++f) {
    const int n = n0 + 16 * f + row;
    wrow[f] = p.qweight + static_cast<int64_t>(n) * (p.K / 2);
    srow[f] = p.scales + static_cast<int64_t>(n) * p.groups;
    zrow[f] = p.zeros + static_cast<int64_t>(n) * p.groups;
  }
  const char* xrow[NT];
  bool xok[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int m = m0 + 16 * t + row;
    xok[t] = m < p.M;
    xrow[t] = p.x + static_cast<int64_t>(xok[t] ? m : 0) * p.x_stride * ESZ;
  }

  floatx4 acc[FT][NT];
#pragma unroll
  for (int f = 0; f < FT; ++f)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[f][t] = floatx4{0.f, 0.f, 0.f, 0.f};

  // NORM: rms_norm(x) = x * rstd(x) * w with rstd = rsqrt(mean(x^2) + eps)
  // per row, so W·rms_norm(x) = rstd(x) * (W·(x * w)).  Each wave (one
  // 128-wide chunk of K, the host guarantees) multiplies its x operands by
  // the norm weight as they arrive, rounding x * w to the model dtype once,
  // and adds up its slice of the rows' sums of squares in fp32; the sums meet
  // in wave 0 with the partial products, which scales the accumulators by
  // rstd before the epilogue.  No barrier stands between the loads and the
  // MFMAs.  Against normalising first (torch's rms_norm rounds x * rstd * w
  // once) an operand rounds at the same relative precision.
  float ss[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) ss[t] = 0.f;
  if constexpr (NORM) {
    const int kb = 128 * wave + 32 * grp;
    const int gi = kb / p.group_size;
    u32x4 codes[FT];
    float scale[FT];
    uint32_t zq[FT];  // converted after the x loads are issued
#pragma unroll
    for (int f = 0; f < FT; ++f) {
      codes[f] = *reinterpret_cast<const u32x4*>(wrow[f] + kb / 2);
      scale[f] = srow[f][gi];
      zq[f] = zrow[f][gi];
    }
    V8 b[4][NT], nw[4];
    // Rows past M read row 0 (unconditional loads, no wait between them);
    // their sums and products only reach outputs that are never stored.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      nw[j] = load16<DT>(static_cast<const char*>(p.norm_weight) + (kb + 8 * j) * ESZ);
#pragma unroll
      for (int t = 0; t < NT; ++t) b[j][t] = load16<DT>(xrow[t] + (kb + 8 * j) * ESZ);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float v = static_cast<float>(b[j][t][e]);
          ss[t] = __builtin_fmaf(v, v, ss[t]);
          b[j][t][e] = to_model<DT>(v * static_cast<float>(nw[j][e]));
        }
#pragma unroll
    for (int f = 0; f < FT; ++f) {
      const float zero = static_cast<float>(zq[f]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const V8 a = dequant8<DT>(codes[f][j], zero, scale[f]);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[f][t] = mfma16x16x32(DT{}, a, b[j][t], acc[f][t]);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      ss[t] += __shfl_xor(ss[t], 16);  // the four lane groups holding this row
      ss[t] += __shfl_xor(ss[t], 32);
    }
  }

  // Whole 128-wide chunks, split between the waves.  The NORM block above has
  // done them all when NORM is set.  Otherwise p.norm_weight is null, and testing
  // it at run time keeps the compiler from deriving the chunk count and the
  // tail steps from K together: with `NORM ? 0 : p.K / 128` the 7-wave kernel
  // needed 74 VGPRs instead of 52 (two feature tiles: 128 instead of 77).
  const bool normed = NORM || p.norm_weight != nullptr;
  const int chunks = normed ? 0 : p.K / 128;
  // Split z of gridDim.z takes chunks [chunks·z/S, chunks·(z+1)/S) (S = 1
  // unless the host asked for split-K); its waves divide them.
  const int S = static_cast<int>(gridDim.z), z = static_cast<int>(blockIdx.z);
  const int cz0 = (chunks * z) / S, czn = (chunks * (z + 1)) / S - cz0;
  const int c_beg = cz0 + (czn * wave) / WAVES;
  const int c_end = cz0 + (czn * (wave + 1)) / WAVES;
  if constexpr (BATCH == 1) {
    // One chunk per wave (K up to 8 chunks): the chunk's codes, scale, zero
    // point and x operands are all issued before any of them is used, so the
    // wave makes one memory round trip.  The zero point stays a raw byte
    // until then (converting it at its load made the wave wait for that
    // load before issuing the next), and rows past M read row 0, whose
    // products only reach outputs that are never stored (no branch, so no
    // wait, between loads).
    for (int c = c_beg; c < c_end; ++c) {
      const int kb = 128 * c + 32 * grp;
      const int gi = kb / p.group_size;
      u32x4 codes[FT];
      float scale[FT];
      uint32_t zq[FT];
#pragma unroll
      for (int f = 0; f < FT; ++f) {
        codes[f] = *reinterpret_cast<const u32x4*>(wrow[f] + kb / 2);
        scale[f] = srow[f][gi];
        zq[f] = zrow[f][gi];
      }
      V8 b[4][NT];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int t = 0; t < NT; ++t) b[j][t] = load16<DT>(xrow[t] + (kb + 8 * j) * ESZ);
      // Loads complete in order: keep them all ahead of the arithmetic.
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int f = 0; f < FT; ++f) {
        const float zero = static_cast<float>(zq[f]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const V8 a = dequant8<DT>(codes[f][j], zero, scale[f]);
#pragma unroll
          for (int t = 0; t < NT; ++t) acc[f][t] = mfma16x16x32(DT{}, a, b[j][t], acc[f][t]);
        }
      }
    }
  } else {
    // Several chunks per wave (down_proj's K = 4864): the codes, scales and
    // zero points of up to BATCH chunks are fetched first, the x operands
    // chunk by chunk.  Issuing every chunk's x at once measured slower
    // (M = 16..64: 8.4 -> 12.3 us): a 16-row load uses half of each line it
    // touches, and with all chunks in flight the lines leave L1 before the
    // load that uses their other half.
    for (int c0 = c_beg; c0 < c_end; c0 += BATCH) {
      const int nb = c_end - c0 < BATCH ? c_end - c0 : BATCH;
      u32x4 codes[BATCH];
      float scale[BATCH], zero[BATCH];
#pragma unroll
      for (int i = 0; i < BATCH; ++i) {
        if (i < nb) {
          const int kb = 128 * (c0 + i) + 32 * grp;
          codes[i] = *reinterpret_cast<const u32x4*>(wrow[0] + kb / 2);
          const int gi = kb / p.group_size;
          scale[i] = srow[0][gi];
          zero[i] = static_cast<float>(zrow[0][gi]);
        }
      }
#pragma unroll
      for (int i = 0; i < BATCH; ++i) {
        if (i < nb) {
          const int kb = 128 * (c0 + i) + 32 * grp;
          V8 b[4][NT];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
              b[j][t] = xok[t] ? load16<DT>(xrow[t] + (kb + 8 * j) * ESZ) : zero8<DT>();
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const V8 a = dequant8<DT>(codes[i][j], zero[i], scale[i]);
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[0][t] = mfma16x16x32(DT{}, a, b[j][t], acc[0][t]);
          }
        }
      }
    }
  }
  // Remaining 32-wide steps when K is not a multiple of 128.
  for (int s = normed || z != S - 1 ? p.K / 32 : 4 * chunks + wave; s < p.K / 32; s += WAVES) {
    const int k = 32 * s + 8 * grp;
    const int gi = k / p.group_size;
    V8 b[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) b[t] = xok[t] ? load16<DT>(xrow[t] + k * ESZ) : zero8<DT>();
#pragma unroll
    for (int f = 0; f < FT; ++f) {
      const uint32_t word = *reinterpret_cast<const uint32_t*>(wrow[f] + k / 2);
      const V8 a = dequant8<DT>(word, static_cast<float>(zrow[f][gi]), srow[f][gi]);
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[f][t] = mfma16x16x32(DT{}, a, b[t], acc[f][t]);
    }
  }

  // Waves 1.. hand their partial sums (and, with NORM, their slices of the
  // rows' sums of squares) to wave 0.
  if constexpr (WAVES > 1) {
    __shared__ floatx4 red[WAVES - 1][FT][NT][64];
    __shared__ float nss[NORM ? WAVES - 1 : 1][NT][16];
    if (wave > 0) {
#pragma unroll
      for (int f = 0; f < FT; ++f)
#pragma unroll
        for (int t = 0; t < NT; ++t) red[wave - 1][f][t][lane] = acc[f][t];
      if constexpr (NORM) {
        if (grp == 0) {
#pragma unroll
          for (int t = 0; t < NT; ++t) nss[wave - 1][t][row] = ss[t];
        }
      }
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int f = 0; f < FT; ++f)
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int w = 0; w < WAVES - 1; ++w) acc[f][t] += red[w][f][t][lane];
      }
    if constexpr (NORM) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int w = 0; w < WAVES - 1; ++w) ss[t] += nss[w][t][row];
    }
  }
  if constexpr (NORM) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float rstd = rsqrtf(ss[t] / static_cast<float>(p.K) + p.norm_eps);
#pragma unroll
      for (int f = 0; f < FT; ++f) acc[f][t] *= rstd;
    }
  }

  if constexpr (BATCH > 1) {
    if (S > 1) {
      // Publish this split's sums, count the arrival; the last split of the
      // tile adds all S partials in split order (its own included, so the
      // result does not depend on which split came last) and resets the counter.
      const int tile = static_cast<int>(blockIdx.y * gridDim.x + blockIdx.x);
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc(p.part, static_cast<short>(0), p.part_bytes, kBufferWord3);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[0][t]), rs,
                                               (((tile * S + z) * NT + t) * 64 + lane) * 16, 0, kSc1);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the partial stores are acknowledged
      unsigned prev = 0;
      if (lane == 0) prev = __hip_atomic_fetch_add(&p.counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      prev = __shfl(prev, 0);
      if (prev != static_cast<unsigned>(S - 1)) return;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        floatx4 sum = {0.f, 0.f, 0.f, 0.f};
        for (int zz = 0; zz < S; ++zz) {
          const int off = (((tile * S + zz) * NT + t) * 64 + lane) * 16;
          floatx4 v;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            v[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off + 4 * r, 0, kSc1));
          sum += v;
        }
        acc[0][t] = sum;
      }
      if (lane == 0) __hip_atomic_store(&p.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // D[4·(lane/16) + r][lane%16] of row tile f: features nf+16f .. +3 of token
  // m.  Each epilogue rounds where the reference's separate tensor ops round.
  if constexpr (ROPE) {
    // y = round(acc + bias) is the projection's output (q, k or v of this
    // head); q and k then rotate as RotaryEmbedding.apply rounds it,
    //   first half:  round(round(x1*cos) - round(x2*sin)),
    //   second half: round(round(x2*cos) + round(x1*sin)),
    // with x1/x2 the dims of the pair in the first/second half, held by this
    // lane and by lane ^ 32 (same token row, so the exchange happens before
    // any row check, with every lane of the wave active).
    const bool second = grp >= 2;
    const int Hq = p.num_heads, Hkv = p.num_kv_heads, D = p.head_dim;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int m = m0 + 16 * t + row;
      float y[4], yp[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        y[r] = from_model<DT>(to_model<DT>(acc[0][t][r] + from_model<DT>(bias_raw[0][r])));
        yp[r] = __shfl_xor(y[r], 32);
      }
      if (m >= p.M) continue;
      typename DT::vec4 o;
      if (head < Hq + Hkv) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float c = from_model<DT>(cos_raw[t][r]), sn = from_model<DT>(sin_raw[t][r]);
          const float a = from_model<DT>(to_model<DT>(y[r] * c));
          const float b = from_model<DT>(to_model<DT>(yp[r] * sn));
          o[r] = to_model<DT>(second ? a + b : a - b);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = to_model<DT>(y[r]);
      }
      T* dst;
      if (head < Hq) {
        dst = static_cast<T*>(p.out) + (static_cast<int64_t>(m) * Hq + head) * D;
      } else {
        if (slot[t] < 0 || slot[t] >= p.num_slots) continue;  // padding / invalid slot: never written
        const int kvh = head < Hq + Hkv ? head - Hq : head - Hq - Hkv;
        T* cache = static_cast<T*>(head < Hq + Hkv ? p.k_cache : p.v_cache);
        dst = cache + (slot[t] * Hkv + kvh) * D;
      }
      *reinterpret_cast<typename DT::vec4*>(dst + dim0) = o;
    }
    return;
  }
#pragma unroll
  for (int f = 0; f < FT; ++f) {
    const int nff = nf + 16 * f;
    float bias[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) bias[r] = from_model<DT>(bias_raw[f][r]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int m = m0 + 16 * t + row;
      if (m >= p.M) continue;
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = from_model<DT>(to_model<DT>(acc[f][t][r] + bias[r]));
      if (p.epilogue == NS_EPILOGUE_SILU_MUL) {
        // Rows (nff, nff+1) and (nff+2, nff+3) are (gate, up) pairs of outputs nff/2, nff/2+1.
        typename DT::T o[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float act = from_model<DT>(to_model<DT>(silu_f32(y[2 * h])));
          o[h] = to_model<DT>(act * y[2 * h + 1]);
        }
        T* dst = static_cast<T*>(p.out) + static_cast<int64_t>(m) * (p.N / 2) + nff / 2;
        dst[0] = o[0];
        dst[1] = o[1];
        continue;
      }
      typename DT::vec4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = to_model<DT>(y[r] + from_model<DT>(resid_raw[f][t][r]));
      *reinterpret_cast<typename DT::vec4*>(static_cast<T*>(p.out) + static_cast<int64_t>(m) * p.N + nff) = o;
    }
  }
}

// Launch shape.  K of up to 2048 (Qwen2.5-0.5B: 896) gets one wave per
// 128-wide chunk, up to 8 waves, each with a single chunk (few registers, so
// many waves fit per SIMD).  Longer K (down_proj's 4864 = 38 chunks) gets 16
// waves per 16-token tile (8 per 64-token tile) that each fetch up to four
// chunks at once.  Single-chunk waves take two feature tiles per workgroup
// when the token tile holds at least 16 rows and the grid keeps at least 256
// workgroups: each x operand then feeds two MFMAs, and the grid holds half as
// many waves re-reading the token tile's x rows.  Measured on MI355X for
// gate|up (N = 9728, K = 896), graph-replayed: 5.53 -> 5.34 us at 16 tokens,
// 7.82 -> 7.39 at 32, 13.49 -> 11.19 at 64; at 8 tokens there is little x to
// share and the halved grid is slower (4.67 -> 5.01 us), and four feature
// tiles are slower than two at 32 and 64 tokens.
struct Shape {
  int waves;
  int batch;
  int ft;
};

Shape shape_for(int M, int N, int K, int mt, int mtiles) {
  const int chunks = K / 128;
  if (chunks >= 1 && chunks <= 8) {
    // (64-token tiles with two feature tiles would spill: 256 VGPRs.)
    const bool two = mt == 16 && M >= 16 && N % 32 == 0 && static_cast<int64_t>(N / 32) * mtiles >= 256;
    return {chunks, 1, two ? 2 : 1};
  }
  if (K <= 2048) return {8, 4, 1};
  return {mt <= 16 ? 16 : 8, 4, 1};
}

template <class DT, int MT, int FT, bool NORM, bool ROPE = false>
const void* one_chunk_kernel(int waves) {
  switch (waves) {
    case 1: return reinterpret_cast<const void*>(&int4_linear_kernel<DT, MT, 1, 1, FT, NORM, ROPE>);
    case 2: return reinterpret_cast<const void*>(&int4_linear_kernel<DT, MT, 2, 1, FT, NORM, ROPE>);
    case 3: return reinterpret_cast<const void*>(&int4_linear_kernel<DT, MT, 3, 1, FT, NORM, ROPE>);
    case 4: return reinterpret_cast<const void*>(&int4_linear_kernel<DT, MT, 4, 1, FT, NORM, ROPE>);
    case 5: return reinterpret_cast<const void*>(&int4_linear_kernel<DT, MT, 5, 1, FT, NORM, ROPE>);
    case 6: return reinterpret_cast<const void*>(&int4_linear_kernel<DT, MT, 6, 1, FT, NORM, ROPE>);
    case 7: return reinterpret_cast<const void*>(&int4_linear_kernel<DT, MT, 7, 1, FT, NORM, ROPE>);
    default: return reinterpret_cast<const void*>(&int4_linear_kernel<DT, MT, 8, 1, FT, NORM, ROPE>);
  }
}

template <class DT, int MT>
const void* kernel_for(Shape sh, bool norm) {
  if (sh.batch == 1) {
    if constexpr (MT == 16) {
      if (sh.ft == 2) return norm ? one_chunk_kernel<DT, MT, 2, true>(sh.waves) : one_chunk_kernel<DT, MT, 2, false>(sh.waves);
    }
    return norm ? one_chunk_kernel<DT, MT, 1, true>(sh.waves) : one_chunk_kernel<DT, MT, 1, false>(sh.waves);
  }
  if constexpr (MT <= 16) {
    if (sh.waves == 16) return reinterpret_cast<const void*>(&int4_linear_kernel<DT, MT, 16, 4, 1, false, false>);
  }
  return reinterpret_cast<const void*>(&int4_linear_kernel<DT, MT, 8, 4, 1, false, false>);
}

template <class DT>
hipError_t launch_int4_linear_rope(const Int4LinearParams& p, hipStream_t stream) {
  void* args[] = {const_cast<Int4LinearParams*>(&p)};
  const int mt = p.M <= 64 ? 16 : 64;
  const int waves = p.K / 128;  // the caller checked 1..8 whole chunks
  const bool norm = p.norm_weight != nullptr;
  const void* fn = mt == 16 ? (norm ? one_chunk_kernel<DT, 16, 1, true, true>(waves)
                                    : one_chunk_kernel<DT, 16, 1, false, true>(waves))
                            : (norm ? one_chunk_kernel<DT, 64, 1, true, true>(waves)
                                    : one_chunk_kernel<DT, 64, 1, false, true>(waves));
  const dim3 grid(static_cast<unsigned>(p.N / 16), static_cast<unsigned>((p.M + mt - 1) / mt));
  return hipLaunchKernel(fn, grid, dim3(64 * waves), args, 0, stream);
}

// Split-K for the multi-chunk kernels: few workgroups (down_proj: N = 896 is
// 56 tiles of 16 features per token tile) each walking 38 chunks leave most
// CUs idle, so each tile's chunks are split over up to 4 workgroups while the
// grid stays within one workgroup per CU (a 16-wave workgroup fills one).
// Measured on MI355X for down_proj + residual, graph-replayed: 8 / 16 tokens
// 7.16 / 8.50 -> 6.62 / 6.99 us with 4 splits; 4 splits at 32 and 64 tokens
// (448 and 896 workgroups, two dispatch rounds) were slower, 8.61 / 8.88 ->
// 9.24 / 12.42 us.
int splitk_for(int N, int K, int64_t mtiles) {
  const int chunks = K / 128;
  if (chunks <= 8 || K <= 2048) return 1;
  const int64_t tiles = static_cast<int64_t>(N / 16) * mtiles;
  return 4 * tiles <= 256 ? 4 : 2 * tiles <= 256 ? 2 : 1;
}

template <class DT>
hipError_t launch_int4_linear(const Int4LinearParams& p, hipStream_t stream, int splits = 1) {
  void* args[] = {const_cast<Int4LinearParams*>(&p)};
  // Up to 64 tokens, 16-token tiles (grid.y tiles side by side) beat wider
  // ones: more waves in flight and fewer registers each (measured on MI355X,
  // M = 32: down_proj 12.9 -> 8.5 us, qkv 4.1 -> 3.3 us).  Beyond that, 64-token
  // tiles amortise the dequantisation over more MFMAs.
  const int mt = p.M <= 64 ? 16 : 64;
  const int mtiles = (p.M + mt - 1) / mt;
  const bool norm = p.norm_weight != nullptr;
  const Shape sh = shape_for(p.M, p.N, p.K, mt, mtiles);
  const void* fn = mt == 16 ? kernel_for<DT, 16>(sh, norm) : kernel_for<DT, 64>(sh, norm);
  const dim3 grid(static_cast<unsigned>(p.N / (16 * sh.ft)), static_cast<unsigned>(mtiles),
                  static_cast<unsigned>(sh.batch > 1 ? splits : 1));
  return hipLaunchKernel(fn, grid, dim3(64 * sh.waves), args, 0, stream);
}

bool aligned(const void* q, uintptr_t a) { return reinterpret_cast<uintptr_t>(q) % a == 0; }

// --------------------------------------------------------------------------
// Token counts of prefill chunks (M above kGemmMinRows): a tiled GEMM whose
// waves dequantise weight codes in registers, straight into the MFMA operand
// layout, and reuse each dequantised fragment over many tokens.  The fused
// kernel above dequantises a weight tile once per 16- or 64-token tile, which
// at prefill sizes makes the dequantisation, not the MFMA, its bound.
//
// Workgroup: 4 waves, BN features x BM tokens; WN waves side by side along
// the features and 4/WN along the tokens, wave (wn, wm) computing WF features
// x WT tokens as MFMA 16x16x32 tiles (A = W rows, B = x^T), so a lane ends
// with four consecutive features of one token, as in the fused kernel, and
// the epilogues are the same.  Each 64-wide K step's x tile, weight codes,
// scales and zero-point words go from HBM into LDS by global_load_lds
// through a ring of NST stages.  Within a step, lane group g of the MFMA
// operands carries k = 16g + 8j .. +7 in sub-step j (a permutation of the 64
// k, the same for both operands), so a lane's two sub-steps of one weight
// row are one 8-byte word pair of codes.  The lane dequantises them with
// dequantize_int4's arithmetic (quant.py:83-95) one step ahead of the MFMAs
// that use them (software pipeline: step s+1's dequantisation and step s's
// MFMAs are independent work in one block).  x rows in LDS are 128 bytes
// with 16-byte unit c of row r at c ^ ((r >> 1) & 7), and code rows swap
// their 16-byte halves when bit 3 of the row is set, so the operand reads of
// a wave meet every bank once.  Every wait for the ring is an explicit vmcnt
// (the loads are issued from asm, invisible to the compiler's wait-count
// pass).
//
// Split-K (tiles past gemm_whole, S = gemm_splits > 1): split z walks steps
// [z*steps/S, (z+1)*steps/S), publishes its fp32 partial tile to the
// workspace and counts its arrival; the last split of the tile adds all S
// partials in split order and applies the epilogue.  The split tiles come
// last in the grid, so when the whole tiles fill the device for some rounds
// the splits share out the last round's tiles over its otherwise idle slots.
// --------------------------------------------------------------------------
constexpr int64_t kGemmMinRows = 128;  // the fused kernel takes M up to here
namespace gemm {
constexpr int BK = 64;
constexpr int WAVES = 4, THREADS = WAVES * 64;
constexpr int ROW_B = BK * 2;  // one LDS row of x: 64 k in the model dtype
// BM tokens x BN features per workgroup; NST stages in the load ring; WN
// waves side by side along the features (4 / WN along the tokens).
template <int BM, int BN, int NST, int WN>
struct Cfg {
  static constexpr int X_B = BM * ROW_B;       // x tile of a stage
  static constexpr int C_B = BN * BK / 2;      // weight codes of a stage (32 bytes a row)
  static constexpr int SZ_B = BN * 4;          // a scale (or zero-point word) per row
  static constexpr int STAGE_B = X_B + C_B + 2 * SZ_B;
  static constexpr int LDS = NST * STAGE_B;
  static constexpr int X_DMA = X_B / 1024 / WAVES;  // 16-byte global_load_lds per wave
  // Besides its x loads, each wave takes an equal share of the stage's other
  // loads: the code loads (1 KiB each), then the scale loads and then the
  // zero-point loads (64 rows each).  No load repeats another.
  static constexpr int CODE_L = C_B / 1024, SZ_L = BN / 64;
  static constexpr int EXTRA = (CODE_L + 2 * SZ_L) / WAVES;
  static constexpr int PS = X_DMA + EXTRA;  // loads per wave and step
  static constexpr int WM = WAVES / WN;
  static constexpr int WF = BN / WN, WT = BM / WM;  // features and tokens of one wave
  static constexpr int FT = WF / 16, TT = WT / 16;  // 16-row MFMA tiles per wave: features, tokens
  static_assert(X_B % (1024 * WAVES) == 0 && C_B % 1024 == 0 && BN % 64 == 0, "whole loads per wave");
  static_assert((CODE_L + 2 * SZ_L) % WAVES == 0, "the waves share the code, scale and zero loads evenly");
  static_assert(NST >= 3, "the loop dequantises one step ahead of its MFMAs");
  static_assert(LDS <= 80 * 1024, "two workgroups fit one CU's LDS");
};
// Split-K: at most this many tiles split (their arrival counters lie at the
// start of the workspace).
constexpr int kMaxSplitTiles = 256;
}  // namespace gemm

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <class DT, int BM, int BN, int NST, int WN>
__global__ __launch_bounds__(gemm::THREADS, 2) void int4_gemm_kernel(Int4LinearParams p) {
  using namespace gemm;
  using C = Cfg<BM, BN, NST, WN>;
  using T = typename DT::T;
  using V8 = typename DT::vec8;
  using V4 = typename DT::vec4;
  constexpr int ESZ = sizeof(T);
  constexpr int TT = C::TT, FT = C::FT;
  __shared__ __attribute__((aligned(16))) char smem[C::LDS];
  auto xst = [&](int st) { return smem + st * C::STAGE_B; };
  auto cst = [&](int st) { return smem + st * C::STAGE_B + C::X_B; };
  auto sst = [&](int st) { return smem + st * C::STAGE_B + C::X_B + C::C_B; };
  auto zst = [&](int st) { return smem + st * C::STAGE_B + C::X_B + C::C_B + C::SZ_B; };

  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = w % WN, wm = w / WN;
  // Grid: work unit b is tile t = (token tile t / gx, feature tile t % gx),
  // so consecutive units share one x row block.  Unit b < gemm_whole takes
  // tile b whole; the rest take split z of tile gemm_whole + st, unit
  // gemm_whole + z * split_tiles + st, so one round of splits covers every
  // split tile.  The dispatcher deals workgroup i to XCD i % 8; workgroup i
  // takes unit b from a contiguous eighth of the units per XCD, so the
  // workgroups of one XCD share x row blocks in that XCD's L2 (down_proj at
  // 1024 tokens 34.4 -> 32.7 us, o_proj at 2048 14.7 -> 13.7 us on MI355X).
  const int gx = p.gemm_gx;
  const int b = [] {
    const int units = gridDim.x, q = units >> 3, r = units & 7, xcd = blockIdx.x & 7;
    return xcd * q + min(xcd, r) + static_cast<int>(blockIdx.x >> 3);
  }();
  const int split_tiles = ((p.M + BM - 1) / BM) * gx - p.gemm_whole;
  int S = 1, z = 0, st = 0, tile = b;
  if (b >= p.gemm_whole) {
    S = p.gemm_splits;
    st = (b - p.gemm_whole) % split_tiles;
    z = (b - p.gemm_whole) / split_tiles;
    tile = p.gemm_whole + st;
  }
  const int n0 = (tile % gx) * BN, m0 = (tile / gx) * BM;
  const int steps = p.K / BK;
  const int s0 = z * steps / S, s1 = (z + 1) * steps / S;

  // Loader roles of this lane (rows past M or N repeat the last one, never
  // stored).  Each load is a uniform base, moved along K per step in scalar
  // registers, plus a per-lane 32-bit byte offset fixed for the whole loop
  // (the host takes this kernel only when every offset fits).  LDS layouts:
  // 16-byte unit c of x row r sits at unit c ^ ((r >> 1) & 7) and the two
  // 16-byte halves of code row r are swapped when bit 3 of r is set, so the
  // operand reads of a wave (16 consecutive rows per quarter-wave) meet every
  // bank once.
  uint32_t xoff[C::X_DMA];
#pragma unroll
  for (int u = 0; u < C::X_DMA; ++u) {
    const int unit = (w * C::X_DMA + u) * 64 + lane;
    const int row = unit >> 3, pos = unit & 7;
    const int m = min(m0 + row, p.M - 1);
    xoff[u] = static_cast<uint32_t>((static_cast<int64_t>(m) * p.x_stride + 8 * (pos ^ ((row >> 1) & 7))) * ESZ);
  }
  // This wave's other loads: load e = w * EXTRA + j is code load e (16-byte
  // unit 64e + lane: row u / 2, LDS half u & 1), or scale / zero-point load
  // e - CODE_L (- SZ_L) of row 64 (e - ...) + lane.  The per-lane part of each
  // address is fixed over the loop.
  int ekind[C::EXTRA];  // 0 code, 1 scale, 2 zero point (uniform)
  uint32_t eoff[C::EXTRA], edst[C::EXTRA];
#pragma unroll
  for (int j = 0; j < C::EXTRA; ++j) {
    const int e = w * C::EXTRA + j;
    if (e < C::CODE_L) {
      const int cu = e * 64 + lane;
      ekind[j] = 0;
      eoff[j] = static_cast<uint32_t>(min(n0 + (cu >> 1), p.N - 1)) * static_cast<uint32_t>(p.K / 2) +
                16u * ((cu & 1) ^ ((cu >> 4) & 1));
      edst[j] = e * 1024;
    } else {
      const int k = e - C::CODE_L, kind = k < C::SZ_L ? 1 : 2, r = (k % C::SZ_L) * 64;
      ekind[j] = kind;
      eoff[j] = static_cast<uint32_t>(min(n0 + r + lane, p.N - 1)) * static_cast<uint32_t>(p.groups) *
                (kind == 1 ? 4u : 1u);
      edst[j] = r * 4;
    }
  }
  // This lane's operand rows: features WF wn + 16 fi + c16 of the tile; the
  // zero-point byte of group gi sits at byte (zrow + gi) & 3 of its word.
  uint32_t zrow[FT];
#pragma unroll
  for (int fi = 0; fi < FT; ++fi)
    zrow[fi] = static_cast<uint32_t>(min(n0 + C::WF * wn + 16 * fi + c16, p.N - 1)) * static_cast<uint32_t>(p.groups);
  auto group_of = [&](int n) -> int {
    return p.gemm_gh == 1 ? n : static_cast<int>(__umulhi(static_cast<uint32_t>(n), p.gemm_ghinv));
  };

  auto dma = [&](int s, int st) {
    const char* xs = p.x + static_cast<int64_t>(BK * ESZ) * s;
#pragma unroll
    for (int u = 0; u < C::X_DMA; ++u) dma_lds16_off(xs, xoff[u], xst(st) + (w * C::X_DMA + u) * 1024);
    const uint32_t gi = static_cast<uint32_t>(group_of(2 * s));
#pragma unroll
    for (int j = 0; j < C::EXTRA; ++j) {
      if (ekind[j] == 0)
        dma_lds16_off(p.qweight + (BK / 2) * s, eoff[j], cst(st) + edst[j]);
      else if (ekind[j] == 1)
        dma_lds4_off(p.scales + gi, eoff[j], sst(st) + edst[j]);
      else  // the aligned word holding the zero point (inside the table: N * groups is a multiple of 16)
        dma_lds4_off(p.zeros, (eoff[j] + gi) & ~3u, zst(st) + edst[j]);
    }
  };

  floatx4 acc[FT][TT];
#pragma unroll
  for (int fi = 0; fi < FT; ++fi)
#pragma unroll
    for (int ti = 0; ti < TT; ++ti) acc[fi][ti] = floatx4{0.f, 0.f, 0.f, 0.f};
  const uint32_t magic = f16_magic_pair();

  auto stage = [&](int s) { return (s - s0) % NST; };
  // Wait until at most n whole steps of this wave's loads are in flight.
  auto wait_steps = [&](int n) {
    if (n >= 2) wait_vm<2 * C::PS>();
    else if (n == 1) wait_vm<C::PS>();
    else wait_vm<0>();
  };
  // The A operands of step s: this lane's codes of rows WF wn + 16 fi + c16,
  // k of the step in one group per lane, dequantised into both sub-steps.
  auto dequant_step = [&](int s, V8 (&a)[FT][2]) {
    const int st = stage(s);
    const uint32_t gi = static_cast<uint32_t>(group_of(2 * s));  // both halves of a step share a group
#pragma unroll
    for (int fi = 0; fi < FT; ++fi) {
      const int r = C::WF * wn + 16 * fi + c16;
      const u32x2 words =
          *reinterpret_cast<const u32x2*>(cst(st) + 32 * r + 16 * ((g >> 1) ^ ((r >> 3) & 1)) + 8 * (g & 1));
      const float scale = *reinterpret_cast<const float*>(sst(st) + 4 * r);
      const uint32_t zword = *reinterpret_cast<const uint32_t*>(zst(st) + 4 * r);
      const uint32_t zb = zero_bias_f16x2((zword >> (8 * ((zrow[fi] + gi) & 3u))) & 0xFFu);
      a[fi][0] = dequant8_mix<DT>(words[0], zb, scale, magic);
      a[fi][1] = dequant8_mix<DT>(words[1], zb, scale, magic);
    }
  };
  // The MFMAs of step s: A from registers, B (x rows of this wave's tokens)
  // read from the step's stage as each token tile's turn comes.
  auto mfma_step = [&](int s, const V8 (&a)[FT][2]) {
    const char* xt = xst(stage(s));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int ti = 0; ti < TT; ++ti) {
        const int row = C::WT * wm + 16 * ti + c16;
        const V8 b = *reinterpret_cast<const V8*>(xt + row * ROW_B + (((2 * g + j) ^ ((row >> 1) & 7)) << 4));
#pragma unroll
        for (int fi = 0; fi < FT; ++fi) acc[fi][ti] = mfma16x16x32(DT{}, a[fi][j], b, acc[fi][ti]);
      }
    }
  };

  // Software pipeline: iteration s dequantises step s+1 while the MFMAs of
  // step s run (independent work in one block, so the two interleave), with
  // the loads of up to NST-2 later steps in flight.
#pragma unroll
  for (int k = 0; k < NST - 1; ++k)
    if (s0 + k < s1) dma(s0 + k, k);
  wait_steps(min(s1 - 1 - s0, NST - 2));
  __syncthreads();
  V8 acur[FT][2];
  dequant_step(s0, acur);
  for (int s = s0; s < s1 - 1; ++s) {
    // Step s+1's loads have landed (those up to step s+NST-2 may fly); past
    // the barrier every wave is done with step s-1, whose stage takes step
    // s+NST-1.
    wait_steps(min(s1 - 1, s + NST - 2) - (s + 1));
    __syncthreads();
    if (s + NST - 1 < s1) dma(s + NST - 1, stage(s + NST - 1));
    V8 anext[FT][2];
    dequant_step(s + 1, anext);
    mfma_step(s, acur);
#pragma unroll
    for (int fi = 0; fi < FT; ++fi) {
      acur[fi][0] = anext[fi][0];
      acur[fi][1] = anext[fi][1];
    }
  }
  mfma_step(s1 - 1, acur);

  if (S > 1) {
    // Publish this split's sums, count the arrival; the last split of the
    // tile adds all S partials in split order (its own included, so the
    // result does not depend on which split came last) and resets the counter.
    __shared__ unsigned last_arrival;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(p.part, static_cast<short>(0), p.part_bytes, kBufferWord3);
    auto off = [&](int zz, int fi, int ti) { return ((((st * S + zz) * WAVES + w) * FT + fi) * TT + ti) * 1024 + lane * 16; };
#pragma unroll
    for (int fi = 0; fi < FT; ++fi)
#pragma unroll
      for (int ti = 0; ti < TT; ++ti)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[fi][ti]), rs, off(z, fi, ti), 0, kSc1);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the partial stores are acknowledged
    __syncthreads();                     // ... by every wave
    if (tid == 0)
      last_arrival = __hip_atomic_fetch_add(&p.counters[st], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     static_cast<unsigned>(S - 1);
    __syncthreads();
    if (!last_arrival) return;
#pragma unroll
    for (int fi = 0; fi < FT; ++fi)
#pragma unroll
      for (int ti = 0; ti < TT; ++ti) {
        floatx4 sum = {0.f, 0.f, 0.f, 0.f};
        for (int zz = 0; zz < S; ++zz)
          sum += __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, off(zz, fi, ti), 0, kSc1));
        acc[fi][ti] = sum;
      }
    if (tid == 0) __hip_atomic_store(&p.counters[st], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // D[4g + r][c16] of tile (fi, ti): features nf .. nf+3 of token m, rounded
  // where the reference's separate tensor ops round (as the fused kernel).
#pragma unroll
  for (int fi = 0; fi < FT; ++fi) {
    const int nf = n0 + C::WF * wn + 16 * fi + 4 * g;
    if (nf >= p.N) continue;
    float bias[4] = {0.f, 0.f, 0.f, 0.f};
    if (p.bias) {
      const V4 b4 = *reinterpret_cast<const V4*>(static_cast<const T*>(p.bias) + nf);
#pragma unroll
      for (int r = 0; r < 4; ++r) bias[r] = from_model<DT>(b4[r]);
    }
#pragma unroll
    for (int ti = 0; ti < TT; ++ti) {
      const int m = m0 + C::WT * wm + 16 * ti + c16;
      if (m >= p.M) continue;
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = from_model<DT>(to_model<DT>(acc[fi][ti][r] + bias[r]));
      if (p.epilogue == NS_EPILOGUE_SILU_MUL) {
        T o[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float act = from_model<DT>(to_model<DT>(silu_f32(y[2 * h])));
          o[h] = to_model<DT>(act * y[2 * h + 1]);
        }
        // Outputs nf/2 and nf/2 + 1 (nf a multiple of 4): one 4-byte store.
        T* dst = static_cast<T*>(p.out) + static_cast<int64_t>(m) * (p.N / 2) + nf / 2;
        *reinterpret_cast<uint32_t*>(dst) = __builtin_bit_cast(uint16_t, o[0]) |
                                            (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, o[1])) << 16);
        continue;
      }
      V4 o;
      if (p.epilogue == NS_EPILOGUE_RESIDUAL) {
        const V4 res = *reinterpret_cast<const V4*>(static_cast<const T*>(p.residual) + static_cast<int64_t>(m) * p.N + nf);
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = to_model<DT>(y[r] + from_model<DT>(res[r]));
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = to_model<DT>(y[r]);
      }
      *reinterpret_cast<V4*>(static_cast<T*>(p.out) + static_cast<int64_t>(m) * p.N + nf) = o;
    }
  }
}

struct GemmShape {
  int bm, bn, nst, wn;
  int64_t tiles, whole;  // all tiles; the first `whole` run unsplit
  int splits;            // K splits of each later tile
};

// MI355X: 256 CUs of 160 KiB LDS; the kernels' LDS (not their registers)
// sets how many workgroups share a CU.
constexpr int kGemmCUs = 256;
constexpr int kLdsPerCU = 160 * 1024;
constexpr int gemm_lds(int bm, int bn, int nst) {
  return nst * (bm * gemm::ROW_B + bn * gemm::BK / 2 + 2 * bn * 4) + 16;
}

// Tile shape and split count of a GEMM call, from measurements on MI355X
// (fp16, Qwen2.5-0.5B projections, graph-replayed).  128 x 128 tiles when
// they still give two workgroups per CU (gate|up from 1024 tokens: 44.8 /
// 66.3 us at 1024 / 2048 tokens against 46.9 / 86.7 with 64 x 128 tiles,
// both unsplit);
// 128-token x 64-feature tiles for long-K layers with enough of them
// (down_proj at 2048 tokens, split twice: 49.1 us against 53.9 with 64 x 128
// tiles); 64 x 64 tiles otherwise, the most workgroups for short calls (qkv /
// o / down at 256 tokens: 10.4 / 10.8 / 21.6 us, against 13.8 / 14.8 / 30.7
// with 64 x 128).  When the caller gave a workspace and the tiles of the last
// dispatch round (all of them, if one round holds every tile) fill at most
// half of the device's slots, those tiles split their K loop, at least 8
// steps a split: shorter splits write and read back more fp32 partials than
// the idle slots win (gate|up at 1024 / 2048 tokens, its last round's 128 x
// 128 tiles split into 4-5 steps: 49.4 / 74.9 us against 39.5 / 64.9 unsplit).
GemmShape gemm_shape(int64_t M, int N, int K, bool can_split) {
  auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  GemmShape s{64, 64, 4, 4, 0, 0, 1};
  if (tiles(128, 128) >= 512) s = {128, 128, 3, 4, 0, 0, 1};
  else if (K >= 2048 && tiles(128, 64) >= 200) s = {128, 64, 3, 4, 0, 0, 1};
  s.tiles = s.whole = tiles(s.bm, s.bn);
  const int64_t slots = int64_t{kGemmCUs} * (kLdsPerCU / gemm_lds(s.bm, s.bn, s.nst));
  const int64_t last = s.tiles - (s.tiles - 1) / slots * slots;  // tiles of the last round
  if (can_split && 2 * last <= slots && last <= gemm::kMaxSplitTiles) {
    const int steps = K / gemm::BK;
    const int64_t sp = std::min<int64_t>(std::min<int64_t>(slots / last, 4), steps / 8);
    if (sp > 1) {
      s.splits = static_cast<int>(sp);
      s.whole = s.tiles - last;
    }
  }
  return s;
}

int64_t gemm_part_bytes(const GemmShape& s) {
  if (s.splits <= 1) return 0;
  return (s.tiles - s.whole) * s.splits * static_cast<int64_t>(s.bm) * s.bn * 4;
}

// Instantiated tile configurations: (BM, BN, NST, WN).
#define NS_INT4_GEMM_CONFIGS(X) \
  X(128, 128, 3, 4)             \
  X(128, 64, 3, 4)              \
  X(64, 64, 4, 4)

template <class DT>
hipError_t launch_int4_gemm(const Int4LinearParams& p, const GemmShape& s, hipStream_t stream) {
  void* args[] = {const_cast<Int4LinearParams*>(&p)};
  const void* fn = nullptr;
#define NS_PICK(BM_, BN_, NST_, WN_) \
  if (s.bm == BM_ && s.bn == BN_ && s.nst == NST_ && s.wn == WN_) \
    fn = reinterpret_cast<const void*>(&int4_gemm_kernel<DT, BM_, BN_, NST_, WN_>);
  NS_INT4_GEMM_CONFIGS(NS_PICK)
#undef NS_PICK
  if (!fn) return hipErrorInvalidValue;
  const int64_t wgs = s.whole + (s.tiles - s.whole) * s.splits;
  if (wgs > 0x7FFFFFFF) return hipErrorInvalidValue;
  return hipLaunchKernel(fn, dim3(static_cast<unsigned>(wgs)), dim3(gemm::THREADS), args, 0, stream);
}

// Whole-weight dequantisation for large token counts, where a library GEMM on
// the model-dtype weight beats re-dequantising each weight tile per token
// tile.  One thread turns one 32-bit word (8 codes) into 16 bytes of weights,
// with dequantize_int4's arithmetic (quant.py:83-95).
template <class DT>
__global__ __launch_bounds__(256) void int4_dequantize_kernel(typename DT::T* out, const uint8_t* qweight,
                                                              const float* scales, const uint8_t* zeros,
                                                              int64_t words, int K, int group_size, int groups) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= words) return;
  const int64_t n = i / (K / 8);
  const int k = static_cast<int>(i % (K / 8)) * 8;
  const uint32_t word = reinterpret_cast<const uint32_t*>(qweight)[i];
  const int gi = k / group_size;
  const typename DT::vec8 w = dequant8<DT>(word, static_cast<float>(zeros[n * groups + gi]), scales[n * groups + gi]);
  *reinterpret_cast<typename DT::vec8*>(out + n * K + k) = w;
}

}  // namespace
}  // namespace ns

namespace ns {
namespace {

// Split-K workspace: a fixed region of u32 arrival counters (one per tile,
// zero between calls), then the partial sums.  The region has the same size
// for every M: the fused kernel only splits when 2 * tiles <= 256 and the
// GEMM splits at most gemm::kMaxSplitTiles tiles, so at most 256 counters exist,
// and the partials of any call start past every counter any other call may
// use.  One workspace can therefore serve calls of every token count in turn
// (a layer's decode steps change M from step to step) without a call's
// partial sums landing on another call's counters.
constexpr int64_t kSplitkCounterBytes = gemm::kMaxSplitTiles * 4;

struct SplitkLayout {
  int splits;
  int64_t counter_bytes, part_bytes;
};

// Token counts above kGemmMinRows take the GEMM (when K is a whole number of
// its steps), the rest the fused kernel with 16 bytes of partials per lane,
// tile and split.
SplitkLayout splitk_layout(int64_t M, int N, int K) {
  SplitkLayout l{1, 0, 0};
  if (M <= 0) return l;
  if (M > kGemmMinRows) {
    if (K % gemm::BK == 0) {
      const GemmShape gs = gemm_shape(M, N, K, true);
      l.splits = gs.splits;
      l.part_bytes = gemm_part_bytes(gs);
    }
  } else {
    const int mt = M <= 64 ? 16 : 64;
    const int64_t tiles = static_cast<int64_t>(N / 16) * ((M + mt - 1) / mt);
    l.splits = splitk_for(N, K, (M + mt - 1) / mt);
    l.part_bytes = l.splits > 1 ? tiles * l.splits * (mt / 16) * 64 * 16 : 0;
  }
  l.counter_bytes = l.splits > 1 ? kSplitkCounterBytes : 0;
  return l;
}
static_assert(kSplitkCounterBytes % 256 == 0, "partials stay 256-byte aligned");

int int4_linear_entry(void* out, const void* x, int64_t x_stride_row, const void* qweight, const void* scales,
                      const void* zeros, const void* bias, const void* residual, int epilogue,
                      const void* norm_weight, float norm_eps, int64_t M, int N, int K, int group_size, int dtype,
                      void* stream, void* workspace, size_t workspace_bytes, bool splitk) {
  if (dtype != NS_DTYPE_F16 && dtype != NS_DTYPE_BF16) return NS_ERR_UNSUPPORTED;
  if (M < 0 || N <= 0 || K <= 0 || group_size <= 0) return NS_ERR_INVALID_ARG;
  if (epilogue != NS_EPILOGUE_NONE && epilogue != NS_EPILOGUE_RESIDUAL && epilogue != NS_EPILOGUE_SILU_MUL)
    return NS_ERR_UNSUPPORTED;
  if (M == 0) return NS_OK;
  if (!out || !x || !qweight || !scales || !zeros) return NS_ERR_INVALID_ARG;
  if (epilogue == NS_EPILOGUE_RESIDUAL && (!residual || !aligned(residual, 8))) return NS_ERR_INVALID_ARG;
  // The fused RMSNorm needs every 128-wide chunk of K on its own wave.
  if (norm_weight && (K % 128 != 0 || K / 128 > 8)) return NS_ERR_UNSUPPORTED;
  if (norm_weight && !aligned(norm_weight, 16)) return NS_ERR_INVALID_ARG;
  // One MFMA row tile per 16 features; a K step of 32 lies inside one group.
  if (N % 16 != 0 || K % 32 != 0 || group_size % 32 != 0 || K % group_size != 0) return NS_ERR_UNSUPPORTED;
  if ((M + 15) / 16 > 65535) return NS_ERR_INVALID_ARG;  // grid.y bound of the smallest tile
  if (x_stride_row < K || x_stride_row % 8 != 0 || !aligned(x, 16) || !aligned(out, 8) ||
      !aligned(qweight, 16) || !aligned(scales, 4) || (bias && !aligned(bias, 2)))
    return NS_ERR_INVALID_ARG;

  Int4LinearParams p{};
  p.out = out;
  p.x = static_cast<const char*>(x);
  p.x_stride = x_stride_row;
  p.qweight = static_cast<const uint8_t*>(qweight);
  p.scales = static_cast<const float*>(scales);
  p.zeros = static_cast<const uint8_t*>(zeros);
  p.bias = bias;
  p.residual = residual;
  p.norm_weight = norm_weight;
  p.norm_eps = norm_eps;
  p.epilogue = epilogue;
  p.M = static_cast<int>(M);
  p.N = N;
  p.K = K;
  p.group_size = group_size;
  p.groups = K / group_size;
  // The GEMM does not fuse the RMSNorm; its epilogue reads bias four at a time
  // and its loads take whole 4-byte words of the zero-point table.
  // Its loads address x, the codes and the scales by 32-bit byte offsets.
  const int64_t esz = 2, lim = int64_t{1} << 32;
  const bool small = (M - 1) * x_stride_row * esz + int64_t{K} * esz < lim && int64_t{N} * (K / 2) < lim &&
                     int64_t{N} * (K / group_size) * 4 < lim;
  // A 64-wide K step of the GEMM lies inside one group.
  const bool use_gemm = M > kGemmMinRows && !norm_weight && K % gemm::BK == 0 && group_size % gemm::BK == 0 &&
                        (!bias || aligned(bias, 8)) && aligned(zeros, 4) && small;
  int splits = 1;
  if (splitk && (use_gemm || M <= kGemmMinRows)) {
    const SplitkLayout l = splitk_layout(M, N, K);
    if (l.splits > 1) {
      if (!workspace || !aligned(workspace, 256) ||
          workspace_bytes < static_cast<size_t>(l.counter_bytes + l.part_bytes) || l.part_bytes > 0x7FFFFFFF)
        return NS_ERR_INVALID_ARG;
      p.counters = static_cast<unsigned*>(workspace);
      p.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + l.counter_bytes);
      p.part_bytes = static_cast<int>(l.part_bytes);
      splits = l.splits;
    }
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (use_gemm) {
    // The same shape splitk_layout sized the workspace for (or none split).
    const GemmShape gs = gemm_shape(M, N, K, splits > 1);
    p.gemm_gx = (N + gs.bn - 1) / gs.bn;
    p.gemm_whole = static_cast<int>(gs.whole);
    p.gemm_splits = gs.splits;
    p.gemm_gh = static_cast<uint32_t>(group_size / 32);
    p.gemm_ghinv = p.gemm_gh == 1 ? 0u : static_cast<uint32_t>(((uint64_t{1} << 32) + p.gemm_gh - 1) / p.gemm_gh);
    e = dtype == NS_DTYPE_F16 ? launch_int4_gemm<F16>(p, gs, s) : launch_int4_gemm<BF16>(p, gs, s);
  } else
    e = dtype == NS_DTYPE_F16 ? launch_int4_linear<F16>(p, s, splits) : launch_int4_linear<BF16>(p, s, splits);
  return e == hipSuccess ? NS_OK : NS_ERR_HIP;
}

}  // namespace
}  // namespace ns

extern "C" int ns_int4_linear(void* out, const void* x, int64_t x_stride_row,
                              const void* qweight, const void* scales, const void* zeros, const void* bias,
                              const void* residual, int epilogue, const void* norm_weight, float norm_eps,
                              int64_t M, int N, int K, int group_size, int dtype, void* stream) {
  return ns::int4_linear_entry(out, x, x_stride_row, qweight, scales, zeros, bias, residual, epilogue, norm_weight,
                               norm_eps, M, N, K, group_size, dtype, stream, nullptr, 0, false);
}

extern "C" size_t ns_int4_linear_splitk_workspace_size(int64_t M, int N, int K) {
  if (M < 0 || N <= 0 || K <= 0) return 0;
  const ns::SplitkLayout l = ns::splitk_layout(M, N, K);
  return static_cast<size_t>(l.counter_bytes + l.part_bytes);
}

extern "C" int ns_int4_linear_splitk(void* out, const void* x, int64_t x_stride_row,
                                     const void* qweight, const void* scales, const void* zeros, const void* bias,
                                     const void* residual, int epilogue, const void* norm_weight, float norm_eps,
                                     int64_t M, int N, int K, int group_size, int dtype,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  return ns::int4_linear_entry(out, x, x_stride_row, qweight, scales, zeros, bias, residual, epilogue, norm_weight,
                               norm_eps, M, N, K, group_size, dtype, stream, workspace, workspace_bytes, true);
}

extern "C" int ns_int4_linear_rope_cache(void* q_out, const void* x, int64_t x_stride_row,
                                         const void* qweight, const void* scales, const void* zeros,
                                         const void* bias, const void* norm_weight, float norm_eps,
                                         const void* cos, const void* sin, int64_t cos_sin_stride_token,
                                         void* k_cache, void* v_cache,
                                         const void* slot_mapping, int slot_mapping_is_int64,
                                         int64_t M, int K, int group_size,
                                         int num_heads, int num_kv_heads, int head_dim,
                                         int block_size, int64_t num_blocks, int dtype, void* stream) {
  using namespace ns;
  if (dtype != NS_DTYPE_F16 && dtype != NS_DTYPE_BF16) return NS_ERR_UNSUPPORTED;
  if (M < 0 || K <= 0 || group_size <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      block_size <= 0 || num_blocks < 0)
    return NS_ERR_INVALID_ARG;
  // 16-row tiles pair dims of the two halves of a head; one 128-wide chunk per wave.
  if (head_dim % 16 != 0 || K % 128 != 0 || K / 128 > 8 || group_size % 32 != 0 || K % group_size != 0)
    return NS_ERR_UNSUPPORTED;
  if (M == 0) return NS_OK;
  if (!q_out || !x || !qweight || !scales || !zeros || !cos || !sin || !k_cache || !v_cache || !slot_mapping)
    return NS_ERR_INVALID_ARG;
  if ((M + 15) / 16 > 65535) return NS_ERR_INVALID_ARG;
  const int64_t n_rows = static_cast<int64_t>(num_heads + 2 * num_kv_heads) * head_dim;
  if (n_rows / 16 > 0x7FFFFFFF) return NS_ERR_INVALID_ARG;
  if (x_stride_row < K || x_stride_row % 8 != 0 || !aligned(x, 16) || !aligned(qweight, 16) ||
      !aligned(scales, 4) || (bias && !aligned(bias, 2)) || (norm_weight && !aligned(norm_weight, 16)) ||
      !aligned(q_out, 8) || !aligned(k_cache, 8) || !aligned(v_cache, 8) || !aligned(cos, 8) ||
      !aligned(sin, 8) || cos_sin_stride_token < head_dim || cos_sin_stride_token % 4 != 0 ||
      !aligned(slot_mapping, slot_mapping_is_int64 ? 8 : 4))
    return NS_ERR_INVALID_ARG;

  Int4LinearParams p{};
  p.out = q_out;
  p.x = static_cast<const char*>(x);
  p.x_stride = x_stride_row;
  p.qweight = static_cast<const uint8_t*>(qweight);
  p.scales = static_cast<const float*>(scales);
  p.zeros = static_cast<const uint8_t*>(zeros);
  p.bias = bias;
  p.residual = nullptr;
  p.norm_weight = norm_weight;
  p.norm_eps = norm_eps;
  p.epilogue = NS_EPILOGUE_NONE;
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(n_rows);
  p.K = K;
  p.group_size = group_size;
  p.groups = K / group_size;
  p.cos = cos;
  p.sin = sin;
  p.cs_stride = cos_sin_stride_token;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.slots = slot_mapping;
  p.slots64 = slot_mapping_is_int64 ? 1 : 0;
  p.num_slots = num_blocks * static_cast<int64_t>(block_size);
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.head_dim = head_dim;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t e =
      dtype == NS_DTYPE_F16 ? launch_int4_linear_rope<F16>(p, s) : launch_int4_linear_rope<BF16>(p, s);
  return e == hipSuccess ? NS_OK : NS_ERR_HIP;
}

extern "C" int ns_int4_dequantize(void* out, const void* qweight, const void* scales, const void* zeros,
                                  int N, int K, int group_size, int dtype, void* stream) {
  using namespace ns;
  if (dtype != NS_DTYPE_F16 && dtype != NS_DTYPE_BF16) return NS_ERR_UNSUPPORTED;
  if (N <= 0 || K <= 0 || group_size <= 0) return NS_ERR_INVALID_ARG;
  if (!out || !qweight || !scales || !zeros) return NS_ERR_INVALID_ARG;
  if (K % 8 != 0 || group_size % 8 != 0 || K % group_size != 0) return NS_ERR_UNSUPPORTED;
  if (!aligned(out, 16) || !aligned(qweight, 4) || !aligned(scales, 4)) return NS_ERR_INVALID_ARG;
  const int64_t words = static_cast<int64_t>(N) * (K / 8);
  const int64_t blocks = (words + 255) / 256;
  if (blocks > 0x7FFFFFFF) return NS_ERR_INVALID_ARG;
  const uint8_t* q = static_cast<const uint8_t*>(qweight);
  const float* sc = static_cast<const float*>(scales);
  const uint8_t* z = static_cast<const uint8_t*>(zeros);
  int k = K, gs = group_size, g = K / group_size;
  void* args[] = {&out, &q, &sc, &z, const_cast<int64_t*>(&words), &k, &gs, &g};
  const void* fn = dtype == NS_DTYPE_F16 ? reinterpret_cast<const void*>(&int4_dequantize_kernel<F16>)
                                         : reinterpret_cast<const void*>(&int4_dequantize_kernel<BF16>);
  const hipError_t e = hipLaunchKernel(fn, dim3(static_cast<unsigned>(blocks)), dim3(256), args, 0,
                                       static_cast<hipStream_t>(stream));
  return e == hipSuccess ? NS_OK : NS_ERR_HIP;
}
