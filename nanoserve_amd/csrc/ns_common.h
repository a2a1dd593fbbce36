// Shared device helpers for the gfx950 paged-attention kernels.
//
// Everything here is written for CDNA4 wave64: 16-byte per-lane global loads,
// the 16x16x32 f16/bf16 MFMA, and cross-lane reductions inside a wave.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nanoserve_paged.h"

namespace ns {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Element-type tags.  `vec8` is the 16-byte MFMA operand of eight elements,
// `vec4` an 8-byte group of four.
struct F16 {
  using T = _Float16;
  using vec8 = half8;
  using vec4 = half4;
  static constexpr int code = NS_DTYPE_F16;
};
struct BF16 {
  using T = __bf16;
  using vec8 = bf16x8;
  using vec4 = bf16x4;
  static constexpr int code = NS_DTYPE_BF16;
};

// D[16x16] += A[16x32] * B[32x16], fp32 accumulate.
// Operand layout (lane l, group g = l / 16): A row l % 16 and B column l % 16,
// each holding the 8 k-slots of group g.  The result layout is
// D[4 * g + r][l % 16] in element r of the returned vector.
__device__ __forceinline__ floatx4 mfma16x16x32(F16, half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma16x16x32(BF16, bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <class DT>
__device__ __forceinline__ typename DT::vec8 load16(const void* p) {
  return __builtin_bit_cast(typename DT::vec8, *reinterpret_cast<const u32x4*>(p));
}

template <class DT>
__device__ __forceinline__ typename DT::vec8 zero8() {
  return __builtin_bit_cast(typename DT::vec8, u32x4{0u, 0u, 0u, 0u});
}

// Load entry i of an int32 or int64 index tensor.
__device__ __forceinline__ int64_t load_index(const void* p, int64_t i, int is64) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i]
              : static_cast<int64_t>(reinterpret_cast<const int32_t*>(p)[i]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Butterfly max / sum over the four 16-lane groups of a wave (lanes l, l^16,
// l^32, l^48 hold the same matrix column in the MFMA result layout).
__device__ __forceinline__ float group4_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}
__device__ __forceinline__ float group4_sum(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// The same reductions with gfx950's row-swap permutes (VALU, no LDS trip).
// With both operands holding v, v_permlane16_swap leaves 16-lane rows
// {0,0,2,2} of v in its first operand and {1,1,3,3} in its second, and
// v_permlane32_swap halves {lo,lo} and {hi,hi}, so one max / add of the pair
// is one butterfly stage.  They are written as asm: the compiler's builtin
// for these swaps folds the second result into the first.
__device__ __forceinline__ void swap_rows16(float& x, float& y) {
  asm volatile("s_nop 4\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
}
__device__ __forceinline__ void swap_halves32(float& x, float& y) {
  asm volatile("s_nop 4\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
}
__device__ __forceinline__ float group4_max_swap(float v) {
  float x = v, y = v;
  swap_rows16(x, y);
  v = fmaxf(x, y);
  x = v;
  y = v;
  swap_halves32(x, y);
  return fmaxf(x, y);
}
__device__ __forceinline__ float group4_sum_swap(float v) {
  float x = v, y = v;
  swap_rows16(x, y);
  v = x + y;
  x = v;
  y = v;
  swap_halves32(x, y);
  return x + y;
}

// Transposing LDS read (ds_read_b64_tr_b16) written as asm.  The builtin
// carries no memory operand, so the compiler's wait-count pass assumes it may
// read the destination of any LDS-DMA load in flight and puts an
// s_waitcnt vmcnt(0) in front of it, which drains every prefetch of a
// global_load_lds ring.  The asm result is not waited for: the caller issues
// lds_wait_all() and then passes each result through lds_ready().
__device__ __forceinline__ u32x2 ds_read_tr16_b64(const void* lds) {
  u32x2 r;
  const uint32_t a =
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(lds)));
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(a));
  return r;
}
// global_load_lds as asm: each lane's `bytes` (4 or 16) at `src` land in
// LDS at lds + bytes * lane.  The compiler does not see these loads, so its
// wait-count pass neither waits for them (the caller does, with explicit
// vmcnt) nor drains them before later LDS or DMA instructions; its own
// waits for its own loads only ever count too few operations in flight,
// which waits longer, never too little.
// M0 is reserved, so listing it as clobbered draws a warning; the compiler
// sets M0 itself right before any instruction of its own that reads it.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_lds16(const void* src, const void* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(lds))));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m) : "memory", "m0");
}
// The same with a uniform base address in an SGPR pair and a per-lane 32-bit
// byte offset (the instruction's saddr form): no 64-bit address arithmetic
// in the vector ALU.
__device__ __forceinline__ void dma_lds16_off(const void* base, uint32_t off, const void* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(lds))));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m)
               : "memory", "m0");
}
__device__ __forceinline__ void dma_lds4_off(const void* base, uint32_t off, const void* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(lds))));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(m)
               : "memory", "m0");
}
__device__ __forceinline__ void dma_lds4(const void* src, const void* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(lds))));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(m) : "memory", "m0");
}
#pragma clang diagnostic pop

// Plain LDS reads as asm, for data that arrived by global_load_lds: the
// compiler's wait-count pass would otherwise wait for every LDS-DMA load in
// flight before any LDS read it cannot prove disjoint from them.
__device__ __forceinline__ u32x4 ds_read_b128(const void* lds) {
  u32x4 r;
  const uint32_t a =
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(lds)));
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
  return r;
}
__device__ __forceinline__ uint32_t ds_read_b32(const void* lds) {
  uint32_t r;
  const uint32_t a =
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(lds)));
  asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(a));
  return r;
}
__device__ __forceinline__ void lds_wait_all() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// Orders every later use of x after the preceding lds_wait_all().
template <class V>
__device__ __forceinline__ void lds_ready(V& x) {
  asm volatile("" : "+v"(x));
}

}  // namespace ns
