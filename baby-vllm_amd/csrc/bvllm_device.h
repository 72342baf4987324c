// Device-side helpers shared by the paged-KV kernels (gfx950 only).
//
// bf16 values travel as raw 16-bit patterns (uint16_t) so that every rounding
// step is explicit; MFMA operands are built from those patterns.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#if !defined(__gfx950__) && defined(__HIP_DEVICE_COMPILE__)
#error "baby-vllm_amd kernels are written for gfx950 (MI355X) only"
#endif

namespace bvllm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// float -> bf16 bits, round to nearest, ties to even; NaN -> canonical quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two floats -> one dword of packed bf16 (lo in bits 0..15), RNE, NaN -> 0x7fc0.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_rne(lo) | (f32_to_bf16_rne(hi) << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 with the hardware converter (v_cvt_pk_bf16_f32,
// round to nearest even). Same bits as pack_bf16x2 for every non-NaN input.
__device__ __forceinline__ uint32_t pack_bf16x2_hw(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Low / high bf16 of a dword as float.
__device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Select the 16-bit half `h` (0 = low, 1 = high) of a and b into one dword: {a.h, b.h}.
__device__ __forceinline__ uint32_t pick_halves(uint32_t a, uint32_t b, int h) {
  return h ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
}

__device__ __forceinline__ f32x4_t mfma_16x16x32(const uint4& a, const uint4& b, f32x4_t c) {
  bf16x8_t av = __builtin_bit_cast(bf16x8_t, a);
  bf16x8_t bv = __builtin_bit_cast(bf16x8_t, b);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4_t mfma_16x16x16(const uint2& a, const uint2& b, f32x4_t c) {
  i16x4_t av = __builtin_bit_cast(i16x4_t, a);
  i16x4_t bv = __builtin_bit_cast(i16x4_t, b);
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bv, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// IEEE maximum (NaN-propagating): lowers to v_maximum3_f32 chains with no
// canonicalising of the operands, which fmaxf (maxnum) needs on every value
// not known to be canonical. Same result as fmaxf for non-NaN operands (a NaN
// score yields a NaN output either way: its exponent poisons the sum).
__device__ __forceinline__ float fmax_prop(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Butterfly over the four 16-lane groups of a wave (lanes n, n+16, n+32, n+48),
// xor 16 then xor 32, with gfx950's permlane swaps (VALU, no LDS round trip).
// permlane16_swap(x, x) leaves {g0, g0, g2, g2} in the first result and
// {g1, g1, g3, g3} in the second (g = 16-lane group); permlane32_swap(x, x)
// leaves {lo, lo} and {hi, hi} (32-lane halves). Combining the two results
// lane by lane is the xor-16 (resp. xor-32) exchange: lane l gets x[l] op
// x[l ^ 16] (resp. x[l ^ 32]), the same operands in some order, and fmax and
// + are commutative, so the bits equal those of the shuffle form.
__device__ __forceinline__ float max_across_groups(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmax_prop(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmax_prop(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_across_groups(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

template <typename T>
__device__ __forceinline__ T uniform(T v) {
  return (T)__builtin_amdgcn_readfirstlane((int)v);
}

// LDS transpose read (ds_read_b64_tr_b16, 8-byte aligned LDS address): within
// each 16-lane group, lane l receives element (l mod 4) of the 4 bf16 that lanes
// 4i + l/4 (i < 4) address, as its element i. So if lane s of group g addresses
// row r0 + 4g + s/4, columns c0 + 4(s mod 4) .. +3 of a row-major bf16 matrix,
// lane l gets column c0 + l of rows r0 + 4g + i, i < 4: a column operand for MFMA.
__device__ __forceinline__ uint2 ld_tr16(const uint16_t* lds_ptr) {
  typedef __attribute__((address_space(3))) i16x4_t* LdsVec;
  const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsVec)(lds_ptr));
  return __builtin_bit_cast(uint2, v);
}

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint2 ld8(const void* p) { return *reinterpret_cast<const uint2*>(p); }
__device__ __forceinline__ void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }
__device__ __forceinline__ void st8(void* p, uint2 v) { *reinterpret_cast<uint2*>(p) = v; }

// 16-byte load with the nontemporal hint, for data a kernel reads exactly once
// (streamed past the caches; a higher read rate on MI355X than plain loads).
__device__ __forceinline__ uint4 ld16_nt(const void* p) {
  typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));
  const u32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 16-byte store with the nontemporal hint, for data the kernel writes once and
// no later work of the same kernel reads.
__device__ __forceinline__ void st16_nt(void* p, uint4 v) {
  typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));
  const u32x4_nt w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_nt*>(p));
}

}  // namespace bvllm
