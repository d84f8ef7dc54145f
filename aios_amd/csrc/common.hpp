// Shared device helpers for the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aios {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

// v_mfma_f32_16x16x32_bf16.  Lane l supplies A[l%16][(l/16)*8 + j] and
// B[(l/16)*8 + j][l%16] for j = 0..7 and receives C[(l/16)*4 + i][l%16]
// for i = 0..3.
__device__ __forceinline__ f32x4 mfma16x16x32(const bf16x8& a, const bf16x8& b,
                                              const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Low / high bf16 of a packed dword as fp32.
__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 pair, packed (a in the low half): one
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// fp32 -> nearest-even bf16 -> fp32.
__device__ __forceinline__ float round_bf16(float x) {
  return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, static_cast<bf16>(x)) << 16);
}

// Eight bf16 as fp32, and back (nearest even).
__device__ __forceinline__ void unpack_bf16x8(const bf16x8& v, float (&f)[8]) {
  const uint4 u = __builtin_bit_cast(uint4, v);
  f[0] = lo_bf16(u.x); f[1] = hi_bf16(u.x); f[2] = lo_bf16(u.y); f[3] = hi_bf16(u.y);
  f[4] = lo_bf16(u.z); f[5] = hi_bf16(u.z); f[6] = lo_bf16(u.w); f[7] = hi_bf16(u.w);
}
__device__ __forceinline__ bf16x8 pack_bf16x8(const float (&f)[8]) {
  return __builtin_bit_cast(bf16x8, make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]),
                                               pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7])));
}

// max(a, b) as v_maximum3_f32 (NaN-propagating, so the compiler adds no
// canonicalising v_max before it as it does for fmaxf; three-input chains
// fuse).  Inputs here are finite or -inf.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// DPP-based sums within each 16-lane row of the wavefront; every lane of the
// row receives the row total.  quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror.
__device__ __forceinline__ float row16_sum(float x) {
  int v;
  v = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false);
  x += __int_as_float(v);
  v = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false);
  x += __int_as_float(v);
  v = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false);
  x += __int_as_float(v);
  v = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false);
  x += __int_as_float(v);
  return x;
}
// The same within each group of 8 lanes (the first three steps: the half
// mirror pairs lane i of a group with lane 7 - i, in its other quad).
__device__ __forceinline__ float row8_sum(float x) {
  int v;
  v = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false);
  x += __int_as_float(v);
  v = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false);
  x += __int_as_float(v);
  v = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false);
  x += __int_as_float(v);
  return x;
}

// Cross-row (lanes l, l^16, l^32, l^48) reductions with the gfx950 lane
// swaps: v_permlane16_swap exchanges the odd 16-lane rows of its first
// operand with the even rows of its second, v_permlane32_swap the upper and
// lower halves; with both operands equal to x, the two results of a swap
// hold x[l] and x[l ^ 16] (resp. x[l ^ 32]) in some order on every lane.
__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xrow_max(float x) { return xor32_max(xor16_max(x)); }
// The cross-row maxima of two values at once, three swaps instead of four:
// swapping a's odd rows with b's even rows and taking the max leaves
// pairwise maxima of a in rows 0 and 2 and of b in rows 1 and 3; the
// half swap completes both (a's in rows 0 and 2, b's in 1 and 3); a last
// row swap hands every lane both.
__device__ __forceinline__ void xrow_max2(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  const float m = vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const float mm = xor32_max(m);
  const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(mm), __float_as_uint(mm), false, false);
  a = __uint_as_float(t[0]);
  b = __uint_as_float(t[1]);
}
__device__ __forceinline__ float xrow_sum(float x) { return xor32_sum(xor16_sum(x)); }

}  // namespace aios
