// MFMA attention building blocks shared by the masked prefill attention and
// the grouped-query decode attention: 32x32x16 MFMAs, packing of
// probabilities, row sums with v_dot2, and the LDS layouts of K and V tiles
// (swizzles and the transpose-read addressing of V^T operands).
#pragma once
#include "common.hpp"

namespace sfl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Two values rounded to T and packed (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
template <typename T> __device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <> __device__ __forceinline__ uint32_t pack2<bf16_t>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}
template <> __device__ __forceinline__ uint32_t pack2<f16_t>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), f16x2_t));
}

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_v __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, f32x16 c);
template <>
__device__ __forceinline__ f32x16 mfma32<bf16_t>(const u32x4& a, const u32x4& b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32<f16_t>(const u32x4& a, const u32x4& b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// acc + lo + hi of a packed pair (v_dot2 with (1, 1)).
template <typename T> __device__ __forceinline__ float add_pair(uint32_t pk, float acc);
template <> __device__ __forceinline__ float add_pair<bf16_t>(uint32_t pk, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, pk), __builtin_bit_cast(bf16x2_v, 0x3f803f80u),
                                         acc, false);
}
template <> __device__ __forceinline__ float add_pair<f16_t>(uint32_t pk, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_v, pk), __builtin_bit_cast(f16x2_v, 0x3c003c00u), acc, false);
}

// V tile layout: row-major [key][8 slots of 16 bytes]; logical slot sg (dims
// 8sg .. 8sg+7) of key row r sits at physical slot 2((sg >> 1) ^ (r & 3)) +
// (sg & 1), so the 4 rows one 16-lane transpose read touches use 4 different
// 32-byte bank groups.
__device__ __forceinline__ unsigned vt_slot(unsigned sg, unsigned r) { return 2u * ((sg >> 1) ^ (r & 3u)) + (sg & 1u); }
// Byte offset, within a tile, of lane l's 8-byte piece for key step 0, dim
// tile t, first key half: key row 4(g >> 1) + (m >> 2), dims 32t + 16(g & 1) +
// 4(m & 3) .. +3, with g = l / 16 and m = l % 16.
template <int D>
__device__ __forceinline__ unsigned vt_lane_offset(int lane, int t) {
  const unsigned g = unsigned(lane) / 16u, m = unsigned(lane) % 16u;
  const unsigned r = 4u * (g >> 1) + (m >> 2);
  const unsigned dim = 32u * unsigned(t) + 16u * (g & 1u) + 4u * (m & 3u);
  return r * (2u * D) + 16u * vt_slot(dim / 8u, r) + 2u * (dim % 8u);
}

// K tile swizzle: row r's logical 16-byte slot s sits at s ^ k_swizzle<D>(r).
// The operand reads take one logical slot of 16 consecutive rows per LDS
// cycle; rows of 128 bytes (D = 64) alternate bank halves, so (r >> 1) & 7
// separates the rest, and rows of 256 bytes (D = 128) all start at bank 0, so
// the slot itself is rotated by r & 15.
template <int D>
__device__ __forceinline__ int k_swizzle(int r) {
  return D == 64 ? (r >> 1) & 7 : r & 15;
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

constexpr float kLazyMax = 8.f;

}  // namespace sfl
