// Activation operand format and layout of the decode GEMVs.
//
// Values, 4 bytes per element in every model dtype:
//   fp32 weights: fp32 values;
//   bf16 weights: hi = x truncated to bf16 and lo = (x - hi) truncated to
//   bf16, so hi + lo keeps ~16 mantissa bits of x (two MFMAs per chunk);
//   fp16 weights: hi = x rounded to fp16 and lo = (x - hi) rounded to fp16
//   (~22 bits while lo stays a normal fp16 number).
// Layout of a [B, K] input: blocks of 16 rows; inside a block, K is cut into
// chunks of chunk_k values (32 for bf16, 16 for fp32) and each chunk is stored
// exactly as a wave loads its MFMA B operand: lane l = 16 * g + r (row r, lane
// group g) owns the chunk's values [g * epl, (g + 1) * epl) of row r in 16
// bytes at lane * 16 (bf16: the hi halves; the lo halves follow 1 KB later).
// A chunk is 1 KB (fp32) or 2 KB (bf16) of contiguous memory, so every GEMV
// load instruction reads whole cache lines.
#pragma once
#include "common.hpp"

namespace sfl {

// Chunk geometry: one 16-byte lane load covers vec_elems<T>() values, a chunk
// covers 4 lane groups.
template <typename T> __host__ __device__ constexpr int chunk_k() { return 4 * vec_elems<T>(); }
template <typename T> __host__ __device__ constexpr int act_chunk_bytes() {
  return sizeof(T) == 2 ? 2048 : 1024;
}
constexpr int kActLoOffset = 1024;  // 16-bit: lo halves of a chunk follow its hi halves

// The (hi, lo) halves of one activation value for 16-bit weights, as raw bits.
template <typename T> __device__ __forceinline__ void split_act(float v, uint32_t& hi, uint32_t& lo);
template <> __device__ __forceinline__ void split_act<bf16_t>(float v, uint32_t& hi, uint32_t& lo) {
  const uint32_t hb = __float_as_uint(v) & 0xffff0000u;
  hi = hb >> 16;
  lo = (__float_as_uint(v - __uint_as_float(hb)) & 0xffff0000u) >> 16;
}
template <> __device__ __forceinline__ void split_act<f16_t>(float v, uint32_t& hi, uint32_t& lo) {
  hi = f32_to_f16_bits(v);
  lo = f32_to_f16_bits(v - f16_bits_to_f32(uint16_t(hi)));
}

// Byte offset of element (b, e) of a [B, K] activation (bf16: of its hi half).
template <typename T>
__device__ __forceinline__ long act_offset(int b, int e, int K) {
  constexpr int KC = chunk_k<T>(), EPL = vec_elems<T>(), ES = sizeof(T) == 2 ? 2 : 4;
  const long block = long(b / 16) * (K / KC) * act_chunk_bytes<T>();
  const int lane = ((e % KC) / EPL) * 16 + b % 16;
  return block + long(e / KC) * act_chunk_bytes<T>() + lane * 16 + (e % EPL) * ES;
}

// One value in the activation format (split halves for 16-bit T).
template <typename T>
__device__ __forceinline__ void store_act1(unsigned char* act, int b, int e, int K, float v) {
  unsigned char* p = act + act_offset<T>(b, e, K);
  if constexpr (sizeof(T) == 2) {
    uint32_t hi, lo;
    split_act<T>(v, hi, lo);
    *reinterpret_cast<uint16_t*>(p) = uint16_t(hi);
    *reinterpret_cast<uint16_t*>(p + kActLoOffset) = uint16_t(lo);
  } else {
    *reinterpret_cast<float*>(p) = v;
  }
}

// Four consecutive values (e % 4 == 0; they share one lane's 16 bytes).
template <typename T>
__device__ __forceinline__ void store_act4(unsigned char* act, int b, int e, int K, const float* v);
template <>
__device__ __forceinline__ void store_act4<float>(unsigned char* act, int b, int e, int K, const float* v) {
  *reinterpret_cast<float4*>(act + act_offset<float>(b, e, K)) = make_float4(v[0], v[1], v[2], v[3]);
}
template <>
__device__ __forceinline__ void store_act4<bf16_t>(unsigned char* act, int b, int e, int K, const float* v) {
  uint32_t hb[4], lb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hb[i] = __float_as_uint(v[i]) & 0xffff0000u;
    lb[i] = __float_as_uint(v[i] - __uint_as_float(hb[i])) & 0xffff0000u;
  }
  unsigned char* g = act + act_offset<bf16_t>(b, e, K);
  *reinterpret_cast<uint2*>(g) = make_uint2((hb[0] >> 16) | hb[1], (hb[2] >> 16) | hb[3]);
  *reinterpret_cast<uint2*>(g + kActLoOffset) = make_uint2((lb[0] >> 16) | lb[1], (lb[2] >> 16) | lb[3]);
}
template <>
__device__ __forceinline__ void store_act4<f16_t>(unsigned char* act, int b, int e, int K, const float* v) {
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) split_act<f16_t>(v[i], hi[i], lo[i]);
  unsigned char* g = act + act_offset<f16_t>(b, e, K);
  *reinterpret_cast<uint2*>(g) = make_uint2(hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16));
  *reinterpret_cast<uint2*>(g + kActLoOffset) = make_uint2(lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16));
}

}  // namespace sfl
