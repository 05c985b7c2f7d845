// Activation operand format and layout of the decode GEMVs, and its producers.
//
// Values, 4 bytes per element in both model dtypes:
//   fp32 weights: fp32 values;
//   bf16 weights: hi = x truncated to bf16 and lo = (x - hi) truncated to
//   bf16, so hi + lo keeps ~16 mantissa bits of x (two MFMAs per chunk).
// Layout of a [B, K] input: blocks of 16 rows; inside a block, K is cut into
// chunks of chunk_k values (32 for bf16, 16 for fp32) and each chunk is stored
// exactly as a wave loads its MFMA B operand: lane l = 16 * g + r (row r, lane
// group g) owns the chunk's values [g * epl, (g + 1) * epl) of row r in 16
// bytes at lane * 16 (bf16: the hi halves; the lo halves follow 1 KB later).
// A chunk is 1 KB (fp32) or 2 KB (bf16) of contiguous memory, so every GEMV
// load instruction reads whole cache lines.
// A normalized consumer (RMSNorm folded into the GEMV) reads x * g in this
// format plus the sums of x^2 over each 16-feature tile of x.
#pragma once
#include "common.hpp"

namespace sfl {

// Four consecutive RMSNorm gains as fp32 (one 8- or 16-byte load).
template <typename T> __device__ __forceinline__ float4 load_gain4(const T* p);
template <> __device__ __forceinline__ float4 load_gain4<float>(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
template <> __device__ __forceinline__ float4 load_gain4<bf16_t>(const bf16_t* p) {
  const uint2 w = *reinterpret_cast<const uint2*>(p);
  return make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
}

// Chunk geometry: one 16-byte lane load covers vec_elems<T>() values, a chunk
// covers 4 lane groups.
template <typename T> __host__ __device__ constexpr int chunk_k() { return 4 * vec_elems<T>(); }
template <typename T> __host__ __device__ constexpr int act_chunk_bytes() {
  return sizeof(T) == 2 ? 2048 : 1024;
}
constexpr int kActLoOffset = 1024;  // bf16: lo halves of a chunk follow its hi halves

// Byte offset of element (b, e) of a [B, K] activation (bf16: of its hi half).
template <typename T>
__device__ __forceinline__ long act_offset(int b, int e, int K) {
  constexpr int KC = chunk_k<T>(), EPL = vec_elems<T>(), ES = sizeof(T) == 2 ? 2 : 4;
  const long block = long(b / 16) * (K / KC) * act_chunk_bytes<T>();
  const int lane = ((e % KC) / EPL) * 16 + b % 16;
  return block + long(e / KC) * act_chunk_bytes<T>() + lane * 16 + (e % EPL) * ES;
}

// One value in the activation format (split-bf16 for T = bf16).
template <typename T>
__device__ __forceinline__ void store_act1(unsigned char* act, int b, int e, int K, float v) {
  unsigned char* p = act + act_offset<T>(b, e, K);
  if constexpr (sizeof(T) == 2) {
    const uint32_t hb = __float_as_uint(v) & 0xffff0000u;
    const uint32_t lb = __float_as_uint(v - __uint_as_float(hb)) & 0xffff0000u;
    *reinterpret_cast<uint16_t*>(p) = uint16_t(hb >> 16);
    *reinterpret_cast<uint16_t*>(p + kActLoOffset) = uint16_t(lb >> 16);
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

// One tile of 16 features of row b: optionally store x, then store x * g in the
// activation format and the tile's sum of squares.
template <typename T>
__device__ __forceinline__ void emit_tile(const float* v, const T* gain, int t, float* x_row,
                                          unsigned char* act, int b, int K, float* ss_row) {
  if (x_row) {
#pragma unroll
    for (int i = 0; i < 16; i += 4)
      *reinterpret_cast<float4*>(x_row + 16 * t + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
  }
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    const float4 g = load_gain4<T>(gain + 16 * t + i);
    const float gx[4] = {v[i] * g.x, v[i + 1] * g.y, v[i + 2] * g.z, v[i + 3] * g.w};
    store_act4<T>(act, b, 16 * t + i, K, gx);
    sq = fmaf(v[i], v[i], fmaf(v[i + 1], v[i + 1], fmaf(v[i + 2], v[i + 2], fmaf(v[i + 3], v[i + 3], sq))));
  }
  ss_row[t] = sq;
}

}  // namespace sfl
