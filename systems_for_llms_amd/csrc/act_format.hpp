// Activation operand format of the decode GEMVs and its producers.
//
// 4 bytes per element in both model dtypes:
//   fp32 weights: plain fp32 values;
//   bf16 weights: each group of 8 consecutive values is stored as 8 "hi" bf16
//   followed by 8 "lo" bf16 (32 bytes), with hi = x truncated to bf16 and
//   lo = (x - hi) truncated to bf16, so hi + lo keeps ~16 mantissa bits of x
//   and one lane's 8-value chunk is exactly two MFMA B operands.
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

// Store 4 consecutive activation values (element index e, e % 4 == 0) of a row.
template <typename T>
__device__ __forceinline__ void store_act4(unsigned char* row, int e, const float* v);
template <>
__device__ __forceinline__ void store_act4<float>(unsigned char* row, int e, const float* v) {
  *reinterpret_cast<float4*>(row + size_t(e) * 4) = make_float4(v[0], v[1], v[2], v[3]);
}
template <>
__device__ __forceinline__ void store_act4<bf16_t>(unsigned char* row, int e, const float* v) {
  uint32_t hb[4], lb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hb[i] = __float_as_uint(v[i]) & 0xffff0000u;
    lb[i] = __float_as_uint(v[i] - __uint_as_float(hb[i])) & 0xffff0000u;
  }
  unsigned char* g = row + size_t(e / 8) * 32 + (e % 8) * 2;
  *reinterpret_cast<uint2*>(g) = make_uint2((hb[0] >> 16) | hb[1], (hb[2] >> 16) | hb[3]);
  *reinterpret_cast<uint2*>(g + 16) = make_uint2((lb[0] >> 16) | lb[1], (lb[2] >> 16) | lb[3]);
}

// One tile of 16 features of a row: optionally store x, then store x * g in the
// activation format and the tile's sum of squares.
template <typename T>
__device__ __forceinline__ void emit_tile(const float* v, const T* gain, int t, float* x_row,
                                          unsigned char* act_row, float* ss_row) {
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
    store_act4<T>(act_row, 16 * t + i, gx);
    sq = fmaf(v[i], v[i], fmaf(v[i + 1], v[i + 1], fmaf(v[i + 2], v[i + 2], fmaf(v[i + 3], v[i + 3], sq))));
  }
  ss_row[t] = sq;
}

}  // namespace sfl
