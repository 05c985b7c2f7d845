// Building blocks of the decode GEMVs, shared by decode_linear.hip and the
// fused attention kernel of decode_attention.hip: the MFMA step over one K
// chunk, the activation-format operands (act_format.hpp), the normalized
// consumers' x * g operands and the 4-value stores of the epilogues.
#pragma once
#include "act_format.hpp"

namespace sfl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ f32x4 mfma_chunk(const uint4& a, const u32x4& b, f32x4 acc);

template <>
__device__ __forceinline__ f32x4 mfma_chunk<bf16_t>(const uint4& a, const u32x4& b, f32x4 acc) {
  const u32x4 av = {a.x, a.y, a.z, a.w};
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                 __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ f32x4 mfma_chunk<f16_t>(const uint4& a, const u32x4& b, f32x4 acc) {
  const u32x4 av = {a.x, a.y, a.z, a.w};
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av), __builtin_bit_cast(f16x8, b), acc, 0,
                                                0, 0);
}

// fp32: the lane's 4 consecutive k values feed 4 MFMA steps; A and B use the
// same (lane group, step) -> k mapping, so the contraction is exact.
template <>
__device__ __forceinline__ f32x4 mfma_chunk<float>(const uint4& a, const u32x4& b, f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
  return acc;
}

template <typename T>
__device__ __forceinline__ void store4(T* dst, const float* v);
template <>
__device__ __forceinline__ void store4<float>(float* dst, const float* v) {
  *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
}
template <>
__device__ __forceinline__ void store4<bf16_t>(bf16_t* dst, const float* v) {
  const uint32_t lo = uint32_t(f32_to_bf16_bits(v[0])) | (uint32_t(f32_to_bf16_bits(v[1])) << 16);
  const uint32_t hi = uint32_t(f32_to_bf16_bits(v[2])) | (uint32_t(f32_to_bf16_bits(v[3])) << 16);
  *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
}
template <>
__device__ __forceinline__ void store4<f16_t>(f16_t* dst, const float* v) {
  const uint32_t lo = uint32_t(f32_to_f16_bits(v[0])) | (uint32_t(f32_to_f16_bits(v[1])) << 16);
  const uint32_t hi = uint32_t(f32_to_f16_bits(v[2])) | (uint32_t(f32_to_f16_bits(v[3])) << 16);
  *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
}

// One lane's chunk of the activation format (act_format.hpp). Producers (the
// residual epilogues, the token step, the SwiGLU epilogue, the attention
// merge) write the format once; the GEMV loop then does no conversion.
template <typename T> struct ActChunk;
template <> struct ActChunk<float> { uint4 v; };
template <> struct ActChunk<bf16_t> { uint4 hi, lo; };
template <> struct ActChunk<f16_t> { uint4 hi, lo; };

template <typename T>
__device__ __forceinline__ ActChunk<T> load_act(const unsigned char* p);
template <>
__device__ __forceinline__ ActChunk<float> load_act<float>(const unsigned char* p) {
  return {load16(p)};
}
template <>
__device__ __forceinline__ ActChunk<bf16_t> load_act<bf16_t>(const unsigned char* p) {
  return {load16(p), load16(p + kActLoOffset)};
}
template <>
__device__ __forceinline__ ActChunk<f16_t> load_act<f16_t>(const unsigned char* p) {
  return {load16(p), load16(p + kActLoOffset)};
}

template <typename T>
__device__ __forceinline__ f32x4 mfma_act(const uint4& w, const ActChunk<T>& x, bool live, f32x4 acc);
template <>
__device__ __forceinline__ f32x4 mfma_act<bf16_t>(const uint4& w, const ActChunk<bf16_t>& x, bool live, f32x4 acc) {
  const u32x4 bh = {live ? x.hi.x : 0u, live ? x.hi.y : 0u, live ? x.hi.z : 0u, live ? x.hi.w : 0u};
  const u32x4 bl = {live ? x.lo.x : 0u, live ? x.lo.y : 0u, live ? x.lo.z : 0u, live ? x.lo.w : 0u};
  acc = mfma_chunk<bf16_t>(w, bh, acc);
  return mfma_chunk<bf16_t>(w, bl, acc);
}
template <>
__device__ __forceinline__ f32x4 mfma_act<f16_t>(const uint4& w, const ActChunk<f16_t>& x, bool live, f32x4 acc) {
  const u32x4 bh = {live ? x.hi.x : 0u, live ? x.hi.y : 0u, live ? x.hi.z : 0u, live ? x.hi.w : 0u};
  const u32x4 bl = {live ? x.lo.x : 0u, live ? x.lo.y : 0u, live ? x.lo.z : 0u, live ? x.lo.w : 0u};
  acc = mfma_chunk<f16_t>(w, bh, acc);
  return mfma_chunk<f16_t>(w, bl, acc);
}
template <>
__device__ __forceinline__ f32x4 mfma_act<float>(const uint4& w, const ActChunk<float>& x, bool live, f32x4 acc) {
  const u32x4 b = {live ? x.v.x : 0u, live ? x.v.y : 0u, live ? x.v.z : 0u, live ? x.v.w : 0u};
  return mfma_chunk<float>(w, b, acc);
}

// A normalized consumer's source: one lane's fp32 values of x for a chunk and
// the matching gains (16-bit weights: 8 values, fp32: 4).
template <typename T> struct NormChunk;
template <> struct NormChunk<bf16_t> { float4 x0, x1; uint4 g; };
template <> struct NormChunk<f16_t> { float4 x0, x1; uint4 g; };
template <> struct NormChunk<float> { float4 x; float4 g; };

template <typename T>
__device__ __forceinline__ NormChunk<T> load_norm(const float* x, const T* g);
template <>
__device__ __forceinline__ NormChunk<bf16_t> load_norm<bf16_t>(const float* x, const bf16_t* g) {
  return {*reinterpret_cast<const float4*>(x), *reinterpret_cast<const float4*>(x + 4), load16(g)};
}
template <>
__device__ __forceinline__ NormChunk<f16_t> load_norm<f16_t>(const float* x, const f16_t* g) {
  return {*reinterpret_cast<const float4*>(x), *reinterpret_cast<const float4*>(x + 4), load16(g)};
}
template <>
__device__ __forceinline__ NormChunk<float> load_norm<float>(const float* x, const float* g) {
  return {*reinterpret_cast<const float4*>(x), *reinterpret_cast<const float4*>(g)};
}

// x * g in the MFMA operand format (for bf16 weights split into hi + lo bf16
// halves, as act_format.hpp defines), adding the lane's x^2 to ss.
template <typename T>
__device__ __forceinline__ ActChunk<T> norm_operand(const NormChunk<T>& s, float& ss);
template <>
__device__ __forceinline__ ActChunk<bf16_t> norm_operand<bf16_t>(const NormChunk<bf16_t>& s, float& ss) {
  const float x[8] = {s.x0.x, s.x0.y, s.x0.z, s.x0.w, s.x1.x, s.x1.y, s.x1.z, s.x1.w};
  const uint32_t gw[4] = {s.g.x, s.g.y, s.g.z, s.g.w};
  uint32_t hb[8], lb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    ss = fmaf(x[i], x[i], ss);
    const float v = x[i] * ((i & 1) ? bf16_hi(gw[i / 2]) : bf16_lo(gw[i / 2]));
    hb[i] = __float_as_uint(v) & 0xffff0000u;
    lb[i] = __float_as_uint(v - __uint_as_float(hb[i])) & 0xffff0000u;
  }
  ActChunk<bf16_t> r;
  r.hi = make_uint4((hb[0] >> 16) | hb[1], (hb[2] >> 16) | hb[3], (hb[4] >> 16) | hb[5], (hb[6] >> 16) | hb[7]);
  r.lo = make_uint4((lb[0] >> 16) | lb[1], (lb[2] >> 16) | lb[3], (lb[4] >> 16) | lb[5], (lb[6] >> 16) | lb[7]);
  return r;
}
template <>
__device__ __forceinline__ ActChunk<f16_t> norm_operand<f16_t>(const NormChunk<f16_t>& s, float& ss) {
  const float x[8] = {s.x0.x, s.x0.y, s.x0.z, s.x0.w, s.x1.x, s.x1.y, s.x1.z, s.x1.w};
  float g[8];
  unpack16<f16_t>(s.g, g);
  uint32_t hb[8], lb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    ss = fmaf(x[i], x[i], ss);
    split_act<f16_t>(x[i] * g[i], hb[i], lb[i]);
  }
  ActChunk<f16_t> r;
  r.hi = make_uint4(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16), hb[4] | (hb[5] << 16), hb[6] | (hb[7] << 16));
  r.lo = make_uint4(lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16), lb[4] | (lb[5] << 16), lb[6] | (lb[7] << 16));
  return r;
}
template <>
__device__ __forceinline__ ActChunk<float> norm_operand<float>(const NormChunk<float>& s, float& ss) {
  ss = fmaf(s.x.x, s.x.x, ss);
  ss = fmaf(s.x.y, s.x.y, ss);
  ss = fmaf(s.x.z, s.x.z, ss);
  ss = fmaf(s.x.w, s.x.w, ss);
  ActChunk<float> r;
  r.v = make_uint4(__float_as_uint(s.x.x * s.g.x), __float_as_uint(s.x.y * s.g.y),
                   __float_as_uint(s.x.z * s.g.z), __float_as_uint(s.x.w * s.g.w));
  return r;
}

template <bool kNorm, typename T> struct SrcOf { using type = ActChunk<T>; };
template <typename T> struct SrcOf<true, T> { using type = NormChunk<T>; };

}  // namespace sfl
