// Shared device helpers for the gfx950 kernels: element types, 16-byte vector
// loads, fp32 <-> storage conversions and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sfl.h"

namespace sfl {

constexpr int kWave = 64;

// Storage types. bf16 and fp16 are carried as raw 16-bit words so every
// conversion is explicit and the same on every path.
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

template <typename T> struct Elem;
template <> struct Elem<float> { static constexpr int bytes = 4; };
template <> struct Elem<bf16_t> { static constexpr int bytes = 2; };
template <> struct Elem<f16_t> { static constexpr int bytes = 2; };

// Elements carried by one 16-byte load.
template <typename T> constexpr int vec_elems() { return 16 / Elem<T>::bytes; }

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 (the rounding torch's .to(bfloat16) uses);
// NaN maps to a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  return *reinterpret_cast<uint16_t*>(&h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  _Float16 h = *reinterpret_cast<_Float16*>(&b);
  return (float)h;
}

// Unpack one 16-byte vector into fp32 values.
template <typename T> __device__ __forceinline__ void unpack16(const uint4& r, float* out);
template <> __device__ __forceinline__ void unpack16<bf16_t>(const uint4& r, float* out) {
  out[0] = bf16_lo(r.x); out[1] = bf16_hi(r.x);
  out[2] = bf16_lo(r.y); out[3] = bf16_hi(r.y);
  out[4] = bf16_lo(r.z); out[5] = bf16_hi(r.z);
  out[6] = bf16_lo(r.w); out[7] = bf16_hi(r.w);
}
template <> __device__ __forceinline__ void unpack16<f16_t>(const uint4& r, float* out) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = f16_bits_to_f32(uint16_t(w[i] & 0xffffu));
    out[2 * i + 1] = f16_bits_to_f32(uint16_t(w[i] >> 16));
  }
}
template <> __device__ __forceinline__ void unpack16<float>(const uint4& r, float* out) {
  out[0] = __uint_as_float(r.x); out[1] = __uint_as_float(r.y);
  out[2] = __uint_as_float(r.z); out[3] = __uint_as_float(r.w);
}

template <typename T> __device__ __forceinline__ float load_scalar(const T* p);
template <> __device__ __forceinline__ float load_scalar<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float load_scalar<bf16_t>(const bf16_t* p) {
  return __uint_as_float(uint32_t(p->bits) << 16);
}
template <> __device__ __forceinline__ float load_scalar<f16_t>(const f16_t* p) { return f16_bits_to_f32(p->bits); }

template <typename T> __device__ __forceinline__ void store_scalar(T* p, float v);
template <> __device__ __forceinline__ void store_scalar<float>(float* p, float v) { *p = v; }
template <> __device__ __forceinline__ void store_scalar<bf16_t>(bf16_t* p, float v) { p->bits = f32_to_bf16_bits(v); }
template <> __device__ __forceinline__ void store_scalar<f16_t>(f16_t* p, float v) { p->bits = f32_to_f16_bits(v); }

// Round an fp32 value through the storage type and back (models a cast to T).
template <typename T> __device__ __forceinline__ float round_to(float v);
template <> __device__ __forceinline__ float round_to<float>(float v) { return v; }
template <> __device__ __forceinline__ float round_to<bf16_t>(float v) {
  return __uint_as_float(uint32_t(f32_to_bf16_bits(v)) << 16);
}
template <> __device__ __forceinline__ float round_to<f16_t>(float v) { return (float)(_Float16)v; }

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 load16(const void* p) {
  const u32x4 r = *reinterpret_cast<const u32x4*>(p);
  return make_uint4(r.x, r.y, r.z, r.w);
}

// Streaming 16-byte load for data read once per call (the KV cache).
__device__ __forceinline__ uint4 load16_stream(const void* p) {
  const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(r.x, r.y, r.z, r.w);
}

// The 32-bit value of lane (lane ^ M), exchanged on the VALU rather than
// through an LDS permute (ds_bpermute, which __shfl_xor compiles to, adds an
// LDS round trip per exchange): DPP inside each row of 16 lanes --
// quad_perm [1,0,3,2] and [2,3,0,1] for M = 1, 2, row_shl:4 / row_shr:4 picked
// per lane for M = 4, row_ror:8 for M = 8 -- and the gfx950 lane swaps across
// rows: v_permlane16_swap / v_permlane32_swap of a value with itself leave the
// even row's (lower half's) value in the first result and the odd row's (upper
// half's) in the second, so a lane takes the one that is not its own. Every
// lane of the wave must be active.
template <int M>
__device__ __forceinline__ uint32_t lane_xor_bits(uint32_t x) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "lane mask");
  if constexpr (M == 1) {
    return __builtin_amdgcn_update_dpp(0, int(x), 0xB1, 0xF, 0xF, true);
  } else if constexpr (M == 2) {
    return __builtin_amdgcn_update_dpp(0, int(x), 0x4E, 0xF, 0xF, true);
  } else if constexpr (M == 4) {
    const uint32_t up = __builtin_amdgcn_update_dpp(0, int(x), 0x104, 0xF, 0xF, true);  // lane + 4
    const uint32_t dn = __builtin_amdgcn_update_dpp(0, int(x), 0x114, 0xF, 0xF, true);  // lane - 4
    return (__lane_id() & 4) ? dn : up;
  } else if constexpr (M == 8) {
    return __builtin_amdgcn_update_dpp(0, int(x), 0x128, 0xF, 0xF, true);
  } else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (__lane_id() & 16) ? r[0] : r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (__lane_id() & 32) ? r[0] : r[1];
  }
}

// lane_xor_bits for a mask known after unrolling (a constant-folded switch).
__device__ __forceinline__ uint32_t lane_xor_bits(uint32_t x, int m) {
  switch (m) {
    case 1: return lane_xor_bits<1>(x);
    case 2: return lane_xor_bits<2>(x);
    case 4: return lane_xor_bits<4>(x);
    case 8: return lane_xor_bits<8>(x);
    case 16: return lane_xor_bits<16>(x);
    default: return lane_xor_bits<32>(x);
  }
}
__device__ __forceinline__ float lane_xor(float v, int m) { return __uint_as_float(lane_xor_bits(__float_as_uint(v), m)); }
__device__ __forceinline__ int lane_xor(int v, int m) { return int(lane_xor_bits(uint32_t(v), m)); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, lane_xor(v, m));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += lane_xor(v, m);
  return v;
}

// Sum over aligned groups of `Width` lanes (Width a power of two <= 64).
template <int Width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = Width / 2; m >= 1; m >>= 1) v += lane_xor(v, m);
  return v;
}

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace sfl

// Host-side status plumbing shared by every entry point.
namespace sfl {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
}  // namespace sfl
