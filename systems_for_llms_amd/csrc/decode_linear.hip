// Decode-step projections as MFMA GEMVs with fused prologues and epilogues.
//
// Every kernel computes out[b, n] = sum_k act[b, k] * W[n, k] for a batch of
// at most 16 rows (one decode token per sequence), with W stored [N, K]
// K-contiguous as the reference's Linear keeps it (src/llmlab/model/layers.py:34-35).
// A workgroup owns 16 output features; its waves split K, stream their weight
// slices straight from HBM into MFMA A-operand registers (16 bytes per lane)
// and feed the activations as the B operand; partial tiles are summed across
// waves in LDS. The MFMA result layout puts 4 consecutive features of one
// batch row in each lane, so RoPE pairs, SwiGLU pairs and vector stores stay
// in-lane.
//
// Precision: weights and the KV cache are in the model dtype; activations,
// the residual stream and every epilogue stay in fp32. For bf16 weights each
// fp32 activation is split into hi + lo bf16 halves and multiplied by two
// MFMAs (the GEMV is bandwidth-bound, so the second MFMA is free), which keeps
// ~16 mantissa bits of the activation instead of 8.
//
// Prologue NORM: act = RMSNorm(x) from the fp32 residual stream, staged in LDS
// (layers.py:133-141: x / sqrt(mean(x^2) + eps) * w). Prologue plain: fp32
// activations read straight from global memory (each wave needs only its own
// K chunks, so there is nothing to share through LDS).
// Epilogues:
//   QKV      RoPE on q and k (attention.py:44-58) with the host-built fp32
//            table; q to an fp32 [B, H, dk] buffer, k/v appended to the
//            model-dtype [B, H, cap, dk] cache at each row's position.
//   RESIDUAL x += W act (transformer.py:46-47).
//   SWIGLU   h = silu(W1 act) * (W3 act) in fp32 (layers.py:114-115).
//   LOGITS   lm_head rows (transformer.py:137-138) plus a per-tile argmax with
//            the lowest index winning ties, taken on the fp32 accumulators.
#include "common.hpp"

namespace sfl {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum Epi { EPI_QKV = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2, EPI_LOGITS = 3 };

constexpr int kWaves = 8;       // waves per workgroup (K split)
constexpr int kTileN = 16;      // output features per workgroup
constexpr int kMaxRows = 16;    // batch rows per launch
constexpr int kChunkGroup = 8;  // weight chunks loaded per wave before computing
constexpr int kPadF = 4;        // LDS row padding (floats) against bank conflicts
constexpr float kEps = 1e-5f;

struct LinearArgs {
  const float* x;        // fp32 residual [B, K] (NORM prologue) / residual base (RESIDUAL)
  const void* act;       // fp32 activations [B, K] (plain prologue)
  const void* norm_w;    // [K]
  const void* w;         // [N, K]
  const void* w3;        // [N, K] second matrix of SWIGLU
  int batch, n, k;
  // QKV
  const float* cos_t;    // [ctx, dk/2] fp32
  const float* sin_t;
  const int32_t* pos;    // [B]
  void* q_out;           // fp32 [B, H, dk]
  void* k_cache;         // [B, H, cap, dk]
  void* v_cache;
  int heads, head_dim, cap, d_model;
  // RESIDUAL
  float* x_out;          // [B, N]
  // SWIGLU
  void* h_out;           // fp32 [B, N]
  // LOGITS
  void* logits;          // fp32 [B, V], optional; row offset pos[b]*logits_pos_stride
  long logits_batch_stride;
  long logits_pos_stride;
  float* best_val;       // [tiles, best_stride]
  int32_t* best_idx;
  int best_stride;
};

// One 16-byte weight chunk of K covers 4 lane groups of vec_elems<T>() values.
template <typename T> constexpr int chunk_k() { return 4 * vec_elems<T>(); }

template <typename T>
__device__ __forceinline__ f32x4 mfma_chunk(const uint4& a, const u32x4& b, f32x4 acc);

template <>
__device__ __forceinline__ f32x4 mfma_chunk<bf16_t>(const uint4& a, const u32x4& b, f32x4 acc) {
  const u32x4 av = {a.x, a.y, a.z, a.w};
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                 __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
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

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// B operand of one chunk from 16 bytes' worth of fp32 activations (8 values for
// bf16, 4 for fp32). bf16 splits each value into hi + lo bf16 parts so the
// activation enters the product with ~16 mantissa bits; fp32 passes through.
template <typename T>
__device__ __forceinline__ f32x4 mfma_act(const uint4& w, const float* f, f32x4 acc);

template <>
__device__ __forceinline__ f32x4 mfma_act<bf16_t>(const uint4& w, const float* f, f32x4 acc) {
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint16_t h0 = f32_to_bf16_bits(f[2 * j]), h1 = f32_to_bf16_bits(f[2 * j + 1]);
    const uint16_t l0 = f32_to_bf16_bits(f[2 * j] - __uint_as_float(uint32_t(h0) << 16));
    const uint16_t l1 = f32_to_bf16_bits(f[2 * j + 1] - __uint_as_float(uint32_t(h1) << 16));
    hi[j] = uint32_t(h0) | (uint32_t(h1) << 16);
    lo[j] = uint32_t(l0) | (uint32_t(l1) << 16);
  }
  const u32x4 bh = {hi[0], hi[1], hi[2], hi[3]};
  const u32x4 bl = {lo[0], lo[1], lo[2], lo[3]};
  acc = mfma_chunk<bf16_t>(w, bh, acc);
  return mfma_chunk<bf16_t>(w, bl, acc);
}

template <>
__device__ __forceinline__ f32x4 mfma_act<float>(const uint4& w, const float* f, f32x4 acc) {
  const u32x4 b = {__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])};
  return mfma_chunk<float>(w, b, acc);
}

template <typename T, int E, bool NORM>
__global__ __launch_bounds__(kWaves * kWave) void linear_kernel(LinearArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int EPL = vec_elems<T>();  // k values per lane per chunk
  constexpr int KC = chunk_k<T>();
  constexpr bool kTwo = (E == EPI_SWIGLU);
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int K = a.k;
  const int ldk = K + kPadF;
  float* act_s = reinterpret_cast<float*>(smem);
  float* red = act_s + (NORM ? kMaxRows * ldk : 0);

  const int n0 = blockIdx.x * kTileN;
  const int row = min(n0 + lane % 16, a.n - 1);
  const int grp = lane / 16;
  const int b = lane % 16;
  const T* wrow = static_cast<const T*>(a.w) + long(row) * K + grp * EPL;
  const T* w3row = kTwo ? static_cast<const T*>(a.w3) + long(row) * K + grp * EPL : nullptr;
  // Plain prologue: this lane's fp32 activation row, read straight from global memory.
  const float* arow = static_cast<const float*>(a.act) + long(min(b, a.batch - 1)) * K + grp * EPL;
  const bool live = b < a.batch;
  const int nchunks = K / KC;

  // Issue the first group of weight (and plain activation) loads up front.
  uint4 wa[kChunkGroup], wb[kTwo ? kChunkGroup : 1];
  float af[NORM ? 1 : kChunkGroup][NORM ? 1 : EPL];
  int c0 = wave;
#pragma unroll
  for (int j = 0; j < kChunkGroup; ++j) {
    const int c = c0 + j * kWaves;
    if (c < nchunks) {
      wa[j] = load16(wrow + long(c) * KC);
      if constexpr (kTwo) wb[j] = load16(w3row + long(c) * KC);
      if constexpr (!NORM) {
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
          const float4 v = *reinterpret_cast<const float4*>(arow + long(c) * KC + e);
          af[j][e] = live ? v.x : 0.f; af[j][e + 1] = live ? v.y : 0.f;
          af[j][e + 2] = live ? v.z : 0.f; af[j][e + 3] = live ? v.w : 0.f;
        }
      }
    }
  }

  if constexpr (NORM) {
    // RMSNorm rows in fp32 into LDS (layers.py:133-141); pad rows are zero.
    const T* nw = static_cast<const T*>(a.norm_w);
    for (int r = wave; r < kMaxRows; r += kWaves) {
      float* dst = act_s + r * ldk;
      if (r < a.batch) {
        const float* xr = a.x + long(r) * K;
        float ss = 0.f;
        for (int i = lane; i < K; i += kWave) ss = fmaf(xr[i], xr[i], ss);
        ss = wave_sum(ss);
        const float rms = sqrtf(ss / float(K) + kEps);
        for (int i = lane; i < K; i += kWave) dst[i] = (xr[i] / rms) * load_scalar<T>(nw + i);
      } else {
        for (int i = lane; i < K; i += kWave) dst[i] = 0.f;
      }
    }
    __syncthreads();
  }

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc3 = {0.f, 0.f, 0.f, 0.f};
  const float* bsrc = act_s + b * ldk + grp * EPL;
  for (;;) {
#pragma unroll
    for (int j = 0; j < kChunkGroup; ++j) {
      const int c = c0 + j * kWaves;
      if (c < nchunks) {
        float f[EPL];
        if constexpr (NORM) {
#pragma unroll
          for (int e = 0; e < EPL; e += 4) {
            const float4 v = *reinterpret_cast<const float4*>(bsrc + c * KC + e);
            f[e] = v.x; f[e + 1] = v.y; f[e + 2] = v.z; f[e + 3] = v.w;
          }
        } else {
#pragma unroll
          for (int e = 0; e < EPL; ++e) f[e] = af[j][e];
        }
        acc = mfma_act<T>(wa[j], f, acc);
        if constexpr (kTwo) acc3 = mfma_act<T>(wb[j], f, acc3);
      }
    }
    c0 += kChunkGroup * kWaves;
    if (c0 >= nchunks) break;
#pragma unroll
    for (int j = 0; j < kChunkGroup; ++j) {
      const int c = c0 + j * kWaves;
      if (c < nchunks) {
        wa[j] = load16(wrow + long(c) * KC);
        if constexpr (kTwo) wb[j] = load16(w3row + long(c) * KC);
        if constexpr (!NORM) {
#pragma unroll
          for (int e = 0; e < EPL; e += 4) {
            const float4 v = *reinterpret_cast<const float4*>(arow + long(c) * KC + e);
            af[j][e] = live ? v.x : 0.f; af[j][e + 1] = live ? v.y : 0.f;
            af[j][e + 2] = live ? v.z : 0.f; af[j][e + 3] = live ? v.w : 0.f;
          }
        }
      }
    }
  }

  // Sum the waves' partial tiles.
  float* mine = red + (wave * kWave + lane) * (kTwo ? 8 : 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    mine[i] = acc[i];
    if constexpr (kTwo) mine[4 + i] = acc3[i];
  }
  __syncthreads();
  if (wave != 0) return;
  float v1[4] = {0.f, 0.f, 0.f, 0.f}, v3[4] = {0.f, 0.f, 0.f, 0.f};
  for (int w = 0; w < kWaves; ++w) {
    const float* p = red + (w * kWave + lane) * (kTwo ? 8 : 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v1[i] += p[i];
      if constexpr (kTwo) v3[i] += p[4 + i];
    }
  }

  const int n = n0 + 4 * grp;  // this lane's features n .. n+3 of batch row b
  if constexpr (E == EPI_LOGITS) {
    // Start from a valid index so a row of NaN logits still yields an in-range token.
    float bv = -INFINITY;
    int bi = min(n, a.n - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (n + i < a.n && better(v1[i], n + i, bv, bi)) { bv = v1[i]; bi = n + i; }
    }
#pragma unroll
    for (int m = 16; m < kWave; m <<= 1) {
      const float ov = __shfl_xor(bv, m, kWave);
      const int oi = __shfl_xor(bi, m, kWave);
      if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (live) {
      if (grp == 0) {
        a.best_val[long(blockIdx.x) * a.best_stride + b] = bv;
        a.best_idx[long(blockIdx.x) * a.best_stride + b] = bi;
      }
      if (a.logits && n < a.n) {
        float* dst = static_cast<float*>(a.logits) + b * a.logits_batch_stride + n;
        if (a.pos) dst += long(a.pos[b]) * a.logits_pos_stride;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n + i < a.n) dst[i] = v1[i];
      }
    }
    return;
  }
  if (!live || n >= a.n) return;
  if constexpr (E == EPI_RESIDUAL) {
    const float* xr = a.x + long(b) * a.n + n;
    float* xo = a.x_out + long(b) * a.n + n;
#pragma unroll
    for (int i = 0; i < 4; ++i) xo[i] = xr[i] + v1[i];
  } else if constexpr (E == EPI_SWIGLU) {
    float h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = v1[i] / (1.f + expf(-v1[i])) * v3[i];
    float* dst = static_cast<float*>(a.h_out) + long(b) * a.n + n;
    *reinterpret_cast<float4*>(dst) = make_float4(h[0], h[1], h[2], h[3]);
  } else {  // EPI_QKV
    const int section = n / a.d_model;  // 0 q, 1 k, 2 v
    const int f = n % a.d_model;
    const int head = f / a.head_dim;
    const int dim = f % a.head_dim;
    const int p = a.pos[b];
    float y[4] = {v1[0], v1[1], v1[2], v1[3]};
    if (section < 2) {
      const int half = a.head_dim / 2;
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const int pair = (dim + i) / 2;
        const float c = a.cos_t[long(p) * half + pair];
        const float s = a.sin_t[long(p) * half + pair];
        const float e = y[i], o = y[i + 1];
        y[i] = e * c - o * s;
        y[i + 1] = e * s + o * c;
      }
    }
    if (section == 0) {
      float* dst = static_cast<float*>(a.q_out) + (long(b) * a.heads + head) * a.head_dim + dim;
      *reinterpret_cast<float4*>(dst) = make_float4(y[0], y[1], y[2], y[3]);
    } else {
      T* cache = static_cast<T*>(section == 1 ? a.k_cache : a.v_cache);
      store4<T>(cache + ((long(b) * a.heads + head) * a.cap + p) * a.head_dim + dim, y);
    }
  }
}

template <typename T, int E, bool NORM>
int launch_linear(const LinearArgs& a, hipStream_t stream, const char* what) {
  const size_t lds = (NORM ? size_t(kMaxRows) * (a.k + kPadF) * sizeof(float) : 0) +
                     size_t(kWaves) * kWave * (E == EPI_SWIGLU ? 8 : 4) * sizeof(float);
  if (lds > 160 * 1024)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: K=%d needs %zu bytes of LDS (max 163840)", what, a.k, lds);
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&linear_kernel<T, E, NORM>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    attr_set = true;
  }
  const unsigned tiles = unsigned((a.n + kTileN - 1) / kTileN);
  hipLaunchKernelGGL((linear_kernel<T, E, NORM>), dim3(tiles), dim3(kWaves * kWave), lds, stream, a);
  return check_launch(what);
}

int check_common(const char* what, int batch, int n, int k, int dtype) {
  if (batch < 1 || batch > kMaxRows)
    return set_error(SFL_ERR_INVALID, "%s: batch must be in [1, %d] per launch", what, kMaxRows);
  if (n < 1 || k < 1) return set_error(SFL_ERR_INVALID, "%s: sizes must be positive", what);
  if (dtype != SFL_DTYPE_F32 && dtype != SFL_DTYPE_BF16)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: model dtype must be F32 or BF16", what);
  const int kc = dtype == SFL_DTYPE_BF16 ? chunk_k<bf16_t>() : chunk_k<float>();
  if (k % kc) return set_error(SFL_ERR_UNSUPPORTED, "%s: K=%d must be a multiple of %d", what, k, kc);
  return SFL_OK;
}

template <int E, bool NORM>
int dispatch_linear(const LinearArgs& a, int dtype, hipStream_t s, const char* what) {
  if (dtype == SFL_DTYPE_BF16) return launch_linear<bf16_t, E, NORM>(a, s, what);
  return launch_linear<float, E, NORM>(a, s, what);
}

}  // namespace
}  // namespace sfl

using namespace sfl;

extern "C" int sfl_rmsnorm_qkv_rope_append(const float* x, const void* norm_w, const void* w_qkv,
                                           const float* cos_t, const float* sin_t,
                                           const int32_t* pos, void* q_out, void* k_cache,
                                           void* v_cache, int batch, int d_model, int heads,
                                           int capacity, int dtype, void* stream) {
  const char* what = "rmsnorm_qkv_rope_append";
  if (!x || !norm_w || !w_qkv || !cos_t || !sin_t || !pos || !q_out || !k_cache || !v_cache)
    return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (heads < 1 || d_model % heads) return set_error(SFL_ERR_INVALID, "%s: d_model must be divisible by heads", what);
  const int dk = d_model / heads;
  if (dk % 16) return set_error(SFL_ERR_UNSUPPORTED, "%s: head dim must be a multiple of 16", what);
  if (capacity < 1) return set_error(SFL_ERR_INVALID, "%s: capacity must be positive", what);
  if (int rc = check_common(what, batch, 3 * d_model, d_model, dtype)) return rc;
  LinearArgs a{};
  a.x = x; a.norm_w = norm_w; a.w = w_qkv; a.batch = batch; a.n = 3 * d_model; a.k = d_model;
  a.cos_t = cos_t; a.sin_t = sin_t; a.pos = pos; a.q_out = q_out; a.k_cache = k_cache;
  a.v_cache = v_cache; a.heads = heads; a.head_dim = dk; a.cap = capacity; a.d_model = d_model;
  return dispatch_linear<EPI_QKV, true>(a, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_linear_residual(const void* act, const void* w, const float* x, float* x_out,
                                   int batch, int n, int k, int dtype, void* stream) {
  const char* what = "linear_residual";
  if (!act || !w || !x || !x_out) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (int rc = check_common(what, batch, n, k, dtype)) return rc;
  if (n % 4) return set_error(SFL_ERR_UNSUPPORTED, "%s: N must be a multiple of 4", what);
  LinearArgs a{};
  a.act = act; a.w = w; a.x = x; a.x_out = x_out; a.batch = batch; a.n = n; a.k = k;
  return dispatch_linear<EPI_RESIDUAL, false>(a, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_rmsnorm_swiglu(const float* x, const void* norm_w, const void* w1, const void* w3,
                                  void* h_out, int batch, int d_model, int d_ff, int dtype,
                                  void* stream) {
  const char* what = "rmsnorm_swiglu";
  if (!x || !norm_w || !w1 || !w3 || !h_out) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (int rc = check_common(what, batch, d_ff, d_model, dtype)) return rc;
  if (d_ff % 4) return set_error(SFL_ERR_UNSUPPORTED, "%s: d_ff must be a multiple of 4", what);
  LinearArgs a{};
  a.x = x; a.norm_w = norm_w; a.w = w1; a.w3 = w3; a.h_out = h_out; a.batch = batch; a.n = d_ff;
  a.k = d_model;
  return dispatch_linear<EPI_SWIGLU, true>(a, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_rmsnorm_lm_head(const float* x, const void* norm_w, const void* w_head,
                                   void* logits, long logits_batch_stride, const int32_t* pos,
                                   long logits_pos_stride, float* best_val, int32_t* best_idx,
                                   int best_stride, int batch, int d_model, int vocab, int dtype,
                                   void* stream) {
  const char* what = "rmsnorm_lm_head";
  if (!x || !norm_w || !w_head || !best_val || !best_idx)
    return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (int rc = check_common(what, batch, vocab, d_model, dtype)) return rc;
  if (best_stride < batch) return set_error(SFL_ERR_INVALID, "%s: best_stride must be >= batch", what);
  LinearArgs a{};
  a.x = x; a.norm_w = norm_w; a.w = w_head; a.logits = logits; a.logits_batch_stride = logits_batch_stride;
  a.pos = pos; a.logits_pos_stride = logits_pos_stride; a.best_val = best_val; a.best_idx = best_idx;
  a.best_stride = best_stride;
  a.batch = batch; a.n = vocab; a.k = d_model;
  return dispatch_linear<EPI_LOGITS, true>(a, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_lm_head_tiles(int vocab) { return (vocab + kTileN - 1) / kTileN; }
