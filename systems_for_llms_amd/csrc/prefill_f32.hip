// Prefill of float32 models: the Linear layers as fp32 MFMA GEMMs and causal
// attention in fp32, so a float32 forward over T positions is one pass.
//
// The reference's float32 TransformerLM.forward (src/llmlab/model/
// transformer.py:121-139) runs every Linear (layers.py:34-35) and the
// attention (attention.py:61-98,187-197) in fp32; these kernels keep every
// product and sum in fp32, so they differ from it only by the order of fp32
// additions.
//
// GEMM: C^T[n][m] = sum_k W[n][k] A[m][k] on v_mfma_f32_32x32x2_f32 (fp32
// operands, fp32 accumulation). A workgroup of 4 waves (2 x 2) computes 64
// features x 64 tokens, a wave one 32 x 32 block; K advances by 32 through two
// LDS stages (rows padded to 36 floats), the next stage's global loads in
// registers while the current one computes. A lane reads 16 bytes -- 4
// consecutive k of its row -- per operand and feeds them to 4 MFMAs: lane
// half h takes k = 8 kq + 4 h + s in step s for both operands, so each
// product pairs equal k (the contraction is exact in any shared order). The
// output layout of the 32x32 MFMA puts features 8q + 4h .. +3 of one token in
// a lane, so the epilogues of the 16-bit GEMMs carry over: RoPE pairs in-lane,
// W1/W3 interleaved in blocks of 8 rows paired in-lane, 16-byte stores.
//
// Attention: one workgroup of 256 threads per 64 queries of one (batch, head);
// four threads per query, each holding a quarter of the head dim of q and of
// the output. Key/value tiles of 32 rows are staged in LDS; for each key the
// four threads add their partial dot products with two shuffles and update an
// exact fp32 online softmax (base 2, the scale folded into q).
#include <math.h>

#include "gemm_f32.hpp"

namespace sfl {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int FT = 64;        // features and tokens per workgroup
constexpr int FK = 32;        // K per LDS stage
constexpr int FLD = FK + 4;   // LDS row stride (floats)
constexpr int kF32Threads = 256;

__device__ __forceinline__ f32x16 mfma32f(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// silu(a) * c with an IEEE exponential (layers.py:102-104,114-115).
__device__ __forceinline__ float silu_mul_f32(float a, float c) { return a / (1.f + expf(-a)) * c; }

template <int E>
__global__ __launch_bounds__(kF32Threads) void gemm_f32_kernel(F32GemmArgs g) {
  __shared__ __align__(16) float ws[2][FT * FLD];
  __shared__ __align__(16) float as[2][FT * FLD];
  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int wn = wave / 2, wm = wave % 2;
  const int l32 = lane % 32, hf = lane / 32;
  const int n0 = blockIdx.x * FT;
  const int m0 = blockIdx.y * FT;
  const int ksteps = (g.k + FK - 1) / FK;

  // Thread tid moves row r = idx / 8, floats 4 c4 .. +3 of a stage, idx = tid + 256 i.
  // Loads are unconditional from clamped rows; columns past K are zeroed per
  // component (a select of whole float4 values is lowered through scratch).
  float4 wr[2], ar[2];
#define SFL_F32_GLOAD(kt)                                                                   \
  _Pragma("unroll") for (int i = 0; i < 2; ++i) {                                           \
    const int idx = tid + i * kF32Threads;                                                  \
    const int r = idx / (FK / 4), c4 = idx % (FK / 4);                                      \
    const int kk = (kt) * FK + 4 * c4;                                                      \
    const bool in = kk < g.k;                                                               \
    const int kc = in ? kk : 0;                                                             \
    const float4 w_ = *reinterpret_cast<const float4*>(g.w + long(min(n0 + r, g.n - 1)) * g.k + kc); \
    const float4 a_ = *reinterpret_cast<const float4*>(g.a + long(min(m0 + r, g.m - 1)) * g.k + kc); \
    wr[i] = make_float4(in ? w_.x : 0.f, in ? w_.y : 0.f, in ? w_.z : 0.f, in ? w_.w : 0.f);  \
    ar[i] = make_float4(in ? a_.x : 0.f, in ? a_.y : 0.f, in ? a_.z : 0.f, in ? a_.w : 0.f);  \
  }
#define SFL_F32_SSTORE(buf)                                                                 \
  _Pragma("unroll") for (int i = 0; i < 2; ++i) {                                           \
    const int idx = tid + i * kF32Threads;                                                  \
    const int r = idx / (FK / 4), c4 = idx % (FK / 4);                                      \
    *reinterpret_cast<float4*>(&ws[buf][r * FLD + 4 * c4]) = wr[i];                         \
    *reinterpret_cast<float4*>(&as[buf][r * FLD + 4 * c4]) = ar[i];                         \
  }

  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  SFL_F32_GLOAD(0)
  SFL_F32_SSTORE(0)
  __syncthreads();
  for (int kt = 0; kt < ksteps; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ksteps) { SFL_F32_GLOAD(kt + 1) }
    const float* wrow = &ws[buf][(32 * wn + l32) * FLD + 4 * hf];
    const float* arow = &as[buf][(32 * wm + l32) * FLD + 4 * hf];
#pragma unroll
    for (int kq = 0; kq < FK / 8; ++kq) {
      const float4 av = *reinterpret_cast<const float4*>(wrow + 8 * kq);
      const float4 bv = *reinterpret_cast<const float4*>(arow + 8 * kq);
      acc = mfma32f(av.x, bv.x, acc);
      acc = mfma32f(av.y, bv.y, acc);
      acc = mfma32f(av.z, bv.z, acc);
      acc = mfma32f(av.w, bv.w, acc);
    }
    if (kt + 1 < ksteps) {
      SFL_F32_SSTORE(buf ^ 1)
      __syncthreads();
    }
  }
#undef SFL_F32_GLOAD
#undef SFL_F32_SSTORE

  // acc[4q + e] holds feature n0 + 32 wn + 8q + 4hf + e of token m0 + 32 wm + l32.
  const int m = m0 + 32 * wm + l32;
  if (m >= g.m) return;
  const int nt = n0 + 32 * wn;
  if constexpr (E == F32_SWIGLU) {
    // Groups q = 0, 2 are W1 rows, q + 1 the W3 rows of the same hidden features
    // nt/2 + 4q + 4hf .. +3.
#pragma unroll
    for (int q = 0; q < 4; q += 2) {
      const int f = nt / 2 + 4 * q + 4 * hf;
      if (f >= g.n / 2) continue;
      float h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = silu_mul_f32(acc[4 * q + e], acc[4 * q + 4 + e]);
      *reinterpret_cast<float4*>(g.h_out + long(m) * (g.n / 2) + f) = make_float4(h[0], h[1], h[2], h[3]);
    }
  } else if constexpr (E == F32_QKV) {
    const int b = m / g.seq, t = m - (m / g.seq) * g.seq;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = nt + 8 * q + 4 * hf;
      if (n >= g.n) continue;
      const int section = n / g.d_model;
      const int fi = n - section * g.d_model;
      const int head = fi / g.head_dim, dim = fi - (fi / g.head_dim) * g.head_dim;
      float y[4] = {acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
      if (section < 2) {  // RoPE pairs (dim, dim+1), (dim+2, dim+3) (attention.py:44-58)
        const long r0 = long(dim / 2) * g.cap + t;
        const float c0 = g.cos_t[r0], c1 = g.cos_t[r0 + g.cap];
        const float s0 = g.sin_t[r0], s1 = g.sin_t[r0 + g.cap];
        const float e0 = y[0], o0 = y[1], e1 = y[2], o1 = y[3];
        y[0] = e0 * c0 - o0 * s0;
        y[1] = e0 * s0 + o0 * c0;
        y[2] = e1 * c1 - o1 * s1;
        y[3] = e1 * s1 + o1 * c1;
      }
      float* dst = section == 0 ? g.q_out + ((long(b) * g.heads + head) * g.seq + t) * g.head_dim + dim
                                : (section == 1 ? g.k_cache : g.v_cache) +
                                      ((long(b) * g.heads + head) * g.cap + t) * g.head_dim + dim;
      *reinterpret_cast<float4*>(dst) = make_float4(y[0], y[1], y[2], y[3]);
    }
  } else {  // F32_PLAIN
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = nt + 8 * q + 4 * hf;
      float* c = g.c + long(m) * g.n + n;
      if (n + 3 < g.n && (g.n & 3) == 0) {
        float4 v = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
        if (g.accumulate) {
          const float4 old = *reinterpret_cast<const float4*>(c);
          v = make_float4(old.x + v.x, old.y + v.y, old.z + v.z, old.w + v.w);
        }
        *reinterpret_cast<float4*>(c) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < g.n) c[e] = (g.accumulate ? c[e] : 0.f) + acc[4 * q + e];
      }
    }
  }
}

struct F32AttnArgs {
  const float *q, *k, *v;
  float* o;
  long qs[3], ks[3], vs[3], os[3];  // strides (elements) of batch, head, sequence
  int batch, heads, n;
  float scale_log2;
};

constexpr int kAttnQ = 64;   // queries per workgroup
constexpr int kAttnK = 32;   // keys per LDS tile

template <int D>
__global__ __launch_bounds__(kF32Threads) void causal_attention_f32_kernel(F32AttnArgs a) {
  constexpr int DQ = D / 4;  // head-dim quarter of a thread
  __shared__ __align__(16) float kt[kAttnK][D];
  __shared__ __align__(16) float vt[kAttnK][D];
  const int nqb = (a.n + kAttnQ - 1) / kAttnQ;
  const int qb = nqb - 1 - int(blockIdx.x % nqb);  // longest rows first
  const int bh = int(blockIdx.x / nqb);
  const int b = bh / a.heads, h = bh % a.heads;
  const int tid = threadIdx.x;
  const int qrow = qb * kAttnQ + tid / 4, part = tid % 4;
  const float* qp = a.q + b * a.qs[0] + h * a.qs[1] + long(min(qrow, a.n - 1)) * a.qs[2] + part * DQ;
  float qv[DQ], o[DQ];
#pragma unroll
  for (int d = 0; d < DQ; ++d) {
    qv[d] = qp[d] * a.scale_log2;
    o[d] = 0.f;
  }
  float m_run = -INFINITY, l_run = 0.f;
  const int kend = min(a.n, qb * kAttnQ + kAttnQ);  // keys 0 .. kend-1 cover every row of the block
  const float* kb = a.k + b * a.ks[0] + h * a.ks[1];
  const float* vb = a.v + b * a.vs[0] + h * a.vs[1];
  for (int k0 = 0; k0 < kend; k0 += kAttnK) {
    __syncthreads();
    for (int idx = tid; idx < kAttnK * D / 4; idx += kF32Threads) {
      const int r = idx / (D / 4), c4 = idx % (D / 4);
      const long key = min(k0 + r, a.n - 1);
      *reinterpret_cast<float4*>(&kt[r][4 * c4]) = *reinterpret_cast<const float4*>(kb + key * a.ks[2] + 4 * c4);
      *reinterpret_cast<float4*>(&vt[r][4 * c4]) = *reinterpret_cast<const float4*>(vb + key * a.vs[2] + 4 * c4);
    }
    __syncthreads();
    const int jn = min(kAttnK, kend - k0);  // uniform over the workgroup
    for (int j = 0; j < jn; ++j) {
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < DQ; ++d) s = fmaf(qv[d], kt[j][part * DQ + d], s);
      s += lane_xor(s, 1);
      s += lane_xor(s, 2);
      if (k0 + j <= qrow) {  // causal (attention.py:187-197)
        if (s > m_run) {
          const float alpha = exp2f(m_run - s);  // 0 for the first key
          l_run *= alpha;
#pragma unroll
          for (int d = 0; d < DQ; ++d) o[d] *= alpha;
          m_run = s;
        }
        const float p = exp2f(s - m_run);
        l_run += p;
#pragma unroll
        for (int d = 0; d < DQ; ++d) o[d] = fmaf(p, vt[j][part * DQ + d], o[d]);
      }
    }
  }
  if (qrow >= a.n) return;
  const float inv = 1.f / l_run;  // key 0 is always admissible: l_run >= 1
  float* op = a.o + b * a.os[0] + h * a.os[1] + long(qrow) * a.os[2] + part * DQ;
#pragma unroll
  for (int d = 0; d < DQ; d += 4)
    *reinterpret_cast<float4*>(op + d) = make_float4(o[d] * inv, o[d + 1] * inv, o[d + 2] * inv, o[d + 3] * inv);
}

}  // namespace

int launch_gemm_f32(const F32GemmArgs& g, int epi, hipStream_t stream, const char* what) {
  if (g.m < 1 || g.n < 1 || g.k < 1) return set_error(SFL_ERR_INVALID, "%s: sizes must be positive", what);
  if (g.k % 4) return set_error(SFL_ERR_UNSUPPORTED, "%s: fp32 K must be a multiple of 4", what);
  const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (!a16(g.a) || !a16(g.w))
    return set_error(SFL_ERR_INVALID, "%s: fp32 operands must be 16-byte aligned", what);
  const dim3 grid(unsigned((g.n + FT - 1) / FT), unsigned((g.m + FT - 1) / FT));
  if (grid.y > 65535) return set_error(SFL_ERR_UNSUPPORTED, "%s: M too large", what);
  switch (epi) {
    case F32_QKV: hipLaunchKernelGGL(gemm_f32_kernel<F32_QKV>, grid, dim3(kF32Threads), 0, stream, g); break;
    case F32_SWIGLU: hipLaunchKernelGGL(gemm_f32_kernel<F32_SWIGLU>, grid, dim3(kF32Threads), 0, stream, g); break;
    default: hipLaunchKernelGGL(gemm_f32_kernel<F32_PLAIN>, grid, dim3(kF32Threads), 0, stream, g); break;
  }
  return check_launch(what);
}

}  // namespace sfl

using namespace sfl;

extern "C" int sfl_causal_attention_f32(const float* q, const float* k, const float* v, float* o, int batch,
                                        int heads, int n, int head_dim, const long* q_strides,
                                        const long* k_strides, const long* v_strides, const long* o_strides,
                                        float scale, void* stream) {
  const char* what = "causal_attention_f32";
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides)
    return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (batch < 1 || heads < 1 || n < 1) return set_error(SFL_ERR_INVALID, "%s: sizes must be positive", what);
  if (!(scale > 0.f) || !__builtin_isfinite(scale))
    return set_error(SFL_ERR_INVALID, "%s: scale must be finite and positive", what);
  for (int i = 0; i < 3; ++i)
    if (q_strides[i] < 0 || k_strides[i] < 0 || v_strides[i] < 0 || o_strides[i] < 0)
      return set_error(SFL_ERR_INVALID, "%s: strides must be non-negative", what);
  const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  bool aligned = a16(k) && a16(v) && a16(o);
  for (int i = 0; i < 3; ++i) aligned = aligned && k_strides[i] % 4 == 0 && v_strides[i] % 4 == 0 && o_strides[i] % 4 == 0;
  if (!aligned) return set_error(SFL_ERR_INVALID, "%s: k, v and o rows must be 16-byte aligned", what);
  if (long((n + kAttnQ - 1) / kAttnQ) * batch * heads > (1L << 31) - 1)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: too many query blocks", what);
  F32AttnArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o;
  for (int i = 0; i < 3; ++i) {
    a.qs[i] = q_strides[i]; a.ks[i] = k_strides[i]; a.vs[i] = v_strides[i]; a.os[i] = o_strides[i];
  }
  a.batch = batch; a.heads = heads; a.n = n; a.scale_log2 = scale * kLog2e;
  const dim3 grid(unsigned((n + kAttnQ - 1) / kAttnQ) * unsigned(batch * heads));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (head_dim) {
    case 16: hipLaunchKernelGGL(causal_attention_f32_kernel<16>, grid, dim3(kF32Threads), 0, s, a); break;
    case 32: hipLaunchKernelGGL(causal_attention_f32_kernel<32>, grid, dim3(kF32Threads), 0, s, a); break;
    case 64: hipLaunchKernelGGL(causal_attention_f32_kernel<64>, grid, dim3(kF32Threads), 0, s, a); break;
    case 128: hipLaunchKernelGGL(causal_attention_f32_kernel<128>, grid, dim3(kF32Threads), 0, s, a); break;
    default: return set_error(SFL_ERR_UNSUPPORTED, "%s: head dim must be 16, 32, 64 or 128", what);
  }
  return check_launch(what);
}
