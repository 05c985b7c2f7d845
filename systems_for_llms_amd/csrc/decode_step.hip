// Token-loop bookkeeping kernels: embedding gather and the greedy next-token step.
//
// The reference has no token loop (its forward always recomputes from
// position 0, src/llmlab/model/transformer.py:121-139); its greedy
// continuation is argmax(forward(ids)[:, -1]), and torch.argmax returns the
// first maximal index. These kernels keep the whole loop on the device so a
// decode step can be captured once and replayed: the next token, the position
// and the attention lengths are advanced in place.
#include "act_format.hpp"

namespace sfl {
namespace {

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// x[b, :] = emb[tokens[b, pos[b]], :] as fp32 (Embedding.forward, layers.py:68-70).
template <typename T>
__global__ __launch_bounds__(256) void embed_kernel(const int64_t* __restrict__ tokens, long stride,
                                                    const int32_t* __restrict__ pos,
                                                    const T* __restrict__ emb, float* __restrict__ x,
                                                    int d) {
  const int b = blockIdx.x;
  const long id = tokens[b * stride + pos[b]];
  const T* src = emb + id * d;
  for (int i = threadIdx.x; i < d; i += blockDim.x) x[long(b) * d + i] = load_scalar<T>(src + i);
}

// One wave per sequence: finish the argmax over the lm_head tiles (lowest
// index on ties), record it, pick the next token (the given one while the
// sequence is still inside its prompt, else the argmax), gather its
// embedding into x (fp32) and advance pos/lengths. The arguments the first
// loads need come first (13 dwords, preloaded into SGPRs with the wave).
template <typename T>
__global__ __launch_bounds__(64) void next_token_kernel(
    const float* __restrict__ best_val, const int32_t* __restrict__ best_idx, int32_t* __restrict__ pos,
    int64_t* __restrict__ tokens, long stride, int tiles, int best_stride, int cap,
    int64_t* __restrict__ predicted, const int32_t* __restrict__ prompt_len, int32_t* __restrict__ lengths,
    const T* __restrict__ emb, float* __restrict__ x, int d) {
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const int p = pos[b];
  const int plen = prompt_len[b];
  const int np = p + 1;
  const long given = np < cap ? tokens[b * stride + np] : 0;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  // Issue kScan independent loads per lane per round (tiles <= 1024 in one round).
  constexpr int kScan = 16;
  for (int t0 = 0; t0 < tiles; t0 += kScan * kWave) {
    float v[kScan];
    int ix[kScan];
#pragma unroll
    for (int j = 0; j < kScan; ++j) {  // unconditional loads from clamped tiles
      const long t = min(t0 + lane + j * kWave, tiles - 1);
      v[j] = best_val[t * best_stride + b];
      ix[j] = best_idx[t * best_stride + b];
    }
#pragma unroll
    for (int j = 0; j < kScan; ++j)
      if (t0 + lane + j * kWave < tiles && better(v[j], ix[j], bv, bi)) { bv = v[j]; bi = ix[j]; }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = lane_xor(bv, m);
    const int oi = lane_xor(bi, m);
    if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if (np >= cap) return;  // context full: the host never steps past capacity
  const bool forced = np < plen;
  const long tok = forced ? given : long(bi);
  const T* src = emb + tok * d;
  constexpr int V = vec_elems<T>();
  float* xr = x + long(b) * d;
  for (int t = lane; t < d / 16; t += kWave) {  // one 16-feature tile per lane per round
    uint4 r[16 / V];
#pragma unroll
    for (int j = 0; j < 16 / V; ++j) r[j] = load16(src + 16 * t + j * V);
    float v[16];
#pragma unroll
    for (int j = 0; j < 16 / V; ++j) unpack16<T>(r[j], v + j * V);
#pragma unroll
    for (int i = 0; i < 16; i += 4)
      *reinterpret_cast<float4*>(xr + 16 * t + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
  }
  if (lane == 0) {
    predicted[b * stride + np] = bi;
    if (!forced) tokens[b * stride + np] = bi;
    pos[b] = np;
    lengths[b] = np + 1;
  }
}

}  // namespace
}  // namespace sfl

using namespace sfl;

extern "C" int sfl_embedding_gather(const int64_t* tokens, long token_stride, const int32_t* pos,
                                    const void* emb, float* x, int batch, int d_model, int dtype,
                                    void* stream) {
  if (!tokens || !pos || !emb || !x) return set_error(SFL_ERR_INVALID, "embedding_gather: null pointer argument");
  if (batch < 1 || d_model < 1) return set_error(SFL_ERR_INVALID, "embedding_gather: sizes must be positive");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == SFL_DTYPE_BF16)
    hipLaunchKernelGGL(embed_kernel<bf16_t>, dim3(batch), dim3(256), 0, s, tokens, token_stride, pos,
                       static_cast<const bf16_t*>(emb), x, d_model);
  else if (dtype == SFL_DTYPE_F16)
    hipLaunchKernelGGL(embed_kernel<f16_t>, dim3(batch), dim3(256), 0, s, tokens, token_stride, pos,
                       static_cast<const f16_t*>(emb), x, d_model);
  else if (dtype == SFL_DTYPE_F32)
    hipLaunchKernelGGL(embed_kernel<float>, dim3(batch), dim3(256), 0, s, tokens, token_stride, pos,
                       static_cast<const float*>(emb), x, d_model);
  else
    return set_error(SFL_ERR_UNSUPPORTED, "embedding_gather: model dtype must be F32, BF16 or F16");
  return check_launch("embedding_gather");
}

extern "C" int sfl_next_token(const float* best_val, const int32_t* best_idx, int tiles,
                              int best_stride, int64_t* tokens, int64_t* predicted, long token_stride,
                              const int32_t* prompt_len, int32_t* pos, int32_t* lengths,
                              const void* emb, float* x, int batch, int d_model, int capacity,
                              int dtype, void* stream) {
  if (!best_val || !best_idx || !tokens || !predicted || !prompt_len || !pos || !lengths || !emb || !x)
    return set_error(SFL_ERR_INVALID, "next_token: null pointer argument");
  if (batch < 1 || tiles < 1 || d_model < 1 || capacity < 1)
    return set_error(SFL_ERR_INVALID, "next_token: sizes must be positive");
  if (d_model % 16) return set_error(SFL_ERR_UNSUPPORTED, "next_token: d_model must be a multiple of 16");
  if (token_stride < capacity)
    return set_error(SFL_ERR_INVALID, "next_token: token_stride must be >= capacity");
  if (best_stride < batch) return set_error(SFL_ERR_INVALID, "next_token: best_stride must be >= batch");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == SFL_DTYPE_BF16)
    hipLaunchKernelGGL(next_token_kernel<bf16_t>, dim3(batch), dim3(64), 0, s, best_val, best_idx, pos, tokens,
                       token_stride, tiles, best_stride, capacity, predicted, prompt_len, lengths,
                       static_cast<const bf16_t*>(emb), x, d_model);
  else if (dtype == SFL_DTYPE_F16)
    hipLaunchKernelGGL(next_token_kernel<f16_t>, dim3(batch), dim3(64), 0, s, best_val, best_idx, pos, tokens,
                       token_stride, tiles, best_stride, capacity, predicted, prompt_len, lengths,
                       static_cast<const f16_t*>(emb), x, d_model);
  else if (dtype == SFL_DTYPE_F32)
    hipLaunchKernelGGL(next_token_kernel<float>, dim3(batch), dim3(64), 0, s, best_val, best_idx, pos, tokens,
                       token_stride, tiles, best_stride, capacity, predicted, prompt_len, lengths,
                       static_cast<const float*>(emb), x, d_model);
  else
    return set_error(SFL_ERR_UNSUPPORTED, "next_token: model dtype must be F32, BF16 or F16");
  return check_launch("next_token");
}
