// Split-KV single-query attention over a contiguous [B, Hkv, cap, D] cache.
//
// Semantics follow attention_lab/cuda_decode/decode.cu: the cache is
// partitioned by capacity into `splits` chunks of ceil(cap/splits) keys
// (decode.cu:50-52), each chunk produces an fp32 (max, sum, numerator) partial,
// and a merge rescales the partials to one softmax (decode.cu:160-183,
// cuda_decode/README.md:72-76). Lengths are clamped to [0, cap] (decode.cu:49)
// and empty rows produce zeros (decode.cu:121-126, 180-182).
//
// The gfx950 design is not the reference's: one wave64 owns one (batch, kv
// head, chunk) item and streams its K/V rows with 16-byte loads, LPT lanes per
// key row; the query is held in registers pre-scaled by scale*log2(e) so the
// softmax runs on exp2. Every group of LPT lanes ("slot") keeps its own online
// softmax over the keys it loads, so the inner loop needs only the short
// intra-row dot-product reduction; the slots are merged once at the end of
// the chunk with xor shuffles. Max and sum are kept in base-2 units.
#include "common.hpp"

namespace sfl {
namespace {

template <typename T, int D, int G>
struct DecodeShape {
  static constexpr int EPL = vec_elems<T>();  // elements per lane per load
  static constexpr int LPT = D / EPL;          // lanes per key row
  static constexpr int TPL = kWave / LPT;      // key rows per wave load
  static constexpr int NL = (G >= 4) ? 4 : 8;  // loads per tile and operand
  static constexpr int TILE = NL * TPL;        // keys per tile
  static_assert(LPT >= 1 && LPT <= kWave, "head dim does not fit a wave");
};

template <typename T, typename TQ, int D, int G>
__global__ __launch_bounds__(256) void decode_partial_kernel(
    const TQ* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int32_t* __restrict__ lengths, float* __restrict__ pmax, float* __restrict__ psum,
    float* __restrict__ pout, int batch, int kv_heads, int cap, int splits, int chunk,
    float qscale) {
  using S = DecodeShape<T, D, G>;
  constexpr int EPL = S::EPL, LPT = S::LPT, TPL = S::TPL, NL = S::NL, TILE = S::TILE;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const long item = long(blockIdx.x) * 4 + wave;
  if (item >= long(batch) * kv_heads * splits) return;
  const int split = int(item % splits);
  const long bh = item / splits;
  const int h = int(bh % kv_heads);
  const int b = int(bh / kv_heads);
  const int len = min(max(lengths[b], 0), cap);
  const int begin = split * chunk;
  if (begin >= len) return;  // the merge reads only chunks below the length
  const int end = min(len, begin + chunk);
  const int slot = lane / LPT;
  const int dg = lane % LPT;
  const int q_heads = kv_heads * G;

  float qv[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const TQ* qp = q + (long(b) * q_heads + h * G + g) * D + dg * EPL;
#pragma unroll
    for (int e = 0; e < EPL; ++e) qv[g][e] = load_scalar<TQ>(qp + e) * qscale;
  }
  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
  }

  const long row0 = (long(b) * kv_heads + h) * cap;
  const T* kb = k + row0 * D + dg * EPL;
  const T* vb = v + row0 * D + dg * EPL;

  for (int t0 = begin; t0 < end; t0 += TILE) {
    uint4 kr[NL], vr[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int tc = min(t0 + i * TPL + slot, cap - 1);
      kr[i] = load16_stream(kb + long(tc) * D);
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int tc = min(t0 + i * TPL + slot, cap - 1);
      vr[i] = load16_stream(vb + long(tc) * D);
    }
    float sc[G][NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      float kf[EPL];
      unpack16<T>(kr[i], kf);
      const bool valid = t0 + i * TPL + slot < end;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) d = fmaf(qv[g][e], kf[e], d);
        d = group_sum<LPT>(d);
        sc[g][i] = valid ? d : -INFINITY;
      }
    }
    float p[G][NL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = sc[g][0];
#pragma unroll
      for (int i = 1; i < NL; ++i) mx = fmaxf(mx, sc[g][i]);
      const float mn = fmaxf(m[g], mx);
      const float ms = mn == -INFINITY ? 0.f : mn;
      const float alpha = exp2f(m[g] - ms);
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        p[g][i] = exp2f(sc[g][i] - ms);
        sum += p[g][i];
      }
      l[g] = l[g] * alpha + sum;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
      m[g] = mn;
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      float vf[EPL];
      unpack16<T>(vr[i], vf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(p[g][i], vf[e], acc[g][e]);
      }
    }
  }

  // Merge the slots' online-softmax states: xor over the slot bits of the lane id.
#pragma unroll
  for (int mask = LPT; mask < kWave; mask <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float om = __shfl_xor(m[g], mask, kWave);
      const float ol = __shfl_xor(l[g], mask, kWave);
      const float mn = fmaxf(m[g], om);
      const float ms = mn == -INFINITY ? 0.f : mn;
      const float a = exp2f(m[g] - ms);
      const float c = exp2f(om - ms);
      l[g] = l[g] * a + ol * c;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float oa = __shfl_xor(acc[g][e], mask, kWave);
        acc[g][e] = acc[g][e] * a + oa * c;
      }
      m[g] = mn;
    }
  }
  if (slot != 0) return;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const long row = (long(b) * q_heads + h * G + g) * splits + split;
    float4* dst = reinterpret_cast<float4*>(pout + row * D + dg * EPL);
#pragma unroll
    for (int e = 0; e < EPL; e += 4) dst[e / 4] = make_float4(acc[g][e], acc[g][e + 1], acc[g][e + 2], acc[g][e + 3]);
    if (dg == 0) {
      pmax[row] = m[g];
      psum[row] = l[g];
    }
  }
}

// One wave per (batch, query head): combine the chunks below the row's length.
template <typename T, int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(
    const float* __restrict__ pmax, const float* __restrict__ psum, const float* __restrict__ pout,
    const int32_t* __restrict__ lengths, T* __restrict__ out, int batch, int q_heads, int cap,
    int splits, int chunk) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const long row = long(blockIdx.x) * 4 + wave;
  if (row >= long(batch) * q_heads) return;
  const int b = int(row / q_heads);
  const int len = min(max(lengths[b], 0), cap);
  const int n = (len + chunk - 1) / chunk;
  const float* rm = pmax + row * splits;
  const float* rl = psum + row * splits;
  float top = -INFINITY;
  for (int s = lane; s < n; s += kWave) top = fmaxf(top, rm[s]);
  top = wave_max(top);
  float den = 0.f;
  if (top != -INFINITY) {
    for (int s = lane; s < n; s += kWave) {
      const float ms = rm[s];
      den += (ms == -INFINITY ? 0.f : exp2f(ms - top)) * rl[s];
    }
  }
  den = wave_sum(den);
#pragma unroll
  for (int d = lane; d < D; d += kWave) {
    float num = 0.f;
    if (top != -INFINITY) {
      for (int s = 0; s < n; ++s) {
        const float ms = rm[s];
        const float w = ms == -INFINITY ? 0.f : exp2f(ms - top);
        num = fmaf(w, pout[(row * splits + s) * D + d], num);
      }
    }
    store_scalar<T>(out + row * D + d, den > 0.f ? num / den : 0.f);
  }
}

template <typename T, typename TQ, int D, int G>
int launch_decode(const void* q, const void* k, const void* v, const int32_t* lengths, float* pmax,
                  float* psum, float* pout, void* out, int batch, int q_heads, int kv_heads,
                  int cap, int splits, float scale, hipStream_t stream) {
  const int chunk = (cap + splits - 1) / splits;
  const long items = long(batch) * kv_heads * splits;
  const long rows = long(batch) * q_heads;
  hipLaunchKernelGGL((decode_partial_kernel<T, TQ, D, G>), dim3(unsigned((items + 3) / 4)), dim3(256), 0,
                     stream, static_cast<const TQ*>(q), static_cast<const T*>(k),
                     static_cast<const T*>(v), lengths, pmax, psum, pout, batch, kv_heads, cap,
                     splits, chunk, scale * kLog2e);
  int rc = check_launch("decode_partial");
  if (rc) return rc;
  hipLaunchKernelGGL((decode_merge_kernel<TQ, D>), dim3(unsigned((rows + 3) / 4)), dim3(256), 0, stream,
                     pmax, psum, pout, lengths, static_cast<TQ*>(out), batch, q_heads, cap, splits,
                     chunk);
  return check_launch("decode_merge");
}

template <typename T, typename TQ, int D>
int dispatch_groups(int groups, const void* q, const void* k, const void* v, const int32_t* lengths,
                    float* pmax, float* psum, float* pout, void* out, int batch, int q_heads,
                    int kv_heads, int cap, int splits, float scale, hipStream_t stream) {
  switch (groups) {
    case 1: return launch_decode<T, TQ, D, 1>(q, k, v, lengths, pmax, psum, pout, out, batch, q_heads, kv_heads, cap, splits, scale, stream);
    case 2: return launch_decode<T, TQ, D, 2>(q, k, v, lengths, pmax, psum, pout, out, batch, q_heads, kv_heads, cap, splits, scale, stream);
    case 4: return launch_decode<T, TQ, D, 4>(q, k, v, lengths, pmax, psum, pout, out, batch, q_heads, kv_heads, cap, splits, scale, stream);
    case 8: return launch_decode<T, TQ, D, 8>(q, k, v, lengths, pmax, psum, pout, out, batch, q_heads, kv_heads, cap, splits, scale, stream);
  }
  return set_error(SFL_ERR_UNSUPPORTED, "decode_attention: unsupported GQA ratio %d", groups);
}

template <typename T, typename TQ>
int dispatch_dim(int dim, int groups, const void* q, const void* k, const void* v,
                 const int32_t* lengths, float* pmax, float* psum, float* pout, void* out, int batch,
                 int q_heads, int kv_heads, int cap, int splits, float scale, hipStream_t stream) {
  switch (dim) {
    case 16: return dispatch_groups<T, TQ, 16>(groups, q, k, v, lengths, pmax, psum, pout, out, batch, q_heads, kv_heads, cap, splits, scale, stream);
    case 32: return dispatch_groups<T, TQ, 32>(groups, q, k, v, lengths, pmax, psum, pout, out, batch, q_heads, kv_heads, cap, splits, scale, stream);
    case 64: return dispatch_groups<T, TQ, 64>(groups, q, k, v, lengths, pmax, psum, pout, out, batch, q_heads, kv_heads, cap, splits, scale, stream);
    case 128: return dispatch_groups<T, TQ, 128>(groups, q, k, v, lengths, pmax, psum, pout, out, batch, q_heads, kv_heads, cap, splits, scale, stream);
  }
  return set_error(SFL_ERR_UNSUPPORTED, "decode_attention: unsupported head dim %d", dim);
}

}  // namespace
}  // namespace sfl

extern "C" int sfl_decode_attention(const void* q, const void* k, const void* v,
                                    const int32_t* lengths, float* partial_max,
                                    float* partial_sum, float* partial_out, void* out, int batch,
                                    int q_heads, int kv_heads, int capacity, int head_dim,
                                    int splits, float scale, int dtype, int io_dtype, void* stream) {
  using namespace sfl;
  if (!q || !k || !v || !lengths || !partial_max || !partial_sum || !partial_out || !out)
    return set_error(SFL_ERR_INVALID, "decode_attention: null pointer argument");
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || capacity <= 0)
    return set_error(SFL_ERR_INVALID, "decode_attention: batch, heads and capacity must be positive");
  if (q_heads % kv_heads)
    return set_error(SFL_ERR_INVALID, "decode_attention: query heads must be divisible by KV heads");
  if (splits < 1 || splits > 1024)
    return set_error(SFL_ERR_INVALID, "decode_attention: splits must be in [1, 1024]");
  if (!(scale > 0.f) || !__builtin_isfinite(scale))
    return set_error(SFL_ERR_INVALID, "decode_attention: scale must be finite and positive");
  if (io_dtype != dtype && io_dtype != SFL_DTYPE_F32)
    return set_error(SFL_ERR_UNSUPPORTED, "decode_attention: q/out dtype must equal the KV dtype or be F32");
  const int groups = q_heads / kv_heads;
  const bool f32_io = io_dtype == SFL_DTYPE_F32;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define SFL_DECODE_ARGS head_dim, groups, q, k, v, lengths, partial_max, partial_sum, partial_out, out, \
    batch, q_heads, kv_heads, capacity, splits, scale, s
  switch (dtype) {
    case SFL_DTYPE_F32: return dispatch_dim<float, float>(SFL_DECODE_ARGS);
    case SFL_DTYPE_BF16:
      return f32_io ? dispatch_dim<bf16_t, float>(SFL_DECODE_ARGS) : dispatch_dim<bf16_t, bf16_t>(SFL_DECODE_ARGS);
    case SFL_DTYPE_F16:
      return f32_io ? dispatch_dim<f16_t, float>(SFL_DECODE_ARGS) : dispatch_dim<f16_t, f16_t>(SFL_DECODE_ARGS);
  }
#undef SFL_DECODE_ARGS
  return set_error(SFL_ERR_UNSUPPORTED, "decode_attention: unsupported dtype %d", dtype);
}
