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
#include <mutex>

#include "act_format.hpp"
#include "attn_mfma.hpp"
#include "lds_dma.hpp"

// Split scratch of sfl_decode_attention_static: one copy per GPU, held from
// module load until the process ends. In host code the name is only a stand-in
// for the symbol; every use goes through the device address that
// hipGetSymbolAddress returns for the current device (static_scratch below).
constexpr long kStaticScratchBytes = 16L << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace sfl {
namespace {

// Tag types of the outputs in the decode GEMVs' activation layout (act_format.hpp):
// split-bf16 values (BF16X2), split-fp16 values (F16X2) and fp32 values (F32X);
// and of the fused output projection, x[b] += attention(b) . W_o^T, accumulated
// into x with atomics.
struct split_t {};
struct split16_t {};
struct f32x_t {};
struct resid_t {};

// kStep: the fused output projection of the model's decode step (one split
// per row). Its D = 64, one-head-per-group tiles are 4 loads deep: the 324M
// decode step measured 1.404 -> 1.360 ms against 8 loads (config 4's split
// launches, which keep 8, measured 1.3% slower with 4; the operator's
// outputs keep 8, so its fp32 and activation-format outputs stay equal).
template <typename T, int D, int G, bool kStep = false>
struct DecodeShape {
  static constexpr int EPL = vec_elems<T>();  // elements per lane per load
  static constexpr int LPT = D / EPL;          // lanes per key row
  static constexpr int TPL = kWave / LPT;      // key rows per wave load
  static constexpr int NL = (G >= 4 || (kStep && G == 1 && D == 64)) ? 4 : 8;  // loads per tile and operand
  static constexpr int TILE = NL * TPL;        // keys per tile
  static_assert(LPT >= 1 && LPT <= kWave, "head dim does not fit a wave");
};

// Store output element f = row * D + d of [batch * q_heads, D] (K = q_heads * D).
template <typename TO>
__device__ __forceinline__ void store_out(void* out, long f, int K, float v);

// Fused output projection (TO = resid_t, one split): the packed W_o of the
// decode GEMVs (decode_linear.hip: 1 KB per 16 rows x one K chunk) is read for
// this kv head's G*D columns, in rounds of kProjRound 16-byte loads per lane.
constexpr int kProjRound = 8;

template <typename T, int D, int G>
struct ProjShape {
  static constexpr int KC = 4 * vec_elems<T>();  // K values per packed chunk
  // Chunks per kv head (a power of two; the host admits G*D % KC == 0 only).
  static constexpr int NCK = G * D >= KC ? G * D / KC : 1;
};

// Unit u of a wave's share: tile wave + (u / NCK) * W, chunk h * NCK + u % NCK.
template <typename T, int D, int G, int W>
__device__ __forceinline__ uint4 load_proj_unit(const unsigned char* w_lane, int u, int wave, int h,
                                                int nchunks_all) {
  using P = ProjShape<T, D, G>;
  const long tile = wave + (u / P::NCK) * W;
  const long c = long(h) * P::NCK + u % P::NCK;
  return load16(w_lane + (tile * nchunks_all + c) * kWave * 16);
}

// One workgroup of W waves per (batch, kv head, split). The split's key
// tiles are dealt round-robin to the waves; each wave streams its tiles with
// the per-slot online softmax, the slots are merged with shuffles, and the W
// wave states are merged through LDS. With one split the workgroup writes the final
// output (or, fused, adds its heads' share of the output projection to x);
// otherwise it writes its (max, sum, numerator) partial for the merge kernel.
// The arguments the prologue and the first loads need come first (14 dwords):
// this file is built with kernel-argument preloading, so they arrive in SGPRs
// with the wave. The index math is 32-bit, and the fused projection (always
// one split) skips the division by the split count: a launch's first
// instructions are fetched cold, so each one ahead of the first load counts.
template <typename T, typename TQ, typename TO, int D, int G, int W>
__global__ __launch_bounds__(W * kWave) void decode_attn_kernel(
    const TQ* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int32_t* __restrict__ lengths, int kv_heads, int cap, int splits, int chunk, float qscale,
    int d_model, float* __restrict__ pmax, float* __restrict__ psum, float* __restrict__ pout,
    void* __restrict__ out, float* __restrict__ x) {
  constexpr bool kProj = std::is_same<TO, resid_t>::value;
  using S = DecodeShape<T, D, G, kProj>;
  constexpr int EPL = S::EPL, LPT = S::LPT, TPL = S::TPL, NL = S::NL, TILE = S::TILE;
  __shared__ float sm[W][G][D + 2];
  __shared__ float os[kProj ? G * D : 1];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const unsigned bh = kProj ? blockIdx.x : blockIdx.x / unsigned(splits);
  const int split = kProj ? 0 : int(blockIdx.x - bh * unsigned(splits));
  const int b = int(bh / unsigned(kv_heads));
  const int h = int(bh - unsigned(b) * unsigned(kv_heads));
  const int q_heads = kv_heads * G;
  const int slot = lane / LPT;
  const int dg = lane % LPT;

  // The query does not depend on the length: issue its loads first.
  float qv[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const TQ* qp = q + (long(b) * q_heads + h * G + g) * D + dg * EPL;
#pragma unroll
    for (int e = 0; e < EPL; ++e) qv[g][e] = load_scalar<TQ>(qp + e);
  }
  const long row0 = (long(b) * kv_heads + h) * cap;
  const T* kb = k + row0 * D + dg * EPL;
  const T* vb = v + row0 * D + dg * EPL;
  const int begin = split * chunk;
  const int t_first = begin + wave * TILE;

  // With one split (the model's path) the first waves issue their first
  // tile's loads before the length is known, rows clamped to the capacity, so
  // their round trip overlaps the q and length loads; rows at or past the
  // length are zeroed once it is known (they may hold stale values, NaN
  // included). The others wait for the length: the speculative loads stay at
  // W/2 tiles of 8 loads (W tiles of 4), so a short row wastes at most that
  // much (with every wave speculating 8-load tiles: ~15.5 us per 324M launch
  // below length 1024 against ~11.5, and no faster at 3584).
  const bool spec = splits == 1 && wave < W * 4 / NL;
  uint4 kr[NL], vr[NL];
  if (spec) {
#pragma unroll
    for (int i = 0; i < NL; ++i) kr[i] = load16_stream(kb + long(min(t_first + i * TPL + slot, cap - 1)) * D);
#pragma unroll
    for (int i = 0; i < NL; ++i) vr[i] = load16_stream(vb + long(min(t_first + i * TPL + slot, cap - 1)) * D);
  }
  const int len = min(max(lengths[b], 0), cap);
  if (splits > 1 && begin >= len) return;  // the merge reads only chunks below the length
  const int end = min(len, begin + chunk);
  if (spec) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      if (t_first + i * TPL + slot >= end) {
        kr[i] = make_uint4(0u, 0u, 0u, 0u);
        vr[i] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  }

#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) qv[g][e] *= qscale;
  }
  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
  }

  // Wave w takes tiles w, w + W, w + 2W, ... of the split, so the workgroup's
  // loads at any time cover one contiguous run of W tiles per operand (two
  // DRAM streams per workgroup instead of two per wave). Rows past the split
  // are clamped to its last row: the masked lanes of the final partial tile
  // re-read a cached row instead of fetching new HBM lines.
  const int last = end - 1;
  // One tile of the wave: scores, per-slot online softmax, V accumulation.
  auto tile = [&](int t0, const uint4 (&kr)[NL], const uint4 (&vr)[NL]) {
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
  };
  const int t_loop = spec ? t_first + W * TILE : t_first;
  if constexpr (kProj && NL == 4) {
    // The fused path's 4-load tiles leave registers for one tile of loads in
    // flight ahead of the tile being computed (324M decode step -0.8%); past
    // the end the loads re-read the split's last row.
    uint4 kc[NL], vc[NL];
    if (t_loop < end) {
#pragma unroll
      for (int i = 0; i < NL; ++i) kc[i] = load16_stream(kb + long(min(t_loop + i * TPL + slot, last)) * D);
#pragma unroll
      for (int i = 0; i < NL; ++i) vc[i] = load16_stream(vb + long(min(t_loop + i * TPL + slot, last)) * D);
    }
    if (spec && t_first < end) tile(t_first, kr, vr);
    for (int t0 = t_loop; t0 < end; t0 += W * TILE) {
      const int t1 = min(t0 + W * TILE, last);
      uint4 kn[NL], vn[NL];
#pragma unroll
      for (int i = 0; i < NL; ++i) kn[i] = load16_stream(kb + long(min(t1 + i * TPL + slot, last)) * D);
#pragma unroll
      for (int i = 0; i < NL; ++i) vn[i] = load16_stream(vb + long(min(t1 + i * TPL + slot, last)) * D);
      tile(t0, kc, vc);
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        kc[i] = kn[i];
        vc[i] = vn[i];
      }
    }
  } else {
    if (spec && t_first < end) tile(t_first, kr, vr);
    for (int t0 = t_loop; t0 < end; t0 += W * TILE) {
      uint4 kn[NL], vn[NL];
#pragma unroll
      for (int i = 0; i < NL; ++i) kn[i] = load16_stream(kb + long(min(t0 + i * TPL + slot, last)) * D);
#pragma unroll
      for (int i = 0; i < NL; ++i) vn[i] = load16_stream(vb + long(min(t0 + i * TPL + slot, last)) * D);
      tile(t0, kn, vn);
    }
  }

  // Fused projection: issue the first round of W_o loads now, so they land
  // while the softmax states are merged. `out` is the packed W_o.
  const unsigned char* w_lane = static_cast<const unsigned char*>(out) + lane * 16;
  const int proj_tiles = d_model / 16;
  const int proj_units = kProj ? max(0, (proj_tiles - wave + W - 1) / W) * ProjShape<T, D, G>::NCK : 0;
  uint4 wr[kProj ? kProjRound : 1];
  if constexpr (kProj) {
#pragma unroll
    for (int j = 0; j < kProjRound; ++j)
      if (proj_units > 0)
        wr[j] = load_proj_unit<T, D, G, W>(w_lane, min(j, proj_units - 1), wave, h, d_model / ProjShape<T, D, G>::KC);
  }

  // Merge the slots' online-softmax states: xor over the slot bits of the lane id.
#pragma unroll
  for (int mask = LPT; mask < kWave; mask <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float om = lane_xor(m[g], mask);
      const float ol = lane_xor(l[g], mask);
      const float mn = fmaxf(m[g], om);
      const float ms = mn == -INFINITY ? 0.f : mn;
      const float a = exp2f(m[g] - ms);
      const float c = exp2f(om - ms);
      l[g] = l[g] * a + ol * c;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float oa = lane_xor(acc[g][e], mask);
        acc[g][e] = acc[g][e] * a + oa * c;
      }
      m[g] = mn;
    }
  }
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) sm[wave][g][dg * EPL + e] = acc[g][e];
      if (dg == 0) {
        sm[wave][g][D] = m[g];
        sm[wave][g][D + 1] = l[g];
      }
    }
  }
  __syncthreads();

  // Merge the W wave states. Output o = (query head g, dim d) is combined by
  // W lanes of one wave (lane = j * W + w holds wave w's state for the wave's
  // j-th output of the round), all waves in parallel: an xor-butterfly over
  // those W lanes takes the maximum, another adds the rescaled sums. (One
  // thread walking the W states one after another, each step waiting on LDS
  // and on the previous one, cost ~1.8 us of the fused decode launch.)
  {
    constexpr int OPW = kWave / W;  // outputs per wave and round
    static_assert(OPW >= 1 && (G * D) % OPW == 0, "outputs per wave");
    const int j = lane / W, w = lane % W;
    for (int o0 = wave * OPW; o0 < G * D; o0 += W * OPW) {  // uniform over the wave
      const int o = o0 + j;
      const int g = o / D, d = o % D;
      const float mw = sm[w][g][D];
      float top = mw;
#pragma unroll
      for (int m = 1; m < W; m <<= 1) top = fmaxf(top, lane_xor(top, m));
      const float c = mw == -INFINITY ? 0.f : exp2f(mw - top);  // every state empty: top = -inf, c = 0
      float den = c * sm[w][g][D + 1];
      float num = c * sm[w][g][d];
#pragma unroll
      for (int m = 1; m < W; m <<= 1) {
        den += lane_xor(den, m);
        num += lane_xor(num, m);
      }
      if (w == 0) {
        const long qrow = long(b) * q_heads + h * G + g;
        if constexpr (kProj) {
          os[o] = den > 0.f ? num / den : 0.f;
        } else if (splits == 1) {
          store_out<TO>(out, qrow * D + d, q_heads * D, den > 0.f ? num / den : 0.f);
        } else {
          const long prow = qrow * splits + split;
          pout[prow * D + d] = num;
          if (d == 0) {
            pmax[prow] = top;
            psum[prow] = den;
          }
        }
      }
    }
  }
  if constexpr (kProj) {
    // x[b, n] += sum_c W_o[n, c] o[c] over this kv head's columns c: each
    // lane takes a 16-byte piece of W_o (row n = tile*16 + lane%16, columns
    // of its lane group), the 4 groups are added with shuffles and lanes 0..15
    // add their row's value to x (16 kv heads add to each element).
    using P = ProjShape<T, D, G>;
    constexpr int EW = vec_elems<T>();
    __syncthreads();
    const int grp = lane / 16;
    float* xb = x + long(b) * d_model;
    float part = 0.f;
    for (int r0 = 0; r0 < proj_units; r0 += kProjRound) {
      if (r0 > 0) {
#pragma unroll
        for (int j = 0; j < kProjRound; ++j)
          wr[j] = load_proj_unit<T, D, G, W>(w_lane, min(r0 + j, proj_units - 1), wave, h, d_model / P::KC);
      }
#pragma unroll
      for (int j = 0; j < kProjRound; ++j) {
        const int u = r0 + j;
        if (u < proj_units) {  // uniform over the wave
          float wv[EW];
          unpack16<T>(wr[j], wv);
          const float* op = os + (u % P::NCK) * P::KC + grp * EW;
#pragma unroll
          for (int e = 0; e < EW; ++e) part = fmaf(wv[e], op[e], part);
          if (u % P::NCK == P::NCK - 1) {
            part += lane_xor(part, 16);
            part += lane_xor(part, 32);
            const int tile = wave + (u / P::NCK) * W;
            if (lane < 16) unsafeAtomicAdd(xb + tile * 16 + lane, part);
            part = 0.f;
          }
        }
      }
    }
  }
}

// Output writers: the KV dtype, fp32, or the GEMV activation layout of a
// [batch, q_heads * D] input (split-bf16 or fp32 values).
template <typename TO>
__device__ __forceinline__ void store_out(void* out, long f, int, float v) {
  store_scalar<TO>(static_cast<TO*>(out) + f, v);
}
template <>
__device__ __forceinline__ void store_out<split_t>(void* out, long f, int K, float v) {
  store_act1<bf16_t>(static_cast<unsigned char*>(out), int(f / K), int(f % K), K, v);
}
template <>
__device__ __forceinline__ void store_out<split16_t>(void* out, long f, int K, float v) {
  store_act1<f16_t>(static_cast<unsigned char*>(out), int(f / K), int(f % K), K, v);
}
template <>
__device__ __forceinline__ void store_out<f32x_t>(void* out, long f, int K, float v) {
  store_act1<float>(static_cast<unsigned char*>(out), int(f / K), int(f % K), K, v);
}

// One wave per (batch, query head): combine the chunks below the row's length.
// Every load of a round of up to kRound = 16 chunks (their max, sum and
// numerators) is issued before any is used, so a merge of <= 16 chunks costs
// one round trip.
// Lane s holds chunk s's max and sum; the numerators are weighted by shuffles.
template <typename TO, int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(
    const float* __restrict__ pmax, const float* __restrict__ psum, const float* __restrict__ pout,
    const int32_t* __restrict__ lengths, void* __restrict__ out, int batch, int q_heads, int cap,
    int splits, int chunk) {
  constexpr int DPL = (D + kWave - 1) / kWave;  // dims per lane
  constexpr int kRound = 16;                     // numerator loads in flight per lane and dim
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const long row = long(blockIdx.x) * 4 + wave;
  if (row >= long(batch) * q_heads) return;
  const int b = int(row / q_heads);
  const int len = min(max(lengths[b], 0), cap);
  const int n = (len + chunk - 1) / chunk;
  const float* rm = pmax + row * splits;
  const float* rl = psum + row * splits;
  const float* ro = pout + row * splits * D;
  float top = -INFINITY, den = 0.f;
  float num[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) num[i] = 0.f;
  for (int s0 = 0; s0 < n; s0 += kRound) {
    // Unconditional loads from clamped indices; masked after they land.
    const int s = s0 + (lane % kRound);
    const bool ok = s < n;
    const float ms_raw = rm[min(s, n - 1)];
    const float ls_raw = rl[min(s, n - 1)];
    float part[kRound][DPL];
#pragma unroll
    for (int j = 0; j < kRound; ++j) {
#pragma unroll
      for (int i = 0; i < DPL; ++i)
        part[j][i] = ro[long(min(s0 + j, n - 1)) * D + min(lane + i * kWave, D - 1)];
    }
    const float ms = ok ? ms_raw : -INFINITY;
    const float ls = ok ? ls_raw : 0.f;
#pragma unroll
    for (int j = 0; j < kRound; ++j) {
#pragma unroll
      for (int i = 0; i < DPL; ++i)
        if (s0 + j >= n) part[j][i] = 0.f;
    }
    // Rescale the running state to the new maximum, then add this round.
    const float round_top = wave_max(ms);
    const float nt = fmaxf(top, round_top);
    if (nt == -INFINITY) continue;
    const float keep = top == -INFINITY ? 0.f : exp2f(top - nt);
    const float w = ms == -INFINITY ? 0.f : exp2f(ms - nt);
    den = den * keep + (lane < kRound ? w * ls : 0.f);
#pragma unroll
    for (int i = 0; i < DPL; ++i) num[i] *= keep;
#pragma unroll
    for (int j = 0; j < kRound; ++j) {
      const float wj = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(w), j));  // lane j's weight
#pragma unroll
      for (int i = 0; i < DPL; ++i) num[i] = fmaf(wj, part[j][i], num[i]);
    }
    top = nt;
  }
  den = wave_sum(den);
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int d = lane + i * kWave;
    if (d < D) store_out<TO>(out, row * D + d, q_heads * D, den > 0.f ? num[i] / den : 0.f);
  }
}

template <typename TO, int D>
int launch_merge(const float* pmax, const float* psum, const float* pout, const int32_t* lengths, void* out,
                 int batch, int q_heads, int cap, int splits, hipStream_t stream) {
  const int chunk = (cap + splits - 1) / splits;
  const long rows = long(batch) * q_heads;
  hipLaunchKernelGGL((decode_merge_kernel<TO, D>), dim3(unsigned((rows + 3) / 4)), dim3(256), 0, stream,
                     pmax, psum, pout, lengths, out, batch, q_heads, cap, splits, chunk);
  return check_launch("decode_merge");
}

// Grouped-query decode on the matrix cores. With G >= 4 query heads per KV
// head the kernel above does G dot products and G multiply-adds per key
// element on the VALU, which takes longer than streaming the element from HBM
// (D = 128, G = 8: ~2 TB/s). Here one 32x32x16 MFMA block holds a 32-key
// tile against all G heads: S^T = K Q^T with the heads as the B operand's
// columns (zero past G), then O^T += V^T P^T, exactly the tile step of the
// masked prefill attention (prefill_attention.hip) with the group's heads in
// place of 32 queries. Each of the 4 waves owns every 4th 32-key tile of the
// split and stages it in its own double-buffered LDS slots through LDS DMA:
// K rows swizzled for the operand reads (k_swizzle), V rows laid out for the
// transpose reads (vt_slot). The buffer range ends at the split's last key,
// so key rows past the length read as zeros and stale cache rows (NaN
// included) never reach the products. The waves' states are merged through
// LDS (reusing the tile buffers) as in decode_attn_kernel, and the workgroup
// writes the output or the same base-2 (max, sum, numerator) partial, which
// decode_merge_kernel combines.
constexpr int kGqaWaves = 4;
constexpr int kGqaTile = 32;  // keys per wave tile

template <typename T, int D, bool kMask>
__device__ __forceinline__ void gqa32_tile(const uint4 (&kt)[kGqaTile][D / 8], const uint4 (&vt)[kGqaTile][D / 8],
                                           const u32x4 (&qreg)[D / 16], f32x16 (&oacc)[D / 32], float& m_run,
                                           float& l_run, int c, int h, int t0, int end, float cs,
                                           const unsigned (&vlane)[D / 32]) {
  f32x16 s;
#pragma unroll
  for (int j = 0; j < 16; ++j) s[j] = 0.f;
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    const uint4 kr = kt[c][(D / 16 * h + ks) ^ k_swizzle<D>(c)];
    s = mfma32<T>(u32x4{kr.x, kr.y, kr.z, kr.w}, qreg[ks], s);
  }
  if constexpr (kMask) {
#pragma unroll
    for (int j = 0; j < 16; ++j) s[j] = t0 + 8 * (j / 4) + 4 * h + j % 4 < end ? s[j] : -INFINITY;
  }
  float mx = fmaxf(s[0], s[1]);
#pragma unroll
  for (int j = 2; j < 16; j += 2) mx = fmaxf(fmaxf(mx, s[j]), s[j + 1]);
  mx = fmaxf(mx, lane_xor(mx, 32));
  // Lazy maximum (as in the prefill tile): m_run moves only when a head's
  // tile maximum exceeds it by more than kLazyMax, so probabilities stay
  // below 2^kLazyMax and O is rescaled only on those tiles.
  const bool grow = mx * cs > m_run + kLazyMax;
  float alpha = 1.f;
  if (__ballot(grow)) {
    const float m_new = grow ? mx * cs : m_run;
    alpha = grow ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < D / 32; ++t) oacc[t] *= alpha;
  }
  const float ms = m_run == -INFINITY ? 0.f : m_run;
  u32x4 pop[2];
  float psum[2] = {0.f, 0.f};
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    uint32_t pk[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j0 = 8 * s2 + 2 * e;
      pk[e] = pack2<T>(__builtin_amdgcn_exp2f(fmaf(s[j0], cs, -ms)), __builtin_amdgcn_exp2f(fmaf(s[j0 + 1], cs, -ms)));
      psum[s2] = add_pair<T>(pk[e], psum[s2]);
    }
    pop[s2] = u32x4{pk[0], pk[1], pk[2], pk[3]};
  }
  l_run = l_run * alpha + (psum[0] + psum[1]);
  const unsigned vbase = lds_offset(&vt[0][0]);
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
    for (int t = 0; t < D / 32; ++t) {
      const unsigned off = vbase + vlane[t] + 32u * D * s2;
      const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(size_t)(off));
      const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(size_t)(off + 16u * D));
      const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
      oacc[t] = mfma32<T>(u32x4{l2.x, l2.y, h2.x, h2.y}, pop[s2], oacc[t]);
    }
  }
}

// One workgroup of 4 waves per (batch, kv head, split), grid order as
// decode_attn_kernel. The host admits 16-byte aligned q/k/v and caches of
// cap * D * 2 < 2^31 bytes per head (32-bit buffer offsets).
// Arguments ordered as decode_attn_kernel's: the prologue's in the preloaded 13 dwords.
template <typename T, typename TO, int D, int G>
__global__ __launch_bounds__(kGqaWaves * kWave) void decode_gqa32_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int32_t* __restrict__ lengths, int kv_heads, int cap, int splits, int chunk, float cs,
    float* __restrict__ pmax, float* __restrict__ psum, float* __restrict__ pout, void* __restrict__ out) {
  constexpr int W = kGqaWaves, BT = kGqaTile;
  constexpr int SL = D / 8;        // 16-byte slots per key row
  constexpr int RPL = kWave / SL;  // key rows one 1 KB DMA load moves
  constexpr int NLD = BT / RPL;    // DMA loads per tile and operand
  static_assert(G <= 32 && NLD * RPL == BT, "tile shape");
  __shared__ __align__(16) uint4 kv_s[W][2][2][BT][SL];  // [wave][buffer][K, V][key][slot]
  typedef float MergeRow[G][D + 2];
  static_assert(sizeof(MergeRow) * W <= sizeof(kv_s), "the merge rows fit the tile buffers");
  MergeRow* sm = reinterpret_cast<MergeRow*>(&kv_s[0][0][0][0][0]);
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
  const int lane = threadIdx.x % kWave;
  const int c = lane % 32, h = lane / 32;
  const unsigned bh = blockIdx.x / unsigned(splits);
  const int split = int(blockIdx.x - bh * unsigned(splits));
  const int b = int(bh / unsigned(kv_heads));
  const int hk = int(bh - unsigned(b) * unsigned(kv_heads));
  const int q_heads = kv_heads * G;

  // Q^T operand of k-step ks: head c's dims (D/2) h + 8 ks .. +7; zero past G.
  // The select waits for the loads here, before the tile prefetch is issued.
  u32x4 qreg[D / 16];
  {
    const T* qp = q + (long(b) * q_heads + hk * G + min(c, G - 1)) * D + (D / 2) * h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const uint4 r = load16(qp + 8 * ks);
      qreg[ks] = c < G ? u32x4{r.x, r.y, r.z, r.w} : u32x4{0u, 0u, 0u, 0u};
    }
  }
  const int len = min(max(__builtin_amdgcn_readfirstlane(lengths[b]), 0), cap);
  const int begin = split * chunk;
  if (splits > 1 && begin >= len) return;  // the merge reads only chunks below the length
  const int end = min(len, begin + chunk);

  const long head0 = (long(b) * kv_heads + hk) * cap * D;
  constexpr unsigned kRow = 2u * D;  // bytes per key row
  const i32x4_t krsrc = buffer_rsrc(k + head0, unsigned(end) * kRow);
  const i32x4_t vrsrc = buffer_rsrc(v + head0, unsigned(end) * kRow);
  // DMA load j of a tile moves rows RPL j .. RPL j + RPL - 1; lane i takes
  // row RPL j + i / SL into physical slot i % SL: the K slot (i % SL) ^
  // k_swizzle(row), the V slot sg with vt_slot(sg, row) == i % SL (row & 3 ==
  // (i / SL) & 3 for every j).
  const int lrr = lane / SL, lpp = lane % SL;
  unsigned kvoff[NLD];
#pragma unroll
  for (int j = 0; j < NLD; ++j) {
    const int r = RPL * j + lrr;
    kvoff[j] = unsigned(r) * kRow + 16u * unsigned(lpp ^ k_swizzle<D>(r));
  }
  const unsigned vvoff = unsigned(lrr) * kRow + 16u * (2u * ((unsigned(lpp) >> 1) ^ (unsigned(lrr) & 3u)) + (unsigned(lpp) & 1u));
  unsigned vlane[D / 32];
#pragma unroll
  for (int t = 0; t < D / 32; ++t) vlane[t] = vt_lane_offset<D>(lane, t);
  auto issue = [&](int tile0, int buf) {
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      lds_load16(krsrc, lds_offset(&kv_s[wave][buf][0][RPL * j][0]), kvoff[j], unsigned(tile0) * kRow);
      lds_load16(vrsrc, lds_offset(&kv_s[wave][buf][1][RPL * j][0]), vvoff, unsigned(tile0 + RPL * j) * kRow);
    }
  };

  float m_run = -INFINITY, l_run = 0.f;
  f32x16 oacc[D / 32];
#pragma unroll
  for (int t = 0; t < D / 32; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) oacc[t][j] = 0.f;

  int t0 = begin + BT * wave;
  if (t0 < end) issue(t0, 0);
  for (int buf = 0; t0 < end; buf ^= 1) {
    const int tn = t0 + BT * W;
    if (tn < end) {
      issue(tn, buf ^ 1);
      __builtin_amdgcn_s_waitcnt(sfl_vmcnt(2 * NLD));  // this tile has landed, the next is in flight
    } else {
      __builtin_amdgcn_s_waitcnt(sfl_vmcnt(0));
    }
    if (t0 + BT <= end)
      gqa32_tile<T, D, false>(kv_s[wave][buf][0], kv_s[wave][buf][1], qreg, oacc, m_run, l_run, c, h, t0, end, cs, vlane);
    else
      gqa32_tile<T, D, true>(kv_s[wave][buf][0], kv_s[wave][buf][1], qreg, oacc, m_run, l_run, c, h, t0, end, cs, vlane);
    t0 = tn;
  }

  const float l_tot = l_run + lane_xor(l_run, 32);
  __syncthreads();  // every wave is done with the tile buffers the merge rows reuse
  if (c < G) {
#pragma unroll
    for (int t = 0; t < D / 32; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) sm[wave][c][32 * t + 8 * (j / 4) + 4 * h + j % 4] = oacc[t][j];
    if (h == 0) {
      sm[wave][c][D] = m_run;
      sm[wave][c][D + 1] = l_tot;
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < G * D; t += W * kWave) {
    const int g = t / D, d = t % D;
    float top = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) top = fmaxf(top, sm[w][g][D]);
    float den = 0.f, num = 0.f;
    if (top != -INFINITY) {
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float mw = sm[w][g][D];
        const float f = mw == -INFINITY ? 0.f : exp2f(mw - top);
        den = fmaf(f, sm[w][g][D + 1], den);
        num = fmaf(f, sm[w][g][d], num);
      }
    }
    const long qrow = long(b) * q_heads + hk * G + g;
    if (splits == 1) {
      store_out<TO>(out, qrow * D + d, q_heads * D, den > 0.f ? num / den : 0.f);
    } else {
      const long prow = qrow * splits + split;
      pout[prow * D + d] = num;
      if (d == 0) {
        pmax[prow] = top;
        psum[prow] = den;
      }
    }
  }
}

struct DecodeCall {
  const void *q, *k, *v;
  const int32_t* lengths;
  float *pmax, *psum, *pout;
  void* out;
  int batch, q_heads, kv_heads, cap, dim, splits;
  float scale;
  hipStream_t stream;
  float* x;     // fused projection: residual stream [batch, d_model]
  int d_model;
};

// Waves per workgroup: as many as keep the kernel within the register budget
// of W waves per CU-quarter (<= 128 VGPRs at W = 16).
template <typename T, int D, int G> constexpr int waves_for() {
  return (G == 1 && D <= 64) ? 16 : ((G <= 2 && D <= 128) ? 8 : 4);
}

// The MFMA kernel takes grouped 16-bit caches with 16-bit queries (G >= 4, D
// of 64 or 128) when q/k/v are 16-byte aligned and a head's cache fits 32-bit
// buffer offsets; everything else runs decode_attn_kernel.
template <typename T, typename TQ, typename TO, int D, int G>
constexpr bool gqa_mfma_shape() {
  return G >= 4 && (D == 64 || D == 128) && std::is_same<T, TQ>::value &&
         (std::is_same<T, bf16_t>::value || std::is_same<T, f16_t>::value) && !std::is_same<TO, resid_t>::value;
}

inline bool gqa_mfma_fits(const DecodeCall& c) {
  const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  return a16(c.q) && a16(c.k) && a16(c.v) && long(c.cap) * c.dim * 2 < (1L << 31);
}

template <typename T, typename TQ, typename TO, int D, int G>
int launch_attn(const DecodeCall& c) {
  if constexpr (gqa_mfma_shape<T, TQ, TO, D, G>()) {
    if (gqa_mfma_fits(c)) {
      const int chunk = (c.cap + c.splits - 1) / c.splits;
      const long groups = long(c.batch) * c.kv_heads * c.splits;
      hipLaunchKernelGGL((decode_gqa32_kernel<T, TO, D, G>), dim3(unsigned(groups)), dim3(kGqaWaves * kWave), 0,
                         c.stream, static_cast<const T*>(c.q), static_cast<const T*>(c.k),
                         static_cast<const T*>(c.v), c.lengths, c.kv_heads, c.cap, c.splits, chunk,
                         c.scale * kLog2e, c.pmax, c.psum, c.pout, c.out);
      return check_launch("decode_attention");
    }
  }
  constexpr int W = waves_for<T, D, G>();
  const int chunk = (c.cap + c.splits - 1) / c.splits;
  const long groups = long(c.batch) * c.kv_heads * c.splits;
  hipLaunchKernelGGL((decode_attn_kernel<T, TQ, TO, D, G, W>), dim3(unsigned(groups)), dim3(W * kWave), 0,
                     c.stream, static_cast<const TQ*>(c.q), static_cast<const T*>(c.k),
                     static_cast<const T*>(c.v), c.lengths, c.kv_heads, c.cap, c.splits, chunk,
                     c.scale * kLog2e, c.d_model, c.pmax, c.psum, c.pout, c.out, c.x);
  return check_launch("decode_attention");
}

template <typename T, typename TQ, typename TO, int D>
int attn_groups(const DecodeCall& c) {
  switch (c.q_heads / c.kv_heads) {
    case 1: return launch_attn<T, TQ, TO, D, 1>(c);
    case 2: return launch_attn<T, TQ, TO, D, 2>(c);
    case 4: return launch_attn<T, TQ, TO, D, 4>(c);
    case 8: return launch_attn<T, TQ, TO, D, 8>(c);
  }
  return set_error(SFL_ERR_UNSUPPORTED, "decode_attention: unsupported GQA ratio %d", c.q_heads / c.kv_heads);
}

template <typename T, typename TQ, typename TO>
int attn_dims(const DecodeCall& c) {
  switch (c.dim) {
    case 16: return attn_groups<T, TQ, TO, 16>(c);
    case 32: return attn_groups<T, TQ, TO, 32>(c);
    case 64: return attn_groups<T, TQ, TO, 64>(c);
    case 128: return attn_groups<T, TQ, TO, 128>(c);
  }
  return set_error(SFL_ERR_UNSUPPORTED, "decode_attention: unsupported head dim %d", c.dim);
}

template <typename TO>
int merge_dims(const DecodeCall& c) {
  switch (c.dim) {
    case 16: return launch_merge<TO, 16>(c.pmax, c.psum, c.pout, c.lengths, c.out, c.batch, c.q_heads, c.cap, c.splits, c.stream);
    case 32: return launch_merge<TO, 32>(c.pmax, c.psum, c.pout, c.lengths, c.out, c.batch, c.q_heads, c.cap, c.splits, c.stream);
    case 64: return launch_merge<TO, 64>(c.pmax, c.psum, c.pout, c.lengths, c.out, c.batch, c.q_heads, c.cap, c.splits, c.stream);
    case 128: return launch_merge<TO, 128>(c.pmax, c.psum, c.pout, c.lengths, c.out, c.batch, c.q_heads, c.cap, c.splits, c.stream);
  }
  return set_error(SFL_ERR_UNSUPPORTED, "decode_attention: unsupported head dim %d", c.dim);
}

// The attention kernel's output type is only used with one split; with more
// splits it writes partials and the merge kernel writes the output type.
template <typename T, typename TQ>
int attn_out(const DecodeCall& c, int out_dtype) {
  if (c.splits > 1) return attn_dims<T, TQ, float>(c);
  switch (out_dtype) {
    case SFL_DTYPE_F32: return attn_dims<T, TQ, float>(c);
    case SFL_DTYPE_BF16X2: return attn_dims<T, TQ, split_t>(c);
    case SFL_DTYPE_F16X2: return attn_dims<T, TQ, split16_t>(c);
    case SFL_DTYPE_F32X: return attn_dims<T, TQ, f32x_t>(c);
    default: return attn_dims<T, TQ, T>(c);
  }
}

template <typename T, int D>
int launch_proj(const DecodeCall& c) {
  return launch_attn<T, float, resid_t, D, 1>(c);
}

template <typename T>
int proj_dims(const DecodeCall& c) {
  switch (c.dim) {
    case 16: if constexpr (sizeof(T) == 4) return launch_proj<T, 16>(c); else break;
    case 32: return launch_proj<T, 32>(c);
    case 64: return launch_proj<T, 64>(c);
    case 128: return launch_proj<T, 128>(c);
  }
  return set_error(SFL_ERR_UNSUPPORTED, "decode_attention_out_proj: unsupported head dim %d", c.dim);
}

}  // namespace
}  // namespace sfl

extern "C" int sfl_decode_attention_out_proj(const float* q, const void* k, const void* v,
                                             const int32_t* lengths, const void* w_out, float* x,
                                             int batch, int heads, int capacity, int head_dim,
                                             float scale, int dtype, void* stream) {
  using namespace sfl;
  const char* what = "decode_attention_out_proj";
  if (!q || !k || !v || !lengths || !w_out || !x) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (batch <= 0 || heads <= 0 || capacity <= 0)
    return set_error(SFL_ERR_INVALID, "%s: batch, heads and capacity must be positive", what);
  if (!(scale > 0.f) || !__builtin_isfinite(scale))
    return set_error(SFL_ERR_INVALID, "%s: scale must be finite and positive", what);
  if (dtype != SFL_DTYPE_F32 && dtype != SFL_DTYPE_BF16 && dtype != SFL_DTYPE_F16)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: model dtype must be F32, BF16 or F16", what);
  const int kc = dtype == SFL_DTYPE_F32 ? 16 : 32;
  if (head_dim % kc || head_dim > 128 || (head_dim & (head_dim - 1)))
    return set_error(SFL_ERR_UNSUPPORTED, "%s: head dim %d must be a power of two in [%d, 128]", what, head_dim, kc);
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w_out) % 16)
    return set_error(SFL_ERR_INVALID, "%s: x and w_out must be 16-byte aligned", what);
  DecodeCall c{q, k, v, lengths, nullptr, nullptr, nullptr, const_cast<void*>(w_out), batch, heads,
               heads, capacity, head_dim, 1, scale, static_cast<hipStream_t>(stream)};
  c.x = x;
  c.d_model = heads * head_dim;
  if (dtype == SFL_DTYPE_BF16) return proj_dims<bf16_t>(c);
  if (dtype == SFL_DTYPE_F16) return proj_dims<f16_t>(c);
  return proj_dims<float>(c);
}

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch`, looked up once per device (with that
// device current) and kept.
int static_scratch(void** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess)
    return sfl::set_error(SFL_ERR_HIP, "decode_attention_static: hipGetDevice: %s", hipGetErrorString(err));
  if (device < 0 || device >= kMaxDevices)
    return sfl::set_error(SFL_ERR_UNSUPPORTED, "decode_attention_static: device %d beyond the %d supported",
                          device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr)
      return sfl::set_error(SFL_ERR_HIP, "decode_attention_static: hipGetSymbolAddress: %s",
                            hipGetErrorString(err));
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return SFL_OK;
}

long align256(long bytes) { return (bytes + 255) / 256 * 256; }

}  // namespace

extern "C" long sfl_decode_attention_static_scratch_bytes(void) { return kStaticScratchBytes; }

extern "C" int sfl_decode_attention_static(const void* q, const void* k, const void* v,
                                           const int32_t* lengths, void* out, int batch, int q_heads,
                                           int kv_heads, int capacity, int head_dim, int splits,
                                           float scale, int kv_dtype, int q_dtype, int out_dtype,
                                           void* stream) {
  using namespace sfl;
  const char* what = "decode_attention_static";
  if (!q || !k || !v || !lengths || !out) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || capacity <= 0)
    return set_error(SFL_ERR_INVALID, "%s: batch, heads and capacity must be positive", what);
  if (splits < 1 || splits > 1024) return set_error(SFL_ERR_INVALID, "%s: splits must be in [1, 1024]", what);
  if (head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: unsupported head dim %d", what, head_dim);
  // Partials as sfl_decode_attention takes them: max and sum [B, Hq, splits],
  // numerator [B, Hq, splits, D], fp32, each 256-byte aligned in the buffer.
  const long parts = long(batch) * q_heads * splits;
  const long max_bytes = align256(parts * 4), out_bytes = align256(parts * head_dim * 4);
  const long need = 2 * max_bytes + out_bytes;
  if (need > kStaticScratchBytes)
    return set_error(SFL_ERR_INVALID,
                     "%s: batch*q_heads*splits*(head_dim+2)*4 = %ld bytes of split scratch exceed the %ld-byte "
                     "static buffer; use fewer splits or sfl_decode_attention with caller scratch",
                     what, parts * (head_dim + 2) * 4, kStaticScratchBytes);
  void* base = nullptr;
  if (int rc = static_scratch(&base)) return rc;
  unsigned char* bytes = static_cast<unsigned char*>(base);
  return sfl_decode_attention(q, k, v, lengths, reinterpret_cast<float*>(bytes),
                              reinterpret_cast<float*>(bytes + max_bytes),
                              reinterpret_cast<float*>(bytes + 2 * max_bytes), out, batch, q_heads, kv_heads,
                              capacity, head_dim, splits, scale, kv_dtype, q_dtype, out_dtype, stream);
}

extern "C" int sfl_decode_attention(const void* q, const void* k, const void* v,
                                    const int32_t* lengths, float* partial_max,
                                    float* partial_sum, float* partial_out, void* out, int batch,
                                    int q_heads, int kv_heads, int capacity, int head_dim,
                                    int splits, float scale, int kv_dtype, int q_dtype,
                                    int out_dtype, void* stream) {
  using namespace sfl;
  if (!q || !k || !v || !lengths || !partial_max || !partial_sum || !partial_out || !out)
    return set_error(SFL_ERR_INVALID, "decode_attention: null pointer argument");
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || capacity <= 0)
    return set_error(SFL_ERR_INVALID, "decode_attention: batch, heads and capacity must be positive");
  if (q_heads % kv_heads)
    return set_error(SFL_ERR_INVALID, "decode_attention: query heads must be divisible by KV heads");
  const int groups = q_heads / kv_heads;
  if (groups != 1 && groups != 2 && groups != 4 && groups != 8)
    return set_error(SFL_ERR_UNSUPPORTED, "decode_attention: unsupported GQA ratio %d", groups);
  if (head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128)
    return set_error(SFL_ERR_UNSUPPORTED, "decode_attention: unsupported head dim %d", head_dim);
  if (splits < 1 || splits > 1024)
    return set_error(SFL_ERR_INVALID, "decode_attention: splits must be in [1, 1024]");
  if (!(scale > 0.f) || !__builtin_isfinite(scale))
    return set_error(SFL_ERR_INVALID, "decode_attention: scale must be finite and positive");
  if (kv_dtype != SFL_DTYPE_F32 && kv_dtype != SFL_DTYPE_BF16 && kv_dtype != SFL_DTYPE_F16)
    return set_error(SFL_ERR_UNSUPPORTED, "decode_attention: unsupported dtype %d", kv_dtype);
  if (q_dtype != kv_dtype && q_dtype != SFL_DTYPE_F32)
    return set_error(SFL_ERR_UNSUPPORTED, "decode_attention: q dtype must equal the KV dtype or be F32");
  const bool split_out = out_dtype == SFL_DTYPE_BF16X2 || out_dtype == SFL_DTYPE_F16X2;
  const bool act_out = split_out || out_dtype == SFL_DTYPE_F32X;
  if (out_dtype != kv_dtype && out_dtype != SFL_DTYPE_F32 && !act_out)
    return set_error(SFL_ERR_UNSUPPORTED,
                     "decode_attention: out dtype must be the KV dtype, F32, BF16X2, F16X2 or F32X");
  if (act_out && (q_heads * head_dim) % (split_out ? 32 : 16))
    return set_error(SFL_ERR_UNSUPPORTED, "decode_attention: activation-layout output needs q_heads*head_dim %% %d == 0",
                     split_out ? 32 : 16);
  const DecodeCall c{q, k, v, lengths, partial_max, partial_sum, partial_out, out, batch, q_heads,
                     kv_heads, capacity, head_dim, splits, scale, static_cast<hipStream_t>(stream)};
  int rc;
  const bool f32q = q_dtype == SFL_DTYPE_F32;
  switch (kv_dtype) {
    case SFL_DTYPE_F32: rc = attn_out<float, float>(c, out_dtype); break;
    case SFL_DTYPE_BF16: rc = f32q ? attn_out<bf16_t, float>(c, out_dtype) : attn_out<bf16_t, bf16_t>(c, out_dtype); break;
    default: rc = f32q ? attn_out<f16_t, float>(c, out_dtype) : attn_out<f16_t, f16_t>(c, out_dtype); break;
  }
  if (rc || splits == 1) return rc;
  switch (out_dtype) {
    case SFL_DTYPE_F32: return merge_dims<float>(c);
    case SFL_DTYPE_BF16: return merge_dims<bf16_t>(c);
    case SFL_DTYPE_F16: return merge_dims<f16_t>(c);
    case SFL_DTYPE_F32X: return merge_dims<f32x_t>(c);
    case SFL_DTYPE_F16X2: return merge_dims<split16_t>(c);
    default: return merge_dims<split_t>(c);
  }
}
