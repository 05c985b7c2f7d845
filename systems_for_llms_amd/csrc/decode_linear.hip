// Decode-step projections as MFMA GEMVs with fused prologues and epilogues.
//
// Every kernel computes out[b, n] = sum_k act[b, k] * W[n, k] for a batch of
// rows (one decode token per sequence), 16 rows -- the MFMA's columns -- per
// workgroup. W is the reference's [N, K]
// Linear weight (src/llmlab/model/layers.py:34-35) repacked once by
// sfl_pack_gemv_weights into the load order of the kernel: for every tile of
// 16 output rows and every K chunk, the 64 lanes' 16-byte A operands are
// stored contiguously (1 KB), as are the activations (act_format.hpp). A
// workgroup owns 16 output features; its waves split K, and every load
// instruction reads whole contiguous cache lines. (Reading the [N, K] rows
// directly touches 16 rows x 64 bytes per instruction and runs at about half
// the speed.) Partial tiles are summed across waves in LDS. The MFMA result
// layout puts 4 consecutive features of one batch row in each lane, so RoPE
// pairs, SwiGLU pairs and vector stores stay in-lane.
//
// Precision: weights and the KV cache are in the model dtype; activations,
// the residual stream and every epilogue stay in fp32. For 16-bit weights each
// fp32 activation is split into hi + lo halves of the weight type and
// multiplied by two MFMAs (the GEMV is bandwidth-bound, so the second MFMA is
// free), which keeps ~16 (bf16) or ~22 (fp16) mantissa bits of the activation
// instead of 8 or 11.
//
// RMSNorm is folded into its consumers (layers.py:133-141): RMSNorm(x) W^T =
// (1/rms(x)) * ((x * g) W^T). The residual stream x stays a plain fp32 [B, K]
// tensor; a normalized consumer (q/k/v, w1/w3, lm_head) reads its K chunks of
// x and the gain g, forms x * g in the MFMA operand format as it goes, adds up
// x^2 on the side, and scales its sums by 1 / sqrt(sum(x^2) / K + eps) once
// the waves' partials are reduced (in a fixed order, so every workgroup
// computes the same scale). Producers of x therefore only add to it, which
// lets them split K over several workgroups and accumulate with atomics.
// Epilogues:
//   QKV      RoPE on q and k (attention.py:44-58) with the host-built fp32
//            table; q to an fp32 [B, H, dk] buffer, k/v appended to the
//            model-dtype [B, H, cap, dk] cache at each row's position.
//   RESIDUAL x += W act (transformer.py:46-47), in place; with K split over
//            several workgroups each adds its partial with fp32 atomics.
//   SWIGLU   h = silu(W1 act) * (W3 act) in fp32 (layers.py:114-115).
//   LOGITS   lm_head rows (transformer.py:137-138) plus a per-tile argmax with
//            the lowest index winning ties, taken on the fp32 accumulators.
#include "gemv_ops.hpp"

namespace sfl {
namespace {


enum Epi { EPI_QKV = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2, EPI_LOGITS = 3 };

constexpr int kWaves = 8;       // waves per workgroup (K split)
constexpr int kTileN = 16;      // output features per workgroup
constexpr int kBlockRows = 16;  // batch rows per MFMA column block (one workgroup)
constexpr int kMaxRows = 1 << 16;  // batch rows per launch
constexpr int kXcds = 8;        // workgroups are dealt to the XCDs round-robin
constexpr float kEps = 1e-5f;
constexpr int kMaxSplitK = 16;  // workgroups per tile along K (RESIDUAL)

struct LinearArgs {
  const void* act;       // RESIDUAL: [B, K] input in the activation format
  const float* x_in;     // normalized consumers: the fp32 residual stream [B, K]
  const void* gain;      // and its RMSNorm gain [K] (model dtype)
  const void* w;         // packed [ceil(N/16)][K/chunk][64 lanes][16 B]
  const void* w3;        // packed second matrix of SWIGLU
  int batch, n, k;
  int ksplit;            // workgroups per 16-row tile along K (1 except RESIDUAL)
  // QKV
  const float* cos_t;    // [ctx, dk/2] fp32
  const float* sin_t;
  const int32_t* pos;    // [B]
  void* q_out;           // fp32 [B, H, dk]
  void* k_cache;         // [B, H, cap, dk]
  void* v_cache;
  int heads, head_dim, cap, d_model;
  // RESIDUAL
  float* x;              // fp32 residual [B, N], updated in place
  // SWIGLU
  void* h_out;           // [B, N] in the activation format
  // LOGITS
  void* logits;          // fp32 [B, V], optional; row offset pos[b]*logits_pos_stride
  long logits_batch_stride;
  long logits_pos_stride;
  float* best_val;       // [tiles, best_stride]
  int32_t* best_idx;
  int best_stride;
};

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}


// CPW: weight chunks each wave loads per round (one round when the workgroup's
// chunks fit kWaves*CPW); chosen on the host so no wave issues more loads than
// it needs. A workgroup owns one (tile, K part) item -- tile = item % tiles,
// part = item / tiles (one part unless RESIDUAL splits K) -- for one block of
// 16 batch rows. With one block (kBlocks false), workgroup w owns item w.
// With several, the blocks of one item go to workgroups w = 8 (g * blocks +
// blk) + x for item 8 g + x: the same XCD (w % 8 == x), so the item's weights
// come from HBM once and from that XCD's L2 for the other blocks.
// The arguments every workgroup needs before its first load come first, as
// scalars: the library builds this file with kernarg preloading, so the
// command processor places these 14 dwords in SGPRs before the waves start
// and the loads issue without waiting for a kernel-argument fetch (one such
// round trip per launch measured 17 us per 324M decode step). `aux` is the
// epilogue's first pointer: pos (QKV, LOGITS), x (RESIDUAL) or h_out (SWIGLU).
// The rest of LinearArgs is read from the kernel arguments as usual.
template <typename T, int E, int CPW, bool kBlocks>
__global__ __launch_bounds__(kWaves * kWave) void linear_kernel(const void* p_w, const void* p_src,
                                                                const void* p_gain, const void* p_w3, void* p_aux,
                                                                int p_batch, int p_n, int p_k, int p_ksplit,
                                                                LinearArgs a) {
  a.w = p_w; a.w3 = p_w3; a.gain = p_gain; a.batch = p_batch; a.n = p_n; a.k = p_k; a.ksplit = p_ksplit;
  if constexpr (E == EPI_RESIDUAL) {
    a.act = p_src;
    a.x = static_cast<float*>(p_aux);
  } else {
    a.x_in = static_cast<const float*>(p_src);
    if constexpr (E == EPI_SWIGLU) a.h_out = p_aux;
    else a.pos = static_cast<const int32_t*>(p_aux);
  }
  constexpr int KC = chunk_k<T>();
  constexpr int EPL = vec_elems<T>();
  // Two accumulators sharing the x operands: W1 and W3 (SWIGLU), or two
  // consecutive 16-row tiles of the lm_head (LOGITS), so one launch round
  // covers the vocabulary with half as many workgroups re-reading x.
  constexpr bool kTwo = (E == EPI_SWIGLU || E == EPI_LOGITS);
  constexpr int kTilesPerItem = E == EPI_LOGITS ? 2 : 1;
  constexpr bool kNorm = (E != EPI_RESIDUAL);
  constexpr int RS = (kTwo ? 8 : 4) + (kNorm ? 1 : 0);  // floats per lane in the cross-wave reduction
  using Src = typename SrcOf<kNorm, T>::type;
  __shared__ float red[kWaves * kWave * RS];
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int K = a.k;

  constexpr int CB = act_chunk_bytes<T>();
  // The loads wait for these indices, and a launch's first instructions are
  // fetched cold: the one-block instantiations of the epilogues that never
  // split K (all but RESIDUAL) compute them without a division.
  constexpr bool kOnePart = E != EPI_RESIDUAL;  // ksplit is 1
  const int tiles = (a.n + kTileN - 1) / kTileN;
  unsigned item = blockIdx.x;
  int blk = 0;
  if constexpr (kBlocks) {
    const unsigned blocks = (unsigned(a.batch) + kBlockRows - 1) / kBlockRows;
    const unsigned r = blockIdx.x / kXcds;
    blk = int(r % blocks);
    item = (r / blocks) * kXcds + blockIdx.x % kXcds;
    if (item >= unsigned((tiles + kTilesPerItem - 1) / kTilesPerItem) * unsigned(a.ksplit))
      return;  // padding of the last group of 8 items
  }
  const int tile = kOnePart ? int(item) * kTilesPerItem : int(item % unsigned(tiles));
  const int part = kOnePart ? 0 : int(item / unsigned(tiles));
  const int n0 = tile * kTileN;
  const int grp = lane / 16;
  const int b = blk * kBlockRows + lane % 16;  // this lane's batch row
  const int nchunks = K / KC;
  const int per = kOnePart ? nchunks : (nchunks + a.ksplit - 1) / a.ksplit;
  const int cb = part * per;
  const int ce = min(nchunks, cb + per);
  if (cb >= ce) return;  // an empty K part (whole workgroup)
  // This lane's 16 bytes of chunk c: w + c*1KB (packed weights); its B operand
  // from act + c*CB (activation format) or from row b of x and the gain.
  const unsigned char* wl = static_cast<const unsigned char*>(a.w) + (long(tile) * nchunks * kWave + lane) * 16;
  const unsigned char* w3l =
      E == EPI_SWIGLU ? static_cast<const unsigned char*>(a.w3) + (long(tile) * nchunks * kWave + lane) * 16
      : E == EPI_LOGITS ? static_cast<const unsigned char*>(a.w) +
                              (long(min(tile + 1, tiles - 1)) * nchunks * kWave + lane) * 16  // masked at the end
                        : nullptr;
  const bool live = b < a.batch;
  const int row = min(b, a.batch - 1);
  const unsigned char* al =
      kNorm ? nullptr : static_cast<const unsigned char*>(a.act) + long(blk) * nchunks * CB + lane * 16;
  const float* xl = kNorm ? a.x_in + long(row) * K + grp * EPL : nullptr;
  const T* gl = kNorm ? static_cast<const T*>(a.gain) + grp * EPL : nullptr;

  // Issue the first group of operand and weight loads up front. Loads are
  // unconditional, from clamped addresses, and masked where they are used: a
  // load whose value is consumed inside its own guard makes the compiler wait
  // for it on the spot, serialising the memory round trips. The operand loads
  // (cache hits) go first, so a normalized consumer forms x * g while the
  // weights are still on their way from HBM. Weights are read once per step
  // and take the non-temporal hint (measured: 1.3% faster decode steps).
  // QKV: load the position before anything else; the RoPE table loads of the
  // epilogue depend on it and are issued right after the weight loads.
  int pre_p = 0;
  if constexpr (E == EPI_QKV) pre_p = a.pos[row];
  uint4 wa[CPW], wb[kTwo ? CPW : 1];
  Src src[CPW];
  int c0 = cb + wave;
  const int last = ce - 1;
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const long c = min(c0 + j * kWaves, last);
    if constexpr (kNorm) src[j] = load_norm<T>(xl + c * KC, gl + c * KC);
    else src[j] = load_act<T>(al + c * CB);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the operand loads ahead of the weight loads
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const long c = min(c0 + j * kWaves, last);
    wa[j] = load16_stream(wl + c * kWave * 16);
    if constexpr (kTwo) wb[j] = load16_stream(w3l + c * kWave * 16);
  }

  // Prefetch what wave 0's epilogue reads, so it overlaps the weight loads.
  const int n = n0 + 4 * grp;  // this lane's features n .. n+3 of batch row b
  const int nl = min(n, a.n - 4);
  float4 pre_x = make_float4(0.f, 0.f, 0.f, 0.f);
  float2 pre_c = make_float2(0.f, 0.f), pre_s = make_float2(0.f, 0.f);
  // QKV: where this lane's features go (section 0 q, 1 k, 2 v), worked out while the loads fly.
  int section = 0;
  void* qkv_dst = nullptr;
  if (wave == 0) {
    if constexpr (E == EPI_RESIDUAL) {
      if (a.ksplit == 1) pre_x = *reinterpret_cast<const float4*>(a.x + long(row) * a.n + nl);
    } else if constexpr (E == EPI_QKV) {
      section = nl / a.d_model;
      const int f = nl - section * a.d_model;
      const int head = f / a.head_dim;
      const int dim = f - head * a.head_dim;
      const long at = long(pre_p) * (a.head_dim / 2) + dim / 2;
      pre_c = *reinterpret_cast<const float2*>(a.cos_t + at);
      pre_s = *reinterpret_cast<const float2*>(a.sin_t + at);
      if (section == 0)
        qkv_dst = static_cast<float*>(a.q_out) + (long(row) * a.heads + head) * a.head_dim + dim;
      else
        qkv_dst = static_cast<T*>(section == 1 ? a.k_cache : a.v_cache) +
                  ((long(row) * a.heads + head) * a.cap + pre_p) * a.head_dim + dim;
    }
  }

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc3 = {0.f, 0.f, 0.f, 0.f};
  float ssum = 0.f;  // this lane's share of sum(x^2) of row b (normalized consumers)
  for (;;) {
    // Operands first (they do not wait for the weights), then the MFMAs. Both
    // are unconditional, with chunks past the part masked to zero, so no load
    // is sunk into a branch behind the others.
    ActChunk<T> op[CPW];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      if constexpr (kNorm) {
        float part = 0.f;
        op[j] = norm_operand<T>(src[j], part);
        ssum += (c0 + j * kWaves < ce) ? part : 0.f;
      } else {
        op[j] = src[j];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const bool use = live && c0 + j * kWaves < ce;
      acc = mfma_act<T>(wa[j], op[j], use, acc);
      if constexpr (kTwo) acc3 = mfma_act<T>(wb[j], op[j], use, acc3);
    }
    c0 += CPW * kWaves;
    if (c0 >= ce) break;
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const long c = min(c0 + j * kWaves, last);
      if constexpr (kNorm) src[j] = load_norm<T>(xl + c * KC, gl + c * KC);
      else src[j] = load_act<T>(al + c * CB);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const long c = min(c0 + j * kWaves, last);
      wa[j] = load16_stream(wl + c * kWave * 16);
      if constexpr (kTwo) wb[j] = load16_stream(w3l + c * kWave * 16);
    }
  }

  // Sum the waves' partial tiles (and partial sums of x^2). Every thread adds
  // up one value of the tile over the waves, in wave order, and leaves the sum
  // in wave 0's slot, which only it reads; wave 0 then reads its lanes' sums.
  // (Wave 0 adding all waves' values by itself waited on ~30 small groups of
  // LDS reads while the other waves had nothing left to do.)
  float* mine = red + (wave * kWave + lane) * RS;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    mine[i] = acc[i];
    if constexpr (kTwo) mine[4 + i] = acc3[i];
  }
  if constexpr (kNorm) mine[RS - 1] = ssum;
  __syncthreads();
  constexpr int NV = kWave * RS;  // values of one wave's partial tile
  for (int q = tid; q < NV; q += kWaves * kWave) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) t += red[w * NV + q];
    red[q] = t;
  }
  __syncthreads();
  if (wave != 0) return;
  float v1[4] = {0.f, 0.f, 0.f, 0.f}, v3[4] = {0.f, 0.f, 0.f, 0.f};
  float sq = 0.f;
  {
    const float* p = red + lane * RS;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v1[i] = p[i];
      if constexpr (kTwo) v3[i] = p[4 + i];
    }
    if constexpr (kNorm) sq = p[RS - 1];
  }
  if constexpr (kNorm) {
    // Lane (row b, group g) holds group g's sum over all of K: add the 4 groups.
    sq += lane_xor(sq, 16);
    sq += lane_xor(sq, 32);
    const float inv = 1.f / sqrtf(sq / float(K) + kEps);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v1[i] *= inv;
      v3[i] *= inv;
    }
  }

  if constexpr (E == EPI_LOGITS) {
#pragma unroll
    for (int t = 0; t < kTilesPerItem; ++t) {
      const int tt = tile + t;
      if (tt >= tiles) break;  // uniform: an odd tile count leaves the last item one tile
      const float* v = t == 0 ? v1 : v3;
      const int nt = tt * kTileN + 4 * grp;  // this lane's features nt .. nt+3
      // Start from a valid index so a row of NaN logits still yields an in-range token.
      float bv = -INFINITY;
      int bi = min(nt, a.n - 1);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (nt + i < a.n && better(v[i], nt + i, bv, bi)) { bv = v[i]; bi = nt + i; }
      }
#pragma unroll
      for (int m = 16; m < kWave; m <<= 1) {
        const float ov = lane_xor(bv, m);
        const int oi = lane_xor(bi, m);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
      }
      if (live) {
        if (grp == 0) {
          a.best_val[long(tt) * a.best_stride + b] = bv;
          a.best_idx[long(tt) * a.best_stride + b] = bi;
        }
        if (a.logits && nt < a.n) {
          float* dst = static_cast<float*>(a.logits) + b * a.logits_batch_stride + nt;
          if (a.pos) dst += long(a.pos[b]) * a.logits_pos_stride;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (nt + i < a.n) dst[i] = v[i];
        }
      }
    }
    return;
  }
  if (!live || n >= a.n) return;
  if constexpr (E == EPI_RESIDUAL) {
    float* dst = a.x + long(b) * a.n + n;
    if (a.ksplit == 1) {
      *reinterpret_cast<float4*>(dst) = make_float4(pre_x.x + v1[0], pre_x.y + v1[1], pre_x.z + v1[2], pre_x.w + v1[3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) unsafeAtomicAdd(dst + i, v1[i]);
    }
  } else if constexpr (E == EPI_SWIGLU) {
    float h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      h[i] = v1[i] * v3[i] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(v1[i] * -1.4426950408889634f));
    store_act4<T>(static_cast<unsigned char*>(a.h_out), b, n, a.n, h);
  } else {  // EPI_QKV
    float y[4] = {v1[0], v1[1], v1[2], v1[3]};
    if (section < 2) {
      // Pairs (dim, dim+1) and (dim+2, dim+3) use table columns dim/2 and dim/2+1.
      const float c[2] = {pre_c.x, pre_c.y}, sn[2] = {pre_s.x, pre_s.y};
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const float e = y[i], o = y[i + 1];
        y[i] = e * c[i / 2] - o * sn[i / 2];
        y[i + 1] = e * sn[i / 2] + o * c[i / 2];
      }
    }
    if (section == 0) *static_cast<float4*>(qkv_dst) = make_float4(y[0], y[1], y[2], y[3]);
    else store4<T>(static_cast<T*>(qkv_dst), y);
  }
}

template <typename T, int E, int CPW>
int launch_linear_cpw(const LinearArgs& a, hipStream_t stream, const char* what) {
  constexpr int kTilesPerItem = E == EPI_LOGITS ? 2 : 1;  // as linear_kernel
  const long items = long(((a.n + kTileN - 1) / kTileN + kTilesPerItem - 1) / kTilesPerItem) * a.ksplit;
  const long blocks = (a.batch + kBlockRows - 1) / kBlockRows;
  const void* src = E == EPI_RESIDUAL ? a.act : static_cast<const void*>(a.x_in);
  void* aux = E == EPI_RESIDUAL ? static_cast<void*>(a.x)
              : E == EPI_SWIGLU ? a.h_out
                                : const_cast<int32_t*>(a.pos);
  if (blocks == 1) {
    hipLaunchKernelGGL((linear_kernel<T, E, CPW, false>), dim3(unsigned(items)), dim3(kWaves * kWave), 0,
                       stream, a.w, src, a.gain, a.w3, aux, a.batch, a.n, a.k, a.ksplit, a);
  } else {
    const long grid = (items + kXcds - 1) / kXcds * kXcds * blocks;
    if (grid > (1L << 31) - 1) return set_error(SFL_ERR_UNSUPPORTED, "%s: too many workgroups", what);
    hipLaunchKernelGGL((linear_kernel<T, E, CPW, true>), dim3(unsigned(grid)), dim3(kWaves * kWave), 0,
                       stream, a.w, src, a.gain, a.w3, aux, a.batch, a.n, a.k, a.ksplit, a);
  }
  return check_launch(what);
}

template <typename T, int E>
int launch_linear(const LinearArgs& a, hipStream_t stream, const char* what) {
  const int per_part = (a.k / chunk_k<T>() + a.ksplit - 1) / a.ksplit;
  const int per_wave = (per_part + kWaves - 1) / kWaves;
  if (per_wave <= 1) return launch_linear_cpw<T, E, 1>(a, stream, what);
  if (per_wave <= 2) return launch_linear_cpw<T, E, 2>(a, stream, what);
  if (per_wave <= 4) return launch_linear_cpw<T, E, 4>(a, stream, what);
  if (per_wave <= 6) return launch_linear_cpw<T, E, 6>(a, stream, what);
  if (per_wave <= 8) return launch_linear_cpw<T, E, 8>(a, stream, what);
  return launch_linear_cpw<T, E, 11>(a, stream, what);  // larger K loops in rounds of 11
}

// vec4: the epilogue moves 4 consecutive features per lane (all but LOGITS).
int check_common(const char* what, int batch, int n, int k, int dtype, bool vec4 = true) {
  if (batch < 1 || batch > kMaxRows)
    return set_error(SFL_ERR_INVALID, "%s: batch must be in [1, %d]", what, kMaxRows);
  if (n < 1 || k < 1) return set_error(SFL_ERR_INVALID, "%s: sizes must be positive", what);
  if (vec4 && n % 4) return set_error(SFL_ERR_UNSUPPORTED, "%s: N must be a multiple of 4", what);
  if (dtype != SFL_DTYPE_F32 && dtype != SFL_DTYPE_BF16 && dtype != SFL_DTYPE_F16)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: model dtype must be F32, BF16 or F16", what);
  const int kc = dtype == SFL_DTYPE_F32 ? chunk_k<float>() : chunk_k<bf16_t>();
  if (k % kc) return set_error(SFL_ERR_UNSUPPORTED, "%s: K=%d must be a multiple of %d", what, k, kc);
  return SFL_OK;
}

// Normalized inputs: x rows are read as float4 (16-byte aligned rows).
int check_normed(const char* what, const float* x, const void* gain) {
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(gain) % 16)
    return set_error(SFL_ERR_INVALID, "%s: x and gain must be 16-byte aligned", what);
  return SFL_OK;
}

template <int E>
int dispatch_linear(LinearArgs a, int dtype, hipStream_t s, const char* what) {
  if (a.ksplit < 1) a.ksplit = 1;
  if (dtype == SFL_DTYPE_BF16) return launch_linear<bf16_t, E>(a, s, what);
  if (dtype == SFL_DTYPE_F16) return launch_linear<f16_t, E>(a, s, what);
  return launch_linear<float, E>(a, s, what);
}

// Packed GEMV weights: 16-byte unit u = (tile * nchunks + c) * 64 + lane holds
// row tile*16 + lane%16, k values [c*KC + (lane/16)*EPL, +EPL) (zeros past N).
template <typename T>
__global__ __launch_bounds__(256) void pack_weights_kernel(const T* __restrict__ w, uint4* __restrict__ packed,
                                                           int n, int k) {
  constexpr int KC = chunk_k<T>(), EPL = vec_elems<T>();
  const int nchunks = k / KC;
  const long units = long((n + kTileN - 1) / kTileN) * nchunks * kWave;
  for (long u = long(blockIdx.x) * 256 + threadIdx.x; u < units; u += long(gridDim.x) * 256) {
    const int lane = int(u % kWave);
    const long tc = u / kWave;
    const int c = int(tc % nchunks);
    const int row = int(tc / nchunks) * kTileN + lane % 16;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < n) v = load16(w + long(row) * k + c * KC + (lane / 16) * EPL);
    packed[u] = v;
  }
}

}  // namespace
}  // namespace sfl

using namespace sfl;

extern "C" int sfl_rmsnorm_qkv_rope_append(const float* x, const void* gain, const void* w_qkv,
                                           const float* cos_t, const float* sin_t,
                                           const int32_t* pos, void* q_out, void* k_cache,
                                           void* v_cache, int batch, int d_model, int heads,
                                           int capacity, int dtype, void* stream) {
  const char* what = "rmsnorm_qkv_rope_append";
  if (!x || !gain || !w_qkv || !cos_t || !sin_t || !pos || !q_out || !k_cache || !v_cache)
    return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (heads < 1 || d_model % heads) return set_error(SFL_ERR_INVALID, "%s: d_model must be divisible by heads", what);
  const int dk = d_model / heads;
  if (dk % 16) return set_error(SFL_ERR_UNSUPPORTED, "%s: head dim must be a multiple of 16", what);
  if (capacity < 1) return set_error(SFL_ERR_INVALID, "%s: capacity must be positive", what);
  if (int rc = check_common(what, batch, 3 * d_model, d_model, dtype)) return rc;
  if (int rc = check_normed(what, x, gain)) return rc;
  LinearArgs a{};
  a.x_in = x; a.gain = gain; a.w = w_qkv; a.batch = batch; a.n = 3 * d_model; a.k = d_model;
  a.cos_t = cos_t; a.sin_t = sin_t; a.pos = pos; a.q_out = q_out; a.k_cache = k_cache;
  a.v_cache = v_cache; a.heads = heads; a.head_dim = dk; a.cap = capacity; a.d_model = d_model;
  return dispatch_linear<EPI_QKV>(a, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_linear_residual(const void* act, const void* w, float* x, int batch, int n, int k,
                                   int ksplit, int dtype, void* stream) {
  const char* what = "linear_residual";
  if (!act || !w || !x) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (int rc = check_common(what, batch, n, k, dtype)) return rc;
  if (ksplit < 1 || ksplit > kMaxSplitK)
    return set_error(SFL_ERR_INVALID, "%s: ksplit must be in [1, %d]", what, kMaxSplitK);
  if (reinterpret_cast<uintptr_t>(x) % 16) return set_error(SFL_ERR_INVALID, "%s: x must be 16-byte aligned", what);
  LinearArgs a{};
  a.act = act; a.w = w; a.x = x; a.batch = batch; a.n = n; a.k = k; a.ksplit = ksplit;
  return dispatch_linear<EPI_RESIDUAL>(a, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_rmsnorm_swiglu(const float* x, const void* gain, const void* w1, const void* w3,
                                  void* h_out, int batch, int d_model, int d_ff, int dtype,
                                  void* stream) {
  const char* what = "rmsnorm_swiglu";
  if (!x || !gain || !w1 || !w3 || !h_out) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (int rc = check_common(what, batch, d_ff, d_model, dtype)) return rc;
  if (int rc = check_normed(what, x, gain)) return rc;
  const int kc = dtype == SFL_DTYPE_F32 ? chunk_k<float>() : chunk_k<bf16_t>();
  if (d_ff % kc)  // h is written in the activation layout, whole chunks per row
    return set_error(SFL_ERR_UNSUPPORTED, "%s: d_ff=%d must be a multiple of %d", what, d_ff, kc);
  LinearArgs a{};
  a.x_in = x; a.gain = gain; a.w = w1; a.w3 = w3; a.h_out = h_out; a.batch = batch; a.n = d_ff;
  a.k = d_model;
  return dispatch_linear<EPI_SWIGLU>(a, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_rmsnorm_lm_head(const float* x, const void* gain, const void* w_head,
                                   void* logits, long logits_batch_stride, const int32_t* pos,
                                   long logits_pos_stride, float* best_val, int32_t* best_idx,
                                   int best_stride, int batch, int d_model, int vocab, int dtype,
                                   void* stream) {
  const char* what = "rmsnorm_lm_head";
  if (!x || !gain || !w_head || !best_val || !best_idx)
    return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (int rc = check_common(what, batch, vocab, d_model, dtype, false)) return rc;
  if (int rc = check_normed(what, x, gain)) return rc;
  if (best_stride < batch) return set_error(SFL_ERR_INVALID, "%s: best_stride must be >= batch", what);
  LinearArgs a{};
  a.x_in = x; a.gain = gain; a.w = w_head; a.logits = logits; a.logits_batch_stride = logits_batch_stride;
  a.pos = pos; a.logits_pos_stride = logits_pos_stride; a.best_val = best_val; a.best_idx = best_idx;
  a.best_stride = best_stride;
  a.batch = batch; a.n = vocab; a.k = d_model;
  return dispatch_linear<EPI_LOGITS>(a, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_lm_head_tiles(int vocab) { return (vocab + kTileN - 1) / kTileN; }

extern "C" long sfl_packed_gemv_elems(int n, int k) { return long((n + kTileN - 1) / kTileN) * kTileN * k; }

extern "C" int sfl_pack_gemv_weights(const void* w, void* packed, int n, int k, int dtype, void* stream) {
  const char* what = "pack_gemv_weights";
  if (!w || !packed) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (n < 1 || k < 1) return set_error(SFL_ERR_INVALID, "%s: sizes must be positive", what);
  if (dtype != SFL_DTYPE_F32 && dtype != SFL_DTYPE_BF16 && dtype != SFL_DTYPE_F16)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: dtype must be F32, BF16 or F16", what);
  const bool half = dtype != SFL_DTYPE_F32;  // 16-bit values pack alike whatever their format
  const int kc = half ? chunk_k<bf16_t>() : chunk_k<float>();
  if (k % kc) return set_error(SFL_ERR_UNSUPPORTED, "%s: K=%d must be a multiple of %d", what, k, kc);
  if (reinterpret_cast<uintptr_t>(w) % 16 || reinterpret_cast<uintptr_t>(packed) % 16)
    return set_error(SFL_ERR_INVALID, "%s: pointers must be 16-byte aligned", what);
  const long units = sfl_packed_gemv_elems(n, k) / (16 / (half ? 2 : 4));
  const unsigned blocks = unsigned(std::min<long>((units + 255) / 256, 4096));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (half)
    hipLaunchKernelGGL(pack_weights_kernel<bf16_t>, dim3(blocks), dim3(256), 0, s, static_cast<const bf16_t*>(w),
                       static_cast<uint4*>(packed), n, k);
  else
    hipLaunchKernelGGL(pack_weights_kernel<float>, dim3(blocks), dim3(256), 0, s, static_cast<const float*>(w),
                       static_cast<uint4*>(packed), n, k);
  return check_launch(what);
}
