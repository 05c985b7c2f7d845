// Masked softmax attention over a block schedule (prefill), bf16/fp16 MFMA.
//
// Semantics follow attention_lab/triton_attention.py: a query tile visits the
// key tiles of its schedule row -- analytic interval bounds
// (interval_attention_forward, :209-321) or a CSR list with full/partial flags
// (csr_attention_forward, :126-197) -- with an online softmax in fp32 whose
// rescale is safe for fully masked rows (:176-183); rows with no admissible
// key produce zeros and LSE -inf (:191-197); LSE is the natural log; full
// tiles skip the elementwise mask except at the sequence tail (:225-234).
// The mask language is attention_lab/masks.py:84-106 plus this build's
// global key prefix: allowed = causal_ok & doc_ok & (window_ok | k < prefix).
//
// gfx950 design: a workgroup of 4 waves owns 64 query rows of one (batch,
// head); each wave owns 16 rows. Key tiles of 64 rows are staged in LDS (K
// row-major, V transposed). Scores are computed transposed, S^T = K Q^T, with
// 16x16x32 MFMAs so each lane holds 16 scores of ONE query: the row max and
// row sum need only two cross-lane steps and the rescale factor is per lane.
// The P V product is O^T = V^T P^T; its key order is chosen so that the B
// operand is exactly the probabilities the lane already holds (the product is
// a sum over keys, so any order both operands share is exact), and V^T rows
// come from LDS as 8-byte runs.
#include <algorithm>
#include <climits>
#include <stdio.h>

#include "attn_mfma.hpp"
#include "lds_dma.hpp"

namespace sfl {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BQ = 64;        // query rows per workgroup
constexpr int BK = 64;        // key rows per tile
constexpr int kThreads = 256;
constexpr int kPadK = 8;      // LDS padding (elements) of K rows and V^T rows

template <typename T>
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma16<bf16_t>(const u32x4& a, const u32x4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16<f16_t>(const u32x4& a, const u32x4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <typename T> __device__ __forceinline__ uint16_t to_bits(float v);
template <> __device__ __forceinline__ uint16_t to_bits<bf16_t>(float v) { return f32_to_bf16_bits(v); }
template <> __device__ __forceinline__ uint16_t to_bits<f16_t>(float v) { return f32_to_f16_bits(v); }

struct MaskArgs {
  int causal;
  int left, right;      // < 0: unbounded
  int prefix;           // global key prefix (0: none)
  const int64_t* docs;  // same-document labels (nullptr: none)
};

struct Sched {
  int mode;             // 0 interval, 1 csr
  int use_full;
  const int32_t* row_ptr;
  const int32_t* col_idx;
  const uint8_t* full;
};

// The CSR entries of one query tile's row, 64 at a time in one VGPR: lane l
// holds entry first + l as 2 * column + full flag. A key tile's entry is then
// a readlane instead of a memory round trip in front of every tile's loads;
// the window moves (one load) every 64 tiles. `it` must be wave-uniform.
struct RowSched {
  const int32_t* col;
  const uint8_t* full;
  int count, first, reg;
  __device__ __forceinline__ void fetch(int f) {
    first = f;
    const int i = f + int(threadIdx.x % kWave);
    reg = i < count ? 2 * col[i] + int(full[i] != 0) : 0;
  }
  __device__ __forceinline__ void at(int it, int& kb, bool& fl) {
    if ((it & ~63) != first) fetch(it & ~63);
    const int e = __builtin_amdgcn_readlane(reg, it & 63);
    kb = e >> 1;
    fl = (e & 1) != 0;
  }
};

struct AttnArgs {
  const void *q, *k, *v;
  void* o;
  float* lse;
  long qs[3], ks[3], vs[3], os[3];  // strides (elements) of batch, head, sequence
  int batch, heads, n;
  float scale_log2;
  MaskArgs m;
  Sched s;
};

__device__ __forceinline__ bool allowed(const MaskArgs& m, int q, int k, int n) {
  if (k >= n || q >= n) return false;
  if (m.causal && k > q) return false;
  if (m.docs && m.docs[q] != m.docs[k]) return false;
  if (k < m.prefix) return true;
  if (m.left >= 0 && q - k > m.left) return false;
  if (m.right >= 0 && k - q > m.right) return false;
  return true;
}

// allowed() without short-circuit branches, with the document labels of q and
// k already loaded (ignored when m.docs is null).
__device__ __forceinline__ bool allowed_flat(const MaskArgs& m, int q, int k, int n, int64_t dq, int64_t dk) {
  const bool in = (k < n) & (q < n);
  const bool causal_ok = !m.causal | (k <= q);
  const bool doc_ok = !m.docs | (dq == dk);
  const bool left_ok = (m.left < 0) | (q - k <= m.left);
  const bool right_ok = (m.right < 0) | (k - q <= m.right);
  return in & causal_ok & doc_ok & ((k < m.prefix) | (left_ok & right_ok));
}

// Workgroup -> (query tile, batch * head) of a 1-D grid, XCD-aware. Workgroups
// are dealt to the 8 XCDs round-robin and each XCD has its own 4 MB L2, so XCD
// x takes a contiguous range of the head-major tile order: the ~100
// workgroups an XCD runs at once then share the K/V of 2-3 heads (0.8 MB per
// head at 3072 x 64 bf16) instead of every XCD streaming every head's K/V.
// Query tiles run last-first, so the longest causal rows start first. When
// the XCD's range is two or more whole heads, it is dealt query-tile major
// across groups of up to kTileOrderHeads heads: the tail of each group (and
// of the range) is then the short rows of several heads, not one head's
// short rows after other heads' long ones, while the heads an XCD runs at
// once stay few enough to share their K/V in its L2 (measured: causal
// 16x16x3072 417 -> 392 us, config 5 125 -> 119 us; 4 or 6 heads per
// group gained less, 12-16 the same, all 32 at once lost the gain).
constexpr int kXcds = 8;
constexpr int kTileOrderHeads = 8;
__device__ __forceinline__ int2 attn_tile(int nqt, int nbh) {
  const int total = nqt * nbh;
  const int blk = int(blockIdx.x);
  const int x = blk % kXcds, idx = blk / kXcds;
  const int base = total / kXcds, extra = total % kXcds;
  const int start = x * base + min(x, extra);
  const int len = base + (x < extra);
  if (len >= 2 * nqt && start % nqt == 0 && len % nqt == 0) {
    constexpr int G = kTileOrderHeads;
    const int heads = len / nqt;
    const int grp = idx / (G * nqt), g = min(G, heads - grp * G), r = idx - grp * G * nqt;
    return make_int2(nqt - 1 - r / g, start / nqt + grp * G + r % g);
  }
  const int t = start + idx;
  return make_int2(nqt - 1 - t % nqt, t / nqt);
}

// Tile geometry of one query tile, as masks.py/_tile_geometry derives it.
struct TileBounds {
  int begin, end, gend;  // window blocks [begin, end), global blocks [0, gend)
  int f_lo, f_hi, gf_hi; // keys admissible for every row: [f_lo, f_hi] U [0, gf_hi]
};

__device__ __forceinline__ TileBounds tile_bounds(const MaskArgs& m, int n, int q0, int q1) {
  const int right = m.causal ? (m.right < 0 ? 0 : min(0, m.right)) : m.right;  // < 0 unbounded when !causal
  const bool has_right = m.causal || m.right >= 0;
  const int w_lo = m.left < 0 ? 0 : max(0, q0 - m.left);
  const int w_hi = has_right ? min(n - 1, q1 + right) : n - 1;
  TileBounds t;
  t.begin = w_lo / BK;
  t.end = w_hi / BK + 1;
  t.f_lo = m.left < 0 ? 0 : max(0, q1 - m.left);
  t.f_hi = has_right ? min(n - 1, q0 + right) : n - 1;
  const int g = min(m.prefix, n);
  const int g_hi = m.causal ? min(g - 1, q1) : g - 1;
  t.gf_hi = m.causal ? min(g - 1, q0) : g - 1;
  t.gend = g_hi >= 0 ? g_hi / BK + 1 : 0;
  return t;
}

// Whether every key of [k0, k1] is admissible for every row of the tile
// (without documents): [k0, k1] inside [0, gf_hi] U [f_lo, f_hi].
__device__ __forceinline__ bool covered(const TileBounds& t, int k0, int k1) {
  int pos = k0;
  if (t.gf_hi >= 0 && pos <= t.gf_hi) pos = t.gf_hi + 1;
  if (pos > k1) return true;
  if (t.f_lo <= pos && pos <= t.f_hi) pos = t.f_hi + 1;
  if (pos > k1) return true;
  // [0, gf_hi] may also cover the tail if f-range came first
  if (t.gf_hi >= 0 && pos <= t.gf_hi) pos = t.gf_hi + 1;
  return pos > k1;
}

template <typename T, int D>
__global__ __launch_bounds__(kThreads) void masked_attention_kernel(AttnArgs a) {
  constexpr int KSTEPS = D / 32;   // MFMA k-steps over the head dim
  constexpr int DT = D / 16;       // 16-wide d tiles of O^T
  constexpr int LDK = D + kPadK;   // K row stride (elements)
  constexpr int LDV = BK + kPadK;  // V^T row stride (elements)
  __shared__ __align__(16) uint16_t k_s[BK * LDK];
  __shared__ __align__(16) uint16_t vt_s[D * LDV];

  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int col = lane % 16, grp = lane / 16;
  const int2 tile = attn_tile((a.n + BQ - 1) / BQ, a.batch * a.heads);
  const int qt = tile.x;
  const int bh = tile.y;
  const int b = bh / a.heads, h = bh % a.heads;
  const int n = a.n;
  const int q0 = qt * BQ;
  const int q1 = min(q0 + BQ, n) - 1;
  const int qrow = q0 + wave * 16 + col;  // this lane's query row

  const uint16_t* qp = static_cast<const uint16_t*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const uint16_t* kp = static_cast<const uint16_t*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const uint16_t* vp = static_cast<const uint16_t*>(a.v) + b * a.vs[0] + h * a.vs[1];

  // Q^T operand: lane holds Q[qrow][32*ks + 8*grp .. +8] for every k-step.
  u32x4 qreg[KSTEPS];
  {
    const uint16_t* qr = qp + long(min(qrow, n - 1)) * a.qs[2];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const uint4 r = load16(qr + 32 * ks + 8 * grp);
      qreg[ks] = u32x4{r.x, r.y, r.z, r.w};
    }
  }

  float m_run = -INFINITY, l_run = 0.f;
  float m_lim = -INFINITY, m_sub = 0.f;  // m_run + kLazyMax and the subtracted maximum
  f32x4 oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const TileBounds tb = tile_bounds(a.m, n, q0, q1);
  int count, base = 0;
  if (a.s.mode == 1) {
    base = a.s.row_ptr[qt];
    count = a.s.row_ptr[qt + 1] - base;
  } else {
    const int lowg = min(tb.gend, tb.begin);
    count = lowg + max(0, max(tb.end, tb.gend) - tb.begin);
  }
  const int lowg = min(tb.gend, tb.begin);
  RowSched rs{a.s.col_idx + base, a.s.full + base, count, 0, 0};
  if (a.s.mode == 1) rs.fetch(0);

  for (int it = 0; it < count; ++it) {
    int kb;
    bool full;
    if (a.s.mode == 1) {
      rs.at(it, kb, full);
    } else {
      kb = it < lowg ? it : tb.begin + (it - lowg);
      full = !a.m.docs && covered(tb, kb * BK, min(kb * BK + BK, n) - 1);
    }
    full = full && a.s.use_full;
    const int k0 = kb * BK;

    // Stage the key tile: K row-major, V transposed.
    __syncthreads();
#pragma unroll
    for (int r = 0; r < (BK * D / 8) / kThreads; ++r) {
      const int idx = tid + r * kThreads;
      const int key = idx / (D / 8), dg = idx % (D / 8);
      const int kr = min(k0 + key, n - 1);
      const uint4 kv = load16(kp + long(kr) * a.ks[2] + dg * 8);
      const uint4 vv = load16(vp + long(kr) * a.vs[2] + dg * 8);
      *reinterpret_cast<uint4*>(k_s + key * LDK + dg * 8) = kv;
      const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vt_s[(dg * 8 + 2 * e) * LDV + key] = uint16_t(w[e] & 0xffffu);
        vt_s[(dg * 8 + 2 * e + 1) * LDV + key] = uint16_t(w[e] >> 16);
      }
    }
    __syncthreads();

    // S^T = K Q^T: subtile j covers keys 16j .. 16j+15; lane holds keys 16j + 4*grp + i.
    f32x4 sacc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const u32x4 ka = *reinterpret_cast<const u32x4*>(k_s + (16 * j + col) * LDK + 32 * ks + 8 * grp);
        sacc[j] = mfma16<T>(ka, qreg[ks], sacc[j]);
      }
    }
    // Unscaled scores (the scale goes into the exponent). Full tiles inside the
    // sequence need no mask (rows past n are never stored); the branch is
    // wave-uniform. Other tiles evaluate the mask without branches: with the
    // short-circuit allowed() inside a per-lane branch, selecting the unchanged
    // accumulator value made the compiler write -inf into that accumulator
    // register for every lane of the branch, the admissible ones included.
    const bool fast = full && k0 + BK <= n;
    float sv[16];
    if (fast) {
#pragma unroll
      for (int e = 0; e < 16; ++e) sv[e] = sacc[e / 4][e % 4];
    } else {
      const int64_t dq = a.m.docs ? a.m.docs[min(qrow, n - 1)] : 0;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = k0 + 16 * (e / 4) + 4 * grp + e % 4;
        const int64_t dk = a.m.docs ? a.m.docs[min(key, n - 1)] : 0;
        const bool ok = full ? (key < n) & (qrow < n) : allowed_flat(a.m, qrow, key, n, dq, dk);
        sv[e] = ok ? sacc[e / 4][e % 4] : -INFINITY;
      }
    }
    float mx = sv[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) mx = fmaxf(mx, sv[e]);
    mx = fmaxf(mx, lane_xor(mx, 16));
    mx = fmaxf(mx, lane_xor(mx, 32));
    // The softmax of the other kernels of this file: a lazy running maximum
    // (it moves only when a tile's maximum exceeds it by more than kLazyMax
    // log2 units), p = 2^(s * c - m) with one FMA, p stored in T for the P V
    // product, and the row sum taken over those stored values, so the output
    // is exactly sum(p v) / sum(p) of the weights the product used.
    const float cs = a.scale_log2;
    const bool grow = mx * cs > m_lim;  // false for a fully masked row (mx = -inf)
    float alpha = 1.f;
    if (grow) {
      alpha = exp2f(m_run - mx * cs);  // 0 for the first admissible tile
      m_run = mx * cs;
      m_lim = m_run + kLazyMax;
      m_sub = m_run;
    }
    if (__ballot(alpha != 1.f)) {  // wave-uniform: skip the rescale while no maximum moves
#pragma unroll
      for (int t = 0; t < DT; ++t) oacc[t] *= alpha;
    }
    uint32_t pk[8];
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pk[e] = pack2<T>(exp2f(fmaf(sv[2 * e], cs, -m_sub)), exp2f(fmaf(sv[2 * e + 1], cs, -m_sub)));
      psum = add_pair<T>(pk[e], psum);
    }
    psum += lane_xor(psum, 16);
    psum += lane_xor(psum, 32);
    l_run = l_run * alpha + psum;

    // O^T += V^T P^T. Step s covers subtiles 2s and 2s+1; element e of the
    // lane's operands is key 16*(2s + e/4) + 4*grp + e%4 for both operands
    // (the pair (4*(2s + e/2) + (2e)%4, +1) of sv is pk[4s + e]).
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const u32x4 pop = {pk[4 * s2], pk[4 * s2 + 1], pk[4 * s2 + 2], pk[4 * s2 + 3]};
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const uint16_t* vrow = vt_s + (16 * t + col) * LDV;
        const uint2 a0 = *reinterpret_cast<const uint2*>(vrow + 16 * (2 * s2) + 4 * grp);
        const uint2 a1 = *reinterpret_cast<const uint2*>(vrow + 16 * (2 * s2 + 1) + 4 * grp);
        const u32x4 vop = {a0.x, a0.y, a1.x, a1.y};
        oacc[t] = mfma16<T>(vop, pop, oacc[t]);
      }
    }
  }

  if (qrow >= n) return;
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  uint16_t* op = static_cast<uint16_t*>(a.o) + b * a.os[0] + h * a.os[1] + long(qrow) * a.os[2];
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    const uint32_t lo = uint32_t(to_bits<T>(oacc[t][0] * inv)) | (uint32_t(to_bits<T>(oacc[t][1] * inv)) << 16);
    const uint32_t hi = uint32_t(to_bits<T>(oacc[t][2] * inv)) | (uint32_t(to_bits<T>(oacc[t][3] * inv)) << 16);
    *reinterpret_cast<uint2*>(op + 16 * t + 4 * grp) = make_uint2(lo, hi);
  }
  if (a.lse && grp == 0) {
    const float lse = l_run > 0.f ? (m_sub + log2f(l_run)) * 0.6931471805599453f : -INFINITY;
    a.lse[(long(b) * a.heads + h) * n + qrow] = lse;
  }
}

// Head dim 64: one workgroup of 2 waves per 64-query tile (its CSR row or
// interval bounds); each wave computes 32 queries (2 MFMA column tiles), so
// the K/V bytes of a tile feed 2x the MFMAs of the 16-queries-per-wave kernel
// above while the registers stay within 256 per lane (2 waves per SIMD, no
// accumulator moves). Each wave reads K straight from global memory into its
// MFMA A operands; the pair loads V together and writes it transposed into a
// double-buffered LDS tile, one barrier per key tile. The next tile's K/V
// loads are issued before the current tile's math. The softmax keeps the
// scores unscaled (scale > 0 commutes with the max) and folds the scale into
// the exponent: p = 2^(s*c - m) with one FMA.
// One key tile of the pair kernel for this wave's QS query subtiles: S^T =
// K Q^T from the K operands `kc`, the masked online softmax, and O^T += V^T P^T
// from the transposed V tile `vt` in LDS.
template <typename T, int QS, int DT, int KSTEPS, int LDV>
__device__ __forceinline__ void tile_math(const AttnArgs& a, const u32x4 (&kc)[4][KSTEPS],
                                          const u32x4 (&qreg)[QS][KSTEPS], const uint16_t* vt,
                                          f32x4 (&oacc)[QS][DT], float (&m_run)[QS], float (&l_run)[QS],
                                          int qw, int col, int grp, int n, int k0, bool full) {
  // V^T operands: element e of step s2 is key 16*(2s2 + e/4) + 4grp + e%4 of dim 16t + col.
  u32x4 vop[2][DT];
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const uint16_t* vrow = &vt[(16 * t + col) * LDV];
      const uint2 a0 = *reinterpret_cast<const uint2*>(vrow + 16 * (2 * s2) + 4 * grp);
      const uint2 a1 = *reinterpret_cast<const uint2*>(vrow + 16 * (2 * s2 + 1) + 4 * grp);
      vop[s2][t] = u32x4{a0.x, a0.y, a1.x, a1.y};
    }
  const bool fast = full && k0 + BK <= n;

#pragma unroll
  for (int qs = 0; qs < QS; ++qs) {
    const int qrow = qw + 16 * qs + col;
    // S^T = K Q^T: lane holds keys 16j + 4grp + i of query qrow.
    f32x4 sacc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) sacc[j] = mfma16<T>(kc[j][ks], qreg[qs][ks], sacc[j]);
    }
    // Full tiles need no mask (rows past n are never stored); the branch is
    // uniform. Other tiles evaluate the mask arithmetically per score.
    float sv[16];
    if (fast) {
#pragma unroll
      for (int e = 0; e < 16; ++e) sv[e] = sacc[e / 4][e % 4];
    } else {
      const int64_t dq = a.m.docs ? a.m.docs[min(qrow, n - 1)] : 0;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = k0 + 16 * (e / 4) + 4 * grp + e % 4;
        const int64_t dk = a.m.docs ? a.m.docs[min(key, n - 1)] : 0;
        const bool ok = full ? (key < n) & (qrow < n) : allowed_flat(a.m, qrow, key, n, dq, dk);
        sv[e] = ok ? sacc[e / 4][e % 4] : -INFINITY;
      }
    }
    float mx = fmaxf(fmaxf(sv[0], sv[1]), sv[2]);
#pragma unroll
    for (int e = 3; e < 15; e += 2) mx = fmaxf(fmaxf(mx, sv[e]), sv[e + 1]);
    mx = fmaxf(mx, sv[15]);
    mx = fmaxf(mx, lane_xor(mx, 16));
    mx = fmaxf(mx, lane_xor(mx, 32));
    // The lazy maximum and stored-probability row sums of masked_attention32_kernel:
    // m_run (the subtracted maximum) moves only when the tile's maximum exceeds
    // it by more than kLazyMax log2 units, and l sums the T-rounded probabilities
    // that the P V product uses.
    const float c = a.scale_log2;
    const bool grow = mx * c > m_run[qs] + kLazyMax;  // false for a fully masked row
    const float alpha = grow ? __builtin_amdgcn_exp2f(m_run[qs] - mx * c) : 1.f;
    if (grow) m_run[qs] = mx * c;
    const float ms = m_run[qs] == -INFINITY ? 0.f : m_run[qs];
    uint32_t pk[8];
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pk[e] = pack2<T>(__builtin_amdgcn_exp2f(fmaf(sv[2 * e], c, -ms)),
                       __builtin_amdgcn_exp2f(fmaf(sv[2 * e + 1], c, -ms)));
      psum = add_pair<T>(pk[e], psum);
    }
    psum += lane_xor(psum, 16);
    psum += lane_xor(psum, 32);
    l_run[qs] = l_run[qs] * alpha + psum;
    if (__ballot(alpha != 1.f)) {  // wave-uniform: skip the rescale while no maximum moves
#pragma unroll
      for (int t = 0; t < DT; ++t) oacc[qs][t] *= alpha;
    }

    // O^T += V^T P^T; the key order makes the B operand the lane's own probabilities
    // (element e of step s2 is the pair pk[4 s2 + e]).
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const u32x4 pop = {pk[4 * s2], pk[4 * s2 + 1], pk[4 * s2 + 2], pk[4 * s2 + 3]};
#pragma unroll
      for (int t = 0; t < DT; ++t) oacc[qs][t] = mfma16<T>(vop[s2][t], pop, oacc[qs][t]);
    }
  }
}

constexpr int kPairWaves = 2;

template <typename T>
__global__ __launch_bounds__(kPairWaves * kWave) __attribute__((amdgpu_waves_per_eu(2))) void masked_attention_pair_kernel(AttnArgs a) {
  constexpr int D = 64, KSTEPS = D / 32, DT = D / 16, QS = BQ / 16 / kPairWaves;
  constexpr int LDV = BK + kPadK;
  __shared__ __align__(16) uint16_t vt_s[2][D * LDV];
  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int col = lane % 16, grp = lane / 16;
  const int n = a.n;
  const int2 tile = attn_tile((a.n + BQ - 1) / BQ, a.batch * a.heads);
  const int qt = tile.x;
  const int bh = tile.y;
  const int b = bh / a.heads, h = bh % a.heads;
  const int q0 = qt * BQ;
  const int q1 = min(q0 + BQ, n) - 1;
  const int qw = q0 + wave * 16 * QS;  // this wave's first query

  const uint16_t* qp = static_cast<const uint16_t*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const uint16_t* kp = static_cast<const uint16_t*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const uint16_t* vp = static_cast<const uint16_t*>(a.v) + b * a.vs[0] + h * a.vs[1];

  // Q^T operands: subtile qs, lane holds Q[qw + 16qs + col][32ks + 8grp .. +8].
  u32x4 qreg[QS][KSTEPS];
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) {
    const uint16_t* qr = qp + long(min(qw + 16 * qs + col, n - 1)) * a.qs[2];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const uint4 r = load16(qr + 32 * ks + 8 * grp);
      qreg[qs][ks] = u32x4{r.x, r.y, r.z, r.w};
    }
  }

  float m_run[QS], l_run[QS];
  f32x4 oacc[QS][DT];
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) {
    m_run[qs] = -INFINITY;
    l_run[qs] = 0.f;
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[qs][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const TileBounds tb = tile_bounds(a.m, n, q0, q1);
  int count, base = 0;
  if (a.s.mode == 1) {
    base = a.s.row_ptr[qt];
    count = a.s.row_ptr[qt + 1] - base;
  } else {
    const int lowg = min(tb.gend, tb.begin);
    count = lowg + max(0, max(tb.end, tb.gend) - tb.begin);
  }
  const int lowg = min(tb.gend, tb.begin);
  RowSched rs{a.s.col_idx + base, a.s.full + base, count, 0, 0};
  if (a.s.mode == 1) rs.fetch(0);

  // Per tile at key block kb: K operands of key subtile j (keys 16j + col),
  // and this thread's share of V: rows 4*(tid % 16) + u (u < 4), dims
  // 8*(tid / 16) .. +8 (128 threads cover 64 keys x 64 dims).
  const int vr0 = 4 * (tid % 16), vd0 = 8 * (tid / 16);
  u32x4 ka[4][KSTEPS], kb2[4][KSTEPS];  // K operands, alternating between tiles
  uint4 vreg[4];
#define SFL_LOAD_TILE(kb, KD)                                                               \
  {                                                                                         \
    const int k0_ = (kb) * BK;                                                              \
    _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                         \
      const uint16_t* kr_ = kp + long(min(k0_ + 16 * j + col, n - 1)) * a.ks[2];            \
      _Pragma("unroll") for (int ks = 0; ks < KSTEPS; ++ks) {                               \
        const uint4 r_ = load16(kr_ + 32 * ks + 8 * grp);                                   \
        KD[j][ks] = u32x4{r_.x, r_.y, r_.z, r_.w};                                          \
      }                                                                                     \
    }                                                                                       \
    _Pragma("unroll") for (int u = 0; u < 4; ++u)                                           \
      vreg[u] = load16(vp + long(min(k0_ + vr0 + u, n - 1)) * a.vs[2] + vd0);               \
  }
#define SFL_TILE_AT(it, kb_, fl_)                                                           \
  if (a.s.mode == 1) {                                                                      \
    rs.at((it), kb_, fl_);                                                                  \
  } else {                                                                                  \
    kb_ = (it) < lowg ? (it) : tb.begin + ((it) - lowg);                                    \
    fl_ = !a.m.docs && covered(tb, kb_ * BK, min(kb_ * BK + BK, n) - 1);                    \
  }
  // V^T tile into LDS buffer `buf`: dims vd0 + e, keys vr0 .. vr0+3 (one 8-byte store each).
#define SFL_STORE_VT(buf)                                                                   \
  {                                                                                         \
    const uint32_t w0_[4] = {vreg[0].x, vreg[0].y, vreg[0].z, vreg[0].w};                  \
    const uint32_t w1_[4] = {vreg[1].x, vreg[1].y, vreg[1].z, vreg[1].w};                  \
    const uint32_t w2_[4] = {vreg[2].x, vreg[2].y, vreg[2].z, vreg[2].w};                  \
    const uint32_t w3_[4] = {vreg[3].x, vreg[3].y, vreg[3].z, vreg[3].w};                  \
    _Pragma("unroll") for (int e = 0; e < 8; ++e) {                                         \
      /* byte permute: the low (e even) or high (e odd) halves of two words */              \
      const uint32_t sel_ = (e & 1) ? 0x07060302u : 0x05040100u;                             \
      const uint32_t k01_ = __builtin_amdgcn_perm(w1_[e / 2], w0_[e / 2], sel_);             \
      const uint32_t k23_ = __builtin_amdgcn_perm(w3_[e / 2], w2_[e / 2], sel_);             \
      *reinterpret_cast<uint2*>(&vt_s[buf][(vd0 + e) * LDV + vr0]) = make_uint2(k01_, k23_); \
    }                                                                                       \
  }

  if (count > 0) {
    int kb0;
    bool f0;
    SFL_TILE_AT(0, kb0, f0)
    (void)f0;
    SFL_LOAD_TILE(kb0, ka)
    SFL_STORE_VT(0)
  }
  __syncthreads();
  // Tile `it` uses the K operands in KC and prefetches tile it+1 into KN; the
  // loop is unrolled twice so the two register sets swap roles without copies.
#define SFL_TILE_STEP(it, KC, KN)                                                           \
  {                                                                                         \
    int kb;                                                                                 \
    bool full;                                                                              \
    SFL_TILE_AT(it, kb, full)                                                               \
    full = full && a.s.use_full;                                                            \
    const int k0 = kb * BK;                                                                 \
    const int buf = (it) & 1;                                                               \
    const bool more = (it) + 1 < count;                                                     \
    if (more) {                                                                             \
      int kbn;                                                                              \
      bool fn;                                                                              \
      SFL_TILE_AT((it) + 1, kbn, fn)                                                        \
      (void)fn;                                                                             \
      SFL_LOAD_TILE(kbn, KN)                                                                \
    }                                                                                       \
    tile_math<T, QS, DT, KSTEPS, LDV>(a, KC, qreg, vt_s[buf], oacc, m_run, l_run, qw, col,  \
                                      grp, n, k0, full);                                    \
    if (more) SFL_STORE_VT(buf ^ 1)                                                         \
    __syncthreads();                                                                        \
  }
  for (int it = 0; it < count; it += 2) {
    SFL_TILE_STEP(it, ka, kb2)
    if (it + 1 >= count) break;
    SFL_TILE_STEP(it + 1, kb2, ka)
  }
#undef SFL_TILE_STEP
#undef SFL_LOAD_TILE
#undef SFL_TILE_AT
#undef SFL_STORE_VT

#pragma unroll
  for (int qs = 0; qs < QS; ++qs) {
    const int qrow = qw + 16 * qs + col;
    if (qrow >= n) continue;
    const float inv = l_run[qs] > 0.f ? 1.f / l_run[qs] : 0.f;
    uint16_t* op = static_cast<uint16_t*>(a.o) + b * a.os[0] + h * a.os[1] + long(qrow) * a.os[2];
#pragma unroll
    for (int t = 0; t < DT; ++t)
      *reinterpret_cast<uint2*>(op + 16 * t + 4 * grp) =
          make_uint2(pack2<T>(oacc[qs][t][0] * inv, oacc[qs][t][1] * inv),
                     pack2<T>(oacc[qs][t][2] * inv, oacc[qs][t][3] * inv));
    if (a.lse && grp == 0) {
      const float lse = l_run[qs] > 0.f ? (m_run[qs] + log2f(l_run[qs])) * 0.6931471805599453f : -INFINITY;
      a.lse[(long(b) * a.heads + h) * n + qrow] = lse;
    }
  }
}

// The keys one query may attend, without document labels, as two intervals:
// the window [lo, hi] (causality and the sequence end folded in) and the
// global prefix [0, phi]; allowed_flat() is "key in either". Returned relative
// to `base` for an unsigned range test per key offset c:
//   allowed(base + c) == (unsigned(c + r.a) <= unsigned(r.w)) | (c <= r.p).
struct KeyRanges { int a, w, p; };
__device__ __forceinline__ KeyRanges key_ranges(const MaskArgs& m, int q, int n, int base, bool all) {
  int lo = 0, hi = n - 1, phi = -1;
  if (!all) {
    if (m.left >= 0) lo = max(0, q - min(m.left, n));
    if (m.right >= 0) hi = min(hi, q + min(m.right, n));
    if (m.causal) hi = min(hi, q);
    phi = min(m.prefix, n) - 1;
    if (m.causal) phi = min(phi, q);
  }
  if (q >= n) { lo = 1; hi = 0; phi = -1; }
  KeyRanges r;
  if (hi < lo) { r.a = 1 << 30; r.w = 0; }  // empty window: no c + a fits in [0, 0]
  else { r.a = base - lo; r.w = hi - lo; }
  r.p = phi - base;
  return r;
}

// Head dim 64 on 32x32x16 MFMAs (twice the rate of 16x16x32 on gfx950). A
// workgroup of 2 waves owns a 64-query tile; a wave owns 32 queries, one per
// lane pair (lanes c and c + 32). S^T = K Q^T per 32-key block: lane
// (c, h = lane/32) ends with 16 scores of query q0 + 32*wave + c, keys
// 8*(j/4) + 4h + j%4 of the block, so the row max needs one exchange with
// the partner lane and the rescale factor is per lane. The head dim is split
// between the lane halves in both K and Q (h takes dims 32h .. 32h+31; a
// contraction is exact in any order both operands share), so a lane reads 64
// contiguous bytes of its key or query row. K tiles go global -> LDS by
// buffer loads that write LDS directly (no registers), rows stored with their
// 16-byte slots XOR-swizzled by (row >> 1) & 7 so that the 32 rows an operand
// read touches hit distinct banks (with row & 7 the 128-bit reads measured
// 2-way conflicts on gfx950); rows past the sequence read as zeros through the
// buffer range check. O^T = V^T P^T: for the 16-key
// step s the P^T operand of lane (c, h) is its own probabilities j = 8(s%2)
// .. +7 of block s/2 (keys 16s + 4h + {0..3} and 16s + 8 + 4h + {0..3}). V
// also goes global -> LDS directly, row-major (key rows, 32-byte units
// XOR-swizzled by the row), and each V^T operand is assembled by two LDS
// transpose reads (ds_read_b64_tr_b16): within each 16 lanes, lane 16g + i
// receives element i%4 of the 8-byte pieces addressed by lanes
// 16g + i/4 + 4k, k = 0..3, so lane 16g + m addresses key 16s + 4(g/2) + m/4
// (+8 for the second read) at dims 32t + 16(g%2) + 4(m%4), and lane l ends
// with dim 32t + l%32 of the 8 keys its P^T partner slots hold. The row sum comes from the packed
// probabilities with dot2 (the sum of exactly the values the P V product
// weights), kept per lane and added with the partner's at the end.
// Max / sum of a value over lanes l and l ^ 32 (the two halves of a 32x32
// MFMA column), exchanged with v_permlane32_swap instead of an LDS permute:
// the swap leaves {v[l], v[l ^ 32]} in the two results in some order, and max
// and + are symmetric.
__device__ __forceinline__ float pair_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Two 16-bit ones (bf16 or fp16 1.0) in one word.
template <typename T> __device__ __forceinline__ uint32_t ones_pair();
template <> __device__ __forceinline__ uint32_t ones_pair<bf16_t>() { return 0x3f803f80u; }
template <> __device__ __forceinline__ uint32_t ones_pair<f16_t>() { return 0x3c003c00u; }
// lo + hi of a packed pair, as add_pair(pk, 0.f) computes it, in the VOP3
// dot2 form with an inline zero addend (the compiler picks the accumulating
// VOP2 form and a register cleared by an extra move for every chain start).
template <typename T> __device__ __forceinline__ float first_pair(uint32_t pk, uint32_t ones);
template <> __device__ __forceinline__ float first_pair<bf16_t>(uint32_t pk, uint32_t ones) {
  float r;
  asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(r) : "v"(pk), "v"(ones));
  return r;
}
template <> __device__ __forceinline__ float first_pair<f16_t>(uint32_t pk, uint32_t ones) {
  float r;
  asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(pk), "v"(ones));
  return r;
}

// One key tile of masked_attention32_kernel for this wave: S^T = K Q^T from the
// swizzled K tile, the online softmax (with the token mask when `masked`), and
// O^T += V^T P^T. One code path for full and masked tiles, the mask a
// wave-uniform branch on the scores alone: with two instantiations of the
// whole tile the compiler kept the O accumulators of one in a second register
// set and copied them every tile (33 moves, and spills at D = 128).
template <typename T, int D>
__device__ __forceinline__ void attn32_tile(const AttnArgs& a, const uint4 (&kt)[BK][D / 8],
                                            const uint4 (&vt)[BK][D / 8], const u32x4 (&qreg)[D / 16],
                                            f32x16 (&oacc)[D / 32], float& m_run, float& l_run, float& m_lim,
                                            float& m_sub, int c, int h, int qrow, int k0, bool full,
                                            const unsigned (&vlane)[D / 32], bool masked) {
  const int n = a.n;
  f32x16 sacc[2];
  // S^T for key block kb2 (keys 32 kb2 .. +31 of the tile).
  auto scores = [&](int kb2) {
#pragma unroll
    for (int j = 0; j < 16; ++j) sacc[kb2][j] = 0.f;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const uint4 kr = kt[32 * kb2 + c][(D / 16 * h + ks) ^ k_swizzle<D>(c)];
      sacc[kb2] = mfma32<T>(u32x4{kr.x, kr.y, kr.z, kr.w}, qreg[ks], sacc[kb2]);
    }
  };
  // The scores are computed inside each branch (the masked one takes the
  // blocks in the other order, so the compiler cannot hoist them above the
  // branch): both branches then define the scores afresh, and the join needs
  // no copy of them (with the MFMAs shared ahead of the branch the full-tile
  // path copied all 32 scores every tile).
  if (!masked) {  // wave-uniform: full tiles skip the token mask
    scores(0);
    scores(1);
  } else {
    scores(1);
    scores(0);
    if (!a.m.docs) {
      const KeyRanges kr = key_ranges(a.m, qrow, n, k0 + 4 * h, full);
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int j = i % 16;
        const int cc = 32 * (i / 16) + 8 * (j / 4) + j % 4;
        const bool ok = (unsigned(cc + kr.a) <= unsigned(kr.w)) | (cc <= kr.p);
        sacc[i / 16][j] = ok ? sacc[i / 16][j] : -INFINITY;
      }
    } else {
      const int64_t dq = a.m.docs[min(qrow, n - 1)];
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int j = i % 16;
        const int key = k0 + 32 * (i / 16) + 8 * (j / 4) + 4 * h + j % 4;
        const int64_t dk = a.m.docs[min(key, n - 1)];
        const bool ok = full ? (key < n) & (qrow < n) : allowed_flat(a.m, qrow, key, n, dq, dk);
        sacc[i / 16][j] = ok ? sacc[i / 16][j] : -INFINITY;
      }
    }
  }
  // Row max: two interleaved chains of 3-input maxima over the lane's 32
  // scores, then the partner lane's.
  float ma = fmaxf(sacc[0][0], sacc[0][1]), mb = fmaxf(sacc[1][0], sacc[1][1]);
#pragma unroll
  for (int j = 2; j < 16; j += 2) {
    ma = fmaxf(fmaxf(ma, sacc[0][j]), sacc[0][j + 1]);
    mb = fmaxf(fmaxf(mb, sacc[1][j]), sacc[1][j + 1]);
  }
  float mx = fmaxf(ma, mb);
  mx = pair_max(mx);
  const float cs = a.scale_log2;
  // Lazy maximum: the subtracted maximum m_run moves only when the tile's
  // maximum exceeds it by more than kLazyMax (log2 units), so the probabilities
  // stay below 2^kLazyMax and the O rescale runs only on the rare tiles where
  // some query's maximum jumps. Any m_run that bounds the exponents gives the
  // same O / l; it only has to keep them from overflowing.
  // m_lim = m_run + kLazyMax and m_sub = the subtracted maximum (0 while
  // m_run is -inf) change only with m_run, so they are kept, not recomputed.
  const bool grow = mx * cs > m_lim;  // false for a fully masked row (mx = -inf)
  float alpha = 1.f;
  if (__ballot(grow)) {  // wave-uniform
    const float m_new = grow ? mx * cs : m_run;
    alpha = grow ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;  // 0 for the first admissible tile
    m_run = m_new;
    m_lim = m_run + kLazyMax;
    m_sub = m_run == -INFINITY ? 0.f : m_run;
    // In place (tied operands): the accumulators keep their registers on both
    // sides of this rare branch, so the common path needs no copies of them.
#pragma unroll
    for (int t = 0; t < D / 32; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(oacc[t][j]) : "v"(alpha));
  }
  const float ms = m_sub;
  u32x4 pop[4];
  float psum[4];  // one accumulator per key step: short dot2 chains
  const uint32_t ones2 = ones_pair<T>();
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2) {
    uint32_t pk[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i0 = 16 * (s2 / 2) + 8 * (s2 % 2) + 2 * e;
      pk[e] = pack2<T>(__builtin_amdgcn_exp2f(fmaf(sacc[i0 / 16][i0 % 16], cs, -ms)),
                       __builtin_amdgcn_exp2f(fmaf(sacc[i0 / 16][i0 % 16 + 1], cs, -ms)));
      // (at head dim 128 the VOP3 start measured 2-4% slower: compiler's form there)
      psum[s2] = e == 0 && D == 64 ? first_pair<T>(pk[e], ones2) : add_pair<T>(pk[e], e == 0 ? 0.f : psum[s2]);
    }
    pop[s2] = u32x4{pk[0], pk[1], pk[2], pk[3]};
  }
  l_run = l_run * alpha + ((psum[0] + psum[1]) + (psum[2] + psum[3]));
  // V^T operands: this lane's piece for step s2 (16 keys of 2D bytes), dim
  // tile t and key half (8 keys) is at byte vlane[t] + 32 D s2 + 16 D half
  // of the tile (vt_lane_offset).
  const unsigned vbase = unsigned(size_t((__attribute__((address_space(3))) const char*)(&vt[0][0])));
  // One address register per dim tile, opaque to the compiler, so the step
  // and half offsets go into the reads' offset fields (otherwise it forms
  // every address with its own VALU add).
  unsigned vaddr[D / 32];
#pragma unroll
  for (int t = 0; t < D / 32; ++t) {
    vaddr[t] = vbase + vlane[t];
    asm volatile("" : "+v"(vaddr[t]));
  }
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2) {
#pragma unroll
    for (int t = 0; t < D / 32; ++t) {
      const unsigned off = vaddr[t] + 32u * D * s2;
      const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(size_t)(off));
      const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(size_t)(off + 16u * D));
      const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
      oacc[t] = mfma32<T>(u32x4{l2.x, l2.y, h2.x, h2.y}, pop[s2], oacc[t]);
    }
  }
}

// The key tiles of one 64-query row of the schedule in increasing order: the
// CSR row (mode 1) or the interval row (global blocks [0, lowg), then window
// blocks [begin, end)). A row that starts past the sequence has none.
struct TileRow {
  const int32_t* col;  // CSR row (mode 1)
  const uint8_t* full;
  TileBounds tb;       // interval row (mode 0)
  int n, lowg, count, i, first, reg;
  bool csr, no_docs;
  __device__ __forceinline__ void init(const AttnArgs& a, int row) {
    n = a.n;
    const int q0 = row * BQ;
    const bool live = q0 < n;
    csr = a.s.mode == 1;
    no_docs = !a.m.docs;
    tb = tile_bounds(a.m, n, q0, min(q0 + BQ, n) - 1);
    lowg = min(tb.gend, tb.begin);
    int base = 0;
    if (!live) {
      count = 0;
    } else if (csr) {
      base = __builtin_amdgcn_readfirstlane(a.s.row_ptr[row]);
      count = __builtin_amdgcn_readfirstlane(a.s.row_ptr[row + 1]) - base;
    } else {
      count = lowg + max(0, max(tb.end, tb.gend) - tb.begin);
    }
    col = a.s.col_idx + base;
    full = a.s.full + base;
    i = 0;
    fill(0);
  }
  // Entries first .. first + 63 of the row into one VGPR (lane l: entry
  // first + l as 2 * key block + full), read from the CSR row or generated
  // from the interval bounds, so every tile's entry is then a readlane.
  __device__ __forceinline__ void fill(int f) {
    first = f;
    const int e = f + int(threadIdx.x % kWave);
    reg = 0;
    if (e < count) {
      if (csr) {
        reg = 2 * col[e] + int(full[e] != 0);
      } else {
        const int kb = e < lowg ? e : tb.begin + (e - lowg);
        reg = 2 * kb + int(no_docs && covered(tb, kb * BK, min(kb * BK + BK, n) - 1));
      }
    }
  }
  // The next tile's key block (INT_MAX when the row is done) and full flag.
  __device__ __forceinline__ int peek(bool& is_full) {
    if (i >= count) {
      is_full = false;
      return INT_MAX;
    }
    if ((i & ~63) != first) fill(i & ~63);
    const int e = __builtin_amdgcn_readlane(reg, i & 63);
    is_full = (e & 1) != 0;
    return e >> 1;
  }
};

// One key tile of a 128-query workgroup: its block and, for each 64-query
// half, whether the half's row lists it and whether it is fully admissible.
struct MergedTile {
  int kb;
  bool in[2], full[2];
};
__device__ __forceinline__ MergedTile next_tile(const AttnArgs&, TileRow (&rows)[1]) {
  MergedTile t;
  t.kb = rows[0].peek(t.full[0]);
  t.in[0] = t.kb != INT_MAX;
  t.in[1] = false;
  t.full[1] = false;
  rows[0].i += t.in[0];
  return t;
}
__device__ __forceinline__ MergedTile next_tile(const AttnArgs& a, TileRow (&rows)[2]) {
  MergedTile t;
  const int c0 = rows[0].peek(t.full[0]);
  const int c1 = rows[1].peek(t.full[1]);
  t.kb = min(c0, c1);
  t.in[0] = c0 == t.kb && c0 != INT_MAX;
  t.in[1] = c1 == t.kb && c1 != INT_MAX;
  rows[0].i += t.in[0];
  rows[1].i += t.in[1];
  return t;
}

constexpr int kA32Waves = 4;

// 4 waves, 128 queries (two 64-query rows of the schedule) per workgroup: the
// waves share each K/V tile in LDS, so a tile's global -> LDS traffic serves
// 128 queries, and the 32 KB of double-buffered tiles per 4 waves leaves the
// register file, not LDS, to bound the waves per CU. The workgroup walks the
// merge of its two rows' tile lists; a wave skips (but still synchronises on)
// a tile its own row does not list, so each row processes exactly its own
// tiles, as the 64-query tiling would.
// Head dim 64: 32 KB of LDS per workgroup, 168 VGPRs, 3 waves per SIMD. Head
// dim 128: the same layout with 256-byte rows (64 KB, two workgroups per CU,
// 2 waves per SIMD), 8 k-steps per score block and 4 dim tiles of O.
template <int D> constexpr int attn32_waves_per_eu() { return D == 64 ? 3 : 2; }

template <typename T, int D, int NW>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(attn32_waves_per_eu<D>())))
void masked_attention32_kernel(AttnArgs a) {
  static_assert(NW == 2 || NW == 4, "one or two 64-query rows per workgroup");
  constexpr int NR = NW / 2;     // 64-query schedule rows per workgroup
  constexpr int QB = NR * BQ;
  constexpr int SL = D / 8;      // 16-byte slots per K/V row
  constexpr int RPL = 64 / SL;   // rows one 1 KB load moves
  __shared__ __align__(16) uint4 k_s[2][BK][SL];  // [key][16-byte slot s at s ^ k_swizzle<D>(key)]
  __shared__ __align__(16) uint4 v_s[2][BK][SL];  // [key][16-byte slot, see vt_slot]
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid % kWave;
  const int half = wave / 2;
  const int c = lane % 32, h = lane / 32;
  const int n = a.n;
  // Tile indices, schedule entries and key offsets are wave-uniform; keeping
  // them in scalar registers keeps their loads off the vector memory counter,
  // which would otherwise make the math wait for the next tile's prefetch.
  const int2 tile = attn_tile((a.n + QB - 1) / QB, a.batch * a.heads);
  const int qt = __builtin_amdgcn_readfirstlane(tile.x);
  const int bh = __builtin_amdgcn_readfirstlane(tile.y);
  const int b = bh / a.heads, hd = bh % a.heads;
  const int q0 = qt * QB;
  const int qrow = q0 + 32 * wave + c;  // this lane's query

  const uint16_t* qp = static_cast<const uint16_t*>(a.q) + b * a.qs[0] + hd * a.qs[1];
  const uint16_t* kp = static_cast<const uint16_t*>(a.k) + b * a.ks[0] + hd * a.ks[1];
  const uint16_t* vp = static_cast<const uint16_t*>(a.v) + b * a.vs[0] + hd * a.vs[1];

  // Q^T operand of k-step ks: Q[qrow][(D/2) h + 8ks .. +8].
  u32x4 qreg[D / 16];
  {
    const uint16_t* qr = qp + long(min(qrow, n - 1)) * a.qs[2] + (D / 2) * h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const uint4 r = load16(qr + 8 * ks);
      qreg[ks] = u32x4{r.x, r.y, r.z, r.w};
    }
  }

  float m_run = -INFINITY, l_run = 0.f;
  float m_lim = -INFINITY, m_sub = 0.f;  // m_run + kLazyMax and the subtracted maximum (attn32_tile)
  f32x16 oacc[D / 32];
#pragma unroll
  for (int t = 0; t < D / 32; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) oacc[t][j] = 0.f;

  TileRow rows[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) rows[r].init(a, NR * qt + r);

  // K tile: BK / RPL loads of RPL rows (1 KB) per tile, shared by the waves;
  // lane i moves row r = RPL ch + i/SL, logical slot (i%SL) ^ k_swizzle(r)
  // into physical slot i%SL (the swizzle under which the 128-bit operand
  // reads are free of LDS bank conflicts; measured). ch is kA32Waves cw +
  // wave, and k_swizzle only sees the low bits of r, so one byte offset per
  // lane serves every load of this wave. The buffer covers this head's rows
  // [0, n): rows past n read as zeros.
  const unsigned krow_bytes = unsigned(a.ks[2]) * 2u;
  const i32x4_t krsrc = buffer_rsrc(kp, unsigned((long(n - 1) * a.ks[2] + D) * 2));
  const int lrr = lane / SL, lpp = lane % SL;
  // k_swizzle sees only the low bits of the row: those of ch & 3 (D 128) or
  // ch & 1 (D 64), so per wave ch = NW cw + wave takes two offsets, by cw & 1
  // (one when NW = 4).
  unsigned kvoff[NW == 4 ? 1 : 2];
#pragma unroll
  for (int par = 0; par < (NW == 4 ? 1 : 2); ++par)
    kvoff[par] = unsigned(lrr) * krow_bytes + 16u * unsigned(lpp ^ k_swizzle<D>(RPL * (par * NW + wave) + lrr));
  // V tile: the same loads; lane i moves row RPL ch + i/SL, logical slot sg
  // with vt_slot(sg, row) == i%SL, into physical slot i%SL (row & 3 == (i/SL) & 3).
  const unsigned vrow_bytes = unsigned(a.vs[2]) * 2u;
  const i32x4_t vrsrc = buffer_rsrc(vp, unsigned((long(n - 1) * a.vs[2] + D) * 2));
  const unsigned vvoff = unsigned(lrr) * vrow_bytes +
                         16u * (2u * ((unsigned(lpp) >> 1) ^ (unsigned(lrr) & 3u)) + (unsigned(lpp) & 1u));
  unsigned vlane[D / 32];
#pragma unroll
  for (int t = 0; t < D / 32; ++t) vlane[t] = vt_lane_offset<D>(lane, t);
#define SFL_A32_LOAD(kb, kbuf)                                                              \
  {                                                                                         \
    const int k0_ = (kb) * BK;                                                              \
    _Pragma("unroll") for (int cw = 0; cw < BK / RPL / NW; ++cw) {                          \
      const int ch_ = cw * NW + wave;                                                       \
      lds_load16(krsrc, lds_offset(&k_s[kbuf][RPL * ch_][0]), kvoff[NW == 4 ? 0 : cw & 1],  \
                 unsigned(k0_ + RPL * ch_) * krow_bytes);                                   \
      lds_load16(vrsrc, lds_offset(&v_s[kbuf][RPL * ch_][0]), vvoff,                        \
                 unsigned(k0_ + RPL * ch_) * vrow_bytes);                                   \
    }                                                                                       \
  }
  // One key tile: S^T, masked online softmax, O^T += V^T P^T.
  MergedTile cur = next_tile(a, rows);
  if (cur.kb != INT_MAX) SFL_A32_LOAD(cur.kb, 0)
  __builtin_amdgcn_s_waitcnt(sfl_vmcnt(0));
  __syncthreads();
  for (int buf = 0; cur.kb != INT_MAX; buf ^= 1) {
    const MergedTile nxt = next_tile(a, rows);
    if (nxt.kb != INT_MAX) SFL_A32_LOAD(nxt.kb, buf ^ 1)
    const int k0 = cur.kb * BK;
    const bool full = (NR == 2 && half ? cur.full[1] : cur.full[0]) && a.s.use_full;
    if (NR == 2 && half ? cur.in[1] : cur.in[0]) {
      attn32_tile<T, D>(a, k_s[buf], v_s[buf], qreg, oacc, m_run, l_run, m_lim, m_sub, c, h, qrow, k0, full, vlane,
                        !(full && k0 + BK <= n));
    }
    __builtin_amdgcn_s_waitcnt(sfl_vmcnt(0));  // the next K and V tiles have landed
    __syncthreads();
    cur = nxt;
  }
#undef SFL_A32_LOAD

  const float l_tot = pair_sum(l_run);
  if (qrow >= n) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  uint16_t* op = static_cast<uint16_t*>(a.o) + b * a.os[0] + hd * a.os[1] + long(qrow) * a.os[2];
#pragma unroll
  for (int t = 0; t < D / 32; ++t)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq)
      *reinterpret_cast<uint2*>(op + 32 * t + 8 * jq + 4 * h) =
          make_uint2(pack2<T>(oacc[t][4 * jq] * inv, oacc[t][4 * jq + 1] * inv),
                     pack2<T>(oacc[t][4 * jq + 2] * inv, oacc[t][4 * jq + 3] * inv));
  if (a.lse && h == 0) {
    const float lse = l_tot > 0.f ? (m_run + log2f(l_tot)) * 0.6931471805599453f : -INFINITY;
    a.lse[(long(b) * a.heads + hd) * n + qrow] = lse;
  }
}

// The kernel a launch runs, chosen from the head dim and the K/V row strides
// (the 32x32 kernel addresses K and V with 32-bit buffer offsets), with its
// grid and workgroup size; shared by the launch and sfl_masked_attention_kernel_info.
struct MaskedLaunch {
  const void* fn;
  const char* name;
  unsigned queries_per_workgroup;
  unsigned threads;
};

// Keys one 64-query row of the mask can see: its window (left + right + one
// tile, clipped to the sequence) plus the global prefix.
inline long row_keys(const MaskArgs& m, long n) {
  const long left = m.left >= 0 ? std::min<long>(m.left, n) : n;
  const long right = m.causal ? 0 : (m.right >= 0 ? std::min<long>(m.right, n) : n);
  return std::min<long>(n, left + right + BQ) + std::min<long>(m.prefix, n);
}
// Rows of at most this many keys (about 8 tiles) run one row per workgroup
// (2 waves, head dim 64): with so few tiles per row the per-tile barrier of 4 waves and
// the two rows' merged tile list cost more than sharing each K/V tile saves.
#ifndef SFL_A32_SHORT_KEYS
#define SFL_A32_SHORT_KEYS 512
#endif
constexpr long kShortRowKeys = SFL_A32_SHORT_KEYS;

template <typename T>
MaskedLaunch select_masked(int dim, long n, long k_row_stride, long v_row_stride, const MaskArgs& m) {
  const bool offsets32 = n * k_row_stride * 2 < (1L << 31) && n * v_row_stride * 2 < (1L << 31);
  const bool one_row = row_keys(m, n) <= kShortRowKeys;
  switch (dim) {
    case 32:
      return {reinterpret_cast<const void*>(&masked_attention_kernel<T, 32>), "masked_attention_kernel<D=32>",
              unsigned(BQ), unsigned(kThreads)};
    case 64:
      if (offsets32 && one_row)
        return {reinterpret_cast<const void*>(&masked_attention32_kernel<T, 64, 2>),
                "masked_attention32_kernel<D=64, 2 waves>", unsigned(BQ), unsigned(2 * kWave)};
      if (offsets32)
        return {reinterpret_cast<const void*>(&masked_attention32_kernel<T, 64, kA32Waves>),
                "masked_attention32_kernel<D=64>", unsigned(2 * BQ), unsigned(kA32Waves * kWave)};
      return {reinterpret_cast<const void*>(&masked_attention_pair_kernel<T>), "masked_attention_pair_kernel<D=64>",
              unsigned(BQ), unsigned(kPairWaves * kWave)};
    case 128:  // (one row per workgroup at D = 128 needs 300 VGPRs: one wave per SIMD)
      if (offsets32)
        return {reinterpret_cast<const void*>(&masked_attention32_kernel<T, 128, kA32Waves>),
                "masked_attention32_kernel<D=128>", unsigned(2 * BQ), unsigned(kA32Waves * kWave)};
      return {reinterpret_cast<const void*>(&masked_attention_kernel<T, 128>), "masked_attention_kernel<D=128>",
              unsigned(BQ), unsigned(kThreads)};
    default: return {nullptr, nullptr, 0u, 0u};
  }
}

template <typename T>
int launch_masked(AttnArgs a, int batch, int dim, hipStream_t stream) {
  const MaskedLaunch l = select_masked<T>(dim, a.n, a.ks[2], a.vs[2], a.m);
  if (!l.fn) return set_error(SFL_ERR_UNSUPPORTED, "masked_attention: head dim must be 32, 64 or 128");
  const dim3 grid(unsigned((a.n + l.queries_per_workgroup - 1) / l.queries_per_workgroup) *
                  unsigned(batch * a.heads));
  void* args[] = {&a};
  const hipError_t err = hipLaunchKernel(l.fn, grid, dim3(l.threads), args, 0, stream);
  if (err != hipSuccess) {
    (void)hipGetLastError();  // clear the launch error
    return set_error(SFL_ERR_HIP, "masked_attention: launch of %s failed: %s", l.name, hipGetErrorString(err));
  }
  return SFL_OK;
}

}  // namespace
}  // namespace sfl

using namespace sfl;

extern "C" int sfl_masked_attention(const void* q, const void* k, const void* v, void* o, float* lse,
                                    int batch, int heads, int n, int head_dim,
                                    const long* q_strides, const long* k_strides,
                                    const long* v_strides, const long* o_strides, float scale,
                                    int causal, int window_left, int window_right, int global_prefix,
                                    const int64_t* document_ids, int schedule_mode,
                                    const int32_t* row_ptr, const int32_t* col_idx,
                                    const uint8_t* full_blocks, int use_full_blocks, int dtype,
                                    void* stream) {
  const char* what = "masked_attention";
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides)
    return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (batch < 1 || heads < 1 || n < 1) return set_error(SFL_ERR_INVALID, "%s: sizes must be positive", what);
  if (!(scale > 0.f) || !__builtin_isfinite(scale)) return set_error(SFL_ERR_INVALID, "%s: scale must be finite and positive", what);
  if (schedule_mode != 0 && schedule_mode != 1) return set_error(SFL_ERR_INVALID, "%s: schedule_mode must be 0 (interval) or 1 (csr)", what);
  if (schedule_mode == 1 && (!row_ptr || !col_idx || !full_blocks))
    return set_error(SFL_ERR_INVALID, "%s: csr schedule arrays are required", what);
  if (schedule_mode == 0 && document_ids)
    return set_error(SFL_ERR_INVALID, "%s: interval schedules do not support document constraints", what);
  if (global_prefix < 0) return set_error(SFL_ERR_INVALID, "%s: global_prefix must be >= 0", what);
  for (int i = 0; i < 3; ++i) {
    if (q_strides[i] < 0 || k_strides[i] < 0 || v_strides[i] < 0 || o_strides[i] < 0)
      return set_error(SFL_ERR_INVALID, "%s: strides must be non-negative", what);
  }
  if (q_strides[2] % 8 || k_strides[2] % 8 || v_strides[2] % 8 || o_strides[2] % 4)
    return set_error(SFL_ERR_INVALID, "%s: row strides must keep 16-byte alignment", what);
  AttnArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o; a.lse = lse;
  for (int i = 0; i < 3; ++i) {
    a.qs[i] = q_strides[i]; a.ks[i] = k_strides[i]; a.vs[i] = v_strides[i]; a.os[i] = o_strides[i];
  }
  a.batch = batch; a.heads = heads; a.n = n; a.scale_log2 = scale * kLog2e;
  if (long((n + BQ - 1) / BQ) * batch * heads > (1L << 31) - 1)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: too many query tiles", what);
  a.m = MaskArgs{causal, window_left, window_right, global_prefix, document_ids};
  a.s = Sched{schedule_mode, use_full_blocks, row_ptr, col_idx, full_blocks};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == SFL_DTYPE_BF16) return launch_masked<bf16_t>(a, batch, head_dim, s);
  if (dtype == SFL_DTYPE_F16) return launch_masked<f16_t>(a, batch, head_dim, s);
  return set_error(SFL_ERR_UNSUPPORTED, "%s: dtype must be BF16 or F16", what);
}

extern "C" int sfl_masked_attention_block(void) { return BQ; }

extern "C" int sfl_masked_attention_kernel_info(int head_dim, int dtype, int n, long k_row_stride,
                                                long v_row_stride, int causal, int window_left,
                                                int window_right, int global_prefix, sfl_kernel_info* info) {
  const char* what = "masked_attention_kernel_info";
  if (!info) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (n < 1 || k_row_stride < 0 || v_row_stride < 0 || global_prefix < 0)
    return set_error(SFL_ERR_INVALID, "%s: bad sizes", what);
  const MaskArgs m{causal, window_left, window_right, global_prefix, nullptr};
  MaskedLaunch l{};
  if (dtype == SFL_DTYPE_BF16) l = select_masked<bf16_t>(head_dim, n, k_row_stride, v_row_stride, m);
  else if (dtype == SFL_DTYPE_F16) l = select_masked<f16_t>(head_dim, n, k_row_stride, v_row_stride, m);
  else return set_error(SFL_ERR_UNSUPPORTED, "%s: dtype must be BF16 or F16", what);
  if (!l.fn) return set_error(SFL_ERR_UNSUPPORTED, "%s: head dim must be 32, 64 or 128", what);
  hipFuncAttributes attr{};
  const hipError_t err = hipFuncGetAttributes(&attr, l.fn);
  if (err != hipSuccess) return set_error(SFL_ERR_HIP, "%s: hipFuncGetAttributes: %s", what, hipGetErrorString(err));
  snprintf(info->name, sizeof(info->name), "%s%s", l.name, dtype == SFL_DTYPE_BF16 ? " bf16" : " f16");
  info->registers = attr.numRegs;
  info->private_bytes = int(attr.localSizeBytes);
  info->shared_bytes = int(attr.sharedSizeBytes);
  info->max_threads = attr.maxThreadsPerBlock;
  info->threads = int(l.threads);
  info->queries_per_workgroup = int(l.queries_per_workgroup);
  return SFL_OK;
}
