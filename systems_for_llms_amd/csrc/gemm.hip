// Prefill projections as 16-bit MFMA GEMMs with fused epilogues, plus the
// row-wise prefill helpers (embedding gather, RMSNorm).
//
// Every GEMM computes C^T[n][m] = sum_k W[n][k] * A[m][k] for A [M, K]
// activations (one row per token) and W [N, K] weights, both K-contiguous as
// the reference's Linear stores them (src/llmlab/model/layers.py:34-35), in
// the model's 16-bit type T (bf16 or fp16; the kernels are templates on T,
// whose 16-bit outputs are stored in T too).
// Features are the MFMA rows, so each lane ends with 4 consecutive features
// of one token: RoPE pairs and SwiGLU pairs are in-lane or one shuffle away
// and stores are 8/16-byte vectors.
//
// Tiling: a workgroup of 4 waves computes a 128-feature x 128-token tile;
// wave (wn, wm) owns 64 x 64 = 4 x 4 MFMA tiles of 16x16x32. K advances in
// steps of 64 through double-buffered LDS tiles (rows padded by 8 elements);
// the next step's global loads are in registers while the current step runs.
// Epilogues:
//   PLAIN     C[m][n] stored as fp32 or bf16 (optionally accumulated into fp32).
//   QKV       RoPE on q and k (attention.py:44-58) from the host fp32 table at
//             position m % T, q to [B, H, T, dk] bf16, k/v to the KV cache.
//   SWIGLU    W is W1/W3 interleaved in blocks of 8 rows; h = silu(a) * c
//             (layers.py:114-115) as bf16 [M, d_ff].
#include "attn_mfma.hpp"
#include "gemm_f32.hpp"
#include "lds_dma.hpp"

namespace sfl {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int TN = 128, TM = 128, TK = 64;
constexpr int LDT = TK + 8;      // LDS row stride (elements)
constexpr int kThreads = 256;

enum GemmEpi { G_PLAIN = 0, G_QKV = 1, G_SWIGLU = 2 };

struct GemmArgs {
  const uint16_t* a;   // [M, K]
  const uint16_t* w;   // [N, K]
  int m, n, k;
  // PLAIN
  void* c;             // [M, N] (ldc = N)
  int c_f32, accumulate;
  // QKV
  const float* cos_t;
  const float* sin_t;
  int seq, heads, head_dim, d_model, cap;
  uint16_t* q_out;     // [B, H, T, dk]
  uint16_t* k_cache;   // [B, H, cap, dk]
  uint16_t* v_cache;
  // SWIGLU
  uint16_t* h_out;     // [M, N/2]
  // PLAIN residual (fp32 C += A W^T) that also prepares the next RMSNorm
  // (norm_gain null: not): norm_act = bf16(C * gain), and per token and
  // 128-feature part the sum of C^2 in norm_ss [ceil(N / 128)][M].
  const uint16_t* norm_gain;
  uint16_t* norm_act;
  float* norm_ss;
  // QKV / SWIGLU fed by such an input: the products are scaled by
  // row_scale[m] = 1 / rms of token m (null: not).
  const float* row_scale;
  // Every bf16 output base is 16-byte aligned: the 32x32 kernel then stores
  // 8 consecutive outputs per lane (lane pairs exchange halves first).
  int vec16;
};

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

// One value rounded to T (round to nearest even), as raw bits.
template <typename T> __device__ __forceinline__ uint16_t bits16(float v);
template <> __device__ __forceinline__ uint16_t bits16<bf16_t>(float v) { return f32_to_bf16_bits(v); }
template <> __device__ __forceinline__ uint16_t bits16<f16_t>(float v) { return f32_to_f16_bits(v); }

// The low and high T values of a packed pair, as fp32.
template <typename T> __device__ __forceinline__ float lo16(uint32_t w);
template <typename T> __device__ __forceinline__ float hi16(uint32_t w);
template <> __device__ __forceinline__ float lo16<bf16_t>(uint32_t w) { return bf16_lo(w); }
template <> __device__ __forceinline__ float hi16<bf16_t>(uint32_t w) { return bf16_hi(w); }
template <> __device__ __forceinline__ float lo16<f16_t>(uint32_t w) { return f16_bits_to_f32(uint16_t(w & 0xffffu)); }
template <> __device__ __forceinline__ float hi16<f16_t>(uint32_t w) { return f16_bits_to_f32(uint16_t(w >> 16)); }

// v, or zeros when !keep. Selected per component: a select of whole uint4
// structs is lowered through scratch memory.
__device__ __forceinline__ uint4 keep16(const uint4& v, bool keep) {
  return make_uint4(keep ? v.x : 0u, keep ? v.y : 0u, keep ? v.z : 0u, keep ? v.w : 0u);
}


// Where a lane's 4 QKV features and its token go: section (0 q, 1 k, 2 v),
// head, dim of the first feature; batch row and position of the token.
// Computed once per feature tile / token tile by the caller (integer
// divisions by runtime sizes are long instruction sequences).
struct QkvFeat { int section, head, dim; };
struct QkvTok { int b, t; };

__device__ __forceinline__ QkvFeat qkv_feat(const GemmArgs& g, int n) {
  const int section = n / g.d_model;
  const int f = n - section * g.d_model;
  const int head = f / g.head_dim;
  return QkvFeat{section, head, f - head * g.head_dim};
}
// qkv_feat of feature nt + off from base = qkv_feat(nt), 0 <= off < 32: the
// head changes at most twice within 32 features (head dims >= 16), so two
// compare-and-wrap steps replace the two integer divisions.
__device__ __forceinline__ QkvFeat qkv_feat_at(const GemmArgs& g, const QkvFeat& base, int off) {
  QkvFeat f{base.section, base.head, base.dim + off};
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    if (f.dim >= g.head_dim) {
      f.dim -= g.head_dim;
      if (++f.head == g.heads) {
        f.head = 0;
        ++f.section;
      }
    }
  }
  return f;
}
__device__ __forceinline__ QkvTok qkv_tok(const GemmArgs& g, int m) {
  const int b = m / g.seq;
  return QkvTok{b, m - b * g.seq};
}

// RoPE (attention.py:44-58) of 4 consecutive q or k features (dims dim ..
// dim+3 of one head: two rotation pairs) of token qt; v features pass through.
__device__ __forceinline__ void rope4(const GemmArgs& g, float (&y)[4], const QkvFeat& qf, const QkvTok& qt) {
  if (qf.section >= 2) return;
  // Feature-major tables [head_dim / 2][cap]: the 32 lanes of a group hold 32
  // consecutive tokens, so each load reads consecutive floats (row-major
  // tables put the 32 tokens on 32 cache lines: 345 -> 330 us on the 324M
  // q/k/v shape, same values).
  const long r0 = long(qf.dim / 2) * g.cap + qt.t;
  const float2 c = make_float2(g.cos_t[r0], g.cos_t[r0 + g.cap]);
  const float2 s = make_float2(g.sin_t[r0], g.sin_t[r0 + g.cap]);
  const float e0 = y[0], o0 = y[1], e1 = y[2], o1 = y[3];
  y[0] = e0 * c.x - o0 * s.x;
  y[1] = e0 * s.x + o0 * c.x;
  y[2] = e1 * c.y - o1 * s.y;
  y[3] = e1 * s.y + o1 * c.y;
}

// Destination of feature qf of token qt: q [B, H, T, dk] or the k / v cache [B, H, cap, dk].
__device__ __forceinline__ uint16_t* qkv_dst(const GemmArgs& g, const QkvFeat& qf, const QkvTok& qt) {
  if (qf.section == 0) return g.q_out + ((long(qt.b) * g.heads + qf.head) * g.seq + qt.t) * g.head_dim + qf.dim;
  uint16_t* cache = qf.section == 1 ? g.k_cache : g.v_cache;
  return cache + ((long(qt.b) * g.heads + qf.head) * g.cap + qt.t) * g.head_dim + qf.dim;
}

// silu(a) * c = a * c / (1 + e^-a) with the hardware base-2 exponential and
// reciprocal (e^-a = 2^(-a log2 e); each ~1 ulp): the bf16 rounding of the
// result dominates their error. a -> -inf gives 2^+inf = inf and a zero
// reciprocal (a signed zero), as the exact form does.
__device__ __forceinline__ float silu_mul(float a, float c) {
  const float e = __builtin_amdgcn_exp2f(a * -1.4426950408889634f);
  return a * c * __builtin_amdgcn_rcpf(1.f + e);
}

// Two packed groups of 4 bf16 outputs, A (lane-local features f .. f+3) and
// B (f+8 .. f+11), where lane l ^ 32 holds f+4 .. f+7 and f+12 .. f+15: one
// v_permlane32_swap per dword gives lanes 0..31 features f .. f+7 (own A,
// partner's A) and lanes 32..63 features f+8 .. f+15 (partner's B, own B),
// one 16-byte store each instead of two 8-byte stores.
__device__ __forceinline__ uint4 pair8(const uint32_t (&a)[2], const uint32_t (&b)[2]) {
  const auto s0 = __builtin_amdgcn_permlane32_swap(a[0], b[0], false, false);
  const auto s1 = __builtin_amdgcn_permlane32_swap(a[1], b[1], false, false);
  return make_uint4(s0[0], s1[0], s0[1], s1[1]);
}

// Epilogue of one 16x16 MFMA tile: v holds features nt + 4*grp + (0..3) of
// token m. Every lane must call it (the SwiGLU pairing shuffles).
template <typename T, int E>
__device__ __forceinline__ void store_tile(const GemmArgs& g, const f32x4& v, int nt, int grp, int m,
                                           QkvFeat qf = QkvFeat{}, QkvTok qt = QkvTok{}) {
  const int n = nt + 4 * grp;
  float y[4] = {v[0], v[1], v[2], v[3]};
  if constexpr (E == G_SWIGLU) {
    // Rows 0..7 of the 16-row tile are W1 features, rows 8..15 the
    // matching W3 features: lane groups 0,1 pair with groups 2,3.
    float c3[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) c3[e] = lane_xor(y[e], 32);
    if (grp >= 2 || m >= g.m) return;
    const int f = nt / 2 + 4 * grp;  // hidden feature index
    if (f >= g.n / 2) return;
    float h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = silu_mul(y[e], c3[e]);
    *reinterpret_cast<uint2*>(g.h_out + long(m) * (g.n / 2) + f) = make_uint2(pack2<T>(h[0], h[1]), pack2<T>(h[2], h[3]));
  } else {
    if (m >= g.m || n >= g.n) return;
    if constexpr (E == G_PLAIN) {
      if (g.c_f32) {
        float* c = static_cast<float*>(g.c) + long(m) * g.n + n;
        if (n + 3 < g.n && (g.n & 3) == 0) {
          float4 old = g.accumulate ? *reinterpret_cast<const float4*>(c) : make_float4(0.f, 0.f, 0.f, 0.f);
          *reinterpret_cast<float4*>(c) = make_float4(old.x + y[0], old.y + y[1], old.z + y[2], old.w + y[3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < g.n) c[e] = (g.accumulate ? c[e] : 0.f) + y[e];
        }
      } else {
        uint16_t* c = static_cast<uint16_t*>(g.c) + long(m) * g.n + n;
        if (n + 3 < g.n && (g.n & 3) == 0) {
          *reinterpret_cast<uint2*>(c) = make_uint2(pack2<T>(y[0], y[1]), pack2<T>(y[2], y[3]));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < g.n) c[e] = bits16<T>(y[e]);
        }
      }
    } else {  // G_QKV
      rope4(g, y, qf, qt);
      *reinterpret_cast<uint2*>(qkv_dst(g, qf, qt)) = make_uint2(pack2<T>(y[0], y[1]), pack2<T>(y[2], y[3]));
    }
  }
}

template <typename T, int E>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmArgs g) {
  __shared__ __align__(16) uint16_t ws[2][TN * LDT];
  __shared__ __align__(16) uint16_t as[2][TM * LDT];
  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int wn = wave / 2, wm = wave % 2;
  const int col = lane % 16, grp = lane / 16;
  const int n0 = blockIdx.x * TN;
  const int m0 = blockIdx.y * TM;
  const int ksteps = (g.k + TK - 1) / TK;

  // Each thread moves 4 x 16 bytes of W and of A per K step: row r, 8-element
  // group cg. Loads are unconditional from clamped addresses; the K tail is
  // zeroed when the registers go to LDS, so no load waits inside its guard.
  uint4 wr[4], ar[4];
  bool kin[4];
#define SFL_GEMM_GLOAD(kt)                                                   \
  _Pragma("unroll") for (int i = 0; i < 4; ++i) {                            \
    const int idx = tid + i * kThreads;                                      \
    const int r = idx / (TK / 8), cg = idx % (TK / 8);                       \
    const int kk = (kt) * TK + cg * 8;                                       \
    kin[i] = kk < g.k;                                                       \
    const int kc = kin[i] ? kk : 0;                                          \
    wr[i] = load16(g.w + long(min(n0 + r, g.n - 1)) * g.k + kc);             \
    ar[i] = load16(g.a + long(min(m0 + r, g.m - 1)) * g.k + kc);             \
  }
#define SFL_GEMM_SSTORE(buf)                                                 \
  _Pragma("unroll") for (int i = 0; i < 4; ++i) {                            \
    const int idx = tid + i * kThreads;                                      \
    const int r = idx / (TK / 8), cg = idx % (TK / 8);                       \
    *reinterpret_cast<uint4*>(&ws[buf][r * LDT + cg * 8]) = keep16(wr[i], kin[i]); \
    *reinterpret_cast<uint4*>(&as[buf][r * LDT + cg * 8]) = keep16(ar[i], kin[i]); \
  }

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  SFL_GEMM_GLOAD(0)
  SFL_GEMM_SSTORE(0)
  __syncthreads();
  for (int kt = 0; kt < ksteps; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ksteps) { SFL_GEMM_GLOAD(kt + 1) }
#pragma unroll
    for (int ks = 0; ks < TK / 32; ++ks) {
      u32x4 af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const u32x4*>(&ws[buf][(wn * 64 + i * 16 + col) * LDT + ks * 32 + grp * 8]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bfr[j] = *reinterpret_cast<const u32x4*>(&as[buf][(wm * 64 + j * 16 + col) * LDT + ks * 32 + grp * 8]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<T>(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < ksteps) {
      SFL_GEMM_SSTORE(buf ^ 1)
      __syncthreads();
    }
  }
#undef SFL_GEMM_GLOAD
#undef SFL_GEMM_SSTORE

  // Epilogue: acc[i][j] holds features n0 + wn*64 + 16i + 4grp + (0..3) of token m0 + wm*64 + 16j + col.
  QkvTok tok[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) tok[j] = E == G_QKV ? qkv_tok(g, m0 + wm * 64 + j * 16 + col) : QkvTok{};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const QkvFeat feat = E == G_QKV ? qkv_feat(g, n0 + wn * 64 + i * 16 + 4 * grp) : QkvFeat{};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      store_tile<T, E>(g, acc[i][j], n0 + wn * 64 + i * 16, grp, m0 + wm * 64 + j * 16 + col, feat, tok[j]);
  }
}

// GEMM for K % 64 == 0 on v_mfma_f32_32x32x16_{bf16,f16} (on gfx950 the 32x32
// form sustains about twice the bf16 rate of the 16x16x32 form used above).
// A workgroup of 4 waves (2 x 2) computes 128 features x 128 tokens; wave
// (wn, wm) owns 2 x 2 MFMA tiles of 32x32. Operands reach LDS through buffer
// loads with an LDS destination (no register staging). A K step stores each
// operand tile row-major, 128 bytes (64 k values) per row in 8 slots of 16
// bytes, slot = (16-byte column) ^ ((row >> 1) & 7): a load instruction moves
// 8 whole rows (1 KB, full cache lines, the lanes of a row in swizzled order)
// and every MFMA operand read -- 32 rows x 2 columns per instruction -- is
// free of bank conflicts. Rows past the matrix read as zeros through the
// buffer range check. K advances by 64 through two LDS stages, the loads of
// the next step in flight while a step computes.
constexpr int K2 = 64;     // K step
constexpr int TB = 128;    // features and tokens per workgroup


template <int TN_, int TM_, int SL_>
struct Stage32 {
  uint4 w[TN_][SL_];  // [row][swizzled 16-byte slot]
  uint4 a[TM_][SL_];
};

// Physical 16-byte slot offset of row r in a stage of SL slots per row: the
// XOR under which the MFMA operand reads (16 consecutive lanes reading rows r
// .. r+15 at one logical slot, 256 bytes per LDS cycle) touch every bank
// once. Rows of 128 bytes already alternate bank halves, rows of 64 bytes
// cycle through bank quarters, so the swizzle only has to separate rows that
// share a half / quarter.
template <int SL>
__device__ __forceinline__ int stage_swizzle(int r) {
  return SL == 8 ? (r >> 1) & 7 : (r >> 2) & 3;
}

// Tile of workgroup b in a 1-D grid of tn x tm tiles, XCD-aware: workgroups
// are dealt to the 8 XCDs round-robin (b % 8) and each XCD has its own L2, so
// XCD x is given a contiguous range of the tile order, and that order walks
// groups of kGroupM token tiles across the feature tiles. The workgroups an
// XCD runs at once then cover about 4 token tiles x 8 feature tiles, whose
// operands stay in (or near) its 4 MB L2 (for 256 x 384 tiles, 448 KB of the
// 2.5 MB a K step requests are distinct).
constexpr int kXcds = 8;
constexpr int kGroupM = 4;

__device__ __forceinline__ int2 xcd_tile(int b, int tn, int tm) {
  const int total = tn * tm;
  const int x = b % kXcds, idx = b / kXcds;
  const int base = total / kXcds, extra = total % kXcds;  // XCD x gets base + (x < extra) tiles
  const int t = x * base + min(x, extra) + idx;
  const int group = t / (kGroupM * tn);
  const int gm0 = group * kGroupM;
  const int gsize = min(kGroupM, tm - gm0);
  const int r = t - group * kGroupM * tn;
  return make_int2(r / gsize, gm0 + r % gsize);  // (feature tile, token tile)
}

// TBN x TBM tiles (features x tokens) per workgroup of WN x WM waves; a wave
// owns (TBN/WN) x (TBM/WM) as blocks of 32 x 32. 128 x 128 with 2 x 2 waves:
// two workgroups per CU (64 KB of LDS each), 64 x 64 per wave. 256 x 384 with
// 4 x 2 waves: one workgroup of 8 waves per CU using all 160 KB of LDS (two
// stages of 80 KB), 64 x 192 per wave (12 accumulator blocks, ~236 VGPRs, no
// spills); per MFMA it stages 5/8 of the bytes of the 128 x 128 tile through
// LDS and reads 2/3 of its LDS operand bytes.
template <typename T, int E, int TBN, int TBM, int WN, int WM, int KS, int NS>
__global__ __launch_bounds__(64 * WN * WM) __attribute__((amdgpu_waves_per_eu(2)))
void gemm32_kernel(GemmArgs g) {
  constexpr int NW = WN * WM;              // waves
  constexpr int NBN = TBN / WN / 32;       // 32x32 blocks per wave along features
  constexpr int NBM = TBM / WM / 32;       // and along tokens
  constexpr int SL = KS / 8;               // 16-byte slots per row of a stage
  constexpr int RPL = kWave / SL;          // rows one 1 KB load instruction moves
  // NS LDS stages of KS k values each; see lds_load16 for why the loads are
  // counted by hand.
  __shared__ Stage32<TBN, TBM, SL> st[NS];
  const int tid = threadIdx.x;
  // readfirstlane: the wave index is uniform, so the LDS destinations live in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid % kWave;
  const int wn = wave / WM, wm = wave % WM;
  const int l32 = lane % 32, hf = lane / 32;
  const int2 tile = xcd_tile(blockIdx.x, (g.n + TBN - 1) / TBN, (g.m + TBM - 1) / TBM);
  const int n0 = tile.x * TBN;
  const int m0 = tile.y * TBM;
  const int ksteps = g.k / KS;

  // Loads: the TBN + TBM rows of a step are chunks of RPL rows; wave w takes
  // chunks w, w + NW, ... Lane i of a chunk moves row RPL c + i/SL into slot
  // i%SL, i.e. column (i%SL) ^ stage_swizzle(row); the swizzle depends on the
  // chunk's parity at most, so two byte offsets per lane cover every chunk.
  const i32x4_t rw = buffer_rsrc(g.w, unsigned(g.n * g.k * 2));
  const i32x4_t ra = buffer_rsrc(g.a, unsigned(g.m * g.k * 2));
  const int rr = lane / SL, pos = lane % SL;
  unsigned voff[2];
#pragma unroll
  for (int par = 0; par < 2; ++par)
    voff[par] = unsigned((rr * g.k + 8 * (pos ^ stage_swizzle<SL>(RPL * par + rr))) * 2);
  constexpr int CHN = TBN / RPL, CHM = TBM / RPL;  // chunks per operand
  constexpr int CPW = (CHN + CHM) / NW;            // load instructions per wave and stage
  static_assert((CHN + CHM) % NW == 0 && CHN % 2 == 0, "chunks per wave");

#define SFL_G32_ISSUE(stage, kt)                                                            \
  {                                                                                         \
    _Pragma("unroll") for (int c0 = 0; c0 < CHN + CHM; c0 += NW) {                          \
      const int c = c0 + wave;                                                              \
      if (c < CHN)                                                                          \
        lds_load16(rw, lds_offset(&stage.w[RPL * c][0]), voff[c & 1],                       \
                   unsigned(((n0 + RPL * c) * g.k + (kt) * KS) * 2));                       \
      else                                                                                  \
        lds_load16(ra, lds_offset(&stage.a[RPL * (c - CHN)][0]), voff[(c - CHN) & 1],       \
                   unsigned(((m0 + RPL * (c - CHN)) * g.k + (kt) * KS) * 2));               \
    }                                                                                       \
  }
  // Operand reads: lane (l32, hf) takes row 32t + l32, column 2kk + hf.
  const int sw = stage_swizzle<SL>(l32);
#define SFL_G32_COMPUTE(stage)                                                              \
  _Pragma("unroll") for (int kk = 0; kk < KS / 16; ++kk) {                                  \
    const int slot = (2 * kk + hf) ^ sw;                                                    \
    u32x4 af[NBN], bfr[NBM];                                                                \
    _Pragma("unroll") for (int t = 0; t < NBN; ++t) {                                       \
      const uint4 ra_ = stage.w[32 * (NBN * wn + t) + l32][slot];                           \
      af[t] = u32x4{ra_.x, ra_.y, ra_.z, ra_.w};                                            \
    }                                                                                       \
    _Pragma("unroll") for (int t = 0; t < NBM; ++t) {                                       \
      const uint4 rb_ = stage.a[32 * (NBM * wm + t) + l32][slot];                           \
      bfr[t] = u32x4{rb_.x, rb_.y, rb_.z, rb_.w};                                           \
    }                                                                                       \
    _Pragma("unroll") for (int i = 0; i < NBN; ++i)                                         \
      _Pragma("unroll") for (int j = 0; j < NBM; ++j) acc[i][j] = mfma32<T>(af[i], bfr[j], acc[i][j]); \
  }

  f32x16 acc[NBN][NBM];
#pragma unroll
  for (int i = 0; i < NBN; ++i)
#pragma unroll
    for (int j = 0; j < NBM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  // Residual accumulation into fp32 C (x += A W^T): the accumulators start
  // from the old C values, loaded now, while the first stages are in flight,
  // so the epilogue only stores. (Unconditional loads from clamped addresses;
  // the values of rows / columns past C are never stored.)
  const bool acc_c = E == G_PLAIN && g.c_f32 && g.accumulate && (g.n & 3) == 0;
  if constexpr (E == G_PLAIN) {
    if (acc_c) {
      const float* c = static_cast<const float*>(g.c);
#pragma unroll
      for (int j = 0; j < NBM; ++j) {
        const long mr = min(m0 + (TBM / WM) * wm + 32 * j + l32, g.m - 1);
#pragma unroll
        for (int i = 0; i < NBN; ++i) {
          const int nt = n0 + (TBN / WN) * wn + 32 * i;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 o = *reinterpret_cast<const float4*>(c + mr * g.n + min(nt + 8 * q + 4 * hf, g.n - 4));
            acc[i][j][4 * q] = o.x;
            acc[i][j][4 * q + 1] = o.y;
            acc[i][j][4 * q + 2] = o.z;
            acc[i][j][4 * q + 3] = o.w;
          }
        }
      }
    }
  }

  // Row scales of the normalized input (q/k/v, SwiGLU), loaded while the
  // first stages are in flight.
  float rsc[NBM];
#pragma unroll
  for (int j = 0; j < NBM; ++j) rsc[j] = 1.f;
  if constexpr (E != G_PLAIN) {
    if (g.row_scale) {
#pragma unroll
      for (int j = 0; j < NBM; ++j) rsc[j] = g.row_scale[min(m0 + (TBM / WM) * wm + 32 * j + l32, g.m - 1)];
    }
  }

  // NS LDS stages in a ring: step kt computes from stage kt % NS while the
  // loads of the next NS - 1 steps are in flight. At step kt the wave waits
  // only for stage kt's loads (the younger stages' CPW each may stay
  // outstanding), the barrier then covers every wave's share, and stage
  // (kt - 1) % NS, last read before that barrier, is refilled with step
  // kt + NS - 1. One loop body, so every accumulator keeps its registers.
#pragma unroll
  for (int p = 0; p < NS - 1; ++p)
    if (p < ksteps) SFL_G32_ISSUE(st[p], p)
  for (int kt = 0; kt < ksteps; ++kt) {
    const int younger = min(NS - 2, ksteps - 1 - kt);  // stages issued after stage kt
    if (NS > 3 && younger >= 2) __builtin_amdgcn_s_waitcnt(sfl_vmcnt(NS > 3 ? 2 * CPW : 0));
    else if (NS > 2 && younger >= 1) __builtin_amdgcn_s_waitcnt(sfl_vmcnt(NS > 2 ? CPW : 0));
    else __builtin_amdgcn_s_waitcnt(sfl_vmcnt(0));
    __syncthreads();  // every wave's loads of this stage landed; stage (kt - 1) % NS is no longer read
    if (kt + NS - 1 < ksteps) SFL_G32_ISSUE(st[(kt + NS - 1) % NS], kt + NS - 1)
    SFL_G32_COMPUTE(st[kt % NS])
  }
#undef SFL_G32_COMPUTE
#undef SFL_G32_ISSUE

  if constexpr (E == G_PLAIN) {
    if (acc_c) {
      float* const c = static_cast<float*>(g.c);
      const bool norm = g.norm_gain != nullptr;  // uniform
      // The next norm's gains for this lane's features (one batch of loads,
      // before any store).
      uint2 gw[NBN][4];
      if (norm) {
#pragma unroll
        for (int i = 0; i < NBN; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            gw[i][q] = *reinterpret_cast<const uint2*>(
                g.norm_gain + min(n0 + (TBN / WN) * wn + 32 * i + 8 * q + 4 * hf, g.n - 4));
      }
      float ssq[NBM];
#pragma unroll
      for (int j = 0; j < NBM; ++j) {
        const int m = m0 + (TBM / WM) * wm + 32 * j + l32;
        ssq[j] = 0.f;
#pragma unroll
        for (int i = 0; i < NBN; ++i) {
          const int nt = n0 + (TBN / WN) * wn + 32 * i;
          uint32_t pk[4][2];  // T(x * gain) of features nt + 8q + 4hf + (0..3)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int n = nt + 8 * q + 4 * hf;
            const float4 v = make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                         acc[i][j][4 * q + 3]);
            const bool in = m < g.m && n < g.n;
            if (in) *reinterpret_cast<float4*>(c + long(m) * g.n + n) = v;
            if (norm) {
              pk[q][0] = pack2<T>(v.x * lo16<T>(gw[i][q].x), v.y * hi16<T>(gw[i][q].x));
              pk[q][1] = pack2<T>(v.z * lo16<T>(gw[i][q].y), v.w * hi16<T>(gw[i][q].y));
              if (in) ssq[j] += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
            }
          }
          if (norm) {
            if (g.vec16) {  // 8 consecutive features per lane (every lane swaps)
#pragma unroll
              for (int q = 0; q < 4; q += 2) {
                const uint4 o = pair8(pk[q], pk[q + 1]);
                const int n = nt + 8 * q + 8 * hf;
                if (m < g.m && n < g.n) *reinterpret_cast<uint4*>(g.norm_act + long(m) * g.n + n) = o;
              }
            } else {
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const int n = nt + 8 * q + 4 * hf;
                if (m < g.m && n < g.n)
                  *reinterpret_cast<uint2*>(g.norm_act + long(m) * g.n + n) = make_uint2(pk[q][0], pk[q][1]);
              }
            }
          }
        }
      }
      if (norm) {
        // Sum of squares per token over each 128-feature part: this lane's 32
        // features, its partner lane's (l ^ 32: the other 4 of each 8), then
        // the wave pair (wn, wn ^ 1) covering the part, in that order.
        float* const part_s = reinterpret_cast<float*>(&st[0]);  // [WN][TBM] (the stages are free now)
        __syncthreads();  // every wave has read the last stage
#pragma unroll
        for (int j = 0; j < NBM; ++j) {
          const float t = ssq[j] + lane_xor(ssq[j], 32);
          if (hf == 0) part_s[wn * TBM + (TBM / WM) * wm + 32 * j + l32] = t;
        }
        __syncthreads();
        static_assert(TBN / WN == 64, "two waves per 128-feature part");
        const int part = (n0 + (TBN / WN) * wn) / 128;
        if ((wn & 1) == 0 && part * 128 < g.n) {
          for (int r = lane; r < TBM / WM; r += kWave) {
            const int row = (TBM / WM) * wm + r;
            const int m = m0 + row;
            if (m < g.m) g.norm_ss[long(part) * g.m + m] = part_s[wn * TBM + row] + part_s[(wn + 1) * TBM + row];
          }
        }
      }
      return;
    }
  }

  // acc[i][j][4q + e] holds feature n0 + (TBN/WN)wn + 32i + 8q + 4hf + e of
  // token m0 + (TBM/WM)wm + 32j + l32.
#pragma unroll
  for (int j = 0; j < NBM; ++j) {
    const int m = m0 + (TBM / WM) * wm + 32 * j + l32;
    const QkvTok tok = E == G_QKV ? qkv_tok(g, m) : QkvTok{};
#pragma unroll
    for (int i = 0; i < NBN; ++i) {
      const int nt = n0 + (TBN / WN) * wn + 32 * i;
      // One division pair per 32-feature block; the lane's features derive from
      // it. With head dims that are multiples of 32 the block is one head of one
      // section: its features share the destination row.
      const QkvFeat fb = E == G_QKV ? qkv_feat(g, nt) : QkvFeat{};
      const bool blk = E == G_QKV && g.head_dim % 32 == 0;
      uint16_t* const base = blk ? qkv_dst(g, fb, tok) : nullptr;
      if constexpr (E == G_SWIGLU) {
        // W1/W3 interleaved in blocks of 8 rows: groups q = 0, 2 are W1 features,
        // q + 1 the matching W3 features, all in this lane. Hidden features
        // nt/2 + 4q + 4hf .. +3; with vec16 the two groups go out as one
        // 16-byte store per lane at nt/2 + 8hf (d_ff % 8 == 0: a group of 8 is
        // wholly inside or outside d_ff).
        uint32_t pk[2][2];
#pragma unroll
        for (int q = 0; q < 4; q += 2) {
          float h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a1 = acc[i][j][4 * q + e] * rsc[j], a3 = acc[i][j][4 * q + 4 + e] * rsc[j];
            h[e] = silu_mul(a1, a3);
          }
          pk[q / 2][0] = pack2<T>(h[0], h[1]);
          pk[q / 2][1] = pack2<T>(h[2], h[3]);
        }
        if (g.vec16) {
          const uint4 v8 = pair8(pk[0], pk[1]);
          const int f = nt / 2 + 8 * hf;
          if (m < g.m && f < g.n / 2) *reinterpret_cast<uint4*>(g.h_out + long(m) * (g.n / 2) + f) = v8;
        } else if (m < g.m) {
#pragma unroll
          for (int q = 0; q < 4; q += 2) {
            const int f = nt / 2 + 4 * q + 4 * hf;  // hidden feature index
            if (f < g.n / 2)
              *reinterpret_cast<uint2*>(g.h_out + long(m) * (g.n / 2) + f) = make_uint2(pk[q / 2][0], pk[q / 2][1]);
          }
        }
      } else if (E != G_PLAIN || (!g.c_f32 && !g.accumulate)) {
        // bf16 outputs (q/k/v, plain bf16): feature groups q and q + 1 of the
        // lane pair go out as 16-byte stores (vec16; whole 32-feature blocks
        // inside N), else 8 bytes per group.
        const bool wide = g.vec16 && nt + 32 <= g.n && (E == G_QKV || g.n % 8 == 0);
#pragma unroll
        for (int q = 0; q < 4; q += 2) {
          uint32_t pk[2][2];
          QkvFeat feat[2];
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            float y[4] = {acc[i][j][4 * (q + r)] * rsc[j], acc[i][j][4 * (q + r) + 1] * rsc[j],
                          acc[i][j][4 * (q + r) + 2] * rsc[j], acc[i][j][4 * (q + r) + 3] * rsc[j]};
            feat[r] = E != G_QKV ? QkvFeat{}
                      : blk ? QkvFeat{fb.section, fb.head, fb.dim + 8 * (q + r) + 4 * hf}
                            : qkv_feat_at(g, fb, 8 * (q + r) + 4 * hf);
            if constexpr (E == G_QKV) rope4(g, y, feat[r], tok);
            pk[r][0] = pack2<T>(y[0], y[1]);
            pk[r][1] = pack2<T>(y[2], y[3]);
          }
          if (wide) {
            const uint4 v8 = pair8(pk[0], pk[1]);
            if (m < g.m) {
              const int f = nt + 8 * q + 8 * hf;  // first of this lane's 8 features
              uint16_t* dst = E == G_QKV ? (blk ? base + 8 * q + 8 * hf : qkv_dst(g, qkv_feat_at(g, fb, 8 * q + 8 * hf), tok))
                                         : static_cast<uint16_t*>(g.c) + long(m) * g.n + f;
              *reinterpret_cast<uint4*>(dst) = v8;
            }
          } else if (m < g.m) {
#pragma unroll
            for (int r = 0; r < 2; ++r) {
              const int n = nt + 8 * (q + r) + 4 * hf;
              if (E == G_QKV) {
                if (n < g.n) *reinterpret_cast<uint2*>(qkv_dst(g, feat[r], tok)) = make_uint2(pk[r][0], pk[r][1]);
              } else if (n + 3 < g.n && (g.n & 3) == 0) {
                *reinterpret_cast<uint2*>(static_cast<uint16_t*>(g.c) + long(m) * g.n + n) =
                    make_uint2(pk[r][0], pk[r][1]);
              } else {
                uint16_t* c = static_cast<uint16_t*>(g.c) + long(m) * g.n + n;
                const uint32_t w[2] = {pk[r][0], pk[r][1]};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  if (n + e < g.n) c[e] = uint16_t(w[e / 2] >> (16 * (e % 2)));
              }
            }
          }
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 v = {acc[i][j][4 * q] * rsc[j], acc[i][j][4 * q + 1] * rsc[j], acc[i][j][4 * q + 2] * rsc[j],
                           acc[i][j][4 * q + 3] * rsc[j]};
          // store_tile's feature index is nt + 4 * grp: grp = 2q + hf.
          const QkvFeat feat = E == G_QKV ? qkv_feat_at(g, fb, 8 * q + 4 * hf) : QkvFeat{};
          store_tile<T, E>(g, v, nt, 2 * q + hf, m, feat, tok);
        }
      }
    }
  }
}

inline bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

template <typename T, int E>
int launch_gemm_t(const GemmArgs& g, hipStream_t s, const char* what) {
  if (g.m < 1 || g.n < 1 || g.k < 1) return set_error(SFL_ERR_INVALID, "%s: sizes must be positive", what);
  if (g.k % 8) return set_error(SFL_ERR_UNSUPPORTED, "%s: K must be a multiple of 8", what);
  if (g.k % K2 == 0 && long(g.m) * g.k < (1L << 30) && long(g.n) * g.k < (1L << 30)) {
    const long tiles = long((g.n + TB - 1) / TB) * ((g.m + TB - 1) / TB);
    if (tiles > (1L << 31) - 1) return set_error(SFL_ERR_UNSUPPORTED, "%s: too many tiles", what);
    // 256 x 384 tiles where they still give every CU more than one workgroup
    // (measured against 256 x 256 on the 324M prefill shapes, bit-identical
    // outputs: q/k/v 437 -> 421 us, output_proj 171 -> 145, w1/w3 640 -> 603,
    // w2 330 -> 308; 2 x 4 waves of 128 x 96 and a ring of 4 stages of K = 32
    // were no better).
    const long big = long((g.n + 255) / 256) * ((g.m + 383) / 384);
    if (big >= 320)
      hipLaunchKernelGGL((gemm32_kernel<T, E, 256, 384, 4, 2, 64, 2>), dim3(unsigned(big)), dim3(512), 0, s, g);
    else
      hipLaunchKernelGGL((gemm32_kernel<T, E, 128, 128, 2, 2, 64, 2>), dim3(unsigned(tiles)), dim3(kThreads), 0, s, g);
    return check_launch(what);
  }
  dim3 grid((g.n + TN - 1) / TN, (g.m + TM - 1) / TM);
  if (grid.y > 65535) return set_error(SFL_ERR_UNSUPPORTED, "%s: M too large", what);
  hipLaunchKernelGGL((gemm_kernel<T, E>), grid, dim3(kThreads), 0, s, g);
  return check_launch(what);
}

// The GEMMs' 16-bit element type: SFL_DTYPE_BF16 or SFL_DTYPE_F16.
template <int E>
int launch_gemm(const GemmArgs& g, int dtype, hipStream_t s, const char* what) {
  if (dtype == SFL_DTYPE_BF16) return launch_gemm_t<bf16_t, E>(g, s, what);
  if (dtype == SFL_DTYPE_F16) return launch_gemm_t<f16_t, E>(g, s, what);
  return set_error(SFL_ERR_UNSUPPORTED, "%s: dtype must be BF16 or F16", what);
}

// Prefill embedding gather: x[m] = emb[ids[m]] in fp32.
template <typename T>
__global__ __launch_bounds__(256) void embed_rows_kernel(const int64_t* ids, const T* emb, float* x, int d) {
  const long m = blockIdx.x;
  const T* src = emb + ids[m] * d;
  for (int i = threadIdx.x; i < d; i += blockDim.x) x[m * d + i] = load_scalar<T>(src + i);
}

// Prefill RMSNorm: out[m] = O(x[m] / sqrt(mean(x[m]^2) + eps) * w) (layers.py:133-141),
// O the GEMMs' 16-bit type.
template <typename T, typename O>
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* x, const T* w, O* out, int d) {
  __shared__ float part[4];
  const long m = blockIdx.x;
  const float* xr = x + m * d;
  float ss = 0.f;
  for (int i = threadIdx.x; i < d; i += 256) ss = fmaf(xr[i], xr[i], ss);
  ss = wave_sum(ss);
  if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = ss;
  __syncthreads();
  const float total = part[0] + part[1] + part[2] + part[3];
  const float inv = 1.f / sqrtf(total / float(d) + 1e-5f);
  for (int i = threadIdx.x; i < d; i += 256) store_scalar<O>(out + m * d + i, (xr[i] * inv) * load_scalar<T>(w + i));
}

// The same for rows of d % 4 == 0 and d <= 4 * 64 * kNormVec with one wave per
// row: the row is read once with 16-byte loads and kept in registers, the sum
// of squares is a wave reduction (no LDS, no barrier), and each lane stores
// four 16-bit values at a time.
constexpr int kNormVec = 8;
// kScaled: out = O(x * w) and rscale[row] = 1 / rms(x), for a consumer GEMM
// that applies the scale to its products.
template <typename T, typename O, bool kScaled = false>
__global__ __launch_bounds__(256) void rmsnorm_rows_wave_kernel(const float* x, const T* w, O* out, int m,
                                                               int d, float* rscale = nullptr) {
  const long row = long(blockIdx.x) * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= m) return;
  const float* xr = x + row * d;
  float4 v[kNormVec];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kNormVec; ++j) {
    const int i = 4 * (j * kWave + lane);
    v[j] = i < d ? *reinterpret_cast<const float4*>(xr + i) : make_float4(0.f, 0.f, 0.f, 0.f);
    ss = fmaf(v[j].x, v[j].x, ss);
    ss = fmaf(v[j].y, v[j].y, ss);
    ss = fmaf(v[j].z, v[j].z, ss);
    ss = fmaf(v[j].w, v[j].w, ss);
  }
  const float inv = 1.f / sqrtf(wave_sum(ss) / float(d) + 1e-5f);
  if (kScaled && lane == 0) rscale[row] = inv;
  const float sc = kScaled ? 1.f : inv;
#pragma unroll
  for (int j = 0; j < kNormVec; ++j) {
    const int i = 4 * (j * kWave + lane);
    if (i < d) {
      float y0 = v[j].x, y1 = v[j].y, y2 = v[j].z, y3 = v[j].w;
      if (!kScaled) {
        y0 *= sc; y1 *= sc; y2 *= sc; y3 *= sc;
      }
      y0 *= load_scalar<T>(w + i); y1 *= load_scalar<T>(w + i + 1);
      y2 *= load_scalar<T>(w + i + 2); y3 *= load_scalar<T>(w + i + 3);
      if constexpr (sizeof(O) == 4)
        *reinterpret_cast<float4*>(out + row * d + i) = make_float4(y0, y1, y2, y3);
      else
        *reinterpret_cast<uint2*>(out + row * d + i) = make_uint2(pack2<O>(y0, y1), pack2<O>(y2, y3));
    }
  }
}

// rscale[m] = 1 / sqrt(sum_p ss[p][m] / d + eps): the inverse RMS from the
// per-part sums of squares a residual GEMM left (parts in a fixed order).
__global__ __launch_bounds__(256) void norm_scale_kernel(const float* __restrict__ ss, int parts, int m, int d,
                                                         float* __restrict__ rscale) {
  const long row = long(blockIdx.x) * 256 + threadIdx.x;
  if (row >= m) return;
  float t = 0.f;
  for (int p = 0; p < parts; ++p) t += ss[long(p) * m + row];
  rscale[row] = 1.f / sqrtf(t / float(d) + 1e-5f);
}

}  // namespace
}  // namespace sfl

using namespace sfl;

// The GEMMs' 16-bit element type (A, W and 16-bit outputs).
static bool gemm_dtype_ok(int dtype) { return dtype == SFL_DTYPE_BF16 || dtype == SFL_DTYPE_F16; }

extern "C" int sfl_gemm(const void* a, const void* w, void* c, int m, int n, int k, int dtype, int c_dtype,
                        int accumulate, void* stream) {
  const char* what = "gemm";
  if (!a || !w || !c) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (dtype == SFL_DTYPE_F32) {  // the fp32 MFMA GEMM (prefill_f32.hip)
    if (c_dtype != SFL_DTYPE_F32) return set_error(SFL_ERR_UNSUPPORTED, "%s: F32 inputs need an F32 output", what);
    F32GemmArgs f{};
    f.a = static_cast<const float*>(a); f.w = static_cast<const float*>(w);
    f.m = m; f.n = n; f.k = k; f.c = static_cast<float*>(c); f.accumulate = accumulate;
    return launch_gemm_f32(f, F32_PLAIN, static_cast<hipStream_t>(stream), what);
  }
  if (!gemm_dtype_ok(dtype)) return set_error(SFL_ERR_UNSUPPORTED, "%s: dtype must be F32, BF16 or F16", what);
  if (c_dtype != SFL_DTYPE_F32 && c_dtype != dtype)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: output dtype must be F32 or the input dtype", what);
  if (accumulate && c_dtype != SFL_DTYPE_F32)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: accumulation needs an F32 output", what);
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(a); g.w = static_cast<const uint16_t*>(w);
  g.m = m; g.n = n; g.k = k; g.c = c; g.c_f32 = c_dtype == SFL_DTYPE_F32; g.accumulate = accumulate;
  g.vec16 = aligned16(c);
  return launch_gemm<G_PLAIN>(g, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_gemm_qkv_rope(const void* a, const void* w_qkv, int m, int seq, int d_model, int heads,
                                 const float* cos_t, const float* sin_t, void* q_out, void* k_cache,
                                 void* v_cache, int capacity, int dtype, void* stream) {
  const char* what = "gemm_qkv_rope";
  if (!a || !w_qkv || !cos_t || !sin_t || !q_out || !k_cache || !v_cache)
    return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (seq < 1 || m % seq) return set_error(SFL_ERR_INVALID, "%s: rows must be batch * seq", what);
  if (heads < 1 || d_model % heads || (d_model / heads) % 16)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: head dim must be a multiple of 16", what);
  if (seq > capacity) return set_error(SFL_ERR_INVALID, "%s: seq exceeds the cache capacity", what);
  if (dtype == SFL_DTYPE_F32) {
    if (!aligned16(q_out) || !aligned16(k_cache) || !aligned16(v_cache))
      return set_error(SFL_ERR_INVALID, "%s: fp32 q and caches must be 16-byte aligned", what);
    F32GemmArgs f{};
    f.a = static_cast<const float*>(a); f.w = static_cast<const float*>(w_qkv);
    f.m = m; f.n = 3 * d_model; f.k = d_model;
    f.cos_t = cos_t; f.sin_t = sin_t; f.seq = seq; f.heads = heads; f.head_dim = d_model / heads;
    f.d_model = d_model; f.cap = capacity;
    f.q_out = static_cast<float*>(q_out); f.k_cache = static_cast<float*>(k_cache);
    f.v_cache = static_cast<float*>(v_cache);
    return launch_gemm_f32(f, F32_QKV, static_cast<hipStream_t>(stream), what);
  }
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(a); g.w = static_cast<const uint16_t*>(w_qkv);
  g.m = m; g.n = 3 * d_model; g.k = d_model;
  g.cos_t = cos_t; g.sin_t = sin_t; g.seq = seq; g.heads = heads; g.head_dim = d_model / heads;
  g.d_model = d_model; g.cap = capacity;
  g.q_out = static_cast<uint16_t*>(q_out); g.k_cache = static_cast<uint16_t*>(k_cache);
  g.v_cache = static_cast<uint16_t*>(v_cache);
  g.vec16 = aligned16(q_out) && aligned16(k_cache) && aligned16(v_cache);
  return launch_gemm<G_QKV>(g, dtype, static_cast<hipStream_t>(stream), what);
}

// The fused-norm entry points need the 32x32 kernels (K % 64 == 0, 32-bit offsets).
static bool gemm32_path(int m, int n, int k) {
  return k % K2 == 0 && long(m) * k < (1L << 30) && long(n) * k < (1L << 30);
}

extern "C" int sfl_gemm_qkv_rope_scaled(const void* a_xg, const void* w_qkv, const float* rscale, int m, int seq,
                                        int d_model, int heads, const float* cos_t, const float* sin_t,
                                        void* q_out, void* k_cache, void* v_cache, int capacity, int dtype,
                                        void* stream) {
  const char* what = "gemm_qkv_rope_scaled";
  if (!rscale) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (!gemm32_path(m, 3 * d_model, d_model))
    return set_error(SFL_ERR_UNSUPPORTED, "%s: d_model must be a multiple of %d", what, K2);
  if (!a_xg || !w_qkv || !cos_t || !sin_t || !q_out || !k_cache || !v_cache)
    return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (seq < 1 || m % seq) return set_error(SFL_ERR_INVALID, "%s: rows must be batch * seq", what);
  if (heads < 1 || d_model % heads || (d_model / heads) % 16)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: head dim must be a multiple of 16", what);
  if (seq > capacity) return set_error(SFL_ERR_INVALID, "%s: seq exceeds the cache capacity", what);
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(a_xg); g.w = static_cast<const uint16_t*>(w_qkv);
  g.m = m; g.n = 3 * d_model; g.k = d_model;
  g.cos_t = cos_t; g.sin_t = sin_t; g.seq = seq; g.heads = heads; g.head_dim = d_model / heads;
  g.d_model = d_model; g.cap = capacity;
  g.q_out = static_cast<uint16_t*>(q_out); g.k_cache = static_cast<uint16_t*>(k_cache);
  g.v_cache = static_cast<uint16_t*>(v_cache);
  g.vec16 = aligned16(q_out) && aligned16(k_cache) && aligned16(v_cache);
  g.row_scale = rscale;
  return launch_gemm<G_QKV>(g, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_gemm_swiglu_scaled(const void* a_xg, const void* w13_interleaved, const float* rscale,
                                      void* h_out, int m, int d_ff, int k, int dtype, void* stream) {
  const char* what = "gemm_swiglu_scaled";
  if (!a_xg || !w13_interleaved || !rscale || !h_out)
    return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (d_ff % 8) return set_error(SFL_ERR_UNSUPPORTED, "%s: d_ff must be a multiple of 8", what);
  if (!gemm32_path(m, 2 * d_ff, k)) return set_error(SFL_ERR_UNSUPPORTED, "%s: K must be a multiple of %d", what, K2);
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(a_xg); g.w = static_cast<const uint16_t*>(w13_interleaved);
  g.m = m; g.n = 2 * d_ff; g.k = k; g.h_out = static_cast<uint16_t*>(h_out);
  g.vec16 = aligned16(h_out);
  g.row_scale = rscale;
  return launch_gemm<G_SWIGLU>(g, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_gemm_residual_norm(const void* a, const void* w, float* x, int m, int n, int k,
                                      const void* gain_next, void* act_xg, float* ss_parts, int dtype,
                                      void* stream) {
  const char* what = "gemm_residual_norm";
  if (!a || !w || !x || !gain_next || !act_xg || !ss_parts)
    return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (m < 1 || n < 1 || k < 1) return set_error(SFL_ERR_INVALID, "%s: sizes must be positive", what);
  if (n % 4) return set_error(SFL_ERR_UNSUPPORTED, "%s: N must be a multiple of 4", what);
  if (!gemm32_path(m, n, k)) return set_error(SFL_ERR_UNSUPPORTED, "%s: K must be a multiple of %d", what, K2);
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(act_xg) % 8 ||
      reinterpret_cast<uintptr_t>(gain_next) % 8)
    return set_error(SFL_ERR_INVALID, "%s: x must be 16-byte and act / gain 8-byte aligned", what);
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(a); g.w = static_cast<const uint16_t*>(w);
  g.m = m; g.n = n; g.k = k; g.c = x; g.c_f32 = 1; g.accumulate = 1;
  g.norm_gain = static_cast<const uint16_t*>(gain_next);
  g.norm_act = static_cast<uint16_t*>(act_xg);
  g.norm_ss = ss_parts;
  g.vec16 = aligned16(act_xg) && n % 8 == 0;  // rows of act start 16-byte aligned
  return launch_gemm<G_PLAIN>(g, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_norm_scale(const float* ss_parts, int parts, int m, int d_model, float* rscale, void* stream) {
  if (!ss_parts || !rscale) return set_error(SFL_ERR_INVALID, "norm_scale: null pointer argument");
  if (parts < 1 || m < 1 || d_model < 1) return set_error(SFL_ERR_INVALID, "norm_scale: sizes must be positive");
  hipLaunchKernelGGL(norm_scale_kernel, dim3(unsigned((m + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), ss_parts, parts, m, d_model, rscale);
  return check_launch("norm_scale");
}

extern "C" int sfl_rmsnorm_rows_scaled(const float* x, const void* w, void* act_xg, float* rscale, int m,
                                       int d_model, int dtype, void* stream) {
  const char* what = "rmsnorm_rows_scaled";
  if (!x || !w || !act_xg || !rscale) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (m < 1 || d_model < 1) return set_error(SFL_ERR_INVALID, "%s: sizes must be positive", what);
  if (!gemm_dtype_ok(dtype)) return set_error(SFL_ERR_UNSUPPORTED, "%s: dtype must be BF16 or F16", what);
  if (d_model % 4 || d_model > 4 * kWave * kNormVec || reinterpret_cast<uintptr_t>(x) % 16 ||
      reinterpret_cast<uintptr_t>(act_xg) % 8)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: d_model must be a multiple of 4 and at most %d, x 16-byte and "
                     "act 8-byte aligned", what, 4 * kWave * kNormVec);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == SFL_DTYPE_BF16)
    hipLaunchKernelGGL((rmsnorm_rows_wave_kernel<bf16_t, bf16_t, true>), dim3((m + 3) / 4), dim3(256), 0, s, x,
                       static_cast<const bf16_t*>(w), static_cast<bf16_t*>(act_xg), m, d_model, rscale);
  else
    hipLaunchKernelGGL((rmsnorm_rows_wave_kernel<f16_t, f16_t, true>), dim3((m + 3) / 4), dim3(256), 0, s, x,
                       static_cast<const f16_t*>(w), static_cast<f16_t*>(act_xg), m, d_model, rscale);
  return check_launch(what);
}

extern "C" int sfl_gemm_swiglu(const void* a, const void* w13_interleaved, void* h_out, int m, int d_ff,
                               int k, int dtype, void* stream) {
  const char* what = "gemm_swiglu";
  if (!a || !w13_interleaved || !h_out) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (d_ff % 8) return set_error(SFL_ERR_UNSUPPORTED, "%s: d_ff must be a multiple of 8", what);
  if (dtype == SFL_DTYPE_F32) {
    if (!aligned16(h_out)) return set_error(SFL_ERR_INVALID, "%s: fp32 h must be 16-byte aligned", what);
    F32GemmArgs f{};
    f.a = static_cast<const float*>(a); f.w = static_cast<const float*>(w13_interleaved);
    f.m = m; f.n = 2 * d_ff; f.k = k; f.h_out = static_cast<float*>(h_out);
    return launch_gemm_f32(f, F32_SWIGLU, static_cast<hipStream_t>(stream), what);
  }
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(a); g.w = static_cast<const uint16_t*>(w13_interleaved);
  g.m = m; g.n = 2 * d_ff; g.k = k; g.h_out = static_cast<uint16_t*>(h_out);
  g.vec16 = aligned16(h_out);
  return launch_gemm<G_SWIGLU>(g, dtype, static_cast<hipStream_t>(stream), what);
}

extern "C" int sfl_embed_rows(const int64_t* ids, const void* emb, float* x, int m, int d_model, int dtype,
                              void* stream) {
  if (!ids || !emb || !x) return set_error(SFL_ERR_INVALID, "embed_rows: null pointer argument");
  if (m < 1 || d_model < 1) return set_error(SFL_ERR_INVALID, "embed_rows: sizes must be positive");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == SFL_DTYPE_BF16)
    hipLaunchKernelGGL(embed_rows_kernel<bf16_t>, dim3(m), dim3(256), 0, s, ids, static_cast<const bf16_t*>(emb), x, d_model);
  else if (dtype == SFL_DTYPE_F16)
    hipLaunchKernelGGL(embed_rows_kernel<f16_t>, dim3(m), dim3(256), 0, s, ids, static_cast<const f16_t*>(emb), x, d_model);
  else if (dtype == SFL_DTYPE_F32)
    hipLaunchKernelGGL(embed_rows_kernel<float>, dim3(m), dim3(256), 0, s, ids, static_cast<const float*>(emb), x, d_model);
  else
    return set_error(SFL_ERR_UNSUPPORTED, "embed_rows: dtype must be F32, BF16 or F16");
  return check_launch("embed_rows");
}

template <typename T, typename O>
static void launch_rmsnorm_rows(const float* x, const void* w, void* out, int m, int d, bool wave_rows, hipStream_t s) {
  if (wave_rows)
    hipLaunchKernelGGL((rmsnorm_rows_wave_kernel<T, O>), dim3((m + 3) / 4), dim3(256), 0, s, x,
                       static_cast<const T*>(w), static_cast<O*>(out), m, d, nullptr);
  else
    hipLaunchKernelGGL((rmsnorm_rows_kernel<T, O>), dim3(m), dim3(256), 0, s, x, static_cast<const T*>(w),
                       static_cast<O*>(out), d);
}

extern "C" int sfl_rmsnorm_rows(const float* x, const void* w, void* out, int m, int d_model, int dtype,
                                int out_dtype, void* stream) {
  const char* what = "rmsnorm_rows";
  if (!x || !w || !out) return set_error(SFL_ERR_INVALID, "%s: null pointer argument", what);
  if (m < 1 || d_model < 1) return set_error(SFL_ERR_INVALID, "%s: sizes must be positive", what);
  if (dtype != SFL_DTYPE_BF16 && dtype != SFL_DTYPE_F16 && dtype != SFL_DTYPE_F32)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: dtype must be F32, BF16 or F16", what);
  if (out_dtype != SFL_DTYPE_BF16 && out_dtype != SFL_DTYPE_F16 && out_dtype != SFL_DTYPE_F32)
    return set_error(SFL_ERR_UNSUPPORTED, "%s: out dtype must be F32, BF16 or F16", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool wave_rows = d_model % 4 == 0 && d_model <= 4 * kWave * kNormVec &&
                         reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(out) % (out_dtype == SFL_DTYPE_F32 ? 16 : 8) == 0;
  const int key = dtype * 8 + out_dtype;
  switch (key) {
    case SFL_DTYPE_BF16 * 8 + SFL_DTYPE_BF16: launch_rmsnorm_rows<bf16_t, bf16_t>(x, w, out, m, d_model, wave_rows, s); break;
    case SFL_DTYPE_F32 * 8 + SFL_DTYPE_BF16: launch_rmsnorm_rows<float, bf16_t>(x, w, out, m, d_model, wave_rows, s); break;
    case SFL_DTYPE_F16 * 8 + SFL_DTYPE_F16: launch_rmsnorm_rows<f16_t, f16_t>(x, w, out, m, d_model, wave_rows, s); break;
    case SFL_DTYPE_F32 * 8 + SFL_DTYPE_F32: launch_rmsnorm_rows<float, float>(x, w, out, m, d_model, wave_rows, s); break;
    default: return set_error(SFL_ERR_UNSUPPORTED, "%s: unsupported weight / output dtype pair", what);
  }
  return check_launch(what);
}
