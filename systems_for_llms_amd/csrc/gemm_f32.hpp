// fp32 prefill GEMMs (prefill_f32.hip): the arguments the 16-bit GEMM entry
// points (gemm.hip) pass through when their dtype is SFL_DTYPE_F32.
#pragma once
#include "common.hpp"

namespace sfl {

enum F32Epi { F32_PLAIN = 0, F32_QKV = 1, F32_SWIGLU = 2 };

struct F32GemmArgs {
  const float* a;  // [M, K]
  const float* w;  // [N, K]
  int m, n, k;
  // PLAIN: C [M, N] fp32, stored or (accumulate) added to
  float* c;
  int accumulate;
  // QKV: RoPE from the feature-major tables [head_dim / 2, cap]; q to
  // [B, H, T, dk], k / v to the [B, H, cap, dk] cache at positions 0..T-1
  const float* cos_t;
  const float* sin_t;
  int seq, heads, head_dim, d_model, cap;
  float* q_out;
  float* k_cache;
  float* v_cache;
  // SWIGLU: W is W1/W3 interleaved in blocks of 8 rows; h [M, N / 2]
  float* h_out;
};

// Launches the fp32 GEMM with epilogue `epi` (argument checks done by the caller).
int launch_gemm_f32(const F32GemmArgs& g, int epi, hipStream_t stream, const char* what);

}  // namespace sfl
