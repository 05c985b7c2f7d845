/*
 * sfl.h -- C ABI of the MI355X (gfx950) decode path of the llmlab decoder.
 *
 * Every entry point takes raw device pointers, sizes and a hipStream_t passed
 * as `void*` (NULL = the null stream), launches asynchronously on that stream
 * and allocates nothing: callers own every buffer, including fp32 scratch.
 * Return value: 0 on success, a negative SFL_ERR_* code otherwise; the message
 * for the last failure on the calling thread is available from
 * sfl_last_error(). Argument checks happen before any launch, so a rejected
 * call leaves every buffer untouched.
 *
 * Tensor layouts are row-major and contiguous unless a stride is passed.
 * Element types are selected by an SFL_DTYPE_* code.
 */
#ifndef SFL_H_
#define SFL_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  SFL_DTYPE_F32 = 0,
  SFL_DTYPE_BF16 = 1,
  SFL_DTYPE_F16 = 2,
};

enum {
  SFL_OK = 0,
  SFL_ERR_INVALID = -1,     /* bad shape, size, pointer or value */
  SFL_ERR_UNSUPPORTED = -2, /* valid request outside the compiled variants */
  SFL_ERR_HIP = -3,         /* HIP runtime reported an error at launch */
};

/* Library version string and the message of the calling thread's last error. */
const char* sfl_version(void);
const char* sfl_last_error(void);

/*
 * Split-KV single-query attention over a contiguous KV cache.
 * Replaces the pybind `run` of attention_lab/cuda_decode/decode.cu:210-256
 * (kernels partial_attention :27-136 and merge_partials :138-184), bound in the
 * reference by attention_lab/cuda_decode/kernel.py:71-77.
 *
 *   q        [B, Hq, D]            dtype
 *   k, v     [B, Hkv, cap, D]      dtype
 *   lengths  [B] int32, clamped to [0, cap]; row b attends to keys [0, lengths[b])
 *   partial_max, partial_sum [B, Hq, splits] fp32 scratch
 *   partial_out              [B, Hq, splits, D] fp32 scratch
 *   out      [B, Hq, D]            dtype; rows with length 0 are zeros
 *
 * The cache is partitioned by capacity into `splits` chunks of
 * ceil(cap/splits) keys (decode.cu:50-52); chunks past a row's length do no
 * work. D in {32, 64, 128}; Hq/Hkv in {1, 2, 4, 8}; splits in [1, 1024].
 * dtype: F32, BF16 or F16; softmax state is fp32.
 */
int sfl_decode_attention(const void* q, const void* k, const void* v, const int32_t* lengths,
                         float* partial_max, float* partial_sum, float* partial_out, void* out,
                         int batch, int q_heads, int kv_heads, int capacity, int head_dim,
                         int splits, float scale, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SFL_H_ */
