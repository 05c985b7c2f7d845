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
 * Element types are selected by an SFL_DTYPE_* code. In the decode-step
 * entry points weights and the KV cache use the model dtype; the residual
 * stream x and q are fp32; the GEMV inputs that other kernels produce (the
 * attention output, the SwiGLU hidden state, x * g) are in the activation
 * layout: SFL_DTYPE_F32X for F32 models, SFL_DTYPE_BF16X2 for BF16 models and
 * SFL_DTYPE_F16X2 for F16 models.
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
  /* Inputs of the decode GEMVs ("activation layout"), 4 bytes per value, for a
   * [B, K] matrix: blocks of 16 rows; each block is K/KC chunks of KC values
   * (KC = 32 for BF16X2, 16 for F32X), and chunk c of a block is stored as 64
   * lanes x 16 bytes, lane l = 16*g + r holding row r's values
   * [c*KC + g*KC/4, c*KC + (g+1)*KC/4). BF16X2 stores each value as hi = the
   * value truncated to bf16 and lo = the remainder truncated to bf16; a
   * chunk's 64 lanes of hi halves (1 KB) are followed by its lo halves (1 KB),
   * hi + lo keeping ~16 mantissa bits. F32X stores fp32 values (1 KB chunks).
   * Buffers hold whole 16-row blocks: ceil(B/16) * 16 * K * 4 bytes. */
  SFL_DTYPE_BF16X2 = 3,
  SFL_DTYPE_F32X = 4,
  /* F16X2: the BF16X2 layout for F16 models; hi = the value rounded to fp16,
   * lo = the remainder rounded to fp16. */
  SFL_DTYPE_F16X2 = 5,
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
 * work. D in {16, 32, 64, 128}; Hq/Hkv in {1, 2, 4, 8}; splits in [1, 1024].
 * kv_dtype: element type of k and v (F32, BF16 or F16); q_dtype: kv_dtype or
 * F32; out_dtype: kv_dtype, F32, BF16X2, F16X2 or F32X (the last three: the
 * GEMV activation layout of [B, Hq*D]). Softmax state is fp32. Cache rows at
 * positions >= lengths[b] are never read into the result (they may hold
 * anything, NaN included). Hq/Hkv >= 4 with D 64 or 128, q_dtype ==
 * kv_dtype in {BF16, F16}, 16-byte aligned q/k/v and cap*D*2 < 2^31 run
 * on the MFMA kernel; all other cases on the VALU kernel.
 */
int sfl_decode_attention(const void* q, const void* k, const void* v, const int32_t* lengths,
                         float* partial_max, float* partial_sum, float* partial_out, void* out,
                         int batch, int q_heads, int kv_heads, int capacity, int head_dim,
                         int splits, float scale, int kv_dtype, int q_dtype, int out_dtype,
                         void* stream);

/*
 * sfl_decode_attention without caller scratch, for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference: its prepare() allocates the
 * split scratch (attention_lab/cuda_decode/kernel.py:107-111). The split
 * partials live in a static device buffer of
 * sfl_decode_attention_static_scratch_bytes() (16 MiB), one per GPU, held
 * until the process ends; a call needing more -- 2*align256(B*Hq*splits*4) +
 * align256(B*Hq*splits*D*4) bytes -- is rejected before any launch. Every call
 * on a GPU shares that GPU's buffer, so calls that overlap on one GPU (two
 * streams, two threads) race; nothing in it needs clearing between calls
 * (the merge reads only the partials its own call wrote). The current HIP
 * device must be the one `stream` belongs to. Arguments, results and errors
 * are otherwise those of sfl_decode_attention.
 */
int sfl_decode_attention_static(const void* q, const void* k, const void* v, const int32_t* lengths,
                                void* out, int batch, int q_heads, int kv_heads, int capacity,
                                int head_dim, int splits, float scale, int kv_dtype, int q_dtype,
                                int out_dtype, void* stream);
long sfl_decode_attention_static_scratch_bytes(void);

/*
 * Decode attention fused with the output projection and residual add:
 *   x[b] += concat_h(attention(q[b, h], k[b, h], v[b, h])) @ w_out^T
 * for multi-head attention (Hq == Hkv == heads) with one split. Replaces
 * attention.py:187-203 (attention, head merge, output_proj) plus the residual
 * add of transformer.py:46 for one position; the softmax is that of
 * sfl_decode_attention. Each (batch, head) workgroup adds its head's share of
 * the projection to x with fp32 atomics, so the summation order varies from
 * call to call.
 *   q        [batch, heads, head_dim] fp32 (RoPE applied)
 *   k, v     [batch, heads, capacity, head_dim] in the model dtype (F32, BF16 or F16)
 *   lengths  [batch] int32; w_out: output_proj packed by sfl_pack_gemv_weights
 *   x        fp32 [batch, heads*head_dim], updated in place (16-byte aligned)
 * head_dim: a power of two in [32, 128] (bf16, fp16) or [16, 128] (fp32).
 */
int sfl_decode_attention_out_proj(const float* q, const void* k, const void* v,
                                  const int32_t* lengths, const void* w_out, float* x, int batch,
                                  int heads, int capacity, int head_dim, float scale, int dtype,
                                  void* stream);


/* ---- decode step of the llmlab decoder (model dtype F32, BF16 or F16) -----
 * One step processes one token per sequence for `batch` <= 65536 sequences.
 * The GEMVs run one workgroup per 16 output features and block of 16 batch
 * rows; the blocks of one weight tile share an XCD, so the weights stream
 * from HBM once per launch whatever the batch. x is the fp32 residual stream
 * [batch, d_model]; weights are the reference's [out, in] matrices in the
 * model dtype.
 */

/*
 * GEMV weights. The decode GEMVs read their [N, K] weights (the reference's
 * Linear layout, layers.py:34-35) repacked by sfl_pack_gemv_weights into
 * sfl_packed_gemv_elems(N, K) elements: for each tile of 16 rows and each K
 * chunk (KC = 32 bf16 or 16 fp32 values), 64 lanes x 16 bytes, lane
 * l = 16*g + r holding row r's values [c*KC + g*KC/4, c*KC + (g+1)*KC/4);
 * rows past N are zero.
 *
 * GEMV inputs. A plain input (the attention output, the SwiGLU hidden state)
 * is in the activation layout. A normalized input is the fp32 residual stream
 * x [batch, d_model] itself plus the RMSNorm gain g [d_model]: the consumer
 * computes RMSNorm(x) @ W^T as (x * g) @ W^T / sqrt(sum(x^2) / d_model + 1e-5)
 * (layers.py:133-141) while it reads x. x and g must be 16-byte aligned.
 * Producers of x only add to it (sfl_linear_residual,
 * sfl_decode_attention_out_proj) or overwrite it (sfl_next_token).
 */

/* Elements of a packed [n, k] GEMV weight, and the packing itself (w and
 * packed 16-byte aligned, k a multiple of the chunk size). */
long sfl_packed_gemv_elems(int n, int k);
int sfl_pack_gemv_weights(const void* w, void* packed, int n, int k, int dtype, void* stream);

/*
 * q/k/v projections of RMSNorm(x) with RoPE and the KV-cache append.
 * Replaces, for one position, TransformerBlock's attn_norm + q/k/v_proj + RoPE
 * (src/llmlab/model/transformer.py:46, layers.py:133-141,
 * attention.py:160-185); the reference recomputes K/V for every position.
 *   x, gain  the fp32 residual stream [batch, d_model] and attn_norm's weight
 *   w_qkv    packed [3*d_model, d_model]: q_proj, k_proj, v_proj rows stacked
 *   cos_t, sin_t [capacity, head_dim/2] fp32 (the table of attention.py:31-42)
 *   pos      [batch] int32 position of this token; k/v are written at pos[b]
 *   q_out    [batch, heads, head_dim] fp32; k_cache, v_cache [batch, heads, capacity, head_dim]
 */
int sfl_rmsnorm_qkv_rope_append(const float* x, const void* gain, const void* w_qkv,
                                const float* cos_t, const float* sin_t, const int32_t* pos,
                                void* q_out, void* k_cache, void* v_cache, int batch,
                                int d_model, int heads, int capacity, int dtype, void* stream);

/*
 * x += act @ w^T in place (act [batch, k] in the activation layout; w packed
 * [n, k]; x fp32 [batch, n], 16-byte aligned). Replaces output_proj + residual
 * and ffn.w2 + residual (transformer.py:46-47, attention.py:199-203,
 * layers.py:114-115). ksplit in [1, 16] workgroups share each 16-row tile
 * along K: with ksplit > 1 they add their partial sums to x with fp32 atomics
 * (more workgroups for small n; the summation order then varies from call to
 * call); ksplit = 1 is deterministic.
 */
int sfl_linear_residual(const void* act, const void* w, float* x, int batch, int n, int k,
                        int ksplit, int dtype, void* stream);

/*
 * h = silu(RMSNorm(x) @ w1^T) * (RMSNorm(x) @ w3^T), h [batch, d_ff] in the
 * activation layout. x, gain: the residual stream and ffn_norm's weight;
 * w1, w3 packed [d_ff, d_model].
 * Replaces ffn_norm + SwiGLU's w1/w3 half (transformer.py:47, layers.py:73-115).
 */
int sfl_rmsnorm_swiglu(const float* x, const void* gain, const void* w1, const void* w3,
                       void* h_out, int batch, int d_model, int d_ff, int dtype, void* stream);

/*
 * logits = RMSNorm(x) @ w_head^T plus a per-tile argmax (lowest index on ties).
 * Replaces ln_final + lm_head (transformer.py:137-138) for the last position.
 *   x, gain  the residual stream and ln_final's weight; w_head packed [vocab, d_model]
 *   logits   optional [.., vocab] fp32; row b is written at
 *            logits + b*logits_batch_stride + pos[b]*logits_pos_stride (pos may be NULL)
 *   best_val, best_idx [sfl_lm_head_tiles(vocab), best_stride]: the tile maxima
 */
int sfl_rmsnorm_lm_head(const float* x, const void* gain, const void* w_head, void* logits,
                        long logits_batch_stride, const int32_t* pos, long logits_pos_stride,
                        float* best_val, int32_t* best_idx, int best_stride, int batch,
                        int d_model, int vocab, int dtype, void* stream);

/* Number of lm_head tiles (rows of best_val/best_idx) for a vocabulary size. */
int sfl_lm_head_tiles(int vocab);

/*
 * x[b] = emb[tokens[b*token_stride + pos[b]]] in fp32 (Embedding.forward, layers.py:68-70).
 * Token ids must lie in [0, vocab): the library does not know vocab and does
 * not check them (the Python layer rejects out-of-range ids, as the
 * reference's nn.Embedding lookup raises).
 */
int sfl_embedding_gather(const int64_t* tokens, long token_stride, const int32_t* pos,
                         const void* emb, float* x, int batch, int d_model, int dtype,
                         void* stream);

/*
 * Greedy step: argmax over the lm_head tiles (first maximal index, as
 * torch.argmax) -- best_val/best_idx [tiles, best_stride] as sfl_rmsnorm_lm_head
 * wrote them, with the same best_stride (>= batch) -- then, with np = pos[b] + 1: predicted[b, np] = argmax;
 * tokens[b, np] = argmax unless np < prompt_len[b] (the prompt token is kept);
 * x[b] = emb[tokens[b, np]] (fp32, d_model % 16 == 0); pos[b] = np; lengths[b] = np + 1.
 * Nothing changes for a row whose np would reach capacity. The reference has
 * no token loop; its greedy continuation is argmax(TransformerLM.forward(ids)[:, -1]).
 */
int sfl_next_token(const float* best_val, const int32_t* best_idx, int tiles, int best_stride, int64_t* tokens,
                   int64_t* predicted, long token_stride, const int32_t* prompt_len, int32_t* pos,
                   int32_t* lengths, const void* emb, float* x, int batch, int d_model,
                   int capacity, int dtype, void* stream);

/* ---- masked prefill attention ----------------------------------------------
 * Replaces attention_lab/triton_attention.py `attention` (:326-438) and its
 * kernels interval_attention_forward (:209-321) and csr_attention_forward
 * (:126-197), bound by the Python wrapper at :389-435.
 *
 *   q, k, v, o   [B, H, N, D] bf16/fp16 addressed by per-tensor strides
 *                {batch, head, sequence} in elements (D contiguous; row
 *                strides multiple of 8 for q/k/v, of 4 for o)
 *   lse          optional fp32 [B, H, N]: natural-log row normalizers,
 *                -inf (with a zero output row) where no key is admissible
 *   scale        score scale (the reference uses D^-0.5)
 *   mask         causal; window_left / window_right (< 0: unbounded);
 *                global_prefix: keys k < prefix pass the windows (not
 *                causality or documents); document_ids int64 [N] or NULL
 *   schedule     mode 0: interval bounds derived on the device (no
 *                documents); mode 1: CSR over 64-row query tiles of 64-key
 *                tiles, row_ptr int32 [ceil(N/64)+1], col_idx int32, full
 *                uint8 (1 = no elementwise mask needed)
 *   use_full_blocks 0 applies the elementwise mask to every tile
 * Tiles are 64 x 64 (sfl_masked_attention_block()). D in {32, 64, 128}.
 */
int sfl_masked_attention(const void* q, const void* k, const void* v, void* o, float* lse,
                         int batch, int heads, int n, int head_dim, const long* q_strides,
                         const long* k_strides, const long* v_strides, const long* o_strides,
                         float scale, int causal, int window_left, int window_right,
                         int global_prefix, const int64_t* document_ids, int schedule_mode,
                         const int32_t* row_ptr, const int32_t* col_idx,
                         const uint8_t* full_blocks, int use_full_blocks, int dtype, void* stream);

/* Query/key tile size of sfl_masked_attention (64). */
int sfl_masked_attention_block(void);

/* Compiler resource data of a kernel (hipFuncGetAttributes), not a profiler measurement. */
typedef struct {
  char name[96];             /* kernel and element type */
  int registers;             /* VGPRs per lane */
  int private_bytes;         /* scratch per lane: register spills (0 = none) */
  int shared_bytes;          /* static LDS per workgroup */
  int max_threads;           /* largest workgroup the code object allows */
  int threads;               /* workgroup size of the launch */
  int queries_per_workgroup; /* query rows one workgroup covers */
} sfl_kernel_info;

/*
 * The kernel sfl_masked_attention launches for this head dim, dtype, sequence
 * length and K/V row strides (elements), with its resource data. Replaces the
 * Triton CompiledKernel metadata the reference records when its caller passes
 * `launch_metadata` (attention_lab/triton_attention.py:39-57,
 * launch_metadata at :326-328). Needs a HIP device; launches nothing.
 */
int sfl_masked_attention_kernel_info(int head_dim, int dtype, int n, long k_row_stride,
                                     long v_row_stride, int causal, int window_left,
                                     int window_right, int global_prefix, sfl_kernel_info* info);

/* ---- prefill (weights in bf16, fp16 or fp32) ---------------------------------
 * C^T = W A^T on MFMAs; A [M, K] row-major (one row per token) and W [N, K]
 * of one type `dtype`: SFL_DTYPE_BF16 or SFL_DTYPE_F16 (16-bit MFMAs; every
 * 16-bit output of these calls has that type too; K % 8 == 0; K % 64 == 0 runs
 * 32x32x16 MFMA tiles of 256 x 384 (grids of >= 320 such tiles) or 128 x 128
 * features x tokens, other K the 16x16x32 kernel on 128 x 128 tiles), or, for
 * sfl_gemm, sfl_gemm_qkv_rope and sfl_gemm_swiglu, SFL_DTYPE_F32 (fp32
 * v_mfma_f32_32x32x2_f32 on 64 x 64 tiles: fp32 products and sums, every
 * output fp32, K % 4 == 0, 16-byte aligned operands and outputs).
 * Replace, for a whole prompt, the Linear layers of one TransformerBlock and
 * the lm_head (src/llmlab/model/layers.py:34-35, attention.py:160-162,199-203,
 * layers.py:114-115, transformer.py:137-138).
 */

/* C = A W^T as fp32 (c_dtype F32; accumulate = 1 adds into C: the residual
 * update) or in the input type (c_dtype == dtype). */
int sfl_gemm(const void* a, const void* w, void* c, int m, int n, int k, int dtype, int c_dtype,
             int accumulate, void* stream);

/* q/k/v = A W_qkv^T with RoPE at position (row % seq) from the fp32 tables
 * cos_t / sin_t in feature-major layout [head_dim / 2, capacity] (the
 * reference's [positions, head_dim / 2] table of attention.py:31-42
 * transposed: lanes holding consecutive tokens read consecutive floats);
 * q to [m/seq, heads, seq, head_dim], k/v written at positions 0..seq-1
 * of the [m/seq, heads, capacity, head_dim] cache. */
int sfl_gemm_qkv_rope(const void* a, const void* w_qkv, int m, int seq, int d_model, int heads,
                      const float* cos_t, const float* sin_t, void* q_out, void* k_cache,
                      void* v_cache, int capacity, int dtype, void* stream);

/* h = silu(A W1^T) * (A W3^T) as [m, d_ff]; w13_interleaved [2*d_ff, k]
 * holds 8 rows of W1 then the same 8 rows of W3, repeatedly. */
int sfl_gemm_swiglu(const void* a, const void* w13_interleaved, void* h_out, int m, int d_ff, int k,
                    int dtype, void* stream);

/* Causal attention of a whole prompt in fp32 (attention.py:61-98 with the
 * causal mask of :187-197), for the prefill of float32 models: q, k, v, o
 * [B, H, N, D] fp32 addressed by per-tensor strides {batch, head, sequence}
 * (elements; D contiguous; k, v and o rows 16-byte aligned), o = softmax(q k^T
 * * scale) v over keys 0..i for query i, every product and sum in fp32.
 * D in {16, 32, 64, 128}. */
int sfl_causal_attention_f32(const float* q, const float* k, const float* v, float* o, int batch, int heads,
                             int n, int head_dim, const long* q_strides, const long* k_strides,
                             const long* v_strides, const long* o_strides, float scale, void* stream);

/* x[r] = emb[ids[r]] in fp32 for r < m (Embedding.forward, layers.py:68-70);
 * emb F32, BF16 or F16; ids in [0, vocab), unchecked as for sfl_embedding_gather. */
int sfl_embed_rows(const int64_t* ids, const void* emb, float* x, int m, int d_model, int dtype,
                   void* stream);

/* out[r] = RMSNorm(x[r]) * w for r < m (layers.py:133-141), rounded once to
 * out_dtype; (w dtype, out_dtype) is (BF16, BF16), (F32, BF16), (F16, F16)
 * or (F32, F32). */
int sfl_rmsnorm_rows(const float* x, const void* w, void* out, int m, int d_model, int dtype,
                     int out_dtype, void* stream);

/* ---- prefill with the RMSNorm folded into the neighbouring GEMMs -------------
 * RMSNorm(x) W^T = (1 / rms(x)) ((x * w) W^T) per token: the norm's input side
 * is xg = T(x * w) plus a per-token scale r = 1 / rms(x) that the consuming
 * GEMM applies to its fp32 products, and the residual GEMM producing x writes
 * xg for the next norm and per-token sums of squares over each 128-feature
 * part, so no separate pass re-reads x. Same layers as above (layers.py:133-141
 * feeding attention.py:160-162 and layers.py:114-115); T = bf16 or fp16 as
 * `dtype` says, d_model and d_ff multiples of 64 (the 32x32 MFMA kernels).
 */

/* act_xg[r] = T(x[r] * w), rscale[r] = 1 / sqrt(mean(x[r]^2) + 1e-5); w of
 * type `dtype` (BF16 or F16), d_model <= 2048. */
int sfl_rmsnorm_rows_scaled(const float* x, const void* w, void* act_xg, float* rscale, int m, int d_model,
                            int dtype, void* stream);

/* x += A W^T (fp32, as sfl_gemm with accumulate) and, from the updated
 * x: act_xg = T(x * gain_next) and ss_parts[p][r] = sum of x[r][f]^2 over
 * the features f of part p = f / 128 (ceil(n / 128) parts). n % 4 == 0.
 * act_xg must not overlap a (other workgroups may still be reading A while
 * one writes its outputs); each part's sum has a fixed order, so results are
 * the same from call to call. */
int sfl_gemm_residual_norm(const void* a, const void* w, float* x, int m, int n, int k, const void* gain_next,
                           void* act_xg, float* ss_parts, int dtype, void* stream);

/* rscale[r] = 1 / sqrt(sum_p ss_parts[p][r] / d_model + 1e-5), parts summed in order. */
int sfl_norm_scale(const float* ss_parts, int parts, int m, int d_model, float* rscale, void* stream);

/* sfl_gemm_qkv_rope on act_xg (same feature-major tables), each token's
 * products scaled by rscale[r] before RoPE and the 16-bit stores. */
int sfl_gemm_qkv_rope_scaled(const void* a_xg, const void* w_qkv, const float* rscale, int m, int seq,
                             int d_model, int heads, const float* cos_t, const float* sin_t, void* q_out,
                             void* k_cache, void* v_cache, int capacity, int dtype, void* stream);

/* sfl_gemm_swiglu on act_xg, both products of a token scaled by rscale[r]
 * before silu(.) * (.). */
int sfl_gemm_swiglu_scaled(const void* a_xg, const void* w13_interleaved, const float* rscale, void* h_out,
                           int m, int d_ff, int k, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SFL_H_ */
