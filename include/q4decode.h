/* Decode-step kernels of the device-resident Qwen2 stage on MI355X (gfx950).
 *
 * These are the device counterparts of the NumPy operations around the int4
 * GEMVs in the reference stage (hetero/cpu_model.py).  The reference runs them
 * on the host; here they run on the GPU so that a whole decode step is one
 * HIP graph replay with every tensor resident in HBM.  They have no
 * counterpart in the reference's kernel ABI (kernel/q4gemv.c), so they sit in
 * a header of their own.
 *
 * All pointers are device pointers; every call is asynchronous on `stream`
 * (a hipStream_t, NULL = the null stream) and capturable in a HIP graph (no
 * allocation, no memset).  The decode position and the token live in device
 * memory (int64), so a captured step is position-independent.
 *
 * Return codes as in q4gemv.h: 0 success, Q4_EHIP, Q4_EARG (text in
 * q4_last_error()).
 */
#ifndef Q4DECODE_H
#define Q4DECODE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Embedding row of token *tok (clamped into [0, n_rows)) dequantised to fp32:
 * out[i] = fma(q, scale, bias) of row *tok of the packed table, as
 * hetero/cpu_model.py:334-338 (Stage.embed) and :67-81 (dequantize) compute
 * it.  w [n_rows][n_in/8], scales/biases fp16 [n_rows][n_in/gs]. */
int q4_embed_dev(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, const int64_t* tok,
                 float* out, int n_rows, int n_in, int gs, void* stream);

/* q4_embed_dev for n_ids tokens: row i of out [n_ids][n_in] is the
 * embedding of ids[i] (hetero/cpu_model.py:334-338 over a prompt's token
 * ids).  n_ids <= 65535. */
int q4_embed_rows_dev(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, const int64_t* ids,
                      int n_ids, float* out, int n_rows, int n_in, int gs, void* stream);

/* Residual add and RMSNorm (hetero/cpu_model.py:164-166 rms_norm, :304-306
 * the residual adds of DecoderLayer): if delta is not NULL, x += delta
 * (in place); then y = x * (1 / sqrt(mean(x*x) + eps)) * w.  n <= 8192. */
int q4_add_rmsnorm_dev(float* x, const float* delta, const float* w, float eps, float* y, int n,
                       void* stream);

/* q4_add_rmsnorm_dev on each row of x, delta, y [rows][n] (the prompt's
 * rows, hetero/cpu_model.py:304-306 with L > 1); row i gives the bits
 * q4_add_rmsnorm_dev gives for that row alone. */
int q4_add_rmsnorm_rows_dev(float* x, const float* delta, const float* w, float eps, float* y, int rows, int n,
                            void* stream);

/* q4_add_rmsnorm_rows_dev with y stored as bf16 bit patterns, each value
 * rounded to nearest even: the x operand the prefill GEMM would round it to
 * (q4_gemm_bf16in_multi_dev, q4_gemm_bf16in_gate_up_silu_dev), written by
 * the norm instead of a separate conversion.  x, delta and w as there. */
int q4_add_rmsnorm_rows_bf16_dev(float* x, const float* delta, const float* w, float eps, uint16_t* y, int rows,
                                 int n, void* stream);

/* The GEMVs that follow a residual add + RMSNorm, with the norm folded into
 * their prologue (every workgroup normalises the input itself, so the
 * separate q4_add_rmsnorm_dev launch goes away):
 *   xs = x + delta (x alone when delta is NULL),
 *   input = xs * (1 / sqrt(mean(xs*xs) + eps)) * norm_w  -- the bits of
 *     q4_add_rmsnorm_dev's y for the same x, delta, norm_w, eps;
 *   x_out (may be NULL; written only when delta is not NULL) receives xs, so a
 *     caller alternates two residual buffers instead of updating x in place.
 * One activation row; gs 64; 64 <= n_in <= 8192; x, delta, norm_w, x_out
 * 16-byte aligned, x_out overlapping neither x nor delta.
 * q4_norm_gemv_multi_dev: out[k] = W_k input as q4_gemv_multi_dev computes
 * it (the q/k/v projections after input_layernorm, hetero/cpu_model.py:305
 * and :271-273; lm_head after the final norm, :355 and :367).
 * q4_norm_gate_up_silu_dev: h = SiLU(W_gate input) * (W_up input) as
 * q4_gate_up_silu_dev computes it (the MLP after post_attention_layernorm,
 * :306 and :292). */
int q4_norm_gemv_multi_dev(int count, const uint32_t* const* w, const uint16_t* const* scales,
                           const uint16_t* const* biases, float* const* out, const int* n_out, const float* x,
                           const float* delta, const float* norm_w, float eps, float* x_out, int n_in, int gs,
                           void* stream);
int q4_norm_gate_up_silu_dev(const uint32_t* gate_w, const uint16_t* gate_s, const uint16_t* gate_b,
                             const uint32_t* up_w, const uint16_t* up_s, const uint16_t* up_b, const float* x,
                             const float* delta, const float* norm_w, float eps, float* x_out, float* h,
                             int n_inter, int n_in, int gs, void* stream);

/* q/k/v projection biases, rotary embedding and the KV-cache write at the
 * position *pos (hetero/cpu_model.py:156-157 QLinear bias, :195-204 RoPE
 * non-traditional half split, :207-230 KVCache.update_and_fetch):
 *   q_out = rope(q + bias[0:nh*d]),  k = rope(k + bias[nh*d : (nh+nkv)*d]),
 *   v = v + bias[(nh+nkv)*d :]; k and v are stored as fp16 (round to nearest
 *   even) at [kv head][*pos][:] of k_cache / v_cache [nkv][cap][d].
 * cos_t / sin_t are the fp32 tables [cap][d/2] (angle = position * inv_freq).
 * Nothing is written when *pos is outside [0, cap). */
int q4_rope_kv_dev(const float* q, const float* k, const float* v, const float* bias, const float* cos_t,
                   const float* sin_t, const int64_t* pos, uint16_t* k_cache, uint16_t* v_cache,
                   float* q_out, int n_heads, int n_kv, int head_dim, int cap, void* stream);

/* q4_rope_kv_dev for the rows of a prompt chunk: row i of q [rows][nh*d],
 * k, v [rows][nkv*d] at position pos0 + i (hetero/cpu_model.py:195-204 with
 * offset = pos0, :216-230 storing L rows), written to q_out [rows][nh*d]
 * and the cache rows pos0 .. pos0 + rows - 1, which must lie in [0, cap).
 * Row i gives the bits q4_rope_kv_dev gives at that position.
 * rows <= 65535. */
int q4_rope_kv_rows_dev(const float* q, const float* k, const float* v, const float* bias, const float* cos_t,
                        const float* sin_t, int64_t pos0, int rows, uint16_t* k_cache, uint16_t* v_cache,
                        float* q_out, int n_heads, int n_kv, int head_dim, int cap, void* stream);

/* h[i] = SiLU(g[i]) * u[i] for i < n (hetero/cpu_model.py:169-170, :291-292),
 * the expression q4_gate_up_silu_dev applies to its two sums. */
int q4_silu_mul_dev(const float* g, const float* u, float* h, long n, void* stream);

/* Causal grouped-query attention of a prompt chunk (hetero/cpu_model.py:
 * 233-252 with causal=True and L > 1): query row i of q [rows][nh*d]
 * (rotated, q4_rope_kv_rows_dev) sits at position pos0 + i and attends to
 * the cache positions [0, pos0 + i], which the caller has written (the
 * chunk's own keys and values by q4_rope_kv_rows_dev first); out
 * [rows][nh*d].  The softmax is evaluated online over 64-position tiles, so
 * results agree with the reference's single max-and-sum to fp32 rounding.
 * head_dim 32, 64 or 128; at most 8 query heads per kv head;
 * pos0 + rows <= cap; q, out and the caches 16-byte aligned. */
int q4_prompt_attention_dev(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out, int rows,
                            int64_t pos0, int n_heads, int n_kv, int head_dim, int cap, float scale, void* stream);

/* q4_prompt_attention_dev with out stored as bf16 bit patterns (each value
 * rounded to nearest even), the x operand of the o projection's prefill
 * GEMM (q4_gemm_bf16in_multi_dev). */
int q4_prompt_attention_bf16_dev(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out,
                                 int rows, int64_t pos0, int n_heads, int n_kv, int head_dim, int cap, float scale,
                                 void* stream);

/* Floats of scratch memory q4_attention_dev needs for these sizes: the
 * chunks' partial results and, at the end, 512 arrival counters (one per
 * 128-byte line: 16384 floats), which must
 * be zero before the first call (allocate the scratch zeroed); every call
 * leaves them zero.  Calls that overlap in time on one scratch race. */
long q4_attention_scratch_floats(int n_heads, int head_dim, int cap);

/* Grouped-query attention of one query token over cache positions
 * [0, *pos] (hetero/cpu_model.py:233-252 sdpa: scores q.k * scale, softmax
 * with the maximum subtracted, weighted sum of v; query head h uses kv head
 * h / (n_heads / n_kv)).  q [n_heads][d] fp32, caches fp16 [nkv][cap][d],
 * out [n_heads][d] fp32.  One launch: the context is split in chunks of 64
 * positions (one workgroup per kv head and chunk) whose partial softmax
 * results go to scratch (q4_attention_scratch_floats); for each query
 * head, the last chunk to finish merges the head's parts.  head_dim 32, 64
 * or 128; at most 8 query heads per kv head, at most 512 query heads;
 * cap <= 65536. */
int q4_attention_dev(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, const int64_t* pos,
                     float* out, float* scratch, int n_heads, int n_kv, int head_dim, int cap, float scale,
                     void* stream);

/* q4_rope_kv_dev followed by q4_attention_dev, in the one launch of
 * q4_attention_dev: q, k, v are the raw projection outputs (fp32 [n_heads*d],
 * [n_kv*d], [n_kv*d]) and bias/cos_t/sin_t are as for q4_rope_kv_dev; the
 * workgroups apply bias and RoPE to the query heads they need, and the one
 * whose chunk holds *pos writes the new key and value rows to the cache and
 * uses them directly.  Results equal the two calls in sequence. */
int q4_attention_rope_dev(const float* q, const float* k, const float* v, const float* bias, const float* cos_t,
                          const float* sin_t, const int64_t* pos, uint16_t* k_cache, uint16_t* v_cache, float* out,
                          float* scratch, int n_heads, int n_kv, int head_dim, int cap, float scale, void* stream);

/* The final norm, the vocabulary projection and the greedy token in one
 * launch: logits as q4_norm_gemv_multi_dev computes them for the one matrix
 * (lm_head after the final norm, hetero/cpu_model.py:355 and :367), then
 * *tok, hist and *pos exactly as q4_argmax_dev(logits, n_out, ...) sets them
 * (hetero/backends.py:106-109).  Each workgroup reduces the rows it stored
 * and the last one to finish reduces those parts, through fixed arrays of
 * the library in device memory: 16 sets per GPU, one for each of the 16
 * streams that called it most recently on that GPU, so calls on different
 * streams do not share them (a call captured in a graph keeps the set of
 * the stream it was captured on; 17 or more streams calling it at once, or
 * such a graph replayed beside the stream's own calls, share sets and
 * race).  The same arguments as q4_norm_gemv_multi_dev with count 1, plus
 * q4_argmax_dev's. */
int q4_norm_gemv_argmax_dev(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, float* logits,
                            int n_out, const float* x, const float* delta, const float* norm_w, float eps,
                            float* x_out, int n_in, int gs, int64_t* tok, int64_t* hist, int64_t* pos, int64_t s0,
                            int hist_len, void* stream);

/* Greedy token (hetero/backends.py:106-109, NumpyBackend.sample: NumPy's
 * argmax, which takes NaN as the largest value -- the first NaN if there is
 * one, else the first index of the maximum) and the step's bookkeeping:
 * *tok = argmax, hist[*pos - s0] = *tok when that index is in [0, hist_len),
 * *pos += 1.  Two launches; the per-slice maxima go through a fixed array
 * of the library in device memory, one set per stream as for
 * q4_norm_gemv_argmax_dev. */
int q4_argmax_dev(const float* logits, int n, int64_t* tok, int64_t* hist, int64_t* pos, int64_t s0,
                  int hist_len, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* Q4DECODE_H */
