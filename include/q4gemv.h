/* C-ABI of the MI355X (gfx950) int4 GEMV library, libq4gemv.so.
 *
 * Weight layout (MLX 4-bit, the reference's kernel/q4gemv.c:7-11):
 *   w       [n_out][n_in/8]   uint32, eight 4-bit values each, low nibble first
 *   scales  [n_out][n_in/gs]  fp16 bit patterns
 *   biases  [n_out][n_in/gs]  fp16 bit patterns
 *   value = q * scale + bias
 *
 * Return codes: 0 success; -1 invalid shape, for exactly the conditions the
 * reference rejects (kernel/q4gemv.c:237, :361), plus gs <= 0; Q4_EHIP a HIP
 * runtime error (no device, launch failure); Q4_ENOMEM device or pinned
 * memory exhausted; Q4_EARG a null pointer, a misaligned device pointer or
 * a size the library does not take.  q4_last_error() describes the last
 * failure of the calling thread.
 *
 * Results: q4_gemv reproduces the reference's x86 arithmetic bit for bit
 * (x quantised to int16 once per call, exact integer dot per group, groups
 * accumulated in ascending order as acc + fma(scale, xscale*dot, bias*xsum)),
 * i.e. the reference built with ROWS=1 -- and with any ROWS when
 * n_out % ROWS == 0.  To replace a build tuned to another ROWS (its
 * kernel/tuning.json "rows"), set HETERO_Q4_ROWS=<rows> (read on first use)
 * or call q4_set_rows: the last n_out % ROWS rows of each matrix then take
 * the reference's fp32 tail path (kernel/q4gemv.c:185-200), in q4_gemv,
 * q4_gemv_batched, q4_gemv_dev, q4_gemv_noalloc_dev and q4_gemv_multi_dev.
 * The fused and chained entry points (gate/up SiLU, MLP, norm prologue,
 * chained programs) always compute every row by the integer path.
 */
#ifndef HETERO_AMD_Q4GEMV_H
#define HETERO_AMD_Q4GEMV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q4_EHIP   (-2)
#define Q4_ENOMEM (-3)
#define Q4_EARG   (-4)

/* ---- drop-in entry points: host pointers, synchronous ------------------- */

/* y = W x for one activation row.  Replaces q4_gemv of the reference,
 * kernel/q4gemv.c:232-233, bound by hetero/cpu_model.py:41-42 as
 * [c_void_p]*5 + [c_int]*4 -> c_int.  All pointers are host addresses.
 * w/scales/biases are uploaded to HBM on first use and kept resident, keyed
 * by their host addresses and shape.  Every call checks them against a
 * fingerprint: 16 sampled words per array by default, so a caller that
 * edits registered weights in place calls q4_release first; with the
 * environment variable Q4_RESIDENCY_CHECK=full, a hash of every byte (an
 * edit anywhere is re-uploaded, as the reference reads host memory on every
 * call, at the cost of one host read of the weights per call).  nthreads is
 * accepted and ignored.  Returns after out[0..n_out) is written. */
int q4_gemv(const uint32_t *w, const uint16_t *scales, const uint16_t *biases,
            const float *x, float *out, int n_out, int n_in, int gs, int nthreads);

/* Rows [row0,row1) of W expanded to fp32, out[(o-row0)*n_in + i] =
 * fma(q, scale, bias).  Replaces q4_dequant, kernel/q4gemv.c:359-360, bound
 * by hetero/cpu_model.py:43-44 as [c_void_p]*4 + [c_int]*5 -> c_int.
 * w/scales/biases are whole-matrix host bases (resident as for q4_gemv);
 * out is a host buffer of (row1-row0)*n_in floats.  Returns 0 without
 * touching out when row1 <= row0. */
int q4_dequant(const uint32_t *w, const uint16_t *scales, const uint16_t *biases,
               float *out, int row0, int row1, int n_in, int gs, int nthreads);

/* m activation rows x[m][n_in] -> out[m][n_out], each row bit-identical to
 * q4_gemv on that row; the weights are read once for all rows.  No
 * counterpart in the reference: it replaces the row-by-row loop of
 * hetero/cpu_model.py:149-153 (QLinear.__call__ for 1 < rows <= 16).  Host
 * pointers, synchronous, same residency rules as q4_gemv. */
int q4_gemv_batched(const uint32_t *w, const uint16_t *scales, const uint16_t *biases,
                    const float *x, float *out, int m, int n_out, int n_in, int gs,
                    int nthreads);

/* Drop the HBM copies registered for host weights at address w (every
 * shape, and every row block q4_dequant registered for the matrix whose
 * base is w); q4_release_all drops every registered matrix on every device.
 * Return the number of entries released. */
int q4_release(const void *w);
int q4_release_all(void);

/* Text of the calling thread's last failure ("" if none). */
const char *q4_last_error(void);

/* ---- device-pointer entry points: asynchronous on `stream` --------------
 * All pointers are device addresses on the current HIP device; `stream` is a
 * hipStream_t (NULL = the null stream).  w must be 16-byte aligned.  Calls
 * that share a device and overlap in time must be issued on one stream: the
 * per-stream x workspace is reused by the next call on that stream. */

/* Batched GEMV over m rows (any m >= 1; rows are processed eight at a time).
 * Same arithmetic as q4_gemv.  x is [m][n_in], out is [m][n_out].  Blocks of
 * 3..8 rows with gs 64 run their integer dots on the int8 matrix cores, with
 * x quantised into the per-stream workspace first; the workspace grows on
 * first use, so run the largest call once on a stream before capturing it
 * in a graph. */
int q4_gemv_dev(const uint32_t *w, const uint16_t *scales, const uint16_t *biases,
                const float *x, float *out, int m, int n_out, int n_in, int gs,
                void *stream);

/* q4_gemv_dev for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  Same arguments, arithmetic and results as
 * q4_gemv_dev, but every scratch buffer (the x planes, group sums and row
 * scales of blocks of 3..8 rows and of group sizes other than 64) is a fixed
 * array in device memory, one per GPU, held until the process ends; the call
 * makes no hipMalloc/hipFree.  Limit: n_in <= 32768 (larger n_in returns
 * Q4_EARG).  Every call on one GPU shares that GPU's array: calls that
 * overlap in time on one GPU (other streams, other threads) race. */
int q4_gemv_noalloc_dev(const uint32_t *w, const uint16_t *scales, const uint16_t *biases,
                        const float *x, float *out, int m, int n_out, int n_in, int gs,
                        void *stream);

/* Up to four matrices that share the activations x (q/k/v, gate/up) in one
 * launch (1..2 rows; 3..8 rows: x quantised once, then one matrix-core launch
 * per matrix): out[k] is [m][n_out[k]] = W_k x, each row bit-identical to
 * q4_gemv.
 * w, scales, biases, out and n_out are host arrays of `count` device
 * pointers / sizes.  No counterpart in the reference, whose caller makes one
 * q4_gemv call per projection (hetero/cpu_model.py:269-275, :291-292). */
int q4_gemv_multi_dev(int count, const uint32_t *const *w, const uint16_t *const *scales,
                      const uint16_t *const *biases, float *const *out, const int *n_out,
                      const float *x, int m, int n_in, int gs, void *stream);

/* Fused gate/up projection with SiLU * mul: h[m][n_inter] =
 * SiLU(W_gate x) * (W_up x), SiLU(g) = g / (1 + exp(-g)) in fp32.  The gate
 * and up rows are the q4_gemv results bit for bit; exp may differ from
 * NumPy's float32 exp in the last place.  Replaces the first half of
 * MLP.__call__, hetero/cpu_model.py:291-292 (two q4_gemv calls and the NumPy
 * silu of :169-170).  Device pointers, asynchronous on `stream`. */
int q4_gate_up_silu_dev(const uint32_t *gate_w, const uint16_t *gate_s, const uint16_t *gate_b,
                        const uint32_t *up_w, const uint16_t *up_s, const uint16_t *up_b,
                        const float *x, float *h, int m, int n_inter, int n_in, int gs,
                        void *stream);

/* The whole MLP block, hetero/cpu_model.py:291-292:
 * out[m][n_hidden] = W_down (SiLU(W_gate x) * W_up x), with h[m][n_inter]
 * as caller-provided scratch (it holds the SiLU * mul activations on
 * return).  Two launches: the fused gate/up/SiLU one and the down GEMV. */
int q4_mlp_dev(const uint32_t *gate_w, const uint16_t *gate_s, const uint16_t *gate_b,
               const uint32_t *up_w, const uint16_t *up_s, const uint16_t *up_b,
               const uint32_t *down_w, const uint16_t *down_s, const uint16_t *down_b,
               const float *x, float *h, float *out, int m, int n_hidden, int n_inter, int gs,
               void *stream);

/* Prefill contraction out[m][n_out] = x[m][n_in] . W^T for prompts (m >
 * 16 rows): W dequantised to bf16 inside the tile load (the value of
 * q4_dequant_bf16_dev), x rounded to bf16, fp32 accumulation on the matrix
 * cores (v_mfma_f32_32x32x16_bf16).  Replaces QLinear._gemm,
 * hetero/cpu_model.py:119-136 (512-row q4_dequant blocks + an fp32 BLAS
 * sgemm); the result differs from it by bf16 rounding of both operands.
 * gs must be 64; w and x 16-byte aligned.  Uses a per-stream workspace (the
 * bf16 copy of x and, when K is split over workgroups, the partial sums)
 * that grows on first use: run the largest call once on a stream before
 * capturing it in a graph. */
int q4_gemm_bf16_dev(const uint32_t *w, const uint16_t *scales, const uint16_t *biases,
                     const float *x, float *out, int m, int n_out, int n_in, int gs,
                     void *stream);

/* Up to four prefill contractions that share x (q/k/v, gate/up) in one
 * launch: out[k] is [m][n_out[k]] = x . W_k^T, each as q4_gemm_bf16_dev
 * computes it (the tiling may differ, so the fp32 sums may differ from a
 * separate call's in the last place).  x is rounded to bf16 once, and the
 * matrices' 256-column tile blocks share one tile space, so small matrices
 * fill the CUs together.  w, scales, biases, out and n_out are host arrays
 * of `count` device pointers / sizes.  No counterpart in the reference,
 * whose caller makes one QLinear._gemm call per projection
 * (hetero/cpu_model.py:119-136, :269-275, :291-292). */
int q4_gemm_bf16_multi_dev(int count, const uint32_t *const *w, const uint16_t *const *scales,
                           const uint16_t *const *biases, float *const *out, const int *n_out,
                           const float *x, int m, int n_in, int gs, void *stream);

/* q4_gemm_bf16_multi_dev with x given as bf16 bit patterns [m][n_in] (16-byte
 * aligned): the call skips its own rounding of x, so for x = bf16(x32)
 * (nearest even) the outputs are those of q4_gemm_bf16_multi_dev on x32, bit
 * for bit.  For producers that write bf16 (q4_add_rmsnorm_rows_bf16_dev,
 * q4_prompt_attention_bf16_dev, q4_gemm_bf16in_gate_up_silu_dev).  Same
 * reference contraction: hetero/cpu_model.py:119-136. */
int q4_gemm_bf16in_multi_dev(int count, const uint32_t *const *w, const uint16_t *const *scales,
                             const uint16_t *const *biases, float *const *out, const int *n_out,
                             const uint16_t *xb, int m, int n_in, int gs, void *stream);

/* The prompt's MLP activations from bf16 x [m][n_in] (hetero/cpu_model.py:
 * 149-153 and :169-170 with both projections as QLinear._gemm, :119-136):
 * h[m][n_inter] = bf16(SiLU(x . Wg^T) * (x . Wu^T)) as bf16 bit patterns,
 * rounded to nearest even -- the down projection's operand.  One launch:
 * each tile holds the same 128 rows of both matrices, so the SiLU * mul is
 * the GEMM's epilogue.  While the 256 x 128 output tiles fit the CUs in
 * one round, each tile is one workgroup and the fp32 sums are those of
 * q4_gemm_bf16in_multi_dev on {gate, up} without split-K (bit for bit);
 * past that (a 512-token prompt at n_inter 18944 has 296 tiles) the tiles'
 * K steps are shared out stream-K over one workgroup per CU and a tile's
 * partial sums are added in a fixed order, which may move a value by one
 * bf16 unit.  Q4_PAIR_PLAN=dp or sk:<P> forces either form.  gs must be
 * 64; w and x 16-byte aligned.  The stream-K form uses the calling
 * stream's workspace, which grows on first use (run the largest call once
 * before capturing it in a graph). */
int q4_gemm_bf16in_gate_up_silu_dev(const uint32_t *gate_w, const uint16_t *gate_s, const uint16_t *gate_b,
                                    const uint32_t *up_w, const uint16_t *up_s, const uint16_t *up_b,
                                    const uint16_t *xb, uint16_t *h, int m, int n_inter, int n_in, int gs,
                                    void *stream);

/* Set the reference ROWS whose tail rows the plain GEMV entry points
 * reproduce (1..64; 1 = every row by the integer path).  Returns the
 * previous setting, or Q4_EARG.  No counterpart in the reference's ABI: the
 * reference fixes ROWS when it is built (kernel/build.sh:7, -DROWS) and its
 * autotuner picks it (kernel/autotune.py:52-63).  Affects later calls only;
 * not to be changed while calls run on other threads. */
int q4_set_rows(int rows);

/* Synchronise `stream` and return how many stream-K partial sums of the
 * prefill calls on it did not arrive within their bounded wait since the
 * last call (0 in a correct run; each such tile was stored as NaN), then
 * clear the count.  No counterpart in the reference: its prefill is one
 * BLAS call (hetero/cpu_model.py:135), which cannot time out. */
int q4_prefill_errors(void *stream);

/* Device q4_dequant: rows [row0,row1) to fp32 [row1-row0][n_in]. */
int q4_dequant_dev(const uint32_t *w, const uint16_t *scales, const uint16_t *biases,
                   float *out, int row0, int row1, int n_in, int gs, void *stream);

/* Rows [row0,row1) to bf16 bit patterns [row1-row0][n_in]: the fp32 value
 * of q4_dequant rounded to nearest even. */
int q4_dequant_bf16_dev(const uint32_t *w, const uint16_t *scales, const uint16_t *biases,
                        uint16_t *out, int row0, int row1, int n_in, int gs, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* HETERO_AMD_Q4GEMV_H */
