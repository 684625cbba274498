// Decode-step kernels of the device-resident Qwen2 stage (gfx950): the
// operations around the int4 GEMVs that the reference's NumPy stage
// (hetero/cpu_model.py) runs on the host.  Declared in q4decode.h.
//
// Elementwise fp32 arithmetic follows the reference's expression order with
// -ffp-contract=off (explicit _rn operations), so RoPE and the bias adds give
// the NumPy bits; the reductions (RMSNorm's mean, the softmax sums, the
// attention dot products) are tree reductions, not NumPy's pairwise order.
#include <mutex>

#include "q4_attn.h"
#include "q4_common.h"
#include "q4decode.h"

namespace q4k {
namespace {

__device__ __forceinline__ uint16_t f2h_rne(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

__device__ __forceinline__ float h2f_bits(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// ------------------------------------------------------------ embedding ---
// hetero/cpu_model.py:334-338 (Stage.embed) / :67-81 (dequantize):
// value 8j+n of the row = q * scale + bias with q * scale exact, so one fma.
// Token blockIdx.y of tok[] into row blockIdx.y of out.
__global__ __launch_bounds__(256) void embed_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ sc,
                                                    const uint16_t* __restrict__ bi, const int64_t* __restrict__ tok,
                                                    float* __restrict__ out, int n_rows, int n_in, int gs) {
    const int wpr = n_in >> 3, G = n_in / gs;
    const int64_t t = tok[blockIdx.y];
    out += static_cast<size_t>(blockIdx.y) * n_in;
    const int row = (t >= 0 && t < n_rows) ? static_cast<int>(t) : (t < 0 ? 0 : n_rows - 1);
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= wpr) return;
    const uint32_t word = w[static_cast<size_t>(row) * wpr + j];
    const size_t si = static_cast<size_t>(row) * G + (8 * j) / gs;
    const float s = h2f_bits(sc[si]), b = h2f_bits(bi[si]);
    float v[8];
#pragma unroll
    for (int n = 0; n < 8; n++) v[n] = __builtin_fmaf(static_cast<float>((word >> (4 * n)) & 0xFu), s, b);
    float4* o4 = reinterpret_cast<float4*>(out + 8 * static_cast<size_t>(j));
    o4[0] = make_float4(v[0], v[1], v[2], v[3]);
    o4[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// ------------------------------------------------ residual add + RMSNorm ---
// hetero/cpu_model.py:164-166: x * (1 / sqrt(mean(x * x) + eps)) * w, after
// the residual add of :304-306.  One workgroup per row (blockIdx.x of
// [rows][n]); n <= 8 * 1024.  Thread t owns the 8 consecutive values of
// word t; the squares are summed in NumPy's order (row_sum_numpy), and the
// streaming GEMV's norm prologue sums them the same way, so its input is y
// bit for bit.  VEC (n a multiple of 8, 16-byte aligned rows): the words
// move as two 16-byte accesses.  BF: y is stored rounded to bf16 (nearest
// even), the operand the prefill GEMM reads.
constexpr int kNormPer = 8;
template <bool VEC, bool BF>
__global__ __launch_bounds__(1024) void add_rmsnorm_kernel(float* __restrict__ x, const float* __restrict__ delta,
                                                          const float* __restrict__ w, float eps,
                                                          void* __restrict__ y_out, int n) {
    __shared__ float red[16];
    __shared__ __attribute__((aligned(16))) float sq_s[kNormPer * 1024];
    const int tid = threadIdx.x;
    const int i0 = tid * kNormPer;
    const size_t row = static_cast<size_t>(blockIdx.x) * n;
    x += row;
    if (delta) delta += row;
    float v[kNormPer], sq[kNormPer], wv[kNormPer];
    if constexpr (VEC) {
        const bool in = i0 < n;
        float4 a0 = make_float4(0.f, 0.f, 0.f, 0.f), a1 = a0, w0 = a0, w1 = a0;
        if (in) {
            a0 = reinterpret_cast<const float4*>(x + i0)[0];
            a1 = reinterpret_cast<const float4*>(x + i0)[1];
            w0 = reinterpret_cast<const float4*>(w + i0)[0];
            w1 = reinterpret_cast<const float4*>(w + i0)[1];
            if (delta) {
                const float4 d0 = reinterpret_cast<const float4*>(delta + i0)[0];
                const float4 d1 = reinterpret_cast<const float4*>(delta + i0)[1];
                a0 = make_float4(__fadd_rn(a0.x, d0.x), __fadd_rn(a0.y, d0.y), __fadd_rn(a0.z, d0.z),
                                 __fadd_rn(a0.w, d0.w));
                a1 = make_float4(__fadd_rn(a1.x, d1.x), __fadd_rn(a1.y, d1.y), __fadd_rn(a1.z, d1.z),
                                 __fadd_rn(a1.w, d1.w));
                reinterpret_cast<float4*>(x + i0)[0] = a0;
                reinterpret_cast<float4*>(x + i0)[1] = a1;
            }
        }
        const float va[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const float wa[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int k = 0; k < kNormPer; k++) {
            v[k] = va[k];
            wv[k] = wa[k];
            sq[k] = __fmul_rn(va[k], va[k]);
        }
    } else {
#pragma unroll
        for (int k = 0; k < kNormPer; k++) {
            const int i = i0 + k;
            v[k] = sq[k] = wv[k] = 0.0f;
            if (i < n) {
                float a = x[i];
                if (delta) {
                    a = __fadd_rn(a, delta[i]);
                    x[i] = a;
                }
                v[k] = a;
                wv[k] = w[i];
                sq[k] = __fmul_rn(a, a);
            }
        }
    }
    const float r = rms_factor(row_sum_numpy(sq, n, sq_s, red), n, eps);
    float o[kNormPer];
#pragma unroll
    for (int k = 0; k < kNormPer; k++) o[k] = __fmul_rn(__fmul_rn(v[k], r), wv[k]);
    if constexpr (BF) {
        uint16_t* y = static_cast<uint16_t*>(y_out) + row;
        if constexpr (VEC) {
            if (i0 < n)
                *reinterpret_cast<uint4*>(y + i0) =
                    make_uint4(bf16x2_rne(o[0], o[1]), bf16x2_rne(o[2], o[3]), bf16x2_rne(o[4], o[5]),
                               bf16x2_rne(o[6], o[7]));
        } else {
#pragma unroll
            for (int k = 0; k < kNormPer; k++)
                if (i0 + k < n) y[i0 + k] = static_cast<uint16_t>(bf16x2_rne(o[k], o[k]) & 0xFFFFu);
        }
    } else {
        float* y = static_cast<float*>(y_out) + row;
        if constexpr (VEC) {
            if (i0 < n) {
                reinterpret_cast<float4*>(y + i0)[0] = make_float4(o[0], o[1], o[2], o[3]);
                reinterpret_cast<float4*>(y + i0)[1] = make_float4(o[4], o[5], o[6], o[7]);
            }
        } else {
#pragma unroll
            for (int k = 0; k < kNormPer; k++)
                if (i0 + k < n) y[i0 + k] = o[k];
        }
    }
}

// ------------------------------------------- bias + RoPE + KV-cache write ---
// hetero/cpu_model.py:156-157 (bias), :195-204 (RoPE: x1*cos - x2*sin,
// x1*sin + x2*cos on the two halves), :207-230 (cache at the position).
// Items: [0, nh*half) query pairs, then nkv*half key pairs, then nkv*d values.
// Row blockIdx.y of q/k/v/q_out ([rows][nh*d], [rows][nkv*d]) at position
// (*pos_p, or pos0 when pos_p is null) + blockIdx.y.
__global__ __launch_bounds__(256) void rope_kv_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                      const float* __restrict__ v, const float* __restrict__ bias,
                                                      const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                                      const int64_t* __restrict__ pos_p, int64_t pos0,
                                                      uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                      float* __restrict__ q_out, int nh, int nkv, int d, int cap) {
    const int64_t pos = (pos_p ? *pos_p : pos0) + blockIdx.y;
    q += static_cast<size_t>(blockIdx.y) * nh * d;
    q_out += static_cast<size_t>(blockIdx.y) * nh * d;
    k += static_cast<size_t>(blockIdx.y) * nkv * d;
    v += static_cast<size_t>(blockIdx.y) * nkv * d;
    const int half = d >> 1;
    const int it = blockIdx.x * blockDim.x + threadIdx.x;
    const int nq = nh * half, nk = nkv * half, nv = nkv * d;
    if (pos < 0 || pos >= cap) {                   // no valid cache row: only q
        if (it >= nq) return;
    }
    const size_t prow = static_cast<size_t>(pos < 0 ? 0 : (pos >= cap ? cap - 1 : pos));
    if (it < nq + nk) {
        const bool is_q = it < nq;
        const int p = is_q ? it : it - nq;
        const int head = p / half, i = p - head * half;
        const float* src = is_q ? q : k;
        const float* bsrc = is_q ? bias : bias + nh * d;
        const int e1 = head * d + i, e2 = e1 + half;
        const float x1 = __fadd_rn(src[e1], bsrc[e1]);
        const float x2 = __fadd_rn(src[e2], bsrc[e2]);
        const float c = cos_t[prow * half + i], s = sin_t[prow * half + i];
        const float o1 = __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, s));
        const float o2 = __fadd_rn(__fmul_rn(x1, s), __fmul_rn(x2, c));
        if (is_q) {
            q_out[e1] = o1;
            q_out[e2] = o2;
        } else {
            uint16_t* row = kc + (static_cast<size_t>(head) * cap + prow) * d;
            row[i] = f2h_rne(o1);
            row[i + half] = f2h_rne(o2);
        }
    } else if (it < nq + nk + nv) {
        const int e = it - nq - nk;
        const int head = e / d, i = e - head * d;
        const float val = __fadd_rn(v[e], bias[(nh + nkv) * d + e]);
        vc[(static_cast<size_t>(head) * cap + prow) * d + i] = f2h_rne(val);
    }
}

// ------------------------------------------------------------ SiLU * up ---
// h = SiLU(g) * u elementwise (hetero/cpu_model.py:169-170, :291-292), the
// expression the fused gate/up GEMV applies to its two sums.
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                       float* __restrict__ h, long n) {
    const long stride = static_cast<long>(gridDim.x) * blockDim.x;
    for (long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        h[i] = silu_mul(g[i], u[i]);
}

// ---------------------------------------------------------- attention ---
// attn_decode of q4_attn.h as one launch over grid (chunk, kv head).
template <bool ROPE, int G, int D>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) char lds[kAttnLdsBytes];
    attn_decode<ROPE, G, D>(a, blockIdx.x, blockIdx.y, lds);
}

template <bool ROPE, int D>
void launch_attention_d(int G, dim3 grid, hipStream_t st, const AttnArgs& a) {
    switch (G) {
#define Q4_ATTN_CASE(g)                                                                                      \
    case g:                                                                                                  \
        hipLaunchKernelGGL((attn_decode_kernel<ROPE, g, D>), grid, dim3(kAttnThreads), 0, st, a);          \
        break;
        Q4_ATTN_CASE(1) Q4_ATTN_CASE(2) Q4_ATTN_CASE(3) Q4_ATTN_CASE(4)
        Q4_ATTN_CASE(5) Q4_ATTN_CASE(6) Q4_ATTN_CASE(7) Q4_ATTN_CASE(8)
#undef Q4_ATTN_CASE
        default: break;                        // the callers check 1 <= G <= kMaxG
    }
}

// head_dim 32, 64 or 128 (the callers check)
template <bool ROPE>
void launch_attention(int G, dim3 grid, hipStream_t st, const AttnArgs& a) {
    if (a.d == 128) launch_attention_d<ROPE, 128>(G, grid, st, a);
    else if (a.d == 64) launch_attention_d<ROPE, 64>(G, grid, st, a);
    else launch_attention_d<ROPE, 32>(G, grid, st, a);
}

// ---------------------------------------------------------------- argmax ---
// hetero/backends.py:106-109: int(z.argmax()) -- NumPy's argmax, which
// takes NaN as the largest value, so the result is the first NaN when there
// is one, else the first index of the maximum.  Two launches: workgroup b
// reduces slice b of the logits to (value, index) in the library's argmax
// scratch, then one workgroup reduces the slices in order and does the
// step's bookkeeping.
constexpr int kArgmaxParts = 256;

__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) { argmax_better(bv, bi, v, i); }

// wave and workgroup reduction of (value, index); the result in thread 0
__device__ __forceinline__ void argmax_reduce(float& bv, int& bi, float* rv, int* ri) {
    const int tid = threadIdx.x, nt = blockDim.x;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        better(bv, bi, ov, oi);
    }
    if ((tid & 63) == 0) {
        rv[tid >> 6] = bv;
        ri[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0)
        for (int w = 1; w < (nt >> 6); w++) better(bv, bi, rv[w], ri[w]);
}

// workgroup b: float4s [b*per4, (b+1)*per4) of the logits (and the tail
// values past the last float4 in the last workgroup)
__global__ __launch_bounds__(256) void argmax_part_kernel(const float* __restrict__ logits, int n, int per4,
                                                          float2* __restrict__ part) {
    __shared__ float rv[4];
    __shared__ int ri[4];
    const int tid = threadIdx.x, b = blockIdx.x;
    float bv = -__builtin_inff();
    int bi = 0x7FFFFFFF;
    const int n4 = n >> 2;
    const int lo = b * per4, hi = lo + per4 < n4 ? lo + per4 : n4;
    const __amdgpu_buffer_rsrc_t lr = buf_rsrc(logits, static_cast<uint32_t>(n4) * 16u);
    constexpr int kU = 4;
    for (int base = lo; base < hi; base += kU * 256) {
        float4 f[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int i = base + u * 256 + tid;
            f[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  lr, i < hi ? static_cast<uint32_t>(i) * 16u : kOutOfRange, 0, 0));
        }
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int i = base + u * 256 + tid;
            if (i < hi) {
                better(bv, bi, f[u].x, 4 * i);
                better(bv, bi, f[u].y, 4 * i + 1);
                better(bv, bi, f[u].z, 4 * i + 2);
                better(bv, bi, f[u].w, 4 * i + 3);
            }
        }
    }
    if (b == gridDim.x - 1)
        for (int i = 4 * n4 + tid; i < n; i += 256) better(bv, bi, logits[i], i);
    argmax_reduce(bv, bi, rv, ri);
    if (tid == 0) part[b] = make_float2(bv, __int_as_float(bi));
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const float2* __restrict__ part, int parts,
                                                           int64_t* __restrict__ tok, int64_t* __restrict__ hist,
                                                           int64_t* __restrict__ pos, int64_t s0, int hist_len) {
    __shared__ float rv[4];
    __shared__ int ri[4];
    const int tid = threadIdx.x;
    float bv = -__builtin_inff();
    int bi = 0x7FFFFFFF;
    for (int k = tid; k < parts; k += 256) {
        const float2 c = part[k];
        better(bv, bi, c.x, __float_as_int(c.y));
    }
    argmax_reduce(bv, bi, rv, ri);
    if (tid == 0) {
        const int best = bi == 0x7FFFFFFF ? 0 : bi;
        *tok = best;
        const int64_t p = *pos;
        const int64_t k = p - s0;
        if (k >= 0 && k < hist_len) hist[k] = best;
        *pos = p + 1;
    }
}

// The argmax partials: a fixed array in device memory, one per GPU.
static __device__ __align__(256) float2 argmax_scratch[kStreamSlots * kArgmaxParts];   // a set per stream slot

// Threads of an add_rmsnorm_kernel workgroup: a word (8 values) each, whole
// waves (the sum's order does not depend on the count: threads past the
// row hold zeros).
int norm_threads(int n) {
    const int words = (n + kNormPer - 1) / kNormPer;
    return ((words + 63) / 64) * 64;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q4_EHIP, "%s launch: %s", what, hipGetErrorString(e));
    return 0;
}

// add_rmsnorm_kernel over `rows` rows, 16-byte accesses where n and every
// pointer allow them.
int launch_add_rmsnorm(float* x, const float* delta, const float* w, float eps, void* y, bool bf, int rows, int n,
                       void* stream, const char* what) {
    const auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool vec = n % 8 == 0 && al(x) && al(w) && al(y) && (!delta || al(delta));
    const dim3 grid(rows), block(norm_threads(n));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (vec) {
        if (bf) hipLaunchKernelGGL((add_rmsnorm_kernel<true, true>), grid, block, 0, st, x, delta, w, eps, y, n);
        else hipLaunchKernelGGL((add_rmsnorm_kernel<true, false>), grid, block, 0, st, x, delta, w, eps, y, n);
    } else {
        if (bf) hipLaunchKernelGGL((add_rmsnorm_kernel<false, true>), grid, block, 0, st, x, delta, w, eps, y, n);
        else hipLaunchKernelGGL((add_rmsnorm_kernel<false, false>), grid, block, 0, st, x, delta, w, eps, y, n);
    }
    return check_launch(what);
}

}  // namespace
}  // namespace q4k

using namespace q4k;

#pragma GCC visibility push(default)
extern "C" {

int q4_embed_dev(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, const int64_t* tok,
                 float* out, int n_rows, int n_in, int gs, void* stream) {
    if (!w || !scales || !biases || !tok || !out) return fail(Q4_EARG, "q4_embed_dev: null pointer");
    if (n_rows <= 0 || n_in <= 0 || gs <= 0 || n_in % gs || gs % 8 || (reinterpret_cast<uintptr_t>(out) & 15))
        return fail(Q4_EARG, "q4_embed_dev: bad sizes (n_rows %d, n_in %d, gs %d) or out not 16-byte aligned",
                    n_rows, n_in, gs);
    const int wpr = n_in / 8;
    hipLaunchKernelGGL(embed_kernel, dim3((wpr + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream), w,
                       scales, biases, tok, out, n_rows, n_in, gs);
    return check_launch("q4_embed_dev");
}

int q4_embed_rows_dev(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, const int64_t* ids,
                      int n_ids, float* out, int n_rows, int n_in, int gs, void* stream) {
    if (n_ids < 0 || n_ids > 65535) return fail(Q4_EARG, "q4_embed_rows_dev: n_ids = %d outside [0, 65535]", n_ids);
    if (!w || !scales || !biases || !ids || !out) return fail(Q4_EARG, "q4_embed_rows_dev: null pointer");
    if (n_rows <= 0 || n_in <= 0 || gs <= 0 || n_in % gs || gs % 8 || (reinterpret_cast<uintptr_t>(out) & 15))
        return fail(Q4_EARG, "q4_embed_rows_dev: bad sizes (n_rows %d, n_in %d, gs %d) or out not 16-byte aligned",
                    n_rows, n_in, gs);
    if (n_ids == 0) return 0;
    const int wpr = n_in / 8;
    hipLaunchKernelGGL(embed_kernel, dim3((wpr + 255) / 256, n_ids), dim3(256), 0, static_cast<hipStream_t>(stream),
                       w, scales, biases, ids, out, n_rows, n_in, gs);
    return check_launch("q4_embed_rows_dev");
}

int q4_add_rmsnorm_dev(float* x, const float* delta, const float* w, float eps, float* y, int n, void* stream) {
    if (!x || !w || !y) return fail(Q4_EARG, "q4_add_rmsnorm_dev: null pointer");
    if (n <= 0 || n > kNormPer * 1024) return fail(Q4_EARG, "q4_add_rmsnorm_dev: n = %d outside [1, %d]", n,
                                                   kNormPer * 1024);
    return launch_add_rmsnorm(x, delta, w, eps, y, false, 1, n, stream, "q4_add_rmsnorm_dev");
}

int q4_add_rmsnorm_rows_dev(float* x, const float* delta, const float* w, float eps, float* y, int rows, int n,
                            void* stream) {
    if (!x || !w || !y) return fail(Q4_EARG, "q4_add_rmsnorm_rows_dev: null pointer");
    if (rows < 0 || n <= 0 || n > kNormPer * 1024)
        return fail(Q4_EARG, "q4_add_rmsnorm_rows_dev: rows = %d, n = %d (n in [1, %d])", rows, n, kNormPer * 1024);
    if (rows == 0) return 0;
    return launch_add_rmsnorm(x, delta, w, eps, y, false, rows, n, stream, "q4_add_rmsnorm_rows_dev");
}

int q4_add_rmsnorm_rows_bf16_dev(float* x, const float* delta, const float* w, float eps, uint16_t* y, int rows,
                                 int n, void* stream) {
    if (!x || !w || !y) return fail(Q4_EARG, "q4_add_rmsnorm_rows_bf16_dev: null pointer");
    if (rows < 0 || n <= 0 || n > kNormPer * 1024)
        return fail(Q4_EARG, "q4_add_rmsnorm_rows_bf16_dev: rows = %d, n = %d (n in [1, %d])", rows, n,
                    kNormPer * 1024);
    if (rows == 0) return 0;
    return launch_add_rmsnorm(x, delta, w, eps, y, true, rows, n, stream, "q4_add_rmsnorm_rows_bf16_dev");
}

int q4_rope_kv_dev(const float* q, const float* k, const float* v, const float* bias, const float* cos_t,
                   const float* sin_t, const int64_t* pos, uint16_t* k_cache, uint16_t* v_cache, float* q_out,
                   int n_heads, int n_kv, int head_dim, int cap, void* stream) {
    if (!q || !k || !v || !bias || !cos_t || !sin_t || !pos || !k_cache || !v_cache || !q_out)
        return fail(Q4_EARG, "q4_rope_kv_dev: null pointer");
    if (n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || head_dim <= 0 || head_dim % 2 || cap <= 0)
        return fail(Q4_EARG, "q4_rope_kv_dev: bad sizes (heads %d, kv heads %d, head_dim %d, cap %d)", n_heads,
                    n_kv, head_dim, cap);
    const int items = n_heads * (head_dim / 2) + n_kv * (head_dim / 2) + n_kv * head_dim;
    hipLaunchKernelGGL(rope_kv_kernel, dim3((items + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                       q, k, v, bias, cos_t, sin_t, pos, int64_t{0}, k_cache, v_cache, q_out, n_heads, n_kv, head_dim,
                       cap);
    return check_launch("q4_rope_kv_dev");
}

int q4_rope_kv_rows_dev(const float* q, const float* k, const float* v, const float* bias, const float* cos_t,
                        const float* sin_t, int64_t pos0, int rows, uint16_t* k_cache, uint16_t* v_cache,
                        float* q_out, int n_heads, int n_kv, int head_dim, int cap, void* stream) {
    if (!q || !k || !v || !bias || !cos_t || !sin_t || !k_cache || !v_cache || !q_out)
        return fail(Q4_EARG, "q4_rope_kv_rows_dev: null pointer");
    if (n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || head_dim <= 0 || head_dim % 2 || cap <= 0)
        return fail(Q4_EARG, "q4_rope_kv_rows_dev: bad sizes (heads %d, kv heads %d, head_dim %d, cap %d)", n_heads,
                    n_kv, head_dim, cap);
    if (rows < 0 || rows > 65535 || pos0 < 0 || pos0 + rows > cap)
        return fail(Q4_EARG, "q4_rope_kv_rows_dev: positions [%lld, %lld) outside the cache [0, %d) or rows > 65535",
                    static_cast<long long>(pos0), static_cast<long long>(pos0 + rows), cap);
    if (rows == 0) return 0;
    const int items = n_heads * (head_dim / 2) + n_kv * (head_dim / 2) + n_kv * head_dim;
    hipLaunchKernelGGL(rope_kv_kernel, dim3((items + 255) / 256, rows), dim3(256), 0,
                       static_cast<hipStream_t>(stream), q, k, v, bias, cos_t, sin_t, nullptr, pos0, k_cache, v_cache,
                       q_out, n_heads, n_kv, head_dim, cap);
    return check_launch("q4_rope_kv_rows_dev");
}

int q4_silu_mul_dev(const float* g, const float* u, float* h, long n, void* stream) {
    if (!g || !u || !h) return fail(Q4_EARG, "q4_silu_mul_dev: null pointer");
    if (n < 0) return fail(Q4_EARG, "q4_silu_mul_dev: n = %ld", n);
    if (n == 0) return 0;
    const long blocks = (n + 255) / 256;
    hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(blocks < 4096 ? blocks : 4096)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), g, u, h, n);
    return check_launch("q4_silu_mul_dev");
}

long q4_attention_scratch_floats(int n_heads, int head_dim, int cap) {
    if (n_heads <= 0 || head_dim <= 0 || cap <= 0) return 0;
    const long n_chunks = (cap + kChunk - 1) / kChunk;
    return static_cast<long>(n_heads) * n_chunks * (head_dim + 2) + kAttnCounters * kCounterStride;
}

int q4_attention_dev(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, const int64_t* pos,
                     float* out, float* scratch, int n_heads, int n_kv, int head_dim, int cap, float scale,
                     void* stream) {
    if (!q || !k_cache || !v_cache || !pos || !out || !scratch) return fail(Q4_EARG, "q4_attention_dev: null pointer");
    if (n_heads <= 0 || n_kv <= 0 || n_heads > kAttnCounters || n_heads % n_kv || n_heads / n_kv > kMaxG ||
        head_dim <= 0 || head_dim % 2 ||
        head_dim > kMaxD || cap <= 0)
        return fail(Q4_EARG, "q4_attention_dev: unsupported sizes (heads %d, kv heads %d, head_dim %d, cap %d)",
                    n_heads, n_kv, head_dim, cap);
    const int n_chunks = (cap + kChunk - 1) / kChunk;
    if (n_chunks > kMaxChunks || head_dim % 32 || 256 % head_dim || (reinterpret_cast<uintptr_t>(q) & 15) ||
        (reinterpret_cast<uintptr_t>(k_cache) & 15) || (reinterpret_cast<uintptr_t>(v_cache) & 15) ||
        (reinterpret_cast<uintptr_t>(scratch) & 7))
        return fail(Q4_EARG, "q4_attention_dev: cap %d over %d, head_dim %d not 32, 64 or 128, "
                             "or a pointer not 16-byte aligned", cap, kMaxChunks * kChunk, head_dim);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const AttnArgs a{q, const_cast<uint16_t*>(k_cache), const_cast<uint16_t*>(v_cache), pos, scratch, out, n_heads,
                     n_kv, head_dim, cap, n_chunks, scale, nullptr, nullptr, nullptr, nullptr, nullptr};
    launch_attention<false>(n_heads / n_kv, dim3(n_chunks, n_kv), st, a);
    return check_launch("q4_attention_dev");
}

int q4_attention_rope_dev(const float* q, const float* k, const float* v, const float* bias, const float* cos_t,
                          const float* sin_t, const int64_t* pos, uint16_t* k_cache, uint16_t* v_cache, float* out,
                          float* scratch, int n_heads, int n_kv, int head_dim, int cap, float scale, void* stream) {
    if (!q || !k || !v || !bias || !cos_t || !sin_t || !pos || !k_cache || !v_cache || !out || !scratch)
        return fail(Q4_EARG, "q4_attention_rope_dev: null pointer");
    if (n_heads <= 0 || n_kv <= 0 || n_heads > kAttnCounters || n_heads % n_kv || n_heads / n_kv > kMaxG ||
        head_dim <= 0 || head_dim % 32 ||
        256 % head_dim || head_dim > kMaxD || cap <= 0 || (cap + kChunk - 1) / kChunk > kMaxChunks ||
        (reinterpret_cast<uintptr_t>(k_cache) & 15) || (reinterpret_cast<uintptr_t>(v_cache) & 15) ||
        (reinterpret_cast<uintptr_t>(scratch) & 7))
        return fail(Q4_EARG, "q4_attention_rope_dev: unsupported sizes (heads %d, kv heads %d, head_dim %d, cap %d) "
                             "or a pointer not aligned", n_heads, n_kv, head_dim, cap);
    const int n_chunks = (cap + kChunk - 1) / kChunk;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const AttnArgs a{q, k_cache, v_cache, pos, scratch, out, n_heads, n_kv, head_dim, cap, n_chunks, scale,
                     k, v, bias, cos_t, sin_t};
    launch_attention<true>(n_heads / n_kv, dim3(n_chunks, n_kv), st, a);
    return check_launch("q4_attention_rope_dev");
}

int q4_argmax_dev(const float* logits, int n, int64_t* tok, int64_t* hist, int64_t* pos, int64_t s0, int hist_len,
                  void* stream) {
    if (!logits || !tok || !pos || (hist_len > 0 && !hist)) return fail(Q4_EARG, "q4_argmax_dev: null pointer");
    if (n <= 0 || (reinterpret_cast<uintptr_t>(logits) & 15)) return fail(Q4_EARG, "q4_argmax_dev: bad n %d or logits not 16-byte aligned", n);
    static std::mutex mu;
    static void* scr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(Q4_EHIP, "q4_argmax_dev: no device");
    void* sp;
    {
        std::lock_guard<std::mutex> lock(mu);
        if (!scr[dev]) {
            void* a = nullptr;
            const hipError_t e = hipGetSymbolAddress(&a, HIP_SYMBOL(argmax_scratch));
            if (e != hipSuccess || !a) return fail(Q4_EHIP, "hipGetSymbolAddress(argmax_scratch): %s", hipGetErrorString(e));
            scr[dev] = a;
        }
        sp = scr[dev];
    }
    int slot = 0;
    if (int rc = stream_slot(static_cast<hipStream_t>(stream), &slot)) return rc;
    sp = static_cast<float2*>(sp) + static_cast<size_t>(slot) * kArgmaxParts;
    const int n4 = n >> 2;
    // at least 1024 float4s per workgroup, at most kArgmaxParts workgroups
    int parts = (n4 + 1023) / 1024;
    parts = parts < 1 ? 1 : (parts > kArgmaxParts ? kArgmaxParts : parts);
    const int per4 = (n4 + parts - 1) / parts;
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(argmax_part_kernel, dim3(parts), dim3(256), 0, st, logits, n, per4, static_cast<float2*>(sp));
    if (int rc = check_launch("q4_argmax_dev")) return rc;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, st, static_cast<const float2*>(sp), parts, tok,
                       hist, pos, s0, hist_len);
    return check_launch("q4_argmax_dev");
}

}  // extern "C"
#pragma GCC visibility pop
