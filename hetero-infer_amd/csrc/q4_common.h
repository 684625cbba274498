// Shared by the translation units of libq4gemv.so: constants and the
// device helpers of the int4 GEMV kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>

#include "q4gemv.h"

namespace q4k {

constexpr int kChunkWords = 256;   // words per wave chunk: 64 lanes x 4 words

// ---------------------------------------------------------------- helpers --

__device__ __forceinline__ float h2f(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// x86 cvttss2si followed by a 16-bit truncation: values outside the int32
// range (and NaN) give 0x80000000, whose low half is 0.
__device__ __forceinline__ int32_t to_i16_like_x86(float r) {
    int32_t v = (r > -2147483648.0f && r < 2147483648.0f) ? static_cast<int32_t>(r)
                                                           : static_cast<int32_t>(0x80000000u);
    return static_cast<int16_t>(v);
}

// Sum of an int over the `lpg` consecutive lanes of a group (lpg a power of
// two, 1..64).  Every lane of the wave must execute it.
__device__ __forceinline__ int group_sum(int v, int lpg) {
    if (lpg >= 2) v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);   // quad_perm 1,0,3,2
    if (lpg >= 4) v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);   // quad_perm 2,3,0,1
    if (lpg >= 8) v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false);  // row_half_mirror
    if (lpg >= 16) v += __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false); // row_mirror
    if (lpg >= 32) v += __shfl_xor(v, 16);
    if (lpg >= 64) v += __shfl_xor(v, 32);
    return v;
}


// Max over the wave (NaN-skipping, like the reference's `v > amax` scan):
// DPP within rows of 16 lanes, then the four row results through SGPRs.
template <int CTRL>
__device__ __forceinline__ float dpp_max(float a) {
    const int o = __builtin_amdgcn_update_dpp(__float_as_int(a), __float_as_int(a), CTRL, 0xF, 0xF, false);
    return fmaxf(a, __int_as_float(o));
}

// Raw buffer resource over [p, p + bytes): loads at an offset >= bytes
// return 0 without a memory access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}
constexpr uint32_t kOutOfRange = 0x80000000u;   // any offset past every resource here

template <int CTRL>
__device__ __forceinline__ float dpp_add(float a) {
    const int o = __builtin_amdgcn_update_dpp(__float_as_int(a), __float_as_int(a), CTRL, 0xF, 0xF, false);
    return __fadd_rn(a, __int_as_float(o));
}

// Sum over the 64 lanes, the same value in every lane: DPP pairs, quads,
// halves and rows of 16 (every lane of a row ends with the row's sum),
// then the four row sums added in row order.
__device__ __forceinline__ float wave_sum(float v) {
    v = dpp_add<0xB1>(v);    // quad_perm 1,0,3,2
    v = dpp_add<0x4E>(v);    // quad_perm 2,3,0,1
    v = dpp_add<0x141>(v);   // row_half_mirror
    v = dpp_add<0x140>(v);   // row_mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return __fadd_rn(__fadd_rn(__fadd_rn(r0, r1), r2), r3);
}

// a in the low half, b in the high half, each rounded to bf16 to nearest
// even: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t bf16x2_rne(float a, float b) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
    const f32x2 p = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(p, bf16x2v));
}

// SiLU(g) * u as hetero/cpu_model.py:169-170 and :291-292 compute it in
// fp32: g / (1 + exp(-g)) * u (expf here; NumPy's float32 exp may differ in
// the last place).
__device__ __forceinline__ float silu_mul(float g, float u) {
    const float e = expf(-g);
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
}

// 1 / sqrt(mean + eps) of RMSNorm from the sum of squares of n values
// (hetero/cpu_model.py:164-166).  NumPy's mean divides the float32 sum by
// the element count, an integer scalar, in float64 and stores the quotient
// as float32 (true_divide with casting='unsafe'); eps then adds in float32.
// The square root is the correctly rounded one (__builtin_sqrtf expands to
// v_sqrt_f32 plus a one-ulp correction; __fsqrt_rn is v_sqrt_f32 alone,
// which is off by an ulp now and then), as np.sqrt's.
__device__ __forceinline__ float rms_factor(float sum_sq, int n, float eps) {
    const float ms = static_cast<float>(static_cast<double>(sum_sq) / static_cast<double>(n));
    return __fdiv_rn(1.0f, __builtin_sqrtf(__fadd_rn(ms, eps)));
}

__device__ __forceinline__ float wave_max(float v) {
    v = dpp_max<0xB1>(v);    // quad_perm 1,0,3,2
    v = dpp_max<0x4E>(v);    // quad_perm 2,3,0,1
    v = dpp_max<0x141>(v);   // row_half_mirror
    v = dpp_max<0x140>(v);   // row_mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// The sum of a row of n non-negative values (sums of squares), thread t
// holding the 8 values of word t (values 8t .. 8t+7; threads past the row
// hold zeros), added in the order of NumPy's float32 reductions
// (np.add.reduce, which x.mean() and x.sum() use): pairwise summation -- a
// row of more than 128 values is split at n2 = n/2 rounded down to a
// multiple of 8 and the two halves' sums are added; a block of
// 8 <= n <= 128 values is added by 8 accumulators, r[j] taking values j,
// j + 8, j + 16, ... in order, combined as ((r0 + r1) + (r2 + r3)) +
// ((r4 + r5) + (r6 + r7)).  When every split is exact (n = L m with L a
// power of two, m <= 128, m % 8 == 0, each halving an exact half) the tree
// is perfect: lane 8b + j adds block b's column j, and pairs of lanes, then
// of lane groups, are added -- that order, IEEE addition being commutative
// -- by DPP within rows of 16 lanes, the 4 rows of a wave by readlane, and
// the waves' sums through LDS; groups past the L blocks hold zeros, which
// add exactly.  Other n fall back to a tree order (wave_sum).  Every
// thread of the workgroup calls it (blockDim.x a multiple of 64 and at
// least n / 8); scratch: n floats of LDS, red: 16 floats of LDS.  Returns
// the sum in every thread, after two workgroup barriers; scratch is free
// for other use on return, red keeps the waves' sums.
__device__ __forceinline__ float row_sum_numpy(const float v[8], int n, float* scratch, float* red) {
    const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wave = tid >> 6;
    int m = n, L = 1;
    bool perfect = n >= 8 && n % 8 == 0;
    while (perfect && m > 128) {
        if (m % 16) perfect = false;
        else { m >>= 1; L <<= 1; }
    }
    if (!perfect || 8 * L > nt) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) ss = __fadd_rn(ss, v[i]);
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int i = 0; i < (nt >> 6); i++) tot = __fadd_rn(tot, red[i]);
        __syncthreads();
        return tot;
    }
    if (tid < (n >> 3)) {
        float4* d = reinterpret_cast<float4*>(scratch + 8 * tid);
        d[0] = make_float4(v[0], v[1], v[2], v[3]);
        d[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();
    float r = 0.0f;
    if (tid < 8 * L) {                                             // block b = tid / 8, accumulator j = tid % 8
        const float* p = scratch + (tid >> 3) * m + (tid & 7);
        r = p[0];
        for (int i = 8; i < m; i += 8) r = __fadd_rn(r, p[i]);
    }
    r = dpp_add<0xB1>(r);                                          // + lane ^ 1: r0 + r1, ...
    r = dpp_add<0x4E>(r);                                          // + lane ^ 2: (r0 + r1) + (r2 + r3)
    r = dpp_add<0x141>(r);                                         // + the half-row's other quad: the block
    r = dpp_add<0x140>(r);                                         // + the row's other half: blocks in pairs
    const float q0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 0));
    const float q1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 16));
    const float q2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 32));
    const float q3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 48));
    const int W = (8 * L + 63) >> 6;                               // waves holding blocks: 1, 2, 4, ..., 16
    if (lane == 0 && wave < W) red[wave] = __fadd_rn(__fadd_rn(q0, q1), __fadd_rn(q2, q3));
    __syncthreads();
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; i++) t[i] = i < W ? red[i] : 0.0f;
#pragma unroll
    for (int s = 1; s < 16; s <<= 1)
#pragma unroll
        for (int i = 0; i < 16; i += 2 * s) t[i] = __fadd_rn(t[i], t[i + s]);
    return t[0];
}

// One packed word of x (8 values, MLX order) -> {xl even, xl odd, xh even,
// xh odd} byte planes of xq = (int16)(x*inv +- 0.5) (kernel/q4gemv.c:266-268).
// a + copysign(0.5, a) is the reference's `a < 0 ? a - 0.5 : a + 0.5` for
// every a whose truncation is defined (the two differ only for -0.0, which
// truncates to 0 either way).  When inv is finite |x*inv| <= 32767.5, so
// v_cvt_i32_f32 is the x86 truncation (NaN -> 0 on both after the 16-bit
// cut); `exact_clamp` selects the out-of-range rule for an infinite inv.
__device__ __forceinline__ uint4 quant_word(const float (&v)[8], float inv, bool exact_clamp) {
    int32_t q[8];
#pragma unroll
    for (int n = 0; n < 8; n++) {
        const float a = __fmul_rn(v[n], inv);
        const float r = __fadd_rn(a, __builtin_copysignf(0.5f, a));
        q[n] = exact_clamp ? to_i16_like_x86(r) : static_cast<int32_t>(r);
    }
    // pack (q0,q2), (q4,q6), (q1,q3), (q5,q7) as int16 pairs, then gather bytes
    const uint32_t e0 = (static_cast<uint32_t>(q[0]) & 0xFFFFu) | (static_cast<uint32_t>(q[2]) << 16);
    const uint32_t e1 = (static_cast<uint32_t>(q[4]) & 0xFFFFu) | (static_cast<uint32_t>(q[6]) << 16);
    const uint32_t o0 = (static_cast<uint32_t>(q[1]) & 0xFFFFu) | (static_cast<uint32_t>(q[3]) << 16);
    const uint32_t o1 = (static_cast<uint32_t>(q[5]) & 0xFFFFu) | (static_cast<uint32_t>(q[7]) << 16);
    // v_perm_b32(hi, lo, sel): byte k of the result = byte sel[k] of {hi:lo}
    const uint32_t le = __builtin_amdgcn_perm(e1, e0, 0x06040200u);   // low bytes of q0,q2,q4,q6
    const uint32_t he = __builtin_amdgcn_perm(e1, e0, 0x07050301u);   // high bytes
    const uint32_t lo = __builtin_amdgcn_perm(o1, o0, 0x06040200u);
    const uint32_t ho = __builtin_amdgcn_perm(o1, o0, 0x07050301u);
    return make_uint4(le, lo, he, ho);
}

// NumPy's argmax order (hetero/backends.py:106-109, z.argmax()): NaN counts
// as the largest value, so the first NaN wins; otherwise the largest value,
// the first index of it on ties.  (v, i) replaces (bv, bi) when it comes
// first in that order -- a total order, so any reduction tree gives the
// same result.
__device__ __forceinline__ void argmax_better(float& bv, int& bi, float v, int i) {
    const bool vn = v != v, bn = bv != bv;
    const bool take = vn ? (!bn || i < bi) : (!bn && (v > bv || (v == bv && i < bi)));
    if (take) { bv = v; bi = i; }
}
constexpr int kArgmaxNone = 0x7FFFFFFF;   // the index of "no value yet"
constexpr int kGreedyMaxParts = 4096;     // workgroups of a launch that takes the greedy token

// The greedy token of a one-matrix, one-row GEMV, taken in the GEMV's own
// launch: each workgroup reduces the rows it stored to (value, index) in
// part[blockIdx.x] and counts itself in *count; the last to arrive reduces
// the parts and does the decode step's bookkeeping (*tok = the index,
// hist[*pos - s0] = *tok when in [0, hist_len), *pos += 1) and sets *count
// back to 0.  part null: no greedy token.
struct GreedyArgs {
    float2* part;
    unsigned* count;
    int64_t* tok;
    int64_t* hist;
    int64_t* pos;
    int64_t s0;
    int hist_len;
};

// host side, defined in q4gemv.hip
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int num_cus();
// Arrays of the library in device memory that a launch uses as its own
// (the greedy token's parts and counter, argmax's parts) come in
// kStreamSlots sets per GPU, one per stream: the kStreamSlots streams that
// used them most recently on a device each hold a set, so calls on
// different streams never share one (calls on one stream are ordered by it).
constexpr int kStreamSlots = 16;
int stream_slot(hipStream_t st, int* slot);

// The matrices of one prefill launch (q4_gemm.hip), up to 4 sharing x:
// matrix k's 256-column blocks are blocks nb0[k] .. nb0[k+1] - 1 of the
// launch (a block never holds two matrices), its columns are columns
// col0[k] .. col0[k] + n_out[k] - 1 of the split-K partials.
struct GemmMats {
    const uint32_t* w[4];
    const uint16_t* s[4];
    const uint16_t* b[4];
    float* out[4];
    int n_out[4];
    int nb0[5];
    int col0[4];
    int count;
};

// The prefill GEMM (q4_gemm.hip), data-parallel: tiles of height bm (256 or
// 128) over every block of gm, S splits of kt_split K steps.  part null:
// each matrix's output directly; else split z into part + z M ldp at the
// matrix's columns.
int gemm_w4(const uint16_t* xb, const GemmMats& gm, float* part, int M, int K, int bm, int S, int kt_split, int ldp,
            hipStream_t st);

// Paired gate/up form (q4_gemm.hip): matrices 0 and 1 of gm, both n_out[0]
// rows, every K step in one workgroup, h[M][n_out[0]] = bf16(SiLU(x Wg^T) *
// (x Wu^T)).
int gemm_w4_pair(const uint16_t* xb, const GemmMats& gm, uint16_t* h, int M, int K, hipStream_t st);

// Stream-K form of the prefill GEMM: P workgroups in nx XCD groups (256 x
// 256 tiles; P a multiple of nx, and P / nx at least a group's tile count,
// ceil(tiles / nx)), each matrix's output directly.  part: P x 256 x 256
// floats of partial sums; flags: 32 P words; ctl: kSkCtlWords control
// words (the epoch, the exit counter and, at kSkCtlErrors, a counter of
// partials that did not arrive in time: their tiles are NaN).  flags and
// ctl are zero when first used and are left consistent by every launch.
int gemm_w4_sk(const uint16_t* xb, const GemmMats& gm, float* part, unsigned* flags, unsigned* ctl, int M, int K,
               int P, int nx, hipStream_t st);

// gemm_w4_pair over a stream-K split of its tiles (the ranges of gemm_w4_sk,
// P workgroups in nx groups, any P up to the CUs and the iterations): the
// owner of each paired tile stores h as gemm_w4_pair does.
int gemm_w4_sk_pair(const uint16_t* xb, const GemmMats& gm, float* part, unsigned* flags, unsigned* ctl, uint16_t* h,
                    int M, int K, int P, int nx, hipStream_t st);
constexpr int kSkCtlWordsHost = 96;   // the control words after the flags (q4_gemm.hip: kSkCtlWords)
constexpr int kSkCtlErrorsHost = 64;  // the error counter among them (kSkCtlErrors)

// Dynamic LDS above 64 KiB needs the kernel's limit raised on each device
// that runs it.  `done` holds one bit per device already raised (0..63; a
// higher device id raises it on every call).
inline int raise_lds_limit(const void* kern, size_t bytes, std::atomic<uint64_t>& done) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(Q4_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t{1} << dev) : 0;
    if (bit && (done.load(std::memory_order_relaxed) & bit)) return 0;
    e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) return fail(Q4_EHIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    done.fetch_or(bit, std::memory_order_relaxed);
    return 0;
}
constexpr size_t kStreamLdsMax = 160 * 1024;

}  // namespace q4k
