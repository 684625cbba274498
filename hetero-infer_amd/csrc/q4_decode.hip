// Decode-step kernels of the device-resident Qwen2 stage (gfx950): the
// operations around the int4 GEMVs that the reference's NumPy stage
// (hetero/cpu_model.py) runs on the host.  Declared in q4decode.h.
//
// Elementwise fp32 arithmetic follows the reference's expression order with
// -ffp-contract=off (explicit _rn operations), so RoPE and the bias adds give
// the NumPy bits; the reductions (RMSNorm's mean, the softmax sums, the
// attention dot products) are tree reductions, not NumPy's pairwise order.
#include <mutex>

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
__global__ __launch_bounds__(256) void embed_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ sc,
                                                    const uint16_t* __restrict__ bi, const int64_t* __restrict__ tok,
                                                    float* __restrict__ out, int n_rows, int n_in, int gs) {
    const int wpr = n_in >> 3, G = n_in / gs;
    const int64_t t = *tok;
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
// the residual add of :304-306.  One workgroup; n <= 8 * 1024.  Thread t
// owns the 8 consecutive values of word t and adds their squares in order;
// the wave sums (wave_sum) are added in wave order.  The streaming GEMV's
// norm prologue sums in exactly this order, so its input is y bit for bit.
constexpr int kNormPer = 8;
__global__ __launch_bounds__(1024) void add_rmsnorm_kernel(float* __restrict__ x, const float* __restrict__ delta,
                                                          const float* __restrict__ w, float eps,
                                                          float* __restrict__ y, int n) {
    __shared__ float red[16];
    const int tid = threadIdx.x, nt = blockDim.x;
    const int i0 = tid * kNormPer;
    float v[kNormPer];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormPer; k++) {
        const int i = i0 + k;
        v[k] = 0.0f;
        if (i < n) {
            float a = x[i];
            if (delta) {
                a = __fadd_rn(a, delta[i]);
                x[i] = a;
            }
            v[k] = a;
            ss = __fadd_rn(ss, __fmul_rn(a, a));
        }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int i = 0; i < (nt >> 6); i++) tot = __fadd_rn(tot, red[i]);
    const float r = rms_factor(tot, n, eps);
#pragma unroll
    for (int k = 0; k < kNormPer; k++) {
        const int i = i0 + k;
        if (i < n) y[i] = __fmul_rn(__fmul_rn(v[k], r), w[i]);
    }
}

// ------------------------------------------- bias + RoPE + KV-cache write ---
// hetero/cpu_model.py:156-157 (bias), :195-204 (RoPE: x1*cos - x2*sin,
// x1*sin + x2*cos on the two halves), :207-230 (cache at the position).
// Items: [0, nh*half) query pairs, then nkv*half key pairs, then nkv*d values.
__global__ __launch_bounds__(256) void rope_kv_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                      const float* __restrict__ v, const float* __restrict__ bias,
                                                      const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                                      const int64_t* __restrict__ pos_p, uint16_t* __restrict__ kc,
                                                      uint16_t* __restrict__ vc, float* __restrict__ q_out, int nh,
                                                      int nkv, int d, int cap) {
    const int64_t pos = *pos_p;
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

// ---------------------------------------------------------- attention ---
// hetero/cpu_model.py:233-252 for one query token: per query head,
// s = (q . k_t) * scale over the positions t <= pos, p = exp(s - max s),
// o = (sum p_t v_t) / (sum p_t).  Workgroup (chunk, kv head) takes 64
// positions and the G = nh / nkv query heads that share the kv head, and
// writes its partial (max, sum, unnormalised o); the combine launch merges
// the chunks (o = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c).
constexpr int kChunk = 64;
constexpr int kMaxG = 8;          // query heads per kv head
constexpr int kMaxD = 128;
constexpr int kRowU4 = kMaxD / 8 + 1;   // LDS row of a chunk: 16 uint4 of fp16 + 1 pad (16-byte reads spread over the banks)
constexpr int kMaxChunks = 1024;        // cap <= 65536

// ROPE: q, k and v are the raw projection outputs; the workgroup applies
// the biases and the rotary embedding to its G query heads (as
// rope_kv_kernel does), and the workgroup whose chunk holds the position
// also rotates the new key, writes the new key and value rows to the cache
// and takes them from registers instead of the cache.
// G: query heads per kv head, a template parameter so that the per-head
// loops unroll and their LDS reads are issued together.  NW: waves (4, or 8
// for head_dim >= 64), which split the head dimension of the scores and the
// positions of the outputs between them.
template <bool ROPE, int G, int NW>
__global__ __launch_bounds__(64 * NW) void attn_partial_kernel(const float* __restrict__ q,
                                                           uint16_t* __restrict__ kc,
                                                           uint16_t* __restrict__ vc,
                                                           const int64_t* __restrict__ pos_p,
                                                           float* __restrict__ part, int nh, int nkv, int d,
                                                           int cap, float scale, const float* __restrict__ kraw,
                                                           const float* __restrict__ vraw,
                                                           const float* __restrict__ bias,
                                                           const float* __restrict__ cos_t,
                                                           const float* __restrict__ sin_t) {
    constexpr int NT = 64 * NW;                              // threads
    constexpr int KV = kChunk * (kMaxD / 8) / NT;            // uint4 of K (and of V) per thread at d = 128
    constexpr int QR = kMaxG * (kMaxD / 2) / NT;             // rounds of the RoPE'd query pairs
    constexpr int PW = kChunk / NW;                          // positions per wave in the output pass
    __shared__ float4 q_s[kMaxG][kMaxD / 4];
    __shared__ uint4 k_s[kChunk][kRowU4];
    __shared__ uint4 v_s[kChunk][kRowU4];
    __shared__ __attribute__((aligned(16))) float p_s[kMaxG][kChunk];
    __shared__ float sc_part[NW][kMaxG][kChunk];
    __shared__ float out_part[NW][kMaxG][kMaxD];
    const int chunk = blockIdx.x, kvh = blockIdx.y, n_chunks = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t pos = *pos_p;
    const int c0 = chunk * kChunk;
    const int64_t lim = pos + 1 < cap ? pos + 1 : cap;      // positions [0, lim)
    const int valid = lim - c0 >= kChunk ? kChunk : static_cast<int>(lim - c0 > 0 ? lim - c0 : 0);
    const int du4 = d >> 3;                                  // uint4 (8 fp16) per row
    float* my = part;                                        // [nh][n_chunks][d + 2]
    if (valid == 0) {                                        // chunk past the position
        for (int e = tid; e < G * (d + 2); e += blockDim.x) {
            const int g = e / (d + 2), i = e - g * (d + 2);
            float* dst = my + (static_cast<size_t>(kvh * G + g) * n_chunks + chunk) * (d + 2);
            dst[i] = i == 0 ? -__builtin_inff() : 0.0f;
        }
        return;
    }
    // the chunk's new row (the position) comes from registers, not the cache
    const bool fresh = ROPE && pos >= c0 && pos < c0 + kChunk && pos < cap;
    // every load up front: q, the chunk's K and V rows (4 uint4 each per
    // thread at d = 128), unconditional, through resources that end with the
    // rows to read: rows past `valid` (and a fresh row) read 0 without an
    // access, and the staging registers stay registers
    const int nkv4 = (fresh ? valid - 1 : valid) * du4;
    const __amdgpu_buffer_rsrc_t kr =
        buf_rsrc(kc + (static_cast<size_t>(kvh) * cap + c0) * d, static_cast<uint32_t>(nkv4) * 16u);
    const __amdgpu_buffer_rsrc_t vr =
        buf_rsrc(vc + (static_cast<size_t>(kvh) * cap + c0) * d, static_cast<uint32_t>(nkv4) * 16u);
    uint4 kv[KV], vv[KV];
    uint16_t fh1 = 0, fh2 = 0;                               // the fresh row's values of this thread
    auto load_kv = [&]() {
#pragma unroll
        for (int r = 0; r < KV; r++) {
            const uint32_t off = static_cast<uint32_t>(r * NT + tid) * 16u;
            kv[r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0));
            vv[r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0));
        }
    };
    if constexpr (ROPE) {
        // hetero/cpu_model.py:156-157 (bias) and :195-204 (RoPE), the same
        // fp32 operations as rope_kv_kernel
        const int half = d >> 1;
        const size_t prow = static_cast<size_t>(pos < 0 ? 0 : (pos >= cap ? cap - 1 : pos));
        float qa[QR][2], qb[QR][2], cs[QR][2];
#pragma unroll
        for (int r = 0; r < QR; r++) {
            const int e = r * NT + tid;
            if (e < G * half) {
                const int g = e / half, i = e - g * half;
                const int e1 = (kvh * G + g) * d + i;
                qa[r][0] = q[e1]; qa[r][1] = q[e1 + half];
                qb[r][0] = bias[e1]; qb[r][1] = bias[e1 + half];
                cs[r][0] = cos_t[prow * half + i]; cs[r][1] = sin_t[prow * half + i];
            }
        }
        float nk[2] = {0.f, 0.f}, nkb[2] = {0.f, 0.f}, nkc[2] = {0.f, 0.f}, nv = 0.f, nvb = 0.f;
        if (fresh) {
            if (tid < half) {
                const int e1 = kvh * d + tid;
                nk[0] = kraw[e1]; nk[1] = kraw[e1 + half];
                nkb[0] = bias[nh * d + e1]; nkb[1] = bias[nh * d + e1 + half];
                nkc[0] = cos_t[prow * half + tid]; nkc[1] = sin_t[prow * half + tid];
            } else if (tid < half + d) {
                const int e = kvh * d + (tid - half);
                nv = vraw[e];
                nvb = bias[(nh + nkv) * d + e];
            }
        }
        load_kv();
        float* qf = reinterpret_cast<float*>(&q_s[0][0]);
#pragma unroll
        for (int r = 0; r < QR; r++) {
            const int e = r * NT + tid;
            if (e < G * half) {
                const int g = e / half, i = e - g * half;
                const float x1 = __fadd_rn(qa[r][0], qb[r][0]), x2 = __fadd_rn(qa[r][1], qb[r][1]);
                const float c = cs[r][0], sn = cs[r][1];
                qf[g * kMaxD + i] = __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, sn));
                qf[g * kMaxD + i + half] = __fadd_rn(__fmul_rn(x1, sn), __fmul_rn(x2, c));
            }
        }
        if (fresh) {
            uint16_t* kg = kc + (static_cast<size_t>(kvh) * cap + pos) * d;
            uint16_t* vg = vc + (static_cast<size_t>(kvh) * cap + pos) * d;
            if (tid < half) {
                const float x1 = __fadd_rn(nk[0], nkb[0]), x2 = __fadd_rn(nk[1], nkb[1]);
                const float c = nkc[0], sn = nkc[1];
                fh1 = f2h_rne(__fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, sn)));
                fh2 = f2h_rne(__fadd_rn(__fmul_rn(x1, sn), __fmul_rn(x2, c)));
                kg[tid] = fh1; kg[tid + half] = fh2;
            } else if (tid < half + d) {
                fh1 = f2h_rne(__fadd_rn(nv, nvb));
                vg[tid - half] = fh1;
            }
        }
    } else {
        const float4* q4p = reinterpret_cast<const float4*>(q + static_cast<size_t>(kvh * G) * d);
        const int nq4 = G * d / 4;
        float4 qv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (tid < nq4) qv = q4p[tid];
        load_kv();
        if (tid < nq4) q_s[tid / (d / 4)][tid % (d / 4)] = qv;
    }
    // all 64 rows but a fresh one: the rows past the ones read (past the
    // position) hold 0, so the output loop needs no bound
    const int frow = fresh ? static_cast<int>(pos - c0) : -1;
#pragma unroll
    for (int r = 0; r < KV; r++) {
        const int e = r * NT + tid;
        if (e < kChunk * du4 && e / du4 != frow) {
            k_s[e / du4][e % du4] = kv[r];
            v_s[e / du4][e % du4] = vv[r];
        }
    }
    if (fresh) {
        const int row = frow, half = d >> 1;
        uint16_t* kl = reinterpret_cast<uint16_t*>(&k_s[row][0]);
        uint16_t* vl = reinterpret_cast<uint16_t*>(&v_s[row][0]);
        if (tid < half) {
            kl[tid] = fh1;
            kl[tid + half] = fh2;
        } else if (tid < half + d) {
            vl[tid - half] = fh1;
        }
    }
    __syncthreads();
    // scores: wave w takes dims [w*d/NW, (w+1)*d/NW) of every position of
    // the chunk (lane = position) for all G heads, so each K element is
    // converted once; the NW partial dots are added in wave order below
    {
        const int s = lane;
        const int c_begin = wave * (du4 / NW), c_end = c_begin + du4 / NW;
        float acc[kMaxG];
#pragma unroll
        for (int g = 0; g < kMaxG; g++) acc[g] = 0.0f;
        for (int c = c_begin; c < c_end; c++) {
            const uint4 kk = k_s[s][c];
            const float kf[8] = {h2f_bits(static_cast<uint16_t>(kk.x)), h2f_bits(static_cast<uint16_t>(kk.x >> 16)),
                                 h2f_bits(static_cast<uint16_t>(kk.y)), h2f_bits(static_cast<uint16_t>(kk.y >> 16)),
                                 h2f_bits(static_cast<uint16_t>(kk.z)), h2f_bits(static_cast<uint16_t>(kk.z >> 16)),
                                 h2f_bits(static_cast<uint16_t>(kk.w)), h2f_bits(static_cast<uint16_t>(kk.w >> 16))};
#pragma unroll
            for (int g = 0; g < kMaxG; g++) {
                if (g < G) {                                         // uniform
                    const float4 qa = q_s[g][2 * c], qb = q_s[g][2 * c + 1];
                    acc[g] = __builtin_fmaf(qa.x, kf[0], acc[g]);
                    acc[g] = __builtin_fmaf(qa.y, kf[1], acc[g]);
                    acc[g] = __builtin_fmaf(qa.z, kf[2], acc[g]);
                    acc[g] = __builtin_fmaf(qa.w, kf[3], acc[g]);
                    acc[g] = __builtin_fmaf(qb.x, kf[4], acc[g]);
                    acc[g] = __builtin_fmaf(qb.y, kf[5], acc[g]);
                    acc[g] = __builtin_fmaf(qb.z, kf[6], acc[g]);
                    acc[g] = __builtin_fmaf(qb.w, kf[7], acc[g]);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < kMaxG; g++)
            if (g < G) sc_part[wave][g][s] = acc[g];
    }
    __syncthreads();
    // softmax over the chunk, heads wave, wave + NW, ... (lane = position)
    for (int g = wave; g < G; g += NW) {
        const int s = lane;
        float dot = sc_part[0][g][s];
#pragma unroll
        for (int w = 1; w < NW; w++) dot = __fadd_rn(dot, sc_part[w][g][s]);
        const float sc = s < valid ? __fmul_rn(dot, scale) : -__builtin_inff();
        const float m = wave_max(sc);
        const float p = s < valid ? expf(__fsub_rn(sc, m)) : 0.0f;
        const float l = wave_sum(p);
        p_s[g][s] = p;
        if (lane == 0) {
            float* dst = my + (static_cast<size_t>(kvh * G + g) * n_chunks + chunk) * (d + 2);
            dst[0] = m;
            dst[1] = l;
        }
    }
    __syncthreads();
    // unnormalised outputs: wave w takes positions [PW*w, PW*w + PW), lane
    // = fp16 pair of the row, all G heads; the NW partial outputs are
    // added in wave order
    {
        const int i = lane, dp = d >> 1;
        float a0[kMaxG], a1[kMaxG];
#pragma unroll
        for (int g = 0; g < kMaxG; g++) a0[g] = a1[g] = 0.0f;
        if (i < dp) {
            const uint32_t* vw = reinterpret_cast<const uint32_t*>(&v_s[0][0]);
            constexpr int kRowW = kRowU4 * 4;
            // p is 0 and the V row is 0 past the valid positions
            for (int s0 = PW * wave; s0 < PW * wave + PW; s0 += 4) {
                uint32_t w2[4];
#pragma unroll
                for (int j = 0; j < 4; j++) w2[j] = vw[(s0 + j) * kRowW + i];
                float4 pg[kMaxG];
#pragma unroll
                for (int g = 0; g < kMaxG; g++)
                    if (g < G) pg[g] = *reinterpret_cast<const float4*>(&p_s[g][s0]);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float v0 = h2f_bits(static_cast<uint16_t>(w2[j]));
                    const float v1 = h2f_bits(static_cast<uint16_t>(w2[j] >> 16));
#pragma unroll
                    for (int g = 0; g < kMaxG; g++) {
                        if (g < G) {
                            const float p = j == 0 ? pg[g].x : j == 1 ? pg[g].y : j == 2 ? pg[g].z : pg[g].w;
                            a0[g] = __builtin_fmaf(p, v0, a0[g]);
                            a1[g] = __builtin_fmaf(p, v1, a1[g]);
                        }
                    }
                }
            }
#pragma unroll
            for (int g = 0; g < kMaxG; g++)
                if (g < G) {
                    out_part[wave][g][2 * i] = a0[g];
                    out_part[wave][g][2 * i + 1] = a1[g];
                }
        }
    }
    __syncthreads();
    for (int e = tid; e < G * d; e += NT) {
        const int g = e / d, j = e - g * d;
        float o = out_part[0][g][j];
#pragma unroll
        for (int w = 1; w < NW; w++) o = __fadd_rn(o, out_part[w][g][j]);
        my[(static_cast<size_t>(kvh * G + g) * n_chunks + chunk) * (d + 2) + 2 + j] = o;
    }
}

template <bool ROPE, int NW>
void launch_partial_nw(int G, dim3 grid, hipStream_t st, const float* q, uint16_t* kc, uint16_t* vc,
                       const int64_t* pos, float* part, int nh, int nkv, int d, int cap, float scale,
                       const float* kraw, const float* vraw, const float* bias, const float* cos_t,
                       const float* sin_t) {
    switch (G) {
#define Q4_ATTN_CASE(g)                                                                                      \
    case g:                                                                                                  \
        hipLaunchKernelGGL((attn_partial_kernel<ROPE, g, NW>), grid, dim3(64 * NW), 0, st, q, kc, vc, pos, part, \
                           nh, nkv, d, cap, scale, kraw, vraw, bias, cos_t, sin_t);                          \
        break;
        Q4_ATTN_CASE(1) Q4_ATTN_CASE(2) Q4_ATTN_CASE(3) Q4_ATTN_CASE(4)
        Q4_ATTN_CASE(5) Q4_ATTN_CASE(6) Q4_ATTN_CASE(7) Q4_ATTN_CASE(8)
#undef Q4_ATTN_CASE
        default: break;                        // the callers check 1 <= G <= kMaxG
    }
}

// 8 waves when every wave gets a whole uint4 of the head dimension (d >= 64)
template <bool ROPE>
void launch_partial(int G, dim3 grid, hipStream_t st, const float* q, uint16_t* kc, uint16_t* vc, const int64_t* pos,
                    float* part, int nh, int nkv, int d, int cap, float scale, const float* kraw, const float* vraw,
                    const float* bias, const float* cos_t, const float* sin_t) {
    if (d >= 64)
        launch_partial_nw<ROPE, 8>(G, grid, st, q, kc, vc, pos, part, nh, nkv, d, cap, scale, kraw, vraw, bias,
                                   cos_t, sin_t);
    else
        launch_partial_nw<ROPE, 4>(G, grid, st, q, kc, vc, pos, part, nh, nkv, d, cap, scale, kraw, vraw, bias,
                                   cos_t, sin_t);
}

// one workgroup per query head: M = max_c m_c, w_c = e^(m_c - M),
// o = sum_c w_c o_c / sum_c w_c l_c.  Every load is issued before the
// first reduction: m and l of chunk c by thread c (c + 256, ...), and thread
// (part k, dim i) prefetches o[i] of its chunks k, k + nparts, ... (nparts =
// 256 / d) -- one round of memory latency instead of three.
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                           int n_chunks, int d) {
    __shared__ float w_s[kMaxChunks];
    __shared__ float red[8];
    const int h = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
    const int stride = d + 2;
    const int i = tid % d, part_k = tid / d;
    const int nparts = nt / d;
    const __amdgpu_buffer_rsrc_t pr = buf_rsrc(part + static_cast<size_t>(h) * n_chunks * stride,
                                               static_cast<uint32_t>(n_chunks * stride) * 4u);
    auto ld = [&](int c, int k) {                 // element k of chunk c (0 past the last chunk)
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             pr, static_cast<uint32_t>(c * stride + k) * 4u, 0, 0));
    };
    constexpr int kPre = 32;                      // o values prefetched per thread
    float ob[kPre];
#pragma unroll
    for (int j = 0; j < kPre; j++) ob[j] = ld(part_k + j * nparts, 2 + i);
    constexpr int kMl = kMaxChunks / 256;         // chunks per thread for m and l
    float mv[kMl], lv[kMl];
#pragma unroll
    for (int r = 0; r < kMl; r++) {
        mv[r] = ld(tid + 256 * r, 0);
        lv[r] = ld(tid + 256 * r, 1);
    }
    float mloc = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < kMl; r++)
        if (tid + 256 * r < n_chunks) mloc = fmaxf(mloc, mv[r]);
    mloc = wave_max(mloc);
    if ((tid & 63) == 0) red[tid >> 6] = mloc;
    __syncthreads();
    float M = -__builtin_inff();
    for (int k = 0; k < (nt >> 6); k++) M = fmaxf(M, red[k]);
    __syncthreads();
    float lloc = 0.0f;
#pragma unroll
    for (int r = 0; r < kMl; r++) {
        const int c = tid + 256 * r;
        if (c < n_chunks) {
            const float wgt = mv[r] == -__builtin_inff() ? 0.0f : expf(__fsub_rn(mv[r], M));
            w_s[c] = wgt;
            lloc = __builtin_fmaf(lv[r], wgt, lloc);
        }
    }
    lloc = wave_sum(lloc);
    if ((tid & 63) == 0) red[tid >> 6] = lloc;
    __syncthreads();
    float L = 0.0f;
    for (int k = 0; k < (nt >> 6); k++) L = __fadd_rn(L, red[k]);
    // the part's chunks in order: the prefetched ones, then any past them
    float O = 0.0f;
#pragma unroll
    for (int j = 0; j < kPre; j++) {
        const int c = part_k + j * nparts;
        if (c < n_chunks) O = __builtin_fmaf(ob[j], w_s[c], O);
    }
    for (int c = part_k + kPre * nparts; c < n_chunks; c += nparts) O = __builtin_fmaf(ld(c, 2 + i), w_s[c], O);
    __syncthreads();
    float* o_s = w_s;                                        // the weights are no longer read
    o_s[part_k * d + i] = O;
    __syncthreads();
    if (part_k == 0) {
        for (int k = 1; k < nparts; k++) O = __fadd_rn(O, o_s[k * d + i]);
        out[static_cast<size_t>(h) * d + i] = __fdiv_rn(O, L);
    }
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
static __device__ __align__(256) float2 argmax_scratch[kArgmaxParts];

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q4_EHIP, "%s launch: %s", what, hipGetErrorString(e));
    return 0;
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

int q4_add_rmsnorm_dev(float* x, const float* delta, const float* w, float eps, float* y, int n, void* stream) {
    if (!x || !w || !y) return fail(Q4_EARG, "q4_add_rmsnorm_dev: null pointer");
    if (n <= 0 || n > kNormPer * 1024) return fail(Q4_EARG, "q4_add_rmsnorm_dev: n = %d outside [1, %d]", n,
                                                   kNormPer * 1024);
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream), x, delta, w,
                       eps, y, n);
    return check_launch("q4_add_rmsnorm_dev");
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
                       q, k, v, bias, cos_t, sin_t, pos, k_cache, v_cache, q_out, n_heads, n_kv, head_dim, cap);
    return check_launch("q4_rope_kv_dev");
}

long q4_attention_scratch_floats(int n_heads, int head_dim, int cap) {
    if (n_heads <= 0 || head_dim <= 0 || cap <= 0) return 0;
    const long n_chunks = (cap + kChunk - 1) / kChunk;
    return static_cast<long>(n_heads) * n_chunks * (head_dim + 2);
}

int q4_attention_dev(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, const int64_t* pos,
                     float* out, float* scratch, int n_heads, int n_kv, int head_dim, int cap, float scale,
                     void* stream) {
    if (!q || !k_cache || !v_cache || !pos || !out || !scratch) return fail(Q4_EARG, "q4_attention_dev: null pointer");
    if (n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || n_heads / n_kv > kMaxG || head_dim <= 0 || head_dim % 2 ||
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
    launch_partial<false>(n_heads / n_kv, dim3(n_chunks, n_kv), st, q, const_cast<uint16_t*>(k_cache),
                          const_cast<uint16_t*>(v_cache), pos, scratch, n_heads, n_kv, head_dim, cap, scale, nullptr,
                          nullptr, nullptr, nullptr, nullptr);
    if (int rc = check_launch("q4_attention_dev (partial)")) return rc;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(n_heads), dim3(256), 0, st, scratch, out, n_chunks, head_dim);
    return check_launch("q4_attention_dev (combine)");
}

int q4_attention_rope_dev(const float* q, const float* k, const float* v, const float* bias, const float* cos_t,
                          const float* sin_t, const int64_t* pos, uint16_t* k_cache, uint16_t* v_cache, float* out,
                          float* scratch, int n_heads, int n_kv, int head_dim, int cap, float scale, void* stream) {
    if (!q || !k || !v || !bias || !cos_t || !sin_t || !pos || !k_cache || !v_cache || !out || !scratch)
        return fail(Q4_EARG, "q4_attention_rope_dev: null pointer");
    if (n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || n_heads / n_kv > kMaxG || head_dim <= 0 || head_dim % 32 ||
        256 % head_dim || head_dim > kMaxD || cap <= 0 || (cap + kChunk - 1) / kChunk > kMaxChunks ||
        (reinterpret_cast<uintptr_t>(k_cache) & 15) || (reinterpret_cast<uintptr_t>(v_cache) & 15) ||
        (reinterpret_cast<uintptr_t>(scratch) & 7))
        return fail(Q4_EARG, "q4_attention_rope_dev: unsupported sizes (heads %d, kv heads %d, head_dim %d, cap %d) "
                             "or a pointer not aligned", n_heads, n_kv, head_dim, cap);
    const int n_chunks = (cap + kChunk - 1) / kChunk;
    hipStream_t st = static_cast<hipStream_t>(stream);
    launch_partial<true>(n_heads / n_kv, dim3(n_chunks, n_kv), st, q, k_cache, v_cache, pos, scratch, n_heads,
                         n_kv, head_dim, cap, scale, k, v, bias, cos_t, sin_t);
    if (int rc = check_launch("q4_attention_rope_dev (partial)")) return rc;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(n_heads), dim3(256), 0, st, scratch, out, n_chunks, head_dim);
    return check_launch("q4_attention_rope_dev (combine)");
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
