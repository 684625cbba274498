// Grouped-query attention of one query token over an fp16 KV cache, as
// device functions: the partial over one (64-position chunk, kv head) job
// and the combine of one query head's chunks.  The decode-step kernels
// (q4_decode.hip) run them as launches of their own; the chained programs
// (q4_chain.hip) run them as phases of one persistent launch.
//
// hetero/cpu_model.py:233-252 for one query token: per query head,
// s = (q . k_t) * scale over the positions t <= pos, p = exp(s - max s),
// o = (sum p_t v_t) / (sum p_t).  Job (chunk, kv head) takes 64 positions
// and the G = nh / nkv query heads that share the kv head, and writes its
// partial (max, sum, unnormalised o); the combine merges the chunks
// (o = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c).
//
// The functions are called by every thread of a workgroup of at least the
// threads they use (64 NW for the partial, 256 for the combine): the others
// pass the same barriers and do no work.  DEV: the values another
// workgroup of the same launch produced or consumes -- the raw q/k/v, the
// partials, the output -- are loaded and stored at device scope (cache
// policy sc1); with separate launches plain accesses suffice.  The
// arithmetic does not depend on DEV.
#pragma once

#include "q4_common.h"

namespace q4k {

constexpr int kChunk = 64;
constexpr int kMaxG = 8;          // query heads per kv head
constexpr int kMaxD = 128;
constexpr int kRowU4 = kMaxD / 8 + 1;   // LDS row of a chunk: 16 uint4 of fp16 + 1 pad (16-byte reads spread over the banks)
constexpr int kMaxChunks = 1024;        // cap <= 65536

__device__ __forceinline__ uint16_t attn_f2h(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

__device__ __forceinline__ float attn_h2f(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

template <bool DEV>
__device__ __forceinline__ float attn_ld(const float* p) {
    if constexpr (DEV) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *p;
}

template <bool DEV>
__device__ __forceinline__ void attn_st(float* p, float v) {
    if constexpr (DEV) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}

// LDS of the partial of NW waves: q [kMaxG][kMaxD], the chunk's K and V rows
// [kChunk][kRowU4] uint4 each, p [kMaxG][kChunk], the waves' partial scores
// [NW][kMaxG][kChunk] and outputs [NW][kMaxG][kMaxD].
template <int NW>
__host__ __device__ constexpr size_t attn_partial_lds_bytes() {
    return static_cast<size_t>(kMaxG) * kMaxD * 4 + 2 * static_cast<size_t>(kChunk) * kRowU4 * 16 +
           static_cast<size_t>(kMaxG) * kChunk * 4 + static_cast<size_t>(NW) * kMaxG * kChunk * 4 +
           static_cast<size_t>(NW) * kMaxG * kMaxD * 4;
}
constexpr size_t kAttnCombineLdsBytes = (kMaxChunks + 8) * 4;

struct AttnArgs {
    const float* q;          // raw projection outputs (ROPE) or rotated queries
    uint16_t* kc;
    uint16_t* vc;
    const int64_t* pos;
    float* part;             // [nh][n_chunks][d + 2]
    float* out;              // [nh][d]
    int nh, nkv, d, cap, n_chunks;
    float scale;
    const float* kraw;       // ROPE: raw k, v, the q/k/v biases, cos/sin tables
    const float* vraw;
    const float* bias;
    const float* cos_t;
    const float* sin_t;
};

// ROPE: q, k and v are the raw projection outputs; the job applies the
// biases and the rotary embedding to its G query heads (as rope_kv_kernel
// does), and the job whose chunk holds the position also rotates the new
// key, writes the new key and value rows to the cache and takes them from
// registers instead of the cache.
// G: query heads per kv head, a template parameter so that the per-head
// loops unroll and their LDS reads are issued together.  NW: waves (4, or 8
// for head_dim >= 64), which split the head dimension of the scores and the
// positions of the outputs between them.
template <bool ROPE, int G, int NW, bool DEV>
__device__ __forceinline__ void attn_partial(const AttnArgs& a, int chunk, int kvh, char* lds) {
    constexpr int NT = 64 * NW;                              // threads that work
    constexpr int KV = kChunk * (kMaxD / 8) / NT;            // uint4 of K (and of V) per thread at d = 128
    constexpr int QR = kMaxG * (kMaxD / 2) / NT;             // rounds of the RoPE'd query pairs
    constexpr int PW = kChunk / NW;                          // positions per wave in the output pass
    typedef float4 QRow[kMaxD / 4];
    typedef uint4 KRow[kRowU4];
    typedef float SRow[kMaxG][kChunk];
    typedef float ORow[kMaxG][kMaxD];
    QRow* q_s = reinterpret_cast<QRow*>(lds);                                          // [kMaxG]
    KRow* k_s = reinterpret_cast<KRow*>(lds + kMaxG * kMaxD * 4);                      // [kChunk]
    KRow* v_s = k_s + kChunk;                                                          // [kChunk]
    float(*p_s)[kChunk] = reinterpret_cast<float(*)[kChunk]>(v_s + kChunk);             // [kMaxG]
    SRow* sc_part = reinterpret_cast<SRow*>(p_s + kMaxG);                              // [NW]
    ORow* out_part = reinterpret_cast<ORow*>(sc_part + NW);                            // [NW]
    const int n_chunks = a.n_chunks, d = a.d, cap = a.cap, nh = a.nh, nkv = a.nkv;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool act = tid < NT;                               // wave-uniform
    const int64_t pos = *a.pos;
    const int c0 = chunk * kChunk;
    const int64_t lim = pos + 1 < cap ? pos + 1 : cap;      // positions [0, lim)
    const int valid = lim - c0 >= kChunk ? kChunk : static_cast<int>(lim - c0 > 0 ? lim - c0 : 0);
    const int du4 = d >> 3;                                  // uint4 (8 fp16) per row
    float* my = a.part;                                      // [nh][n_chunks][d + 2]
    if (valid == 0) {                                        // chunk past the position (uniform)
        if (act)
            for (int e = tid; e < G * (d + 2); e += NT) {
                const int g = e / (d + 2), i = e - g * (d + 2);
                float* dst = my + (static_cast<size_t>(kvh * G + g) * n_chunks + chunk) * (d + 2);
                attn_st<DEV>(dst + i, i == 0 ? -__builtin_inff() : 0.0f);
            }
        return;
    }
    // the chunk's new row (the position) comes from registers, not the cache
    const bool fresh = ROPE && pos >= c0 && pos < c0 + kChunk && pos < cap;
    const int frow = fresh ? static_cast<int>(pos - c0) : -1;
    if (act) {
        // every load up front: q, the chunk's K and V rows (4 uint4 each per
        // thread at d = 128), unconditional, through resources that end with
        // the rows to read: rows past `valid` (and a fresh row) read 0
        // without an access, and the staging registers stay registers
        const int nkv4 = (fresh ? valid - 1 : valid) * du4;
        const __amdgpu_buffer_rsrc_t kr =
            buf_rsrc(a.kc + (static_cast<size_t>(kvh) * cap + c0) * d, static_cast<uint32_t>(nkv4) * 16u);
        const __amdgpu_buffer_rsrc_t vr =
            buf_rsrc(a.vc + (static_cast<size_t>(kvh) * cap + c0) * d, static_cast<uint32_t>(nkv4) * 16u);
        uint4 kv[KV], vv[KV];
        uint16_t fh1 = 0, fh2 = 0;                           // the fresh row's values of this thread
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
                    qa[r][0] = attn_ld<DEV>(a.q + e1); qa[r][1] = attn_ld<DEV>(a.q + e1 + half);
                    qb[r][0] = a.bias[e1]; qb[r][1] = a.bias[e1 + half];
                    cs[r][0] = a.cos_t[prow * half + i]; cs[r][1] = a.sin_t[prow * half + i];
                }
            }
            float nk[2] = {0.f, 0.f}, nkb[2] = {0.f, 0.f}, nkc[2] = {0.f, 0.f}, nv = 0.f, nvb = 0.f;
            if (fresh) {
                if (tid < half) {
                    const int e1 = kvh * d + tid;
                    nk[0] = attn_ld<DEV>(a.kraw + e1); nk[1] = attn_ld<DEV>(a.kraw + e1 + half);
                    nkb[0] = a.bias[nh * d + e1]; nkb[1] = a.bias[nh * d + e1 + half];
                    nkc[0] = a.cos_t[prow * half + tid]; nkc[1] = a.sin_t[prow * half + tid];
                } else if (tid < half + d) {
                    const int e = kvh * d + (tid - half);
                    nv = attn_ld<DEV>(a.vraw + e);
                    nvb = a.bias[(nh + nkv) * d + e];
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
                uint16_t* kg = a.kc + (static_cast<size_t>(kvh) * cap + pos) * d;
                uint16_t* vg = a.vc + (static_cast<size_t>(kvh) * cap + pos) * d;
                if (tid < half) {
                    const float x1 = __fadd_rn(nk[0], nkb[0]), x2 = __fadd_rn(nk[1], nkb[1]);
                    const float c = nkc[0], sn = nkc[1];
                    fh1 = attn_f2h(__fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, sn)));
                    fh2 = attn_f2h(__fadd_rn(__fmul_rn(x1, sn), __fmul_rn(x2, c)));
                    kg[tid] = fh1; kg[tid + half] = fh2;
                } else if (tid < half + d) {
                    fh1 = attn_f2h(__fadd_rn(nv, nvb));
                    vg[tid - half] = fh1;
                }
            }
        } else {
            const int nq4 = G * d / 4;
            float4 qv = make_float4(0.f, 0.f, 0.f, 0.f);
            if (tid < nq4) {
                const float* qp = a.q + static_cast<size_t>(kvh * G) * d + 4 * tid;
                qv = make_float4(attn_ld<DEV>(qp), attn_ld<DEV>(qp + 1), attn_ld<DEV>(qp + 2), attn_ld<DEV>(qp + 3));
            }
            load_kv();
            if (tid < nq4) q_s[tid / (d / 4)][tid % (d / 4)] = qv;
        }
        // all 64 rows but a fresh one: the rows past the ones read (past the
        // position) hold 0, so the output loop needs no bound
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
    }
    __syncthreads();
    // scores: wave w takes dims [w*d/NW, (w+1)*d/NW) of every position of
    // the chunk (lane = position) for all G heads, so each K element is
    // converted once; the NW partial dots are added in wave order below
    if (act) {
        const int s = lane;
        const int c_begin = wave * (du4 / NW), c_end = c_begin + du4 / NW;
        float acc[kMaxG];
#pragma unroll
        for (int g = 0; g < kMaxG; g++) acc[g] = 0.0f;
        for (int c = c_begin; c < c_end; c++) {
            const uint4 kk = k_s[s][c];
            const float kf[8] = {attn_h2f(static_cast<uint16_t>(kk.x)), attn_h2f(static_cast<uint16_t>(kk.x >> 16)),
                                 attn_h2f(static_cast<uint16_t>(kk.y)), attn_h2f(static_cast<uint16_t>(kk.y >> 16)),
                                 attn_h2f(static_cast<uint16_t>(kk.z)), attn_h2f(static_cast<uint16_t>(kk.z >> 16)),
                                 attn_h2f(static_cast<uint16_t>(kk.w)), attn_h2f(static_cast<uint16_t>(kk.w >> 16))};
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
    if (act) {
        for (int g = wave; g < G; g += NW) {
            const int s = lane;
            float dot = sc_part[0][g][s];
#pragma unroll
            for (int w = 1; w < NW; w++) dot = __fadd_rn(dot, sc_part[w][g][s]);
            const float sc = s < valid ? __fmul_rn(dot, a.scale) : -__builtin_inff();
            const float m = wave_max(sc);
            const float p = s < valid ? expf(__fsub_rn(sc, m)) : 0.0f;
            const float l = wave_sum(p);
            p_s[g][s] = p;
            if (lane == 0) {
                float* dst = my + (static_cast<size_t>(kvh * G + g) * n_chunks + chunk) * (d + 2);
                attn_st<DEV>(dst, m);
                attn_st<DEV>(dst + 1, l);
            }
        }
    }
    __syncthreads();
    // unnormalised outputs: wave w takes positions [PW*w, PW*w + PW), lane
    // = fp16 pair of the row, all G heads; the NW partial outputs are
    // added in wave order
    if (act) {
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
                    const float v0 = attn_h2f(static_cast<uint16_t>(w2[j]));
                    const float v1 = attn_h2f(static_cast<uint16_t>(w2[j] >> 16));
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
    if (act)
        for (int e = tid; e < G * d; e += NT) {
            const int g = e / d, j = e - g * d;
            float o = out_part[0][g][j];
#pragma unroll
            for (int w = 1; w < NW; w++) o = __fadd_rn(o, out_part[w][g][j]);
            attn_st<DEV>(my + (static_cast<size_t>(kvh * G + g) * n_chunks + chunk) * (d + 2) + 2 + j, o);
        }
}

// The combine of query head h: M = max_c m_c, w_c = e^(m_c - M),
// o = sum_c w_c o_c / sum_c w_c l_c, on 256 threads.  Every load is issued
// before the first reduction: m and l of chunk c by thread c (c + 256, ...),
// and thread (part k, dim i) prefetches o[i] of its chunks k, k + nparts, ...
// (nparts = 256 / d) -- one round of memory latency instead of three.
// lds: kAttnCombineLdsBytes.
template <bool DEV>
__device__ __forceinline__ void attn_combine(const AttnArgs& a, int h, char* lds) {
    constexpr int NT = 256;
    float* w_s = reinterpret_cast<float*>(lds);                       // [kMaxChunks]
    float* red = w_s + kMaxChunks;                                    // [8]
    const int tid = threadIdx.x;
    const bool act = tid < NT;                                        // wave-uniform
    const int n_chunks = a.n_chunks, d = a.d;
    const int stride = d + 2;
    const int i = tid % d, part_k = tid / d;
    const int nparts = NT / d;
    constexpr int kAux = DEV ? 16 : 0;                                // sc1 when DEV
    const __amdgpu_buffer_rsrc_t pr = buf_rsrc(a.part + static_cast<size_t>(h) * n_chunks * stride,
                                               static_cast<uint32_t>(n_chunks * stride) * 4u);
    auto ld = [&](int c, int k) {                 // element k of chunk c (0 past the last chunk)
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             pr, static_cast<uint32_t>(c * stride + k) * 4u, 0, kAux));
    };
    constexpr int kPre = 32;                      // o values prefetched per thread
    constexpr int kMl = kMaxChunks / NT;          // chunks per thread for m and l
    float ob[kPre], mv[kMl], lv[kMl];
    if (act) {
#pragma unroll
        for (int j = 0; j < kPre; j++) ob[j] = ld(part_k + j * nparts, 2 + i);
#pragma unroll
        for (int r = 0; r < kMl; r++) {
            mv[r] = ld(tid + NT * r, 0);
            lv[r] = ld(tid + NT * r, 1);
        }
        float mloc = -__builtin_inff();
#pragma unroll
        for (int r = 0; r < kMl; r++)
            if (tid + NT * r < n_chunks) mloc = fmaxf(mloc, mv[r]);
        mloc = wave_max(mloc);
        if ((tid & 63) == 0) red[tid >> 6] = mloc;
    }
    __syncthreads();
    float M = -__builtin_inff();
    for (int k = 0; k < (NT >> 6); k++) M = fmaxf(M, red[k]);
    __syncthreads();
    if (act) {
        float lloc = 0.0f;
#pragma unroll
        for (int r = 0; r < kMl; r++) {
            const int c = tid + NT * r;
            if (c < n_chunks) {
                const float wgt = mv[r] == -__builtin_inff() ? 0.0f : expf(__fsub_rn(mv[r], M));
                w_s[c] = wgt;
                lloc = __builtin_fmaf(lv[r], wgt, lloc);
            }
        }
        lloc = wave_sum(lloc);
        if ((tid & 63) == 0) red[tid >> 6] = lloc;
    }
    __syncthreads();
    float L = 0.0f;
    for (int k = 0; k < (NT >> 6); k++) L = __fadd_rn(L, red[k]);
    // the part's chunks in order: the prefetched ones, then any past them
    float O = 0.0f;
    if (act) {
#pragma unroll
        for (int j = 0; j < kPre; j++) {
            const int c = part_k + j * nparts;
            if (c < n_chunks) O = __builtin_fmaf(ob[j], w_s[c], O);
        }
        for (int c = part_k + kPre * nparts; c < n_chunks; c += nparts) O = __builtin_fmaf(ld(c, 2 + i), w_s[c], O);
    }
    __syncthreads();
    float* o_s = w_s;                                        // the weights are no longer read
    if (act) o_s[part_k * d + i] = O;
    __syncthreads();
    if (act && part_k == 0) {
        for (int k = 1; k < nparts; k++) O = __fadd_rn(O, o_s[k * d + i]);
        attn_st<DEV>(a.out + static_cast<size_t>(h) * d + i, __fdiv_rn(O, L));
    }
}

}  // namespace q4k
