// Grouped-query attention of one query token over an fp16 KV cache, as one
// launch (the decode-step kernels of q4_decode.hip).
//
// hetero/cpu_model.py:233-252 for one query token: per query head,
// s = (q . k_t) * scale over the positions t <= pos, p = exp(s - max s),
// o = (sum p_t v_t) / (sum p_t).  Workgroup (chunk, kv head) takes 64
// positions and the G = nh / nkv query heads that share the kv head:
// wave g is query head g -- for the scores and the softmax lane j takes
// position j of the chunk (all in registers), for the weighted sum of v
// lane i the dimensions 2i, 2i + 1.  Each wave writes its head's partial
// result (max m, sum l, unnormalised o) and arrives at the head's counter;
// the wave of the last chunk to arrive merges the head's parts
// (o = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c, the o sum in chunk
// order, the l sum a fixed lane tree), so there is no second launch.  The
// result does not depend on which chunk arrives last.
#pragma once

#include "q4_common.h"

namespace q4k {

constexpr int kChunk = 64;
constexpr int kMaxG = 8;          // query heads per kv head
constexpr int kMaxD = 128;
constexpr int kRowU4 = kMaxD / 8 + 1;   // LDS row of a chunk: 16 uint4 of fp16 + 1 pad (16-byte reads spread over the banks)
constexpr int kMaxChunks = 1024;        // cap <= 65536
constexpr int kAttnThreads = 64 * kMaxG;   // a wave per query head
constexpr int kAttnCounters = 512;      // arrival counters after the partials (one per query head)
constexpr int kCounterStride = 32;      // words between counters: each on its own 128-byte line
constexpr int kMergeBatch = 36;         // chunks merged per round of loads (2304 positions in one round)
constexpr int kAttnCoherent = 16;       // cache policy sc1: device-scope stores and loads of the parts

__device__ __forceinline__ uint16_t attn_f2h(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

__device__ __forceinline__ float attn_h2f(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// LDS of the kernel: q [kMaxG][kMaxD], the chunk's K and V rows
// [kChunk][kRowU4] uint4 each, p [kMaxG][kChunk].
constexpr size_t kAttnLdsBytes = static_cast<size_t>(kMaxG) * kMaxD * 4 +
                                 2 * static_cast<size_t>(kChunk) * kRowU4 * 16 +
                                 static_cast<size_t>(kMaxG) * kChunk * 4;

struct AttnArgs {
    const float* q;          // raw projection outputs (ROPE) or rotated queries
    uint16_t* kc;
    uint16_t* vc;
    const int64_t* pos;
    float* part;             // [nh][n_chunks][d + 2], then kAttnCounters arrival counters
    float* out;              // [nh][d]
    int nh, nkv, d, cap, n_chunks;
    float scale;
    const float* kraw;       // ROPE: raw k, v, the q/k/v biases, cos/sin tables
    const float* vraw;
    const float* bias;
    const float* cos_t;
    const float* sin_t;
};

// ROPE: q, k and v are the raw projection outputs; the workgroup applies
// the biases and the rotary embedding to its G query heads (as
// rope_kv_kernel does), and the one whose chunk holds the position also
// rotates the new key, writes the new key and value rows to the cache and
// takes them from registers instead of the cache.  G: query heads per kv
// head, D: head_dim (32, 64 or 128; a.d), template parameters so that the
// loops over them unroll and their LDS reads are issued together.  Called
// by the kAttnThreads threads of the workgroup.
template <bool ROPE, int G, int D>
__device__ __forceinline__ void attn_decode(const AttnArgs& a, int chunk, int kvh, char* lds) {
    static_assert(D == 32 || D == 64 || D == 128, "head_dim 32, 64 or 128");
    constexpr int NT = kAttnThreads;
    constexpr int KV = kChunk * (kMaxD / 8) / NT;            // uint4 of K (and of V) per thread at d = 128
    constexpr int QR = (G * (kMaxD / 2) + NT - 1) / NT;      // rounds of the RoPE'd query pairs
    typedef float4 QRow[kMaxD / 4];
    typedef uint4 KRow[kRowU4];
    QRow* q_s = reinterpret_cast<QRow*>(lds);                                          // [kMaxG]
    KRow* k_s = reinterpret_cast<KRow*>(lds + kMaxG * kMaxD * 4);                      // [kChunk]
    KRow* v_s = k_s + kChunk;                                                          // [kChunk]
    float(*p_s)[kChunk] = reinterpret_cast<float(*)[kChunk]>(v_s + kChunk);             // [kMaxG]
    const int n_chunks = a.n_chunks, cap = a.cap, nh = a.nh, nkv = a.nkv;
    constexpr int d = D;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: the wave's resources stay scalar
    const int64_t pos = *a.pos;
    const int c0 = chunk * kChunk;
    const int64_t lim = pos + 1 < cap ? pos + 1 : cap;      // positions [0, lim)
    if (lim <= c0) return;                                   // past the position: no part, no arrival
    const int valid = lim - c0 >= kChunk ? kChunk : static_cast<int>(lim - c0);
    const int n_act = static_cast<int>((lim + kChunk - 1) / kChunk);   // chunks that arrive
    constexpr int du4 = d >> 3;                              // uint4 (8 fp16) per row
    // the chunk's new row (the position) comes from registers, not the cache
    const bool fresh = ROPE && pos >= c0 && pos < c0 + kChunk && pos < cap;
    const int frow = fresh ? static_cast<int>(pos - c0) : -1;
    // every load up front: q, the chunk's K and V rows, unconditional,
    // through resources that end with the rows to read: rows past `valid`
    // (and a fresh row) read 0 without an access
    {
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
                    qa[r][0] = a.q[e1]; qa[r][1] = a.q[e1 + half];
                    qb[r][0] = a.bias[e1]; qb[r][1] = a.bias[e1 + half];
                    cs[r][0] = a.cos_t[prow * half + i]; cs[r][1] = a.sin_t[prow * half + i];
                }
            }
            float nk[2] = {0.f, 0.f}, nkb[2] = {0.f, 0.f}, nkc[2] = {0.f, 0.f}, nv = 0.f, nvb = 0.f;
            if (fresh) {
                if (tid < half) {
                    const int e1 = kvh * d + tid;
                    nk[0] = a.kraw[e1]; nk[1] = a.kraw[e1 + half];
                    nkb[0] = a.bias[nh * d + e1]; nkb[1] = a.bias[nh * d + e1 + half];
                    nkc[0] = a.cos_t[prow * half + tid]; nkc[1] = a.sin_t[prow * half + tid];
                } else if (tid < half + d) {
                    const int e = kvh * d + (tid - half);
                    nv = a.vraw[e];
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
            if (tid < nq4) qv = reinterpret_cast<const float4*>(a.q + static_cast<size_t>(kvh * G) * d)[tid];
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
            const int half = d >> 1;
            uint16_t* kl = reinterpret_cast<uint16_t*>(&k_s[frow][0]);
            uint16_t* vl = reinterpret_cast<uint16_t*>(&v_s[frow][0]);
            if (tid < half) {
                kl[tid] = fh1;
                kl[tid + half] = fh2;
            } else if (tid < half + d) {
                vl[tid - half] = fh1;
            }
        }
    }
    __syncthreads();
    const int g = wave;                                      // this wave's query head (uniform)
    const int h = kvh * G + g;
    const int stride = d + 2;
    const int i = lane;
    constexpr int dp = d >> 1;
    if (g >= G) return;
    {
        // scores: lane j = position c0 + j, the dimensions in four
        // interleaved partial sums
        const int j = lane;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < du4; c++) {
            const uint4 kk = k_s[j][c];
            const float4 qa = q_s[g][2 * c], qb = q_s[g][2 * c + 1];
            acc[0] = __builtin_fmaf(qa.x, attn_h2f(static_cast<uint16_t>(kk.x)), acc[0]);
            acc[1] = __builtin_fmaf(qa.y, attn_h2f(static_cast<uint16_t>(kk.x >> 16)), acc[1]);
            acc[2] = __builtin_fmaf(qa.z, attn_h2f(static_cast<uint16_t>(kk.y)), acc[2]);
            acc[3] = __builtin_fmaf(qa.w, attn_h2f(static_cast<uint16_t>(kk.y >> 16)), acc[3]);
            acc[0] = __builtin_fmaf(qb.x, attn_h2f(static_cast<uint16_t>(kk.z)), acc[0]);
            acc[1] = __builtin_fmaf(qb.y, attn_h2f(static_cast<uint16_t>(kk.z >> 16)), acc[1]);
            acc[2] = __builtin_fmaf(qb.z, attn_h2f(static_cast<uint16_t>(kk.w)), acc[2]);
            acc[3] = __builtin_fmaf(qb.w, attn_h2f(static_cast<uint16_t>(kk.w >> 16)), acc[3]);
        }
        const float dot = __fadd_rn(__fadd_rn(acc[0], acc[1]), __fadd_rn(acc[2], acc[3]));
        // softmax over the chunk (lane = position; position c0 is visible, so
        // m is finite)
        const float sc = j < valid ? __fmul_rn(dot, a.scale) : -__builtin_inff();
        const float m = wave_max(sc);
        const float p = j < valid ? expf(__fsub_rn(sc, m)) : 0.0f;
        const float l = wave_sum(p);
        p_s[g][j] = p;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        // unnormalised output: lane i = dimensions 2i, 2i + 1; positions in
        // order (p is 0 and the V row is 0 past the valid positions); stored
        // at device scope
        float* my = a.part + (static_cast<size_t>(h) * n_chunks + chunk) * stride;
        const __amdgpu_buffer_rsrc_t pr = buf_rsrc(my, static_cast<uint32_t>(stride) * 4u);
        using u32x2 = unsigned int __attribute__((ext_vector_type(2)));
        if (i < dp) {
            const uint32_t* vw = reinterpret_cast<const uint32_t*>(&v_s[0][0]);
            constexpr int kRowW = kRowU4 * 4;
            float a0 = 0.0f, a1 = 0.0f;
            // 16 positions' V words and p values per round, loaded together
#pragma unroll
            for (int s0 = 0; s0 < kChunk; s0 += 16) {
                uint32_t w2[16];
                float4 p4[4];
#pragma unroll
                for (int t = 0; t < 16; t++) w2[t] = vw[(s0 + t) * kRowW + i];
#pragma unroll
                for (int k = 0; k < 4; k++) p4[k] = *reinterpret_cast<const float4*>(&p_s[g][s0 + 4 * k]);
#pragma unroll
                for (int t = 0; t < 16; t++) {
                    const float4 q4 = p4[t >> 2];
                    const float pv = (t & 3) == 0 ? q4.x : (t & 3) == 1 ? q4.y : (t & 3) == 2 ? q4.z : q4.w;
                    a0 = __builtin_fmaf(pv, attn_h2f(static_cast<uint16_t>(w2[t])), a0);
                    a1 = __builtin_fmaf(pv, attn_h2f(static_cast<uint16_t>(w2[t] >> 16)), a1);
                }
            }
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(a0), __float_as_uint(a1)}, pr,
                                                  (2 + 2 * i) * 4u, 0, kAttnCoherent);
        }
        if (lane == 0)
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(m), __float_as_uint(l)}, pr, 0u, 0,
                                                  kAttnCoherent);
        __builtin_amdgcn_s_waitcnt(0x0F70);                  // vmcnt(0): this wave's part is stored
    }
    // the query head's arrival: one per chunk, the last merges (each wave
    // on its own: no workgroup barrier after the staging)
    unsigned* count = reinterpret_cast<unsigned*>(a.part + static_cast<size_t>(nh) * n_chunks * stride) +
                      h * kCounterStride;
    int last = 0;
    if (lane == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        last = __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               static_cast<unsigned>(n_act - 1);
        if (last) __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!__builtin_amdgcn_readfirstlane(last)) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    {
    // the merge of query head h: lane c takes the (m, l) of chunks c,
    // c + 64, ...: the maximum M over all chunks, the weights e^(m_c - M)
    // and the lane tree of the w_c l_c; lane i then adds w_c o_c for its
    // dimensions 2i, 2i + 1 in chunk order, w_c read from lane c.  The first
    // kMergeBatch chunks' o and the first 64 chunks' (m, l) are loaded in
    // one round; loads past the arrived chunks read 0 and their weights are
    // 0, so they add exactly nothing.
    const float* ph = a.part + static_cast<size_t>(h) * n_chunks * stride;
    const __amdgpu_buffer_rsrc_t hr = buf_rsrc(ph, static_cast<uint32_t>(n_act * stride) * 4u);
    auto ld_ml = [&](int c) {                    // (m, l) of chunk c; (0, 0) past the arrived chunks
        return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                                              hr, static_cast<uint32_t>(c * stride) * 4u, 0, kAttnCoherent));
    };
    auto ld_o = [&](int c) {                     // o[2i], o[2i + 1] of chunk c
        return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                                              hr, static_cast<uint32_t>(c * stride + 2 + 2 * i) * 4u, 0,
                                              kAttnCoherent));
    };
    float2 ob[kMergeBatch];
#pragma unroll
    for (int c = 0; c < kMergeBatch; c++) ob[c] = ld_o(c);
    const float2 ml0 = ld_ml(lane);
    float mloc = lane < n_act ? ml0.x : -__builtin_inff();
    for (int c = lane + 64; c < n_act; c += 64) mloc = fmaxf(mloc, ld_ml(c).x);
    const float M = wave_max(mloc);
    auto weight = [&](float2 ml, int c) {
        return c < n_act && ml.x != -__builtin_inff() ? expf(__fsub_rn(ml.x, M)) : 0.0f;
    };
    float w = weight(ml0, lane);                 // lane c: the weight of chunk c (of this round of 64)
    float lloc = __fmul_rn(ml0.y, w);
    float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int c = 0; c < kMergeBatch; c++) {
        const float wc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), c));
        o0 = __builtin_fmaf(ob[c].x, wc, o0);
        o1 = __builtin_fmaf(ob[c].y, wc, o1);
    }
    for (int c = kMergeBatch; c < n_act; c++) {
        if (c % 64 == 0) {                       // the next round of 64 chunks' weights
            const float2 ml = ld_ml(c + lane);
            w = weight(ml, c + lane);
            lloc = __builtin_fmaf(ml.y, w, lloc);
        }
        const float wc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), c % 64));
        const float2 o = ld_o(c);
        o0 = __builtin_fmaf(o.x, wc, o0);
        o1 = __builtin_fmaf(o.y, wc, o1);
    }
    const float L = wave_sum(lloc);
    if (i < dp) {
        float* dst = a.out + static_cast<size_t>(h) * d + 2 * i;
        dst[0] = __fdiv_rn(o0, L);
        dst[1] = __fdiv_rn(o1, L);
    }
    }
}

}  // namespace q4k
