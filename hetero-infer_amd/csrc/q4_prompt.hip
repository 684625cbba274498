// Causal grouped-query attention of a prompt chunk over the fp16 KV cache
// (gfx950), the attention of the device-resident prompt forward.  Declared
// in q4decode.h (q4_prompt_attention_dev).
//
// hetero/cpu_model.py:233-252 (sdpa with causal=True, L > 1): query row r
// of a chunk that starts at position pos0 sits at position pos0 + r and
// sees the positions [0, pos0 + r] -- the reference's mask
// `arange(S) <= arange(L) + (S - L)` with S = pos0 + L; query head h reads
// kv head h / (nh / nkv); s = (q . k) * scale, softmax over the visible
// positions, o = sum p v.
//
// A workgroup takes one kv head and four consecutive query rows (one per
// wave) for all G query heads that share the kv head, and walks the cache
// in tiles of 64 positions up to the last position its rows see: the tile's
// K and V rows are staged in LDS once for the 4 x G queries.  Per tile a
// wave computes the scores of its row with lane = position (the K row from
// LDS, the query broadcast from LDS), updates a running softmax (running
// maximum m, sum l, and the output rescaled by e^(m_old - m_new)), and adds
// p v with lane = pair of output dimensions.  The softmax is therefore
// evaluated online, tile by tile, not as the reference's one max and one
// sum over the whole row: the results agree to fp32 rounding, not bit for
// bit.  Workgroups of the last rows, which see the most positions, are
// launched first.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "q4_common.h"
#include "q4decode.h"

namespace q4k {
namespace {

constexpr int kPTile = 64;                  // positions per tile
constexpr int kPRows = 4;                   // query rows per workgroup: one per wave
constexpr int kPMaxG = 8;                   // query heads per kv head
constexpr int kPMaxD = 128;
constexpr int kPRowU4 = kPMaxD / 8 + 1;     // LDS row of K / V: 16 uint4 of fp16 + 1 pad (reads spread over the banks)

struct PromptAttnArgs {
    const float* q;          // [rows][nh * d], rotated queries
    const uint16_t* kc;      // [nkv][cap][d] fp16
    const uint16_t* vc;
    void* out;               // [rows][nh * d], fp32 or (BF) bf16
    int rows;
    int64_t pos0;
    int nh, nkv, d, cap;
    float scale;
};

__device__ __forceinline__ float p_h2f(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// LDS stores by some lanes of a wave are visible to the other lanes' later
// loads (the wave's LDS operations complete in order).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

template <int G, int D, bool BF>
__global__ __launch_bounds__(64 * kPRows) void prompt_attn_kernel(PromptAttnArgs a) {
    __shared__ uint4 k_s[kPTile][kPRowU4];
    __shared__ uint4 v_s[kPTile][kPRowU4];
    __shared__ float4 q_s[kPRows][G][kPMaxD / 4];
    __shared__ float4 p_s[kPRows][G][kPTile / 4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: the row's branches stay scalar
    const int kvh = blockIdx.y;
    const int r0 = (static_cast<int>(gridDim.x) - 1 - static_cast<int>(blockIdx.x)) * kPRows;
    const int r = r0 + wave;                                   // this wave's query row
    const bool row_ok = r < a.rows;                            // wave-uniform
    constexpr int d = D, du4 = d >> 3, dp = d >> 1, dq = d >> 2;
    const int hd = a.nh * d;
    const int last_row = (r0 + kPRows < a.rows ? r0 + kPRows : a.rows) - 1;
    const int64_t wg_last = a.pos0 + last_row;                 // the last position a row of the workgroup sees
    const int64_t my_last = a.pos0 + r;                        // the last position this row sees
    const int n_tiles = static_cast<int>(wg_last / kPTile) + 1;
    if (row_ok) {
        const float4* src = reinterpret_cast<const float4*>(a.q + static_cast<size_t>(r) * hd +
                                                            static_cast<size_t>(kvh) * G * d);
        for (int e = lane; e < G * dq; e += 64) q_s[wave][e / dq][e % dq] = src[e];
    }
    float m[G], l[G], o0[G], o1[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -__builtin_inff();
        l[g] = o0[g] = o1[g] = 0.0f;
    }
    const size_t head_row0 = static_cast<size_t>(kvh) * a.cap;
    for (int t = 0; t < n_tiles; t++) {
        const int64_t c0 = static_cast<int64_t>(t) * kPTile;
        const int valid = static_cast<int>(wg_last + 1 - c0 < kPTile ? wg_last + 1 - c0 : kPTile);
        __syncthreads();                                       // the last tile's K, V and p are read
        // K and V rows [c0, c0 + valid); the rows past them read 0 (past the
        // end of the buffer resource), so p = 0 never meets a stale value
        const uint32_t bytes = static_cast<uint32_t>(valid) * static_cast<uint32_t>(d) * 2u;
        const __amdgpu_buffer_rsrc_t kr = buf_rsrc(a.kc + (head_row0 + c0) * d, bytes);
        const __amdgpu_buffer_rsrc_t vr = buf_rsrc(a.vc + (head_row0 + c0) * d, bytes);
        for (int e = tid; e < kPTile * du4; e += 64 * kPRows) {
            const int row = e / du4, c = e - row * du4;
            const uint32_t off = static_cast<uint32_t>(e) * 16u;
            k_s[row][c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0));
            v_s[row][c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0));
        }
        __syncthreads();
        if (!row_ok || c0 > my_last) continue;                 // wave-uniform: nothing this row sees
        // scores: lane j = position c0 + j; dims in ascending order
        const int j = lane;
        float acc[G];
#pragma unroll
        for (int g = 0; g < G; g++) acc[g] = 0.0f;
#pragma unroll
        for (int c = 0; c < du4; c++) {
            const uint4 kk = k_s[j][c];
            const float kf[8] = {p_h2f(kk.x), p_h2f(kk.x >> 16), p_h2f(kk.y), p_h2f(kk.y >> 16),
                                 p_h2f(kk.z), p_h2f(kk.z >> 16), p_h2f(kk.w), p_h2f(kk.w >> 16)};
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float4 qa = q_s[wave][g][2 * c], qb = q_s[wave][g][2 * c + 1];
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
        // the running softmax (every tile a row reaches holds position c0 <=
        // my_last, so the tile's maximum is finite)
        const bool vis = c0 + j <= my_last;
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float s = vis ? __fmul_rn(acc[g], a.scale) : -__builtin_inff();
            const float mn = fmaxf(m[g], wave_max(s));
            const float corr = expf(__fsub_rn(m[g], mn));       // 0 on the row's first tile
            const float p = vis ? expf(__fsub_rn(s, mn)) : 0.0f;
            l[g] = __fadd_rn(__fmul_rn(l[g], corr), wave_sum(p));
            o0[g] = __fmul_rn(o0[g], corr);
            o1[g] = __fmul_rn(o1[g], corr);
            m[g] = mn;
            reinterpret_cast<float*>(&p_s[wave][g][0])[j] = p;
        }
        wave_lds_sync();
        // o += p v: lane = pair of dimensions; positions in ascending order
        if (lane < dp) {
            const uint32_t* vw = reinterpret_cast<const uint32_t*>(&v_s[0][0]);
            constexpr int kRowW = kPRowU4 * 4;
            // every position of the tile: p is 0 past the row's last one
#pragma unroll 4
            for (int j0 = 0; j0 < kPTile; j0 += 4) {
                uint32_t w2[4];
#pragma unroll
                for (int jj = 0; jj < 4; jj++) w2[jj] = vw[(j0 + jj) * kRowW + lane];
                float4 pg[G];
#pragma unroll
                for (int g = 0; g < G; g++) pg[g] = p_s[wave][g][j0 >> 2];
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const float v0 = p_h2f(w2[jj]), v1 = p_h2f(w2[jj] >> 16);
#pragma unroll
                    for (int g = 0; g < G; g++) {
                        const float p = jj == 0 ? pg[g].x : jj == 1 ? pg[g].y : jj == 2 ? pg[g].z : pg[g].w;
                        o0[g] = __builtin_fmaf(p, v0, o0[g]);
                        o1[g] = __builtin_fmaf(p, v1, o1[g]);
                    }
                }
            }
        }
        wave_lds_sync();
    }
    if (row_ok && lane < dp) {
        const size_t at = static_cast<size_t>(r) * hd + static_cast<size_t>(kvh) * G * d + 2 * lane;
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float v0 = __fdiv_rn(o0[g], l[g]), v1 = __fdiv_rn(o1[g], l[g]);
            if constexpr (BF) {
                *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.out) + at + g * d) = bf16x2_rne(v0, v1);
            } else {
                float* dst = static_cast<float*>(a.out) + at + g * d;
                dst[0] = v0;
                dst[1] = v1;
            }
        }
    }
}

// ---------------------------------------------------------------------
// head_dim 128 on the matrix cores (v_mfma_f32_16x16x32_f16).  A workgroup
// takes one kv head and 16 consecutive query rows, a wave per query head of
// the kv head (G waves), and walks the cache in tiles of 64 positions; the
// tile's K rows (k_s, row-major) and V rows (vt_s, transposed: [dim][pos])
// are staged in LDS once for the G heads, the next tile's loads in flight
// while the current one is multiplied.
//
// Per tile and wave, with lane l: c = l % 16 (a query row of the block),
// qd = l / 16:
//   S^T = K Q^T: 4 x 4 MFMAs; lane l ends with query row c's scores at
//     positions 16 mt + 4 qd + v (mt, v = 0..3);
//   the running softmax of row c (its 64 scores sit in lanes c, c + 16,
//     c + 32, c + 48: a max and a sum over the lane's 16, then across the
//     four lanes);
//   O^T += V^T P^T: 8 x 2 MFMAs; lane l holds query row c's outputs at
//     dims 16 dt + 4 qd + v, rescaled by the row's correction in place.
// The MFMA operands are fp16, the sums fp32.  Exact fp16 operands: the
// cache is fp16, and q and p enter as two fp16 terms each (pa_split), two
// MFMAs per product -- x to about 2^-21 of its value (or 2^-25
// absolutely), so the scores and weighted sums keep fp32 accuracy.  q is multiplied by scale * log2(e) first and the softmax
// taken with exp2, which is exp of the scaled score.
constexpr int kMRows = 16;                  // query rows per workgroup
constexpr int kKRowH = kPMaxD + 8;          // k_s row: 128 fp16 + 8 pad (272 bytes: 16-byte reads spread)
constexpr int kVRowH = kPTile + 4;          // vt_s row: 64 fp16 + 4 pad (136 bytes)
constexpr int kKChunks = kPTile * kPMaxD / 8;      // 16-byte chunks of a K tile (1024)
constexpr int kVPairs = kPTile / 2 * kPMaxD / 8;   // (position pair, 8 dims) items of a V tile (512)

typedef _Float16 pa_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 pa_h4 __attribute__((ext_vector_type(4)));
typedef float pa_f4 __attribute__((ext_vector_type(4)));

template <int NT>
struct PaStage {                            // one thread's share of a tile's loads
    uint4 k[(kKChunks + NT - 1) / NT];
    uint4 v0[(kVPairs + NT - 1) / NT], v1[(kVPairs + NT - 1) / NT];
};

template <int NT>
__device__ __forceinline__ void pa_load(PaStage<NT>& st, const PromptAttnArgs& a, size_t head_row0, int64_t c0,
                                        int valid, int tid) {
    const uint32_t bytes = static_cast<uint32_t>(valid) * kPMaxD * 2u;
    const __amdgpu_buffer_rsrc_t kr = buf_rsrc(a.kc + (head_row0 + c0) * kPMaxD, bytes);
    const __amdgpu_buffer_rsrc_t vr = buf_rsrc(a.vc + (head_row0 + c0) * kPMaxD, bytes);
#pragma unroll
    for (int i = 0; i < (kKChunks + NT - 1) / NT; i++) {
        const int e = tid + i * NT;
        const uint32_t off = e < kKChunks ? static_cast<uint32_t>(e) * 16u : kOutOfRange;
        st.k[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < (kVPairs + NT - 1) / NT; i++) {
        const int e = tid + i * NT;                 // pair pp = e / 16 (positions 2 pp, 2 pp + 1), dims 8 (e % 16) ..
        const uint32_t off = e < kVPairs ? static_cast<uint32_t>((e >> 4) * 2 * kPMaxD + (e & 15) * 8) * 2u
                                         : kOutOfRange;
        st.v0[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0));
        st.v1[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, off + kPMaxD * 2, 0, 0));
    }
}

template <int NT>
__device__ __forceinline__ void pa_store(const PaStage<NT>& st, _Float16* k_s, _Float16* vt_s, int tid) {
#pragma unroll
    for (int i = 0; i < (kKChunks + NT - 1) / NT; i++) {
        const int e = tid + i * NT;
        if (e < kKChunks) *reinterpret_cast<uint4*>(k_s + (e >> 4) * kKRowH + (e & 15) * 8) = st.k[i];
    }
#pragma unroll
    for (int i = 0; i < (kVPairs + NT - 1) / NT; i++) {
        const int e = tid + i * NT;
        if (e < kVPairs) {
            const int pp = e >> 4, d0 = (e & 15) * 8;
            const uint32_t a[4] = {st.v0[i].x, st.v0[i].y, st.v0[i].z, st.v0[i].w};
            const uint32_t b[4] = {st.v1[i].x, st.v1[i].y, st.v1[i].z, st.v1[i].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                // dims d0 + 2j and d0 + 2j + 1: (pos 2pp, pos 2pp + 1) each
                *reinterpret_cast<uint32_t*>(vt_s + (d0 + 2 * j) * kVRowH + 2 * pp) =
                    __builtin_amdgcn_perm(b[j], a[j], 0x05040100u);
                *reinterpret_cast<uint32_t*>(vt_s + (d0 + 2 * j + 1) * kVRowH + 2 * pp) =
                    __builtin_amdgcn_perm(b[j], a[j], 0x07060302u);
            }
        }
    }
}

// x = hi + lo in fp16: hi is x with its low 13 significand bits cleared,
// which fp16 holds exactly whenever |x| >= 2^-14, so no conversion of it can
// round (the compiler may convert it again, packed, for the MFMA operand:
// any rounding mode gives the same value); lo = fp16(x - hi), x - hi exact
// in fp32.  Below 2^-14 the pair is within 2^-25 of x.
__device__ __forceinline__ void pa_split(float x, _Float16& hi, _Float16& lo) {
    const float h = __uint_as_float(__float_as_uint(x) & 0xFFFFE000u);
    hi = static_cast<_Float16>(h);
    lo = static_cast<_Float16>(__fsub_rn(x, h));
}

template <int G, bool BF>
__global__ __launch_bounds__(64 * G) void prompt_attn_mfma_kernel(PromptAttnArgs a) {
    constexpr int NT = 64 * G, D = kPMaxD;
    __shared__ __attribute__((aligned(16))) _Float16 k_s[kPTile * kKRowH];
    __shared__ __attribute__((aligned(16))) _Float16 vt_s[D * kVRowH];
    const int tid = threadIdx.x, lane = tid & 63;
    const int h = __builtin_amdgcn_readfirstlane(tid >> 6);     // query head h of the kv head
    const int c = lane & 15, qd = lane >> 4;
    const int kvh = blockIdx.y;
    const int r0 = (static_cast<int>(gridDim.x) - 1 - static_cast<int>(blockIdx.x)) * kMRows;
    const int last_row = (r0 + kMRows < a.rows ? r0 + kMRows : a.rows) - 1;
    const int64_t wg_last = a.pos0 + last_row;
    const int r = r0 + c;                                      // lane's query row
    const int64_t my_last = a.pos0 + (r < last_row ? r : last_row);
    const int n_tiles = static_cast<int>(wg_last / kPTile) + 1;
    const int hd = a.nh * D;
    const size_t head_row0 = static_cast<size_t>(kvh) * a.cap;

    PaStage<NT> st;
    pa_load<NT>(st, a, head_row0, 0, static_cast<int>(wg_last + 1 < kPTile ? wg_last + 1 : kPTile), tid);

    // q of row r, head kvh G + h, as the B operand of S^T: dims 32 ks + 8 qd ..
    const float qs = __fmul_rn(a.scale, 1.44269504088896341f);
    pa_h8 qh[4], ql[4];
    {
        const float* src = a.q + static_cast<size_t>(r) * hd + static_cast<size_t>(kvh * G + h) * D + 8 * qd;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
            if (r < a.rows) {
                x0 = reinterpret_cast<const float4*>(src + 32 * ks)[0];
                x1 = reinterpret_cast<const float4*>(src + 32 * ks)[1];
            }
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                _Float16 hi, lo;
                pa_split(__fmul_rn(xv[i], qs), hi, lo);
                qh[ks][i] = hi;
                ql[ks][i] = lo;
            }
        }
    }
    pa_f4 o[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++) o[dt] = pa_f4{0.f, 0.f, 0.f, 0.f};
    float m = -__builtin_inff(), l = 0.0f;

    for (int t = 0; t < n_tiles; t++) {
        const int64_t c0 = static_cast<int64_t>(t) * kPTile;
        __syncthreads();                                       // every wave is done with the last tile
        pa_store<NT>(st, k_s, vt_s, tid);
        __syncthreads();
        if (t + 1 < n_tiles) {
            const int64_t c1 = c0 + kPTile;
            pa_load<NT>(st, a, head_row0, c1, static_cast<int>(wg_last + 1 - c1 < kPTile ? wg_last + 1 - c1 : kPTile),
                        tid);
        }
        // S^T = K Q^T: s[mt][v] = score of row r at position c0 + 16 mt + 4 qd + v
        pa_f4 s[4];
#pragma unroll
        for (int mt = 0; mt < 4; mt++) {
            s[mt] = pa_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const pa_h8 kf = *reinterpret_cast<const pa_h8*>(k_s + (16 * mt + c) * kKRowH + 32 * ks + 8 * qd);
                s[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[ks], s[mt], 0, 0, 0);
                s[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[ks], s[mt], 0, 0, 0);
            }
        }
        // the running softmax of row r
        float mx = -__builtin_inff();
#pragma unroll
        for (int mt = 0; mt < 4; mt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const bool vis = c0 + 16 * mt + 4 * qd + v <= my_last;
                s[mt][v] = vis ? s[mt][v] : -__builtin_inff();
                mx = fmaxf(mx, s[mt][v]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);                         // finite: position 0 is in every row's first tile
        const float corr = __builtin_amdgcn_exp2f(__fsub_rn(m, mn));
        m = mn;
        float ps = 0.0f;
        pa_h8 ph[2], pl[2];
#pragma unroll
        for (int mt = 0; mt < 4; mt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float p = __builtin_amdgcn_exp2f(__fsub_rn(s[mt][v], mn));   // 0 where masked
                ps = __fadd_rn(ps, p);
                _Float16 hi, lo;
                pa_split(p, hi, lo);
                ph[mt >> 1][(mt & 1) * 4 + v] = hi;
                pl[mt >> 1][(mt & 1) * 4 + v] = lo;
            }
        ps = __fadd_rn(ps, __shfl_xor(ps, 16));
        ps = __fadd_rn(ps, __shfl_xor(ps, 32));
        l = __fadd_rn(__fmul_rn(l, corr), ps);
        // O^T = O^T corr + V^T P^T; k index 8 qd + i of step kk is position
        // 32 kk + 4 qd + i (i < 4) or 32 kk + 16 + 4 qd + i - 4
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            o[dt] *= corr;
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                const _Float16* vrow = vt_s + (16 * dt + c) * kVRowH + 32 * kk + 4 * qd;
                const pa_h4 v0 = *reinterpret_cast<const pa_h4*>(vrow);
                const pa_h4 v1 = *reinterpret_cast<const pa_h4*>(vrow + 16);
                const pa_h8 vf = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, ph[kk], o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl[kk], o[dt], 0, 0, 0);
            }
        }
    }
    if (r < a.rows) {
        const size_t at = static_cast<size_t>(r) * hd + static_cast<size_t>(kvh * G + h) * D + 4 * qd;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const float v0 = __fdiv_rn(o[dt][0], l), v1 = __fdiv_rn(o[dt][1], l);
            const float v2 = __fdiv_rn(o[dt][2], l), v3 = __fdiv_rn(o[dt][3], l);
            if constexpr (BF) {
                *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + at + 16 * dt) =
                    make_uint2(bf16x2_rne(v0, v1), bf16x2_rne(v2, v3));
            } else {
                *reinterpret_cast<float4*>(static_cast<float*>(a.out) + at + 16 * dt) = make_float4(v0, v1, v2, v3);
            }
        }
    }
}

int launch_failed(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q4_EHIP, "%s launch: %s", what, hipGetErrorString(e));
    return 0;
}

}  // namespace
}  // namespace q4k

using namespace q4k;

namespace {

int prompt_attention(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, void* out, bool bf, int rows,
                     int64_t pos0, int n_heads, int n_kv, int head_dim, int cap, float scale, void* stream) {
    if (!q || !k_cache || !v_cache || !out) return fail(Q4_EARG, "q4_prompt_attention_dev: null pointer");
    if (n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || n_heads / n_kv > kPMaxG ||
        (head_dim != 32 && head_dim != 64 && head_dim != 128) || cap <= 0)
        return fail(Q4_EARG, "q4_prompt_attention_dev: unsupported sizes (heads %d, kv heads %d, head_dim %d, cap %d)",
                    n_heads, n_kv, head_dim, cap);
    if (rows < 0 || pos0 < 0 || pos0 + rows > cap)
        return fail(Q4_EARG, "q4_prompt_attention_dev: rows at positions [%lld, %lld) outside the cache [0, %d)",
                    static_cast<long long>(pos0), static_cast<long long>(pos0 + rows), cap);
    if ((reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(out) & 15) ||
        (reinterpret_cast<uintptr_t>(k_cache) & 15) || (reinterpret_cast<uintptr_t>(v_cache) & 15))
        return fail(Q4_EARG, "q4_prompt_attention_dev: q, out and the caches must be 16-byte aligned");
    if (rows == 0) return 0;
    const PromptAttnArgs a{q, k_cache, v_cache, out, rows, pos0, n_heads, n_kv, head_dim, cap, scale};
    const dim3 grid((rows + kPRows - 1) / kPRows, n_kv);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (head_dim == 128) {
        const dim3 mgrid((rows + kMRows - 1) / kMRows, n_kv);
        switch (n_heads / n_kv) {
#define Q4_PROMPT_M(g)                                                                                         \
    case g:                                                                                                    \
        if (bf) hipLaunchKernelGGL((prompt_attn_mfma_kernel<g, true>), mgrid, dim3(64 * g), 0, st, a);        \
        else hipLaunchKernelGGL((prompt_attn_mfma_kernel<g, false>), mgrid, dim3(64 * g), 0, st, a);          \
        break;
            Q4_PROMPT_M(1) Q4_PROMPT_M(2) Q4_PROMPT_M(3) Q4_PROMPT_M(4)
            Q4_PROMPT_M(5) Q4_PROMPT_M(6) Q4_PROMPT_M(7) Q4_PROMPT_M(8)
#undef Q4_PROMPT_M
            default: break;
        }
        return launch_failed("q4_prompt_attention_dev");
    }
    switch (n_heads / n_kv) {
#define Q4_PROMPT_D(g, dd)                                                                                  \
    if (bf) hipLaunchKernelGGL((prompt_attn_kernel<g, dd, true>), grid, dim3(64 * kPRows), 0, st, a);          \
    else hipLaunchKernelGGL((prompt_attn_kernel<g, dd, false>), grid, dim3(64 * kPRows), 0, st, a);
#define Q4_PROMPT_CASE(g)                                                                                   \
    case g:                                                                                                 \
        if (head_dim == 128) { Q4_PROMPT_D(g, 128) }                                                         \
        else if (head_dim == 64) { Q4_PROMPT_D(g, 64) }                                                      \
        else { Q4_PROMPT_D(g, 32) }                                                                          \
        break;
        Q4_PROMPT_CASE(1) Q4_PROMPT_CASE(2) Q4_PROMPT_CASE(3) Q4_PROMPT_CASE(4)
        Q4_PROMPT_CASE(5) Q4_PROMPT_CASE(6) Q4_PROMPT_CASE(7) Q4_PROMPT_CASE(8)
#undef Q4_PROMPT_CASE
#undef Q4_PROMPT_D
        default: break;
    }
    return launch_failed("q4_prompt_attention_dev");
}

}  // namespace

#pragma GCC visibility push(default)
extern "C" {

int q4_prompt_attention_dev(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out, int rows,
                            int64_t pos0, int n_heads, int n_kv, int head_dim, int cap, float scale, void* stream) {
    return prompt_attention(q, k_cache, v_cache, out, false, rows, pos0, n_heads, n_kv, head_dim, cap, scale, stream);
}

int q4_prompt_attention_bf16_dev(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out,
                                 int rows, int64_t pos0, int n_heads, int n_kv, int head_dim, int cap, float scale,
                                 void* stream) {
    return prompt_attention(q, k_cache, v_cache, out, true, rows, pos0, n_heads, n_kv, head_dim, cap, scale, stream);
}

}  // extern "C"
#pragma GCC visibility pop
