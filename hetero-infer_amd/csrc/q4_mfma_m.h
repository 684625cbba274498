// Small-M GEMV on the int8 matrix cores (up to 8 activation rows, gs 64; the
// library takes it from 3 rows, below which the streaming kernel is faster).
//
// The arithmetic is the reference's x86 path of kernel/q4gemv.c:232-301 for
// every row of x: x quantised to int16 once per row (:244-270), an exact
// integer dot per group of 64 (:80-111), and per output
//   acc = acc + fma(scale, xscale * (float)idot, bias * xsum[g])   (:173-180)
// in ascending group order.  Only the integer dots move to the MFMA; the fp32
// steps stay in the order above, so the result is bit-identical to the
// streaming kernel and to the reference.
//
// Integer dots.  v_mfma_i32_32x32x32_i8 takes A (32 x 32, int8) from x and
// B (32 x 32, int8) from the weights.  A row of A is one byte plane of one
// activation row; the 32 columns of B are 32 weight rows.  xq = 256 * xh + xl
// with xh the signed high byte and xl the unsigned low byte; A carries
// xl ^ 0x80 (= xl - 128, a signed byte) and xh, plus two rows of ones, so
//   idot = D[xl] + 256 * D[xh] + 128 * D[ones]          (exact in int32)
// Weights are 0..15, already valid signed bytes: the low and high nibbles of
// each packed word go to two MFMAs (even and odd k), and the A operand holds
// the matching even/odd bytes of x.  A rows: 0..7 xl of activation rows
// 0..7, 8..15 xh (loaded), 16 and 20 ones (made in registers), the rest
// zero, which puts every plane an output needs into the same lane of D.
//
// Work split.  A workgroup owns a tile of 32 weight rows (16 when 32-row
// tiles would leave CUs idle; PAIR: 32 gate rows and the same 32 up rows,
// one A operand for both) and runs S waves over K
// in windows of kMfRing*S groups, kMfRing consecutive groups per wave, each
// wave streaming its groups through a register ring of kMfRing (the next
// window's loads are in flight while the window's terms are chained).  Each group's
// fp32 term goes to an LDS table; after a barrier one lane per (activation
// row, weight row) adds the window's terms in ascending group order.  The K
// split keeps enough waves in flight for the 3584-row shapes; the ordered
// chain keeps it exact.
//
// Loads per pair of groups and wave: per matrix two loads of 16 rows x 64
// contiguous bytes (the two groups of each row; 32-byte pieces per row made
// twice the L2 requests), turned into the B operands of the two groups by
// v_permlane16_swap and v_permlane32_swap; per group the A operand (the 32
// lanes of rows 0..15, 32 bytes each) and the xsum of the lane's four
// activation rows.  Scales and biases come once per window: the lane's
// row, 8 groups in 16 bytes (the window's kMfRing of them used), scales in
// k-half 0 and biases in k-half 1, exchanged across the halves (when the
// group count is a multiple of 8; else one 2-byte load each per group).
#pragma once

#include "q4_common.h"

namespace q4k {

// groups per wave and window (ring: 2 slots of 2 groups).  8 groups (4
// slots) measured slower: q_proj at 8 rows 11.45 against 10.9 us, the MLP
// block 61.6 against 61.2 us -- fewer loads queued per CU wait less.
constexpr int kMfRing = 4;
constexpr int kMfArows = 16;        // A rows stored per (group, k-half): xl 0..7, xh 8..15

// x of up to 8 rows, prepared for the small-M MFMA kernel.  Grid (P, 8):
// workgroup (p, m) takes row slot m (slots >= M write zeros) and the p-th
// slice of its groups.  The fp32 steps are xprep_kernel's:
//   xa[((g*2 + h)*16 + r)*8 + s]  uint32: A row r, k-half h of group g;
//                                 s 0..3 even-k bytes of words 4h..4h+3 of
//                                 the group, 4..7 the odd-k bytes
//   xsum_t[g*8 + m], xscale[m]
// Every workgroup of a row stages the whole row in LDS by 16-byte loads all
// issued at once (one memory round trip) and takes its amax; the group sums
// and the quantisation of its slice then read LDS.
constexpr int kMfPrepMaxK = 32768;           // floats of one x row staged in LDS
__global__ __launch_bounds__(1024) void xprep_mf_kernel(const float* __restrict__ x, int M, int n_in,
                                                        uint32_t* __restrict__ xa, float* __restrict__ xsum_t,
                                                        float* __restrict__ xscale_out) {
    extern __shared__ float4 xrow4[];                            // [n_in / 4]
    const int m = blockIdx.y;
    const int tid = threadIdx.x, nt = blockDim.x;
    const int G = n_in >> 6;
    const int gs = (G + gridDim.x - 1) / gridDim.x;              // groups per slice
    const int g0 = blockIdx.x * gs, g1 = g0 + gs < G ? g0 + gs : G;
    if (m >= M) {
        for (int i = g0 * 16 + tid; i < g1 * 16; i += nt) {
            const int s = i & 7, gh = i >> 3;
            xa[(static_cast<size_t>(gh) * kMfArows + m) * 8 + s] = 0u;
            xa[(static_cast<size_t>(gh) * kMfArows + 8 + m) * 8 + s] = 0u;
        }
        for (int g = g0 + tid; g < g1; g += nt) xsum_t[static_cast<size_t>(g) * 8 + m] = 0.0f;
        if (tid == 0 && blockIdx.x == 0) xscale_out[m] = 1.0f;
        return;
    }
    __shared__ float red[16];
    __shared__ float s_inv;
    const float4* xr4 = reinterpret_cast<const float4*>(x + static_cast<size_t>(m) * n_in);
    const int n4 = n_in >> 2;

    // stage the row; amax on the way (kernel/q4gemv.c:258-259, NaN-skipping)
    float amax = 0.0f;
    constexpr int kPer = kMfPrepMaxK / 4 / 1024;                // float4 per thread at most
    float4 v[kPer];
#pragma unroll
    for (int r = 0; r < kPer; r++) {
        const int i = r * nt + tid;
        v[r] = i < n4 ? xr4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int r = 0; r < kPer; r++) {
        const int i = r * nt + tid;
        if (i < n4) {
            xrow4[i] = v[r];
            const float a[4] = {v[r].x, v[r].y, v[r].z, v[r].w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float t = a[k] < 0 ? -a[k] : a[k];
                amax = t > amax ? t : amax;
            }
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        float o = __shfl_xor(amax, off);
        amax = o > amax ? o : amax;
    }
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    if (tid == 0) {
        float a = 0.0f;
        for (int i = 0; i < (nt >> 6); i++) a = red[i] > a ? red[i] : a;
        const float sc = a > 0.0f ? __fdiv_rn(a, 32767.0f) : 1.0f;   // :260
        if (blockIdx.x == 0) xscale_out[m] = sc;
        s_inv = __fdiv_rn(1.0f, sc);                                  // :261
    }
    for (int g = g0 + tid; g < g1; g += nt) {                    // kernel/q4gemv.c:244-248
        const float4* p = xrow4 + g * 16;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float4 q = p[i];
            s = __fadd_rn(s, q.x);
            s = __fadd_rn(s, q.y);
            s = __fadd_rn(s, q.z);
            s = __fadd_rn(s, q.w);
        }
        xsum_t[static_cast<size_t>(g) * 8 + m] = s;
    }
    __syncthreads();
    const float inv = s_inv;
    const float* xl = reinterpret_cast<const float*>(xrow4);
    for (int j = g0 * 8 + tid; j < g1 * 8; j += nt) {
        uint32_t le = 0, lo = 0, he = 0, ho = 0;
#pragma unroll
        for (int n = 0; n < 8; n++) {
            const float a = __fmul_rn(xl[8 * j + n], inv);             // :266
            const float r = a < 0 ? __fsub_rn(a, 0.5f) : __fadd_rn(a, 0.5f);  // :267-268
            const int32_t q = to_i16_like_x86(r);
            const uint32_t xlb = static_cast<uint32_t>(q) & 0xFFu;
            const uint32_t xhb = static_cast<uint32_t>(q >> 8) & 0xFFu;
            const int sh = 8 * (n >> 1);
            if (n & 1) { lo |= xlb << sh; ho |= xhb << sh; }
            else       { le |= xlb << sh; he |= xhb << sh; }
        }
        const int g = j >> 3, h = (j >> 2) & 1, wd = j & 3;
        uint32_t* base = xa + static_cast<size_t>(g * 2 + h) * kMfArows * 8;
        base[m * 8 + wd] = le ^ 0x80808080u;
        base[m * 8 + 4 + wd] = lo ^ 0x80808080u;
        base[(8 + m) * 8 + wd] = he;
        base[(8 + m) * 8 + 4 + wd] = ho;
    }
}

// One ring slot: a pair of consecutive groups.
template <bool PAIR>
struct MfSlot {
    uint4 w[PAIR ? 2 : 1][2];   // per matrix: rows 0..15 and 16..31 of the tile, 64 bytes of each row
                                //   (the pair's two groups) over four lanes; permuted into B at use
    uint4 xe[2], xo[2];         // per group: A operand, even and odd k
    float4 xs[2];               // per group: xsum of activation rows 4h..4h+3
    uint32_t s[PAIR ? 2 : 1][2], b[PAIR ? 2 : 1][2];   // per matrix and group without SB8 (fp16, low half)
};

typedef int mf_v4i __attribute__((ext_vector_type(4)));
typedef int mf_v16i __attribute__((ext_vector_type(16)));

// Weight-side arguments: one matrix, or (PAIR) gate in 0 and up in 1.
struct MfMats {
    const uint32_t* w[2];
    const uint16_t* s[2];
    const uint16_t* b[2];
};

__device__ __forceinline__ mf_v4i lo_nibbles(const uint4& w) {
    return {static_cast<int>(w.x & 0x0F0F0F0Fu), static_cast<int>(w.y & 0x0F0F0F0Fu),
            static_cast<int>(w.z & 0x0F0F0F0Fu), static_cast<int>(w.w & 0x0F0F0F0Fu)};
}
__device__ __forceinline__ mf_v4i hi_nibbles(const uint4& w) {
    return {static_cast<int>((w.x >> 4) & 0x0F0F0F0Fu), static_cast<int>((w.y >> 4) & 0x0F0F0F0Fu),
            static_cast<int>((w.z >> 4) & 0x0F0F0F0Fu), static_cast<int>((w.w >> 4) & 0x0F0F0F0Fu)};
}

// [a0 a1 a2 a3], [b0 b1 b2 b3] (quarters of 16 lanes) -> [a0 b0 a1 b1],
// [a2 b2 a3 b3]: the odd quarters of the first swap with the even quarters
// of the second, then the upper halves of the first with the lower halves
// of the second.
__device__ __forceinline__ void pair_permute(uint32_t i0, uint32_t i1, uint32_t& b0, uint32_t& b1) {
    const auto pq = __builtin_amdgcn_permlane16_swap(i0, i1, false, false);    // [a0 b0 a2 b2], [a1 b1 a3 b3]
    const auto r = __builtin_amdgcn_permlane32_swap(pq[0], pq[1], false, false);
    b0 = r[0];
    b1 = r[1];
}

// fp16 k of the 8 packed in a uint4 (k = 0..7, wave-uniform)
__device__ __forceinline__ uint32_t half_of(const uint4& v, int k) {
    const uint32_t d = k < 2 ? v.x : k < 4 ? v.y : k < 6 ? v.z : v.w;
    return (k & 1) ? d >> 16 : d & 0xFFFFu;
}

// out[m][row] for m < M (PAIR: h[m][row] = SiLU(gate) * up), row stride ldo.
// Grid: one workgroup per tile of TR rows; block: 64 * S threads (S = 4 or
// 8: with the x operand in the ring, two waves per SIMD).
// SB8: the group count is a multiple of 8 (scales/biases by window).
// TR: weight rows per tile, 32, or 16 (B columns 16..31 dead) to spread a
// matrix of few rows over twice the workgroups.
template <bool PAIR, int S, bool SB8, int TR>
__global__ __launch_bounds__(64 * S) void gemv_mfma_kernel(MfMats mt, int N, int K, int M,
                                                         const uint32_t* __restrict__ xa,
                                                         const float* __restrict__ xsum_t,
                                                         const float* __restrict__ xscale,
                                                         float* __restrict__ out, int ldo) {
    constexpr int NM = PAIR ? 2 : 1;
    static_assert(S == 4 || S == 8, "the chain lanes are waves 0..3; the ring fits two waves per SIMD");
    constexpr int GW = kMfRing * S;
    // terms of one window, [NM][GW][8 activation rows][32 weight rows]: a
    // term store (fixed group and row of x) and a chain load (fixed group)
    // touch 32 consecutive floats per half wave, so no bank conflict past
    // the two halves
    extern __shared__ float tbl[];
    const int tid = threadIdx.x;
    const int lane = tid & 63, j = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = K >> 6;
    const int nwin = (G + GW - 1) / GW;
    const uint32_t rowb = static_cast<uint32_t>(K) >> 1;          // bytes of a weight row

    // the lane's weight row; rows past N read 0 and are not stored
    static_assert(TR == 32 || (TR == 16 && !PAIR), "16-row tiles for one matrix");
    const int row = blockIdx.x * TR + j;
    const bool live = row < N && j < TR;
    __amdgpu_buffer_rsrc_t rw[NM], rs[NM], rb[NM];
#pragma unroll
    for (int k = 0; k < NM; k++) {
        rw[k] = buf_rsrc(mt.w[k], static_cast<uint32_t>(N) * rowb);
        rs[k] = buf_rsrc(mt.s[k], static_cast<uint32_t>(N) * G * 2u);
        rb[k] = buf_rsrc(mt.b[k], static_cast<uint32_t>(N) * G * 2u);
    }
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(xa, static_cast<uint32_t>(G) * 2u * kMfArows * 32u);
    const __amdgpu_buffer_rsrc_t rxs = buf_rsrc(xsum_t, static_cast<uint32_t>(G) * 32u);
    // per-lane offsets at group 0, each below 2^31 (the host checks the
    // matrix sizes), and a dead bit OR-ed in after the group's offset is
    // added: rows past N and the A rows not stored read 0 without an access.
    // A group past the last one adds 2^31 itself; the sum of two in-range
    // parts never reaches 2^32.
    // Weight loads: lane l reads row (l % 16) (+16 for the second load) at
    // byte 16 * (l / 16) of the pair's 64 bytes.
    const int lrow = blockIdx.x * TR + (lane & 15);
    const uint32_t olw = static_cast<uint32_t>(lrow < N ? lrow : 0) * rowb + static_cast<uint32_t>(lane >> 4) * 16u;
    const uint32_t deadw0 = lrow < N ? 0u : kOutOfRange, deadw1 = lrow + 16 < N ? 0u : kOutOfRange;
    const uint32_t row16 = 16u * rowb;
    const uint32_t rowc = live ? static_cast<uint32_t>(row) : 0u;
    const uint32_t og = rowc * static_cast<uint32_t>(G) * 2u;
    const uint32_t dead = live ? 0u : kOutOfRange;
    const uint32_t ox = static_cast<uint32_t>(h * kMfArows + (j & 15)) * 32u;
    const uint32_t deadx = j < kMfArows ? 0u : kOutOfRange;
    const uint32_t onesv = (j == 16 || j == 20) ? 0x01010101u : 0u;   // A rows 16 and 20
    const uint32_t oxs = static_cast<uint32_t>(h) * 16u;

    // slot of groups (g, g + 1), g even
    auto load = [&](MfSlot<PAIR>& sl, int g) {
        const bool gv = g < G;                                       // uniform
        const uint32_t dw = gv ? static_cast<uint32_t>(g) * 32u : kOutOfRange;
        __builtin_amdgcn_sched_barrier(0);
        // default cache policy: the 64 bytes a lane group reads share their
        // 128-byte line with the row's next pair, read by the next slot
#pragma unroll
        for (int k = 0; k < NM; k++) {
            sl.w[k][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw[k], (olw + dw) | deadw0, 0, 0));
            if constexpr (TR == 32)
                sl.w[k][1] = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(rw[k], (olw + row16 + dw) | deadw1, 0, 0));
            else
                sl.w[k][1] = make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const bool ge = g + e < G;                               // uniform
            const uint32_t dg = ge ? static_cast<uint32_t>(g + e) * 2u : kOutOfRange;
            const uint32_t dx = ge ? static_cast<uint32_t>(g + e) * (2u * kMfArows * 32u) : kOutOfRange;
            const uint32_t dxs = ge ? static_cast<uint32_t>(g + e) * 32u : kOutOfRange;
            if constexpr (!SB8) {
#pragma unroll
                for (int k = 0; k < NM; k++) {
                    sl.s[k][e] = __builtin_amdgcn_raw_buffer_load_b16(rs[k], (og + dg) | dead, 0, 0);
                    sl.b[k][e] = __builtin_amdgcn_raw_buffer_load_b16(rb[k], (og + dg) | dead, 0, 0);
                }
            }
            sl.xe[e] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, (ox + dx) | deadx, 0, 0));
            sl.xo[e] = __builtin_bit_cast(uint4,
                                          __builtin_amdgcn_raw_buffer_load_b128(rx, (ox + dx + 16u) | deadx, 0, 0));
            sl.xs[e] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rxs, oxs + dxs, 0, 0));
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // SB8: 8 groups of scales (k-half 0) or biases (k-half 1) of the lane's
    // row in 16 bytes, from the window's first group of the wave
    auto load_sb = [&](uint4 (&sb)[NM], int g) {
        const bool gv = g < G;                                       // uniform
        const uint32_t dg = gv ? static_cast<uint32_t>(g) * 2u : kOutOfRange;
        __builtin_amdgcn_sched_barrier(0);
        // both loads on every lane, the other half's through a dead offset:
        // no divergent branch around a load
        const uint32_t ds = h == 0 ? dead : kOutOfRange, db = h == 0 ? kOutOfRange : dead;
#pragma unroll
        for (int k = 0; k < NM; k++) {
            const uint4 a = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs[k], (og + dg) | ds, 0, 0));
            const uint4 c = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rb[k], (og + dg) | db, 0, 0));
            sb[k] = make_uint4(a.x | c.x, a.y | c.y, a.z | c.z, a.w | c.w);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // xscale of the lane's four activation rows (4h .. 4h+3): the eight
    // values by scalar loads (uniform addresses), picked per k-half.  A
    // vector load here would be one more vector-memory result the loop
    // header's wait accounting merges with the ring, and the first group of
    // every window then waited for the whole ring.
    float xsc[4];
    {
        // a bit mask, not a select: a select of the two loads became one
        // load at a per-lane index, i.e. an array in scratch memory
        const uint32_t hm = 0u - static_cast<uint32_t>(h);
#pragma unroll
        for (int mm = 0; mm < 4; mm++)
            xsc[mm] = __uint_as_float((__float_as_uint(xscale[4 + mm]) & hm) | (__float_as_uint(xscale[mm]) & ~hm));
    }

    constexpr int kSlots = kMfRing / 2;
    MfSlot<PAIR> ring[kSlots];
    uint4 sb_next[NM];
    const int g_wave = wave * kMfRing;                               // the wave's first group of a window
    if constexpr (SB8) load_sb(sb_next, g_wave);
#pragma unroll
    for (int d = 0; d < kSlots; d++) load(ring[d], g_wave + 2 * d);

    // chain lanes: waves 0..3, activation row 2*wave + h, weight row j
    const int cm = 2 * wave + h;
    const bool chain = wave < 4 && 2 * wave < M;                     // uniform
    float acc[NM];
#pragma unroll
    for (int k = 0; k < NM; k++) acc[k] = 0.0f;
    for (int t = 0; t < nwin; t++) {
        const int g0 = t * GW + g_wave;
        // this window's scales and biases: own half plus the other half's
        uint4 sv[NM], bv[NM];
        if constexpr (SB8) {
#pragma unroll
            for (int k = 0; k < NM; k++) {
                uint4 other;
                other.x = __shfl_xor(sb_next[k].x, 32);
                other.y = __shfl_xor(sb_next[k].y, 32);
                other.z = __shfl_xor(sb_next[k].z, 32);
                other.w = __shfl_xor(sb_next[k].w, 32);
                sv[k] = h == 0 ? sb_next[k] : other;
                bv[k] = h == 0 ? other : sb_next[k];
            }
            load_sb(sb_next, g0 + GW);
        }
#pragma unroll
        for (int d = 0; d < kSlots; d++) {
            const MfSlot<PAIR>& sl = ring[d];
            // B operands of the slot's two groups: from [a0 a1 a2 a3] (rows
            // 0..15) and [b0 b1 b2 b3] (rows 16..31), quarters of 16 lanes,
            // to [a0 b0 a1 b1] (first group) and [a2 b2 a3 b3] (second)
            mf_v4i bw[NM][2][2];                                     // [matrix][group][even, odd k]
#pragma unroll
            for (int k = 0; k < NM; k++) {
                uint4 b0, b1;
                pair_permute(sl.w[k][0].x, sl.w[k][1].x, b0.x, b1.x);
                pair_permute(sl.w[k][0].y, sl.w[k][1].y, b0.y, b1.y);
                pair_permute(sl.w[k][0].z, sl.w[k][1].z, b0.z, b1.z);
                pair_permute(sl.w[k][0].w, sl.w[k][1].w, b0.w, b1.w);
                bw[k][0][0] = lo_nibbles(b0);
                bw[k][0][1] = hi_nibbles(b0);
                bw[k][1][0] = lo_nibbles(b1);
                bw[k][1][1] = hi_nibbles(b1);
            }
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint4 xe = make_uint4(sl.xe[e].x | onesv, sl.xe[e].y | onesv, sl.xe[e].z | onesv,
                                            sl.xe[e].w | onesv);
                const uint4 xo = make_uint4(sl.xo[e].x | onesv, sl.xo[e].y | onesv, sl.xo[e].z | onesv,
                                            sl.xo[e].w | onesv);
                const mf_v4i ae = __builtin_bit_cast(mf_v4i, xe), ao = __builtin_bit_cast(mf_v4i, xo);
                const float xs4[4] = {sl.xs[e].x, sl.xs[e].y, sl.xs[e].z, sl.xs[e].w};
                const int gi = 2 * d + e;                            // group of the wave's 8
                const int gl = wave * kMfRing + gi;                  // group within the window
#pragma unroll
                for (int k = 0; k < NM; k++) {
                    mf_v16i D = {};
                    D = __builtin_amdgcn_mfma_i32_32x32x32_i8(ae, bw[k][e][0], D, 0, 0, 0);
                    D = __builtin_amdgcn_mfma_i32_32x32x32_i8(ao, bw[k][e][1], D, 0, 0, 0);
                    uint32_t sraw, braw;
                    if constexpr (SB8) {
                        sraw = half_of(sv[k], gi);
                        braw = half_of(bv[k], gi);
                    } else {
                        sraw = sl.s[k][e];
                        braw = sl.b[k][e];
                    }
                    const float sc = h2f(static_cast<uint16_t>(sraw)), bi = h2f(static_cast<uint16_t>(braw));
                    float* tk = tbl + (k * GW + gl) * 256;
#pragma unroll
                    for (int mm = 0; mm < 4; mm++) {
                        // kernel/q4gemv.c:173-180 with xq = 256 xh + (xl' + 128)
                        const int32_t idot = D[mm] + D[4 + mm] * 256 + D[8] * 128;
                        const float dot = __fmul_rn(xsc[mm], static_cast<float>(idot));
                        const float bx = __fmul_rn(bi, xs4[mm]);
                        tk[(4 * h + mm) * 32 + j] = __fmaf_rn(sc, dot, bx);
                    }
                }
            }
            load(ring[d], g0 + GW + 2 * d);                          // the next window's pair
        }
        __syncthreads();
        if (chain) {
            const int n = G - t * GW < GW ? G - t * GW : GW;
#pragma unroll
            for (int k = 0; k < NM; k++) {
                const float* tp = tbl + k * GW * 256 + cm * 32 + j;
                float a = acc[k];
                int g = 0;
                for (; g + 8 <= n; g += 8) {
                    float v[8];
#pragma unroll
                    for (int i = 0; i < 8; i++) v[i] = tp[(g + i) * 256];
#pragma unroll
                    for (int i = 0; i < 8; i++) a = __fadd_rn(a, v[i]);
                }
                for (; g < n; g++) a = __fadd_rn(a, tp[g * 256]);
                acc[k] = a;
            }
        }
        __syncthreads();
    }
    if (!chain || !live || cm >= M) return;
    if constexpr (PAIR)
        out[static_cast<size_t>(cm) * ldo + row] = silu_mul(acc[0], acc[1]);
    else
        out[static_cast<size_t>(cm) * ldo + row] = acc[0];
}

}  // namespace q4k
