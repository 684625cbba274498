// MI355X (gfx950 / CDNA4) int4 GEMV library: kernels and the C-ABI.
//
// What is computed is the reference kernel/q4gemv.c on x86, bit for bit:
//   prologue (kernel/q4gemv.c:242-272): xsum[g] sequential fp32 sum of each
//     group, xscale = amax/32767 (1 if amax == 0), inv = 1/xscale,
//     xq[i] = (int16)(x*inv +- 0.5) truncated;
//   per row o (kernel/q4gemv.c:158-183):
//     acc = 0; for g ascending:
//       idot = sum_{i in g} q[o][i]*xq[i]            (exact int32)
//       acc  = acc + fma(scale, xscale*(float)idot, bias*xsum[g])
// The integer part is order-free, so it is computed wide across lanes; only
// the per-row chain over groups keeps the reference order, and it is run with
// one lane per row after a transpose through LDS.
//
// Kernel layout (decode is an HBM stream of packed weights):
//   * a chunk is 256 consecutive words (2048 values) of one row; lane l of a
//     wave loads words [4l, 4l+4) of the chunk as one 128-bit load, so one
//     wave-load instruction moves 1 KiB of one row, fully coalesced;
//   * x is pre-split once per call into int8 high and uint8 low planes laid
//     out to match the nibble split of a weight word (w & 0x0F0F0F0F gives
//     the even values, (w >> 4) & 0x0F0F0F0F the odd ones), so a word costs
//     two bit ops and four v_dot4 (sdot4 on the high plane, udot4 on the low);
//     each wave keeps its chunk's x planes in registers and reuses them
//     across every row of the workgroup's row tile;
//   * the lanes of one group combine their partial integer dots with DPP,
//     the group's leader lane forms the fp32 term and writes it to an LDS
//     table T[m][row][group]; after a barrier one lane per (m, row) adds the
//     row's terms in ascending group order.
//
// Everything is compiled with -ffp-contract=off: the only fused multiply-adds
// are the explicit fmaf calls that mirror the reference's own contractions.

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "q4gemv.h"

namespace {

constexpr int kChunkWords = 256;   // words per wave chunk: 64 lanes x 4 words
constexpr int kMaxM = 8;           // activation rows per main-kernel launch
constexpr int kLdsBudget = 64 * 1024;

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

// --------------------------------------------------------------- prologue --
//
// One workgroup per activation row.  Writes, for row m:
//   planes[m][j] = {xl even, xl odd, xh even, xh odd} bytes of word j
//   xsum[m][g], xscale[m]
__global__ __launch_bounds__(1024) void xprep_kernel(
    const float* __restrict__ x, int n_in, int gs, uint4* __restrict__ planes,
    float* __restrict__ xsum, float* __restrict__ xscale_out) {
    const int m = blockIdx.x;
    const float* xr = x + static_cast<size_t>(m) * n_in;
    const int tid = threadIdx.x, nt = blockDim.x;
    __shared__ float red[16];
    __shared__ float s_inv;

    float amax = 0.0f;                                  // kernel/q4gemv.c:258-259
    for (int i = tid; i < n_in; i += nt) {
        float v = xr[i];
        v = v < 0 ? -v : v;
        amax = v > amax ? v : amax;
    }
    for (int off = 32; off > 0; off >>= 1) {
        float o = __shfl_xor(amax, off);
        amax = o > amax ? o : amax;
    }
    if ((tid & 63) == 0) red[tid >> 6] = amax;

    const int n_groups = n_in / gs;                     // kernel/q4gemv.c:244-248
    for (int g = tid; g < n_groups; g += nt) {
        const float* p = xr + static_cast<size_t>(g) * gs;
        float s = 0.0f;
        for (int base = 0; base < gs; base += 32) {   // gs % 64 == 0; 32 loads in flight
            float v[32];
#pragma unroll
            for (int i = 0; i < 32; i++) v[i] = p[base + i];
#pragma unroll
            for (int i = 0; i < 32; i++) s = __fadd_rn(s, v[i]);
        }
        xsum[static_cast<size_t>(m) * n_groups + g] = s;
    }
    __syncthreads();
    if (tid == 0) {
        float a = 0.0f;
        for (int i = 0; i < (nt >> 6); i++) a = red[i] > a ? red[i] : a;
        const float sc = a > 0.0f ? __fdiv_rn(a, 32767.0f) : 1.0f;   // :260
        xscale_out[m] = sc;
        s_inv = __fdiv_rn(1.0f, sc);                                  // :261
    }
    __syncthreads();
    const float inv = s_inv;
    const int wpr = n_in >> 3;
    for (int j = tid; j < wpr; j += nt) {
        uint32_t le = 0, lo = 0, he = 0, ho = 0;
#pragma unroll
        for (int n = 0; n < 8; n++) {
            const float a = __fmul_rn(xr[8 * j + n], inv);             // :266
            const float r = a < 0 ? __fsub_rn(a, 0.5f) : __fadd_rn(a, 0.5f);  // :267-268
            const int32_t q = to_i16_like_x86(r);
            const uint32_t xl = static_cast<uint32_t>(q) & 0xFFu;
            const uint32_t xh = static_cast<uint32_t>(q >> 8) & 0xFFu;
            const int sh = 8 * (n >> 1);
            if (n & 1) { lo |= xl << sh; ho |= xh << sh; }
            else       { le |= xl << sh; he |= xh << sh; }
        }
        planes[static_cast<size_t>(m) * wpr + j] = make_uint4(le, lo, he, ho);
    }
}

// ------------------------------------------------------------ main GEMV ----
//
// grid.x = ceil(n_out / R); block = 64 * nwaves.  Wave w handles chunks
// w, w + nwaves, ...; for each it loads the chunk's x planes once and runs
// every row of the tile.  Requires gs a power of two in [64, 2048] (groups
// never straddle a chunk) and w 16-byte aligned.
template <int MR>
constexpr int main_threads() { return MR <= 2 ? 1024 : (MR <= 4 ? 512 : 256); }

template <int MR>
__global__ __launch_bounds__(main_threads<MR>()) void gemv_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ sc,
    const uint16_t* __restrict__ bi, const uint4* __restrict__ planes,
    const float* __restrict__ xsum, const float* __restrict__ xscale,
    float* __restrict__ out, int n_out, int n_in, int gs, int R, int Gp) {
    extern __shared__ float T[];                 // [MR][R][Gp]
    const int wpr = n_in >> 3, n_groups = n_in / gs;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int row0 = blockIdx.x * R;
    const int n_chunks = (wpr + kChunkWords - 1) / kChunkWords;
    const int wpg = gs >> 3;                     // words per group
    const int lpg = gs >> 5;                     // lanes per group

    for (int c = wave; c < n_chunks; c += nwaves) {
        const int word0 = c * kChunkWords + lane * 4;
        const bool active = word0 < wpr;
        const int g = word0 / wpg;
        const bool leader = active && (lane & (lpg - 1)) == 0;

        uint32_t xle[MR][4], xlo[MR][4], xhe[MR][4], xho[MR][4];
        float xs[MR], xsc[MR];
#pragma unroll
        for (int m = 0; m < MR; m++) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                uint4 p = active ? planes[static_cast<size_t>(m) * wpr + word0 + t]
                                 : make_uint4(0, 0, 0, 0);
                xle[m][t] = p.x; xlo[m][t] = p.y; xhe[m][t] = p.z; xho[m][t] = p.w;
            }
            xs[m] = leader ? xsum[static_cast<size_t>(m) * n_groups + g] : 0.0f;
            xsc[m] = xscale[m];
        }

        for (int r = 0; r < R; r += 4) {
            uint4 wv[4];
            uint16_t s16[4], b16[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int o = row0 + r + u;
                const bool valid = active && (r + u < R) && o < n_out;
                wv[u] = valid ? *reinterpret_cast<const uint4*>(w + static_cast<size_t>(o) * wpr + word0)
                              : make_uint4(0, 0, 0, 0);
                const size_t si = static_cast<size_t>(valid ? o : 0) * n_groups + g;
                s16[u] = (valid && leader) ? sc[si] : uint16_t(0);
                b16[u] = (valid && leader) ? bi[si] : uint16_t(0);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t wd[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
                uint32_t lo4[4], hi4[4];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    lo4[t] = wd[t] & 0x0F0F0F0Fu;          // values 8j+0,2,4,6
                    hi4[t] = (wd[t] >> 4) & 0x0F0F0F0Fu;   // values 8j+1,3,5,7
                }
                int part[MR];
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    int ah = 0;
                    uint32_t al = 0;
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        ah = __builtin_amdgcn_sdot4(static_cast<int>(lo4[t]), static_cast<int>(xhe[m][t]), ah, false);
                        ah = __builtin_amdgcn_sdot4(static_cast<int>(hi4[t]), static_cast<int>(xho[m][t]), ah, false);
                        al = __builtin_amdgcn_udot4(lo4[t], xle[m][t], al, false);
                        al = __builtin_amdgcn_udot4(hi4[t], xlo[m][t], al, false);
                    }
                    part[m] = static_cast<int>(static_cast<uint32_t>(ah) * 256u + al);
                    part[m] = group_sum(part[m], lpg);
                }
                const int rr = r + u;
                if (leader && rr < R && row0 + rr < n_out) {
                    const float sf = h2f(s16[u]), bf = h2f(b16[u]);
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        const float dot = __fmul_rn(xsc[m], static_cast<float>(part[m]));
                        const float bx = __fmul_rn(bf, xs[m]);
                        T[(m * R + rr) * Gp + g] = __builtin_fmaf(sf, dot, bx);
                    }
                }
            }
        }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < MR * R; t += blockDim.x) {
        const int m = t / R, r = t - m * R, o = row0 + r;
        if (o < n_out) {
            const float* p = T + static_cast<size_t>(m * R + r) * Gp;
            float acc = 0.0f;
            for (int g = 0; g < n_groups; g++) acc = __fadd_rn(acc, p[g]);
            out[static_cast<size_t>(m) * n_out + o] = acc;
        }
    }
}

// Any gs with gs % 64 == 0 (the reference's x86 condition): one thread per
// (m, row), scalar.  Used only for group sizes the tiled kernel does not take.
__global__ void gemv_generic_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ sc,
    const uint16_t* __restrict__ bi, const uint4* __restrict__ planes,
    const float* __restrict__ xsum, const float* __restrict__ xscale,
    float* __restrict__ out, int m_rows, int n_out, int n_in, int gs) {
    const long t = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= static_cast<long>(m_rows) * n_out) return;
    const int m = static_cast<int>(t / n_out), o = static_cast<int>(t % n_out);
    const int wpr = n_in >> 3, n_groups = n_in / gs;
    const uint32_t* row = w + static_cast<size_t>(o) * wpr;
    const uint4* xp = planes + static_cast<size_t>(m) * wpr;
    float acc = 0.0f;
    for (int g = 0; g < n_groups; g++) {
        uint32_t idot = 0;
        for (int i = 0; i < gs; i++) {
            const int k = g * gs + i, j = k >> 3, n = k & 7;
            const uint32_t q = (row[j] >> (4 * n)) & 0xFu;
            const uint4 p = xp[j];
            const int sh = 8 * (n >> 1);
            const uint32_t xl = ((n & 1) ? p.y : p.x) >> sh & 0xFFu;
            const int32_t xh = static_cast<int8_t>(((n & 1) ? p.w : p.z) >> sh & 0xFFu);
            idot += q * static_cast<uint32_t>(xh * 256 + static_cast<int32_t>(xl));
        }
        const size_t si = static_cast<size_t>(o) * n_groups + g;
        const float dot = __fmul_rn(xscale[m], static_cast<float>(static_cast<int32_t>(idot)));
        const float bx = __fmul_rn(h2f(bi[si]), xsum[static_cast<size_t>(m) * n_groups + g]);
        acc = __fadd_rn(acc, __builtin_fmaf(h2f(sc[si]), dot, bx));
    }
    out[static_cast<size_t>(m) * n_out + o] = acc;
}

// ---------------------------------------------- streaming single-launch GEMV --
//
// One launch per call; weights are streamed row-contiguously (a wave-load
// moves 1 KiB of one row: 64 lanes x 16 bytes).  Group size 64.
//   * The x prologue runs once per workgroup.  Every x load is issued before
//     the first weight load and x is read once: vector-memory results return
//     in issue order, so an x load issued behind the weight stream would wait
//     for it.  Each thread loads whole packed words (8 values), stages them
//     in LDS and takes amax; after one barrier one thread per group chains
//     the group sum in ascending order from LDS while every thread writes
//     the int8/uint8 planes of its words of the int16 x into LDS.
//   * Then every wave works alone on a flat stream of 1 KiB items: the items
//     of its units (UB consecutive rows; PAIR: UB rows of matrix 0 and the
//     same UB rows of matrix 1), chunk-major within a unit so consecutive
//     items share x planes.  A ring of RING items is in flight (the host
//     picks RING no larger than any working wave's item count): the item
//     RING ahead is issued right after an item is consumed, from straight-
//     line code while every refill is live, so each wait is a partial
//     vmcnt; the last 1..2*RING items run through a tail with conditional
//     refills, so nothing past the wave's last item is ever loaded.  Lanes
//     past a row end read through a buffer range that ends with the row:
//     0, no memory access.
//   * Each group's fp32 term goes to a wave-private LDS table; when a unit
//     is done one lane per (m, row) adds its row's terms in ascending group
//     order -- no workgroup barrier in the main loop.
// The row a wave works on is wave-uniform (kept in SGPRs), so choosing the
// matrix of a grouped launch (q/k/v, gate/up: up to kMaxMats sharing x) is
// scalar work.
constexpr int kMaxMats = 4;
constexpr int kEarly = 2;           // ring items issued before the x prologue has its data
constexpr int kUnitItems = 4;       // rows per unit grow until a unit has this many items

struct MatList {
    const uint32_t* w[kMaxMats];
    const uint16_t* s[kMaxMats];
    const uint16_t* b[kMaxMats];
    float* out[kMaxMats];
    int n_out[kMaxMats];
    int row_begin[kMaxMats + 1];   // prefix sums of n_out
    int count;
};

// Row stride of the per-wave term table: a multiple of 4 floats (16-byte
// reads) that is 4 mod 8 words, so lanes reading different rows spread over
// the banks.
__host__ __device__ inline int term_stride(int G) { return ((G + 3) & ~3) | 4; }

// Staged x floats: group g of row m at (m*G + g) * kStageStride floats, so
// the 16-byte reads of one lane per group land on distinct banks.
constexpr int kStageStride = 68;

size_t stream_lds_bytes(int mr, int n_chunks, int G, int nwaves, int NU) {
    const size_t terms = static_cast<size_t>(nwaves) * mr * NU * term_stride(G) * 4;
    const size_t stage = static_cast<size_t>(mr) * G * kStageStride * 4;
    return static_cast<size_t>(mr) * n_chunks * 256 * 16                 // x planes
         + static_cast<size_t>(mr) * ((G + 3) & ~3) * 4                  // group sums
         + static_cast<size_t>(mr) * 16 * 4                              // amax per wave
         + (terms > stage ? terms : stage);                              // term tables | staged x
}

__device__ __forceinline__ int mat_of_row(const MatList& ml, int gr) {
    int p = 0;
#pragma unroll
    for (int k = 1; k < kMaxMats; k++) p += (k < ml.count && gr >= ml.row_begin[k]) ? 1 : 0;
    return p;
}

// x[p] for a wave-uniform p in an SGPR, as scalar compare/selects in asm: a
// select written in C++ is folded back into an indexed kernel-argument load,
// which puts a scalar memory round trip in front of every weight load.
__device__ __forceinline__ uint64_t sel4(int p, uint64_t a0, uint64_t a1, uint64_t a2, uint64_t a3) {
    uint64_t r;
    asm volatile(
        "s_cmp_eq_u32 %1, 1\n\t"
        "s_cselect_b64 %0, %3, %2\n\t"
        "s_cmp_eq_u32 %1, 2\n\t"
        "s_cselect_b64 %0, %4, %0\n\t"
        "s_cmp_eq_u32 %1, 3\n\t"
        "s_cselect_b64 %0, %5, %0"
        : "=&s"(r) : "s"(p), "s"(a0), "s"(a1), "s"(a2), "s"(a3) : "scc");
    return r;
}
__device__ __forceinline__ int sel4(int p, int a0, int a1, int a2, int a3) {
    int r;
    asm volatile(
        "s_cmp_eq_u32 %1, 1\n\t"
        "s_cselect_b32 %0, %3, %2\n\t"
        "s_cmp_eq_u32 %1, 2\n\t"
        "s_cselect_b32 %0, %4, %0\n\t"
        "s_cmp_eq_u32 %1, 3\n\t"
        "s_cselect_b32 %0, %5, %0"
        : "=&s"(r) : "s"(p), "s"(a0), "s"(a1), "s"(a2), "s"(a3) : "scc");
    return r;
}
template <typename T>
__device__ __forceinline__ T* pick(T* const (&a)[kMaxMats], int p) {
    return reinterpret_cast<T*>(sel4(p, reinterpret_cast<uint64_t>(a[0]), reinterpret_cast<uint64_t>(a[1]),
                                     reinterpret_cast<uint64_t>(a[2]), reinterpret_cast<uint64_t>(a[3])));
}

struct Item {
    uint4 w;
    uint16_t s, b;
};

// Raw buffer resource over [p, p + bytes): loads at an offset >= bytes
// return 0 without a memory access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}
constexpr uint32_t kOutOfRange = 0x80000000u;   // any offset past every resource here

// Issue the loads of item (chunk c, row slot r) of unit `unit`.  The row is
// wave-uniform: each array gets a resource over that row alone, so lanes
// past the row end read 0 and cost no memory access, and `live` false (a
// prefetch past the wave's last item) gives an empty resource: every lane
// reads 0.  No branch, so the waits on earlier loads stay exact.
template <bool PAIR>
__device__ __forceinline__ void load_item(Item& it, const MatList& ml, int unit, int c, int r, int UB,
                                          int n_total, int wpr, int G, int lane, bool live) {
    const int u = PAIR ? (r < UB ? r : r - UB) : r;
    int gr = unit * UB + u;
    gr = gr < n_total ? gr : n_total - 1;
    // p is wave-uniform; readfirstlane makes that explicit, so the
    // kernel-argument reads below are scalar loads
    const int p = __builtin_amdgcn_readfirstlane(PAIR ? (r < UB ? 0 : 1) : mat_of_row(ml, gr));
    const int o = __builtin_amdgcn_readfirstlane(
        PAIR ? gr : gr - sel4(p, ml.row_begin[0], ml.row_begin[1], ml.row_begin[2], ml.row_begin[3]));
    const uint32_t wbytes = live ? static_cast<uint32_t>(wpr) * 4u : 0u;
    const uint32_t gbytes = live ? static_cast<uint32_t>(G) * 2u : 0u;
    const int word0 = c * kChunkWords + lane * 4;
    it.w = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
        buf_rsrc(pick(ml.w, p) + static_cast<size_t>(o) * wpr, wbytes), word0 * 4, 0, 0));
    const int go = (word0 >> 3) * 2;
    it.s = __builtin_amdgcn_raw_buffer_load_b16(buf_rsrc(pick(ml.s, p) + static_cast<size_t>(o) * G, gbytes), go, 0, 0);
    it.b = __builtin_amdgcn_raw_buffer_load_b16(buf_rsrc(pick(ml.b, p) + static_cast<size_t>(o) * G, gbytes), go, 0, 0);
}

// Sequential fp32 sum of n terms (ascending), four 16-byte LDS reads in flight.
__device__ __forceinline__ float chain_sum(const float* tp, int n) {
    const float4* t4 = reinterpret_cast<const float4*>(tp);
    float acc = 0.0f;
    int g = 0;
    for (; g + 16 <= n; g += 16) {
        const float4 a0 = t4[g / 4], a1 = t4[g / 4 + 1], a2 = t4[g / 4 + 2], a3 = t4[g / 4 + 3];
        const float vals[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                                a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
#pragma unroll
        for (int i = 0; i < 16; i++) acc = __fadd_rn(acc, vals[i]);
    }
    for (; g < n; g++) acc = __fadd_rn(acc, tp[g]);
    return acc;
}

// SiLU(g) * u as hetero/cpu_model.py:169-170 and :291-292 compute it in
// fp32: g / (1 + exp(-g)) * u (expf here; NumPy's float32 exp may differ in
// the last place).
__device__ __forceinline__ float silu_mul(float g, float u) {
    const float e = expf(-g);
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
}

// Words of x per thread and activation row that the word pass keeps in
// registers (RW rounds of blockDim.x words); the host picks the instance.
template <int MR>
__host__ __device__ constexpr int stream_max_rounds() { return MR == 1 ? 4 : 2; }

// PAIR: matrices 0 and 1 (gate, up) are computed row for row and the output
// is out[0] = SiLU(gate) * up.
// Host guarantees: MR * (n_in / 64) <= blockDim.x (one thread per group
// item), chunks * 256 <= RW * blockDim.x, n_in % 64 == 0, x 16-byte aligned.
template <int MR, int RW, bool PAIR, int RING>
__global__ __launch_bounds__(1024) void gemv_stream_kernel(MatList ml, const float* __restrict__ x,
                                                          int n_in, int UB) {
    extern __shared__ uint4 lds4[];
    constexpr int lpg = 2;                                        // lanes per group
    const int wpr = n_in >> 3, G = n_in >> 6;
    const int C = (wpr + kChunkWords - 1) / kChunkWords;
    const int Gr = (G + 3) & ~3, Ts = term_stride(G);
    const int tid = threadIdx.x, nt = blockDim.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);    // wave-uniform
    const int nwaves = nt >> 6;
    uint4* xpl = lds4;                                            // [MR][C*256] swizzled
    float* xsum_lds = reinterpret_cast<float*>(xpl + MR * C * 256);   // [MR][Gr]
    float* red = xsum_lds + MR * Gr;                              // [MR][16]
    const int NU = PAIR ? 2 * UB : UB;                            // rows per unit
    float* Tw = red + MR * 16 + wave * (MR * NU * Ts);            // this wave: [MR][NU][Ts]
    const int n_total = PAIR ? ml.n_out[0] : ml.row_begin[ml.count];
    const int n_units = (n_total + UB - 1) / UB;
    const int tw = gridDim.x * nwaves;
    const int items = NU * C;

    // ---- x loads: thread t owns words t, t + nt, ... of every row, 8 values
    //      each, through a resource over x (words at or past the row end read
    //      0); waves with no word in a round issue nothing.  These are the
    //      first loads of the kernel, so the waits further down stay exact.
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(x, static_cast<uint32_t>(MR * n_in) * 4u);
    float4 wv[MR][RW][2];
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int r = 0; r < RW; r++)
            if (r * nt + wave * 64 < wpr) {                       // uniform
                const int j = r * nt + tid;
                const uint32_t off = j < wpr ? static_cast<uint32_t>(m * n_in + 8 * j) * 4u : kOutOfRange;
                wv[m][r][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
                wv[m][r][1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16, 0, 0));
            }

    // ---- the wave's item stream: units gw, gw + tw, ...; item i of a unit
    //      is (chunk i / NU, row slot i % NU).  Up to kEarly items are
    //      issued now, the rest of the ring once x is in: a full ring from
    //      every wave at once would queue ahead of the x loads of later
    //      waves.  A wave without units loads through empty ranges.
    const int gw = blockIdx.x * nwaves + wave;
    const int nu_w = gw < n_units ? (n_units - gw + tw - 1) / tw : 0;
    const int Q = nu_w * items;
    constexpr int kE = RING < kEarly ? RING : kEarly;
    Item ring[RING];
    int pf_unit = gw, pf_c = 0, pf_r = 0, pf_q = 0;               // prefetch cursor (uniform)
#pragma unroll
    for (int d = 0; d < kE; d++) {
        load_item<PAIR>(ring[d], ml, pf_unit, pf_c, pf_r, UB, n_total, wpr, G, lane, pf_q < Q);
        pf_q++;
        if (++pf_r == NU) { pf_r = 0; if (++pf_c == C) { pf_c = 0; pf_unit += tw; } }
    }

    // ---- stage the floats in LDS (the term tables' space, free until the
    //      main loop) and take the running max |x| (kernel/q4gemv.c:258-259,
    //      NaN-skipping) per row
    float* stage = red + MR * 16;
#pragma unroll
    for (int m = 0; m < MR; m++) {
        float amax = 0.0f;
#pragma unroll
        for (int r = 0; r < RW; r++)
            if (r * nt + wave * 64 < wpr) {                       // uniform
                const int j = r * nt + tid;
                if (j < wpr) {
                    float4* dst = reinterpret_cast<float4*>(stage + (m * G + (j >> 3)) * kStageStride + 8 * (j & 7));
                    dst[0] = wv[m][r][0];
                    dst[1] = wv[m][r][1];
                }
                const float4 a = wv[m][r][0], b = wv[m][r][1];  // 0 past the row end
                amax = fmaxf(amax, fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                                         fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w)))));
            }
        amax = wave_max(amax);
        if (lane == 0) red[m * 16 + wave] = amax;
    }
#pragma unroll
    for (int d = kE; d < RING; d++) {
        load_item<PAIR>(ring[d], ml, pf_unit, pf_c, pf_r, UB, n_total, wpr, G, lane, pf_q < Q);
        pf_q++;
        if (++pf_r == NU) { pf_r = 0; if (++pf_c == C) { pf_c = 0; pf_unit += tw; } }
    }
    __syncthreads();

    // ---- group sums: one thread per (row, group) chains its 64 values in
    //      ascending order (kernel/q4gemv.c:244-248)
    if (tid < MR * G) {
        const float4* gp = reinterpret_cast<const float4*>(stage + tid * kStageStride);
        float sum = 0.0f;
#pragma unroll
        for (int i0 = 0; i0 < 16; i0 += 4) {
            const float4 v0 = gp[i0], v1 = gp[i0 + 1], v2 = gp[i0 + 2], v3 = gp[i0 + 3];
            const float vals[16] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w,
                                    v2.x, v2.y, v2.z, v2.w, v3.x, v3.y, v3.z, v3.w};
#pragma unroll
            for (int i = 0; i < 16; i++) sum = __fadd_rn(sum, vals[i]);
        }
        const int m = tid / G;
        xsum_lds[m * Gr + (tid - m * G)] = sum;
    }

    // ---- int16 x (kernel/q4gemv.c:260-270) as byte planes in LDS
    float xsc[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) {
        float a = 0.0f;
        for (int i = 0; i < nwaves; i++) a = fmaxf(a, red[m * 16 + i]);
        xsc[m] = a > 0.0f ? __fdiv_rn(a, 32767.0f) : 1.0f;        // kernel/q4gemv.c:260
        const float inv = __fdiv_rn(1.0f, xsc[m]);                 // :261
        const bool exact_clamp = __builtin_isinf(inv);
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const int j = r * nt + tid;
            if (r * nt + wave * 64 < C * kChunkWords) {           // uniform
                uint4 pl = make_uint4(0, 0, 0, 0);
                if (r * nt + wave * 64 < wpr) {                   // uniform
                    const float vv[8] = {wv[m][r][0].x, wv[m][r][0].y, wv[m][r][0].z, wv[m][r][0].w,
                                         wv[m][r][1].x, wv[m][r][1].y, wv[m][r][1].z, wv[m][r][1].w};
                    pl = exact_clamp ? quant_word(vv, inv, true) : quant_word(vv, inv, false);
                    if (j >= wpr) pl = make_uint4(0, 0, 0, 0);
                }
                const int cc = j >> 8, jj = j & 255;
                xpl[(m * C + cc) * 256 + (jj & 3) * 64 + (jj >> 2)] = pl;
            }
        }
    }
    __syncthreads();

    // ---- main loop: consume the ring, refill each slot RING items ahead
    int cu_unit = gw, cu_c = 0, cu_r = 0;                         // consume cursor (uniform)
    int cprev = -1;
    uint32_t xle[MR][4], xlo[MR][4], xhe[MR][4], xho[MR][4];
    auto consume = [&](const Item& itm) {
        const int c = cu_c, u = cu_r;
        const int word0 = c * kChunkWords + lane * 4;
        const bool lead = word0 < wpr && (lane & (lpg - 1)) == lpg - 1;
        const int g = word0 >> 3;
        if (c != cprev) {                                 // uniform: planes of chunk c
#pragma unroll
            for (int m = 0; m < MR; m++)
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const uint4 pl = xpl[(m * C + c) * 256 + t * 64 + lane];
                    xle[m][t] = pl.x; xlo[m][t] = pl.y; xhe[m][t] = pl.z; xho[m][t] = pl.w;
                }
            cprev = c;
        }
        const uint32_t wd[4] = {itm.w.x, itm.w.y, itm.w.z, itm.w.w};
        uint32_t lo4[4], hi4[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            lo4[t] = wd[t] & 0x0F0F0F0Fu;          // values 8j+0,2,4,6
            hi4[t] = (wd[t] >> 4) & 0x0F0F0F0Fu;   // values 8j+1,3,5,7
        }
        const float sf = h2f(itm.s), bf = h2f(itm.b);
#pragma unroll
        for (int m = 0; m < MR; m++) {
            int ah = 0;
            uint32_t al = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                ah = __builtin_amdgcn_sdot4(static_cast<int>(lo4[t]), static_cast<int>(xhe[m][t]), ah, false);
                ah = __builtin_amdgcn_sdot4(static_cast<int>(hi4[t]), static_cast<int>(xho[m][t]), ah, false);
                al = __builtin_amdgcn_udot4(lo4[t], xle[m][t], al, false);
                al = __builtin_amdgcn_udot4(hi4[t], xlo[m][t], al, false);
            }
            const int part = group_sum(static_cast<int>(static_cast<uint32_t>(ah) * 256u + al), lpg);
            if (lead) {
                const float dot = __fmul_rn(xsc[m], static_cast<float>(part));
                const float bx = __fmul_rn(bf, xsum_lds[m * Gr + g]);
                Tw[(m * NU + u) * Ts + g] = __builtin_fmaf(sf, dot, bx);
            }
        }
        if (++cu_r == NU) {
            cu_r = 0;
            if (++cu_c == C) {                            // unit done: ordered chains
                cu_c = 0;
                const int unit = cu_unit;
                cu_unit += tw;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
                if (lane < MR * UB) {
                    const int m = lane / UB, uu = lane - m * UB, gr = unit * UB + uu;
                    if (gr < n_total) {
                        const float acc = chain_sum(Tw + (m * NU + uu) * Ts, G);
                        if constexpr (PAIR) {
                            const float up = chain_sum(Tw + (m * NU + UB + uu) * Ts, G);
                            ml.out[0][static_cast<size_t>(m) * ml.n_out[0] + gr] = silu_mul(acc, up);
                        } else {
                            // the host picks UB dividing every n_out, so a unit
                            // never straddles two matrices and p is wave-uniform
                            const int p = __builtin_amdgcn_readfirstlane(mat_of_row(ml, unit * UB));
                            const int no = sel4(p, ml.n_out[0], ml.n_out[1], ml.n_out[2], ml.n_out[3]);
                            const int rb = sel4(p, ml.row_begin[0], ml.row_begin[1], ml.row_begin[2],
                                                ml.row_begin[3]);
                            pick(ml.out, p)[static_cast<size_t>(m) * no + (gr - rb)] = acc;
                        }
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            }
        }
    };
    auto refill = [&](Item& slot) {
        load_item<PAIR>(slot, ml, pf_unit, pf_c, pf_r, UB, n_total, wpr, G, lane, true);
        if (++pf_r == NU) { pf_r = 0; if (++pf_c == C) { pf_c = 0; pf_unit += tw; } }
    };
    // steady state: every refill is live and unconditional (exact waits)
    int q0 = 0;
    for (; q0 + 2 * RING <= Q; q0 += RING) {
#pragma unroll
        for (int d = 0; d < RING; d++) {
            consume(ring[d]);
            refill(ring[d]);
        }
    }
    // tail: RING..2*RING-1 items left (a working wave has Q >= RING)
    if (q0 < Q) {                                                 // uniform
#pragma unroll
        for (int d = 0; d < RING; d++) {
            consume(ring[d]);
            if (q0 + RING + d < Q) refill(ring[d]);               // uniform
        }
#pragma unroll
        for (int d = 0; d < RING; d++)
            if (q0 + RING + d < Q) consume(ring[d]);              // uniform
    }
}

// h = SiLU(g) * u elementwise (fallback of the fused gate/up launch).
__global__ void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                float* __restrict__ h, long n) {
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) h[i] = silu_mul(g[i], u[i]);
}

__global__ void fill_zero_kernel(float* __restrict__ p, long n) {
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

// ---------------------------------------------------------------- dequant --
//
// One thread per packed word: 8 values of one row, written as two 16-byte
// stores.  out[(o-row0)][i] = fma(q, scale, bias) (kernel/q4gemv.c:331-334).
template <bool kBf16>
__global__ __launch_bounds__(256) void dequant_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ sc,
    const uint16_t* __restrict__ bi, void* __restrict__ out, int row0, int rows,
    int n_in, int gs) {
    const int wpr = n_in >> 3, n_groups = n_in / gs;
    const long idx = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<long>(rows) * wpr) return;
    const int rr = static_cast<int>(idx / wpr), j = static_cast<int>(idx % wpr);
    const int o = row0 + rr, g = (8 * j) / gs;
    const uint32_t word = w[static_cast<size_t>(o) * wpr + j];
    const size_t si = static_cast<size_t>(o) * n_groups + g;
    const float s = h2f(sc[si]), b = h2f(bi[si]);
    float v[8];
#pragma unroll
    for (int n = 0; n < 8; n++)
        v[n] = __builtin_fmaf(static_cast<float>((word >> (4 * n)) & 0xFu), s, b);
    const size_t base = static_cast<size_t>(rr) * n_in + 8 * static_cast<size_t>(j);
    if constexpr (kBf16) {
        uint32_t pk[4];
#pragma unroll
        for (int n = 0; n < 4; n++) {
            uint32_t h[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t bits = __builtin_bit_cast(uint32_t, v[2 * n + e]);
                const bool nan = (bits & 0x7FFFFFFFu) > 0x7F800000u;
                h[e] = nan ? ((bits >> 16) | 0x40u) : ((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
            }
            pk[n] = h[0] | (h[1] << 16);
        }
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + base) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    } else {
        float* o4 = static_cast<float*>(out) + base;
        *reinterpret_cast<float4*>(o4) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(o4 + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// ------------------------------------------------ prefill GEMM (bf16 MFMA) --
//
// out[M][N] = x[M][K] . W^T for the prompt (M > 16 rows), the contraction the
// reference hands to BLAS after q4_dequant (hetero/cpu_model.py:119-136).
// W is dequantised to bf16 inside the B-tile load (fma(q, scale, bias) in
// fp32, rounded to nearest even: exactly q4_dequant_bf16), x is rounded to
// bf16 in the A-tile load, and v_mfma_f32_32x32x16_bf16 accumulates in fp32.
//   * tile BM x BN x 64 (one quantisation group per k-step, so each B row of
//     a tile has one scale/bias pair), 4 waves as 2 x 2, each wave owning a
//     (BM/2) x (BN/2) block of 32 x 32 MFMA tiles;
//   * LDS double-buffered; the next tile's global loads are in flight while
//     the current tile is multiplied;
//   * blockIdx.x walks the M blocks: with 4 M blocks and WGs dealt round-robin
//     to the 8 XCDs, each XCD keeps one M block of x in its L2 and the W tile
//     of a column of workgroups is read by them back to back.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kGemmLdsK = 72;            // LDS row stride in bf16 (64 + 8 pad: conflict-free)

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const __bf16 ha = static_cast<__bf16>(a), hb = static_cast<__bf16>(b);   // RNE
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, ha)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hb)) << 16);
}

template <int BM, int BN>
__global__ __launch_bounds__(256) void gemm_q4_bf16_kernel(
    const float* __restrict__ x, const uint32_t* __restrict__ w, const uint16_t* __restrict__ sc,
    const uint16_t* __restrict__ bi, float* __restrict__ out, int M, int N, int K) {
    extern __shared__ uint4 gemm_lds[];
    uint16_t* As = reinterpret_cast<uint16_t*>(gemm_lds);          // [2][BM][72]
    uint16_t* Bs = As + 2 * BM * kGemmLdsK;                        // [2][BN][72]
    constexpr int TM = BM / 64, TN = BN / 64;                      // 32x32 tiles per wave
    constexpr int A_PER = BM * 16 / 256;                           // float4 of x per thread
    constexpr int B_PER = BN * 2 / 256;                            // uint4 of w per thread (may be < 1)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
    const int G = K >> 6, wpr = K >> 3;

    float4 ra[A_PER];
    uint4 rb[B_PER > 0 ? B_PER : 1];
    uint16_t rs[B_PER > 0 ? B_PER : 1], rbb[B_PER > 0 ? B_PER : 1];
    auto gload = [&](int kt) {
#pragma unroll
        for (int i = 0; i < A_PER; i++) {
            const int idx = tid + 256 * i, row = idx >> 4, c4 = idx & 15;
            const int gm = m0 + row < M ? m0 + row : M - 1;
            ra[i] = reinterpret_cast<const float4*>(x + static_cast<size_t>(gm) * K + 64 * kt)[c4];
        }
#pragma unroll
        for (int i = 0; i < (B_PER > 0 ? B_PER : 1); i++) {
            const int idx = tid + 256 * i, row = idx >> 1, half = idx & 1;
            if (B_PER > 0 || row < BN) {
                const int gn = n0 + row < N ? n0 + row : N - 1;
                rb[i] = *reinterpret_cast<const uint4*>(w + static_cast<size_t>(gn) * wpr + 8 * kt + 4 * half);
                rs[i] = sc[static_cast<size_t>(gn) * G + kt];
                rbb[i] = bi[static_cast<size_t>(gn) * G + kt];
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_PER; i++) {
            const int idx = tid + 256 * i, row = idx >> 4, c4 = idx & 15;
            uint2 v;
            v.x = pack_bf16x2(ra[i].x, ra[i].y);
            v.y = pack_bf16x2(ra[i].z, ra[i].w);
            *reinterpret_cast<uint2*>(As + (buf * BM + row) * kGemmLdsK + 4 * c4) = v;
        }
#pragma unroll
        for (int i = 0; i < (B_PER > 0 ? B_PER : 1); i++) {
            const int idx = tid + 256 * i, row = idx >> 1, half = idx & 1;
            if (B_PER > 0 || row < BN) {
                const float s = h2f(rs[i]), b = h2f(rbb[i]);
                const uint32_t wd[4] = {rb[i].x, rb[i].y, rb[i].z, rb[i].w};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    // even values in the bytes of lo, odd ones in hi; v_cvt_f32_ubyteN
                    // turns each byte into a float in one instruction
                    const uint32_t lo = wd[t] & 0x0F0F0F0Fu, hi = (wd[t] >> 4) & 0x0F0F0F0Fu;
                    float v[8];
#pragma unroll
                    for (int n = 0; n < 4; n++) {
                        v[2 * n] = __builtin_fmaf(static_cast<float>((lo >> (8 * n)) & 0xFFu), s, b);
                        v[2 * n + 1] = __builtin_fmaf(static_cast<float>((hi >> (8 * n)) & 0xFFu), s, b);
                    }
                    uint4 pk;
                    pk.x = pack_bf16x2(v[0], v[1]); pk.y = pack_bf16x2(v[2], v[3]);
                    pk.z = pack_bf16x2(v[4], v[5]); pk.w = pack_bf16x2(v[6], v[7]);
                    *reinterpret_cast<uint4*>(Bs + (buf * BN + row) * kGemmLdsK + 32 * half + 8 * t) = pk;
                }
            }
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;

    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < G; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < G) gload(kt + 1);
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            bf16x8 a[TM], bv[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int row = wm * (BM / 2) + i * 32 + (lane & 31);
                a[i] = *reinterpret_cast<const bf16x8*>(As + (cur * BM + row) * kGemmLdsK + 16 * ks + 8 * (lane >> 5));
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int row = wn * (BN / 2) + j * 32 + (lane & 31);
                bv[j] = *reinterpret_cast<const bf16x8*>(Bs + (cur * BN + row) * kGemmLdsK + 16 * ks + 8 * (lane >> 5));
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bv[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < G) lstore(cur ^ 1);
        __syncthreads();
    }
    // C tile layout: lane l, register v holds row 8*(v/4) + 4*(l/32) + v%4, column l%32
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = m0 + wm * (BM / 2) + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                const int col = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
                if (row < M && col < N) out[static_cast<size_t>(row) * N + col] = acc[i][j][v];
            }
}

// ============================================================ host side ===

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

#define HIP_TRY(expr)                                                              \
    do {                                                                           \
        hipError_t e_ = (expr);                                                    \
        if (e_ != hipSuccess) {                                                    \
            return fail(e_ == hipErrorOutOfMemory ? Q4_ENOMEM : Q4_EHIP, "%s: %s", \
                        #expr, hipGetErrorString(e_));                             \
        }                                                                          \
    } while (0)

bool pow2_gs(int gs) { return gs >= 64 && gs <= 2048 && (gs & (gs - 1)) == 0; }

// Per-stream x workspace (prologue outputs).  Grows only; before freeing an
// old buffer the stream is drained, since earlier launches may still read it.
struct Workspace {
    uint4* planes = nullptr;
    float* xsum = nullptr;
    float* xscale = nullptr;
    size_t cap_words = 0, cap_groups = 0;
    float* tmp = nullptr;                       // up-projection rows of the unfused MLP
    size_t cap_tmp = 0;
};

int ensure_tmp(Workspace& ws, hipStream_t st, size_t n) {
    if (n <= ws.cap_tmp && ws.tmp) return 0;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(st, &cap));
    if (cap != hipStreamCaptureStatusNone)
        return fail(Q4_EARG, "MLP workspace of this stream must grow during graph capture: "
                             "run the largest call once on the stream before capturing");
    HIP_TRY(hipStreamSynchronize(st));
    (void)hipFree(ws.tmp);
    ws.tmp = nullptr;
    ws.cap_tmp = 0;
    HIP_TRY(hipMalloc(&ws.tmp, n * sizeof(float)));
    ws.cap_tmp = n;
    return 0;
}

struct DevState {
    hipStream_t stream = nullptr;               // stream of the host-pointer calls
    std::map<hipStream_t, Workspace> ws;
    float* pin_x = nullptr;                     // pinned staging
    float* pin_out = nullptr;
    size_t pin_x_cap = 0, pin_out_cap = 0;
    float* dev_x = nullptr;
    float* dev_out = nullptr;
    size_t dev_x_cap = 0, dev_out_cap = 0;
};

struct Resident {
    uint32_t* w = nullptr;
    uint16_t* s = nullptr;
    uint16_t* b = nullptr;
    uint64_t fp = 0;
};

// (device, w, scales, biases, n_out, n_in, gs)
using ResKey = std::tuple<int, const void*, const void*, const void*, int, int, int>;

std::mutex g_mu;                       // serialises every host-pointer call
std::map<int, DevState> g_dev;
std::map<ResKey, Resident> g_res;

int ensure_ws(Workspace& ws, hipStream_t st, size_t words, size_t groups) {
    if (words <= ws.cap_words && groups <= ws.cap_groups && ws.planes) return 0;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(st, &cap));
    if (cap != hipStreamCaptureStatusNone)
        return fail(Q4_EARG, "x workspace of this stream must grow during graph capture: "
                             "run the largest call once on the stream before capturing");
    HIP_TRY(hipStreamSynchronize(st));
    (void)hipFree(ws.planes);
    (void)hipFree(ws.xsum);
    (void)hipFree(ws.xscale);
    ws.planes = nullptr;
    ws.xsum = nullptr;
    ws.xscale = nullptr;
    ws.cap_words = ws.cap_groups = 0;
    size_t cw = words < 4096 ? 4096 : words, cg = groups < 1024 ? 1024 : groups;
    HIP_TRY(hipMalloc(&ws.planes, cw * sizeof(uint4)));
    HIP_TRY(hipMalloc(&ws.xsum, cg * sizeof(float)));
    HIP_TRY(hipMalloc(&ws.xscale, kMaxM * sizeof(float)));
    ws.cap_words = cw;
    ws.cap_groups = cg;
    return 0;
}

template <int MR>
hipError_t launch_main(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                       const Workspace& ws, float* out, int n_out, int n_in, int gs,
                       hipStream_t st) {
    const int wpr = n_in / 8, n_groups = n_in / gs;
    const int n_chunks = (wpr + kChunkWords - 1) / kChunkWords;
    const int max_waves = main_threads<MR>() / 64;
    const int nwaves = n_chunks < max_waves ? n_chunks : max_waves;
    const int Gp = n_groups | 1;                        // odd stride: no LDS bank conflicts
    int R = n_out >= 32768 ? 16 : 4;
    while (R > 1 && static_cast<size_t>(MR) * R * Gp * sizeof(float) > kLdsBudget) R >>= 1;
    if (static_cast<size_t>(MR) * R * Gp * sizeof(float) > kLdsBudget) return hipErrorInvalidValue;
    const int grid = (n_out + R - 1) / R;
    const size_t lds = static_cast<size_t>(MR) * R * Gp * sizeof(float);
    hipLaunchKernelGGL(gemv_kernel<MR>, dim3(grid), dim3(64 * nwaves), lds, st, w, s, b,
                       ws.planes, ws.xsum, ws.xscale, out, n_out, n_in, gs, R, Gp);
    return hipGetLastError();
}

int num_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

constexpr size_t kStreamLdsMax = 160 * 1024;

template <int MR, int RW, bool PAIR, int RING>
int launch_stream_k(const MatList& ml, const float* x, int n_in, int UB, int nwaves, size_t lds, int grid,
                    hipStream_t st) {
    auto kern = gemv_stream_kernel<MR, RW, PAIR, RING>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t ea = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            static_cast<int>(kStreamLdsMax));
        if (ea != hipSuccess) return fail(Q4_EHIP, "hipFuncSetAttribute: %s", hipGetErrorString(ea));
        attr_set = true;
    }
    hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * nwaves), lds, st, ml, x, n_in, UB);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q4_EHIP, "stream gemv launch: %s", hipGetErrorString(e));
    return 1;
}

template <int MR, int RW, bool PAIR>
int launch_stream_rw(const MatList& ml, const float* x, int n_in, int UB, int nwaves, size_t lds, int n_units,
                     int items, hipStream_t st) {
    // occupancy of the largest ring (the most registers)
    int per_cu = 0;
    hipError_t eo = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &per_cu, gemv_stream_kernel<MR, RW, PAIR, 4>, 64 * nwaves, lds);
    if (eo != hipSuccess || per_cu < 1) per_cu = 1;
    const int want = (n_units + nwaves - 1) / nwaves;
    const int cap = num_cus() * per_cu;                 // every workgroup resident at once
    const int grid = want < cap ? want : cap;
    // ring: the largest of 8, 2, 1 items that every working wave has
    const int per_wave = n_units / (grid * nwaves);
    const int qmin = (per_wave > 0 ? per_wave : 1) * items;
    if (qmin >= 4) return launch_stream_k<MR, RW, PAIR, 4>(ml, x, n_in, UB, nwaves, lds, grid, st);
    if (qmin >= 2) return launch_stream_k<MR, RW, PAIR, 2>(ml, x, n_in, UB, nwaves, lds, grid, st);
    return launch_stream_k<MR, RW, PAIR, 1>(ml, x, n_in, UB, nwaves, lds, grid, st);
}

template <int MR, bool PAIR = false>
int launch_stream(const MatList& ml, const float* x, int n_in, hipStream_t st) {
    constexpr int kWavesPerCu = 16;                     // 4 waves per SIMD at <= 128 VGPRs
    constexpr int rmax = stream_max_rounds<MR>();
    const int G = n_in / 64;
    const int C = (n_in / 8 + kChunkWords - 1) / kChunkWords;
    const int n_total = PAIR ? ml.n_out[0] : ml.row_begin[ml.count];
    const int cus = num_cus();
    // smallest workgroup the prologue accepts: one thread per (row, group)
    // item, and at most rmax words of x per thread and row
    int minw = (MR * G + 63) / 64;
    const int wr = (C * kChunkWords + 64 * rmax - 1) / (64 * rmax);
    if (wr > minw) minw = wr;
    if (minw > 16) return 0;
    // rows per unit: 1, or more when rows are plentiful and short
    int UB = 1;
    while (UB < 4 && UB * C * (PAIR ? 2 : 1) < kUnitItems && n_total >= 2 * UB * kWavesPerCu * cus) UB *= 2;
    while (MR * UB > 64) UB >>= 1;
    for (int k = 0; k < ml.count; k++)                 // a unit must not straddle matrices
        while (ml.n_out[k] % UB) UB >>= 1;
    const int n_units = (n_total + UB - 1) / UB;
    // one unit per wave while the units fit on the chip at once, the waves
    // spread evenly over the CUs (3584 rows: 256 workgroups of 14 waves)
    const int target = n_units < kWavesPerCu * cus ? n_units : kWavesPerCu * cus;
    int nwaves = (target + cus - 1) / cus;
    if (nwaves < minw) nwaves = minw;
    if (nwaves > 16) nwaves = 16;
    const size_t lds = stream_lds_bytes(MR, C, G, nwaves, (PAIR ? 2 : 1) * UB);
    if (lds > kStreamLdsMax) return 0;
    const int rw = (C * kChunkWords + 64 * nwaves - 1) / (64 * nwaves);
    const int items = (PAIR ? 2 : 1) * UB * C;
    switch (rw) {
        case 1: return launch_stream_rw<MR, 1, PAIR>(ml, x, n_in, UB, nwaves, lds, n_units, items, st);
        case 2: return launch_stream_rw<MR, 2, PAIR>(ml, x, n_in, UB, nwaves, lds, n_units, items, st);
        // (3 and 4 words per thread: the single-matrix launches of one row)
        case 3: if constexpr (rmax >= 3 && !PAIR) return launch_stream_rw<MR, 3, PAIR>(ml, x, n_in, UB, nwaves, lds, n_units, items, st);
                return 0;
        case 4: if constexpr (rmax >= 4 && !PAIR) return launch_stream_rw<MR, 4, PAIR>(ml, x, n_in, UB, nwaves, lds, n_units, items, st);
                return 0;
        default: return 0;
    }
}

// The streaming path takes gs 64, x 16-byte aligned and at most 16 chunks
// (n_in <= 32768).  Returns 1 if it launched, 0 if the call must take
// the split path, <0 on error.
template <int MR>
int try_fused(const MatList& ml, const float* x, int n_in, int gs, hipStream_t st) {
    if (gs != 64 || n_in == 0 || (reinterpret_cast<uintptr_t>(x) & 15)) return 0;
    const int C = (n_in / 8 + kChunkWords - 1) / kChunkWords;
    if (C > 16) return 0;
    return launch_stream<MR>(ml, x, n_in, st);
}

int try_fused_m(const MatList& ml, const float* x, int m, int n_in, int gs, hipStream_t st) {
    switch (m) {
        case 1: return try_fused<1>(ml, x, n_in, gs, st);
        case 2: return try_fused<2>(ml, x, n_in, gs, st);
        default: return 0;      // 3..8 rows: split path (the streaming kernel would spill)
    }
}

// Split path: prologue kernel, then the main kernel reading x planes from a
// per-stream workspace.  Takes every shape the fused path does not.
int gemv_split(const uint32_t* w, const uint16_t* s, const uint16_t* b, const float* x,
               float* out, int m, int n_out, int n_in, int gs, hipStream_t st, Workspace& ws) {
    const int wpr = n_in / 8, n_groups = n_in / gs;
    int rc = ensure_ws(ws, st, static_cast<size_t>(m) * wpr, static_cast<size_t>(m) * n_groups);
    if (rc) return rc;
    hipLaunchKernelGGL(xprep_kernel, dim3(m), dim3(1024), 0, st, x, n_in, gs, ws.planes, ws.xsum,
                       ws.xscale);
    HIP_TRY(hipGetLastError());
    if (n_in == 0) {
        // n_in == 0: every row is an empty sum (no memset: callers may capture)
        const long n = static_cast<long>(m) * n_out;
        hipLaunchKernelGGL(fill_zero_kernel, dim3((n + 255) / 256), dim3(256), 0, st, out, n);
        HIP_TRY(hipGetLastError());
        return 0;
    }
    hipError_t e = hipSuccess;
    if (!pow2_gs(gs)) {
        const long total = static_cast<long>(m) * n_out;
        hipLaunchKernelGGL(gemv_generic_kernel, dim3((total + 255) / 256), dim3(256), 0, st, w, s, b,
                           ws.planes, ws.xsum, ws.xscale, out, m, n_out, n_in, gs);
        e = hipGetLastError();
    } else {
        switch (m) {
            case 1: e = launch_main<1>(w, s, b, ws, out, n_out, n_in, gs, st); break;
            case 2: e = launch_main<2>(w, s, b, ws, out, n_out, n_in, gs, st); break;
            case 3: e = launch_main<3>(w, s, b, ws, out, n_out, n_in, gs, st); break;
            case 4: e = launch_main<4>(w, s, b, ws, out, n_out, n_in, gs, st); break;
            case 5: e = launch_main<5>(w, s, b, ws, out, n_out, n_in, gs, st); break;
            case 6: e = launch_main<6>(w, s, b, ws, out, n_out, n_in, gs, st); break;
            case 7: e = launch_main<7>(w, s, b, ws, out, n_out, n_in, gs, st); break;
            default: e = launch_main<8>(w, s, b, ws, out, n_out, n_in, gs, st); break;
        }
    }
    if (e != hipSuccess) return fail(Q4_EHIP, "gemv launch: %s", hipGetErrorString(e));
    return 0;
}

// GEMV of m (<= kMaxM) rows already on the device: fused when possible.
int gemv_rows(const uint32_t* w, const uint16_t* s, const uint16_t* b, const float* x,
              float* out, int m, int n_out, int n_in, int gs, hipStream_t st, Workspace& ws) {
    MatList ml{};
    ml.w[0] = w; ml.s[0] = s; ml.b[0] = b; ml.out[0] = out; ml.n_out[0] = n_out;
    ml.row_begin[0] = 0;
    for (int k = 1; k <= kMaxMats; k++) ml.row_begin[k] = n_out;
    ml.count = 1;
    int rc = try_fused_m(ml, x, m, n_in, gs, st);
    if (rc < 0) return rc;
    if (rc == 1) return 0;
    return gemv_split(w, s, b, x, out, m, n_out, n_in, gs, st, ws);
}

int check_gemv_shape(int n_out, int n_in, int gs) {
    if (gs <= 0 || n_in % gs || gs % 64) return fail(-1, "invalid shape n_in=%d gs=%d", n_in, gs);
    if (n_out < 0 || n_in < 0) return fail(-1, "negative size");
    return 0;
}

int current_device(int* dev) {
    HIP_TRY(hipGetDevice(dev));
    return 0;
}

int dev_state(DevState** out) {
    int dev;
    int rc = current_device(&dev);
    if (rc) return rc;
    DevState& d = g_dev[dev];
    if (!d.stream) HIP_TRY(hipStreamCreateWithFlags(&d.stream, hipStreamNonBlocking));
    *out = &d;
    return 0;
}

template <typename T>
int grow_pinned(T** p, size_t* cap, size_t n) {
    if (n <= *cap && *p) return 0;
    if (*p) (void)hipHostFree(*p);
    *p = nullptr;
    *cap = 0;
    size_t c = n < 65536 ? 65536 : n;
    HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(p), c * sizeof(T), hipHostMallocDefault));
    *cap = c;
    return 0;
}

template <typename T>
int grow_dev(T** p, size_t* cap, size_t n) {
    if (n <= *cap && *p) return 0;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    size_t c = n < 65536 ? 65536 : n;
    HIP_TRY(hipMalloc(reinterpret_cast<void**>(p), c * sizeof(T)));
    *cap = c;
    return 0;
}

// Sampled fingerprint of the host weights: catches a matrix replaced at the
// same address without reading all of it on every call.
uint64_t fingerprint(const void* p, size_t bytes) {
    const uint8_t* c = static_cast<const uint8_t*>(p);
    uint64_t h = 1469598103934665603ull ^ bytes;
    auto mix = [&](size_t off) {
        uint64_t v = 0;
        size_t n = bytes - off < 8 ? bytes - off : 8;
        memcpy(&v, c + off, n);
        h = (h ^ v) * 1099511628211ull;
        h ^= h >> 29;
    };
    if (bytes == 0) return h;
    const int samples = 16;
    for (int i = 0; i < samples; i++) mix((bytes - 1) * static_cast<size_t>(i) / (samples - 1));
    return h;
}

int resident(const uint32_t* w, const uint16_t* s, const uint16_t* b, int n_out, int n_in,
             int gs, int dev, Resident** out) {
    const size_t wb = static_cast<size_t>(n_out) * (n_in / 8) * 4;
    const size_t gb = static_cast<size_t>(n_out) * (n_in / gs) * 2;
    const uint64_t fp = fingerprint(w, wb) * 31 + fingerprint(s, gb) * 7 + fingerprint(b, gb);
    Resident& r = g_res[ResKey{dev, w, s, b, n_out, n_in, gs}];
    if (r.w && r.fp == fp) {
        *out = &r;
        return 0;
    }
    if (!r.w) {
        HIP_TRY(hipMalloc(&r.w, wb ? wb : 16));
        HIP_TRY(hipMalloc(&r.s, gb ? gb : 16));
        HIP_TRY(hipMalloc(&r.b, gb ? gb : 16));
    }
    if (wb) HIP_TRY(hipMemcpy(r.w, w, wb, hipMemcpyHostToDevice));
    if (gb) HIP_TRY(hipMemcpy(r.s, s, gb, hipMemcpyHostToDevice));
    if (gb) HIP_TRY(hipMemcpy(r.b, b, gb, hipMemcpyHostToDevice));
    r.fp = fp;
    *out = &r;
    return 0;
}

void free_resident(Resident& r) {
    (void)hipFree(r.w);
    (void)hipFree(r.s);
    (void)hipFree(r.b);
}

int gemv_host(const uint32_t* w, const uint16_t* s, const uint16_t* b, const float* x,
              float* out, int m, int n_out, int n_in, int gs) {
    int rc = check_gemv_shape(n_out, n_in, gs);
    if (rc) return rc;
    if (m < 0) return fail(Q4_EARG, "m=%d", m);
    if (n_out == 0 || m == 0) return 0;
    if (!w || !s || !b || !x || !out) return fail(Q4_EARG, "null pointer");
    std::lock_guard<std::mutex> lock(g_mu);
    DevState* d;
    if ((rc = dev_state(&d))) return rc;
    int dev;
    if ((rc = current_device(&dev))) return rc;
    Resident* r;
    if ((rc = resident(w, s, b, n_out, n_in, gs, dev, &r))) return rc;
    const size_t nx = static_cast<size_t>(m) * n_in, ny = static_cast<size_t>(m) * n_out;
    if ((rc = grow_pinned(&d->pin_x, &d->pin_x_cap, nx))) return rc;
    if ((rc = grow_pinned(&d->pin_out, &d->pin_out_cap, ny))) return rc;
    if ((rc = grow_dev(&d->dev_x, &d->dev_x_cap, nx))) return rc;
    if ((rc = grow_dev(&d->dev_out, &d->dev_out_cap, ny))) return rc;
    memcpy(d->pin_x, x, nx * sizeof(float));
    HIP_TRY(hipMemcpyAsync(d->dev_x, d->pin_x, nx * sizeof(float), hipMemcpyHostToDevice, d->stream));
    Workspace& ws = d->ws[d->stream];
    for (int m0 = 0; m0 < m; m0 += kMaxM) {
        const int mm = m - m0 < kMaxM ? m - m0 : kMaxM;
        rc = gemv_rows(r->w, r->s, r->b, d->dev_x + static_cast<size_t>(m0) * n_in,
                       d->dev_out + static_cast<size_t>(m0) * n_out, mm, n_out, n_in, gs,
                       d->stream, ws);
        if (rc) return rc;
    }
    HIP_TRY(hipMemcpyAsync(d->pin_out, d->dev_out, ny * sizeof(float), hipMemcpyDeviceToHost, d->stream));
    HIP_TRY(hipStreamSynchronize(d->stream));
    memcpy(out, d->pin_out, ny * sizeof(float));
    return 0;
}

int check_dequant_shape(int n_in, int gs) {
    if (gs <= 0 || n_in % gs || gs % 8) return fail(-1, "invalid shape n_in=%d gs=%d", n_in, gs);
    if (n_in < 0) return fail(-1, "negative size");
    return 0;
}

template <bool kBf16>
int dequant_launch(const uint32_t* w, const uint16_t* s, const uint16_t* b, void* out,
                   int row0, int rows, int n_in, int gs, hipStream_t st) {
    const long words = static_cast<long>(rows) * (n_in / 8);
    if (words == 0) return 0;
    hipLaunchKernelGGL(dequant_kernel<kBf16>, dim3((words + 255) / 256), dim3(256), 0, st, w, s, b,
                       out, row0, rows, n_in, gs);
    HIP_TRY(hipGetLastError());
    return 0;
}


template <int BM, int BN>
int launch_gemm(const uint32_t* w, const uint16_t* s, const uint16_t* b, const float* x, float* out,
                int M, int N, int K, hipStream_t st) {
    auto kern = gemm_q4_bf16_kernel<BM, BN>;
    const size_t lds = static_cast<size_t>(2) * (BM + BN) * kGemmLdsK * 2;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t ea = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (ea != hipSuccess) return fail(Q4_EHIP, "hipFuncSetAttribute: %s", hipGetErrorString(ea));
        attr_set = true;
    }
    dim3 grid((M + BM - 1) / BM, (N + BN - 1) / BN);
    hipLaunchKernelGGL(kern, grid, dim3(256), lds, st, x, w, s, b, out, M, N, K);
    HIP_TRY(hipGetLastError());
    return 0;
}

}  // namespace

// ================================================================ C-ABI ====

extern "C" {

int q4_gemv(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, const float* x,
            float* out, int n_out, int n_in, int gs, int nthreads) {
    (void)nthreads;
    return gemv_host(w, scales, biases, x, out, 1, n_out, n_in, gs);
}

int q4_gemv_batched(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                    const float* x, float* out, int m, int n_out, int n_in, int gs, int nthreads) {
    (void)nthreads;
    return gemv_host(w, scales, biases, x, out, m, n_out, n_in, gs);
}

int q4_dequant(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, float* out,
               int row0, int row1, int n_in, int gs, int nthreads) {
    (void)nthreads;
    int rc = check_dequant_shape(n_in, gs);
    if (rc) return rc;
    const int rows = row1 - row0;
    if (rows <= 0) return 0;
    if (row0 < 0) return fail(Q4_EARG, "row0=%d", row0);
    if (!w || !scales || !biases || !out) return fail(Q4_EARG, "null pointer");
    std::lock_guard<std::mutex> lock(g_mu);
    DevState* d;
    if ((rc = dev_state(&d))) return rc;
    int dev;
    if ((rc = current_device(&dev))) return rc;
    // The reference indexes whole-matrix bases with rows [row0,row1)
    // (kernel/q4gemv.c:372).  The caller walks a matrix block by block
    // (hetero/cpu_model.py:129-135), so each row block is registered as its
    // own resident matrix, keyed by the block's first-row addresses; a block
    // that is the whole matrix shares q4_gemv's entry.
    const size_t wpr = static_cast<size_t>(n_in / 8), ng = static_cast<size_t>(n_in / gs);
    Resident* r;
    if ((rc = resident(w + row0 * wpr, scales + row0 * ng, biases + row0 * ng, rows, n_in, gs, dev, &r)))
        return rc;
    const size_t ny = static_cast<size_t>(rows) * n_in;
    if ((rc = grow_pinned(&d->pin_out, &d->pin_out_cap, ny))) return rc;
    if ((rc = grow_dev(&d->dev_out, &d->dev_out_cap, ny))) return rc;
    if ((rc = dequant_launch<false>(r->w, r->s, r->b, d->dev_out, 0, rows, n_in, gs, d->stream)))
        return rc;
    HIP_TRY(hipMemcpyAsync(d->pin_out, d->dev_out, ny * sizeof(float), hipMemcpyDeviceToHost, d->stream));
    HIP_TRY(hipStreamSynchronize(d->stream));
    memcpy(out, d->pin_out, ny * sizeof(float));
    return 0;
}

int q4_release(const void* w) {
    std::lock_guard<std::mutex> lock(g_mu);
    int n = 0;
    for (auto it = g_res.begin(); it != g_res.end();) {
        if (std::get<1>(it->first) == w) {
            int cur = 0;
            (void)hipGetDevice(&cur);
            (void)hipSetDevice(std::get<0>(it->first));
            free_resident(it->second);
            (void)hipSetDevice(cur);
            it = g_res.erase(it);
            n++;
        } else {
            ++it;
        }
    }
    return n;
}

int q4_release_all(void) {
    std::lock_guard<std::mutex> lock(g_mu);
    int n = 0, cur = 0;
    (void)hipGetDevice(&cur);
    for (auto& kv : g_res) {
        (void)hipSetDevice(std::get<0>(kv.first));
        free_resident(kv.second);
        n++;
    }
    (void)hipSetDevice(cur);
    g_res.clear();
    return n;
}

const char* q4_last_error(void) { return g_err; }

int q4_gemv_dev(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, const float* x,
                float* out, int m, int n_out, int n_in, int gs, void* stream) {
    int rc = check_gemv_shape(n_out, n_in, gs);
    if (rc) return rc;
    if (m < 0) return fail(Q4_EARG, "m=%d", m);
    if (n_out == 0 || m == 0) return 0;
    if (!w || !scales || !biases || !x || !out) return fail(Q4_EARG, "null pointer");
    if (reinterpret_cast<uintptr_t>(w) & 15) return fail(Q4_EARG, "w must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    Workspace* ws;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        int dev;
        if ((rc = current_device(&dev))) return rc;
        ws = &g_dev[dev].ws[st];
    }
    for (int m0 = 0; m0 < m; m0 += kMaxM) {
        const int mm = m - m0 < kMaxM ? m - m0 : kMaxM;
        rc = gemv_rows(w, scales, biases, x + static_cast<size_t>(m0) * n_in,
                       out + static_cast<size_t>(m0) * n_out, mm, n_out, n_in, gs, st, *ws);
        if (rc) return rc;
    }
    return 0;
}

int q4_gemv_multi_dev(int count, const uint32_t* const* w, const uint16_t* const* scales,
                      const uint16_t* const* biases, float* const* out, const int* n_out,
                      const float* x, int m, int n_in, int gs, void* stream) {
    if (count < 1 || count > kMaxMats || !w || !scales || !biases || !out || !n_out)
        return fail(Q4_EARG, "count=%d (1..%d) or null array", count, kMaxMats);
    int rc;
    for (int k = 0; k < count; k++) {
        if ((rc = check_gemv_shape(n_out[k], n_in, gs))) return rc;
        if (!w[k] || !scales[k] || !biases[k] || !out[k]) return fail(Q4_EARG, "null pointer in matrix %d", k);
        if (reinterpret_cast<uintptr_t>(w[k]) & 15) return fail(Q4_EARG, "w[%d] must be 16-byte aligned", k);
    }
    if (m < 0) return fail(Q4_EARG, "m=%d", m);
    if (m == 0) return 0;
    if (!x) return fail(Q4_EARG, "null x");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (m <= kMaxM) {
        MatList ml{};
        ml.row_begin[0] = 0;
        for (int k = 0; k < kMaxMats; k++) {
            const int kk = k < count ? k : count - 1;
            ml.w[k] = w[kk]; ml.s[k] = scales[kk]; ml.b[k] = biases[kk]; ml.out[k] = out[kk];
            ml.n_out[k] = k < count ? n_out[k] : 0;
            ml.row_begin[k + 1] = ml.row_begin[k] + ml.n_out[k];
        }
        ml.count = count;
        if (ml.row_begin[count] == 0) return 0;
        rc = try_fused_m(ml, x, m, n_in, gs, st);
        if (rc < 0) return rc;
        if (rc == 1) return 0;
    }
    for (int k = 0; k < count; k++)
        if ((rc = q4_gemv_dev(w[k], scales[k], biases[k], x, out[k], m, n_out[k], n_in, gs, stream)))
            return rc;
    return 0;
}

int q4_gate_up_silu_dev(const uint32_t* gate_w, const uint16_t* gate_s, const uint16_t* gate_b,
                        const uint32_t* up_w, const uint16_t* up_s, const uint16_t* up_b,
                        const float* x, float* h, int m, int n_inter, int n_in, int gs,
                        void* stream) {
    int rc = check_gemv_shape(n_inter, n_in, gs);
    if (rc) return rc;
    if (m < 0) return fail(Q4_EARG, "m=%d", m);
    if (m == 0 || n_inter == 0) return 0;
    if (!gate_w || !gate_s || !gate_b || !up_w || !up_s || !up_b || !x || !h)
        return fail(Q4_EARG, "null pointer");
    if ((reinterpret_cast<uintptr_t>(gate_w) | reinterpret_cast<uintptr_t>(up_w)) & 15)
        return fail(Q4_EARG, "w must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    for (int m0 = 0; m0 < m; m0 += 2) {
        const int mm = m - m0 < 2 ? m - m0 : 2;
        const float* xm = x + static_cast<size_t>(m0) * n_in;
        float* hm = h + static_cast<size_t>(m0) * n_inter;
        MatList ml{};
        ml.w[0] = gate_w; ml.s[0] = gate_s; ml.b[0] = gate_b; ml.out[0] = hm; ml.n_out[0] = n_inter;
        ml.w[1] = up_w;   ml.s[1] = up_s;   ml.b[1] = up_b;   ml.out[1] = hm; ml.n_out[1] = n_inter;
        for (int k = 2; k < kMaxMats; k++) {
            ml.w[k] = up_w; ml.s[k] = up_s; ml.b[k] = up_b; ml.out[k] = hm; ml.n_out[k] = 0;
        }
        ml.row_begin[0] = 0;
        for (int k = 0; k < kMaxMats; k++) ml.row_begin[k + 1] = ml.row_begin[k] + ml.n_out[k];
        ml.count = 2;
        int done = 0;
        if (gs == 64 && n_in > 0 && !(reinterpret_cast<uintptr_t>(xm) & 15) &&
            (n_in / 8 + kChunkWords - 1) / kChunkWords <= 16) {
            done = mm == 1 ? launch_stream<1, true>(ml, xm, n_in, st)
                           : launch_stream<2, true>(ml, xm, n_in, st);
            if (done < 0) return done;
        }
        if (!done) {        // unfused: gate into h, up into the workspace, then SiLU * mul
            Workspace* ws;
            {
                std::lock_guard<std::mutex> lock(g_mu);
                int dev;
                if ((rc = current_device(&dev))) return rc;
                ws = &g_dev[dev].ws[st];
            }
            const size_t n = static_cast<size_t>(mm) * n_inter;
            if ((rc = ensure_tmp(*ws, st, n))) return rc;
            if ((rc = q4_gemv_dev(gate_w, gate_s, gate_b, xm, hm, mm, n_inter, n_in, gs, stream))) return rc;
            if ((rc = q4_gemv_dev(up_w, up_s, up_b, xm, ws->tmp, mm, n_inter, n_in, gs, stream))) return rc;
            hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, st, hm, ws->tmp, hm,
                               static_cast<long>(n));
            HIP_TRY(hipGetLastError());
        }
    }
    return 0;
}

int q4_mlp_dev(const uint32_t* gate_w, const uint16_t* gate_s, const uint16_t* gate_b,
               const uint32_t* up_w, const uint16_t* up_s, const uint16_t* up_b,
               const uint32_t* down_w, const uint16_t* down_s, const uint16_t* down_b,
               const float* x, float* h, float* out, int m, int n_hidden, int n_inter, int gs,
               void* stream) {
    int rc = check_gemv_shape(n_hidden, n_inter, gs);
    if (rc) return rc;
    if ((rc = q4_gate_up_silu_dev(gate_w, gate_s, gate_b, up_w, up_s, up_b, x, h, m, n_inter,
                                  n_hidden, gs, stream)))
        return rc;
    return q4_gemv_dev(down_w, down_s, down_b, h, out, m, n_hidden, n_inter, gs, stream);
}


int q4_gemm_bf16_dev(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                     const float* x, float* out, int m, int n_out, int n_in, int gs, void* stream) {
    int rc = check_gemv_shape(n_out, n_in, gs);
    if (rc) return rc;
    if (gs != 64) return fail(Q4_EARG, "q4_gemm_bf16_dev takes gs = 64 (got %d)", gs);
    if (m < 0) return fail(Q4_EARG, "m=%d", m);
    if (m == 0 || n_out == 0) return 0;
    if (!w || !scales || !biases || !x || !out) return fail(Q4_EARG, "null pointer");
    if ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x)) & 15)
        return fail(Q4_EARG, "w and x must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (n_in == 0) {
        const long n = static_cast<long>(m) * n_out;
        hipLaunchKernelGGL(fill_zero_kernel, dim3((n + 255) / 256), dim3(256), 0, st, out, n);
        HIP_TRY(hipGetLastError());
        return 0;
    }
    // 128 x 128 tiles once there are enough of them for the CUs, else 128 x 64
    const long tiles128 = static_cast<long>((m + 127) / 128) * ((n_out + 127) / 128);
    if (tiles128 >= 2L * num_cus()) return launch_gemm<128, 128>(w, scales, biases, x, out, m, n_out, n_in, st);
    return launch_gemm<128, 64>(w, scales, biases, x, out, m, n_out, n_in, st);
}

int q4_dequant_dev(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, float* out,
                   int row0, int row1, int n_in, int gs, void* stream) {
    int rc = check_dequant_shape(n_in, gs);
    if (rc) return rc;
    if (row1 - row0 <= 0) return 0;
    if (row0 < 0) return fail(Q4_EARG, "row0=%d", row0);
    if (!w || !scales || !biases || !out) return fail(Q4_EARG, "null pointer");
    if (reinterpret_cast<uintptr_t>(out) & 15) return fail(Q4_EARG, "out must be 16-byte aligned");
    return dequant_launch<false>(w, scales, biases, out, row0, row1 - row0, n_in, gs,
                                 static_cast<hipStream_t>(stream));
}

int q4_dequant_bf16_dev(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                        uint16_t* out, int row0, int row1, int n_in, int gs, void* stream) {
    int rc = check_dequant_shape(n_in, gs);
    if (rc) return rc;
    if (row1 - row0 <= 0) return 0;
    if (row0 < 0) return fail(Q4_EARG, "row0=%d", row0);
    if (!w || !scales || !biases || !out) return fail(Q4_EARG, "null pointer");
    if (reinterpret_cast<uintptr_t>(out) & 15) return fail(Q4_EARG, "out must be 16-byte aligned");
    return dequant_launch<true>(w, scales, biases, out, row0, row1 - row0, n_in, gs,
                                static_cast<hipStream_t>(stream));
}

}  // extern "C"
