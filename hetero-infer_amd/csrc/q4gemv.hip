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

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <type_traits>
#include <mutex>
#include <tuple>
#include <vector>

#include "q4_stream.h"
#include "q4_mfma_m.h"
#include "q4decode.h"

namespace q4k {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
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

// The stream slots of each device: the stream holding each slot and when it
// last used it; a stream new to the table takes a free slot, else the
// least recently used one.
struct SlotTable {
    hipStream_t stream[kStreamSlots] = {};
    uint64_t used[kStreamSlots] = {};
    bool taken[kStreamSlots] = {};
    uint64_t tick = 0;
};
std::mutex g_slot_mu;
std::map<int, SlotTable> g_slots;

int stream_slot(hipStream_t st, int* slot) {
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(Q4_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    std::lock_guard<std::mutex> lock(g_slot_mu);
    SlotTable& t = g_slots[dev];
    int pick = -1;
    for (int i = 0; i < kStreamSlots && pick < 0; i++)
        if (t.taken[i] && t.stream[i] == st) pick = i;
    if (pick < 0) {
        int free_i = -1, lru = -1;
        for (int i = 0; i < kStreamSlots; i++) {
            if (!t.taken[i]) {
                if (free_i < 0) free_i = i;
            } else if (lru < 0 || t.used[i] < t.used[lru]) {
                lru = i;
            }
        }
        pick = free_i >= 0 ? free_i : lru;
        t.taken[pick] = true;
        t.stream[pick] = st;
    }
    t.used[pick] = ++t.tick;
    *slot = pick;
    return 0;
}

// The streaming kernel's instances are compiled in q4_stream_inst.hip
// (a build with -DQ4_SINGLE_TU instantiates them here instead).
#ifndef Q4_SINGLE_TU
#define Q4_STREAM_EXTERN(MR, RW, PAIR, RING, NORM, GSH)                                            \
    extern template int launch_stream_k<MR, RW, PAIR, RING, NORM, GSH>(const MatList&, const float*,   \
                                                                       const NormArgs&, int, int, int, \
                                                                       size_t, int, int, hipStream_t);
#define Q4_STREAM_RINGS(MR, RW, PAIR, NORM, GSH)                                                    \
    Q4_STREAM_EXTERN(MR, RW, PAIR, 1, NORM, GSH) Q4_STREAM_EXTERN(MR, RW, PAIR, 2, NORM, GSH)
#define Q4_STREAM_GS(GSH)                                                                           \
    Q4_STREAM_RINGS(1, 1, false, false, GSH) Q4_STREAM_RINGS(1, 2, false, false, GSH)              \
    Q4_STREAM_RINGS(1, 3, false, false, GSH) Q4_STREAM_RINGS(1, 4, false, false, GSH)              \
    Q4_STREAM_EXTERN(1, 1, false, 5, false, GSH) Q4_STREAM_EXTERN(1, 2, false, 5, false, GSH)      \
    Q4_STREAM_EXTERN(1, 3, false, 5, false, GSH) Q4_STREAM_EXTERN(1, 4, false, 5, false, GSH)      \
    Q4_STREAM_RINGS(1, 1, true, false, GSH) Q4_STREAM_RINGS(1, 2, true, false, GSH)                \
    Q4_STREAM_RINGS(2, 1, false, false, GSH) Q4_STREAM_RINGS(2, 2, false, false, GSH)              \
    Q4_STREAM_RINGS(2, 1, true, false, GSH) Q4_STREAM_RINGS(2, 2, true, false, GSH)
Q4_STREAM_GS(0)
Q4_STREAM_GS(1)
Q4_STREAM_RINGS(1, 1, false, true, 0) Q4_STREAM_EXTERN(1, 1, false, 5, true, 0)
Q4_STREAM_RINGS(1, 1, true, true, 0)
#undef Q4_STREAM_GS
#undef Q4_STREAM_RINGS
#undef Q4_STREAM_EXTERN
#endif

}  // namespace q4k

namespace {

using namespace q4k;

constexpr int kMaxM = 8;           // activation rows per main-kernel launch
constexpr int kLdsBudget = 64 * 1024;

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

// The reference's fp32 path for the rows past its last ROWS block
// (kernel/q4gemv.c:185-200; rows [row0, n_out) of an m-row GEMV): one wave
// per (row, activation row).  Lane l takes groups l, l + 64, ..; for its
// group it adds the 64 values of x in ascending order (the xsum of
// :244-248), chains s = fma(q, x, s) over the group's values in ascending
// order (:192-195; clang contracts the reference's `s += q * x`), and forms
// the term fma(scale, s, bias * xsum) (:196-197).  Lane 0 then adds the
// terms to the row's sum in ascending group order.
__global__ __launch_bounds__(64) void tail_rows_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ sc, const uint16_t* __restrict__ bi,
    const float* __restrict__ x, float* __restrict__ out, int row0, int n_out, int n_in, int gs) {
    __shared__ float terms[64];
    const int o = row0 + blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
    const int G = n_in / gs, wpr = n_in >> 3, wpg = gs >> 3;
    const float* xr = x + static_cast<size_t>(m) * n_in;
    const uint32_t* wr = w + static_cast<size_t>(o) * wpr;
    float acc = 0.0f;
    for (int g0 = 0; g0 < G; g0 += 64) {
        const int g = g0 + lane;
        float term = 0.0f;
        if (g < G) {
            float xs = 0.0f, sd = 0.0f;
            for (int i = 0; i < gs; i++) xs = __fadd_rn(xs, xr[g * gs + i]);
            for (int k = 0; k < wpg; k++) {
                const uint32_t d = wr[g * wpg + k];
                for (int n = 0; n < 8; n++)
                    sd = __builtin_fmaf(static_cast<float>((d >> (4 * n)) & 0xFu), xr[g * gs + 8 * k + n], sd);
            }
            const size_t si = static_cast<size_t>(o) * G + g;
            term = __builtin_fmaf(h2f(sc[si]), sd, __fmul_rn(h2f(bi[si]), xs));
        }
        terms[lane] = term;
        __syncthreads();
        if (lane == 0) {
            const int n = G - g0 < 64 ? G - g0 : 64;
            for (int i = 0; i < n; i++) acc = __fadd_rn(acc, terms[i]);
        }
        __syncthreads();
    }
    if (lane == 0) out[static_cast<size_t>(m) * n_out + o] = acc;
}

// h = SiLU(g) * u elementwise (fallback of the fused gate/up launch).
__global__ void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                float* __restrict__ h, long n) {
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) h[i] = silu_mul(g[i], u[i]);
}

__global__ void fill_zero_u16_kernel(uint16_t* __restrict__ p, long n) {
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
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
// reference hands to BLAS after q4_dequant (hetero/cpu_model.py:119-136): x
// is rounded to bf16 once per call (x_to_bf16_kernel), W stays 4-bit up to
// the matrix cores (gemm_w4_kernel, q4_gemm.hip), where it becomes
// bf16(fma(q, scale, bias)) -- exactly q4_dequant_bf16 -- and
// v_mfma_f32_32x32x16_bf16 accumulates in fp32; split-K partials are added
// in split order (splitk_sum_kernel).
// a in the low half, b in the high half, each rounded to nearest even: one
// v_cvt_pk_bf16_f32 (two scalar conversions became a conversion each plus
// shifts and ors)
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
    const f32x2 p = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(p, bf16x2v));
}

// x rounded to bf16 (RNE) once per call, 8 values per thread.
__global__ __launch_bounds__(256) void x_to_bf16_kernel(const float* __restrict__ x, uint4* __restrict__ xb,
                                                        long n8) {
    const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n8) {
        const float4 a = reinterpret_cast<const float4*>(x)[2 * i], b = reinterpret_cast<const float4*>(x)[2 * i + 1];
        uint4 o;
        o.x = pack_bf16x2(a.x, a.y);
        o.y = pack_bf16x2(a.z, a.w);
        o.z = pack_bf16x2(b.x, b.y);
        o.w = pack_bf16x2(b.z, b.w);
        xb[i] = o;
    }
}

// The S split-K partials part[s][r][c] (r < M, c < W: the matrices' columns
// side by side) summed in split order into the output of column c's
// matrix.
__global__ __launch_bounds__(256) void splitk_sum_kernel(const float* __restrict__ part, GemmMats gm, int M, int W,
                                                         int S) {
    const long n = static_cast<long>(M) * W;
    const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) {
        float a = part[i];
        for (int s = 1; s < S; s++) a = __fadd_rn(a, part[static_cast<long>(s) * n + i]);
        const long r = i / W;
        const int c = static_cast<int>(i - r * W);
        int k = 0;
        for (int j = 1; j < gm.count; j++) k += c >= gm.col0[j] ? 1 : 0;
        gm.out[k][r * gm.n_out[k] + (c - gm.col0[k])] = a;
    }
}

// ============================================================ host side ===

#define HIP_TRY(expr)                                                              \
    do {                                                                           \
        hipError_t e_ = (expr);                                                    \
        if (e_ != hipSuccess) {                                                    \
            return fail(e_ == hipErrorOutOfMemory ? Q4_ENOMEM : Q4_EHIP, "%s: %s", \
                        #expr, hipGetErrorString(e_));                             \
        }                                                                          \
    } while (0)

bool pow2_gs(int gs) { return gs >= 64 && gs <= 2048 && (gs & (gs - 1)) == 0; }

// Per-stream workspace: the x prologue's outputs (byte planes, group sums,
// scales), the unfused MLP's up rows, and the prefill's bf16 copy of x,
// partial sums and stream-K flags.  Buffers only grow.  A buffer that a call used while
// its stream was being captured may be baked into a graph, so when it has to
// grow later it is retired -- kept allocated until the process ends --
// instead of freed; a buffer no graph holds is freed once the stream has
// drained (earlier launches may still read it).  A `fixed` workspace is the
// library's static scratch (q4_gemv_noalloc_dev): it never grows.
struct Workspace {
    uint4* planes = nullptr;
    float* xsum = nullptr;
    float* xscale = nullptr;
    float* tmp = nullptr;                       // up-projection rows of the unfused MLP
    void* xbf = nullptr;                        // prefill: bf16 copy of x
    void* part = nullptr;                       // prefill: split-K / stream-K partial sums
    unsigned* sk = nullptr;                     // prefill: stream-K flags, then its control words
    size_t cap[7] = {0, 0, 0, 0, 0, 0, 0};      // bytes, in the order above
    bool in_graph[7] = {false, false, false, false, false, false, false};
    bool fixed = false;
    std::vector<void*> retired;
};
enum WsBuf { kWsPlanes, kWsXsum, kWsXscale, kWsTmp, kWsXbf, kWsPart, kWsSk };

// Make buffer `which` (pointer p) of the workspace hold `bytes`.  Growing is
// refused while the stream is captured (an allocation cannot be recorded).
template <typename T>
int grow(Workspace& ws, T*& p, WsBuf which, size_t bytes, hipStream_t st, const char* what) {
    size_t& cap = ws.cap[which];
    if (ws.fixed) {
        if (bytes <= cap) return 0;
        return fail(Q4_EARG, "%s: needs %zu bytes of scratch, above the library's fixed %zu", what, bytes, cap);
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(st, &cs));
    const bool capturing = cs != hipStreamCaptureStatusNone;
    if (bytes <= cap && p) {
        if (capturing) ws.in_graph[which] = true;
        return 0;
    }
    if (capturing)
        return fail(Q4_EARG, "%s workspace of this stream must grow during graph capture: "
                             "run the largest call once on the stream before capturing", what);
    HIP_TRY(hipStreamSynchronize(st));
    if (p) {
        if (ws.in_graph[which]) ws.retired.push_back(static_cast<void*>(p));
        else (void)hipFree(static_cast<void*>(p));
    }
    p = nullptr;
    cap = 0;
    ws.in_graph[which] = false;
    void* np = nullptr;
    HIP_TRY(hipMalloc(&np, bytes));
    p = static_cast<T*>(np);
    cap = bytes;
    return 0;
}

// The stream-K control words of the workspace: after one flag line per CU.
unsigned* sk_ctl(Workspace& ws) { return ws.sk + static_cast<size_t>(num_cus()) * 32; }

int ensure_tmp(Workspace& ws, hipStream_t st, size_t n) {
    return grow(ws, ws.tmp, kWsTmp, n * sizeof(float), st, "MLP");
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

// HBM copy of host weights.  `base` is the host address of the whole
// matrix's packed weights: q4_dequant registers row blocks under their own
// addresses, and q4_release(base) must find them too.
struct Resident {
    uint32_t* w = nullptr;
    uint16_t* s = nullptr;
    uint16_t* b = nullptr;
    uint64_t fp = 0;
    const void* base = nullptr;
};

// (device, w, scales, biases, n_out, n_in, gs)
using ResKey = std::tuple<int, const void*, const void*, const void*, int, int, int>;

std::mutex g_mu;                       // serialises every host-pointer call
std::map<int, DevState> g_dev;
std::map<ResKey, Resident> g_res;

// words: uint4 of planes; groups: floats of group sums
int ensure_ws(Workspace& ws, hipStream_t st, size_t words, size_t groups) {
    const size_t cw = words < 4096 ? 4096 : words, cg = groups < 1024 ? 1024 : groups;
    if (int rc = grow(ws, ws.planes, kWsPlanes, (ws.fixed ? words : cw) * sizeof(uint4), st, "x")) return rc;
    if (int rc = grow(ws, ws.xsum, kWsXsum, (ws.fixed ? groups : cg) * sizeof(float), st, "x")) return rc;
    return grow(ws, ws.xscale, kWsXscale, kMaxM * sizeof(float), st, "x");
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


template <int MR, int RW, bool PAIR, bool NORM, int GSH>
int launch_stream_rw(const MatList& ml, const float* x, const NormArgs& na, int n_in, int UB, int nwaves,
                     size_t lds, int sep, int n_units, int items, hipStream_t st) {
    // one unit per wave, capped by the launch at what is resident at once
    const int grid = (n_units + nwaves - 1) / nwaves;
    // ring: a divisor of the unit's items (units change only between rings),
    // two items where they divide it.  Deeper rings were slower on every
    // large shape (same-box, down 18944 -> 3584: 13.5 us at 5 items,
    // 15.6 us at 10, 12.5 us at 2, 14.7 us at 1; gate+up 17.3 us at 4,
    // 16.3 us at 2), the more loads a CU has queued the longer each waits.
    if (items % 2 == 0)
        return launch_stream_k<MR, RW, PAIR, 2, NORM, GSH>(ml, x, na, n_in, UB, nwaves, lds, sep, grid, st);
    if constexpr (MR == 1 && !PAIR)
        if (items % 5 == 0)
            return launch_stream_k<MR, RW, PAIR, 5, NORM, GSH>(ml, x, na, n_in, UB, nwaves, lds, sep, grid, st);
    return launch_stream_k<MR, RW, PAIR, 1, NORM, GSH>(ml, x, na, n_in, UB, nwaves, lds, sep, grid, st);
}

// GSH: group size 64 << GSH.  NORM: the norm prologue (group size 64; one
// row; one word of x per thread, so at least
// n_in / 512 waves -- n_in <= 8192).  Returns 0 if the shape does not fit.
template <int MR, bool PAIR = false, bool NORM = false, int GSH = 0>
int launch_stream(const MatList& ml, const float* x, int n_in, hipStream_t st, const NormArgs& na = NormArgs{}) {
    static_assert(!NORM || MR == 1, "the norm prologue takes one row");
    constexpr int kWavesPerCu = stream_waves_per_cu<MR>();
    constexpr int rmax = NORM ? 1 : stream_max_rounds<MR>();
    const int G = n_in / (64 << GSH);
    const int C = (n_in / 8 + kChunkWords - 1) / kChunkWords;
    const int n_total = PAIR ? ml.n_out[0] : ml.row_begin[ml.count];
    const int cus = num_cus();
    // smallest workgroup the prologue accepts: at most rmax words of x per
    // thread and row
    const int minw = (C * kChunkWords + 64 * rmax - 1) / (64 * rmax);
    if (minw > kWavesPerCu) return 0;
    // rows per unit: 1, or more when rows are plentiful and short -- up to 8
    // rows and kUnitItems items, while every wave still gets two units (the
    // end of a unit costs a serial chain, a unit too many per wave a tail)
    int UB = 1;
    while (UB < 8 && UB * C * (PAIR ? 2 : 1) < kUnitItems && n_total >= 4 * UB * kWavesPerCu * cus) UB *= 2;
    while (MR * UB > 64) UB >>= 1;
    for (int k = 0; k < ml.count; k++)                 // a unit must not straddle matrices
        while (ml.n_out[k] % UB) UB >>= 1;
    const int n_units = (n_total + UB - 1) / UB;
    // one unit per wave while the units fit on the chip at once, the waves
    // spread evenly over the CUs (3584 rows: 256 workgroups of 14 waves)
    const int target = n_units < kWavesPerCu * cus ? n_units : kWavesPerCu * cus;
    int nwaves = (target + cus - 1) / cus;
    if (nwaves < minw) nwaves = minw;
    if (nwaves > kWavesPerCu) nwaves = kWavesPerCu;
    const int rw = (C * kChunkWords + 64 * nwaves - 1) / (64 * nwaves);
    // the x staging in LDS of its own while that keeps two workgroups per CU
    // possible: one barrier fewer in the prologue
    const size_t lds_sep = stream_lds_bytes(MR, C, G, nwaves, (PAIR ? 2 : 1) * UB, rw, GSH, true);
    const int sep = lds_sep <= kStreamLdsMax / 2 ? 1 : 0;
    const size_t lds = sep ? lds_sep : stream_lds_bytes(MR, C, G, nwaves, (PAIR ? 2 : 1) * UB, rw, GSH);
    if (lds > kStreamLdsMax) return 0;
    const int items = (PAIR ? 2 : 1) * UB * C;
    if constexpr (NORM)
        return rw == 1 && GSH == 0
                   ? launch_stream_rw<MR, 1, PAIR, true, 0>(ml, x, na, n_in, UB, nwaves, lds, sep, n_units, items, st)
                   : 0;
    switch (rw) {
        case 1: return launch_stream_rw<MR, 1, PAIR, false, GSH>(ml, x, na, n_in, UB, nwaves, lds, sep, n_units, items, st);
        case 2:
            if constexpr (rmax >= 2)
                return launch_stream_rw<MR, 2, PAIR, false, GSH>(ml, x, na, n_in, UB, nwaves, lds, sep, n_units, items, st);
            return 0;
        // (3 and 4 words per thread: the single-matrix launches of one row)
        case 3:
            if constexpr (rmax >= 3 && !PAIR)
                return launch_stream_rw<MR, 3, PAIR, false, GSH>(ml, x, na, n_in, UB, nwaves, lds, sep, n_units, items, st);
            return 0;
        case 4:
            if constexpr (rmax >= 4 && !PAIR)
                return launch_stream_rw<MR, 4, PAIR, false, GSH>(ml, x, na, n_in, UB, nwaves, lds, sep, n_units, items, st);
            return 0;
        default: return 0;
    }
}

// The streaming path takes gs 64 or 128, x 16-byte aligned and at most 16
// chunks (n_in <= 32768).  Returns 1 if it launched, 0 if the call must
// take the split path, <0 on error.
bool stream_takes(const float* x, int n_in, int gs) {
    if ((gs != 64 && gs != 128) || n_in == 0 || (reinterpret_cast<uintptr_t>(x) & 15)) return false;
    return (n_in / 8 + kChunkWords - 1) / kChunkWords <= 16;
}

template <int MR, bool PAIR = false>
int launch_stream_gs(const MatList& ml, const float* x, int n_in, int gs, hipStream_t st) {
    return gs == 128 ? launch_stream<MR, PAIR, false, 1>(ml, x, n_in, st) : launch_stream<MR, PAIR, false, 0>(ml, x, n_in, st);
}

template <int MR>
int try_fused(const MatList& ml, const float* x, int n_in, int gs, hipStream_t st) {
    if (!stream_takes(x, n_in, gs)) return 0;
    return launch_stream_gs<MR>(ml, x, n_in, gs, st);
}

// One or two rows: the streaming kernel's instance of that row count.
int try_fused_m(const MatList& ml, const float* x, int m, int n_in, int gs, hipStream_t st) {
    MatList mm = ml;
    mm.mrows = m;
    switch (m) {
        case 1: return try_fused<1>(mm, x, n_in, gs, st);
        case 2: return try_fused<2>(mm, x, n_in, gs, st);
        // (3..8 rows take the matrix cores, or the split path where those
        // decline the shape)
        default: return 0;
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

template <bool PAIR, int S, bool SB8, int TR>
int launch_mfma_k(const q4k::MfMats& mt, int n, int n_in, int m, const Workspace& ws, float* out, hipStream_t st) {
    auto kern = q4k::gemv_mfma_kernel<PAIR, S, SB8, TR>;
    constexpr size_t lds = (PAIR ? 2 : 1) * 256 * q4k::kMfRing * S * sizeof(float);
    static std::atomic<uint64_t> lds_raised{0};
    if (int rc = q4k::raise_lds_limit(reinterpret_cast<const void*>(kern), lds, lds_raised)) return rc;
    const int tiles = (n + TR - 1) / TR;
    hipLaunchKernelGGL(kern, dim3(tiles), dim3(64 * S), lds, st, mt, n, n_in, m,
                       reinterpret_cast<const uint32_t*>(ws.planes), ws.xsum, ws.xscale, out, n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q4_EHIP, "mfma gemv launch: %s", hipGetErrorString(e));
    return 1;
}

template <bool PAIR, bool SB8>
int launch_mfma_s(const q4k::MfMats& mt, int n, int n_in, int m, const Workspace& ws, float* out, hipStream_t st) {
    // One workgroup per CU holds a fixed number of weight bytes in flight
    // (the register ring), so the workgroups must cover the CUs: 16-row
    // tiles of 8 waves when 32-row tiles would leave CUs idle (one matrix of
    // 3584 rows: 224 tiles), 32-row tiles of 8 waves while they do not fill
    // the CUs twice, else 4 waves.
    const int tiles = (n + 31) / 32, cus = num_cus();
    if constexpr (!PAIR)
        if (tiles < cus) return launch_mfma_k<PAIR, 8, SB8, 16>(mt, n, n_in, m, ws, out, st);
    return tiles < 2 * cus ? launch_mfma_k<PAIR, 8, SB8, 32>(mt, n, n_in, m, ws, out, st)
                           : launch_mfma_k<PAIR, 4, SB8, 32>(mt, n, n_in, m, ws, out, st);
}

// Rows of x from which the matrix-core path is used.  Its cost does not
// depend on the row count; the streaming kernel's grows with it (Qwen2.5-7B
// MLP block: 60 us at 2 rows and 80 us at 3-4 rows streaming, 64 us on the
// matrix cores; q_proj about even at 3-4 rows).
constexpr int kMfMinRows = 3;

// Small-M GEMV on the int8 matrix cores (q4_mfma_m.h): kMfMinRows <= m <= kMaxM,
// gs 64, n_in <= 32768, x 16-byte aligned, every byte offset into the
// matrix below 2^31.  PAIR: mt holds gate and up, out receives
// SiLU(gate) * up.  x is prepared into the stream's workspace by
// xprep_mf_kernel.  Returns 1 if it launched, 0 if the shape is not one it
// takes, <0 on error.
bool mfma_takes(int m, int n, int n_in, int gs, const float* x) {
    if (m < kMfMinRows || m > kMaxM || gs != 64 || n_in <= 0 || n <= 0 || n_in > q4k::kMfPrepMaxK) return false;
    if (reinterpret_cast<uintptr_t>(x) & 15) return false;
    // (n + 32 rows: a tile's second weight load starts 16 rows past the first)
    const long G = n_in / 64;
    return static_cast<long>(n + 32) * (n_in / 2) < (1L << 31) && static_cast<long>(n) * G * 2 < (1L << 31);
}

// x of m rows quantised into the stream's workspace for the matrix-core
// kernel (xprep_mf_kernel); every later launch on the stream reads it.
int mfma_prep(const float* x, int m, int n_in, hipStream_t st, Workspace& ws) {
    const long G = n_in / 64;
    int rc = ensure_ws(ws, st, static_cast<size_t>(G) * 2 * q4k::kMfArows * 2, static_cast<size_t>(G) * 8);
    if (rc) return rc;
    static std::atomic<uint64_t> prep_raised{0};
    if ((rc = q4k::raise_lds_limit(reinterpret_cast<const void*>(q4k::xprep_mf_kernel),
                                   q4k::kMfPrepMaxK * sizeof(float), prep_raised)))
        return rc;
    // each row's groups in slices of at least 32 over up to 8 workgroups
    // (every workgroup of a row reads the whole row for its amax)
    const int slices = static_cast<int>(G / 32 < 1 ? 1 : (G / 32 > 8 ? 8 : G / 32));
    hipLaunchKernelGGL(q4k::xprep_mf_kernel, dim3(slices, kMaxM), dim3(1024), static_cast<size_t>(n_in) * sizeof(float),
                       st, x, m, n_in, reinterpret_cast<uint32_t*>(ws.planes), ws.xsum, ws.xscale);
    HIP_TRY(hipGetLastError());
    return 0;
}

// The matrix-core GEMV on x prepared by mfma_prep.  Returns 1 (launched) or <0.
int mfma_main(const q4k::MfMats& mt, bool pair, float* out, int m, int n, int n_in, hipStream_t st,
              const Workspace& ws) {
    const bool sb8 = (n_in / 64) % 8 == 0;
    if (pair) return sb8 ? launch_mfma_s<true, true>(mt, n, n_in, m, ws, out, st)
                         : launch_mfma_s<true, false>(mt, n, n_in, m, ws, out, st);
    return sb8 ? launch_mfma_s<false, true>(mt, n, n_in, m, ws, out, st)
               : launch_mfma_s<false, false>(mt, n, n_in, m, ws, out, st);
}

int gemv_mfma(const q4k::MfMats& mt, bool pair, const float* x, float* out, int m, int n, int n_in, int gs,
              hipStream_t st, Workspace& ws) {
    if (!mfma_takes(m, n, n_in, gs, x)) return 0;
    if (int rc = mfma_prep(x, m, n_in, st, ws)) return rc;
    return mfma_main(mt, pair, out, m, n, n_in, st, ws);
}

// ROWS of the reference build being replaced (kernel/build.sh:7, -DROWS):
// HETERO_Q4_ROWS, read on first use, or q4_set_rows.  1..64.
constexpr int kMaxRowsBlock = 64;
std::atomic<int> g_rows{0};                    // 0: not read yet

int rows_block(int* out) {
    int r = g_rows.load(std::memory_order_relaxed);
    if (r == 0) {
        const char* e = std::getenv("HETERO_Q4_ROWS");
        char* end = nullptr;
        const long v = e && *e ? std::strtol(e, &end, 10) : 1;
        if (e && *e && (*end != 0 || v < 1 || v > kMaxRowsBlock))
            return fail(Q4_EARG, "HETERO_Q4_ROWS=%s: expected an integer in [1, %d]", e, kMaxRowsBlock);
        r = static_cast<int>(v);
        int expect = 0;
        g_rows.compare_exchange_strong(expect, r, std::memory_order_relaxed);
        r = g_rows.load(std::memory_order_relaxed);
    }
    *out = r;
    return 0;
}

// The last n_out % ROWS rows of an m-row GEMV by the reference's fp32 tail
// path (kernel/q4gemv.c:185-200, rows past the last ROWS block): after the
// integer path has written every row, they are computed again and
// overwritten.  Nothing to do for ROWS = 1 or n_out % ROWS == 0.
int tail_rows(const uint32_t* w, const uint16_t* s, const uint16_t* b, const float* x, float* out, int m,
              int n_out, int n_in, int gs, hipStream_t st) {
    int R = 1;
    if (int rc = rows_block(&R)) return rc;
    const int tail = n_out % R;
    if (tail == 0 || m == 0 || n_in == 0) return 0;
    hipLaunchKernelGGL(tail_rows_kernel, dim3(tail, m), dim3(64), 0, st, w, s, b, x, out, n_out - tail, n_out, n_in,
                       gs);
    HIP_TRY(hipGetLastError());
    return 0;
}

// The tail rows of each matrix of a grouped call (each matrix is a q4_gemv
// call of its own in the reference).
int multi_tails(int count, const uint32_t* const* w, const uint16_t* const* scales, const uint16_t* const* biases,
                float* const* out, const int* n_out, const float* x, int m, int n_in, int gs, hipStream_t st) {
    for (int k = 0; k < count; k++)
        if (int rc = tail_rows(w[k], scales[k], biases[k], x, out[k], m, n_out[k], n_in, gs, st)) return rc;
    return 0;
}

int gemv_rows_int(const uint32_t* w, const uint16_t* s, const uint16_t* b, const float* x,
                  float* out, int m, int n_out, int n_in, int gs, hipStream_t st, Workspace& ws);

// GEMV of m (<= kMaxM) rows already on the device, as the reference build
// with ROWS = rows_block() computes it: the integer path, then the tail rows.
int gemv_rows(const uint32_t* w, const uint16_t* s, const uint16_t* b, const float* x,
              float* out, int m, int n_out, int n_in, int gs, hipStream_t st, Workspace& ws) {
    if (int rc = gemv_rows_int(w, s, b, x, out, m, n_out, n_in, gs, st, ws)) return rc;
    return tail_rows(w, s, b, x, out, m, n_out, n_in, gs, st);
}

// The integer path for every row: the matrix cores for kMfMinRows..8 rows,
// else fused when possible.
int gemv_rows_int(const uint32_t* w, const uint16_t* s, const uint16_t* b, const float* x,
                  float* out, int m, int n_out, int n_in, int gs, hipStream_t st, Workspace& ws) {
    if (m >= kMfMinRows) {
        const q4k::MfMats mt{{w, w}, {s, s}, {b, b}};
        const int rc = gemv_mfma(mt, false, x, out, m, n_out, n_in, gs, st, ws);
        if (rc < 0) return rc;
        if (rc == 1) return 0;
    }
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

// Hash of every byte (four independent multiply-xor lanes over 8-byte
// words, so the host reads at memory speed): the exact check of
// Q4_RESIDENCY_CHECK=full.
uint64_t content_hash(const void* p, size_t bytes) {
    const uint8_t* c = static_cast<const uint8_t*>(p);
    uint64_t h[4] = {1469598103934665603ull ^ bytes, 0x9E3779B97F4A7C15ull, 0xC2B2AE3D27D4EB4Full,
                     0x165667B19E3779F9ull};
    size_t i = 0;
    for (; i + 32 <= bytes; i += 32) {
        uint64_t v[4];
        memcpy(v, c + i, 32);
        for (int k = 0; k < 4; k++) h[k] = (h[k] ^ v[k]) * 1099511628211ull;
    }
    for (int k = 0; k < 4 && i + 8 * k < bytes; k++) {           // the last 0..31 bytes, zero-padded
        uint64_t v = 0;
        const size_t n = bytes - i - 8 * k < 8 ? bytes - i - 8 * k : 8;
        memcpy(&v, c + i + 8 * k, n);
        h[k] = (h[k] ^ v) * 1099511628211ull;
    }
    return (h[0] ^ (h[1] >> 1)) * 31 + (h[2] ^ (h[3] << 1));
}

// Q4_RESIDENCY_CHECK=full makes every host-pointer call hash all of its
// weights (the reference reads them on every call, so an in-place edit
// anywhere shows); the default samples 16 words per array.
bool residency_check_full() {
    const char* e = std::getenv("Q4_RESIDENCY_CHECK");
    return e && std::strcmp(e, "full") == 0;
}

// base: the host address of the whole matrix's packed weights (w itself
// unless w is a row block of it)
int resident(const uint32_t* w, const uint16_t* s, const uint16_t* b, int n_out, int n_in,
             int gs, int dev, Resident** out, const void* base = nullptr) {
    const size_t wb = static_cast<size_t>(n_out) * (n_in / 8) * 4;
    const size_t gb = static_cast<size_t>(n_out) * (n_in / gs) * 2;
    auto h = residency_check_full() ? content_hash : fingerprint;
    const uint64_t fp = h(w, wb) * 31 + h(s, gb) * 7 + h(b, gb);
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
    r.base = base ? base : static_cast<const void*>(w);
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


// The arguments of the norm-prologue entry points: gs 64, n_in in
// [64, 8192], the vectors 16-byte aligned, x_out overlapping neither input.
int check_norm_args(const char* who, const float* x, const float* delta, const float* norm_w, const float* x_out,
                    int n_in, int gs) {
    if (!x || !norm_w) return fail(Q4_EARG, "%s: null x or norm weights", who);
    if (gs != 64) return fail(Q4_EARG, "%s takes gs = 64 (got %d)", who, gs);
    if (n_in <= 0 || n_in > 8192) return fail(Q4_EARG, "%s: n_in = %d outside [64, 8192]", who, n_in);
    const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(delta) |
                         reinterpret_cast<uintptr_t>(norm_w) | reinterpret_cast<uintptr_t>(x_out);
    if (al & 15) return fail(Q4_EARG, "%s: x, delta, norm_w and x_out must be 16-byte aligned", who);
    auto overlap = [n_in](const float* a, const float* b) { return a && b && a < b + n_in && b < a + n_in; };
    if (overlap(x_out, x) || overlap(x_out, delta))
        return fail(Q4_EARG, "%s: x_out overlaps x or delta", who);
    return 0;
}

// ---------------------------------------------------- static scratch ----
//
// The workspace of q4_gemv_noalloc_dev: a fixed array in device memory, so
// that call allocates nothing.  Sized for up to 8 rows at a time of
// n_in <= kNoAllocMaxIn: the x planes (8 rows x n_in/8 words as uint4 for
// the split path; 64 uint4 per group for the matrix-core prep -- both
// 32768 uint4 at the limit), the group sums (8 rows x 512 groups) and the
// 8 row scales.  Each GPU holds its own copy for the life of the process.
constexpr int kNoAllocMaxIn = 32768;
constexpr size_t kScrPlanes = static_cast<size_t>(kMaxM) * (kNoAllocMaxIn / 8);   // uint4
constexpr size_t kScrXsum = static_cast<size_t>(kMaxM) * (kNoAllocMaxIn / 64);    // floats
constexpr size_t kScrXscale = 64;                                                  // floats
static_assert(kScrPlanes >= static_cast<size_t>(kNoAllocMaxIn / 64) * 2 * q4k::kMfArows * 2,
              "the matrix-core prep fits the planes");
static __device__ __align__(256) uint4 scratch[kScrPlanes + (kScrXsum + kScrXscale) / 4];

// Device address of `scratch` per device (the array's name is only a host
// stand-in), looked up once per device with that device current.
std::mutex g_scr_mu;
void* g_scr_ptr[64] = {};

// q4_norm_gemv_argmax_dev's per-workgroup (value, index) parts and arrival
// counter: fixed arrays in device memory, kStreamSlots sets per GPU (zero at
// load; the last workgroup of each launch sets its counter back to zero).
static __device__ __align__(256) float2 greedy_part[kStreamSlots * kGreedyMaxParts];
static __device__ __align__(256) unsigned greedy_count[kStreamSlots * 64];   // counter [64 s]: a 256-byte line each
std::mutex g_greedy_mu;
void* g_greedy_part[64] = {};
void* g_greedy_count[64] = {};

int scratch_workspace(Workspace* ws) {
    int dev;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return fail(Q4_EARG, "device %d: the static scratch is kept for devices 0..63", dev);
    void* p;
    {
        std::lock_guard<std::mutex> lock(g_scr_mu);
        if (!g_scr_ptr[dev]) {
            void* a = nullptr;
            HIP_TRY(hipGetSymbolAddress(&a, HIP_SYMBOL(scratch)));
            if (!a) return fail(Q4_EHIP, "hipGetSymbolAddress(scratch) gave a null address");
            g_scr_ptr[dev] = a;
        }
        p = g_scr_ptr[dev];
    }
    uint4* base = static_cast<uint4*>(p);
    ws->fixed = true;
    ws->planes = base;
    ws->xsum = reinterpret_cast<float*>(base + kScrPlanes);
    ws->xscale = ws->xsum + kScrXsum;
    ws->cap[kWsPlanes] = kScrPlanes * sizeof(uint4);
    ws->cap[kWsXsum] = kScrXsum * sizeof(float);
    ws->cap[kWsXscale] = kScrXscale * sizeof(float);
    return 0;
}

// The prefill GEMM's plan: data-parallel tiles of height bm (256 or 128)
// with K split S ways (S > 1: partial planes and a sum launch), or, when
// sk_p > 0, stream-K over sk_p workgroups of 256 x 256 tiles.
struct PrefillPlan {
    int bm = 256, S = 1, sk_p = 0, sk_nx = 1;
};

// XCD groups of a stream-K launch of P workgroups over `tiles` tiles: one per
// XCD when P spreads evenly over 8 of them and there are tiles for each.
int sk_groups(int P, long tiles) { return P % 8 == 0 && tiles >= 8 ? 8 : 1; }

bool sk_ok(int P, long tiles, long T, int cus) {
    const int nx = sk_groups(P, tiles);
    return P >= 1 && P <= cus && P <= T && P / nx >= (tiles + nx - 1) / nx;
}

// From a cost model of the kernels measured at M = 512: a K step of a
// 256 x 256 tile takes about 2.3 us, of a 128 x 256 tile 2.0 us, plus about
// two steps of pipeline fill per workgroup; data-parallel workgroups run in
// rounds of one per CU, and split partials cost a write and a read of
// M x N floats each (about 4.5 TB/s) plus the sum launch.  Stream-K keeps
// every CU busy, where a step takes about 2.7 us (the clock drops), and a
// tile's owner adds one 256 KiB partial per range before it in the tile
// (about 5 us each, serially), plus about 20 us of partial stores, restarts
// and imbalance: it wins only where each tile has one or two ranges
// (gate/up of a 512-token prompt: 124 us against 132 us).
// Q4_GEMM_PLAN="dp:<bm>:<S>" or "sk:<P>" sets the plan instead (for tests
// and measurement).
// nblocks: 256-column blocks of the launch; ncols: its columns.
int plan_prefill(int m, int nblocks, int ncols, int n_in, PrefillPlan* out) {
    const int cus = num_cus();
    const int G = n_in / 64;
    const long tiles256 = static_cast<long>((m + 255) / 256) * nblocks;
    const long T = tiles256 * G;
    auto splits_ok = [&](int S) { return S >= 1 && S <= G && (G + (G + S - 1) / S - 1) / ((G + S - 1) / S) == S; };
    if (const char* env = getenv("Q4_GEMM_PLAN")) {
        PrefillPlan p;
        char tail = 0;
        if (sscanf(env, "sk:%d%c", &p.sk_p, &tail) == 1) {
            if (!sk_ok(p.sk_p, tiles256, T, cus))
                return fail(Q4_EARG, "Q4_GEMM_PLAN=%s: P must lie in [%ld, %ld] here, with P / 8 >= %ld when P is "
                            "a multiple of 8", env, tiles256, std::min<long>(cus, T), (tiles256 + 7) / 8);
            p.sk_nx = sk_groups(p.sk_p, tiles256);
        } else if (sscanf(env, "dp:%d:%d%c", &p.bm, &p.S, &tail) == 2) {
            if ((p.bm != 256 && p.bm != 128) || !splits_ok(p.S))
                return fail(Q4_EARG, "Q4_GEMM_PLAN=%s: bm is 128 or 256, and S splits of %d K steps must all be "
                                     "non-empty", env, G);
        } else {
            return fail(Q4_EARG, "Q4_GEMM_PLAN=%s: expected dp:<bm>:<S> or sk:<P>", env);
        }
        *out = p;
        return 0;
    }
    PrefillPlan best_plan;
    double best = 1e30;
    for (int bm : {256, 128}) {
        const long tiles = static_cast<long>((m + bm - 1) / bm) * nblocks;
        const double t_step = bm == 256 ? 2.3 : 2.0;
        for (int S = 1; S <= 16 && G / S >= 2; S++) {
            if (!splits_ok(S)) continue;
            const int kts = (G + S - 1) / S;
            const long rounds = (tiles * S + cus - 1) / cus;
            const double est = static_cast<double>(rounds) * (kts + 2) * t_step +
                               (S > 1 ? static_cast<double>(S) * m * ncols * 8.0 / 4.5e6 + 3.0 : 0.0);
            if (est < best) {
                best = est;
                best_plan = PrefillPlan{bm, S, 0};
            }
        }
    }
    for (int P = 8; P <= cus; P += 8) {
        if (!sk_ok(P, tiles256, T, cus) || sk_groups(P, tiles256) != 8) continue;
        const long Tg = (tiles256 + 7) / 8 * G, Pg = P / 8;
        const long L = (Tg + Pg - 1) / Pg, Lmin = Tg / Pg;
        const long partials = (G + Lmin - 1) / Lmin - 1;            // per owner, at most
        const double est = static_cast<double>(L + 4) * 2.7 + static_cast<double>(partials) * 5.0 + 20.0;
        if (est < best) {
            best = est;
            best_plan = PrefillPlan{256, 1, P, 8};
        }
    }
    *out = best_plan;
    return 0;
}

}  // namespace

// ================================================================ C-ABI ====

#pragma GCC visibility push(default)
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
    // own resident matrix, keyed by the block's first-row addresses and
    // tagged with the matrix base w, which q4_release(w) matches; a block
    // that is the whole matrix shares q4_gemv's entry.
    const size_t wpr = static_cast<size_t>(n_in / 8), ng = static_cast<size_t>(n_in / gs);
    Resident* r;
    if ((rc = resident(w + row0 * wpr, scales + row0 * ng, biases + row0 * ng, rows, n_in, gs, dev, &r, w)))
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
        if (std::get<1>(it->first) == w || it->second.base == w) {
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

int q4_set_rows(int rows) {
    if (rows < 1 || rows > kMaxRowsBlock) return fail(Q4_EARG, "rows=%d: expected [1, %d]", rows, kMaxRowsBlock);
    int prev = 1;
    if (rows_block(&prev)) prev = 1;                 // an unreadable HETERO_Q4_ROWS is replaced
    g_rows.store(rows, std::memory_order_relaxed);
    return prev;
}

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

int q4_gemv_noalloc_dev(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, const float* x,
                        float* out, int m, int n_out, int n_in, int gs, void* stream) {
    int rc = check_gemv_shape(n_out, n_in, gs);
    if (rc) return rc;
    if (m < 0) return fail(Q4_EARG, "m=%d", m);
    if (n_in > kNoAllocMaxIn)
        return fail(Q4_EARG, "q4_gemv_noalloc_dev takes n_in <= %d (got %d): its scratch is fixed", kNoAllocMaxIn,
                    n_in);
    if (n_out == 0 || m == 0) return 0;
    if (!w || !scales || !biases || !x || !out) return fail(Q4_EARG, "null pointer");
    if (reinterpret_cast<uintptr_t>(w) & 15) return fail(Q4_EARG, "w must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    Workspace ws;
    if ((rc = scratch_workspace(&ws))) return rc;
    for (int m0 = 0; m0 < m; m0 += kMaxM) {
        const int mm = m - m0 < kMaxM ? m - m0 : kMaxM;
        rc = gemv_rows(w, scales, biases, x + static_cast<size_t>(m0) * n_in,
                       out + static_cast<size_t>(m0) * n_out, mm, n_out, n_in, gs, st, ws);
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
    if (m < kMfMinRows) {  // one grouped streaming launch; more rows: a matrix-core launch per matrix
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
        if (rc == 1) return multi_tails(count, w, scales, biases, out, n_out, x, m, n_in, gs, st);
    }
    // 3..8 rows on the matrix cores: x prepared once for every matrix
    bool all_mf = m <= kMaxM, any = false;
    for (int k = 0; k < count && all_mf; k++) {
        all_mf = n_out[k] == 0 || mfma_takes(m, n_out[k], n_in, gs, x);
        any = any || n_out[k] > 0;
    }
    if (all_mf && any) {
        Workspace* ws;
        {
            std::lock_guard<std::mutex> lock(g_mu);
            int dev;
            if ((rc = current_device(&dev))) return rc;
            ws = &g_dev[dev].ws[st];
        }
        if ((rc = mfma_prep(x, m, n_in, st, *ws))) return rc;
        for (int k = 0; k < count; k++) {
            if (n_out[k] == 0) continue;
            const q4k::MfMats mt{{w[k], w[k]}, {scales[k], scales[k]}, {biases[k], biases[k]}};
            if ((rc = mfma_main(mt, false, out[k], m, n_out[k], n_in, st, *ws)) < 0) return rc;
        }
        return multi_tails(count, w, scales, biases, out, n_out, x, m, n_in, gs, st);
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
    for (int m0 = 0; m0 < m; m0 += kMaxM) {
        const int mm = m - m0 < kMaxM ? m - m0 : kMaxM;
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
        ml.mrows = mm;
        int done = 0;
        if (mm >= kMfMinRows) {
            Workspace* ws;
            {
                std::lock_guard<std::mutex> lock(g_mu);
                int dev;
                if ((rc = current_device(&dev))) return rc;
                ws = &g_dev[dev].ws[st];
            }
            const q4k::MfMats mt{{gate_w, up_w}, {gate_s, up_s}, {gate_b, up_b}};
            done = gemv_mfma(mt, true, xm, hm, mm, n_inter, n_in, gs, st, *ws);
            if (done < 0) return done;
        }
        if (!done && mm <= 2 && stream_takes(xm, n_in, gs)) {
            done = mm == 1 ? launch_stream_gs<1, true>(ml, xm, n_in, gs, st)
                           : launch_stream_gs<2, true>(ml, xm, n_in, gs, st);
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

int q4_norm_gemv_multi_dev(int count, const uint32_t* const* w, const uint16_t* const* scales,
                           const uint16_t* const* biases, float* const* out, const int* n_out, const float* x,
                           const float* delta, const float* norm_w, float eps, float* x_out, int n_in, int gs,
                           void* stream) {
    if (count < 1 || count > kMaxMats || !w || !scales || !biases || !out || !n_out)
        return fail(Q4_EARG, "q4_norm_gemv_multi_dev: count=%d (1..%d) or null array", count, kMaxMats);
    int rc;
    for (int k = 0; k < count; k++) {
        if ((rc = check_gemv_shape(n_out[k], n_in, gs))) return rc;
        if (!w[k] || !scales[k] || !biases[k] || !out[k]) return fail(Q4_EARG, "null pointer in matrix %d", k);
        if (reinterpret_cast<uintptr_t>(w[k]) & 15) return fail(Q4_EARG, "w[%d] must be 16-byte aligned", k);
    }
    if ((rc = check_norm_args("q4_norm_gemv_multi_dev", x, delta, norm_w, x_out, n_in, gs))) return rc;
    MatList ml{};
    ml.row_begin[0] = 0;
    for (int k = 0; k < kMaxMats; k++) {
        const int kk = k < count ? k : count - 1;
        ml.w[k] = w[kk]; ml.s[k] = scales[kk]; ml.b[k] = biases[kk]; ml.out[k] = out[kk];
        ml.n_out[k] = k < count ? n_out[k] : 0;
        ml.row_begin[k + 1] = ml.row_begin[k] + ml.n_out[k];
    }
    ml.count = count;
    ml.mrows = 1;
    if (ml.row_begin[count] == 0) return fail(Q4_EARG, "q4_norm_gemv_multi_dev: no output rows");
    const NormArgs na{delta, norm_w, x_out, eps};
    rc = launch_stream<1, false, true>(ml, x, n_in, static_cast<hipStream_t>(stream), na);
    if (rc == 0) return fail(Q4_EARG, "q4_norm_gemv_multi_dev: n_in = %d does not fit the norm prologue", n_in);
    return rc < 0 ? rc : 0;
}

int q4_norm_gemv_argmax_dev(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, float* logits,
                            int n_out, const float* x, const float* delta, const float* norm_w, float eps,
                            float* x_out, int n_in, int gs, int64_t* tok, int64_t* hist, int64_t* pos, int64_t s0,
                            int hist_len, void* stream) {
    int rc = check_gemv_shape(n_out, n_in, gs);
    if (rc) return rc;
    if (n_out == 0) return fail(Q4_EARG, "q4_norm_gemv_argmax_dev: no output rows");
    if (!w || !scales || !biases || !logits || !tok || !pos || (hist_len > 0 && !hist))
        return fail(Q4_EARG, "q4_norm_gemv_argmax_dev: null pointer");
    if (reinterpret_cast<uintptr_t>(w) & 15) return fail(Q4_EARG, "w must be 16-byte aligned");
    if ((rc = check_norm_args("q4_norm_gemv_argmax_dev", x, delta, norm_w, x_out, n_in, gs))) return rc;
    int dev;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return fail(Q4_EARG, "device %d: the greedy-token arrays are kept for devices 0..63", dev);
    void *part, *count;
    {
        std::lock_guard<std::mutex> lock(g_greedy_mu);
        if (!g_greedy_part[dev]) {
            void *a = nullptr, *b = nullptr;
            HIP_TRY(hipGetSymbolAddress(&a, HIP_SYMBOL(greedy_part)));
            HIP_TRY(hipGetSymbolAddress(&b, HIP_SYMBOL(greedy_count)));
            if (!a || !b) return fail(Q4_EHIP, "hipGetSymbolAddress(greedy arrays) gave a null address");
            g_greedy_part[dev] = a;
            g_greedy_count[dev] = b;
        }
        part = g_greedy_part[dev];
        count = g_greedy_count[dev];
    }
    int slot = 0;
    if ((rc = stream_slot(static_cast<hipStream_t>(stream), &slot))) return rc;
    part = static_cast<float2*>(part) + static_cast<size_t>(slot) * kGreedyMaxParts;
    count = static_cast<unsigned*>(count) + static_cast<size_t>(slot) * 64;
    MatList ml{};
    for (int k = 0; k < kMaxMats; k++) {
        ml.w[k] = w; ml.s[k] = scales; ml.b[k] = biases; ml.out[k] = logits;
        ml.n_out[k] = k == 0 ? n_out : 0;
    }
    ml.row_begin[0] = 0;
    for (int k = 0; k < kMaxMats; k++) ml.row_begin[k + 1] = ml.row_begin[k] + ml.n_out[k];
    ml.count = 1;
    ml.mrows = 1;
    NormArgs na{delta, norm_w, x_out, eps};
    na.greedy = GreedyArgs{static_cast<float2*>(part), static_cast<unsigned*>(count), tok, hist, pos, s0,
                           hist_len > 0 ? hist_len : 0};
    rc = launch_stream<1, false, true>(ml, x, n_in, static_cast<hipStream_t>(stream), na);
    if (rc == 0) return fail(Q4_EARG, "q4_norm_gemv_argmax_dev: n_in = %d does not fit the norm prologue", n_in);
    return rc < 0 ? rc : 0;
}

int q4_norm_gate_up_silu_dev(const uint32_t* gate_w, const uint16_t* gate_s, const uint16_t* gate_b,
                             const uint32_t* up_w, const uint16_t* up_s, const uint16_t* up_b, const float* x,
                             const float* delta, const float* norm_w, float eps, float* x_out, float* h,
                             int n_inter, int n_in, int gs, void* stream) {
    int rc = check_gemv_shape(n_inter, n_in, gs);
    if (rc) return rc;
    if (n_inter == 0) return fail(Q4_EARG, "q4_norm_gate_up_silu_dev: no output rows");
    if (!gate_w || !gate_s || !gate_b || !up_w || !up_s || !up_b || !h)
        return fail(Q4_EARG, "q4_norm_gate_up_silu_dev: null pointer");
    if ((reinterpret_cast<uintptr_t>(gate_w) | reinterpret_cast<uintptr_t>(up_w)) & 15)
        return fail(Q4_EARG, "w must be 16-byte aligned");
    if ((rc = check_norm_args("q4_norm_gate_up_silu_dev", x, delta, norm_w, x_out, n_in, gs))) return rc;
    MatList ml{};
    ml.w[0] = gate_w; ml.s[0] = gate_s; ml.b[0] = gate_b; ml.out[0] = h; ml.n_out[0] = n_inter;
    ml.w[1] = up_w;   ml.s[1] = up_s;   ml.b[1] = up_b;   ml.out[1] = h; ml.n_out[1] = n_inter;
    for (int k = 2; k < kMaxMats; k++) {
        ml.w[k] = up_w; ml.s[k] = up_s; ml.b[k] = up_b; ml.out[k] = h; ml.n_out[k] = 0;
    }
    ml.row_begin[0] = 0;
    for (int k = 0; k < kMaxMats; k++) ml.row_begin[k + 1] = ml.row_begin[k] + ml.n_out[k];
    ml.count = 2;
    ml.mrows = 1;
    const NormArgs na{delta, norm_w, x_out, eps};
    rc = launch_stream<1, true, true>(ml, x, n_in, static_cast<hipStream_t>(stream), na);
    if (rc == 0) return fail(Q4_EARG, "q4_norm_gate_up_silu_dev: n_in = %d does not fit the norm prologue", n_in);
    return rc < 0 ? rc : 0;
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


}  // extern "C"

namespace {

// The calling stream's workspace on the current device.
int stream_workspace(hipStream_t st, Workspace** ws) {
    std::lock_guard<std::mutex> lock(g_mu);
    int dev;
    if (int rc = current_device(&dev)) return rc;
    *ws = &g_dev[dev].ws[st];
    return 0;
}

// Room for P stream-K partial slots (256 x 256 floats each) and the flags
// of up to one workgroup per CU, then the control words; flags and control
// words start at zero once, and every launch leaves them consistent (the
// epoch scheme of q4_gemm.hip).
int sk_workspace(Workspace& ws, int P, hipStream_t st) {
    int rc;
    const size_t flag_words = static_cast<size_t>(num_cus()) * 32 + kSkCtlWordsHost;
    if ((rc = grow(ws, ws.part, kWsPart, static_cast<size_t>(P) * 256 * 256 * 4, st, "prefill"))) return rc;
    const size_t cap_before = ws.cap[kWsSk];
    if ((rc = grow(ws, ws.sk, kWsSk, flag_words * 4, st, "prefill"))) return rc;
    if (ws.cap[kWsSk] != cap_before) {
        const long n = static_cast<long>(ws.cap[kWsSk] / 4);
        hipLaunchKernelGGL(fill_zero_kernel, dim3((n + 255) / 256), dim3(256), 0, st, reinterpret_cast<float*>(ws.sk),
                           n);
        HIP_TRY(hipGetLastError());
    }
    return 0;
}

// q4_gemm_bf16_multi_dev on x given in fp32 (x, rounded to bf16 into the
// workspace first) or already in bf16 (xb).
int gemm_bf16_multi(int count, const uint32_t* const* w, const uint16_t* const* scales,
                    const uint16_t* const* biases, float* const* out, const int* n_out, const float* x,
                    const uint16_t* xb_in, int m, int n_in, int gs, void* stream) {
    if (count < 1 || count > 4) return fail(Q4_EARG, "count=%d (1..4)", count);
    if (!w || !scales || !biases || !out || !n_out) return fail(Q4_EARG, "null array");
    int rc;
    for (int k = 0; k < count; k++)
        if ((rc = check_gemv_shape(n_out[k], n_in, gs))) return rc;
    if (gs != 64) return fail(Q4_EARG, "the prefill GEMM takes gs = 64 (got %d)", gs);
    if (m < 0) return fail(Q4_EARG, "m=%d", m);
    GemmMats gm{};
    int ncols = 0, nblocks = 0;
    for (int k = 0; k < count; k++) {
        if (n_out[k] == 0) continue;                          // a matrix of no rows takes no block
        gm.w[gm.count] = w[k];
        gm.s[gm.count] = scales[k];
        gm.b[gm.count] = biases[k];
        gm.out[gm.count] = out[k];
        gm.n_out[gm.count] = n_out[k];
        gm.nb0[gm.count] = nblocks;
        gm.col0[gm.count] = ncols;
        nblocks += (n_out[k] + 255) / 256;
        ncols += n_out[k];
        ++gm.count;
    }
    gm.nb0[gm.count] = nblocks;
    if (m == 0 || gm.count == 0) return 0;
    for (int k = 0; k < gm.count; k++) {
        if (!gm.w[k] || !gm.s[k] || !gm.b[k] || !gm.out[k]) return fail(Q4_EARG, "null pointer");
        if (reinterpret_cast<uintptr_t>(gm.w[k]) & 15) return fail(Q4_EARG, "w and x must be 16-byte aligned");
    }
    const void* xin = xb_in ? static_cast<const void*>(xb_in) : static_cast<const void*>(x);
    if (!xin || (reinterpret_cast<uintptr_t>(xin) & 15)) return fail(Q4_EARG, "w and x must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (n_in == 0) {
        for (int k = 0; k < gm.count; k++) {
            const long n = static_cast<long>(m) * gm.n_out[k];
            hipLaunchKernelGGL(fill_zero_kernel, dim3((n + 255) / 256), dim3(256), 0, st, gm.out[k], n);
            HIP_TRY(hipGetLastError());
        }
        return 0;
    }
    Workspace* ws;
    if ((rc = stream_workspace(st, &ws))) return rc;
    PrefillPlan plan;
    if ((rc = plan_prefill(m, nblocks, ncols, n_in, &plan))) return rc;
    const size_t mk = static_cast<size_t>(m) * n_in, mn = static_cast<size_t>(m) * ncols;
    if (!xb_in && (rc = grow(*ws, ws->xbf, kWsXbf, mk * 2, st, "prefill"))) return rc;
    if (plan.sk_p > 0) {
        if ((rc = sk_workspace(*ws, plan.sk_p, st))) return rc;
    } else if (plan.S > 1 && (rc = grow(*ws, ws->part, kWsPart, plan.S * mn * 4, st, "prefill"))) {
        return rc;
    }
    const uint16_t* xb = xb_in;
    if (!xb) {
        const long n8 = static_cast<long>(mk / 8);
        hipLaunchKernelGGL(x_to_bf16_kernel, dim3(static_cast<unsigned>((n8 + 255) / 256)), dim3(256), 0, st, x,
                           static_cast<uint4*>(ws->xbf), n8);
        HIP_TRY(hipGetLastError());
        xb = static_cast<const uint16_t*>(ws->xbf);
    }
    if (plan.sk_p > 0) {
        return gemm_w4_sk(xb, gm, static_cast<float*>(ws->part), ws->sk, sk_ctl(*ws), m, n_in, plan.sk_p,
                          plan.sk_nx, st);
    }
    const int S = plan.S, kt_split = (n_in / 64 + S - 1) / S;
    float* part = S > 1 ? static_cast<float*>(ws->part) : nullptr;
    if ((rc = gemm_w4(xb, gm, part, m, n_in, plan.bm, S, kt_split, ncols, st))) return rc;
    if (S == 1) return 0;
    const long n = static_cast<long>(mn);
    hipLaunchKernelGGL(splitk_sum_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st,
                       static_cast<const float*>(ws->part), gm, m, ncols, S);
    HIP_TRY(hipGetLastError());
    return 0;
}

}  // namespace

extern "C" {

int q4_gemm_bf16_multi_dev(int count, const uint32_t* const* w, const uint16_t* const* scales,
                           const uint16_t* const* biases, float* const* out, const int* n_out, const float* x,
                           int m, int n_in, int gs, void* stream) {
    return gemm_bf16_multi(count, w, scales, biases, out, n_out, x, nullptr, m, n_in, gs, stream);
}

int q4_gemm_bf16in_multi_dev(int count, const uint32_t* const* w, const uint16_t* const* scales,
                             const uint16_t* const* biases, float* const* out, const int* n_out, const uint16_t* xb,
                             int m, int n_in, int gs, void* stream) {
    return gemm_bf16_multi(count, w, scales, biases, out, n_out, nullptr, xb, m, n_in, gs, stream);
}

int q4_gemm_bf16in_gate_up_silu_dev(const uint32_t* gate_w, const uint16_t* gate_s, const uint16_t* gate_b,
                                    const uint32_t* up_w, const uint16_t* up_s, const uint16_t* up_b,
                                    const uint16_t* xb, uint16_t* h, int m, int n_inter, int n_in, int gs,
                                    void* stream) {
    int rc = check_gemv_shape(n_inter, n_in, gs);
    if (rc) return rc;
    if (gs != 64) return fail(Q4_EARG, "the prefill GEMM takes gs = 64 (got %d)", gs);
    if (m < 0) return fail(Q4_EARG, "m=%d", m);
    if (!gate_w || !gate_s || !gate_b || !up_w || !up_s || !up_b || !xb || !h)
        return fail(Q4_EARG, "q4_gemm_bf16in_gate_up_silu_dev: null pointer");
    if ((reinterpret_cast<uintptr_t>(gate_w) & 15) || (reinterpret_cast<uintptr_t>(up_w) & 15) ||
        (reinterpret_cast<uintptr_t>(xb) & 15))
        return fail(Q4_EARG, "w and x must be 16-byte aligned");
    if (m == 0 || n_inter == 0) return 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (n_in == 0) {                                   // SiLU(0) * 0
        const long n = static_cast<long>(m) * n_inter;
        hipLaunchKernelGGL(fill_zero_u16_kernel, dim3((n + 255) / 256), dim3(256), 0, st, h, n);
        HIP_TRY(hipGetLastError());
        return 0;
    }
    GemmMats gm{};
    gm.w[0] = gate_w;
    gm.s[0] = gate_s;
    gm.b[0] = gate_b;
    gm.w[1] = up_w;
    gm.s[1] = up_s;
    gm.b[1] = up_b;
    gm.n_out[0] = gm.n_out[1] = n_inter;
    gm.count = 2;
    // one 256 x (128 + 128) tile per workgroup while the tiles fit the CUs
    // in one round; past that, stream-K over one workgroup per CU, so that
    // a last partial round does not double the time (Q4_PAIR_PLAN=dp or
    // sk:<P> chooses)
    const int cus = num_cus();
    const long tiles = static_cast<long>((m + 255) / 256) * ((n_inter + 127) / 128);
    const long T = tiles * (n_in / 64);
    int P = tiles > cus ? static_cast<int>(std::min<long>(cus >= 8 ? cus / 8 * 8 : cus, T)) : 0;
    if (const char* env = getenv("Q4_PAIR_PLAN")) {
        char tail = 0;
        int p = 0;
        if (std::strcmp(env, "dp") == 0) P = 0;
        else if (sscanf(env, "sk:%d%c", &p, &tail) == 1 && p >= 1 && p <= cus && p <= T) P = p;
        else return fail(Q4_EARG, "Q4_PAIR_PLAN=%s: expected dp or sk:<P> with P in [1, %ld]", env,
                         std::min<long>(cus, T));
    }
    if (P == 0) return gemm_w4_pair(xb, gm, h, m, n_in, st);
    Workspace* ws;
    if ((rc = stream_workspace(st, &ws))) return rc;
    if ((rc = sk_workspace(*ws, P, st))) return rc;
    return gemm_w4_sk_pair(xb, gm, static_cast<float*>(ws->part), ws->sk, sk_ctl(*ws), h, m, n_in, P,
                           sk_groups(P, tiles), st);
}

int q4_gemm_bf16_dev(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                     const float* x, float* out, int m, int n_out, int n_in, int gs, void* stream) {
    return q4_gemm_bf16_multi_dev(1, &w, &scales, &biases, &out, &n_out, x, m, n_in, gs, stream);
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

int q4_prefill_errors(void* stream) {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    unsigned* ctl = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        int dev;
        if (int rc = current_device(&dev)) return rc;
        auto d = g_dev.find(dev);
        if (d == g_dev.end()) return 0;
        auto w = d->second.ws.find(st);
        if (w == d->second.ws.end() || !w->second.sk) return 0;
        ctl = sk_ctl(w->second);
    }
    HIP_TRY(hipStreamSynchronize(st));
    unsigned n = 0;
    HIP_TRY(hipMemcpy(&n, ctl + kSkCtlErrorsHost, sizeof(n), hipMemcpyDeviceToHost));
    if (n) {
        const unsigned zero = 0;
        HIP_TRY(hipMemcpy(ctl + kSkCtlErrorsHost, &zero, sizeof(zero), hipMemcpyHostToDevice));
    }
    return static_cast<int>(n);
}

}  // extern "C"
#pragma GCC visibility pop
