// Prefill GEMM on the matrix cores with the 4-bit weights kept 4-bit up to
// the MFMA: out[M][N] = bf16(x)[M][K] . bf16(dequant W)[N][K]^T, fp32
// accumulation on v_mfma_f32_32x32x16_bf16.
//
// Workgroup tile BM x 256 (BM 256 or 128), NW waves in 2 x NW/2, each wave
// (BM/2) x (512/NW) -- TM x TN MFMA tiles of 32 x 32.  One K step is 64 = one
// quantisation group, so each weight row has one scale/bias pair per step.
// Every operand reaches LDS by global->LDS copies (buffer_load ... lds, 16 or
// 2 bytes a lane), into a ring of three stages, each holding one K step:
//   * A: the bf16 copy of x, BM rows x 128 bytes, 16-byte chunk c of row r
//     at r * 128 + (c ^ (r & 7)) * 16 (the XOR spreads a fragment read by 32
//     rows over the banks);
//   * B: the packed weights as they are in memory, 256 rows x 8 words;
//   * the 256 rows' scales, then their biases, a zero-extended word each.
// B is dequantised in registers right before the MFMA that consumes it:
// one packed word (word 2 ks + lane/32 of the row) is exactly one lane's
// 8-value B fragment of K slice ks, and its value is bf16(fma(q, scale,
// bias)) -- what q4_dequant_bf16_dev writes.  Staging B 4-bit keeps its LDS
// traffic a quarter of bf16's, and a dequantised word feeds TM MFMAs.
// Pipeline: step k + 2's copies are issued while step k is multiplied; at
// the top of a step each wave waits for its own copies of the step (the
// next step's stay in flight) and one barrier publishes everyone's.
// Every copy goes through a buffer resource bounded to the tile's rows:
// rows past M or N and steps past the workgroup's K range read 0 and cost
// no access.  Split-K: blockIdx.z takes steps [z kt_split, (z+1) kt_split)
// and writes its partial sums to out + z M ldo.
#include "q4_common.h"

namespace q4k {

typedef __bf16 gemm_bf16x8 __attribute__((ext_vector_type(8)));
typedef float gemm_f32x16 __attribute__((ext_vector_type(16)));

// One stage of the LDS ring: A (BM rows x 128 bytes), B (256 rows x 32
// bytes), then the 256 rows' scales and biases (a word each).
__host__ __device__ constexpr int w4_stage_bytes(int bm) { return bm * 128 + 8192 + 2048; }

__device__ __forceinline__ uint32_t w4_pack_bf16(float a, float b) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
    const f32x2 p = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(p, bf16x2v));
}

// The 8 values of one packed word (element e in bits 4e..4e+3), each
// bf16(fma(q_e, s, b)), in element order.
__device__ __forceinline__ gemm_bf16x8 w4_dequant8(uint32_t w, float s, float b) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;   // even / odd elements, a byte each
    float v[8];
#pragma unroll
    for (int n = 0; n < 4; n++) {
        v[2 * n] = __builtin_fmaf(static_cast<float>((lo >> (8 * n)) & 0xFFu), s, b);
        v[2 * n + 1] = __builtin_fmaf(static_cast<float>((hi >> (8 * n)) & 0xFFu), s, b);
    }
    const uint4 p = make_uint4(w4_pack_bf16(v[0], v[1]), w4_pack_bf16(v[2], v[3]), w4_pack_bf16(v[4], v[5]),
                               w4_pack_bf16(v[6], v[7]));
    return __builtin_bit_cast(gemm_bf16x8, p);
}

// The copies of one K step (kt) into a stage of the LDS ring (a plain device
// function: the copy builtin in a lambda of the kernel keeps the compiler
// from emitting the kernel's host stub).  NW waves share them: A in 1 KiB
// copies of 8 rows, B in 8 copies of 32 rows, the 256 scales and biases in
// 4 copies of 64 rows each.  `live` false (a step past the workgroup's K
// range) reads zeros without an access.
template <int BM, int NW>
__device__ __forceinline__ void w4_issue(char* st, __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t wr,
                                         __amdgpu_buffer_rsrc_t sr, __amdgpu_buffer_rsrc_t br,
                                         const uint32_t* a_src, const uint32_t* b_src,
                                         uint32_t g_src, int kt, bool live, int wave) {
    typedef __attribute__((address_space(3))) void* lds_ptr;
    constexpr int A_DMA = BM / (8 * NW), B_DMA = 8 / NW;
    const uint32_t dead = __builtin_amdgcn_readfirstlane(live ? 0u : kOutOfRange);
#pragma unroll
    for (int i = 0; i < A_DMA; i++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_ptr)(st + (wave * A_DMA + i) * 1024), 16,
                                                 a_src[i] + static_cast<uint32_t>(kt) * 128u + dead, 0, 0, 0);
#pragma unroll
    for (int q = 0; q < B_DMA; q++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_ptr)(st + BM * 128 + (B_DMA * wave + q) * 1024), 16,
                                                 b_src[q] + static_cast<uint32_t>(kt) * 32u + dead, 0, 0, 2);
    const uint32_t go = g_src + static_cast<uint32_t>(kt) * 2u + dead;
    if constexpr (NW == 4) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_ptr)(st + BM * 128 + 8192 + wave * 256), 2, go, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(br, (lds_ptr)(st + BM * 128 + 9216 + wave * 256), 2, go, 0, 0, 0);
    } else {                                                       // waves 0-3 scales, 4-7 biases
        if (wave < 4)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_ptr)(st + BM * 128 + 8192 + wave * 256), 2, go, 0, 0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(br, (lds_ptr)(st + BM * 128 + 9216 + (wave - 4) * 256), 2, go, 0,
                                                     0, 0);
    }
}

// NW waves as 2 x NW/2: each wave (BM/2) x (512/NW) columns.
template <int BM, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_w4_kernel(const uint16_t* __restrict__ xb, const uint32_t* __restrict__ w,
                                                          const uint16_t* __restrict__ sc,
                                                          const uint16_t* __restrict__ bi, float* __restrict__ out,
                                                          int M, int N, int K, int kt_split, int nb0, int ldo) {
    constexpr int BN = 256, WN = NW / 2, WC = BN / WN;             // waves along N, columns per wave
    constexpr int TM = BM / 64, TN = WC / 32;                      // 32 x 32 tiles per wave
    constexpr int A_DMA = BM / (8 * NW), B_DMA = 8 / NW;
    constexpr int PER_STEP = A_DMA + B_DMA + (NW == 4 ? 2 : 1);    // copies per wave and step
    constexpr int STAGE = w4_stage_bytes(BM);
    extern __shared__ uint4 w4_lds[];
    char* lds = reinterpret_cast<char*>(w4_lds);
    const int tid = threadIdx.x, lane = tid & 63, hb = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.x * BM, n0 = (blockIdx.y + nb0) * BN;
    const int G = K >> 6, wpr = K >> 3;
    const int kt0 = blockIdx.z * kt_split;
    const int nk = G - kt0 < kt_split ? G - kt0 : kt_split;
    const int mrows = M - m0 < BM ? M - m0 : BM, nrows = N - n0 < BN ? N - n0 : BN;
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(xb + static_cast<size_t>(m0) * K, static_cast<uint32_t>(mrows * K) * 2u);
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(w + static_cast<size_t>(n0) * wpr, static_cast<uint32_t>(nrows * wpr) * 4u);
    const __amdgpu_buffer_rsrc_t sr = buf_rsrc(sc + static_cast<size_t>(n0) * G, static_cast<uint32_t>(nrows * G) * 2u);
    const __amdgpu_buffer_rsrc_t br = buf_rsrc(bi + static_cast<size_t>(n0) * G, static_cast<uint32_t>(nrows * G) * 2u);

    // per-lane source offsets of the step's copies (step kt adds kt * 128,
    // kt * 32 and kt * 2 bytes).  A: copy i of wave w moves rows
    // 8 (w A_DMA + i) .. + 8, lane -> (row, 16-byte chunk c), reading chunk
    // c ^ (row & 7) of the row: the stage holds row r's chunk c at
    // r * 128 + (c ^ (r & 7)) * 16.  B: copy q moves rows 32 (B_DMA w + q) ..
    // + 32, two lanes per row.  Scales / biases: one row per lane, a
    // zero-extended word each.
    uint32_t a_src[A_DMA];
#pragma unroll
    for (int i = 0; i < A_DMA; i++) {
        const int r = (wave * A_DMA + i) * 8 + (lane >> 3), c = lane & 7;
        a_src[i] = static_cast<uint32_t>(r * K + (c ^ (r & 7)) * 8) * 2u;
    }
    uint32_t b_src[B_DMA];
#pragma unroll
    for (int q = 0; q < B_DMA; q++) {
        const int r = (B_DMA * wave + q) * 32 + (lane >> 1);
        b_src[q] = static_cast<uint32_t>(r * wpr + (lane & 1) * 4) * 4u;
    }
    const uint32_t g_src = static_cast<uint32_t>(((NW == 4 ? wave : wave & 3) * 64 + lane) * G) * 2u;

    gemm_f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;

    w4_issue<BM, NW>(lds, xr, wr, sr, br, a_src, b_src, g_src, kt0, 0 < nk, wave);
    w4_issue<BM, NW>(lds + STAGE, xr, wr, sr, br, a_src, b_src, g_src, kt0 + 1, 1 < nk, wave);
    for (int it = 0; it < nk; it++) {
        // step it's copies are done (only step it + 1's may be in flight)
        __builtin_amdgcn_s_waitcnt(0x0F70 | PER_STEP);
        // a bare barrier: every wave's copies of step it are in LDS and every
        // wave is past step it - 1, whose stage step it + 2 refills (a fence
        // would also wait for the copies of step it + 1)
        __builtin_amdgcn_s_barrier();
        w4_issue<BM, NW>(lds + ((it + 2) % 3) * STAGE, xr, wr, sr, br, a_src, b_src, g_src, kt0 + it + 2, it + 2 < nk,
                         wave);
        const char* st = lds + (it % 3) * STAGE;
        const uint16_t* As = reinterpret_cast<const uint16_t*>(st);
        const uint32_t* Bs = reinterpret_cast<const uint32_t*>(st + BM * 128);
        const uint32_t* Ss = reinterpret_cast<const uint32_t*>(st + BM * 128 + 8192);
        const uint32_t* Ts = reinterpret_cast<const uint32_t*>(st + BM * 128 + 9216);
        float sf[TN], bf[TN];
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int row = wn * WC + j * 32 + (lane & 31);
            sf[j] = h2f(static_cast<uint16_t>(Ss[row]));
            bf[j] = h2f(static_cast<uint16_t>(Ts[row]));
        }
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            gemm_bf16x8 av[TM], bv[TN];
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int row = wn * WC + j * 32 + (lane & 31);
                bv[j] = w4_dequant8(Bs[row * 8 + 2 * ks + hb], sf[j], bf[j]);
            }
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int row = wm * (BM / 2) + i * 32 + (lane & 31);
                const int c = (2 * ks + hb) ^ (row & 7);
                av[i] = *reinterpret_cast<const gemm_bf16x8*>(As + row * 64 + c * 8);
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
    }
    // C tile: lane l, register v holds row 8 (v / 4) + 4 (l / 32) + v % 4,
    // column l % 32.  out: this split's [M][ldo] block, whose column 0 is
    // column nb0 * BN of the product
    float* o = out + static_cast<size_t>(blockIdx.z) * M * ldo;
    const int c0 = nb0 * BN;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = m0 + wm * (BM / 2) + i * 32 + 8 * (v >> 2) + 4 * hb + (v & 3);
                const int col = n0 + wn * WC + j * 32 + (lane & 31);
                if (row < M && col < N) o[static_cast<size_t>(row) * ldo + (col - c0)] = acc[i][j][v];
            }
    // the last copies issued (past the K range) read nothing; wait for them
    // before the workgroup's LDS is released
    __builtin_amdgcn_s_waitcnt(0x0F70);
}

template <int BM, int NW>
size_t w4_lds_bytes() {
    return static_cast<size_t>(3) * w4_stage_bytes(BM);
}

template <int BM, int NW>
int launch_w4(const uint16_t* xb, const uint32_t* w, const uint16_t* s, const uint16_t* b, float* out, int M, int N,
              int K, int S, int kt_split, int nb0, int nblocks, int ldo, hipStream_t st) {
    auto kern = gemm_w4_kernel<BM, NW>;
    const size_t lds = w4_lds_bytes<BM, NW>();
    static std::atomic<uint64_t> lds_raised{0};
    if (int rc = raise_lds_limit(reinterpret_cast<const void*>(kern), lds, lds_raised)) return rc;
    hipLaunchKernelGGL(kern, dim3((M + BM - 1) / BM, nblocks, S), dim3(64 * NW), lds, st, xb, w, s, b, out, M, N, K,
                       kt_split, nb0, ldo);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q4_EHIP, "prefill gemm launch: %s", hipGetErrorString(e));
    return 0;
}

int gemm_w4(const uint16_t* xb, const uint32_t* w, const uint16_t* s, const uint16_t* b, float* out, int M, int N,
            int K, int bm, int S, int kt_split, int nb0, int nblocks, int ldo, hipStream_t st) {
    // 256-row tiles: 4 waves of 128 x 128 (a dequantised weight word feeds 4
    // MFMAs); 128-row tiles: 8 waves of 64 x 64
    return bm == 256 ? launch_w4<256, 4>(xb, w, s, b, out, M, N, K, S, kt_split, nb0, nblocks, ldo, st)
                     : launch_w4<128, 8>(xb, w, s, b, out, M, N, K, S, kt_split, nb0, nblocks, ldo, st);
}

}  // namespace q4k
