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
// Paired tiles (gate/up of the MLP): the tile's 256 weight rows are rows
// [n0, n0 + 128) of the gate matrix, then the same rows of the up matrix,
// and wave w's 64 columns are gate rows n0 + 32 w .. and the same up rows,
// so one lane holds gate and up of every output it writes: the epilogue
// stores bf16(SiLU(gate) * up), the down projection's bf16 operand.
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

// The operands of one tile (M block mt, N block nt): buffer resources over
// its rows of x, W, scales and biases.
struct W4Tile {
    __amdgpu_buffer_rsrc_t xr, wr, sr, br;
    __amdgpu_buffer_rsrc_t wr2, sr2, br2;    // paired tiles: the up matrix's rows
    int m0, n0;
};

// The copies of one K step (kt) into a stage of the LDS ring (a plain device
// function: the copy builtin in a lambda of the kernel keeps the compiler
// from emitting the kernel's host stub).  NW waves share them: A in 1 KiB
// copies of 8 rows, B in 8 copies of 32 rows, the 256 scales and biases in
// 4 copies of 64 rows each.  `live` false (a step past the workgroup's K
// range) reads zeros without an access.
template <int BM, int NW, bool PAIR>
__device__ __forceinline__ void w4_issue(char* st, const W4Tile& t, const uint32_t* a_src, const uint32_t* b_src,
                                         uint32_t g_src, int kt, bool live, int wave) {
    typedef __attribute__((address_space(3))) void* lds_ptr;
    constexpr int A_DMA = BM / (8 * NW), B_DMA = 8 / NW;
    static_assert(!PAIR || NW == 4, "paired tiles: waves 0-1 copy the gate rows, 2-3 the up rows");
    const uint32_t dead = __builtin_amdgcn_readfirstlane(live ? 0u : kOutOfRange);
    const __amdgpu_buffer_rsrc_t xr = t.xr;
    const __amdgpu_buffer_rsrc_t wr = PAIR && wave >= 2 ? t.wr2 : t.wr;     // wave-uniform choice
    const __amdgpu_buffer_rsrc_t sr = PAIR && wave >= 2 ? t.sr2 : t.sr;
    const __amdgpu_buffer_rsrc_t br = PAIR && wave >= 2 ? t.br2 : t.br;
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

template <int BM>
__device__ __forceinline__ W4Tile w4_tile(const uint16_t* xb, const uint32_t* w, const uint16_t* sc, const uint16_t* bi,
                                          int M, int N, int K, int mt, int nt) {
    constexpr int BN = 256;
    W4Tile t;
    t.m0 = mt * BM;
    t.n0 = nt * BN;
    const int G = K >> 6, wpr = K >> 3;
    const int mrows = M - t.m0 < BM ? M - t.m0 : BM, nrows = N - t.n0 < BN ? N - t.n0 : BN;
    t.xr = buf_rsrc(xb + static_cast<size_t>(t.m0) * K, static_cast<uint32_t>(mrows * K) * 2u);
    t.wr = buf_rsrc(w + static_cast<size_t>(t.n0) * wpr, static_cast<uint32_t>(nrows * wpr) * 4u);
    t.sr = buf_rsrc(sc + static_cast<size_t>(t.n0) * G, static_cast<uint32_t>(nrows * G) * 2u);
    t.br = buf_rsrc(bi + static_cast<size_t>(t.n0) * G, static_cast<uint32_t>(nrows * G) * 2u);
    t.wr2 = t.wr;
    t.sr2 = t.sr;
    t.br2 = t.br;
    return t;
}

// A paired tile: output columns [nt 128, nt 128 + 128) of N, weight rows of
// matrix 0 (gate) and matrix 1 (up) of gm.
template <int BM>
__device__ __forceinline__ W4Tile w4_tile_pair(const uint16_t* xb, const GemmMats& gm, int M, int N, int K, int mt,
                                               int nt) {
    W4Tile t;
    t.m0 = mt * BM;
    t.n0 = nt * 128;
    const int G = K >> 6, wpr = K >> 3;
    const int mrows = M - t.m0 < BM ? M - t.m0 : BM, nrows = N - t.n0 < 128 ? N - t.n0 : 128;
    const size_t wo = static_cast<size_t>(t.n0) * wpr, go = static_cast<size_t>(t.n0) * G;
    const uint32_t wb = static_cast<uint32_t>(nrows * wpr) * 4u, gb = static_cast<uint32_t>(nrows * G) * 2u;
    t.xr = buf_rsrc(xb + static_cast<size_t>(t.m0) * K, static_cast<uint32_t>(mrows * K) * 2u);
    t.wr = buf_rsrc(gm.w[0] + wo, wb);
    t.sr = buf_rsrc(gm.s[0] + go, gb);
    t.br = buf_rsrc(gm.b[0] + go, gb);
    t.wr2 = buf_rsrc(gm.w[1] + wo, wb);
    t.sr2 = buf_rsrc(gm.s[1] + go, gb);
    t.br2 = buf_rsrc(gm.b[1] + go, gb);
    return t;
}

// Per-lane source offsets of a step's copies (step kt adds kt * 128, kt * 32
// and kt * 2 bytes).  A: copy i of wave w moves rows 8 (w A_DMA + i) .. + 8,
// lane -> (row, 16-byte chunk c), reading chunk c ^ (row & 7) of the row:
// the stage holds row r's chunk c at r * 128 + (c ^ (r & 7)) * 16.  B: copy
// q moves rows 32 (B_DMA w + q) .. + 32, two lanes per row.  Scales /
// biases: one row per lane, a zero-extended word each.
template <int BM, int NW>
struct W4Src {
    uint32_t a[BM / (8 * NW)];
    uint32_t b[8 / NW];
    uint32_t g;
};

template <int BM, int NW, bool PAIR>
__device__ __forceinline__ void w4_src(W4Src<BM, NW>& src, int K, int wave, int lane) {
    constexpr int A_DMA = BM / (8 * NW), B_DMA = 8 / NW;
    const int G = K >> 6, wpr = K >> 3;
#pragma unroll
    for (int i = 0; i < A_DMA; i++) {
        const int r = (wave * A_DMA + i) * 8 + (lane >> 3), c = lane & 7;
        src.a[i] = static_cast<uint32_t>(r * K + (c ^ (r & 7)) * 8) * 2u;
    }
#pragma unroll
    for (int q = 0; q < B_DMA; q++) {
        const int r = ((B_DMA * wave + q) * 32 + (lane >> 1)) & (PAIR ? 127 : 255);   // row of its matrix
        src.b[q] = static_cast<uint32_t>(r * wpr + (lane & 1) * 4) * 4u;
    }
    src.g = static_cast<uint32_t>(((PAIR ? wave & 1 : NW == 4 ? wave : wave & 3) * 64 + lane) * G) * 2u;
}

// How NW waves split a BM x 256 tile: WM x WN waves of RW rows x WC
// columns, TM x TN MFMA tiles of 32 x 32 each.  256-row tiles: 1 x 4 waves
// of 256 x 64 -- each weight word is dequantised once and feeds 8 MFMAs
// (a 2 x 2 split dequantises every word twice and measured 12% slower per
// K step); 128-row tiles: 2 x 4 waves of 64 x 64.
template <int BM, int NW>
struct W4Layout {
    static constexpr int WN = BM == 256 ? NW : NW / 2, WM = NW / WN;
    static constexpr int RW = BM / WM, WC = 256 / WN;
    static constexpr int TM = RW / 32, TN = WC / 32;
};

template <int BM, int NW>
using W4Acc = gemm_f32x16[W4Layout<BM, NW>::TM][W4Layout<BM, NW>::TN];

// The stage row (of 256) of weight column block j of wave column wn: WC
// consecutive rows per wave; paired tiles: gate rows wn 32 .. (j = 0) and
// the same up rows, 128 further (j = 1).
template <bool PAIR, int WC>
__device__ __forceinline__ int w4_brow(int wn, int j, int lane) {
    return PAIR ? j * 128 + wn * 32 + (lane & 31) : wn * WC + j * 32 + (lane & 31);
}

// K steps [k0, k0 + nk) of one tile into acc (which it adds to): the copy
// pipeline starts and drains inside, and on return every wave is past its
// last LDS read and no copy is in flight, so the next segment may reuse the
// ring.
template <int BM, int NW, bool PAIR = false>
__device__ __forceinline__ void w4_segment(W4Acc<BM, NW>& acc, char* lds, const W4Tile& t, const W4Src<BM, NW>& src,
                                           int k0, int nk, int wave, int lane) {
    using L = W4Layout<BM, NW>;
    constexpr int WN = L::WN, WC = L::WC, RW = L::RW, TM = L::TM, TN = L::TN;
    constexpr int A_DMA = BM / (8 * NW), B_DMA = 8 / NW;
    constexpr int PER_STEP = A_DMA + B_DMA + (NW == 4 ? 2 : 1);    // copies per wave and step
    constexpr int STAGE = w4_stage_bytes(BM);
    const int hb = lane >> 5;
    const int wm = wave / WN, wn = wave % WN;
    w4_issue<BM, NW, PAIR>(lds, t, src.a, src.b, src.g, k0, 0 < nk, wave);
    w4_issue<BM, NW, PAIR>(lds + STAGE, t, src.a, src.b, src.g, k0 + 1, 1 < nk, wave);
    for (int it = 0; it < nk; it++) {
        // step it's copies are done (only step it + 1's may be in flight)
        __builtin_amdgcn_s_waitcnt(0x0F70 | PER_STEP);
        // a bare barrier: every wave's copies of step it are in LDS and every
        // wave is past step it - 1, whose stage step it + 2 refills (a fence
        // would also wait for the copies of step it + 1)
        __builtin_amdgcn_s_barrier();
        w4_issue<BM, NW, PAIR>(lds + ((it + 2) % 3) * STAGE, t, src.a, src.b, src.g, k0 + it + 2, it + 2 < nk, wave);
        const char* st = lds + (it % 3) * STAGE;
        const uint16_t* As = reinterpret_cast<const uint16_t*>(st);
        const uint32_t* Bs = reinterpret_cast<const uint32_t*>(st + BM * 128);
        const uint32_t* Ss = reinterpret_cast<const uint32_t*>(st + BM * 128 + 8192);
        const uint32_t* Ts = reinterpret_cast<const uint32_t*>(st + BM * 128 + 9216);
        float sf[TN], bf[TN];
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int row = w4_brow<PAIR, WC>(wn, j, lane);
            sf[j] = h2f(static_cast<uint16_t>(Ss[row]));
            bf[j] = h2f(static_cast<uint16_t>(Ts[row]));
        }
        // four K slices of 16; slice ks + 1's operands are read while slice
        // ks multiplies, and its dequant is spread over the last of slice
        // ks's MFMAs (fences pin the order), so the VALU work runs under the
        // matrix core instead of before it
        constexpr int NM = TM * TN, NPC = TN * 4;                  // MFMAs, dequant pieces per slice
        auto a_frag = [&](int ks, int i) {
            const int row = wm * RW + i * 32 + (lane & 31);
            const int c = (2 * ks + hb) ^ (row & 7);
            return *reinterpret_cast<const gemm_bf16x8*>(As + row * 64 + c * 8);
        };
        auto b_word = [&](int ks, int j) { return Bs[w4_brow<PAIR, WC>(wn, j, lane) * 8 + 2 * ks + hb]; };
        gemm_bf16x8 av[2][TM], bv[2][TN];
        uint32_t bw[TN], blo[TN], bhi[TN], pk[TN][4];
#pragma unroll
        for (int j = 0; j < TN; j++) bv[0][j] = w4_dequant8(b_word(0, j), sf[j], bf[j]);
#pragma unroll
        for (int i = 0; i < TM; i++) av[0][i] = a_frag(0, i);
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int cu = ks & 1, nx = cu ^ 1;
            if (ks < 3) {
#pragma unroll
                for (int j = 0; j < TN; j++) bw[j] = b_word(ks + 1, j);
#pragma unroll
                for (int i = 0; i < TM; i++) av[nx][i] = a_frag(ks + 1, i);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const int i = m / TN, j = m % TN;
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[cu][i], bv[cu][j], acc[i][j], 0, 0, 0);
                if (ks < 3) {
                    constexpr int M0 = NPC < NM ? NM - NPC : 0, NR = NM - M0;   // pieces in the last NR MFMAs
#pragma unroll
                    for (int pc = m < M0 ? 0 : (m - M0) * NPC / NR; pc < (m < M0 ? 0 : (m - M0 + 1) * NPC / NR); pc++) {
                        const int jj = pc / 4, q = pc % 4;
                        if (q == 0) {
                            blo[jj] = bw[jj] & 0x0F0F0F0Fu;          // even / odd elements, a byte each
                            bhi[jj] = (bw[jj] >> 4) & 0x0F0F0F0Fu;
                        }
                        pk[jj][q] = w4_pack_bf16(
                            __builtin_fmaf(static_cast<float>((blo[jj] >> (8 * q)) & 0xFFu), sf[jj], bf[jj]),
                            __builtin_fmaf(static_cast<float>((bhi[jj] >> (8 * q)) & 0xFFu), sf[jj], bf[jj]));
                        if (q == 3)
                            bv[nx][jj] = __builtin_bit_cast(gemm_bf16x8,
                                                            make_uint4(pk[jj][0], pk[jj][1], pk[jj][2], pk[jj][3]));
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    // the last copies issued (past the segment) read nothing; wait for them,
    // and for every wave's last LDS reads
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
}

// C tile: lane l, register v holds row 8 (v / 4) + 4 (l / 32) + v % 4,
// column l % 32.  o: a [M][ldo] block whose column 0 is column c0 of the
// product.
template <int BM, int NW>
__device__ __forceinline__ void w4_store(const W4Acc<BM, NW>& acc, float* o, const W4Tile& t, int M, int N, int ldo,
                                         int c0, int wave, int lane) {
    using L = W4Layout<BM, NW>;
    constexpr int WN = L::WN, WC = L::WC, RW = L::RW, TM = L::TM, TN = L::TN;
    const int hb = lane >> 5, wm = wave / WN, wn = wave % WN;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = t.m0 + wm * RW + i * 32 + 8 * (v >> 2) + 4 * hb + (v & 3);
                const int col = t.n0 + wn * WC + j * 32 + (lane & 31);
                if (row < M && col < N) o[static_cast<size_t>(row) * ldo + (col - c0)] = acc[i][j][v];
            }
}

// Part h of NP of w4_store's tiles (i TN + j in [h TM TN / NP, (h + 1) TM TN
// / NP)), into a [M][N] output; NaN in place of every value if `poison`.
template <int BM, int NW, int NP>
__device__ __forceinline__ void w4_store_rows(const W4Acc<BM, NW>& acc, float* o, const W4Tile& t, int M, int N, int h,
                                              bool poison, int wave, int lane) {
    using L = W4Layout<BM, NW>;
    constexpr int WN = L::WN, WC = L::WC, RW = L::RW, TM = L::TM, TN = L::TN;
    const int hb = lane >> 5, wm = wave / WN, wn = wave % WN;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            if ((i * TN + j) / (TM * TN / NP) != h) continue;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = t.m0 + wm * RW + i * 32 + 8 * (v >> 2) + 4 * hb + (v & 3);
                const int col = t.n0 + wn * WC + j * 32 + (lane & 31);
                if (row < M && col < N)
                    o[static_cast<size_t>(row) * N + col] = poison ? __builtin_nanf("") : acc[i][j][v];
            }
        }
}

template <int BM, int NW>
__device__ __forceinline__ void w4_zero(W4Acc<BM, NW>& acc) {
    constexpr int TM = W4Layout<BM, NW>::TM, TN = W4Layout<BM, NW>::TN;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;
}

// The matrix of launch block nt (uniform).
__device__ __forceinline__ int gm_mat(const GemmMats& gm, int nt) {
    int k = 0;
#pragma unroll
    for (int i = 1; i < 4; i++) k += (i < gm.count && nt >= gm.nb0[i]) ? 1 : 0;
    return __builtin_amdgcn_readfirstlane(k);
}

// Data-parallel: workgroup (mt, nt, z) computes K steps [z kt_split,
// (z+1) kt_split) of tile (mt, nt): into its matrix's output, or (part)
// into part + z M ldp at the matrix's columns.
template <int BM, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_w4_kernel(const uint16_t* __restrict__ xb, GemmMats gm,
                                                          float* __restrict__ part, int M, int K, int kt_split,
                                                          int ldp) {
    extern __shared__ uint4 w4_lds[];
    char* lds = reinterpret_cast<char*>(w4_lds);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = K >> 6;
    const int kt0 = blockIdx.z * kt_split;
    const int nk = G - kt0 < kt_split ? G - kt0 : kt_split;
    const int k = gm_mat(gm, blockIdx.y);
    const int N = gm.n_out[k];
    const W4Tile t = w4_tile<BM>(xb, gm.w[k], gm.s[k], gm.b[k], M, N, K, blockIdx.x, blockIdx.y - gm.nb0[k]);
    W4Src<BM, NW> src;
    w4_src<BM, NW, false>(src, K, wave, lane);
    W4Acc<BM, NW> acc;
    w4_zero<BM, NW>(acc);
    w4_segment<BM, NW>(acc, lds, t, src, kt0, nk, wave, lane);
    if (part)
        w4_store<BM, NW>(acc, part + static_cast<size_t>(blockIdx.z) * M * ldp + gm.col0[k], t, M, N, ldp, 0, wave,
                         lane);
    else
        w4_store<BM, NW>(acc, gm.out[k], t, M, N, N, 0, wave, lane);
}

// Paired gate/up tiles (blockIdx.y = block of 128 output columns), every K
// step: h[r][c] = bf16(SiLU(x W_gate^T) * (x W_up^T)), rounded to nearest
// even -- the fp32 products of two gemm_w4_kernel calls through silu_mul,
// then the bf16 rounding the down projection applies to its x.
template <int BM, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_w4_pair_kernel(const uint16_t* __restrict__ xb, GemmMats gm,
                                                               uint16_t* __restrict__ h, int M, int K) {
    static_assert(BM == 256 && NW == 4, "paired tiles: 4 waves of 256 x (32 gate + 32 up) columns");
    using L = W4Layout<BM, NW>;
    constexpr int TM = L::TM;
    extern __shared__ uint4 w4_lds[];
    char* lds = reinterpret_cast<char*>(w4_lds);
    const int lane = threadIdx.x & 63, hb = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int N = gm.n_out[0];
    const W4Tile t = w4_tile_pair<BM>(xb, gm, M, N, K, blockIdx.x, blockIdx.y);
    W4Src<BM, NW> src;
    w4_src<BM, NW, true>(src, K, wave, lane);
    W4Acc<BM, NW> acc;
    w4_zero<BM, NW>(acc);
    w4_segment<BM, NW, true>(acc, lds, t, src, 0, K >> 6, wave, lane);
    const int col = t.n0 + wave * 32 + (lane & 31);
    if (col >= N) return;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int row = t.m0 + i * 32 + 8 * (v >> 2) + 4 * hb + (v & 3);
            if (row < M) {
                const float a = silu_mul(acc[i][0][v], acc[i][1][v]);
                h[static_cast<size_t>(row) * N + col] = static_cast<uint16_t>(w4_pack_bf16(a, a) & 0xFFFFu);
            }
        }
}

// Stream-K: the tiles (m block major) are split into nx contiguous groups,
// one per XCD, and each group's T = tiles x G (tile, K step) iterations,
// tile-major and K-minor, into P equal contiguous ranges, one per workgroup
// of that XCD.  A range splits at tile boundaries into segments: a tile's
// tail, whole tiles, the next tile's head; the workgroup runs them last to
// first.  A segment that does not reach its tile's end (only a range's last
// one can be such) is a partial: it goes to the workgroup's slot in `part`
// at device scope, then its flag is set to the launch's epoch.  The segment
// that ends a tile (its owner's) adds the partials of the workgroups before
// it in its group that cover the rest of the tile, nearest first, and
// stores the tile.  Waits point only to lower-numbered workgroups, which
// are dispatched first, and a partial is a workgroup's first segment, so an
// owner, which reaches its first segment last, rarely waits.  With at
// least as many workgroups as tiles a range is at most G iterations long
// (two segments); with fewer, each tile has at most one partial.
// Paired gate/up tiles (PAIR) take the same route, the owner's store being
// the SiLU * up epilogue of gemm_w4_pair_kernel.
//
// The epoch makes a flag mean "this launch's partial is in": every
// workgroup reads it from ctl[0] when it starts, and the last workgroup to
// leave advances it.  A flag is never lowered, so a partial that arrives
// after its owner gave up waiting (an error, its tile stored as NaN) holds
// an old epoch that no later launch waits for.  Stream-ordered launches on
// one workspace, captured ones included, each see their own epoch.
//
// A slot holds 256 x 256 floats as [block b][quad q][thread] of 16 bytes,
// block b = i TN + j of the accumulators, quad q = v / 4: every store and
// LDS read of a wave is 1 KiB contiguous.  The owner cannot add a whole
// partial in registers (the accumulators live in AGPRs, which VALU adds do
// not read), so it brings each quarter of a slot into the drained LDS ring by
// global->LDS copies and adds it from there, storing each quarter of the
// tile once its partials are in.
constexpr int kSkParts = 4;                                        // the owner adds a slot in 4 parts
constexpr int kSkFlagStride = 32;                                  // flags 128 bytes apart
constexpr long long kSkSpinTicks = 20000000;                       // 200 ms at 100 MHz
// The control words after the flags (each on its own 128-byte line): the
// epoch counter, the exit counter, the error counter.
constexpr int kSkCtlGen = 0, kSkCtlExited = 32, kSkCtlErrors = 64, kSkCtlWords = 96;
static_assert(kSkCtlWords == kSkCtlWordsHost && kSkCtlErrors == kSkCtlErrorsHost, "one layout of the control words");

// A workgroup's stream-K group: the tiles [t0, t0 + T / G) of XCD `xcd`
// (tiles m-block major, split into nx contiguous groups; workgroup i runs
// on XCD i mod nx, so an XCD's L2 holds only its group's rows of x), run
// by the P workgroups xcd, xcd + nx, .. (slots 0 .. P - 1).
struct SkGroup {
    long T;
    int P, slot, xcd, nx, t0;
    __device__ int phys(int s) const { return xcd + nx * s; }
};

// Part hp of NP of a paired tile's outputs: h = bf16(SiLU(gate) * up) of
// the accumulator rows i with i TN / (TM TN / NP) = hp; NaN if `poison`.
template <int BM, int NW, int NP>
__device__ __forceinline__ void w4_store_pair_rows(const W4Acc<BM, NW>& acc, uint16_t* h, const W4Tile& t, int M,
                                                   int N, int hp, bool poison, int wave, int lane) {
    constexpr int TM = W4Layout<BM, NW>::TM, TN = W4Layout<BM, NW>::TN;
    static_assert(TN == 2, "paired tiles hold a gate and an up block per wave");
    const int hb = lane >> 5;
    const int col = t.n0 + wave * 32 + (lane & 31);
    if (col >= N) return;
#pragma unroll
    for (int i = 0; i < TM; i++) {
        if ((i * TN) / (TM * TN / NP) != hp) continue;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int row = t.m0 + i * 32 + 8 * (v >> 2) + 4 * hb + (v & 3);
            if (row < M) {
                const float a = silu_mul(acc[i][0][v], acc[i][1][v]);
                h[static_cast<size_t>(row) * N + col] =
                    poison ? static_cast<uint16_t>(0x7FC0u) : static_cast<uint16_t>(w4_pack_bf16(a, a) & 0xFFFFu);
            }
        }
    }
}

// Segment [it, stop) of a stream-K range (stop at most its tile's end).
// NTL: tiles per block row (the N blocks of gm, or of the paired columns).
template <int BM, int NW, bool PAIR>
__device__ __forceinline__ void w4_sk_segment(char* lds, const uint16_t* xb, const GemmMats& gm, float* part,
                                              uint16_t* hout, unsigned* flags, unsigned* errors, unsigned epoch,
                                              int M, int K, int NTL, const SkGroup& gp, long it, long stop,
                                              const W4Src<BM, NW>& src, int tid, int wave, int lane) {
    typedef __attribute__((address_space(3))) void* lds_ptr;
    constexpr int TM = W4Layout<BM, NW>::TM, TN = W4Layout<BM, NW>::TN, NB = TM * TN;
    constexpr int NT = 64 * NW;
    constexpr int kDevice = 16;                                    // sc1: device-coherent
    constexpr uint32_t kSlotBytes = 256u * 256u * 4u;
    using u32x4 = unsigned int __attribute__((__vector_size__(16)));
    const int G = K >> 6;
    const long T = gp.T;
    const int P = gp.P, wg = gp.slot;
    W4Acc<BM, NW> acc;
    const int k0 = static_cast<int>(it % G);
    const int nk = static_cast<int>(stop - it);
    const long tile_start = it - k0;                               // in the group's iterations
    const int tile = gp.t0 + static_cast<int>(it / G);
    const int nt = tile % NTL, mk = PAIR ? 0 : gm_mat(gm, nt);
    const int N = gm.n_out[mk];
    float* const out = gm.out[mk];
    const W4Tile t = PAIR ? w4_tile_pair<BM>(xb, gm, M, N, K, tile / NTL, nt)
                          : w4_tile<BM>(xb, gm.w[mk], gm.s[mk], gm.b[mk], M, N, K, tile / NTL, nt - gm.nb0[mk]);
    w4_zero<BM, NW>(acc);
    w4_segment<BM, NW, PAIR>(acc, lds, t, src, k0, nk, wave, lane);
    if (stop < tile_start + G) {
        const __amdgpu_buffer_rsrc_t pr =
            buf_rsrc(part + static_cast<size_t>(gp.phys(wg)) * (kSlotBytes / 4), kSlotBytes);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int v = 0; v < 16; v += 4) {
                    // by value: a bit cast of a vector element would read element 0
                    const u32x4 q = {__float_as_uint(acc[i][j][v]), __float_as_uint(acc[i][j][v + 1]),
                                     __float_as_uint(acc[i][j][v + 2]), __float_as_uint(acc[i][j][v + 3])};
                    const uint32_t o = static_cast<uint32_t>(((i * TN + j) * 4 + v / 4) * NT + tid) * 16u;
                    __builtin_amdgcn_raw_buffer_store_b128(q, pr, o, 0, kDevice);
                }
        __builtin_amdgcn_s_waitcnt(0x0F70);                    // this thread's stores have landed
        __syncthreads();
        if (tid == 0)
            __hip_atomic_store(flags + gp.phys(wg) * kSkFlagStride, epoch, __ATOMIC_RELEASE,
                               __HIP_MEMORY_SCOPE_AGENT);
    } else {
        // the partials of workgroups wg - 1, wg - 2, .. j1, whose ranges
        // end inside this tile
        int j1 = wg;
        while (j1 > 0 && T * j1 / P > tile_start) j1--;
        int missing = 0;
        if (tid == 0) {
            for (int j = wg - 1; j >= j1; j--) {
                if (T * (j + 1) / P == T * j / P) continue;        // an empty range
                const long long t0 = __builtin_amdgcn_s_memrealtime();
                while (__hip_atomic_load(flags + gp.phys(j) * kSkFlagStride, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT) != epoch) {
                    if (__builtin_amdgcn_s_memrealtime() - t0 > kSkSpinTicks) {
                        __hip_atomic_fetch_add(errors, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        missing = 1;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
            }
        }
        // a tile whose partials did not all arrive is stored as NaN
        const bool poison = __syncthreads_or(missing) != 0;
        // the partials, not stale cache lines (only when there are any: the
        // invalidate also drops the operand lines the XCD's other
        // workgroups are streaming)
        if (j1 < wg) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        // part h of the tile (blocks h NB / kSkParts ..): each partial's part
        // in turn through LDS, then the part is stored, so only a quarter of
        // the accumulators is ever live in VGPRs
        constexpr int PB = NB / kSkParts;                          // blocks per part
        constexpr int PCH = PB * 16;                               // 1 KiB chunks per part
#pragma unroll
        for (int h = 0; h < kSkParts; h++) {
            for (int j = wg - 1; j >= j1; j--) {
                if (T * (j + 1) / P == T * j / P) continue;
                const __amdgpu_buffer_rsrc_t pr =
                    buf_rsrc(part + static_cast<size_t>(gp.phys(j)) * (kSlotBytes / 4), kSlotBytes);
#pragma unroll
                for (int c = 0; c < PCH / NW; c++) {
                    const int chunk = wave * (PCH / NW) + c;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        pr, (lds_ptr)(lds + chunk * 1024), 16, static_cast<uint32_t>(lane) * 16u,
                        static_cast<uint32_t>((h * PCH + chunk) * 1024), 0, kDevice);
                }
                __builtin_amdgcn_s_waitcnt(0x0F70);
                __syncthreads();
                const float4* hp = reinterpret_cast<const float4*>(lds);
#pragma unroll
                for (int b = 0; b < PB; b++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int blk = h * PB + b, i = blk / TN, jj = blk % TN;
                        const float4 p4 = hp[(b * 4 + q) * NT + tid];
                        acc[i][jj][4 * q] = __fadd_rn(acc[i][jj][4 * q], p4.x);
                        acc[i][jj][4 * q + 1] = __fadd_rn(acc[i][jj][4 * q + 1], p4.y);
                        acc[i][jj][4 * q + 2] = __fadd_rn(acc[i][jj][4 * q + 2], p4.z);
                        acc[i][jj][4 * q + 3] = __fadd_rn(acc[i][jj][4 * q + 3], p4.w);
                    }
                __syncthreads();                               // before the next copies overwrite LDS
            }
            if constexpr (PAIR) w4_store_pair_rows<BM, NW, kSkParts>(acc, hout, t, M, N, h, poison, wave, lane);
            else w4_store_rows<BM, NW, kSkParts>(acc, out, t, M, N, h, poison, wave, lane);
        }
    }
}

template <int BM, int NW, bool PAIR>
__global__ __launch_bounds__(64 * NW) void gemm_w4_sk_kernel(const uint16_t* __restrict__ xb, GemmMats gm,
                                                             float* __restrict__ part, unsigned* __restrict__ flags,
                                                             unsigned* __restrict__ ctl, int M, int K, int nx,
                                                             uint16_t* __restrict__ hout) {
    static_assert(BM == 256 && NW == 4, "stream-K slots assume 256 x 256 tiles of 4 waves");
    extern __shared__ uint4 w4_lds[];
    char* lds = reinterpret_cast<char*>(w4_lds);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = K >> 6;
    const int NTL = PAIR ? (gm.n_out[0] + 127) / 128 : gm.nb0[gm.count];
    const int tiles = ((M + BM - 1) / BM) * NTL;
    SkGroup gp;
    gp.xcd = blockIdx.x % nx;
    gp.nx = nx;
    gp.slot = blockIdx.x / nx;
    gp.P = gridDim.x / nx;
    gp.t0 = tiles * gp.xcd / nx;
    gp.T = static_cast<long>(tiles * (gp.xcd + 1) / nx - gp.t0) * G;
    const long begin = gp.T * gp.slot / gp.P, end = gp.T * (gp.slot + 1) / gp.P;
    // this launch's epoch (never 0: the flags start at 0)
    const unsigned epoch =
        __builtin_amdgcn_readfirstlane(__hip_atomic_load(ctl + kSkCtlGen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) +
        1u;
    unsigned* errors = ctl + kSkCtlErrors;
    if (begin < end) {
        W4Src<BM, NW> src;
        w4_src<BM, NW, PAIR>(src, K, wave, lane);
        // the segments, last to first: [max(tile start, begin), seg_end)
        for (long seg_end = end; seg_end > begin;) {
            const long tile_start = (seg_end - 1) / G * G;
            const long seg_start = tile_start > begin ? tile_start : begin;
            w4_sk_segment<BM, NW, PAIR>(lds, xb, gm, part, hout, flags, errors, epoch, M, K, NTL, gp, seg_start,
                                        seg_end, src, tid, wave, lane);
            seg_end = seg_start;
        }
    }
    // the last workgroup to leave advances the epoch (every workgroup has
    // read it by then: the release orders that read before the count)
    if (tid == 0) {
        const unsigned left =
            __hip_atomic_fetch_add(ctl + kSkCtlExited, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (left == gridDim.x - 1) {
            __hip_atomic_store(ctl + kSkCtlExited, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // epoch - 1 is the stored value; skip the one whose epoch would be 0
            const unsigned next = epoch == 0xFFFFFFFFu ? 0u : epoch;
            __hip_atomic_store(ctl + kSkCtlGen, next, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int BM, int NW>
size_t w4_lds_bytes() {
    return static_cast<size_t>(3) * w4_stage_bytes(BM);
}

template <int BM, int NW>
int launch_w4(const uint16_t* xb, const GemmMats& gm, float* part, int M, int K, int S, int kt_split, int ldp,
              hipStream_t st) {
    auto kern = gemm_w4_kernel<BM, NW>;
    const size_t lds = w4_lds_bytes<BM, NW>();
    static std::atomic<uint64_t> lds_raised{0};
    if (int rc = raise_lds_limit(reinterpret_cast<const void*>(kern), lds, lds_raised)) return rc;
    hipLaunchKernelGGL(kern, dim3((M + BM - 1) / BM, gm.nb0[gm.count], S), dim3(64 * NW), lds, st, xb, gm, part, M, K,
                       kt_split, ldp);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q4_EHIP, "prefill gemm launch: %s", hipGetErrorString(e));
    return 0;
}

template <int BM, int NW, bool PAIR>
int launch_w4_sk(const uint16_t* xb, const GemmMats& gm, float* part, unsigned* flags, unsigned* ctl, int M, int K,
                 int P, int nx, uint16_t* hout, hipStream_t st) {
    auto kern = gemm_w4_sk_kernel<BM, NW, PAIR>;
    const size_t lds = w4_lds_bytes<BM, NW>();
    static_assert(256 * 256 * 4 / kSkParts <= 3 * w4_stage_bytes(BM), "a part of a slot fits the LDS ring");
    static std::atomic<uint64_t> lds_raised{0};
    if (int rc = raise_lds_limit(reinterpret_cast<const void*>(kern), lds, lds_raised)) return rc;
    hipLaunchKernelGGL(kern, dim3(P), dim3(64 * NW), lds, st, xb, gm, part, flags, ctl, M, K, nx, hout);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q4_EHIP, "prefill gemm (stream-K) launch: %s", hipGetErrorString(e));
    return 0;
}

int gemm_w4_pair(const uint16_t* xb, const GemmMats& gm, uint16_t* h, int M, int K, hipStream_t st) {
    auto kern = gemm_w4_pair_kernel<256, 4>;
    const size_t lds = w4_lds_bytes<256, 4>();
    static std::atomic<uint64_t> lds_raised{0};
    if (int rc = raise_lds_limit(reinterpret_cast<const void*>(kern), lds, lds_raised)) return rc;
    hipLaunchKernelGGL(kern, dim3((M + 255) / 256, (gm.n_out[0] + 127) / 128), dim3(256), lds, st, xb, gm, h, M, K);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q4_EHIP, "prefill gate/up gemm launch: %s", hipGetErrorString(e));
    return 0;
}

int gemm_w4(const uint16_t* xb, const GemmMats& gm, float* part, int M, int K, int bm, int S, int kt_split, int ldp,
            hipStream_t st) {
    // 256-row tiles: 4 waves of 256 x 64 (a dequantised weight word feeds 8
    // MFMAs); 128-row tiles: 8 waves of 64 x 64
    return bm == 256 ? launch_w4<256, 4>(xb, gm, part, M, K, S, kt_split, ldp, st)
                     : launch_w4<128, 8>(xb, gm, part, M, K, S, kt_split, ldp, st);
}

int gemm_w4_sk(const uint16_t* xb, const GemmMats& gm, float* part, unsigned* flags, unsigned* ctl, int M, int K,
               int P, int nx, hipStream_t st) {
    return launch_w4_sk<256, 4, false>(xb, gm, part, flags, ctl, M, K, P, nx, nullptr, st);
}

int gemm_w4_sk_pair(const uint16_t* xb, const GemmMats& gm, float* part, unsigned* flags, unsigned* ctl, uint16_t* h,
                    int M, int K, int P, int nx, hipStream_t st) {
    return launch_w4_sk<256, 4, true>(xb, gm, part, flags, ctl, M, K, P, nx, h, st);
}

}  // namespace q4k
