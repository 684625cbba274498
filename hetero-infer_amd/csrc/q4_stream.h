// The streaming single-launch GEMV kernel and its launch, shared by
// q4gemv.hip (which picks the instance) and q4_stream_inst.hip (which
// compiles the instances, one object per (rows, pair, ring) in parallel).
#pragma once

#include "q4_common.h"

namespace q4k {

// ---------------------------------------------- streaming single-launch GEMV --
//
// One launch per call; weights are streamed row-contiguously (a wave-load
// moves 1 KiB of one row: 64 lanes x 16 bytes).  Group size 64.
//   * The x prologue runs once per workgroup.  Every x load is issued before
//     the first weight load and x is read once: vector-memory results return
//     in issue order, so an x load issued behind the weight stream would wait
//     for it.  Each thread loads whole packed words (8 values), one per
//     round of blockDim.x words, and takes amax; the 8 lanes of a group
//     chain its sum in ascending order, lane after lane, one chain per
//     round; after one barrier every thread writes the int8/uint8 planes of
//     its words of the int16 x into LDS.
//   * Then every wave works alone on a flat stream of 1 KiB items: the items
//     of its units (UB consecutive rows; PAIR: UB rows of matrix 0 and the
//     same UB rows of matrix 1), chunk-major within a unit so consecutive
//     items share x planes.  Units are handed to the waves of a workgroup
//     from an LDS counter as they free up.  A ring of RING items is in
//     flight (RING divides a unit's items): the item RING ahead is issued
//     right after an item is consumed, from straight-line code, so each wait
//     is a partial vmcnt; after the wave's last unit the ring drains without
//     loads, so nothing past it is ever loaded.  Lanes past a row end read
//     through a buffer range that ends with the row: 0, no memory access.
//   * Each group's fp32 term goes to a wave-private LDS table; when a unit
//     is done one lane per (m, row) adds its row's terms in ascending group
//     order -- no workgroup barrier in the main loop.
// The row a wave works on is wave-uniform (kept in SGPRs), so choosing the
// matrix of a grouped launch (q/k/v, gate/up: up to kMaxMats sharing x) is
// scalar work.
constexpr int kMaxMats = 4;
constexpr int kEarly = 2;           // ring items issued before the x prologue has its data
constexpr int kUnitItems = 16;      // rows per unit grow until a unit has this many items

struct MatList {
    const uint32_t* w[kMaxMats];
    const uint16_t* s[kMaxMats];
    const uint16_t* b[kMaxMats];
    float* out[kMaxMats];
    int n_out[kMaxMats];
    int row_begin[kMaxMats + 1];   // prefix sums of n_out
    int count;
    int mrows;                     // activation rows present (<= MR): the rest read 0 and are not stored
};

// The norm prologue (NORM instances): the kernel's input is
// rmsnorm(x + delta) * w, computed by every workgroup from x, delta (NULL:
// x alone) and w; workgroup 0 also stores x + delta to x_out (if not NULL).
struct NormArgs {
    const float* delta;
    const float* w;
    float* x_out;
    float eps;
    GreedyArgs greedy;   // one matrix, one row, no pair: the greedy token of the outputs
};

// Row stride of the per-wave term table, which holds one chunk's group
// terms (at most 32) per row: a multiple of 4 floats (16-byte reads) that is
// 4 mod 8 words, so lanes reading different rows spread over the banks.
constexpr int kTermStride = 36;

// x staged for the group sums: one group's values per LDS row, padded by 4
// floats so that lanes reading different groups spread over the banks.
__host__ __device__ constexpr int stage_stride(int gsh) { return (64 << gsh) + 4; }

// LDS of the streaming kernel: a header (group sums [mr][Gr], amax per wave
// [mr][16], the unit counter, the norm prologue's wave sums [16]), then the
// x planes and the per-wave term
// tables -- where the prologue first stages one row of x in fp32.
// rw: words of x per thread and row (the register rounds of the x prologue).
// sep: the staging after the term tables instead of over them (the planes
// may then be written while the group sums still read the staging).
inline size_t stream_lds_bytes(int mr, int n_chunks, int G, int nwaves, int NU, int rw, int gsh = 0, bool sep = false) {
    (void)rw;
    const size_t header = static_cast<size_t>(mr) * ((G + 3) & ~3) * 4 + static_cast<size_t>(mr) * 16 * 4 + 16 + 64;
    const size_t planes = static_cast<size_t>(mr) * n_chunks * 256 * 16;
    const size_t terms = static_cast<size_t>(nwaves) * mr * NU * kTermStride * 4;
    const size_t stage = static_cast<size_t>(G) * stage_stride(gsh) * 4;
    if (sep) return header + planes + terms + stage;
    return header + (planes + terms > stage ? planes + terms : stage);
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
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint64_t sel4(int p, uint64_t a0, uint64_t a1, uint64_t a2, uint64_t a3) {
    // uniform operands, kept in SGPRs (see the 32-bit form below)
    a0 = uniform64(a0);
    a1 = uniform64(a1);
    a2 = uniform64(a2);
    a3 = uniform64(a3);
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
    // the operands are uniform; readfirstlane keeps them in SGPRs where the
    // compiler would otherwise hold a loop-invariant copy in a VGPR
    a0 = __builtin_amdgcn_readfirstlane(a0);
    a1 = __builtin_amdgcn_readfirstlane(a1);
    a2 = __builtin_amdgcn_readfirstlane(a2);
    a3 = __builtin_amdgcn_readfirstlane(a3);
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
    int unit;                       // wave-uniform
};


// The rows of the unit the prefetch cursor is in: its matrix's w/s/b
// advanced to the unit's first row (PAIR: index 1 holds the same rows of
// matrix 1).  Resolved once per unit -- the host picks UB dividing every
// n_out, so a unit never straddles two matrices -- and wave-uniform, so an
// item's loads only add the row slot to scalar pointers.
struct UnitRows {
    const uint32_t* w[2];
    const uint16_t* s[2];
    const uint16_t* b[2];
};

template <bool PAIR>
__device__ __forceinline__ void unit_rows(UnitRows& ur, const MatList& ml, int unit, int UB, int wpr, int G) {
    const int gr = unit * UB;
    if constexpr (PAIR) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            ur.w[k] = ml.w[k] + static_cast<size_t>(gr) * wpr;
            ur.s[k] = ml.s[k] + static_cast<size_t>(gr) * G;
            ur.b[k] = ml.b[k] + static_cast<size_t>(gr) * G;
        }
    } else {
        // p is wave-uniform; readfirstlane makes that explicit, so the
        // kernel-argument reads are scalar loads
        const int p = __builtin_amdgcn_readfirstlane(mat_of_row(ml, gr));
        const int o = __builtin_amdgcn_readfirstlane(
            gr - sel4(p, ml.row_begin[0], ml.row_begin[1], ml.row_begin[2], ml.row_begin[3]));
        ur.w[0] = pick(ml.w, p) + static_cast<size_t>(o) * wpr;
        ur.s[0] = pick(ml.s, p) + static_cast<size_t>(o) * G;
        ur.b[0] = pick(ml.b, p) + static_cast<size_t>(o) * G;
    }
}

// Issue the loads of item (chunk c, row slot r) of the unit whose rows `ur`
// holds.  The row is wave-uniform: each array gets a resource that starts at
// the chunk and ends with the row, so lanes past the row end read 0 and cost
// no memory access, and `live` false (a prefetch past the wave's last item)
// gives an empty resource: every lane reads 0.  The chunk moves the
// resource's base (scalar work); the lanes' offsets are the same for every
// item.  No branch, so the waits on earlier loads stay exact.
template <bool PAIR, int GSH>
__device__ __forceinline__ void load_item(Item& it, const UnitRows& ur, int unit, int c, int r, int UB,
                                          int wpr, int G, uint32_t vo_w, uint32_t vo_g, bool live) {
    it.unit = unit;
    const bool second = PAIR && r >= UB;
    const int u = second ? r - UB : r;
    const uint32_t* wp = second ? ur.w[1] : ur.w[0];
    const uint16_t* sp = second ? ur.s[1] : ur.s[0];
    const uint16_t* bp = second ? ur.b[1] : ur.b[0];
    // byte offsets from the unit's first row, 32-bit (a unit is at most 8
    // rows of at most 16 KiB): row slot u, then chunk c
    const uint32_t cw = static_cast<uint32_t>(c) * kChunkWords * 4u;      // bytes of the row before chunk c
    const uint32_t cg = static_cast<uint32_t>(c) * (kChunkWords / (8 << GSH)) * 2u;  // bytes of its scales before it
    const uint32_t ow = static_cast<uint32_t>(u * wpr) * 4u + cw;
    const uint32_t og = static_cast<uint32_t>(u * G) * 2u + cg;
    const uint32_t wbytes = live ? static_cast<uint32_t>(wpr) * 4u - cw : 0u;
    const uint32_t gbytes = live ? static_cast<uint32_t>(G) * 2u - cg : 0u;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(reinterpret_cast<const char*>(wp) + ow, wbytes);
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(reinterpret_cast<const char*>(sp) + og, gbytes);
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(reinterpret_cast<const char*>(bp) + og, gbytes);
    // the three loads in a fixed order wherever an item is loaded: the
    // partial waits on the ring are computed from the issue order, which
    // must then be the same on entry to the main loop as around it.  The
    // weights are read once, so non-temporal (cache policy nt): the stream
    // does not push x and the outputs out of L2 and the last-level cache.
    // Scales and biases keep the default policy: an item reads a 64-byte
    // window of them that shares its edge sectors with the row's next item
    // and with the neighbouring rows.
    constexpr int kNonTemporal = 2;
    __builtin_amdgcn_sched_barrier(0);
    it.w = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, vo_w, 0, kNonTemporal));
    __builtin_amdgcn_sched_barrier(0);
    it.s = __builtin_amdgcn_raw_buffer_load_b16(rs, vo_g, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    it.b = __builtin_amdgcn_raw_buffer_load_b16(rb, vo_g, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
}

// acc + tp[0] + tp[1] + ... + tp[N-1], added in that order (fp32), all N
// terms read from LDS at once.  The running sum of a row's groups goes
// through this one chunk at a time: the same additions in the same order as
// one pass over the row's groups.
template <int N>
__device__ __forceinline__ float chain_add(float acc, const float* tp) {
    static_assert(N % 4 == 0, "whole float4 reads");
    const float4* t4 = reinterpret_cast<const float4*>(tp);
    float4 v[N / 4];
#pragma unroll
    for (int i = 0; i < N / 4; i++) v[i] = t4[i];
#pragma unroll
    for (int i = 0; i < N / 4; i++) {
        acc = __fadd_rn(acc, v[i].x);
        acc = __fadd_rn(acc, v[i].y);
        acc = __fadd_rn(acc, v[i].z);
        acc = __fadd_rn(acc, v[i].w);
    }
    return acc;
}

// Words of x per thread and activation row that the word pass keeps in
// registers (RW rounds of blockDim.x words); the host picks the instance.
template <int MR>
__host__ __device__ constexpr int stream_max_rounds() { return MR == 1 ? 4 : MR <= 4 ? 2 : 1; }

// Waves per CU the instance runs at: 4 per SIMD (<= 128 VGPRs), 2 for eight
// rows (<= 256 VGPRs, workgroups of at most 512 threads).
template <int MR>
__host__ __device__ constexpr int stream_waves_per_cu() { return MR >= 8 ? 8 : 16; }

// PAIR: matrices 0 and 1 (gate, up) are computed row for row and the output
// is out[0] = SiLU(gate) * up.
// NORM: the input is the RMSNorm of a residual sum (NormArgs), with the sum
// of squares taken in the order of add_rmsnorm_kernel (one word per thread,
// wave sums in wave order), so the input is bit for bit the one that
// kernel writes.  MR = 1 and RW = 1 only.
// Rows of x past ml.mrows (an M below MR) read 0 and their outputs are not
// stored.
// GSH: the group size is 64 << GSH (64 or 128): a group is 8 << GSH
// packed words, 2 << GSH lanes of an item.
// Host guarantees: chunks * 256 <= RW * blockDim.x, n_in % (64 << GSH) == 0,
// x 16-byte aligned.
// The greedy token's end of a launch (GreedyArgs): (bv, bi) is the lane's
// best stored row.  The wave's and then the workgroup's best go to
// g.part[blockIdx.x] through a device-coherent store; once the store is
// complete the workgroup counts itself, and the one that finds every other
// workgroup counted reduces the parts.  rv / ri: nwaves free LDS words each.
// Every thread of the workgroup calls it.
__device__ __forceinline__ void greedy_tail(float bv, int bi, const GreedyArgs& g, float* rv, int* ri, int lane,
                                            int wave, int nwaves) {
    constexpr int kCoherent = 16;                                 // cache policy sc1: device scope
    auto wave_best = [&](float& v, int& i) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const float ov = __shfl_xor(v, o);
            const int oi = __shfl_xor(i, o);
            argmax_better(v, i, ov, oi);
        }
    };
    wave_best(bv, bi);                                            // every lane: the wave's best
    if (lane == 0) {
        rv[wave] = bv;
        ri[wave] = bi;
    }
    __syncthreads();
    if (wave != 0) return;
    for (int w = 1; w < nwaves; w++) argmax_better(bv, bi, rv[w], ri[w]);
    const uint32_t parts = gridDim.x;
    const __amdgpu_buffer_rsrc_t pr = buf_rsrc(g.part, parts * 8u);
    using u32x2 = unsigned int __attribute__((ext_vector_type(2)));
    int last = 0;
    if (lane == 0) {
        const u32x2 v = {__float_as_uint(bv), static_cast<uint32_t>(bi)};
        __builtin_amdgcn_raw_buffer_store_b64(v, pr, blockIdx.x * 8u, 0, kCoherent);
        __builtin_amdgcn_s_waitcnt(0x0F70);                       // vmcnt(0): the part is stored
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        last = __hip_atomic_fetch_add(g.count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == parts - 1;
    }
    if (!__builtin_amdgcn_readfirstlane(last)) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    float fv = -__builtin_inff();
    int fi = kArgmaxNone;
    for (uint32_t k = lane; k < parts; k += 64) {
        const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(pr, k * 8u, 0, kCoherent));
        argmax_better(fv, fi, __uint_as_float(v.x), static_cast<int>(v.y));
    }
    wave_best(fv, fi);
    if (lane == 0) {
        // hetero/backends.py:106-109 and the decode loop's bookkeeping
        // (hetero/cpu_model.py:357-368): the token, its history slot, the
        // next position
        const int best = fi == kArgmaxNone ? 0 : fi;
        *g.tok = best;
        const int64_t p = *g.pos;
        const int64_t k = p - g.s0;
        if (k >= 0 && k < g.hist_len) g.hist[k] = best;
        *g.pos = p + 1;
        __hip_atomic_store(g.count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int MR, int RW, bool PAIR, int RING, bool NORM, int GSH>
__global__ __launch_bounds__(64 * stream_waves_per_cu<MR>()) void gemv_stream_kernel(MatList ml,
                                                                                     const float* __restrict__ x,
                                                                                     int n_in, int UB, int sep,
                                                                                     NormArgs na) {
    static_assert(!NORM || (MR == 1 && RW == 1 && GSH == 0), "the norm prologue takes one row, one word per thread");
    static_assert(GSH == 0 || GSH == 1, "group size 64 or 128");
    extern __shared__ uint4 lds4[];
    constexpr int lpg = 2 << GSH;                                 // lanes per group in an item
    constexpr int WPG = 8 << GSH;                                 // packed words per group
    const int wpr = n_in >> 3, G = n_in >> (6 + GSH);
    const int C = (wpr + kChunkWords - 1) / kChunkWords;
    const int Gr = (G + 3) & ~3;
    const int tid = threadIdx.x, nt = blockDim.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);    // wave-uniform
    const int nwaves = nt >> 6;
    float* xsum_lds = reinterpret_cast<float*>(lds4);             // [MR][Gr]
    float* red = xsum_lds + MR * Gr;                              // [MR][16]
    int* claim_ctr = reinterpret_cast<int*>(red + MR * 16);       // units handed out past the first
    float* stage = red + MR * 16 + 4;                              // NORM: the wave sums [16]
    uint4* xpl = reinterpret_cast<uint4*>(stage + 16);            // [MR][C*256] swizzled
    const int NU = PAIR ? 2 * UB : UB;                            // rows per unit
    float* Tw = reinterpret_cast<float*>(xpl + MR * C * 256) + wave * (MR * NU * kTermStride);
                                                                  // this wave: [MR][NU][kTermStride]
    // x staged for the group sums ([G][stage_stride], the prologue only):
    // after every wave's term tables (sep), so the planes need not wait for
    // the sums to have read it, or over the planes
    float* xstage = sep ? reinterpret_cast<float*>(xpl + MR * C * 256) + nwaves * MR * NU * kTermStride
                        : reinterpret_cast<float*>(xpl);
    if (tid == 0) *claim_ctr = 0;                                 // published by the prologue's first barrier

    // ---- x loads: thread t owns words t, t + nt, ... of every row, 8 values
    //      each, through a resource over x (words at or past the row end read
    //      0).  These are the first loads of the kernel, so the waits further
    //      down stay exact.
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(x, static_cast<uint32_t>(ml.mrows * n_in) * 4u);
    // unconditional (a wave with no word in a round reads past the range: 0,
    // no access), so the loads depend on nothing but x, n_in and mrows and
    // go out after the first round of kernel-argument reads
    float4 wv[MR][RW][2];
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const int j = r * nt + tid;
            const uint32_t off = j < wpr ? static_cast<uint32_t>(m * n_in + 8 * j) * 4u : kOutOfRange;
            wv[m][r][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
            wv[m][r][1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16, 0, 0));
        }
    // nothing below (the indexed row_begin read in particular) may be
    // scheduled ahead of these loads
    __builtin_amdgcn_sched_barrier(0);
    const int n_total = PAIR ? ml.n_out[0] : ml.row_begin[ml.count];
    const int n_units = (n_total + UB - 1) / UB;
    const int items = NU * C;
    // NORM: the thread's word of delta and of the norm weights (a NULL
    // delta reads through an empty range: no access)
    float4 nd[2], nw[2];
    if constexpr (NORM) {
        const uint32_t nb = static_cast<uint32_t>(n_in) * 4u;
        const __amdgpu_buffer_rsrc_t dr = buf_rsrc(na.delta ? na.delta : x, na.delta ? nb : 0u);
        const __amdgpu_buffer_rsrc_t wr = buf_rsrc(na.w, nb);
        if (wave * 64 < wpr) {                                    // uniform
            const uint32_t off = tid < wpr ? static_cast<uint32_t>(8 * tid) * 4u : kOutOfRange;
            nd[0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(dr, off, 0, 0));
            nd[1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(dr, off + 16, 0, 0));
            nw[0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
            nw[1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(wr, off + 16, 0, 0));
        }
    }

    // ---- the wave's item stream.  Workgroup b owns units b, b + grid, ...;
    //      wave w starts with its k = w-th one and claims further k from an
    //      LDS counter as it goes: issue arbitration favours a SIMD's oldest
    //      wave, so a fixed share per wave would leave the youngest waves
    //      finishing long after the others.  Item i of a unit is (chunk
    //      i / NU, row slot i % NU).  Up to kEarly items of the first ring are
    //      issued now, the rest once x is in (a full ring from every wave at
    //      once would queue ahead of the x loads of later waves).  A wave
    //      without a first unit loads through empty ranges.
    const int grid = gridDim.x;
    const int first_unit = blockIdx.x + wave * grid;
    const bool has_work = first_unit < n_units;                   // uniform
    constexpr int kE = RING < kEarly ? RING : kEarly;
    Item ring[RING];
    // the lane's byte offsets inside an item: its 16 bytes of weights, the
    // fp16 scale/bias of its group (two lanes per group)
    const uint32_t vo_w = static_cast<uint32_t>(lane) * 16u, vo_g = static_cast<uint32_t>(lane >> (1 + GSH)) * 2u;
    int pf_unit = first_unit, pf_c = 0, pf_r = 0;                 // prefetch cursor (uniform)
    UnitRows pf_rows;
    unit_rows<PAIR>(pf_rows, ml, pf_unit, UB, wpr, G);
#pragma unroll
    for (int d = 0; d < kE; d++) {
        load_item<PAIR, GSH>(ring[d], pf_rows, pf_unit, pf_c, pf_r, UB, wpr, G, vo_w, vo_g, has_work);
        if (++pf_r == NU) { pf_r = 0; ++pf_c; }
    }

    // ---- group sums (kernel/q4gemv.c:244-248: the group's 64 values added
    //      in ascending order) and the running max |x| (:258-259,
    //      NaN-skipping) per row.  The row is staged in LDS with one group
    //      per (padded) row, then one lane per group adds its values in
    //      order: a sequential sum with no cross-lane chain.
    if constexpr (NORM) {
        // hetero/cpu_model.py:304-306 (x + delta) and :164-166 (RMSNorm); the
        // squares are summed in NumPy's order (row_sum_numpy, as
        // add_rmsnorm_kernel does) through the x staging space and the
        // 16-float slot after red (both free until the x staging below); the
        // amax slots stay untouched
        float sq[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        float v[8] = {wv[0][0][0].x, wv[0][0][0].y, wv[0][0][0].z, wv[0][0][0].w,
                      wv[0][0][1].x, wv[0][0][1].y, wv[0][0][1].z, wv[0][0][1].w};
        if (wave * 64 < wpr) {                                    // uniform
            if (na.delta) {                                       // uniform
                const float d8[8] = {nd[0].x, nd[0].y, nd[0].z, nd[0].w, nd[1].x, nd[1].y, nd[1].z, nd[1].w};
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = __fadd_rn(v[i], d8[i]);
                if (na.x_out && blockIdx.x == 0) {                // uniform
                    const __amdgpu_buffer_rsrc_t xo = buf_rsrc(na.x_out, static_cast<uint32_t>(n_in) * 4u);
                    const uint32_t off = tid < wpr ? static_cast<uint32_t>(8 * tid) * 4u : kOutOfRange;
                    using u32x4 = unsigned int __attribute__((__vector_size__(16)));
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(u32x4, make_float4(v[0], v[1], v[2], v[3])), xo, off, 0, 0);
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(u32x4, make_float4(v[4], v[5], v[6], v[7])), xo, off + 16, 0, 0);
                }
            }
            if (tid < wpr) {
#pragma unroll
                for (int i = 0; i < 8; i++) sq[i] = __fmul_rn(v[i], v[i]);
            }
        }
        const float r = rms_factor(row_sum_numpy(sq, n_in, xstage, stage), n_in, na.eps);
        const float w8[8] = {nw[0].x, nw[0].y, nw[0].z, nw[0].w, nw[1].x, nw[1].y, nw[1].z, nw[1].w};
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = __fmul_rn(__fmul_rn(v[i], r), w8[i]);
        wv[0][0][0] = make_float4(v[0], v[1], v[2], v[3]);
        wv[0][0][1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    constexpr int SS = stage_stride(GSH);                         // staged floats per group
#pragma unroll
    for (int m = 0; m < MR; m++) {
        float amax = 0.0f;
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const float4 a = wv[m][r][0], b = wv[m][r][1];
            amax = fmaxf(amax, fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                                     fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w)))));
        }
        amax = wave_max(amax);
        if (lane == 0) red[m * 16 + wave] = amax;
        // row m staged in fp32, one group per LDS row: word j of group g at
        // xstage[g * SS + (j % WPG) * 8] (row m-1's sums are read first)
        if (m > 0) __syncthreads();
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const int j = r * nt + tid;
            if (r * nt + wave * 64 < wpr && j < wpr) {            // the wave's round has words; this one
                float4* dst = reinterpret_cast<float4*>(xstage + (j / WPG) * SS + (j % WPG) * 8);
                dst[0] = wv[m][r][0];
                dst[1] = wv[m][r][1];
            }
        }
        __syncthreads();
        // one lane per group adds its 64 << GSH values in ascending order
        for (int g = tid; g < G; g += nt) {
            float acc = 0.0f;
#pragma unroll
            for (int h = 0; h < (64 << GSH) / 32; h++) acc = chain_add<32>(acc, xstage + g * SS + h * 32);
            xsum_lds[m * Gr + g] = acc;
        }
    }
#pragma unroll
    for (int d = kE; d < RING; d++) {
        load_item<PAIR, GSH>(ring[d], pf_rows, pf_unit, pf_c, pf_r, UB, wpr, G, vo_w, vo_g, has_work);
        if (++pf_r == NU) { pf_r = 0; ++pf_c; }
    }
    if (!sep) __syncthreads();                                    // the staging is read: the planes may overwrite it

    // the claim for the wave's second unit, in flight during the rest of the prologue
    auto claim = [&]() -> int {
        int v = 0;
        if (lane == 0) v = __hip_atomic_fetch_add(claim_ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return v + nwaves;                                        // lane 0's value counts
    };
    int claimed = claim();

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

    // ---- main loop: consume the ring, refill each slot RING items ahead.
    //      A unit is a whole number of ring cycles (the host picks RING
    //      dividing the items of a unit), so units change -- the claim of the
    //      next one, the ordered chains of the finished one -- only between
    //      cycles, and a cycle is straight-line code: its refills are
    //      unconditional (exact waits).  After the wave's last unit the ring
    //      drains without loads.
    // one item: the integer dots of chunk c against row slot u, one fp32
    // term per group written by the group's last lane into the chunk's row of
    // the term table -- +0.0 for a group past the row end: added to a running
    // sum that starts at +0.0 (and so is never -0.0) it changes nothing
    constexpr int GPC = kChunkWords / WPG;                        // groups per chunk
    auto consume = [&](const Item& itm, int c, int u) {
        // group g = c * GPC + lane / lpg: a uniform part and a lane part
        const int lim = wpr - c * kChunkWords;                    // uniform
        const bool lead = (lane & (lpg - 1)) == lpg - 1;
        const bool in_row = lane * 4 < lim;
        const int gl = lane >> (1 + GSH);
        const int g = c * GPC + gl;
        uint32_t xle[MR][4], xlo[MR][4], xhe[MR][4], xho[MR][4];
#pragma unroll
        for (int m = 0; m < MR; m++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint4 pl = xpl[(m * C + c) * 256 + t * 64 + lane];
                xle[m][t] = pl.x; xlo[m][t] = pl.y; xhe[m][t] = pl.z; xho[m][t] = pl.w;
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
                float term = 0.0f;
                if (in_row) {
                    const float dot = __fmul_rn(xsc[m], static_cast<float>(part));
                    const float bx = __fmul_rn(bf, xsum_lds[m * Gr + g]);
                    term = __builtin_fmaf(sf, dot, bx);
                }
                Tw[(m * NU + u) * kTermStride + gl] = term;
            }
        }
    };
    // lane L < MR * NU keeps the running sum of row slot L % NU of x row
    // L / NU over the chunks done so far (kernel/q4gemv.c:286-293: the
    // groups in ascending order); a chunk's terms are added as soon as its
    // last row slot is consumed, so the end of a unit adds one chunk only
    float row_acc = 0.0f;
    auto chunk_done = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        if (lane < MR * NU) row_acc = chain_add<GPC>(row_acc, Tw + lane * kTermStride);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    };
    // GreedyArgs (one row, no pair): the lane's best stored row so far
    const bool greedy = MR == 1 && !PAIR && na.greedy.part != nullptr;   // uniform
    float g_bv = -__builtin_inff();
    int g_bi = kArgmaxNone;
    // a finished unit: its rows' sums are complete; one lane per (m, row)
    // stores the row's output
    auto finish = [&](int unit) {
        // (m, uu) = (lane / UB, lane % UB); its sum sits in lane m * NU + uu
        // (PAIR: the up row's in lane m * NU + UB + uu)
        const int src = (lane / UB) * NU + (lane % UB);
        const float acc = PAIR ? __shfl(row_acc, src & 63) : row_acc;
        const float up = PAIR ? __shfl(row_acc, (src + UB) & 63) : 0.0f;
        row_acc = 0.0f;
        if (lane < MR * UB) {
            const int m = lane / UB, uu = lane - m * UB, gr = unit * UB + uu;
            if (gr < n_total && m < ml.mrows) {
                if constexpr (PAIR) {
                    ml.out[0][static_cast<size_t>(m) * ml.n_out[0] + gr] = silu_mul(acc, up);
                } else {
                    // the host picks UB dividing every n_out, so a unit
                    // never straddles two matrices and p is wave-uniform
                    const int p = __builtin_amdgcn_readfirstlane(mat_of_row(ml, unit * UB));
                    const int no = sel4(p, ml.n_out[0], ml.n_out[1], ml.n_out[2], ml.n_out[3]);
                    const int rb = sel4(p, ml.row_begin[0], ml.row_begin[1], ml.row_begin[2],
                                        ml.row_begin[3]);
                    // through a buffer resource: a store through the selected
                    // pointer would be a flat store, which makes every later
                    // wait on the ring a full one
                    const __amdgpu_buffer_rsrc_t ro =
                        buf_rsrc(pick(ml.out, p), static_cast<uint32_t>(MR * no) * 4u);
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc), ro,
                                                          (m * no + (gr - rb)) * 4, 0, 0);
                    if (greedy) argmax_better(g_bv, g_bi, acc, gr - rb);
                }
            }
        }
    };
    if (has_work) {                                               // uniform
        const int cyc_per_unit = items / RING;
        int cyc_pf = 1;                                           // the first ring: cycle 0
        int cyc_cu = 0, cu_c = 0, cu_r = 0;                       // consume cursor (uniform)
        int cu_unit = first_unit;
        // the prefetch cursor has issued every cycle of its unit: move it to
        // the claimed unit, or report that the wave has none left
        auto next_unit = [&]() -> bool {
            const int u = blockIdx.x + __builtin_amdgcn_readfirstlane(claimed) * grid;
            if (u >= n_units) return false;
            pf_unit = u;
            unit_rows<PAIR>(pf_rows, ml, pf_unit, UB, wpr, G);
            pf_c = 0;
            pf_r = 0;
            cyc_pf = 0;
            claimed = claim();
            return true;
        };
        // one exit, at the bottom: the ring keeps its registers across cycles
        bool more = cyc_pf < cyc_per_unit || next_unit();
        while (more) {
#pragma unroll
            for (int d = 0; d < RING; d++) {
                consume(ring[d], cu_c, cu_r);
                // the refill may not be scheduled above the consume of its
                // slot, so that the slot keeps its registers
                __builtin_amdgcn_sched_barrier(0);
                load_item<PAIR, GSH>(ring[d], pf_rows, pf_unit, pf_c, pf_r, UB, wpr, G, vo_w, vo_g, true);
                if (++pf_r == NU) { pf_r = 0; ++pf_c; }
                if (++cu_r == NU) { chunk_done(); cu_r = 0; ++cu_c; }
            }
            ++cyc_pf;
            if (++cyc_cu == cyc_per_unit) {                       // uniform: unit done
                finish(cu_unit);
                cu_unit = pf_unit;
                cyc_cu = 0;
                cu_c = 0;
                cu_r = 0;
            }
            more = cyc_pf < cyc_per_unit || next_unit();
        }
        // the last cycle of the last unit
#pragma unroll
        for (int d = 0; d < RING; d++) {
            consume(ring[d], cu_c, cu_r);
            if (++cu_r == NU) { chunk_done(); cu_r = 0; ++cu_c; }
        }
        finish(cu_unit);
    }
    // the prologue's amax and wave-sum slots are free past its last barrier
    if constexpr (MR == 1 && !PAIR)
        if (greedy) greedy_tail(g_bv, g_bi, na.greedy, red, reinterpret_cast<int*>(stage), lane, wave, nwaves);
}

// Launch the instance: `want` workgroups, capped at what is resident at
// once for this instance (its own occupancy: rings differ in registers), so
// that every workgroup runs in the first round.
template <int MR, int RW, bool PAIR, int RING, bool NORM, int GSH>
int launch_stream_k(const MatList& ml, const float* x, const NormArgs& na, int n_in, int UB, int nwaves,
                    size_t lds, int sep, int want, hipStream_t st) {
    auto kern = gemv_stream_kernel<MR, RW, PAIR, RING, NORM, GSH>;
    static std::atomic<uint64_t> lds_raised{0};
    if (int rc = raise_lds_limit(reinterpret_cast<const void*>(kern), kStreamLdsMax, lds_raised)) return rc;
    int per_cu = 0;
    const hipError_t oe = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 64 * nwaves, lds);
    if (oe != hipSuccess || per_cu < 1) per_cu = 1;
    const int cap = num_cus() * per_cu;
    const int grid = want < cap ? want : cap;
    if (na.greedy.part && (MR != 1 || PAIR || grid > kGreedyMaxParts))
        return fail(Q4_EARG, "greedy token: one matrix, one row and at most %d workgroups", kGreedyMaxParts);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * nwaves), lds, st, ml, x, n_in, UB, sep, na);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q4_EHIP, "stream gemv launch: %s", hipGetErrorString(e));
    return 1;
}

}  // namespace q4k
