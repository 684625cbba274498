// Chained GEMV program: a sequence of dependent M=1 GEMV phases (the
// projections of a decode step, in order) in ONE persistent launch.
//
// Each phase is what one q4_gemv_multi_dev / q4_gate_up_silu_dev launch of
// one row computes, with the same arithmetic as the streaming kernel
// (q4_stream.h), bit for bit.  Between phases a grid barrier stands where
// the stream order of separate launches stood: phase p reads its x only
// after every workgroup has finished phase p-1.  What the single launch
// changes is what a wave may do before that barrier: the weights of phase p
// do not depend on x, so each wave issues its first ring of phase-p weight
// loads as soon as it is done with phase p-1, and they are in flight while
// the barrier completes and the x prologue runs -- the HBM stream does not
// stop at every dependency the way it does at a kernel boundary.
//
// Launch: one workgroup of 16 waves per CU, all resident at once (the grid
// barrier needs every workgroup running; the dynamic LDS is sized so that
// no CU holds two).  Every barrier wait is bounded in time: a wait that runs
// out records an error in the plan's sync words and the workgroup goes on
// (its results are then invalid; q4_chain_errors reports it), so the kernel
// always ends.
//
// Memory: outputs are stored, and x is loaded, at device scope (cache policy
// sc1): a phase's outputs are written on one XCD and read as x on all
// eight, whose L2s are not coherent with each other (an x that no phase
// writes is loaded through the L2, where it stays between phases).  Before a workgroup
// signals a barrier after which a phase reads (or writes over) what an
// earlier phase stored, each of its waves has waited for its own stores.
// x that the phase just before does not write is loaded, and its prologue
// run, before the barrier, as the weights are.  x that no phase writes is
// prepared at the program's start: one workgroup per such phase runs the
// phase's x prologue and stores the int16 planes, group sums and scale
// (device scope); after one more grid barrier the phase only copies them
// into LDS.  The last workgroup to reach a barrier then starts its stream
// after a copy instead of a whole prologue.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "q4_stream.h"
#include "q4chain.h"

namespace q4k {

constexpr int kChainWaves = 16;               // waves per workgroup (one workgroup per CU)
constexpr int kChainGroup = 32;               // workgroups per barrier counter
constexpr int kChainMaxGroups = 16;
constexpr int kChainRounds = 3;               // words of x per thread: n_in <= 3 * 1024 * 8
constexpr int kChainMaxIn = kChainRounds * kChainWaves * 64 * 8;
constexpr size_t kChainLdsFloor = 81 * 1024;  // > half the CU's LDS: one workgroup per CU
constexpr int kStoreDevice = 16;              // cache policy sc1: device-scope coherent
constexpr long long kChainSpinTicks = 2000000;  // 20 ms of the 100 MHz clock per barrier wait
// Event times a plan can record (q4_chain_stamps), per phase and workgroup,
// kChainStamps words each: 1 the workgroup done with the phase before (its
// waves' stores complete) and arriving at the barrier, 2 the barrier
// released, 3 x staged in LDS, 4 the int16 planes ready, 5 wave 0 done with
// its items.  Kept in LDS during the phase (words 2..5) and written out by
// thread 0 at the next arrival.
constexpr int kChainStamps = 8;
constexpr int kChainLdsHead = 80;             // the failure flag, then 8 event words

struct ChainPhase {
    MatList ml;
    const float* x;
    int n_in;
    int UB;          // rows per unit
    int ring;        // ring size: 1, 2, 4 or 5, dividing the unit's items
    int pair;        // gate/up: out[0] = SiLU(W0 x) * (W1 x)
    int n_total;     // rows of the phase: n_out[0] (pair) or the sum of n_out
    int sep_stage;   // x staged for the group sums in LDS of its own (else over the planes)
    int x_early;     // the phase before does not write x: x and its prologue before the barrier (ring 2)
    int x_cached;    // no phase writes x: x loaded through the L2
    int ack_stores;  // every wave's stores complete before the arrival at the next barrier
    const uint4* prep;   // x prepared at the program's start (prep_bytes), or null
};

using v4u32 = unsigned int __attribute__((__vector_size__(16)));

// How a phase gets its x planes: loaded and quantised after its barrier, or
// before it (the phase before does not write x), or prepared once at the
// program's start (no phase writes x) and only copied into LDS.
constexpr int kXLate = 0, kXEarly = 1, kXPrep = 2;

// A prepared x: the int16 planes in the LDS layout ([C][256] words of 16
// bytes, swizzled as the prologue stores them), the group sums [Gr] and the
// x scale, padded to 256 bytes.
__host__ __device__ constexpr size_t prep_bytes(int C, int Gr) {
    return (static_cast<size_t>(C) * 256 * 16 + static_cast<size_t>(Gr) * 4 + 16 + 255) & ~static_cast<size_t>(255);
}

// Barrier state, every word on its own 128-byte line.  Zero between launches:
// the last workgroup to leave resets it.
struct ChainSync {
    unsigned group[kChainMaxGroups][32];     // arrivals of the workgroups of group g
    unsigned exited[32];
    unsigned errors[32];
};

// The phase table is read through the constant address space: the host
// writes it once, so its words may be read with scalar loads whenever they
// are needed (as kernel arguments are), instead of being held in SGPRs for
// the whole phase.
#define Q4_CONST_AS __attribute__((address_space(4)))
typedef const Q4_CONST_AS ChainPhase CPhase;

__device__ __forceinline__ int c_mat_of_row(CPhase* ph, int gr) {
    int p = 0;
#pragma unroll
    for (int k = 1; k < kMaxMats; k++) p += (k < ph->ml.count && gr >= ph->ml.row_begin[k]) ? 1 : 0;
    return p;
}

// unit_rows of q4_stream.h over a phase-table entry
template <bool PAIR>
__device__ __forceinline__ void c_unit_rows(UnitRows& ur, CPhase* ph, int unit, int UB, int wpr, int G) {
    const int gr = unit * UB;
    if constexpr (PAIR) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            ur.w[k] = ph->ml.w[k] + static_cast<size_t>(gr) * wpr;
            ur.s[k] = ph->ml.s[k] + static_cast<size_t>(gr) * G;
            ur.b[k] = ph->ml.b[k] + static_cast<size_t>(gr) * G;
        }
    } else {
        const int p = __builtin_amdgcn_readfirstlane(c_mat_of_row(ph, gr));
        const int o = __builtin_amdgcn_readfirstlane(
            gr - sel4(p, ph->ml.row_begin[0], ph->ml.row_begin[1], ph->ml.row_begin[2], ph->ml.row_begin[3]));
        auto pk = [&](auto const Q4_CONST_AS(&a)[kMaxMats]) {
            return sel4(p, reinterpret_cast<uint64_t>(a[0]), reinterpret_cast<uint64_t>(a[1]),
                        reinterpret_cast<uint64_t>(a[2]), reinterpret_cast<uint64_t>(a[3]));
        };
        ur.w[0] = reinterpret_cast<const uint32_t*>(pk(ph->ml.w)) + static_cast<size_t>(o) * wpr;
        ur.s[0] = reinterpret_cast<const uint16_t*>(pk(ph->ml.s)) + static_cast<size_t>(o) * G;
        ur.b[0] = reinterpret_cast<const uint16_t*>(pk(ph->ml.b)) + static_cast<size_t>(o) * G;
    }
}

// Workgroup barrier that orders LDS only: a full __syncthreads would also
// wait for this wave's outstanding global loads -- the next phase's weights.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ void wait_own_stores() {
    // vmcnt(0), expcnt and lgkmcnt left alone (gfx9 encoding)
    __builtin_amdgcn_s_waitcnt(0x0F70);
}

// Event e of the current phase, in LDS (thread 0).
__device__ __forceinline__ void chain_event(unsigned long long* stamps, unsigned long long* st, int e) {
    if (stamps && threadIdx.x == 0) st[e] = __builtin_amdgcn_s_memrealtime();
}

// The phase's events out of LDS, and event 1 (the arrival) of phase p + 1.
__device__ __forceinline__ void chain_flush_events(unsigned long long* stamps, const unsigned long long* st, int p) {
    if (stamps && threadIdx.x == 0) {
        unsigned long long* row = stamps + (static_cast<size_t>(p) * gridDim.x + blockIdx.x) * kChainStamps;
        for (int e = 2; e <= 5; e++) row[e] = st[e];
        stamps[(static_cast<size_t>(p + 1) * gridDim.x + blockIdx.x) * kChainStamps + 1] =
            __builtin_amdgcn_s_memrealtime();
    }
}

// Workgroup b's arrival at barrier k (after phase k-1): every wave has waited
// for its stores; one atomic per workgroup, no return value needed.
__device__ __forceinline__ void chain_arrive(ChainSync* s, unsigned long long* stamps, const unsigned long long* st,
                                             int p) {
    lds_barrier();
    chain_flush_events(stamps, st, p);
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(&s->group[blockIdx.x / kChainGroup][0], 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until every workgroup has arrived at barrier k: lane g of wave 0
// polls group g's counter.  Bounded: past kChainSpinTicks the workgroup
// records an error and stops waiting at this and every later barrier.
__device__ __forceinline__ void chain_wait(ChainSync* s, unsigned k, int* failed) {
    if (threadIdx.x < 64) {                                      // wave 0
        const int lane = threadIdx.x;
        const int ng = (gridDim.x + kChainGroup - 1) / kChainGroup;
        const bool active = lane < ng;
        const unsigned gsz = active ? min(kChainGroup, static_cast<int>(gridDim.x) - lane * kChainGroup) : 0u;
        const unsigned target = k * gsz;
        if (!*failed) {
            const long long t0 = __builtin_amdgcn_s_memrealtime();
            for (;;) {
                const unsigned v = active ? __hip_atomic_load(&s->group[lane][0], __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT)
                                          : 0u;
                if (__builtin_amdgcn_ballot_w64(v < target) == 0) break;
                if (__builtin_amdgcn_s_memrealtime() - t0 > kChainSpinTicks) {
                    if (lane == 0) {
                        __hip_atomic_fetch_add(&s->errors[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        *failed = 1;
                    }
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
    }
    lds_barrier();
}

// Thread t's words t, t + nt, t + 2nt of x (8 floats each), device-scope
// loads unless no phase of the program writes x (cached).
__device__ __forceinline__ void chain_load_x(float4 (&wv)[kChainRounds][2], const float* x, int n_in, bool cached) {
    constexpr int nt = 64 * kChainWaves;
    const int wpr = n_in >> 3;
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(x, static_cast<uint32_t>(n_in) * 4u);
#pragma unroll
    for (int r = 0; r < kChainRounds; r++) {
        const int j = r * nt + threadIdx.x;
        const uint32_t off = j < wpr ? static_cast<uint32_t>(8 * j) * 4u : kOutOfRange;
        if (cached) {
            wv[r][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
            wv[r][1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16, 0, 0));
        } else {
            wv[r][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, kStoreDevice));
            wv[r][1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16, 0, kStoreDevice));
        }
    }
}

// The x prologue's first half, as the streaming kernel's: the unit counter
// zeroed, x staged in LDS, max |x| per wave (kernel/q4gemv.c:258-259) and,
// after a barrier, the group sums in ascending order (:244-248), one lane
// per group.
__device__ __forceinline__ void chain_sums(const float4 (&wv)[kChainRounds][2], int wpr, int G, float* xsum_lds,
                                           float* red, float* xstage, int* claim_ctr, unsigned long long* stamps,
                                           unsigned long long* st) {
    constexpr int WPG = 8;                                        // packed words per group
    constexpr int nt = 64 * kChainWaves;
    constexpr int SS = stage_stride(0);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (tid == 0) *claim_ctr = 0;
    float amax = 0.0f;
#pragma unroll
    for (int r = 0; r < kChainRounds; r++) {
        if (r * nt + wave * 64 < wpr) {                           // uniform: the wave has words this round
            const float4 a = wv[r][0], b = wv[r][1];
            amax = fmaxf(amax, fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                                     fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w)))));
            const int j = r * nt + tid;
            if (j < wpr) {
                float4* dst = reinterpret_cast<float4*>(xstage + (j / WPG) * SS + (j % WPG) * 8);
                dst[0] = a;
                dst[1] = b;
            }
        }
    }
    amax = wave_max(amax);
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    chain_event(stamps, st, 3);
    for (int g = tid; g < G; g += nt)
        xsum_lds[g] = chain_add<32>(chain_add<32>(0.0f, xstage + g * SS), xstage + g * SS + 32);
}

// The second half: the x scale (kernel/q4gemv.c:260-261) and int16 x
// (:262-270) as byte planes in LDS, word j of chunk c at
// c*256 + (j%4)*64 + (j%256)/4.  Returns the x scale.
__device__ __forceinline__ float chain_quant(const float4 (&wv)[kChainRounds][2], int wpr, int C, const float* red,
                                             uint4* xpl) {
    constexpr int nt = 64 * kChainWaves;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    float a = 0.0f;
    for (int i = 0; i < kChainWaves; i++) a = fmaxf(a, red[i]);
    const float xsc = a > 0.0f ? __fdiv_rn(a, 32767.0f) : 1.0f;   // kernel/q4gemv.c:260
    const float inv = __fdiv_rn(1.0f, xsc);                        // :261
    const bool exact_clamp = __builtin_isinf(inv);
#pragma unroll
    for (int r = 0; r < kChainRounds; r++) {
        const int j = r * nt + tid;
        if (r * nt + wave * 64 < C * kChunkWords) {               // uniform
            uint4 pl = make_uint4(0, 0, 0, 0);
            if (r * nt + wave * 64 < wpr) {                       // uniform
                const float vv[8] = {wv[r][0].x, wv[r][0].y, wv[r][0].z, wv[r][0].w,
                                     wv[r][1].x, wv[r][1].y, wv[r][1].z, wv[r][1].w};
                pl = exact_clamp ? quant_word(vv, inv, true) : quant_word(vv, inv, false);
                if (j >= wpr) pl = make_uint4(0, 0, 0, 0);
            }
            const int cc = j >> 8, jj = j & 255;
            xpl[cc * 256 + (jj & 3) * 64 + (jj >> 2)] = pl;
        }
    }
    return xsc;
}

// The program's first stage: phase ph's x through the whole prologue (as
// the phase itself would run it), then its planes, group sums and scale
// stored to ph->prep at device scope.  Every phase that reads it copies them
// after the barrier that ends this stage.
__device__ __forceinline__ void chain_prepare(CPhase* ph, uint4* lds4) {
    constexpr int nt = 64 * kChainWaves;
    const int n_in = ph->n_in;
    const int wpr = n_in >> 3, G = n_in >> 6;
    const int C = (wpr + kChunkWords - 1) / kChunkWords;
    const int Gr = (G + 3) & ~3;
    const int NU = ph->pair ? 2 * ph->UB : ph->UB;
    float* xsum_lds = reinterpret_cast<float*>(lds4);
    float* red = xsum_lds + Gr;
    int* claim_ctr = reinterpret_cast<int*>(red + 16);
    uint4* xpl = reinterpret_cast<uint4*>(red + 16 + 4 + 16);
    const bool sep = ph->sep_stage;
    float* xstage = sep ? reinterpret_cast<float*>(xpl + C * 256) + kChainWaves * NU * kTermStride
                        : reinterpret_cast<float*>(xpl);
    float4 wv[kChainRounds][2];
    chain_load_x(wv, ph->x, n_in, ph->x_cached);
    chain_sums(wv, wpr, G, xsum_lds, red, xstage, claim_ctr, nullptr, nullptr);
    if (!sep) __syncthreads();
    const float xsc = chain_quant(wv, wpr, C, red, xpl);
    __syncthreads();
    const int tid = threadIdx.x;
    const __amdgpu_buffer_rsrc_t sr = buf_rsrc(ph->prep, static_cast<uint32_t>(prep_bytes(C, Gr)));
    for (int i = tid; i < C * 256; i += nt)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32, xpl[i]), sr, static_cast<uint32_t>(i) * 16u,
                                               0, kStoreDevice);
    if (tid < Gr / 4)
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(v4u32, reinterpret_cast<const float4*>(xsum_lds)[tid]), sr,
            static_cast<uint32_t>(C * 256 * 16 + tid * 16), 0, kStoreDevice);
    if (tid == 0)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, xsc), sr,
                                              static_cast<uint32_t>(C * 256 * 16 + Gr * 4), 0, kStoreDevice);
    __syncthreads();                                              // the LDS is read: the next user may write it
}

// One phase.  The body follows gemv_stream_kernel<1, RW, PAIR, RING, false, 0>
// (q4_stream.h) step for step; the differences: the whole first ring is
// issued before the barrier and the x loads, x is loaded and the outputs
// stored at device scope, the rounds of x words are guarded at run time,
// and the phase ends with the waves' stores complete and the workgroup's
// arrival at the next barrier.  Barrier k is the k-th arrival of every
// workgroup: base (1 when the program starts with a preparation stage, else
// 0) plus the phases before.
template <int RING, bool PAIR, int XM>
__device__ __forceinline__ void chain_phase(CPhase* ph, int p, int base, ChainSync* sync,
                                            int* failed, uint4* lds4, bool arrive_after,
                                            unsigned long long* stamps, unsigned long long* st) {
    constexpr int lpg = 2;                                        // lanes per group in an item
    constexpr int WPG = 8;                                        // packed words per group
    const float* __restrict__ x = ph->x;
    const int n_in = ph->n_in, UB = ph->UB;
    const int wpr = n_in >> 3, G = n_in >> 6;
    const int C = (wpr + kChunkWords - 1) / kChunkWords;
    const int Gr = (G + 3) & ~3;
    // the launch shape is fixed: blockDim.x would be a 16-bit load from the
    // dispatch packet, a vector-memory round trip (and a wait for every
    // store still in flight) at the start of every phase
    constexpr int nt = 64 * kChainWaves;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nwaves = nt >> 6;
    // the streaming kernel's LDS layout for one row (stream_lds_bytes)
    float* xsum_lds = reinterpret_cast<float*>(lds4);             // [Gr]
    float* red = xsum_lds + Gr;                                   // [16]
    int* claim_ctr = reinterpret_cast<int*>(red + 16);
    uint4* xpl = reinterpret_cast<uint4*>(red + 16 + 4 + 16);     // [C*256] swizzled
    const int NU = PAIR ? 2 * UB : UB;
    float* Tw = reinterpret_cast<float*>(xpl + C * 256) + wave * (NU * kTermStride);   // [NU][kTermStride]
    // x staged for the group sums ([G][stage_stride(0)], the prologue only):
    // after every wave's term table when it fits (sep_stage), so the planes
    // may be written while the sums still read it; else over the planes,
    // which then wait for a barrier after the sums
    const bool sep = ph->sep_stage;                               // uniform
    float* xstage = sep ? reinterpret_cast<float*>(xpl + C * 256) + nwaves * NU * kTermStride
                        : reinterpret_cast<float*>(xpl);
    const int n_total = ph->n_total;
    const int n_units = (n_total + UB - 1) / UB;
    const int items = NU * C;
    const int grid = gridDim.x;
    const int first_unit = blockIdx.x + wave * grid;
    const bool has_work = first_unit < n_units;                   // uniform

    // ---- 1. x, first when the phase before does not write it (kXEarly):
    //         then x does not depend on that phase either, and its loads
    //         and the whole prologue run before the barrier as the weights'
    //         do.  x loads are the wave's oldest then, so the prologue waits
    //         for them alone, not for the weights issued after them (a code
    //         path of its own: one shared with the other order would wait
    //         for both).  A prepared x (kXPrep) is loaded the same way, as
    //         its planes, group sums and scale; phase 0 first waits for the
    //         stage that prepared it.
    float4 wv[kChainRounds][2];
    uint4 pv[kChainRounds];
    float4 gv;
    float xsc_v;
    if constexpr (XM == kXEarly) chain_load_x(wv, x, n_in, ph->x_cached);
    if constexpr (XM == kXPrep) {
        if (p == 0) {
            chain_wait(sync, static_cast<unsigned>(base), failed);
            chain_event(stamps, st, 2);
        }
        // through the L2: the stage before the barrier wrote the prepared x
        // at device scope, and no L2 holds a line of it from before (none is
        // read before that barrier, and the launch starts with the L2s
        // coherent), so the first workgroup of an XCD fetches it and the
        // others hit
        const int n_pl = C * 256;
        const __amdgpu_buffer_rsrc_t sr = buf_rsrc(ph->prep, static_cast<uint32_t>(prep_bytes(C, Gr)));
#pragma unroll
        for (int r = 0; r < kChainRounds; r++) {
            const int j = r * nt + tid;
            const uint32_t off = j < n_pl ? static_cast<uint32_t>(j) * 16u : kOutOfRange;
            pv[r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(sr, off, 0, 0));
        }
        const uint32_t goff = tid < Gr / 4 ? static_cast<uint32_t>(n_pl * 16 + tid * 16) : kOutOfRange;
        gv = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(sr, goff, 0, 0));
        xsc_v = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                              sr, static_cast<uint32_t>(n_pl * 16 + Gr * 4), 0, 0));
    }

    // ---- 2. the first ring of this phase: weights only, no dependency
    Item ring[RING];
    const uint32_t vo_w = static_cast<uint32_t>(lane) * 16u, vo_g = static_cast<uint32_t>(lane >> 1) * 2u;
    int pf_unit = first_unit, pf_c = 0, pf_r = 0;
    UnitRows pf_rows;
    c_unit_rows<PAIR>(pf_rows, ph, pf_unit, UB, wpr, G);
#pragma unroll
    for (int d = 0; d < RING; d++) {
        load_item<PAIR, 0>(ring[d], pf_rows, pf_unit, pf_c, pf_r, UB, wpr, G, vo_w, vo_g, has_work);
        if (++pf_r == NU) { pf_r = 0; ++pf_c; }
    }

    // ---- 3. otherwise every workgroup must be done with the phase before
    //         (x is one of its outputs) before x is loaded
    if constexpr (XM == kXLate) {
        if (p > 0) chain_wait(sync, static_cast<unsigned>(p + base), failed);
        chain_event(stamps, st, 2);
        chain_load_x(wv, x, n_in, ph->x_cached);
    }

    // ---- 4. the x prologue (the unit counter is free again: every wave of
    //         the workgroup is past the phase before)
    auto claim = [&]() -> int {
        int v = 0;
        if (lane == 0) v = __hip_atomic_fetch_add(claim_ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return v + nwaves;                                        // lane 0's value counts
    };
    int claimed;
    float xsc;
    if constexpr (XM == kXPrep) {
        if (tid == 0) *claim_ctr = 0;
#pragma unroll
        for (int r = 0; r < kChainRounds; r++)
            if (r * nt + wave * 64 < C * 256) xpl[r * nt + tid] = pv[r];   // uniform: 256 words per chunk
        if (tid < Gr / 4) reinterpret_cast<float4*>(xsum_lds)[tid] = gv;
        xsc = xsc_v;
        __syncthreads();
        chain_event(stamps, st, 3);
        claimed = claim();
    } else {
        chain_sums(wv, wpr, G, xsum_lds, red, xstage, claim_ctr, stamps, st);
        if (!sep) __syncthreads();                                // the staging is read: the planes may overwrite it
        claimed = claim();
        xsc = chain_quant(wv, wpr, C, red, xpl);
        __syncthreads();
    }
    chain_event(stamps, st, 4);
    if constexpr (XM != kXLate) {
        if (p > 0) chain_wait(sync, static_cast<unsigned>(p + base), failed);
        if (XM == kXEarly || p > 0) chain_event(stamps, st, 2);
    }

    // ---- 5. the item stream (as gemv_stream_kernel)
    constexpr int GPC = kChunkWords / WPG;                        // groups per chunk
    auto consume = [&](const Item& itm, int c, int u) {
        const int lim = wpr - c * kChunkWords;                    // uniform
        const bool lead = (lane & (lpg - 1)) == lpg - 1;
        const bool in_row = lane * 4 < lim;
        const int gl = lane >> 1;
        const int g = c * GPC + gl;
        uint32_t xle[4], xlo[4], xhe[4], xho[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint4 pl = xpl[c * 256 + t * 64 + lane];
            xle[t] = pl.x; xlo[t] = pl.y; xhe[t] = pl.z; xho[t] = pl.w;
        }
        const uint32_t wd[4] = {itm.w.x, itm.w.y, itm.w.z, itm.w.w};
        int ah = 0;
        uint32_t al = 0;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t lo4 = wd[t] & 0x0F0F0F0Fu;              // values 8j+0,2,4,6
            const uint32_t hi4 = (wd[t] >> 4) & 0x0F0F0F0Fu;       // values 8j+1,3,5,7
            ah = __builtin_amdgcn_sdot4(static_cast<int>(lo4), static_cast<int>(xhe[t]), ah, false);
            ah = __builtin_amdgcn_sdot4(static_cast<int>(hi4), static_cast<int>(xho[t]), ah, false);
            al = __builtin_amdgcn_udot4(lo4, xle[t], al, false);
            al = __builtin_amdgcn_udot4(hi4, xlo[t], al, false);
        }
        const float sf = h2f(itm.s), bf = h2f(itm.b);
        const int part = group_sum(static_cast<int>(static_cast<uint32_t>(ah) * 256u + al), lpg);
        if (lead) {
            float term = 0.0f;                                    // +0.0 past the row end
            if (in_row) {
                const float dot = __fmul_rn(xsc, static_cast<float>(part));
                const float bx = __fmul_rn(bf, xsum_lds[g]);
                term = __builtin_fmaf(sf, dot, bx);
            }
            Tw[u * kTermStride + gl] = term;
        }
    };
    // running sums per row slot (lane), one chunk at a time (as the
    // streaming kernel)
    float row_acc = 0.0f;
    auto chunk_done = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        if (lane < NU) row_acc = chain_add<GPC>(row_acc, Tw + lane * kTermStride);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    };
    auto finish = [&](int unit) {
        const float acc = row_acc;
        const float up = PAIR ? __shfl(row_acc, (lane + UB) & 63) : 0.0f;
        row_acc = 0.0f;
        if (lane < UB) {
            const int uu = lane, gr = unit * UB + uu;
            if (gr < n_total) {
                if constexpr (PAIR) {
                    const __amdgpu_buffer_rsrc_t ro =
                        buf_rsrc(ph->ml.out[0], static_cast<uint32_t>(ph->ml.n_out[0]) * 4u);
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, silu_mul(acc, up)), ro,
                                                          gr * 4, 0, kStoreDevice);
                } else {
                    const int pm = __builtin_amdgcn_readfirstlane(c_mat_of_row(ph, unit * UB));
                    const int no = sel4(pm, ph->ml.n_out[0], ph->ml.n_out[1], ph->ml.n_out[2], ph->ml.n_out[3]);
                    const int rb = sel4(pm, ph->ml.row_begin[0], ph->ml.row_begin[1], ph->ml.row_begin[2],
                                        ph->ml.row_begin[3]);
                    float* op = reinterpret_cast<float*>(sel4(pm, reinterpret_cast<uint64_t>(ph->ml.out[0]),
                                                              reinterpret_cast<uint64_t>(ph->ml.out[1]),
                                                              reinterpret_cast<uint64_t>(ph->ml.out[2]),
                                                              reinterpret_cast<uint64_t>(ph->ml.out[3])));
                    const __amdgpu_buffer_rsrc_t ro = buf_rsrc(op, static_cast<uint32_t>(no) * 4u);
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc), ro, (gr - rb) * 4, 0,
                                                          kStoreDevice);
                }
            }
        }
    };
    if (has_work) {                                               // uniform
        const int cyc_per_unit = items / RING;
        int cyc_pf = 1;
        int cyc_cu = 0, cu_c = 0, cu_r = 0;
        int cu_unit = first_unit;
        auto next_unit = [&]() -> bool {
            const int u = blockIdx.x + __builtin_amdgcn_readfirstlane(claimed) * grid;
            if (u >= n_units) return false;
            pf_unit = u;
            c_unit_rows<PAIR>(pf_rows, ph, pf_unit, UB, wpr, G);
            pf_c = 0;
            pf_r = 0;
            cyc_pf = 0;
            claimed = claim();
            return true;
        };
        bool more = cyc_pf < cyc_per_unit || next_unit();
        while (more) {
#pragma unroll
            for (int d = 0; d < RING; d++) {
                consume(ring[d], cu_c, cu_r);
                __builtin_amdgcn_sched_barrier(0);
                load_item<PAIR, 0>(ring[d], pf_rows, pf_unit, pf_c, pf_r, UB, wpr, G, vo_w, vo_g, true);
                if (++pf_r == NU) { pf_r = 0; ++pf_c; }
                if (++cu_r == NU) { chunk_done(); cu_r = 0; ++cu_c; }
            }
            ++cyc_pf;
            if (++cyc_cu == cyc_per_unit) {
                finish(cu_unit);
                cu_unit = pf_unit;
                cyc_cu = 0;
                cu_c = 0;
                cu_r = 0;
            }
            more = cyc_pf < cyc_per_unit || next_unit();
        }
#pragma unroll
        for (int d = 0; d < RING; d++) {
            consume(ring[d], cu_c, cu_r);
            if (++cu_r == NU) { chunk_done(); cu_r = 0; ++cu_c; }
        }
        finish(cu_unit);
    }

    chain_event(stamps, st, 5);

    // ---- 6. the workgroup arrives at the next barrier (the LDS of this
    //         phase is free once every wave is past it), each wave's stores
    //         complete first where a later phase reads what was stored
    //         before that barrier (ack_stores); else the stores only need to
    //         be complete at the kernel's end, which they are
    if (ph->ack_stores) wait_own_stores();
    if (arrive_after) {
        chain_arrive(sync, stamps, st, p);
    } else {
        lds_barrier();
        chain_flush_events(stamps, st, p);
    }
}

__global__ __launch_bounds__(64 * kChainWaves) void gemv_chain_kernel(const ChainPhase* __restrict__ phases,
                                                                      int n_phases, int prepare,
                                                                      ChainSync* __restrict__ sync,
                                                                      unsigned long long* __restrict__ stamps) {
    extern __shared__ uint4 lds_all[];
    int* failed = reinterpret_cast<int*>(lds_all);               // read and written by thread 0 only
    unsigned long long* st = reinterpret_cast<unsigned long long*>(lds_all + 1);   // this phase's events
    uint4* lds4 = lds_all + kChainLdsHead / 16;
    if (threadIdx.x == 0) *failed = 0;
    CPhase* table = (CPhase*)phases;
    // the preparation stage: workgroup b prepares the x of phases b, b + grid,
    // ... that take a prepared x, then arrives at barrier 1
    int base = 0;
    if (prepare) {
        for (int q = blockIdx.x; q < n_phases; q += gridDim.x)
            if (table[q].prep) chain_prepare(table + q, lds4);
        wait_own_stores();
        lds_barrier();
        if (threadIdx.x == 0)
            __hip_atomic_fetch_add(&sync->group[blockIdx.x / kChainGroup][0], 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        base = 1;
    }
    for (int p = 0; p < n_phases; p++) {
        CPhase* ph = table + p;
        const int pair = ph->pair, ring = ph->ring;                  // uniform
        const int xm = ph->prep ? kXPrep : ph->x_early ? kXEarly : kXLate;
        const bool arrive = p + 1 < n_phases;
        if (pair) {
            if (ring == 4) chain_phase<4, true, kXLate>(ph, p, base, sync, failed, lds4, arrive, stamps, st);
            else if (xm == kXPrep) chain_phase<2, true, kXPrep>(ph, p, base, sync, failed, lds4, arrive, stamps, st);
            else if (xm == kXEarly) chain_phase<2, true, kXEarly>(ph, p, base, sync, failed, lds4, arrive, stamps, st);
            else chain_phase<2, true, kXLate>(ph, p, base, sync, failed, lds4, arrive, stamps, st);
        } else if (ring == 1) {
            chain_phase<1, false, kXLate>(ph, p, base, sync, failed, lds4, arrive, stamps, st);
        } else if (ring == 2) {
            if (xm == kXPrep) chain_phase<2, false, kXPrep>(ph, p, base, sync, failed, lds4, arrive, stamps, st);
            else if (xm == kXEarly) chain_phase<2, false, kXEarly>(ph, p, base, sync, failed, lds4, arrive, stamps, st);
            else chain_phase<2, false, kXLate>(ph, p, base, sync, failed, lds4, arrive, stamps, st);
        } else if (ring == 4) {
            chain_phase<4, false, kXLate>(ph, p, base, sync, failed, lds4, arrive, stamps, st);
        } else {
            chain_phase<5, false, kXLate>(ph, p, base, sync, failed, lds4, arrive, stamps, st);
        }
    }
    // every workgroup is past its last barrier wait once it gets here; the
    // last one to leave returns the counters to zero for the next launch
    if (threadIdx.x == 0) {
        const unsigned left = __hip_atomic_fetch_add(&sync->exited[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (left == gridDim.x - 1) {
            for (int g = 0; g < kChainMaxGroups; g++)
                __hip_atomic_store(&sync->group[g][0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&sync->exited[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace q4k

using namespace q4k;

struct q4_chain_plan {
    int device = 0;
    int n_phases = 0;
    int grid = 0;
    size_t lds = 0;
    int prepare = 0;             // phases with a prepared x: the program starts with their preparation
    unsigned long long* stamps = nullptr;
    ChainPhase* d_phases = nullptr;
    ChainSync* d_sync = nullptr;
    void* d_prep = nullptr;      // the prepared x of those phases
};

namespace {

// Whether phase `ph` writes any byte of [lo, hi) (every out[k] of its
// matrices counts as written, out[1] of a gate/up pair too).
bool phase_writes(const q4_chain_phase& ph, uintptr_t lo, uintptr_t hi) {
    for (int k = 0; k < ph.count; k++) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(ph.out[k]);
        const uintptr_t b = a + static_cast<uintptr_t>(ph.n_out[k]) * 4u;
        if (a < hi && lo < b) return true;
    }
    return false;
}

// Rows per unit and ring size of a phase, as launch_stream picks them for
// one row at 16 waves per CU.
int plan_phase(const q4_chain_phase& in, ChainPhase& out, int cus, size_t& lds) {
    std::memset(&out, 0, sizeof(out));
    const int count = in.count;
    if (in.pair ? count != 2 : (count < 1 || count > kMaxMats))
        return fail(Q4_EARG, "count=%d (1..%d; 2 with pair)", count, kMaxMats);
    if (!in.x) return fail(Q4_EARG, "null x");
    if (reinterpret_cast<uintptr_t>(in.x) & 15) return fail(Q4_EARG, "x must be 16-byte aligned");
    if (in.gs != 64) return fail(Q4_EARG, "gs=%d: the chained program takes group size 64", in.gs);
    if (in.n_in <= 0 || in.n_in % 64 || in.n_in > kChainMaxIn)
        return fail(Q4_EARG, "n_in=%d (a positive multiple of 64, at most %d)", in.n_in, kChainMaxIn);
    int rb = 0;
    for (int k = 0; k < count; k++) {
        if (!in.w[k] || !in.scales[k] || !in.biases[k] || !in.out[k])
            return fail(Q4_EARG, "null pointer in matrix %d", k);
        if (reinterpret_cast<uintptr_t>(in.w[k]) & 15) return fail(Q4_EARG, "w[%d] must be 16-byte aligned", k);
        if (in.n_out[k] <= 0) return fail(Q4_EARG, "n_out[%d]=%d", k, in.n_out[k]);
        out.ml.w[k] = in.w[k];
        out.ml.s[k] = in.scales[k];
        out.ml.b[k] = in.biases[k];
        out.ml.out[k] = in.out[k];
        out.ml.n_out[k] = in.n_out[k];
        out.ml.row_begin[k] = rb;
        rb += in.n_out[k];
    }
    if (in.pair && in.n_out[0] != in.n_out[1]) return fail(Q4_EARG, "pair: n_out %d != %d", in.n_out[0], in.n_out[1]);
    {
        // a workgroup may store its rows while another still loads x
        const uintptr_t lo = reinterpret_cast<uintptr_t>(in.x);
        if (phase_writes(in, lo, lo + static_cast<uintptr_t>(in.n_in) * 4u))
            return fail(Q4_EARG, "an output overlaps x");
    }
    for (int k = count; k <= kMaxMats; k++) out.ml.row_begin[k] = rb;
    out.ml.count = count;
    out.ml.mrows = 1;
    out.x = in.x;
    out.n_in = in.n_in;
    out.pair = in.pair ? 1 : 0;
    const int C = (in.n_in / 8 + kChunkWords - 1) / kChunkWords;
    const int G = in.n_in / 64;
    const int n_total = in.pair ? in.n_out[0] : rb;
    out.n_total = n_total;
    const int mult = in.pair ? 2 : 1;
    int UB = 1;
    while (UB < 8 && UB * C * mult < kUnitItems && n_total >= 4 * UB * kChainWaves * cus) UB *= 2;
    for (int k = 0; k < count; k++)
        while (in.n_out[k] % UB) UB >>= 1;
    const int items = mult * UB * C;
    int ring = 0;
    // two items in flight per wave where they divide the unit: deeper
    // rings measured slower (more loads queued per CU)
    if (items % 2 == 0) ring = 2;
    else if (!in.pair && items % 5 == 0) ring = 5;
    else if (!in.pair) ring = 1;
    if (!ring) return fail(Q4_EARG, "no ring size divides %d items", items);
    out.UB = UB;
    out.ring = ring;
    // the x staging in LDS of its own when it fits beside the planes and
    // every wave's term table: one barrier fewer in the x prologue (the
    // sweep 1.248 -> 1.227 ms, same box)
    const size_t shared = kChainLdsHead + stream_lds_bytes(1, C, G, kChainWaves, mult * UB, kChainRounds, 0);
    const size_t header = static_cast<size_t>((G + 3) & ~3) * 4 + 16 * 4 + 16 + 64;
    const size_t separate = kChainLdsHead + header + static_cast<size_t>(C) * 256 * 16 +
                            static_cast<size_t>(kChainWaves) * mult * UB * kTermStride * 4 +
                            static_cast<size_t>(G) * stage_stride(0) * 4;
    out.sep_stage = separate <= kStreamLdsMax ? 1 : 0;
    const size_t need = out.sep_stage ? separate : shared;
    if (need > lds) lds = need;
    return 0;
}

// What each barrier must order, from the buffers the phases read and write:
//  - x_early[j]: phase j-1 writes no byte of x_j, so x_j may be loaded (and
//    its prologue run) before barrier j; every phase before j-1 is past
//    barrier j-1 by then.  Only the ring-2 phases have that code path; the
//    others load x after the barrier, which orders at least as much.
//  - x_cached[j]: no phase writes x_j, so the L2 of any XCD holds no stale
//    copy of it (the launch starts with the L2s coherent).
//  - ack_stores[b-1]: the waves wait for their stores before arriving at
//    barrier b when a read or a write after b must see them: x_j written by
//    an earlier phase is read after barrier j (j-1 when early), and a phase
//    writing what an earlier phase wrote stores after its own barrier.
void plan_dependencies(const q4_chain_phase* in, std::vector<ChainPhase>& out) {
    const int n = static_cast<int>(out.size());
    for (int j = 0; j < n; j++) {
        const uintptr_t lo = reinterpret_cast<uintptr_t>(in[j].x);
        const uintptr_t hi = lo + static_cast<uintptr_t>(in[j].n_in) * 4u;
        out[j].x_early = out[j].ring == 2 && (j == 0 || !phase_writes(in[j - 1], lo, hi));
        bool read_dep = false, write_dep = false;
        out[j].x_cached = 1;
        for (int i = 0; i < n && out[j].x_cached; i++)
            if (phase_writes(in[i], lo, hi)) out[j].x_cached = 0;
        for (int i = 0; i < j; i++) {
            read_dep = read_dep || phase_writes(in[i], lo, hi);
            for (int k = 0; k < in[j].count && !write_dep; k++) {
                const uintptr_t a = reinterpret_cast<uintptr_t>(in[j].out[k]);
                write_dep = phase_writes(in[i], a, a + static_cast<uintptr_t>(in[j].n_out[k]) * 4u);
            }
        }
        // a read before barrier j-1 needs phase j-2's stores at the latest,
        // whose arrival is barrier j-1: the arrival after phase j-2
        if (read_dep) out[out[j].x_early ? j - 2 : j - 1].ack_stores = 1;
        if (write_dep) out[j - 1].ack_stores = 1;
    }
}

}  // namespace

#pragma GCC visibility push(default)
extern "C" {

int q4_chain_create(const q4_chain_phase* phases, int n_phases, q4_chain_plan** plan) {
    if (!plan) return fail(Q4_EARG, "null plan");
    *plan = nullptr;
    if (!phases || n_phases <= 0) return fail(Q4_EARG, "n_phases=%d", n_phases);
    std::vector<ChainPhase> host(n_phases);
    size_t lds = kChainLdsFloor;
    // arguments first, before any device call (launch shapes for one CU)
    for (int p = 0; p < n_phases; p++) {
        if (int rc = plan_phase(phases[p], host[p], 1, lds)) {
            char why[400];
            std::snprintf(why, sizeof(why), "%s", q4_last_error());
            return fail(rc, "phase %d: %s", p, why);
        }
    }
    const int cus = num_cus();
    if (cus <= 0) return fail(Q4_EHIP, "no device");
    if ((cus + kChainGroup - 1) / kChainGroup > kChainMaxGroups) return fail(Q4_EARG, "%d CUs", cus);
    lds = kChainLdsFloor;
    for (int p = 0; p < n_phases; p++) {
        if (int rc = plan_phase(phases[p], host[p], cus, lds)) {
            char why[400];
            std::snprintf(why, sizeof(why), "%s", q4_last_error());
            return fail(rc, "phase %d: %s", p, why);
        }
    }
    if (lds > kStreamLdsMax) return fail(Q4_EARG, "phases need %zu bytes of LDS", lds);
    plan_dependencies(phases, host);
    // an x that no phase writes is prepared once, at the program's start, by
    // one workgroup per phase (ring-2 phases: the code path exists for those)
    std::vector<size_t> prep_off(n_phases, SIZE_MAX);
    size_t prep_total = 0;
    for (int p = 0; p < n_phases; p++) {
        if (!host[p].x_cached || host[p].ring != 2) continue;
        const int wpr = host[p].n_in / 8, G = host[p].n_in / 64;
        prep_off[p] = prep_total;
        prep_total += prep_bytes((wpr + kChunkWords - 1) / kChunkWords, (G + 3) & ~3);
    }
    static std::atomic<uint64_t> lds_raised{0};
    if (int rc = raise_lds_limit(reinterpret_cast<const void*>(gemv_chain_kernel), kStreamLdsMax, lds_raised))
        return rc;
    int per_cu = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_chain_kernel, 64 * kChainWaves, lds);
    if (e != hipSuccess || per_cu < 1)
        return fail(Q4_EHIP, "the chained kernel does not fit a CU (%s)", hipGetErrorString(e));
    int device = 0;
    e = hipGetDevice(&device);
    if (e != hipSuccess) return fail(Q4_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    auto* pl = new q4_chain_plan;
    pl->device = device;
    pl->n_phases = n_phases;
    pl->grid = cus;
    pl->lds = lds;
    e = hipMalloc(&pl->d_phases, sizeof(ChainPhase) * n_phases);
    if (e == hipSuccess) e = hipMalloc(&pl->d_sync, sizeof(ChainSync));
    if (e == hipSuccess && prep_total) e = hipMalloc(&pl->d_prep, prep_total);
    if (e == hipSuccess && prep_total) {
        pl->prepare = 1;
        for (int p = 0; p < n_phases; p++)
            if (prep_off[p] != SIZE_MAX)
                host[p].prep = reinterpret_cast<const uint4*>(static_cast<char*>(pl->d_prep) + prep_off[p]);
    }
    if (e == hipSuccess) e = hipMemcpy(pl->d_phases, host.data(), sizeof(ChainPhase) * n_phases, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(pl->d_sync, 0, sizeof(ChainSync));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(pl->d_phases);
        (void)hipFree(pl->d_sync);
        (void)hipFree(pl->d_prep);
        delete pl;
        return fail(e == hipErrorOutOfMemory ? Q4_ENOMEM : Q4_EHIP, "chain plan: %s", hipGetErrorString(e));
    }
    *plan = pl;
    return 0;
}

int q4_chain_run(q4_chain_plan* plan, void* stream) {
    if (!plan) return fail(Q4_EARG, "null plan");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(Q4_EHIP, "hipGetDevice failed");
    if (dev != plan->device) return fail(Q4_EARG, "plan made on device %d, current device %d", plan->device, dev);
    hipLaunchKernelGGL(gemv_chain_kernel, dim3(plan->grid), dim3(64 * kChainWaves), plan->lds,
                       static_cast<hipStream_t>(stream), plan->d_phases, plan->n_phases, plan->prepare, plan->d_sync,
                       plan->stamps);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q4_EHIP, "chain launch: %s", hipGetErrorString(e));
    return 0;
}

int q4_chain_stamps(q4_chain_plan* plan, unsigned long long* stamps, long words) {
    if (!plan) return fail(Q4_EARG, "null plan");
    const long need = static_cast<long>(plan->n_phases + 1) * plan->grid * kChainStamps;
    if (stamps && words < need) return fail(Q4_EARG, "stamps: %ld words, the plan records %ld", words, need);
    plan->stamps = stamps;
    return 0;
}

int q4_chain_errors(q4_chain_plan* plan) {
    if (!plan) return fail(Q4_EARG, "null plan");
    unsigned n = 0;
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(&n, plan->d_sync->errors, sizeof(n), hipMemcpyDeviceToHost);
    // a wait that ran out may have left counters behind: start clean
    if (e == hipSuccess && n) e = hipMemset(plan->d_sync, 0, sizeof(ChainSync));
    if (e == hipSuccess && n) e = hipDeviceSynchronize();
    if (e != hipSuccess) return fail(Q4_EHIP, "chain errors: %s", hipGetErrorString(e));
    return static_cast<int>(n);
}

int q4_chain_destroy(q4_chain_plan* plan) {
    if (!plan) return 0;
    // free everything whatever fails; report the first failure
    hipError_t e = hipDeviceSynchronize();
    for (void* ptr : {static_cast<void*>(plan->d_phases), static_cast<void*>(plan->d_sync), plan->d_prep}) {
        const hipError_t f = hipFree(ptr);
        if (e == hipSuccess) e = f;
    }
    delete plan;
    if (e != hipSuccess) return fail(Q4_EHIP, "chain destroy: %s", hipGetErrorString(e));
    return 0;
}

}  // extern "C"
#pragma GCC visibility pop
