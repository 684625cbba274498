/* CPU oracle for the fused int4 GEMV path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain scalar C, the arithmetic of the reference
 * kernel kernel/q4gemv.c as it runs on x86 (the AVX2/F16C/FMA build made by
 * kernel/build.sh with clang).  It is the checker that the HIP library is
 * compared against; nothing in the product links, loads or calls it.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
 *
 * Every function cites the reference lines it follows.  How each one is
 * pinned (golden vectors from the reference compiled from source, closed
 * forms, exhaustive checks) is listed in the tests that exercise it:
 *   tests/test_oracle.py.
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off; every fused
 * multiply-add of the reference is written as an explicit fmaf here, and no
 * other operation may be contracted).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* fp16 bit pattern -> fp32, exact, from the IEEE 754 binary16 definition:
 * subnormals are m * 2^-24, exponent 31 is inf/nan with the payload kept.
 * Follows the semantics of f16_to_f32, kernel/q4gemv.c:56-70 (F16C
 * _cvtsh_ss on x86, which is exact for every input). */
float oq_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 0) {
        float f = (float)m * 0x1p-24f;          /* exact: m < 2^10 */
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* The 4-bit value at position k of row o (MLX layout, low nibble first):
 * kernel/q4gemv.c:7-11, hetero/cpu_model.py:69-74. */
static inline uint32_t nib(const uint32_t *row, int k) {
    return (row[k >> 3] >> (4 * (k & 7))) & 0xFu;
}

/* The per-call x prologue of q4_gemv on x86, kernel/q4gemv.c:242-272:
 *   xsum[g]  sequential fp32 sum of group g            (:244-248)
 *   amax     max |x_i|                                  (:258-259)
 *   xscale   amax > 0 ? amax / 32767 : 1                (:260)
 *   inv      1 / xscale                                 (:261)
 *   xq[i]    (int16)(a < 0 ? a - 0.5 : a + 0.5), a = x[i]*inv  (:266-268)
 * xq is returned in natural index order (the reference stores it permuted
 * evens-then-odds per 64-block, :262-270, which changes no value). */
void oq_xprep(const float *x, int n_in, int gs, int16_t *xq, float *xsum,
              float *xscale_out) {
    const int n_groups = n_in / gs;
    for (int g = 0; g < n_groups; g++) {
        float s = 0.0f;
        for (int i = 0; i < gs; i++) s = s + x[g * gs + i];
        xsum[g] = s;
    }
    float amax = 0.0f;
    for (int i = 0; i < n_in; i++) {
        float v = x[i] < 0 ? -x[i] : x[i];
        if (v > amax) amax = v;
    }
    const float xscale = amax > 0.0f ? amax / 32767.0f : 1.0f;
    const float inv = 1.0f / xscale;
    for (int i = 0; i < n_in; i++) {
        float a = x[i] * inv;
        float r = a < 0 ? a - 0.5f : a + 0.5f;
        xq[i] = (int16_t)(int32_t)r;          /* truncation, as cvttss2si */
    }
    *xscale_out = xscale;
}

/* One output row by the integer path, kernel/q4gemv.c:158-183 with the hot
 * loop group_rows_i16 (:80-111):
 *   idot  = sum_{i in g} q_i * xq_i            exact int32
 *   dot   = xscale * (float)idot               (:173)
 *   acc   = acc + fma(scale, dot, bias*xsum[g])  (:179-180; clang contracts
 *           the first product into an fmuladd and keeps the += separate)   */
static float row_int(const uint32_t *row, const uint16_t *sc, const uint16_t *bi,
                     const int16_t *xq, const float *xsum, float xscale,
                     int n_in, int gs) {
    const int n_groups = n_in / gs;
    float acc = 0.0f;
    for (int g = 0; g < n_groups; g++) {
        /* int32 lanes that wrap, like _mm256_add_epi32 (only reachable for
           group sizes above 4368, where 15*32767*gs exceeds 2^31) */
        uint32_t acc_u = 0;
        for (int i = 0; i < gs; i++)
            acc_u += (uint32_t)((int32_t)nib(row, g * gs + i) * (int32_t)xq[g * gs + i]);
        const int32_t idot = (int32_t)acc_u;
        float dot = xscale * (float)idot;
        float b_x = oq_f16_to_f32(bi[g]) * xsum[g];
        acc = acc + fmaf(oq_f16_to_f32(sc[g]), dot, b_x);
    }
    return acc;
}

/* One output row by the fp32 path the reference uses for rows past the last
 * ROWS block, kernel/q4gemv.c:185-199:
 *   s   = fma(q, x, s) sequentially over the group    (:192-195)
 *   acc = acc + fma(scale, s, bias*xsum[g])           (:196-197)        */
static float row_f32(const uint32_t *row, const uint16_t *sc, const uint16_t *bi,
                     const float *x, const float *xsum, int n_in, int gs) {
    const int n_groups = n_in / gs;
    float acc = 0.0f;
    for (int g = 0; g < n_groups; g++) {
        float s = 0.0f;
        for (int i = 0; i < gs; i++)
            s = fmaf((float)nib(row, g * gs + i), x[g * gs + i], s);
        float b_x = oq_f16_to_f32(bi[g]) * xsum[g];
        acc = acc + fmaf(oq_f16_to_f32(sc[g]), s, b_x);
    }
    return acc;
}

/* q4_gemv, x86 semantics, kernel/q4gemv.c:232-301.  rows_block is the
 * reference build's ROWS: rows at index >= n_out - n_out % rows_block take
 * the fp32 tail path (:185-200); every other row takes the integer path.
 * Returns -1 exactly when the reference does (:237). */
int oq_q4_gemv(const uint32_t *w, const uint16_t *scales, const uint16_t *biases,
               const float *x, float *out, int n_out, int n_in, int gs,
               int rows_block) {
    if (gs <= 0 || n_in % gs || gs % 64) return -1;
    if (rows_block < 1) rows_block = 1;
    const int n_groups = n_in / gs, wpr = n_in / 8;
    int16_t *xq = (int16_t *)malloc(sizeof(int16_t) * (size_t)(n_in > 0 ? n_in : 1));
    float *xsum = (float *)malloc(sizeof(float) * (size_t)(n_groups > 0 ? n_groups : 1));
    float xscale;
    oq_xprep(x, n_in, gs, xq, xsum, &xscale);
    const int tail0 = n_out - n_out % rows_block;
    for (int o = 0; o < n_out; o++) {
        const uint32_t *row = w + (size_t)o * wpr;
        const uint16_t *sc = scales + (size_t)o * n_groups;
        const uint16_t *bi = biases + (size_t)o * n_groups;
        out[o] = o < tail0 ? row_int(row, sc, bi, xq, xsum, xscale, n_in, gs)
                           : row_f32(row, sc, bi, x, xsum, n_in, gs);
    }
    free(xq);
    free(xsum);
    return 0;
}

/* q4_dequant, kernel/q4gemv.c:316-379: rows [row0,row1) expanded to fp32
 * out[(o-row0)][i] = fma(q, scale, bias) (:331-334).  q*scale is exact in
 * fp32 (4-bit q times an 11-bit significand), so this equals q*scale+bias
 * with one rounding.  Returns -1 when the reference does (:361), 0 for an
 * empty range (:363). */
int oq_q4_dequant(const uint32_t *w, const uint16_t *scales, const uint16_t *biases,
                  float *out, int row0, int row1, int n_in, int gs) {
    if (gs <= 0 || n_in % gs || gs % 8) return -1;
    if (row1 - row0 <= 0) return 0;
    const int n_groups = n_in / gs, wpr = n_in / 8;
    for (int o = row0; o < row1; o++) {
        const uint32_t *row = w + (size_t)o * wpr;
        float *dst = out + (size_t)(o - row0) * n_in;
        for (int g = 0; g < n_groups; g++) {
            const float s = oq_f16_to_f32(scales[(size_t)o * n_groups + g]);
            const float b = oq_f16_to_f32(biases[(size_t)o * n_groups + g]);
            for (int i = 0; i < gs; i++)
                dst[g * gs + i] = fmaf((float)nib(row, g * gs + i), s, b);
        }
    }
    return 0;
}

/* Integer nibble unpack of rows [row0,row1) into bytes, [rows][n_in]:
 * the closed form (w >> 4j) & 0xF of kernel/q4gemv.c:7-11. */
void oq_unpack(const uint32_t *w, uint8_t *out, int row0, int row1, int n_in) {
    const int wpr = n_in / 8;
    for (int o = row0; o < row1; o++)
        for (int k = 0; k < n_in; k++)
            out[(size_t)(o - row0) * n_in + k] = (uint8_t)nib(w + (size_t)o * wpr, k);
}
