/* Chained GEMV programs on MI355X (gfx950): a sequence of dependent
 * one-row GEMV phases -- the projections of a decode step, in order -- run
 * as ONE persistent launch.
 *
 * No counterpart in the reference's kernel ABI (kernel/q4gemv.c): the
 * reference's caller makes one q4_gemv call per projection per token
 * (hetero/cpu_model.py:269-275, :291-292, :367), each one a full round trip.
 * A phase here computes exactly what one q4_gemv_multi_dev (or, with `pair`,
 * q4_gate_up_silu_dev) call of one row computes, bit for bit; phase p
 * stores its outputs only after every workgroup has finished phase p-1, and
 * reads an x that phase p-1 writes only then, so a phase may read the
 * outputs of the phases before it.  Within the launch each wave issues the
 * weight loads of the next phase before it waits for that dependency, so the
 * weight stream does not pause at each one; an x that phase p-1 does not
 * write (found from the pointers at q4_chain_create) is loaded and
 * quantised before the wait too.  An x that no phase writes is quantised
 * once per phase at the program's start (its int16 planes, group sums and
 * scale, computed as the phase's own prologue computes them, into memory
 * the plan holds), and the phase only copies them, before its wait.  So x
 * must not change while the program runs, which no phase can do.  A
 * phase's outputs must not overlap its own x (Q4_EARG).
 *
 * All pointers are device pointers on the device current at q4_chain_create.
 * A plan holds its phase table, barrier state and the prepared x in device
 * memory (2 bytes per x element of each such phase, n_in rounded up to a
 * multiple of 2048, plus 4 per group); it runs
 * asynchronously on `stream` (a hipStream_t, NULL = the null stream), makes
 * no allocation or memset when it runs, and can be captured in a HIP graph.
 * One plan must not run on two streams at once (its barrier state is shared).
 *
 * Return codes as in q4gemv.h: 0 success, Q4_EHIP, Q4_ENOMEM, Q4_EARG (text in
 * q4_last_error()).
 */
#ifndef Q4CHAIN_H
#define Q4CHAIN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One phase: out[k][0..n_out[k]) = W_k x for count (1..4) matrices sharing
 * x[0..n_in), or with pair = 1 and count = 2 the gate/up pair,
 * out[0][i] = SiLU((W_0 x)[i]) * (W_1 x)[i] (out[1] unused).  gs must be 64,
 * n_in a multiple of 64 up to 24576, w and x 16-byte aligned. */
typedef struct {
    int count;
    int pair;
    const uint32_t *w[4];
    const uint16_t *scales[4];
    const uint16_t *biases[4];
    float *out[4];
    int n_out[4];
    const float *x;
    int n_in;
    int gs;
} q4_chain_phase;

typedef struct q4_chain_plan q4_chain_plan;

/* Check the phases, choose each one's launch shape and upload the table.
 * Synchronous.  *plan is NULL on failure. */
int q4_chain_create(const q4_chain_phase *phases, int n_phases, q4_chain_plan **plan);

/* Run every phase, in order, in one launch on `stream`. */
int q4_chain_run(q4_chain_plan *plan, void *stream);

/* Measurement: with `stamps` a device buffer of at least
 * (n_phases + 1) * workgroups * 8 words (workgroups = the device's CU count),
 * later runs record, for each phase p and workgroup b, the 100 MHz clock
 * (s_memrealtime) at stamps[(p * workgroups + b) * 8 + e] for the events
 * e = 1: the workgroup done with phase p - 1, arriving at the grid barrier
 * (every wave's stores complete when a later phase depends on them); 2: the
 * barrier released; 3: p's x staged in LDS (a prepared x: its planes, group
 * sums and scale copied into LDS); 4: p's int16 planes ready (3 and 4 come
 * before 2 when phase p - 1 does not write p's x); 5: wave 0 done with
 * its items of p (row n_phases holds event 1 only: the end).  NULL stops
 * recording.  Returns Q4_EARG when `words` is too small. */
int q4_chain_stamps(q4_chain_plan *plan, unsigned long long *stamps, long words);

/* Synchronise the device and return how many barrier waits ran out of time
 * since the last call (0 in a correct run; then clears the count and the
 * barrier state).  A run with a nonzero count produced invalid outputs. */
int q4_chain_errors(q4_chain_plan *plan);

/* Synchronise the device and free the plan (NULL is a no-op). */
int q4_chain_destroy(q4_chain_plan *plan);

#ifdef __cplusplus
}
#endif

#endif /* Q4CHAIN_H */
