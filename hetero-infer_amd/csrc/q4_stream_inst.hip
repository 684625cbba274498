// Instances of the streaming GEMV kernel, one object per (activation rows,
// gate/up pair, ring size, group size), one-row objects with the norm
// prologue too: the build compiles this file once per -DQ4_MR=<1|2>
// -DQ4_PAIR=<0|1> -DQ4_RING=<1|2|5> -DQ4_GSH=<0|1> (group size 64 << GSH),
// in parallel.
#include "q4_stream.h"

#if !defined(Q4_MR) || !defined(Q4_PAIR) || !defined(Q4_RING) || !defined(Q4_GSH)
#error "define Q4_MR, Q4_PAIR, Q4_RING and Q4_GSH"
#endif

namespace q4k {

#define Q4_STREAM_INST(RW, NORM)                                                                      \
    template int launch_stream_k<Q4_MR, RW, static_cast<bool>(Q4_PAIR), Q4_RING, NORM, Q4_GSH>(      \
        const MatList&, const float*, const NormArgs&, int, int, int, size_t, int, int, hipStream_t);

Q4_STREAM_INST(1, false)
#if Q4_MR <= 4
Q4_STREAM_INST(2, false)
#endif
#if Q4_MR == 1 && Q4_PAIR == 0
Q4_STREAM_INST(3, false)
Q4_STREAM_INST(4, false)
#endif
#if Q4_MR == 1 && Q4_GSH == 0
Q4_STREAM_INST(1, true)   // the norm prologue: one row, one word per thread, group size 64
#endif

}  // namespace q4k
