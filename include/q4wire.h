/* Activation wire codec on MI355X (gfx950).
 *
 * A pipeline stage hands its hidden state to the next stage as a frame whose
 * payload is the activation encoded as fp16 or as int8 with one fp32 scale
 * per row (hetero/transport.py:193-225).  The reference encodes on the host
 * after copying the activation out of its backend; these entry points encode
 * the device-resident fp32 hidden state in HBM, so only the payload (half or
 * a quarter of the fp32 bytes) has to cross to the host, and decode a
 * received payload straight into a device fp32 hidden state.
 *
 * They fuse the NumPy backend's conversions either side of the codec
 * (hetero/backends.py:100-104), so on finite inputs, byte for byte:
 *   q4_wire_encode_dev(x)  == transport.encode(NumpyBackend.to_wire(x), codec)[1]
 *   q4_wire_decode_dev(p)  == NumpyBackend.from_wire(transport.decode(hdr, p))
 * The reference's output for NaN or infinite activations depends on the
 * host's float-to-int8 conversion; these calls give a fixed result for them
 * but do not claim to match it.
 *
 * All pointers are device pointers; calls are asynchronous on `stream` (a
 * hipStream_t, NULL = the null stream), allocate nothing and are capturable
 * in a HIP graph.  rows = 0 is a no-op.  Return codes as in q4gemv.h:
 * 0 success, Q4_EHIP, Q4_EARG (text in q4_last_error()).
 */
#ifndef Q4WIRE_H
#define Q4WIRE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* codec ids: the reference's codec names "fp16" and "int8"
 * (hetero/transport.py:200, :203; hetero/cli.py:27) */
#define Q4_WIRE_FP16 0
#define Q4_WIRE_INT8 1

/* Payload bytes of rows x hidden activations: 2*rows*hidden (fp16) or
 * 4*rows + rows*hidden (int8: the scales, then the rows;
 * hetero/transport.py:210-211, :220-222).  -1 for an unknown codec or a bad
 * shape.  Host-only arithmetic: no device access. */
long long q4_wire_payload_bytes(int codec, int rows, int hidden);

/* Replaces hetero/transport.py:198-211 (encode) applied to
 * hetero/backends.py:100-101 (to_wire) of an fp32 [rows][hidden] activation.
 * x fp32 [rows][hidden]; payload: q4_wire_payload_bytes bytes, 4-byte
 * aligned.  int8: hidden <= 32768. */
int q4_wire_encode_dev(const float* x, int rows, int hidden, int codec, void* payload, void* stream);

/* Replaces hetero/transport.py:214-225 (decode) followed by
 * hetero/backends.py:103-104 (from_wire): out fp32 [rows][hidden] =
 * fp32(fp16 value) (fp16 codec) or fp32(fp16(fp32(q) * scale)) (int8).
 * payload 4-byte aligned. */
int q4_wire_decode_dev(const void* payload, int rows, int hidden, int codec, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* Q4WIRE_H */
