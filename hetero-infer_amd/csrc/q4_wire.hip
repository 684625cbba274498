// Activation wire codec on the GPU (gfx950): the hidden state a pipeline
// stage hands to the next one, encoded where it lives (HBM) so that only the
// payload crosses to the host.  Declared in q4wire.h.
//
// The reference encodes on the host (hetero/transport.py:198-225) after the
// NumPy backend's to_wire (hetero/backends.py:100-101: fp32 -> fp16) and
// decodes before its from_wire (:103-104: -> fp32).  These kernels fuse those
// conversions, so for an fp32 hidden state x:
//   encode(x, codec)  == transport.encode(backend.to_wire(x), codec)
//   decode(payload)   == backend.from_wire(transport.decode(header, payload))
// byte for byte on finite inputs.  Every step is exact or one IEEE-rounded
// operation (fp16 round-to-nearest-even, fp32 division and product, rint
// half-to-even), and max is order-free, so there is nothing to reorder.
#include "q4_common.h"
#include "q4wire.h"

namespace q4k {
namespace {


__device__ __forceinline__ float round_f16(float f) {        // fp32 -> fp16 (RNE) -> fp32
    return static_cast<float>(static_cast<_Float16>(f));
}
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(a))) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(b))) << 16);
}
__device__ __forceinline__ float h_lo(uint32_t w) { return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w))); }
__device__ __forceinline__ float h_hi(uint32_t w) { return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16))); }

// q = clip(rint(v / scale), -127, 127) as int8 (hetero/transport.py:208)
__device__ __forceinline__ uint32_t q8(float v, float scale) {
    const float r = __builtin_rintf(__fdiv_rn(v, scale));
    const float c = fminf(fmaxf(r, -127.0f), 127.0f);
    return static_cast<uint32_t>(static_cast<int32_t>(c)) & 0xFFu;
}

// --------------------------------------------------------------- fp16 ---
// hetero/transport.py:200-202 after backends.py:100-101: the payload is the
// fp16 array.  Elementwise over n values: 8 per thread through two 16-byte
// loads and one 16-byte store (VEC: n % 8 == 0 and both pointers 16-byte
// aligned, checked on the host), else one value per thread.
template <bool VEC>
__global__ __launch_bounds__(256) void wire_f16_encode_kernel(const float* __restrict__ x, uint16_t* __restrict__ out,
                                                              long long n) {
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; t < (VEC ? n >> 3 : n);
         t += stride) {
        if constexpr (VEC) {
            const float4 a = reinterpret_cast<const float4*>(x)[2 * t];
            const float4 b = reinterpret_cast<const float4*>(x)[2 * t + 1];
            reinterpret_cast<uint4*>(out)[t] =
                make_uint4(pack_h2(a.x, a.y), pack_h2(a.z, a.w), pack_h2(b.x, b.y), pack_h2(b.z, b.w));
        } else {
            out[t] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x[t]));
        }
    }
}

// backends.py:103-104 after transport.py:216-217: fp16 payload -> fp32
template <bool VEC>
__global__ __launch_bounds__(256) void wire_f16_decode_kernel(const uint16_t* __restrict__ in, float* __restrict__ out,
                                                              long long n) {
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; t < (VEC ? n >> 3 : n);
         t += stride) {
        if constexpr (VEC) {
            const uint4 h = reinterpret_cast<const uint4*>(in)[t];
            reinterpret_cast<float4*>(out)[2 * t] = make_float4(h_lo(h.x), h_hi(h.x), h_lo(h.y), h_hi(h.y));
            reinterpret_cast<float4*>(out)[2 * t + 1] = make_float4(h_lo(h.z), h_hi(h.z), h_lo(h.w), h_hi(h.w));
        } else {
            out[t] = static_cast<float>(__builtin_bit_cast(_Float16, in[t]));
        }
    }
}

// --------------------------------------------------------------- int8 ---
// hetero/transport.py:203-211 after backends.py:100-101.  One workgroup per
// row: the row's values, rounded to fp16 and back (to_wire then
// np.asarray(..., float32)), stay in registers -- KC chunks of 8 values per
// thread -- between the max |v| reduction and the quantisation.
//   scale = max|v| / 127 (0 -> 1), q = clip(rint(v / scale), -127, 127)
// Payload: the rows' fp32 scales, then the int8 rows (transport.py:210-211).
// VEC: hidden % 8 == 0 and x 16-byte aligned (whole chunks, aligned rows);
// else every value is loaded on its own with a bounds check.
template <int KC, bool VEC>
__global__ __launch_bounds__(1024) void wire_i8_encode_kernel(const float* __restrict__ x, uint8_t* __restrict__ payload,
                                                              int rows, int hidden) {
    __shared__ float red[16];
    const int row = blockIdx.x;
    const int tid = threadIdx.x, nt = blockDim.x;
    const int n_chunks = (hidden + 7) >> 3;
    const float* xr = x + static_cast<size_t>(row) * hidden;
    float v[KC][8];
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < KC; k++) {
        const int c = k * nt + tid;
#pragma unroll
        for (int i = 0; i < 8; i++) v[k][i] = 0.0f;
        if (c < n_chunks) {
            if constexpr (VEC) {
                const float4 a = reinterpret_cast<const float4*>(xr)[2 * c];
                const float4 b = reinterpret_cast<const float4*>(xr)[2 * c + 1];
                v[k][0] = a.x; v[k][1] = a.y; v[k][2] = a.z; v[k][3] = a.w;
                v[k][4] = b.x; v[k][5] = b.y; v[k][6] = b.z; v[k][7] = b.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (8 * c + i < hidden) v[k][i] = xr[8 * c + i];
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                v[k][i] = round_f16(v[k][i]);
                amax = fmaxf(amax, fabsf(v[k][i]));
            }
        }
    }
    amax = wave_max(amax);
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    float m = 0.0f;
    for (int i = 0; i < (nt >> 6); i++) m = fmaxf(m, red[i]);
    float scale = __fdiv_rn(m, 127.0f);                              // transport.py:206
    scale = scale == 0.0f ? 1.0f : scale;                            // :207
    if (tid == 0) reinterpret_cast<float*>(payload)[row] = scale;
    // the int8 rows start after the scales: 4-byte aligned, so 32-bit stores
    uint8_t* qr = payload + static_cast<size_t>(rows) * 4 + static_cast<size_t>(row) * hidden;
#pragma unroll
    for (int k = 0; k < KC; k++) {
        const int c = k * nt + tid;
        if (c < n_chunks) {
            uint32_t b[8];
#pragma unroll
            for (int i = 0; i < 8; i++) b[i] = q8(v[k][i], scale);
            if constexpr (VEC) {
                uint32_t* q4 = reinterpret_cast<uint32_t*>(qr + 8 * c);
                q4[0] = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
                q4[1] = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (8 * c + i < hidden) qr[8 * c + i] = static_cast<uint8_t>(b[i]);
            }
        }
    }
}

// hetero/transport.py:218-224 then backends.py:103-104:
// fp32(fp16(fp32(q) * scale)).  One workgroup per row, grid-strided over
// the row's chunks of 8.
template <bool VEC>
__global__ __launch_bounds__(256) void wire_i8_decode_kernel(const uint8_t* __restrict__ payload, float* __restrict__ out,
                                                             int rows, int hidden) {
    const int row = blockIdx.x;
    const float scale = reinterpret_cast<const float*>(payload)[row];
    const int8_t* qr = reinterpret_cast<const int8_t*>(payload + static_cast<size_t>(rows) * 4 +
                                                        static_cast<size_t>(row) * hidden);
    float* orow = out + static_cast<size_t>(row) * hidden;
    const int n_chunks = (hidden + 7) >> 3;
    for (int c = threadIdx.x; c < n_chunks; c += blockDim.x) {
        float r[8];
        if constexpr (VEC) {
            const uint32_t* q4 = reinterpret_cast<const uint32_t*>(qr + 8 * c);
            const uint32_t w0 = q4[0], w1 = q4[1];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                r[i] = static_cast<float>(static_cast<int8_t>(w0 >> (8 * i)));
                r[4 + i] = static_cast<float>(static_cast<int8_t>(w1 >> (8 * i)));
            }
#pragma unroll
            for (int i = 0; i < 8; i++) r[i] = round_f16(__fmul_rn(r[i], scale));
            reinterpret_cast<float4*>(orow)[2 * c] = make_float4(r[0], r[1], r[2], r[3]);
            reinterpret_cast<float4*>(orow)[2 * c + 1] = make_float4(r[4], r[5], r[6], r[7]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (8 * c + i < hidden)
                    orow[8 * c + i] = round_f16(__fmul_rn(static_cast<float>(qr[8 * c + i]), scale));
        }
    }
}

int wire_check(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(Q4_EHIP, "%s launch: %s", what, hipGetErrorString(e));
    return 0;
}

int elementwise_grid(long long items) {
    const long long cap = 8LL * num_cus();                  // a few waves of workgroups, then grid-stride
    const long long need = (items + 255) / 256;
    return static_cast<int>(need < 1 ? 1 : (need > cap ? cap : need));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// workgroup size and chunks per thread of the int8 encode: the fewest
// threads (a whole number of waves, at most 1024) that hold the row in at
// most four chunks of 8 per thread
int i8_threads(int hidden, int* kc) {
    const int chunks = (hidden + 7) / 8;
    for (int k = 1; k <= 4; k *= 2) {
        const int t = ((chunks + k - 1) / k + 63) / 64 * 64;
        if (t <= 1024) {
            *kc = k;
            return t < 64 ? 64 : t;
        }
    }
    return 0;
}

template <int KC>
void launch_i8_encode(bool vec, int rows, int nt, hipStream_t st, const float* x, uint8_t* p, int hidden) {
    if (vec)
        hipLaunchKernelGGL((wire_i8_encode_kernel<KC, true>), dim3(rows), dim3(nt), 0, st, x, p, rows, hidden);
    else
        hipLaunchKernelGGL((wire_i8_encode_kernel<KC, false>), dim3(rows), dim3(nt), 0, st, x, p, rows, hidden);
}

}  // namespace
}  // namespace q4k

using namespace q4k;

#pragma GCC visibility push(default)
extern "C" {

long long q4_wire_payload_bytes(int codec, int rows, int hidden) {
    if (rows < 0 || hidden <= 0) return -1;
    const long long n = static_cast<long long>(rows) * hidden;
    if (codec == Q4_WIRE_FP16) return 2 * n;
    if (codec == Q4_WIRE_INT8) return 4LL * rows + n;
    return -1;
}

int q4_wire_encode_dev(const float* x, int rows, int hidden, int codec, void* payload, void* stream) {
    if (codec != Q4_WIRE_FP16 && codec != Q4_WIRE_INT8) return fail(Q4_EARG, "q4_wire_encode_dev: unknown codec %d", codec);
    if (rows < 0 || hidden <= 0) return fail(Q4_EARG, "q4_wire_encode_dev: bad shape (%d rows of %d)", rows, hidden);
    if (rows == 0) return 0;
    if (!x || !payload) return fail(Q4_EARG, "q4_wire_encode_dev: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const long long n = static_cast<long long>(rows) * hidden;
    if (codec == Q4_WIRE_FP16) {
        const bool vec = n % 8 == 0 && aligned16(x) && aligned16(payload);
        uint16_t* out = static_cast<uint16_t*>(payload);
        if (vec)
            hipLaunchKernelGGL(wire_f16_encode_kernel<true>, dim3(elementwise_grid(n >> 3)), dim3(256), 0, st, x, out, n);
        else
            hipLaunchKernelGGL(wire_f16_encode_kernel<false>, dim3(elementwise_grid(n)), dim3(256), 0, st, x, out, n);
        return wire_check("q4_wire_encode_dev (fp16)");
    }
    int kc = 0;
    const int nt = i8_threads(hidden, &kc);
    if (!nt) return fail(Q4_EARG, "q4_wire_encode_dev: hidden %d over the int8 row limit of 32768", hidden);
    if (reinterpret_cast<uintptr_t>(payload) & 3) return fail(Q4_EARG, "q4_wire_encode_dev: payload not 4-byte aligned");
    const bool vec = hidden % 8 == 0 && aligned16(x);
    uint8_t* p = static_cast<uint8_t*>(payload);
    switch (kc) {
        case 1: launch_i8_encode<1>(vec, rows, nt, st, x, p, hidden); break;
        case 2: launch_i8_encode<2>(vec, rows, nt, st, x, p, hidden); break;
        default: launch_i8_encode<4>(vec, rows, nt, st, x, p, hidden); break;
    }
    return wire_check("q4_wire_encode_dev (int8)");
}

int q4_wire_decode_dev(const void* payload, int rows, int hidden, int codec, float* out, void* stream) {
    if (codec != Q4_WIRE_FP16 && codec != Q4_WIRE_INT8) return fail(Q4_EARG, "q4_wire_decode_dev: unknown codec %d", codec);
    if (rows < 0 || hidden <= 0) return fail(Q4_EARG, "q4_wire_decode_dev: bad shape (%d rows of %d)", rows, hidden);
    if (rows == 0) return 0;
    if (!payload || !out) return fail(Q4_EARG, "q4_wire_decode_dev: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const long long n = static_cast<long long>(rows) * hidden;
    if (codec == Q4_WIRE_FP16) {
        const uint16_t* in = static_cast<const uint16_t*>(payload);
        if (n % 8 == 0 && aligned16(payload) && aligned16(out))
            hipLaunchKernelGGL(wire_f16_decode_kernel<true>, dim3(elementwise_grid(n >> 3)), dim3(256), 0, st, in, out, n);
        else
            hipLaunchKernelGGL(wire_f16_decode_kernel<false>, dim3(elementwise_grid(n)), dim3(256), 0, st, in, out, n);
        return wire_check("q4_wire_decode_dev (fp16)");
    }
    if (reinterpret_cast<uintptr_t>(payload) & 3) return fail(Q4_EARG, "q4_wire_decode_dev: payload not 4-byte aligned");
    const uint8_t* p = static_cast<const uint8_t*>(payload);
    if (hidden % 8 == 0 && aligned16(out))
        hipLaunchKernelGGL(wire_i8_decode_kernel<true>, dim3(rows), dim3(256), 0, st, p, out, rows, hidden);
    else
        hipLaunchKernelGGL(wire_i8_decode_kernel<false>, dim3(rows), dim3(256), 0, st, p, out, rows, hidden);
    return wire_check("q4_wire_decode_dev (int8)");
}

}  // extern "C"
#pragma GCC visibility pop
