// Device-side encoding of tensor data for checkpoints.
//
// The reference's binary format stores a Tensor's Vec<f32> as an Array of
// tagged F32 values (serialization/core/impls.rs:278-288 builds the array;
// binary/structs.rs:193-196 writes each element as the type tag 10 followed by
// the f32's bits, little-endian; binary/writer.rs:218-220).  Each element is
// therefore a 5-byte record, and 4 records are exactly 5 dwords:
//
//   bytes  0..3  = 10 | a << 8                       a, b, c, d = float bits
//   bytes  4..7  = a >> 24 | 10 << 8  | b << 16
//   bytes  8..11 = b >> 16 | 10 << 16 | c << 24
//   bytes 12..15 = c >> 8  | 10 << 24
//   bytes 16..19 = d
//
// so a thread turns one float4 into five aligned dword stores (and back),
// without byte-granular traffic.  HBM-bound: 9 bytes moved per element.
#include "ts_hip_internal.h"

namespace tship {

constexpr uint32_t kF32Tag = 10;

__global__ __launch_bounds__(kBlock) void encode_records(const float *__restrict__ src, size_t n,
                                                         uint32_t *__restrict__ dst) {
    const size_t groups = n / 4;
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    const float4 *s4 = reinterpret_cast<const float4 *>(src);
    for (size_t g = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; g < groups; g += stride) {
        const float4 q = s4[g];
        const uint32_t a = __float_as_uint(q.x), b = __float_as_uint(q.y);
        const uint32_t c = __float_as_uint(q.z), d = __float_as_uint(q.w);
        uint32_t *o = dst + 5 * g;
        o[0] = kF32Tag | (a << 8);
        o[1] = (a >> 24) | (kF32Tag << 8) | (b << 16);
        o[2] = (b >> 16) | (kF32Tag << 16) | (c << 24);
        o[3] = (c >> 8) | (kF32Tag << 24);
        o[4] = d;
    }
    // the last n % 4 records, byte by byte
    if (blockIdx.x == 0 && threadIdx.x < n - 4 * groups) {
        const size_t i = 4 * groups + threadIdx.x;
        const uint32_t v = __float_as_uint(src[i]);
        uint8_t *o = reinterpret_cast<uint8_t *>(dst) + 5 * i;
        o[0] = static_cast<uint8_t>(kF32Tag);
        o[1] = static_cast<uint8_t>(v);
        o[2] = static_cast<uint8_t>(v >> 8);
        o[3] = static_cast<uint8_t>(v >> 16);
        o[4] = static_cast<uint8_t>(v >> 24);
    }
}

__global__ __launch_bounds__(kBlock) void decode_records(const uint32_t *__restrict__ src, size_t n,
                                                         float *__restrict__ dst,
                                                         unsigned long long *bad_index) {
    const size_t groups = n / 4;
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    float4 *d4 = reinterpret_cast<float4 *>(dst);
    for (size_t g = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; g < groups; g += stride) {
        const uint32_t *w = src + 5 * g;
        const uint32_t w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3], w4 = w[4];
        if (bad_index) {
            const bool t0 = (w0 & 0xFFu) == kF32Tag, t1 = ((w1 >> 8) & 0xFFu) == kF32Tag;
            const bool t2 = ((w2 >> 16) & 0xFFu) == kF32Tag, t3 = (w3 >> 24) == kF32Tag;
            if (!(t0 && t1 && t2 && t3)) {
                const size_t first = 4 * g + (t0 ? (t1 ? (t2 ? 3 : 2) : 1) : 0);
                atomicMin(bad_index, static_cast<unsigned long long>(first));
            }
        }
        float4 q;
        q.x = __uint_as_float((w0 >> 8) | (w1 << 24));
        q.y = __uint_as_float((w1 >> 16) | (w2 << 16));
        q.z = __uint_as_float((w2 >> 24) | (w3 << 8));
        q.w = __uint_as_float(w4);
        d4[g] = q;
    }
    if (blockIdx.x == 0 && threadIdx.x < n - 4 * groups) {
        const size_t i = 4 * groups + threadIdx.x;
        const uint8_t *r = reinterpret_cast<const uint8_t *>(src) + 5 * i;
        if (bad_index && r[0] != kF32Tag) atomicMin(bad_index, static_cast<unsigned long long>(i));
        const uint32_t v = static_cast<uint32_t>(r[1]) | (static_cast<uint32_t>(r[2]) << 8) |
                           (static_cast<uint32_t>(r[3]) << 16) | (static_cast<uint32_t>(r[4]) << 24);
        dst[i] = __uint_as_float(v);
    }
}

}  // namespace tship

using namespace tship;

extern "C" {

int ts_hip_encode_f32_records(const float *src, size_t n, void *dst, void *stream) {
    if (n == 0) return TS_HIP_OK;
    if (!src || !dst) return TS_HIP_EINVAL;
    // float4 loads and dword stores
    if (!aligned16(src) || (reinterpret_cast<uintptr_t>(dst) & 3u) != 0) return TS_HIP_EINVAL;
    launch(encode_records, dim3(grid_for(n / 4 + 1)), dim3(kBlock), 0, as_stream(stream),
                       src, n, static_cast<uint32_t *>(dst));
    return launch_status();
}

int ts_hip_decode_f32_records(const void *src, size_t n, float *dst, unsigned long long *bad_index,
                              void *stream) {
    if (n == 0) return TS_HIP_OK;
    if (!src || !dst) return TS_HIP_EINVAL;
    if (!aligned16(dst) || (reinterpret_cast<uintptr_t>(src) & 3u) != 0) return TS_HIP_EINVAL;
    launch(decode_records, dim3(grid_for(n / 4 + 1)), dim3(kBlock), 0, as_stream(stream),
                       static_cast<const uint32_t *>(src), n, dst, bad_index);
    return launch_status();
}

}  // extern "C"
