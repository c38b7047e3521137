// softmax along one axis (tensor/ops/softmax.rs:4-60) and its backward
// (grad_fn/ops/softmax.rs:4-38).  The tensor is viewed as [outer, reduce,
// inner]; one thread owns a slice (o, i) and walks its `reduce` elements in
// the reference's order -- max, then exp and a sequential fp32 sum, then a
// scale by 1/sum; backward a sequential fp32 dot then y * (go - dot) -- so
// the results are those of the reference's loops, element for element.
#include "ts_hip_internal.h"
#include "ts_hip_libm.h"

namespace tship {

// f32::exp of the reference: the host libm's expf, restated (ts_hip_libm.h)
__device__ inline float softmax_exp(float x) { return libm::expf_glibc(x); }

__global__ __launch_bounds__(kBlock) void softmax_fwd(const float *__restrict__ x, float *__restrict__ y,
                                                      size_t outer, size_t reduce, size_t inner) {
    const size_t slices = outer * inner;
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t t = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; t < slices; t += stride) {
        const size_t o = t / inner, i = t % inner;
        const size_t base = o * reduce * inner + i;
        float maxv = -__builtin_inff();
        for (size_t j = 0; j < reduce; ++j) {
            const float v = x[base + j * inner];
            if (v > maxv) maxv = v;
        }
        float sum = 0.0f;
        for (size_t j = 0; j < reduce; ++j) {
            const float e = softmax_exp(x[base + j * inner] - maxv);
            y[base + j * inner] = e;
            sum += e;
        }
        const float inv = 1.0f / sum;
        for (size_t j = 0; j < reduce; ++j) y[base + j * inner] *= inv;
    }
}

__global__ __launch_bounds__(kBlock) void softmax_bwd(const float *__restrict__ y, const float *__restrict__ go,
                                                      float *__restrict__ gi, size_t outer, size_t reduce,
                                                      size_t inner) {
    const size_t slices = outer * inner;
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t t = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; t < slices; t += stride) {
        const size_t o = t / inner, i = t % inner;
        const size_t base = o * reduce * inner + i;
        float dot = 0.0f;
        for (size_t j = 0; j < reduce; ++j) {
            const size_t off = base + j * inner;
            dot += go[off] * y[off];
        }
        for (size_t j = 0; j < reduce; ++j) {
            const size_t off = base + j * inner;
            gi[off] = y[off] * (go[off] - dot);
        }
    }
}

}  // namespace tship

using namespace tship;

extern "C" {

int ts_hip_softmax(const float *x, float *y, size_t outer, size_t reduce, size_t inner, void *stream) {
    const size_t slices = outer * inner;
    if (slices == 0 || reduce == 0) return reduce == 0 && slices ? TS_HIP_EINVAL : TS_HIP_OK;
    if (!x || !y) return TS_HIP_EINVAL;
    launch(softmax_fwd, dim3(grid_for(slices)), dim3(kBlock), 0, as_stream(stream), x, y, outer,
                       reduce, inner);
    return launch_status();
}

int ts_hip_softmax_backward(const float *y, const float *go, float *gi, size_t outer, size_t reduce,
                            size_t inner, void *stream) {
    const size_t slices = outer * inner;
    if (slices == 0 || reduce == 0) return TS_HIP_OK;
    if (!y || !go || !gi) return TS_HIP_EINVAL;
    launch(softmax_bwd, dim3(grid_for(slices)), dim3(kBlock), 0, as_stream(stream), y, go, gi,
                       outer, reduce, inner);
    return launch_status();
}

}  // extern "C"
