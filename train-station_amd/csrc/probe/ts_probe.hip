// A stand-alone gfx950 code object for the module entries of ts_hip.h
// (ts_hip_module_load_data / _get_function / _launch): built by the package
// Makefile into ts_probe.hsaco, loaded and launched by the tests.
#include <hip/hip_runtime.h>

// y[i] = a * x[i] + y[i] for i < n (a multiply then an add: no contraction)
extern "C" __global__ void ts_probe_axpy(float a, const float *x, float *y, unsigned long long n) {
    const unsigned long long i = static_cast<unsigned long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = a * x[i] + y[i];
}
