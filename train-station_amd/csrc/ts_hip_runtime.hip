// Runtime half of the C-ABI: device selection, memory, copies, streams,
// events.  Replaces the host-only stub train-station/src/cuda/cuda_wrapper.cpp
// (whose "device" memory is host `new float[]`, :37-52) with real HIP calls.
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "ts_hip_internal.h"

namespace tship {

static std::mutex g_cu_mutex;
static std::vector<int> g_cu_count;  // per device, 0 = not queried yet

int device_cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(g_cu_mutex);
    if (static_cast<size_t>(dev) >= g_cu_count.size()) g_cu_count.resize(dev + 1, 0);
    if (g_cu_count[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        g_cu_count[dev] = cus;
    }
    return g_cu_count[dev];
}

static thread_local TimingWindow g_window;
static thread_local bool g_window_open = false;

TimingWindow *timing_window() { return g_window_open ? &g_window : nullptr; }

// A HIP status returned to the caller is also consumed from HIP's per-thread
// last error, so that a failure reported here is not reported again by the
// next kernel launch's status check.
static int status_of(hipError_t e) {
    if (e != hipSuccess) (void)hipGetLastError();
    return static_cast<int>(e);
}

static hipMemcpyKind copy_kind(int kind, bool *ok) {
    *ok = true;
    switch (kind) {
        case 0: return hipMemcpyHostToDevice;
        case 1: return hipMemcpyDeviceToHost;
        case 2: return hipMemcpyDeviceToDevice;
        default: *ok = false; return hipMemcpyDefault;
    }
}

}  // namespace tship

using namespace tship;

namespace {
// Stream work below that is not a kernel launch (copies, synchronisation,
// events, graphs, module kernels) goes after any products a launch group holds.
void flush_held() {
    if (tship::launch_group_holding()) tship::flush_launch_group();
}
}  // namespace

extern "C" {

int ts_hip_initialize(void) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return tship::status_of(e);
    if (count <= 0) return TS_HIP_ENODEVICE;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, 0);
    if (e != hipSuccess) return tship::status_of(e);
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return TS_HIP_ENODEVICE;
    e = hipSetDevice(0);
    if (e != hipSuccess) return tship::status_of(e);
    device_cu_count();
    return TS_HIP_OK;
}

void ts_hip_cleanup(void) {
    flush_held();
    (void)hipDeviceSynchronize();
}

int ts_hip_get_device_count(int *count) {
    if (!count) return TS_HIP_EINVAL;
    *count = 0;
    hipError_t e = hipGetDeviceCount(count);
    if (e == hipErrorNoDevice) { *count = 0; return TS_HIP_OK; }
    return tship::status_of(e);
}

int ts_hip_set_device(int device_id) { return tship::status_of(hipSetDevice(device_id)); }

int ts_hip_get_device(int *device_id) {
    if (!device_id) return TS_HIP_EINVAL;
    return tship::status_of(hipGetDevice(device_id));
}

int ts_hip_malloc(float **ptr, size_t n_floats) {
    if (!ptr) return TS_HIP_EINVAL;
    *ptr = nullptr;
    if (n_floats == 0) return TS_HIP_OK;
    return tship::status_of(hipMalloc(reinterpret_cast<void **>(ptr), n_floats * sizeof(float)));
}

int ts_hip_free(float *ptr) {
    if (!ptr) return TS_HIP_OK;
    return tship::status_of(hipFree(ptr));
}

int ts_hip_memcpy(float *dst, const float *src, size_t n_floats, int kind) {
    flush_held();
    bool ok;
    hipMemcpyKind k = copy_kind(kind, &ok);
    if (!ok || (n_floats && (!dst || !src))) return TS_HIP_EINVAL;
    if (n_floats == 0) return TS_HIP_OK;
    return tship::status_of(hipMemcpy(dst, src, n_floats * sizeof(float), k));
}

int ts_hip_memcpy_async(float *dst, const float *src, size_t n_floats, int kind, void *stream) {
    flush_held();
    bool ok;
    hipMemcpyKind k = copy_kind(kind, &ok);
    if (!ok || (n_floats && (!dst || !src))) return TS_HIP_EINVAL;
    if (n_floats == 0) return TS_HIP_OK;
    return tship::status_of(
        hipMemcpyAsync(dst, src, n_floats * sizeof(float), k, as_stream(stream)));
}

int ts_hip_memcpy_bytes(void *dst, const void *src, size_t bytes, int kind, void *stream) {
    flush_held();
    bool ok;
    hipMemcpyKind k = copy_kind(kind, &ok);
    if (!ok || (bytes && (!dst || !src))) return TS_HIP_EINVAL;
    if (bytes == 0) return TS_HIP_OK;
    return tship::status_of(hipMemcpyAsync(dst, src, bytes, k, as_stream(stream)));
}

int ts_hip_host_malloc(void **ptr, size_t bytes) {
    if (!ptr) return TS_HIP_EINVAL;
    *ptr = nullptr;
    if (bytes == 0) return TS_HIP_OK;
    return tship::status_of(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
}

int ts_hip_host_free(void *ptr) {
    if (!ptr) return TS_HIP_OK;
    return tship::status_of(hipHostFree(ptr));
}

int ts_hip_stream_create(void **stream) {
    if (!stream) return TS_HIP_EINVAL;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    *stream = s;
    return tship::status_of(e);
}

int ts_hip_stream_destroy(void *stream) {
    if (!stream) return TS_HIP_OK;
    return tship::status_of(hipStreamDestroy(as_stream(stream)));
}

int ts_hip_stream_synchronize(void *stream) {
    flush_held();
    return tship::status_of(hipStreamSynchronize(as_stream(stream)));
}

int ts_hip_device_synchronize(void) {
    flush_held();
    return tship::status_of(hipDeviceSynchronize());
}

int ts_hip_event_create(void **event) {
    if (!event) return TS_HIP_EINVAL;
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreate(&ev);
    *event = ev;
    return tship::status_of(e);
}

int ts_hip_event_destroy(void *event) {
    if (!event) return TS_HIP_OK;
    return tship::status_of(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
}

int ts_hip_event_record(void *event, void *stream) {
    flush_held();
    if (!event) return TS_HIP_EINVAL;
    return tship::status_of(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)));
}

int ts_hip_event_synchronize(void *event) {
    if (!event) return TS_HIP_EINVAL;
    return tship::status_of(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)));
}

int ts_hip_event_elapsed_ms(float *ms, void *start, void *stop) {
    if (!ms || !start || !stop) return TS_HIP_EINVAL;
    return tship::status_of(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                                reinterpret_cast<hipEvent_t>(stop)));
}

int ts_hip_timing_begin(void *start, void *stop) {
    if (!start || !stop) return TS_HIP_EINVAL;
    tship::g_window = {reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop), 0};
    tship::g_window_open = true;
    return TS_HIP_OK;
}

int ts_hip_timing_end(int *kernels) {
    if (!kernels) return TS_HIP_EINVAL;
    *kernels = tship::g_window_open ? tship::g_window.kernels : 0;
    tship::g_window_open = false;
    return TS_HIP_OK;
}

int ts_hip_module_load_data(const void *image, void **module) {
    if (!image || !module) return TS_HIP_EINVAL;
    hipModule_t m = nullptr;
    const hipError_t e = hipModuleLoadData(&m, image);
    *module = e == hipSuccess ? m : nullptr;
    return tship::status_of(e);
}

int ts_hip_module_unload(void *module) {
    if (!module) return TS_HIP_OK;
    return tship::status_of(hipModuleUnload(reinterpret_cast<hipModule_t>(module)));
}

int ts_hip_module_get_function(void *module, const char *name, void **function) {
    if (!module || !name || !function) return TS_HIP_EINVAL;
    hipFunction_t f = nullptr;
    const hipError_t e = hipModuleGetFunction(&f, reinterpret_cast<hipModule_t>(module), name);
    *function = e == hipSuccess ? f : nullptr;
    return tship::status_of(e);
}

int ts_hip_module_launch(void *function, unsigned grid_x, unsigned grid_y, unsigned grid_z, unsigned block_x,
                         unsigned block_y, unsigned block_z, unsigned lds_bytes, void *stream,
                         void **kernel_params) {
    flush_held();
    if (!function || !grid_x || !grid_y || !grid_z || !block_x || !block_y || !block_z) return TS_HIP_EINVAL;
    if (static_cast<unsigned long long>(block_x) * block_y * block_z > 1024) return TS_HIP_EINVAL;
    return tship::status_of(hipModuleLaunchKernel(reinterpret_cast<hipFunction_t>(function), grid_x, grid_y,
                                                  grid_z, block_x, block_y, block_z, lds_bytes,
                                                  as_stream(stream), kernel_params, nullptr));
}

int ts_hip_stream_begin_capture(void *stream) {
    if (!stream) return TS_HIP_EINVAL;  // the null stream cannot be recorded
    return tship::status_of(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeRelaxed));
}

int ts_hip_stream_end_capture(void *stream, void **graph_exec) {
    flush_held();
    if (!stream || !graph_exec) return TS_HIP_EINVAL;
    *graph_exec = nullptr;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(as_stream(stream), &graph);
    if (e != hipSuccess) return tship::status_of(e);
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);  // the executable graph keeps its own copy
    if (e != hipSuccess) return tship::status_of(e);
    *graph_exec = exec;
    return TS_HIP_OK;
}

int ts_hip_stream_is_capturing(void *stream, int *capturing) {
    if (!capturing) return TS_HIP_EINVAL;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(as_stream(stream), &st);
    *capturing = st == hipStreamCaptureStatusActive ? 1 : 0;
    return tship::status_of(e);
}

int ts_hip_graph_launch(void *graph_exec, void *stream) {
    flush_held();
    if (!graph_exec) return TS_HIP_EINVAL;
    return tship::status_of(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph_exec), as_stream(stream)));
}

int ts_hip_graph_destroy(void *graph_exec) {
    if (!graph_exec) return TS_HIP_OK;
    return tship::status_of(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph_exec)));
}

const char *ts_hip_error_string(int status) {
    switch (status) {
        case TS_HIP_OK: return "success";
        case TS_HIP_EINVAL: return "invalid argument (shape, pointer, alignment or copy kind)";
        case TS_HIP_ENODEVICE: return "no gfx950 device visible";
        case TS_HIP_EWORKSPACE: return "workspace smaller than the size the kernel needs";
        case TS_HIP_ESCRATCH: return "product needs more scratch than the allocation-free entry point holds";
        default: return hipGetErrorString(static_cast<hipError_t>(status));
    }
}

int ts_hip_mem_info(size_t *free_bytes, size_t *total_bytes) {
    if (!free_bytes || !total_bytes) return TS_HIP_EINVAL;
    return tship::status_of(hipMemGetInfo(free_bytes, total_bytes));
}

}  // extern "C"
