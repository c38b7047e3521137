// Fused Adam::step for one parameter tensor: one read of p, g, m, v and one
// write of p, m, v per element (28 bytes), replacing the reference's five
// passes and three temporary clones (optimizers/adam/mod.rs:485-1007) while
// keeping its per-element fp32 operation order bit for bit.
#include <cmath>

#include "ts_hip_internal.h"

namespace tship {

struct AdamArgs {
    float *p;
    const float *g;
    float *m;
    float *v;
    float *vmax;  // AMSGrad running max of v_hat, or nullptr
    size_t n, n4, tail_start;
    int amsgrad_first;
    float b1, c1, b2, c2, cf1, cf2, lr, eps, wd;
};

// vmax: the AMSGrad running max of v_hat for this element (read and updated
// only when a.vmax is set).
__device__ inline void adam_elem(const AdamArgs &a, size_t i, float &p, float g, float &m,
                                 float &v, float &vmax) {
    if (a.wd > 0.0f) g = g + a.wd * p;                        // adam/mod.rs:567-620
    m = a.b1 * m + a.c1 * g;                                  // :634-696
    v = (i < a.tail_start) ? a.b2 * v + a.c2 * (g * g)        // :709-774 AVX2 body
                           : a.b2 * v + (a.c2 * g) * g;       //          scalar tail
    const float mh = m * a.cf1;                               // :790-833 bias_correct
    float vh = v * a.cf2;
    if (a.vmax) {                                             // :534-541 AMSGrad
        const float old = a.amsgrad_first ? vh : vmax;
        vh = old > vh ? old : vh;
        vmax = vh;
    }
    const float den = sqrtf(vh) + a.eps;                      // :913-1007
    p = p - (a.lr * mh) / den;
}

// Thread t updates float4 group t (elements 4t .. 4t+3) when t < n4, and
// element 4*n4 + t of the scalar remainder.  The gradient is read once per
// step, so it is loaded with the non-temporal policy.  NT: p, m and v too are
// loaded and stored non-temporally -- for tensors too large to come back from
// the 256 MB last-level cache (MALL) anyway.  Measured: one 256M-parameter
// tensor 753 -> 824 steps/s with NT; the six 16.7M-parameter weights of a
// training step 0.484 -> 0.50 ms, so NT is chosen by size (kAdamNtMin).
template <bool NT>
__device__ inline void adam_unit(const AdamArgs &a, size_t t) {
    if (t < a.n4) {
        float4 *p4 = reinterpret_cast<float4 *>(a.p);
        float4 *m4 = reinterpret_cast<float4 *>(a.m);
        float4 *v4 = reinterpret_cast<float4 *>(a.v);
        float4 *vm4 = reinterpret_cast<float4 *>(a.vmax);
        float4 p = NT ? load_nt(p4 + t) : p4[t], m = NT ? load_nt(m4 + t) : m4[t];
        float4 v = NT ? load_nt(v4 + t) : v4[t];
        const float4 g = load_nt(reinterpret_cast<const float4 *>(a.g) + t);
        float4 vm = a.vmax ? (NT ? load_nt(vm4 + t) : vm4[t]) : make_float4(0, 0, 0, 0);
        adam_elem(a, 4 * t + 0, p.x, g.x, m.x, v.x, vm.x);
        adam_elem(a, 4 * t + 1, p.y, g.y, m.y, v.y, vm.y);
        adam_elem(a, 4 * t + 2, p.z, g.z, m.z, v.z, vm.z);
        adam_elem(a, 4 * t + 3, p.w, g.w, m.w, v.w, vm.w);
        if (NT) {
            store_nt(p4 + t, p);
            store_nt(m4 + t, m);
            store_nt(v4 + t, v);
            if (a.vmax) store_nt(vm4 + t, vm);
        } else {
            p4[t] = p;
            m4[t] = m;
            v4[t] = v;
            if (a.vmax) vm4[t] = vm;
        }
    }
    const size_t i = 4 * a.n4 + t;
    if (i < a.n) {
        float p = a.p[i], m = a.m[i], v = a.v[i], vm = a.vmax ? a.vmax[i] : 0.0f;
        adam_elem(a, i, p, a.g[i], m, v, vm);
        a.p[i] = p;
        a.m[i] = m;
        a.v[i] = v;
        if (a.vmax) a.vmax[i] = vm;
    }
}

// Threads needed by one tensor: its float4 groups or its scalar remainder.
inline size_t adam_threads(size_t n, size_t n4) {
    const size_t rest = n - 4 * n4;
    return n4 > rest ? n4 : rest;
}

// Parameters per tensor from which p, m and v take the non-temporal policy:
// 64M floats, 256 MB per operand array.
constexpr size_t kAdamNtMin = size_t(1) << 26;

template <bool NT>
__global__ __launch_bounds__(kBlock) void adam_kernel(AdamArgs a) {
    adam_unit<NT>(a, static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x);
}

// adam/mod.rs:524-531: (1 - (beta as f64).powf(step as f32 as f64)) as f32,
// then bias_correct's 1.0 / bc in f32.
static float correction_factor(float beta, uint64_t step_count) {
    const float t = static_cast<float>(step_count);
    const double bc = 1.0 - std::pow(static_cast<double>(beta), static_cast<double>(t));
    return 1.0f / static_cast<float>(bc);
}

}  // namespace tship

using namespace tship;

struct MultiArgs {
    ts_hip_adam_param prm[TS_HIP_ADAM_MAX_PARAMS];
    int vec[TS_HIP_ADAM_MAX_PARAMS];
    int nt[TS_HIP_ADAM_MAX_PARAMS];  // tensor j takes the non-temporal policy (n >= kAdamNtMin)
    unsigned first_block[TS_HIP_ADAM_MAX_PARAMS + 1];  // workgroups of tensor j: [first_block[j], first_block[j+1])
    int count;
    float b1, c1, b2, c2, cf1, cf2, lr, eps, wd;
    // When set, the bias corrections are cf_table[2*s], cf_table[2*s+1] with
    // s = *cf_slot instead of cf1 / cf2 (a step recorded once and replayed);
    // with cf_ticket instead of cf_slot, wave w of the launch adds 1 to
    // cf_ticket[w] and s = its value before the add (the launches it has run
    // since the tickets were cleared: one word per wave, so no two waves
    // contend for an address).
    const float *cf_table;
    const unsigned *cf_slot;
    unsigned *cf_ticket;
};

// One flat grid over all tensors: workgroup b finds its tensor in the
// (uniform) prefix table, then works as adam_kernel does on that tensor.
__global__ __launch_bounds__(kBlock) void adam_multi_kernel(MultiArgs A) {
    int j = 0;
    while (j + 1 < A.count && blockIdx.x >= A.first_block[j + 1]) ++j;
    const ts_hip_adam_param &q = A.prm[j];
    AdamArgs a{};
    a.p = q.p; a.g = q.g; a.m = q.m; a.v = q.v; a.vmax = q.v_hat_max;
    a.n = q.n;
    a.n4 = A.vec[j] ? q.n / 4 : 0;
    a.tail_start = (q.n / 8) * 8;
    a.amsgrad_first = q.amsgrad_first;
    a.b1 = A.b1; a.c1 = A.c1; a.b2 = A.b2; a.c2 = A.c2;
    a.cf1 = A.cf1; a.cf2 = A.cf2; a.lr = A.lr; a.eps = A.eps; a.wd = A.wd;
    if (A.cf_table) {  // vector loads at device scope: the slot changes between launches
        unsigned sl;
        if (A.cf_ticket) {  // one vector atomic per wave on its own word, its result read from lane 0
            unsigned tk = 0;
            const unsigned w = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
            if ((threadIdx.x & 63) == 0) tk = atomicAdd(A.cf_ticket + w, 1u);
            sl = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(tk)));
        } else {
            sl = __hip_atomic_load(A.cf_slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        a.cf1 = __hip_atomic_load(A.cf_table + 2 * sl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.cf2 = __hip_atomic_load(A.cf_table + 2 * sl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const size_t t = static_cast<size_t>(blockIdx.x - A.first_block[j]) * kBlock + threadIdx.x;
    if (A.nt[j])  // uniform per workgroup
        adam_unit<true>(a, t);
    else
        adam_unit<false>(a, t);
}

// *slot += 1 by one lane, with vector memory operations.
__global__ void slot_advance_kernel(unsigned *slot) {
    if (threadIdx.x == 0) {
        const unsigned v = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(slot, v + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

extern "C" int ts_hip_adam_step(float *p, const float *g, float *m, float *v, float *v_hat_max,
                                size_t n, float lr, float beta1, float beta2, float eps,
                                float weight_decay, uint64_t step_count, size_t tail_start,
                                int amsgrad_first, void *stream) {
    if (n == 0) return TS_HIP_OK;
    if (!p || !g || !m || !v || step_count == 0) return TS_HIP_EINVAL;
    AdamArgs a{};
    a.p = p; a.g = g; a.m = m; a.v = v; a.vmax = v_hat_max;
    a.n = n;
    a.amsgrad_first = amsgrad_first;
    const bool vec = aligned16(p) && aligned16(g) && aligned16(m) && aligned16(v) &&
                     (!v_hat_max || aligned16(v_hat_max));
    a.n4 = vec ? n / 4 : 0;
    a.tail_start = tail_start;
    a.b1 = beta1; a.c1 = 1.0f - beta1;
    a.b2 = beta2; a.c2 = 1.0f - beta2;
    a.cf1 = correction_factor(beta1, step_count);
    a.cf2 = correction_factor(beta2, step_count);
    a.lr = lr; a.eps = eps; a.wd = weight_decay;
    const size_t blocks = (adam_threads(n, a.n4) + kBlock - 1) / kBlock;
    if (blocks > 0x7fffffffULL) return TS_HIP_EINVAL;
    if (n >= kAdamNtMin)
        launch(adam_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                           as_stream(stream), a);
    else
        launch(adam_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                           as_stream(stream), a);
    return launch_status();
}

// Workgroups of the one multi-tensor launch over params (0 for a bad list).
static size_t adam_multi_blocks(const ts_hip_adam_param *params, size_t count) {
    if (!params || count == 0 || count > TS_HIP_ADAM_MAX_PARAMS) return 0;
    size_t blocks = 0;
    for (size_t i = 0; i < count; ++i) {
        const ts_hip_adam_param &q = params[i];
        const bool vec = aligned16(q.p) && aligned16(q.g) && aligned16(q.m) && aligned16(q.v) &&
                         (!q.v_hat_max || aligned16(q.v_hat_max));
        blocks += (adam_threads(q.n, vec ? q.n / 4 : 0) + kBlock - 1) / kBlock;
    }
    return blocks;
}

static int adam_multi(const ts_hip_adam_param *params, size_t count, float lr, float beta1, float beta2,
                      float eps, float weight_decay, float cf1, float cf2, const float *cf_table,
                      const unsigned *cf_slot, void *stream, unsigned *cf_ticket = nullptr) {
    if (count == 0) return TS_HIP_OK;
    if (!params || count > TS_HIP_ADAM_MAX_PARAMS) return TS_HIP_EINVAL;
    MultiArgs A{};
    size_t blocks = 0;
    for (size_t i = 0; i < count; ++i) {
        const ts_hip_adam_param &q = params[i];
        if (q.n && (!q.p || !q.g || !q.m || !q.v)) return TS_HIP_EINVAL;
        A.prm[i] = q;
        A.vec[i] = aligned16(q.p) && aligned16(q.g) && aligned16(q.m) && aligned16(q.v) &&
                   (!q.v_hat_max || aligned16(q.v_hat_max));
        A.nt[i] = q.n >= kAdamNtMin;
        A.first_block[i] = static_cast<unsigned>(blocks);
        blocks += (adam_threads(q.n, A.vec[i] ? q.n / 4 : 0) + kBlock - 1) / kBlock;
        if (blocks > 0x7fffffffULL) return TS_HIP_EINVAL;
    }
    A.first_block[count] = static_cast<unsigned>(blocks);
    A.count = static_cast<int>(count);
    if (blocks == 0) return TS_HIP_OK;
    A.b1 = beta1; A.c1 = 1.0f - beta1;
    A.b2 = beta2; A.c2 = 1.0f - beta2;
    A.cf1 = cf1;
    A.cf2 = cf2;
    A.cf_table = cf_table;
    A.cf_slot = cf_slot;
    A.cf_ticket = cf_ticket;
    A.lr = lr; A.eps = eps; A.wd = weight_decay;
    launch(adam_multi_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                       as_stream(stream), A);
    return launch_status();
}

extern "C" int ts_hip_adam_step_multi(const ts_hip_adam_param *params, size_t count, float lr,
                                      float beta1, float beta2, float eps, float weight_decay,
                                      uint64_t step_count, void *stream) {
    if (step_count == 0) return TS_HIP_EINVAL;
    return adam_multi(params, count, lr, beta1, beta2, eps, weight_decay, correction_factor(beta1, step_count),
                      correction_factor(beta2, step_count), nullptr, nullptr, stream);
}

extern "C" int ts_hip_adam_step_multi_table(const ts_hip_adam_param *params, size_t count, float lr,
                                            float beta1, float beta2, float eps, float weight_decay,
                                            const float *bias_corrections, const unsigned *slot, void *stream) {
    if (!bias_corrections || !slot) return TS_HIP_EINVAL;
    return adam_multi(params, count, lr, beta1, beta2, eps, weight_decay, 0.0f, 0.0f, bias_corrections, slot,
                      stream);
}

extern "C" size_t ts_hip_adam_multi_waves(const ts_hip_adam_param *params, size_t count) {
    return adam_multi_blocks(params, count) * (kBlock / 64);
}

extern "C" int ts_hip_adam_step_multi_ticket(const ts_hip_adam_param *params, size_t count, float lr,
                                             float beta1, float beta2, float eps, float weight_decay,
                                             const float *bias_corrections, unsigned *tickets, void *stream) {
    if (!bias_corrections || !tickets) return TS_HIP_EINVAL;
    if ((reinterpret_cast<uintptr_t>(tickets) & 3u) != 0) return TS_HIP_EINVAL;
    return adam_multi(params, count, lr, beta1, beta2, eps, weight_decay, 0.0f, 0.0f, bias_corrections, nullptr,
                      stream, tickets);
}

extern "C" int ts_hip_adam_bias_corrections(float beta1, float beta2, uint64_t first_step, size_t count,
                                            float *out) {
    if (!out || first_step == 0) return TS_HIP_EINVAL;
    for (size_t i = 0; i < count; ++i) {
        out[2 * i] = correction_factor(beta1, first_step + i);
        out[2 * i + 1] = correction_factor(beta2, first_step + i);
    }
    return TS_HIP_OK;
}

extern "C" int ts_hip_slot_advance(unsigned *slot, void *stream) {
    if (!slot) return TS_HIP_EINVAL;
    launch(slot_advance_kernel, dim3(1), dim3(64), 0, as_stream(stream), slot);
    return launch_status();
}
