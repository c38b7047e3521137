// C handle API (include/ts_gradtrack.h) over the C++ host classes.
#include <cstdlib>
#include <cstring>
#include <exception>
#include <string>

#include "ts_gradtrack.h"
#include "ts_hip.h"
#include "ts_host.h"

struct ts_tensor {
    ts::Tensor t;
};
struct ts_adam {
    ts::Adam a;
};

struct ts_step_graph {
    std::unique_ptr<ts::StepGraph> g;
};

namespace {

thread_local std::string g_last_error;

template <class F>
auto guard_ptr(F &&f) -> decltype(f()) {
    try {
        g_last_error.clear();
        return f();
    } catch (const std::exception &e) {
        g_last_error = e.what();
    } catch (...) {
        g_last_error = "unknown error";
    }
    return nullptr;
}

template <class F>
int guard_int(F &&f) {
    try {
        g_last_error.clear();
        f();
        return 0;
    } catch (const std::exception &e) {
        g_last_error = e.what();
    } catch (...) {
        g_last_error = "unknown error";
    }
    return -1;
}

ts_tensor *wrap(ts::Tensor &&t) { return new ts_tensor{std::move(t)}; }

std::vector<size_t> dims_of(const size_t *dims, size_t rank) {
    if (rank && !dims) throw ts::Error("dims pointer is NULL");
    return std::vector<size_t>(dims, dims + rank);
}

const ts::Tensor &T(const ts_tensor *h) {
    if (!h) throw ts::Error("tensor handle is NULL");
    return h->t;
}

std::vector<ts::Tensor *> param_list(ts_tensor *const *params, size_t count) {
    if (count && !params) throw ts::Error("parameter list is NULL");
    std::vector<ts::Tensor *> v;
    v.reserve(count);
    for (size_t i = 0; i < count; ++i) {
        if (!params[i]) throw ts::Error("parameter handle is NULL");
        v.push_back(&params[i]->t);
    }
    return v;
}

}  // namespace

extern "C" {

const char *ts_last_error(void) { return g_last_error.c_str(); }

ts_tensor *ts_tensor_new(const size_t *dims, size_t rank) {
    return guard_ptr([&] { return wrap(ts::Tensor::new_uninit(dims_of(dims, rank))); });
}
ts_tensor *ts_tensor_zeros(const size_t *dims, size_t rank) {
    return guard_ptr([&] { return wrap(ts::Tensor::zeros(dims_of(dims, rank))); });
}
ts_tensor *ts_tensor_ones(const size_t *dims, size_t rank) {
    return guard_ptr([&] { return wrap(ts::Tensor::ones(dims_of(dims, rank))); });
}
ts_tensor *ts_tensor_from_slice(const float *data, size_t len, const size_t *dims, size_t rank) {
    return guard_ptr([&] {
        if (len && !data) throw ts::Error("data pointer is NULL");
        return wrap(ts::Tensor::from_slice(data, len, dims_of(dims, rank)));
    });
}
ts_tensor *ts_tensor_randn(const size_t *dims, size_t rank, uint64_t seed, int has_seed) {
    return guard_ptr([&] { return wrap(ts::Tensor::randn(dims_of(dims, rank), has_seed ? &seed : nullptr)); });
}
int ts_tensor_fill_randn(ts_tensor *t, uint64_t seed, int has_seed) {
    return guard_int([&] {
        if (!t) throw ts::Error("tensor handle is NULL");
        t->t.fill_randn(has_seed ? &seed : nullptr);
    });
}
ts_tensor *ts_tensor_clone(const ts_tensor *t) {
    return guard_ptr([&] { return wrap(T(t).clone()); });
}
void ts_tensor_free(ts_tensor *t) { delete t; }

uint64_t ts_tensor_id(const ts_tensor *t) { return t ? t->t.id() : 0; }
size_t ts_tensor_rank(const ts_tensor *t) { return t ? t->t.dims().size() : 0; }
size_t ts_tensor_dims(const ts_tensor *t, size_t *out, size_t cap) {
    if (!t) return 0;
    const auto &d = t->t.dims();
    for (size_t i = 0; i < d.size() && i < cap; ++i) out[i] = d[i];
    return d.size();
}
size_t ts_tensor_size(const ts_tensor *t) { return t ? t->t.size() : 0; }
const float *ts_tensor_device_ptr(const ts_tensor *t) {
    return guard_ptr([&]() -> const float * { return t ? t->t.dev() : nullptr; });
}

int ts_tensor_with_requires_grad(ts_tensor *t) {
    return guard_int([&] {
        if (!t) throw ts::Error("tensor handle is NULL");
        t->t.with_requires_grad();
    });
}
int ts_tensor_set_requires_grad(ts_tensor *t, int r) {
    return guard_int([&] {
        if (!t) throw ts::Error("tensor handle is NULL");
        t->t.set_requires_grad(r != 0);
    });
}
int ts_tensor_requires_grad(const ts_tensor *t) { return t && t->t.requires_grad() ? 1 : 0; }

#define TS_BINARY(name, method)                                                   \
    ts_tensor *name(const ts_tensor *a, const ts_tensor *b) {                     \
        return guard_ptr([&] { return wrap(T(a).method(T(b))); });                \
    }
TS_BINARY(ts_tensor_add_tensor, add_tensor)
TS_BINARY(ts_tensor_sub_tensor, sub_tensor)
TS_BINARY(ts_tensor_mul_tensor, mul_tensor)
TS_BINARY(ts_tensor_div_tensor, div_tensor)
TS_BINARY(ts_tensor_matmul, matmul)
#undef TS_BINARY

#define TS_SCALAR(name, method)                                                   \
    ts_tensor *name(const ts_tensor *a, float s) {                                \
        return guard_ptr([&] { return wrap(T(a).method(s)); });                   \
    }
TS_SCALAR(ts_tensor_add_scalar, add_scalar)
TS_SCALAR(ts_tensor_sub_scalar, sub_scalar)
TS_SCALAR(ts_tensor_mul_scalar, mul_scalar)
TS_SCALAR(ts_tensor_div_scalar, div_scalar)
TS_SCALAR(ts_tensor_pow_scalar, pow_scalar)
#undef TS_SCALAR

ts_tensor *ts_tensor_relu(const ts_tensor *a) {
    return guard_ptr([&] { return wrap(T(a).relu()); });
}
ts_tensor *ts_tensor_exp(const ts_tensor *a) { return guard_ptr([&] { return wrap(T(a).exp()); }); }
ts_tensor *ts_tensor_log(const ts_tensor *a) { return guard_ptr([&] { return wrap(T(a).log()); }); }
ts_tensor *ts_tensor_sqrt(const ts_tensor *a) { return guard_ptr([&] { return wrap(T(a).sqrt()); }); }
ts_tensor *ts_tensor_tanh(const ts_tensor *a) { return guard_ptr([&] { return wrap(T(a).tanh()); }); }
ts_tensor *ts_tensor_sigmoid(const ts_tensor *a) { return guard_ptr([&] { return wrap(T(a).sigmoid()); }); }
ts_tensor *ts_tensor_leaky_relu(const ts_tensor *a, float negative_slope) {
    return guard_ptr([&] { return wrap(T(a).leaky_relu(negative_slope)); });
}
ts_tensor *ts_tensor_softmax(const ts_tensor *a, size_t dim) {
    return guard_ptr([&] { return wrap(T(a).softmax(dim)); });
}
ts_tensor *ts_tensor_sum_dims(const ts_tensor *a, const size_t *dims, size_t ndims, int keepdim) {
    return guard_ptr([&] { return wrap(T(a).sum_dims(dims_of(dims, ndims), keepdim != 0)); });
}
ts_tensor *ts_tensor_mean_dims(const ts_tensor *a, const size_t *dims, size_t ndims, int keepdim) {
    return guard_ptr([&] { return wrap(T(a).mean_dims(dims_of(dims, ndims), keepdim != 0)); });
}
ts_tensor *ts_tensor_transpose(const ts_tensor *a, size_t dim0, size_t dim1) {
    return guard_ptr([&] { return wrap(T(a).transpose(dim0, dim1)); });
}
ts_tensor *ts_tensor_t(const ts_tensor *a) { return guard_ptr([&] { return wrap(T(a).t()); }); }
ts_tensor *ts_tensor_contiguous(const ts_tensor *a) {
    return guard_ptr([&] { return wrap(T(a).contiguous()); });
}
int ts_tensor_is_contiguous(const ts_tensor *a) { return a && a->t.is_contiguous() ? 1 : 0; }
int ts_tensor_fill(ts_tensor *t, float value) {
    return guard_int([&] {
        if (!t) throw ts::Error("tensor handle is NULL");
        t->t.fill(value);
    });
}
ts_tensor *ts_tensor_sum(const ts_tensor *a) {
    return guard_ptr([&] { return wrap(T(a).sum()); });
}
ts_tensor *ts_tensor_mean(const ts_tensor *a) {
    return guard_ptr([&] { return wrap(T(a).mean()); });
}

int ts_tensor_backward(ts_tensor *t, const ts_tensor *grad_output) {
    return guard_int([&] {
        if (!t) throw ts::Error("tensor handle is NULL");
        t->t.backward(grad_output ? &grad_output->t : nullptr);
    });
}

ts_tensor *ts_tensor_grad(const ts_tensor *t) {
    return guard_ptr([&]() -> ts_tensor * {
        const ts::Tensor *g = T(t).grad_direct();
        if (!g) return nullptr;
        return wrap(g->view());
    });
}

ts_tensor *ts_tensor_grad_by_value(const ts_tensor *t) {
    return guard_ptr([&]() -> ts_tensor * {
        auto g = T(t).grad_by_value();
        if (!g) return nullptr;
        return wrap(std::move(*g));
    });
}

int ts_tensor_set_grad(ts_tensor *t, const ts_tensor *grad) {
    return guard_int([&] {
        if (!t) throw ts::Error("tensor handle is NULL");
        t->t.set_grad(T(grad).clone());
    });
}
int ts_tensor_zero_grad(ts_tensor *t) {
    return guard_int([&] {
        if (!t) throw ts::Error("tensor handle is NULL");
        t->t.zero_grad();
    });
}

int ts_tensor_data(const ts_tensor *t, float *out, size_t len) {
    return guard_int([&] {
        if (len && !out) throw ts::Error("output pointer is NULL");
        T(t).copy_to_host(out, len);
    });
}
int ts_tensor_value(const ts_tensor *t, float *out) {
    return guard_int([&] {
        if (!out) throw ts::Error("output pointer is NULL");
        *out = T(t).value();
    });
}

void ts_clear_gradients(void) { ts::clear_gradients(); }
void ts_no_grad_push(void) { ts::push_grad_enabled(false); }
void ts_no_grad_pop(void) { ts::pop_grad_enabled(); }
int ts_is_grad_enabled(void) { return ts::is_grad_enabled() ? 1 : 0; }
void ts_set_grad_enabled(int enabled) { ts::set_grad_enabled(enabled != 0); }

ts_adam *ts_adam_new(void) {
    return guard_ptr([&] { return new ts_adam{ts::Adam()}; });
}
ts_adam *ts_adam_with_config(float lr, float b1, float b2, float eps, float wd, int amsgrad) {
    return guard_ptr([&] {
        ts::AdamConfig c;
        c.learning_rate = lr;
        c.beta1 = b1;
        c.beta2 = b2;
        c.eps = eps;
        c.weight_decay = wd;
        c.amsgrad = amsgrad != 0;
        return new ts_adam{ts::Adam::with_config(c)};
    });
}
ts_adam *ts_adam_with_learning_rate(float lr) {
    return guard_ptr([&] { return new ts_adam{ts::Adam::with_learning_rate(lr)}; });
}
void ts_adam_free(ts_adam *opt) { delete opt; }

int ts_adam_add_parameter(ts_adam *opt, const ts_tensor *param) {
    return guard_int([&] {
        if (!opt) throw ts::Error("optimizer handle is NULL");
        opt->a.add_parameter(T(param));
    });
}
int ts_adam_step(ts_adam *opt, ts_tensor *const *params, size_t count) {
    return guard_int([&] {
        if (!opt) throw ts::Error("optimizer handle is NULL");
        opt->a.step(param_list(params, count));
    });
}
int ts_adam_zero_grad(ts_adam *opt, ts_tensor *const *params, size_t count) {
    return guard_int([&] {
        if (!opt) throw ts::Error("optimizer handle is NULL");
        opt->a.zero_grad(param_list(params, count));
    });
}
float ts_adam_learning_rate(const ts_adam *opt) { return opt ? opt->a.learning_rate() : 0.0f; }
void ts_adam_set_learning_rate(ts_adam *opt, float lr) {
    if (opt) opt->a.set_learning_rate(lr);
}
uint64_t ts_adam_step_count(const ts_adam *opt) { return opt ? opt->a.step_count() : 0; }

int ts_adam_state(const ts_adam *opt, const ts_tensor *param, int which, float *out, size_t len) {
    return guard_int([&] {
        if (!opt) throw ts::Error("optimizer handle is NULL");
        const ts::Tensor &p = T(param);
        const float *src = which == 0 ? opt->a.state_m(p.id()) : opt->a.state_v(p.id());
        if (!src) throw ts::Error("parameter is not linked to this optimizer");
        if (len != p.size()) throw ts::Error("state buffer length mismatch");
        ts::refuse_while_recording("adam state");
        ts::check(ts_hip_memcpy_async(out, src, len, 1, ts::Runtime::get().stream()),
                  "ts_hip_memcpy_async");
        ts::Runtime::get().sync();
    });
}

// ---- checkpoint / resume ------------------------------------------------------------

void ts_buffer_free(void *data) { std::free(data); }

}  // extern "C"

namespace {

template <class Bytes>
void give_bytes(const Bytes &b, uint8_t **data, size_t *len) {
    if (!data || !len) throw ts::Error("output pointer is NULL");
    void *p = std::malloc(b.size() ? b.size() : 1);
    if (!p) throw ts::Error("out of host memory");
    if (b.size()) std::memcpy(p, b.data(), b.size());
    *data = static_cast<uint8_t *>(p);
    *len = b.size();
}

void give_text(const std::string &s, char **out, size_t *len) {
    if (!out || !len) throw ts::Error("output pointer is NULL");
    char *p = static_cast<char *>(std::malloc(s.size() + 1));
    if (!p) throw ts::Error("out of host memory");
    std::memcpy(p, s.data(), s.size());
    p[s.size()] = '\0';
    *out = p;
    *len = s.size();
}

std::string text_of(const char *json, size_t len) {
    if (len && !json) throw ts::Error("JSON pointer is NULL");
    return std::string(json ? json : "", len);
}

const char *path_of(const char *path) {
    if (!path) throw ts::Error("path is NULL");
    return path;
}

ts::Adam &A(ts_adam *h) {
    if (!h) throw ts::Error("optimizer handle is NULL");
    return h->a;
}
const ts::Adam &A(const ts_adam *h) {
    if (!h) throw ts::Error("optimizer handle is NULL");
    return h->a;
}

ts::AdamConfig config_of(const float *v, int amsgrad) {
    if (!v) throw ts::Error("config values pointer is NULL");
    ts::AdamConfig c;
    c.learning_rate = v[0];
    c.beta1 = v[1];
    c.beta2 = v[2];
    c.eps = v[3];
    c.weight_decay = v[4];
    c.amsgrad = amsgrad != 0;
    return c;
}

void put_config(const ts::AdamConfig &c, float *v, int *amsgrad) {
    if (!v || !amsgrad) throw ts::Error("output pointer is NULL");
    v[0] = c.learning_rate;
    v[1] = c.beta1;
    v[2] = c.beta2;
    v[3] = c.eps;
    v[4] = c.weight_decay;
    *amsgrad = c.amsgrad ? 1 : 0;
}

}  // namespace

extern "C" {

int ts_tensor_to_binary(const ts_tensor *t, uint8_t **data, size_t *len) {
    return guard_int([&] { give_bytes(T(t).to_binary(), data, len); });
}
ts_tensor *ts_tensor_from_binary(const uint8_t *data, size_t len) {
    return guard_ptr([&] {
        if (len && !data) throw ts::Error("data pointer is NULL");
        return wrap(ts::Tensor::from_binary(data, len));
    });
}
int ts_tensor_to_json(const ts_tensor *t, char **json, size_t *len) {
    return guard_int([&] { give_text(T(t).to_json(), json, len); });
}
ts_tensor *ts_tensor_from_json(const char *json, size_t len) {
    return guard_ptr([&] { return wrap(ts::Tensor::from_json(text_of(json, len))); });
}
int ts_tensor_save_binary(const ts_tensor *t, const char *path) {
    return guard_int([&] { T(t).save_binary(path_of(path)); });
}
int ts_tensor_save_json(const ts_tensor *t, const char *path) {
    return guard_int([&] { T(t).save_json(path_of(path)); });
}
ts_tensor *ts_tensor_load_binary(const char *path) {
    return guard_ptr([&] { return wrap(ts::Tensor::load_binary(path_of(path))); });
}
ts_tensor *ts_tensor_load_json(const char *path) {
    return guard_ptr([&] { return wrap(ts::Tensor::load_json(path_of(path))); });
}

int ts_adam_to_binary(const ts_adam *opt, uint8_t **data, size_t *len) {
    return guard_int([&] { give_bytes(A(opt).to_binary(), data, len); });
}
ts_adam *ts_adam_from_binary(const uint8_t *data, size_t len) {
    return guard_ptr([&] {
        if (len && !data) throw ts::Error("data pointer is NULL");
        return new ts_adam{ts::Adam::from_binary(data, len)};
    });
}
int ts_adam_to_json(const ts_adam *opt, char **json, size_t *len) {
    return guard_int([&] { give_text(A(opt).to_json(), json, len); });
}
ts_adam *ts_adam_from_json(const char *json, size_t len) {
    return guard_ptr([&] { return new ts_adam{ts::Adam::from_json(text_of(json, len))}; });
}
int ts_adam_save_binary(const ts_adam *opt, const char *path) {
    return guard_int([&] { A(opt).save_binary(path_of(path)); });
}
int ts_adam_save_json(const ts_adam *opt, const char *path) {
    return guard_int([&] { A(opt).save_json(path_of(path)); });
}
ts_adam *ts_adam_load_binary(const char *path) {
    return guard_ptr([&] { return new ts_adam{ts::Adam::load_binary(path_of(path))}; });
}
ts_adam *ts_adam_load_json(const char *path) {
    return guard_ptr([&] { return new ts_adam{ts::Adam::load_json(path_of(path))}; });
}
int ts_adam_relink_parameters(ts_adam *opt, const ts_tensor *const *params, size_t count) {
    return guard_int([&] {
        if (count && !params) throw ts::Error("parameter list is NULL");
        std::vector<const ts::Tensor *> ps;
        for (size_t i = 0; i < count; ++i) ps.push_back(&T(params[i]));
        A(opt).relink_parameters(ps);
    });
}
size_t ts_adam_saved_parameter_count(const ts_adam *opt) { return opt ? opt->a.saved_parameter_count() : 0; }
uint64_t ts_adam_parameter_step(const ts_adam *opt, const ts_tensor *param) {
    return (opt && param) ? opt->a.parameter_step(param->t.id()) : 0;
}
int ts_adam_config(const ts_adam *opt, float *values5, int *amsgrad) {
    return guard_int([&] { put_config(A(opt).config(), values5, amsgrad); });
}
int ts_adam_config_to_binary(const float *values5, int amsgrad, uint8_t **data, size_t *len) {
    return guard_int([&] { give_bytes(ts::adam_config_to_binary(config_of(values5, amsgrad)), data, len); });
}
int ts_adam_config_from_binary(const uint8_t *data, size_t len, float *values5, int *amsgrad) {
    return guard_int([&] {
        if (len && !data) throw ts::Error("data pointer is NULL");
        put_config(ts::adam_config_from_binary(data, len), values5, amsgrad);
    });
}
int ts_adam_config_to_json(const float *values5, int amsgrad, char **json, size_t *len) {
    return guard_int([&] { give_text(ts::adam_config_to_json(config_of(values5, amsgrad)), json, len); });
}
int ts_adam_config_from_json(const char *json, size_t len, float *values5, int *amsgrad) {
    return guard_int([&] { put_config(ts::adam_config_from_json(text_of(json, len)), values5, amsgrad); });
}

void ts_fusion_enable(int on) { ts::set_fusion(on != 0); }
int ts_fusion_enabled(void) { return ts::fusion_enabled() ? 1 : 0; }

int ts_step_graph_begin(void) {
    return guard_int([&] { ts::StepRecorder::get().begin(); });
}
ts_step_graph *ts_step_graph_end(void) {
    return guard_ptr([&] { return new ts_step_graph{std::unique_ptr<ts::StepGraph>(ts::StepRecorder::get().end())}; });
}
void ts_step_graph_abort(void) {
    try {
        ts::StepRecorder::get().abort();
    } catch (...) {
    }
}
int ts_step_graph_recording(void) { return ts::StepRecorder::get().open() ? 1 : 0; }
int ts_step_graph_replay(ts_step_graph *g, size_t times) {
    return guard_int([&] {
        if (!g) throw ts::Error("null step graph");
        g->g->replay(times);
    });
}
void ts_step_graph_free(ts_step_graph *g) { delete g; }

int ts_synchronize(void) {
    return guard_int([&] { ts::Runtime::get().sync(); });
}
void *ts_stream(void) {
    try {
        return ts::Runtime::get().stream();
    } catch (...) {
        return nullptr;
    }
}
size_t ts_pool_live_bytes(void) { return ts::DevicePool::get().live_bytes(); }
size_t ts_pool_cached_bytes(void) { return ts::DevicePool::get().cached_bytes(); }
void ts_pool_empty_cache(void) {
    try {
        ts::Runtime::get().sync();
    } catch (...) {
    }
    ts::DevicePool::get().empty_cache();
}

void ts_profile_classes(unsigned mask) { ts::Profiler::get().set_classes(mask); }

void ts_profile_enable(int on) {
    try {
        ts::Profiler::get().enable(on != 0);
    } catch (const std::exception &e) {
        g_last_error = e.what();
    }
}
void ts_profile_reset(void) {
    try {
        ts::Profiler::get().reset();
    } catch (const std::exception &e) {
        g_last_error = e.what();
    }
}
int ts_profile_read(int k, double *ms, double *work, uint64_t *launches) {
    return guard_int([&] {
        if (k < 0 || k >= static_cast<int>(ts::KernelClass::kCount))
            throw ts::Error("kernel class out of range");
        ts::Profiler::get().collect();
        ts::ClassStats s = ts::Profiler::get().stats(static_cast<ts::KernelClass>(k));
        if (ms) *ms = s.ms;
        if (work) *work = s.work;
        if (launches) *launches = s.launches;
    });
}

}  // extern "C"
