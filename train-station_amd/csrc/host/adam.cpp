// Adam optimizer over device parameters (optimizers/adam/mod.rs).  Per-param
// state m / v (and v_hat_max under AMSGrad) lives in pooled device buffers;
// each step is one fused kernel per parameter.
#include <cstdio>
#include <optional>

#include "ts_hip.h"
#include "ts_host.h"

namespace ts {

Adam Adam::with_config(AdamConfig c) {
    Adam a;
    a.config_ = c;
    return a;
}

Adam Adam::with_learning_rate(float lr) {
    AdamConfig c;
    c.learning_rate = lr;
    return with_config(c);
}

// adam/mod.rs:287-307
void Adam::add_parameter(const Tensor &p) {
    if (!p.requires_grad()) throw Error("Parameter must require gradients");
    if (states_.count(p.id())) return;
    // the state's zero fill would be recorded and so rerun by every replay
    if (StepRecorder::get().open())
        throw Error("add_parameter: link parameters to the optimizer before recording a step");
    State s;
    s.n = p.size();
    s.dims = p.dims();
    if (s.n) {
        s.m = std::make_shared<Allocation>(s.n);
        s.v = std::make_shared<Allocation>(s.n);
        void *st = Runtime::get().stream();
        check(ts_hip_fill(s.m->get(), 0.0f, s.n, st), "ts_hip_fill");
        check(ts_hip_fill(s.v->get(), 0.0f, s.n, st), "ts_hip_fill");
    }
    states_.emplace(p.id(), std::move(s));
    insertion_order_.push_back(p.id());
}

void Adam::add_parameters(const std::vector<const Tensor *> &ps) {
    for (const Tensor *p : ps) add_parameter(*p);
}

void Adam::settle() const {
    if (ledger_->param_delta.empty()) return;
    for (const auto &d : ledger_->param_delta) {
        auto it = states_.find(d.first);
        if (it != states_.end()) it->second.step += static_cast<uint64_t>(d.second);  // wraps correctly for < 0
    }
    ledger_->param_delta.clear();
}

void Adam::step(const std::vector<Tensor *> &params) {
    settle();
    // While a step is being recorded, the launches read their bias
    // corrections from the recording's table (each replay is a later step).
    StepRecorder &rec = StepRecorder::get();
    const bool recording = rec.open();
    if (recording && config_.amsgrad)  // a replay would restart the running maximum every step
        for (Tensor *p : params) {
            auto it = states_.find(p->id());
            if (it != states_.end() && p->grad_ref() && it->second.n && !it->second.v_hat_max)
                throw Error("record an AMSGrad step only after the optimizer's first step");
        }
    // registered before anything is counted, so the end or abort of the
    // recording takes back exactly what this call counted
    std::optional<StepRecorder::AdamSlot> slot;
    if (recording) slot = rec.adam_step(config_.beta1, config_.beta2, ledger_);
    ledger_->step_count += 1;  // adam/mod.rs:1037
    const uint64_t step_count = ledger_->step_count;
    std::vector<ts_hip_adam_param> batch;
    double bytes = 0.0;
    auto flush = [&]() {
        if (batch.empty()) return;
        launch(KernelClass::Adam, bytes, "ts_hip_adam_step_multi", [&] {
            void *st = Runtime::get().stream();
            if (slot)
                return ts_hip_adam_step_multi_ticket(batch.data(), batch.size(), config_.learning_rate,
                                                     config_.beta1, config_.beta2, config_.eps,
                                                     config_.weight_decay, slot->table,
                                                     rec.adam_tickets(ts_hip_adam_multi_waves(batch.data(), batch.size())),
                                                     st);
            return ts_hip_adam_step_multi(batch.data(), batch.size(), config_.learning_rate, config_.beta1,
                                          config_.beta2, config_.eps, config_.weight_decay, step_count, st);
        });
        batch.clear();
        bytes = 0.0;
    };
    for (Tensor *p : params) {
        auto it = states_.find(p->id());
        if (it == states_.end())  // adam/mod.rs:489-492
            throw Error(
                "Parameter must be linked to optimizer before stepping. Use add_parameter() first.");
        const Tensor *g = p->grad_ref();
        if (!g) {  // adam/mod.rs:1040-1042
            std::fprintf(stderr, "Warning: Failed to update parameter: Parameter %zu has no gradient\n",
                         p->id());
            continue;
        }
        State &s = it->second;
        if (g->size() != p->size() || s.n != p->size())
            throw Error("Momentum and gradient size mismatch");
        s.step += 1;
        if (slot) rec.adam_param(slot->use, p->id());
        int first = 0;
        if (config_.amsgrad && !s.v_hat_max && s.n) {
            s.v_hat_max = std::make_shared<Allocation>(s.n);
            first = 1;
        }
        if (!s.n) continue;
        // p is updated in place: deferred products reading it run first
        if (p->allocation()) p->allocation()->before_write();
        // parameters are independent: one launch steps up to 16 of them; a
        // parameter listed twice is stepped twice in order, so it starts a new launch
        for (const ts_hip_adam_param &q : batch)
            if (q.p == p->dev_mut()) {
                flush();
                break;
            }
        batch.push_back(ts_hip_adam_param{p->dev_mut(), g->dev(), s.m->get(), s.v->get(),
                                          config_.amsgrad ? s.v_hat_max->get() : nullptr, s.n, first});
        bytes += 28.0 * s.n + (config_.amsgrad ? 8.0 * s.n : 0.0);
        if (batch.size() == TS_HIP_ADAM_MAX_PARAMS) flush();
    }
    flush();
}

void Adam::zero_grad(const std::vector<Tensor *> &params) {
    for (Tensor *p : params) p->zero_grad();
    clear_gradients();
}

uint64_t Adam::parameter_step(size_t id) const {
    settle();
    auto it = states_.find(id);
    return it == states_.end() ? 0 : it->second.step;
}

const float *Adam::state_m(size_t id) const {
    auto it = states_.find(id);
    return (it == states_.end() || !it->second.m) ? nullptr : it->second.m->get();
}

const float *Adam::state_v(size_t id) const {
    auto it = states_.find(id);
    return (it == states_.end() || !it->second.v) ? nullptr : it->second.v->get();
}

}  // namespace ts
