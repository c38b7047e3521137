// gradtrack engine: the recorded graph, the no-grad switch and the backward
// worklist (gradtrack/engine.rs, gradtrack/no_grad_track.rs).
#include <algorithm>
#include <unordered_map>
#include <utility>
#include <vector>

#include "ts_hip.h"
#include "ts_host.h"

namespace ts {

namespace {

// engine.rs:175-187: operations id -> (input ids, GradFn); gradients id -> Tensor.
struct Graph {
    std::unordered_map<size_t, std::pair<std::vector<size_t>, GradFn>> operations;
    std::unordered_map<size_t, Tensor> gradients;
};

// Thread-local, as GRADTRACK_GRAPH (engine.rs:697-699).
Graph &graph() {
    thread_local Graph g;
    return g;
}

// no_grad_track.rs:16-22: thread-local stack, enabled by default.
std::vector<bool> &grad_stack() {
    thread_local std::vector<bool> s{true};
    return s;
}

// engine.rs:514-524: existing + new, in a new buffer.
void accumulate_gradient(size_t id, Tensor g) {
    auto &grads = graph().gradients;
    auto it = grads.find(id);
    if (it == grads.end()) {
        grads.emplace(id, std::move(g));
        return;
    }
    Tensor &existing = it->second;
    existing = add_gradients(existing, g);
}

}  // namespace

bool is_grad_enabled() { return grad_stack().back(); }
void push_grad_enabled(bool on) { grad_stack().push_back(on); }
void pop_grad_enabled() {
    std::vector<bool> &s = grad_stack();
    if (s.size() > 1) s.pop_back();
    else s.assign(1, true);  // an unbalanced pop restores the default state
}
void set_grad_enabled(bool on) { grad_stack().back() = on; }
bool gradients_pending() { return !graph().gradients.empty(); }

void clear_gradients() {
    graph().operations.clear();
    graph().gradients.clear();
}

void register_operation(size_t output_id, std::vector<size_t> input_ids, GradFn fn) {
    graph().operations.insert_or_assign(output_id, std::make_pair(std::move(input_ids), std::move(fn)));
}

const Tensor *accumulated_gradient(size_t id) {
    auto &grads = graph().gradients;
    auto it = grads.find(id);
    return it == grads.end() ? nullptr : &it->second;
}

namespace {
thread_local int g_backward_depth = 0;  // backward calls running on this thread
struct BackwardScope {
    BackwardScope() { ++g_backward_depth; }
    ~BackwardScope() { --g_backward_depth; }
};
}  // namespace

bool in_backward() { return g_backward_depth > 0; }

// engine.rs:962-1047
void engine_backward(Tensor &root, const Tensor *grad_output) {
    const BackwardScope scope;
    // backward(None) seeds ones; deferred, the seed is a constant of the
    // programs that read it and is written only if read elsewhere
    Tensor init = grad_output ? grad_output->alias() : Tensor::constant(root.dims(), 1.0f);
    if (init.dims() != root.dims() && init.size() != root.size())
        throw Error("backward: gradient shape does not match the tensor");
    root.accumulate_grad(init.alias());
    graph().gradients.insert_or_assign(root.id(), init.alias());  // store_gradient overwrites

    std::vector<size_t> worklist;
    worklist.reserve(128);
    worklist.push_back(root.id());
    while (!worklist.empty()) {
        const size_t node = worklist.back();
        worklist.pop_back();
        auto op = graph().operations.find(node);
        if (op == graph().operations.end()) continue;  // leaf: keep its gradient
        auto git = graph().gradients.find(node);
        if (git == graph().gradients.end()) continue;
        Tensor current = std::move(git->second);
        graph().gradients.erase(git);
        // operations is not modified below, so the reference stays valid
        const std::vector<size_t> &input_ids = op->second.first;
        std::vector<std::optional<Tensor>> grads = op->second.second.apply(current);
        for (size_t idx = 0; idx < input_ids.size(); ++idx) {
            if (idx >= grads.size() || !grads[idx]) continue;
            const size_t input_id = input_ids[idx];
            accumulate_gradient(input_id, std::move(*grads[idx]));
            grads[idx].reset();
            if (graph().operations.count(input_id)) worklist.push_back(input_id);
        }
    }
    // The gradients left are the leaves'; those still deferred run now, in as
    // few passes as they fit (they share their inputs): backward returns with
    // every gradient computed, as the reference's does.  They are merged in
    // tensor-id order: the map's own order follows its bucket history, and a
    // different merge order is a different program (and, for the programs
    // compiled at run time, a new compile) for the same step.
    std::vector<std::pair<size_t, std::shared_ptr<Allocation>>> leaves;
    for (auto &kv : graph().gradients)
        if (kv.second.allocation() && kv.second.allocation()->map) leaves.emplace_back(kv.first, kv.second.allocation());
    std::sort(leaves.begin(), leaves.end(),
              [](const auto &x, const auto &y) { return x.first < y.first; });
    std::vector<std::shared_ptr<Allocation>> deferred;
    for (auto &l : leaves) deferred.push_back(std::move(l.second));
    // (the root's seed, a deferred constant, reads no buffer and stays
    // deferred until read)
    if (root.grad_ref() && root.grad_ref()->allocation() && root.grad_ref()->allocation()->map &&
        !root.grad_ref()->allocation()->map->constant())
        deferred.push_back(root.grad_ref()->allocation());
    materialize_maps(deferred);
    // and the column sums (bias gradients) no weight-gradient product produced
    for (auto &kv : graph().gradients)
        if (kv.second.allocation() && kv.second.allocation()->colsum) kv.second.allocation()->get();
    if (root.grad_ref() && root.grad_ref()->allocation() && root.grad_ref()->allocation()->colsum)
        root.grad_ref()->allocation()->get();
}

}  // namespace ts
