// Recording one training step as a HIP graph and replaying it (no
// counterpart in the reference, whose steps run eagerly on the CPU).  For
// steps short enough that host work and launch latency dominate, a replay
// issues the whole recorded step as one graph launch.
//
// The recording is HIP stream capture of the library stream: the ops,
// backward and Adam::step issued between begin and end are recorded, not
// run.  Everything the recorded launches touch stays valid for the graph's
// life: the pool pins every block acquired or used while recording and
// parks, instead of reusing, any of them released meanwhile.  Adam's bias
// corrections depend on the step count, so a recorded Adam::step reads them
// from a device table: each wave of a recorded Adam launch counts its own
// launches in a ticket word and reads the entry of its replay, so no launch of
// its own advances a counter; before each run of replays the host clears the
// tickets and fills the table with the values eager steps would use from the
// optimizer's count at that moment.
#include <algorithm>

#include "ts_hip.h"
#include "ts_host.h"

namespace ts {

StepRecorder &StepRecorder::get() {
    static StepRecorder *r = new StepRecorder();
    return *r;
}

void StepRecorder::begin() {
    if (graph_) throw Error("a step recording is already open");
    if (Profiler::get().enabled()) throw Error("disable the profiler before recording a step");
    if (gradients_pending())
        throw Error("a step can be recorded only while no gradients are held: call zero_grad (or "
                    "clear_gradients) first, and end the recorded step with zero_grad");
    Runtime &rt = Runtime::get();
    rt.sync();  // work queued before the recording runs eagerly, first
    auto g = std::make_unique<StepGraph>();
    DevicePool::get().pin_begin(&g->pins);
    const int st = ts_hip_stream_begin_capture(rt.stream());
    if (st != TS_HIP_OK) DevicePool::get().pin_end();
    check(st, "ts_hip_stream_begin_capture");
    graph_ = std::move(g);
}

StepRecorder::AdamSlot StepRecorder::adam_step(float beta1, float beta2, const std::shared_ptr<AdamLedger> &ledger) {
    if (!graph_) throw Error("no step recording is open");
    StepGraph::AdamUse u;
    u.table = std::make_shared<Allocation>(2 * kReplayChunk);
    u.beta1 = beta1;
    u.beta2 = beta2;
    u.ledger = ledger;
    for (const StepGraph::AdamUse &o : graph_->adams)
        if (o.ledger == ledger) ++u.order;
    graph_->adams.push_back(std::move(u));
    const StepGraph::AdamUse &b = graph_->adams.back();
    return {b.table->get(), graph_->adams.size() - 1};
}

unsigned *StepRecorder::adam_tickets(size_t waves) {
    if (!graph_) throw Error("no step recording is open");
    graph_->tickets.push_back(std::make_shared<Allocation>(waves));  // pinned: acquired while recording
    return reinterpret_cast<unsigned *>(graph_->tickets.back()->get());
}

void StepRecorder::adam_param(size_t use, size_t param_id) {
    if (!graph_ || use >= graph_->adams.size()) throw Error("no recorded optimizer step to add a parameter to");
    graph_->adams[use].params.push_back(param_id);
}

void StepRecorder::take_back(StepGraph &g) {
    for (StepGraph::AdamUse &u : g.adams) {
        u.ledger->step_count -= 1;
        for (size_t id : u.params) u.ledger->param_delta[id] -= 1;
    }
    for (StepGraph::AdamUse &u : g.adams) {
        u.per_replay = 0;
        for (const StepGraph::AdamUse &o : g.adams)
            if (o.ledger == u.ledger) ++u.per_replay;
    }
}

StepGraph *StepRecorder::end() {
    if (!graph_) throw Error("no step recording is open");
    std::unique_ptr<StepGraph> g = std::move(graph_);
    take_back(*g);
    void *stream = Runtime::get().stream();
    void *exec = nullptr;
    const int st = ts_hip_stream_end_capture(stream, &exec);
    DevicePool::get().pin_end();
    g->exec = exec;
    if (st != TS_HIP_OK) {
        g.reset();  // unpins
        check(st, "recording the step");
    }
    return g.release();
}

void StepRecorder::abort() {
    if (!graph_) return;
    std::unique_ptr<StepGraph> g = std::move(graph_);
    take_back(*g);
    void *exec = nullptr;
    (void)ts_hip_stream_end_capture(Runtime::get().stream(), &exec);
    DevicePool::get().pin_end();
    g->exec = exec;
}

StepGraph::~StepGraph() {
    if (exec) {
        // replays may still be running
        (void)ts_hip_stream_synchronize(Runtime::get().stream());
        (void)ts_hip_graph_destroy(exec);
    }
    DevicePool::get().unpin(pins);
}

void StepGraph::replay(size_t times) {
    if (StepRecorder::get().open()) throw Error("cannot replay a step while another is being recorded");
    if (!exec) throw Error("the step graph holds no recording");
    Runtime &rt = Runtime::get();
    std::vector<float> cf;
    for (size_t done = 0; done < times;) {
        const size_t chunk = std::min(times - done, StepRecorder::kReplayChunk);
        if (!adams.empty()) {
            rt.sync();  // earlier replays have read their tables and tickets
            cf.resize(2 * chunk);
            for (AdamUse &u : adams) {
                // replay i runs this optimizer's recorded steps as its steps
                // count + i*per_replay + 1 .. + per_replay, in recorded order,
                // from the count it has now (eager steps and other graphs
                // included)
                const uint64_t base = u.ledger->step_count + u.order + 1;
                if (u.per_replay == 1) {
                    check(ts_hip_adam_bias_corrections(u.beta1, u.beta2, base, chunk, cf.data()),
                          "ts_hip_adam_bias_corrections");
                } else {
                    for (size_t i = 0; i < chunk; ++i)
                        check(ts_hip_adam_bias_corrections(u.beta1, u.beta2, base + i * u.per_replay, 1,
                                                           cf.data() + 2 * i),
                              "ts_hip_adam_bias_corrections");
                }
                check(ts_hip_memcpy(u.table->get(), cf.data(), 2 * chunk, 0), "ts_hip_memcpy");
            }
            for (auto &t : tickets) {
                const std::vector<float> zeros(t->n, 0.0f);  // all bits 0: tickets of 0
                check(ts_hip_memcpy(t->get(), zeros.data(), t->n, 0), "ts_hip_memcpy");
            }
        }
        for (size_t i = 0; i < chunk; ++i) check(ts_hip_graph_launch(exec, rt.stream()), "ts_hip_graph_launch");
        executed += chunk;
        for (AdamUse &u : adams) {
            u.ledger->step_count += chunk;
            for (size_t id : u.params) u.ledger->param_delta[id] += static_cast<int64_t>(chunk);
        }
        done += chunk;
    }
}

}  // namespace ts
