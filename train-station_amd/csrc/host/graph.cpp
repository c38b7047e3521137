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
// from a device table indexed by a replay counter that the graph's last node
// advances; the host fills the table before each run of replays with the
// values an eager step would use.
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
    Runtime &rt = Runtime::get();
    rt.sync();  // work queued before the recording runs eagerly, first
    auto g = std::make_unique<StepGraph>();
    DevicePool::get().pin_begin(&g->pins);
    const int st = ts_hip_stream_begin_capture(rt.stream());
    if (st != TS_HIP_OK) DevicePool::get().pin_end();
    check(st, "ts_hip_stream_begin_capture");
    graph_ = std::move(g);
}

StepRecorder::AdamSlot StepRecorder::adam_step(float beta1, float beta2, uint64_t step,
                                               std::vector<size_t> params) {
    if (!graph_) throw Error("no step recording is open");
    if (!graph_->slot) graph_->slot = std::make_shared<Allocation>(1);  // pinned: acquired while recording
    StepGraph::AdamUse u;
    u.table = std::make_shared<Allocation>(2 * kReplayChunk);
    u.beta1 = beta1;
    u.beta2 = beta2;
    u.first_step = step;
    u.steps = std::make_shared<ReplaySteps>();
    u.steps->params = std::move(params);
    graph_->adams.push_back(u);
    return {u.table->get(), reinterpret_cast<const unsigned *>(graph_->slot->get()), u.steps};
}

StepGraph *StepRecorder::end() {
    if (!graph_) throw Error("no step recording is open");
    std::unique_ptr<StepGraph> g = std::move(graph_);
    void *stream = Runtime::get().stream();
    // the last node moves the replay counter on to the next table entry
    const int adv = g->slot ? ts_hip_slot_advance(reinterpret_cast<unsigned *>(g->slot->get()), stream)
                            : TS_HIP_OK;
    void *exec = nullptr;
    const int st = ts_hip_stream_end_capture(stream, &exec);
    DevicePool::get().pin_end();
    g->exec = exec;
    if (adv != TS_HIP_OK || st != TS_HIP_OK) {
        g.reset();  // unpins
        check(adv != TS_HIP_OK ? adv : st, "recording the step");
    }
    return g.release();
}

void StepRecorder::abort() {
    if (!graph_) return;
    std::unique_ptr<StepGraph> g = std::move(graph_);
    void *exec = nullptr;
    (void)ts_hip_stream_end_capture(Runtime::get().stream(), &exec);
    DevicePool::get().pin_end();
    g->exec = exec;  // destroyed with g, which takes back the recorded step's count
}

StepGraph::~StepGraph() {
    // the optimizer counted the recorded step when it was recorded; a graph
    // that never ran (aborted, failed or freed unreplayed) takes that back
    if (!executed)
        for (AdamUse &u : adams) u.steps->pending -= 1;
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
        if (slot) {
            rt.sync();  // earlier replays have read their tables
            cf.resize(2 * chunk);
            for (AdamUse &u : adams) {
                check(ts_hip_adam_bias_corrections(u.beta1, u.beta2, u.first_step + executed, chunk, cf.data()),
                      "ts_hip_adam_bias_corrections");
                check(ts_hip_memcpy(u.table->get(), cf.data(), 2 * chunk, 0), "ts_hip_memcpy");
            }
            const unsigned zero = 0;
            check(ts_hip_memcpy(slot->get(), reinterpret_cast<const float *>(&zero), 1, 0), "ts_hip_memcpy");
        }
        for (size_t i = 0; i < chunk; ++i) check(ts_hip_graph_launch(exec, rt.stream()), "ts_hip_graph_launch");
        // the optimizer counted the recorded step when it was recorded; every
        // further replay is one more step
        const uint64_t extra_before = executed ? executed - 1 : 0;
        executed += chunk;
        for (AdamUse &u : adams) u.steps->pending += static_cast<int64_t>((executed - 1) - extra_before);
        done += chunk;
    }
}

}  // namespace ts
