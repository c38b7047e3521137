// Runtime pieces of the host library: status checking, the library stream,
// the division-by-zero word, the device buffer pool and the event profiler.
#include <cstdio>
#include <cstring>
#include <mutex>

#include "ts_hip.h"
#include "ts_host.h"

namespace ts {

void check(int status, const char *what) {
    if (status != TS_HIP_OK)
        throw Error(std::string(what) + ": " + ts_hip_error_string(status) + " (status " +
                    std::to_string(status) + ")");
}

static const unsigned long long kNoZero = ~0ull;

Runtime::Runtime() {
    check(ts_hip_initialize(), "ts_hip_initialize");
    check(ts_hip_stream_create(&stream_), "ts_hip_stream_create");
    float *w = nullptr;
    check(ts_hip_malloc(&w, 2), "ts_hip_malloc(zero index)");
    zero_index_ = reinterpret_cast<unsigned long long *>(w);
    check(ts_hip_memcpy(w, reinterpret_cast<const float *>(&kNoZero), 2, 0), "ts_hip_memcpy");
}

Runtime &Runtime::get() {
    // Never destroyed: tensors may outlive static destruction order.
    static Runtime *rt = new Runtime();
    return *rt;
}

void Runtime::sync() {
    if (StepRecorder::get().open())
        throw Error("a step being recorded cannot wait for or read device results: end the recording first");
    run_division_checks();  // quotients never read still check their divisors
    check(ts_hip_stream_synchronize(stream_), "ts_hip_stream_synchronize");
    unsigned long long idx = kNoZero;
    check(ts_hip_memcpy(reinterpret_cast<float *>(&idx),
                        reinterpret_cast<const float *>(zero_index_), 2, 1),
          "ts_hip_memcpy");
    if (idx != kNoZero) {
        check(ts_hip_memcpy(reinterpret_cast<float *>(zero_index_),
                            reinterpret_cast<const float *>(&kNoZero), 2, 0),
              "ts_hip_memcpy");
        // ops/div.rs:383-416
        throw Error("Division by zero detected at index " + std::to_string(idx));
    }
}

// ---- pool ---------------------------------------------------------------------

static std::mutex g_pool_mutex;

static size_t round_floats(size_t n) {
    if (n <= 1024) return (n + 63) & ~size_t(63);            // 256-byte granules
    if (n <= (size_t(1) << 20)) return (n + 1023) & ~size_t(1023);
    return (n + 65535) & ~size_t(65535);                      // 256 KiB granules
}

DevicePool &DevicePool::get() {
    static DevicePool *p = new DevicePool();
    return *p;
}

float *DevicePool::acquire(size_t n_floats, size_t *rounded) {
    Runtime::get();
    const size_t r = round_floats(n_floats == 0 ? 1 : n_floats);
    *rounded = r;
    {
        std::lock_guard<std::mutex> lock(g_pool_mutex);
        auto it = free_.find(r);
        if (it != free_.end() && !it->second.empty()) {
            float *p = it->second.back();
            it->second.pop_back();
            cached_ -= r * sizeof(float);
            live_ += r * sizeof(float);
            if (sink_) pin(p);
            return p;
        }
    }
    float *p = nullptr;
    int st = ts_hip_malloc(&p, r);
    // Return cached blocks to the device and retry once.  That needs a wait
    // for queued work, which a step being recorded cannot do: there the
    // allocation failure itself is reported.
    if (st != TS_HIP_OK && !pinning_.load(std::memory_order_relaxed)) {
        Runtime::get().sync();
        empty_cache();
        st = ts_hip_malloc(&p, r);
    }
    if (st != TS_HIP_OK)
        throw Error("ts_hip_malloc of " + std::to_string(r * sizeof(float)) + " bytes failed (" +
                    ts_hip_error_string(st) + ")");
    std::lock_guard<std::mutex> lock(g_pool_mutex);
    live_ += r * sizeof(float);
    if (sink_) pin(p);
    return p;
}

void DevicePool::release(float *p, size_t rounded) {
    if (!p) return;
    std::lock_guard<std::mutex> lock(g_pool_mutex);
    if (pins_.count(p)) {  // a recorded step still uses it: park until unpinned
        parked_[p] = rounded;
        return;
    }
    free_[rounded].push_back(p);
    live_ -= rounded * sizeof(float);
    cached_ += rounded * sizeof(float);
}

void DevicePool::pin_begin(std::vector<float *> *sink) {
    std::lock_guard<std::mutex> lock(g_pool_mutex);
    sink_ = sink;
    sink_set_.clear();
    pinning_.store(true, std::memory_order_relaxed);
}

void DevicePool::pin_end() {
    std::lock_guard<std::mutex> lock(g_pool_mutex);
    sink_ = nullptr;
    sink_set_.clear();
    pinning_.store(false, std::memory_order_relaxed);
}

void DevicePool::pin_locked(float *p) {
    std::lock_guard<std::mutex> lock(g_pool_mutex);
    if (sink_) pin(p);
}

void DevicePool::pin(float *p) {
    if (!p || !sink_set_.insert(p).second) return;  // once per recording
    ++pins_[p];
    sink_->push_back(p);
}

void DevicePool::unpin(const std::vector<float *> &blocks) {
    std::lock_guard<std::mutex> lock(g_pool_mutex);
    for (float *p : blocks) {
        auto it = pins_.find(p);
        if (it == pins_.end() || --it->second > 0) continue;
        pins_.erase(it);
        auto pk = parked_.find(p);
        if (pk == parked_.end()) continue;  // still owned: released normally later
        free_[pk->second].push_back(p);
        live_ -= pk->second * sizeof(float);
        cached_ += pk->second * sizeof(float);
        parked_.erase(pk);
    }
}

void DevicePool::empty_cache() {
    std::lock_guard<std::mutex> lock(g_pool_mutex);
    for (auto &kv : free_)
        for (float *p : kv.second) ts_hip_free(p);
    free_.clear();
    cached_ = 0;
}

Allocation::Allocation(size_t n_floats) : n(n_floats) {
    ptr_ = DevicePool::get().acquire(n_floats, &rounded);
}

Allocation::~Allocation() { DevicePool::get().release(ptr_, rounded); }

float *Allocation::get() {
    if (pending) materialize(*this);
    else if (map) materialize_map(*this);
    else if (colsum) materialize_colsum(*this);
    else if (transpose) materialize_transpose(*this);
    else if (reduce) materialize_reduce(*this);
    else if (sibling) run_sibling(*this);
    DevicePool::get().note_use(ptr_);
    return ptr_;
}

void Allocation::before_write() {
    std::vector<std::weak_ptr<Allocation>> rs;
    rs.swap(readers);
    for (auto &w : rs)
        if (auto r = w.lock()) {
            if (r->pending) materialize(*r);
            else if (r->map) materialize_map(*r);
            else if (r->colsum) materialize_colsum(*r);
            else if (r->transpose) materialize_transpose(*r);
            else if (r->reduce) materialize_reduce(*r);
            else if (r->sibling) run_sibling(*r);
        }
}

// ---- profiler -----------------------------------------------------------------

Profiler &Profiler::get() {
    static Profiler *p = new Profiler();
    return *p;
}

void Profiler::enable(bool on) {
    if (on && StepRecorder::get().open()) throw Error("the profiler cannot time a step being recorded");
    if (!on && enabled_) collect();
    while (!open_.empty()) abort();
    enabled_ = on;
}

void *Profiler::event() {
    void *ev = nullptr;
    if (!spare_.empty()) { ev = spare_.back(); spare_.pop_back(); }
    else check(ts_hip_event_create(&ev), "ts_hip_event_create");
    return ev;
}

// A segment is a timing window of the HIP library: the kernels launched while
// it is open carry its events in their own dispatches, so the elapsed time is
// that of the kernels (first start to last end), not of separately queued
// event records around them.
void Profiler::open_segment(Segments &segs) {
    Segment seg;
    seg.start = event();
    seg.stop = event();
    segs.push_back(seg);
    check(ts_hip_timing_begin(seg.start, seg.stop), "ts_hip_timing_begin");
}

void Profiler::close_segment(Segments &segs) {
    if (segs.empty() || segs.back().kernels >= 0) return;
    int n = 0;
    check(ts_hip_timing_end(&n), "ts_hip_timing_end");
    segs.back().kernels = n;
}

// Launches can nest: a deferred product runs when a later launch first reads
// its result, inside that launch's window.  The innermost timed window that
// encloses a timed launch is closed for its duration and a new segment opened
// after it, so each timed launch is charged its own kernels only.  (An
// untimed launch inside a timed window is charged to it; nested launches are
// deferred products, GEMMs, so that happens only when the GEMM class is not
// timed.)
void Profiler::pause_enclosing() {
    for (size_t i = open_.size(); i-- > 0;)
        if (open_[i].timed) {
            close_segment(open_[i].segments);
            return;
        }
}

void Profiler::resume_enclosing() {
    for (size_t i = open_.size(); i-- > 0;)
        if (open_[i].timed) {
            open_segment(open_[i].segments);
            return;
        }
}

void Profiler::begin(KernelClass k) {
    if (!enabled_) return;
    const bool timed = (classes_ >> static_cast<int>(k)) & 1u;
    if (timed) pause_enclosing();
    Frame f{timed, {}};
    open_.push_back(std::move(f));
    if (timed) open_segment(open_.back().segments);
}

void Profiler::abort() {
    if (!enabled_ || open_.empty()) return;
    close_segment(open_.back().segments);
    Frame f = std::move(open_.back());
    open_.pop_back();
    for (auto &seg : f.segments) {
        spare_.push_back(seg.start);
        spare_.push_back(seg.stop);
    }
    if (f.timed) resume_enclosing();
}

void Profiler::end(KernelClass k, double work) {
    if (!enabled_ || open_.empty()) return;
    close_segment(open_.back().segments);
    Frame f = std::move(open_.back());
    open_.pop_back();
    if (!f.timed) return;
    pending_.push_back(Pending{std::move(f.segments), k, work});
    resume_enclosing();
}

void Profiler::collect() {
    if (pending_.empty()) return;
    check(ts_hip_stream_synchronize(Runtime::get().stream()), "ts_hip_stream_synchronize");
    for (auto &p : pending_) {
        double ms = 0.0;
        for (auto &seg : p.segments) {
            if (seg.kernels > 0) {
                float part = 0.0f;
                check(ts_hip_event_elapsed_ms(&part, seg.start, seg.stop), "ts_hip_event_elapsed_ms");
                ms += part;
            }
            spare_.push_back(seg.start);
            spare_.push_back(seg.stop);
        }
        auto &t = totals_[static_cast<int>(p.k)];
        t.ms += ms;
        t.work += p.work;
        t.launches += 1;
    }
    pending_.clear();
}

void Profiler::reset() {
    collect();
    for (auto &t : totals_) t = ClassStats{};
}

}  // namespace ts
