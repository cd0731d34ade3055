// fg_telemetry.cpp -- device memory telemetry: a background sampler of the
// device's memory usage and budget.
//
// Replaces the gpu_telemetry 0.2 monitor the reference's example harness
// uses (crates/ferrograd/examples/matmul_chain3.rs:145-171: GpuMonitor::
// start(interval) ... stop() -> samples of per-heap usage and budget, from
// which it prints the average usage and the largest budget).  The crate is
// not vendored; its contract is restated here for one device heap: every
// interval a thread records (time, used bytes = total - free, budget bytes =
// total) from hipMemGetInfo on the context's device.
#include <hip/hip_runtime.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <vector>

#include "fg_internal.h"

namespace {

struct Sample {
    double t_s;
    uint64_t used;
    uint64_t budget;
};

}  // namespace

struct fg_monitor {
    int device = 0;
    int interval_us = 10000;
    std::vector<Sample> samples;
    std::mutex mu;
    std::condition_variable cv;
    bool stop = false;
    int error = FG_OK;
    std::thread worker;
};

namespace {

void sample_loop(fg_monitor *m) {
    const auto t0 = std::chrono::steady_clock::now();
    if (hipSetDevice(m->device) != hipSuccess) {
        std::lock_guard<std::mutex> lk(m->mu);
        m->error = FG_ERR_DEVICE;
        return;
    }
    std::unique_lock<std::mutex> lk(m->mu);
    for (;;) {
        lk.unlock();
        size_t free_b = 0, total_b = 0;
        const hipError_t e = hipMemGetInfo(&free_b, &total_b);
        const double t = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        lk.lock();
        if (e != hipSuccess) {
            m->error = FG_ERR_DEVICE;
            return;
        }
        m->samples.push_back(Sample{t, (uint64_t)(total_b - free_b), (uint64_t)total_b});
        if (m->cv.wait_for(lk, std::chrono::microseconds(m->interval_us), [m] { return m->stop; }))
            return;
    }
}

}  // namespace

FG_API int fg_monitor_start(fg_ctx *ctx, int interval_us, fg_monitor **out) {
    FG_REQUIRE(ctx && out, FG_ERR_INVALID_ARGUMENT, "fg_monitor_start: NULL argument");
    FG_REQUIRE(interval_us >= 100, FG_ERR_INVALID_ARGUMENT,
               "fg_monitor_start: interval %d us is below 100 us", interval_us);
    fg_monitor *m = new fg_monitor;
    m->device = ctx->device;
    m->interval_us = interval_us;
    try {
        m->worker = std::thread(sample_loop, m);
    } catch (...) {
        delete m;
        fg::set_error("fg_monitor_start: cannot start the sampling thread");
        return FG_ERR_INTERNAL;
    }
    *out = m;
    return FG_OK;
}

// Stops sampling (one last sample is always present); the samples stay
// readable until fg_monitor_destroy.
FG_API int fg_monitor_stop(fg_monitor *m, int *n_samples) {
    FG_REQUIRE(m, FG_ERR_INVALID_ARGUMENT, "fg_monitor_stop: NULL monitor");
    {
        std::lock_guard<std::mutex> lk(m->mu);
        m->stop = true;
    }
    m->cv.notify_all();
    if (m->worker.joinable()) m->worker.join();
    if (n_samples) *n_samples = (int)m->samples.size();
    if (m->error) {
        fg::set_error("fg_monitor_stop: hipMemGetInfo failed on device %d", m->device);
        return m->error;
    }
    return FG_OK;
}

FG_API int fg_monitor_sample(const fg_monitor *m, int index, double *t_s, uint64_t *used,
                             uint64_t *budget) {
    FG_REQUIRE(m, FG_ERR_INVALID_ARGUMENT, "fg_monitor_sample: NULL monitor");
    FG_REQUIRE(!m->worker.joinable(), FG_ERR_INVALID_ARGUMENT,
               "fg_monitor_sample: stop the monitor first");
    FG_REQUIRE(index >= 0 && index < (int)m->samples.size(), FG_ERR_OUT_OF_BOUNDS,
               "fg_monitor_sample: sample %d of %zu", index, m->samples.size());
    const Sample &s = m->samples[index];
    if (t_s) *t_s = s.t_s;
    if (used) *used = s.used;
    if (budget) *budget = s.budget;
    return FG_OK;
}

FG_API int fg_monitor_destroy(fg_monitor *m) {
    if (!m) return FG_OK;
    if (m->worker.joinable()) fg_monitor_stop(m, nullptr);
    delete m;
    return FG_OK;
}
