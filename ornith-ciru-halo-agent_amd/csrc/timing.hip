// Event-pair timing of kernel launches (timed_launch in timing.hpp) and its C
// entry points.
#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "timing.hpp"
#include "../../include/ornith_timing.h"

namespace ornith {
namespace {

struct Record {
    std::string name;
    hipEvent_t start = nullptr, stop = nullptr;
};

struct TimingState {
    std::mutex mu;
    std::string pattern;
    std::vector<Record> records;    // pre-created event pairs
    int used = 0;
};

TimingState& state() {
    static TimingState s;
    return s;
}

void release(TimingState& s) {
    for (Record& r : s.records) {
        if (r.start) (void)hipEventDestroy(r.start);
        if (r.stop) (void)hipEventDestroy(r.stop);
    }
    s.records.clear();
    s.used = 0;
}

}  // namespace

std::atomic<bool> g_timing_armed{false};

bool timing_claim(const char* name, hipEvent_t* start, hipEvent_t* stop) {
    TimingState& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (!g_timing_armed.load(std::memory_order_relaxed) || s.used >= int(s.records.size())) return false;
    if (s.pattern != "*" && s.pattern != name) return false;
    Record& r = s.records[s.used++];
    r.name = name;
    *start = r.start;
    *stop = r.stop;
    return true;
}

}  // namespace ornith

using ornith::state;

extern "C" hipError_t ornith_mi355x_timing_arm(const char* kernel, int capacity) {
    auto& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    ornith::g_timing_armed.store(false);
    ornith::release(s);
    if (kernel == nullptr || capacity <= 0) return hipSuccess;
    if (capacity > (1 << 20)) return hipErrorInvalidValue;
    s.records.resize(size_t(capacity));
    for (auto& r : s.records) {
        hipError_t e = hipEventCreate(&r.start);
        if (e == hipSuccess) e = hipEventCreate(&r.stop);
        if (e != hipSuccess) {
            ornith::release(s);
            return e;
        }
    }
    s.pattern = kernel;
    ornith::g_timing_armed.store(true);
    return hipSuccess;
}

extern "C" hipError_t ornith_mi355x_timing_read(const char* kernel, int* launches, double* total_ms) {
    if (kernel == nullptr || launches == nullptr || total_ms == nullptr) return hipErrorInvalidValue;
    auto& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    *launches = 0;
    *total_ms = 0.0;
    for (int i = 0; i < s.used; ++i) {
        const auto& r = s.records[i];
        if (std::strcmp(kernel, "*") != 0 && r.name != kernel) continue;
        hipError_t e = hipEventSynchronize(r.stop);
        if (e != hipSuccess) return e;
        float ms = 0.f;
        e = hipEventElapsedTime(&ms, r.start, r.stop);
        if (e != hipSuccess) return e;
        *launches += 1;
        *total_ms += ms;
    }
    return hipSuccess;
}

extern "C" int ornith_mi355x_timing_names(char* out, int capacity) {
    // distinct recorded kernel names, comma separated; returns the length needed
    auto& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    std::string all;
    for (int i = 0; i < s.used; ++i) {
        const std::string& n = s.records[i].name;
        bool seen = false;
        for (int j = 0; j < i && !seen; ++j) seen = s.records[j].name == n;
        if (seen) continue;
        if (!all.empty()) all += ',';
        all += n;
    }
    if (out != nullptr && capacity > 0) {
        const size_t n = std::min(all.size(), size_t(capacity - 1));
        std::memcpy(out, all.data(), n);
        out[n] = '\0';
    }
    return int(all.size());
}
