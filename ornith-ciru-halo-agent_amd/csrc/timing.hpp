// Per-kernel launch timing for measurement.
//
// Every kernel of the library is launched through timed_launch.  While the
// timing hook is armed (ornith_mi355x_timing_arm) and the launch's name
// matches the armed name ("*" = every kernel), the launch goes through
// hipExtLaunchKernelGGL with a start/stop event pair attached to the kernel's
// own dispatch on its stream; otherwise it is a plain launch.  The kernels
// and their work are the same either way; an unarmed launch costs one
// relaxed atomic load.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <atomic>

namespace ornith {

extern std::atomic<bool> g_timing_armed;

// Claims the next event pair for a launch of `name`; false when unarmed, not
// matching or full.
bool timing_claim(const char* name, hipEvent_t* start, hipEvent_t* stop);

template <typename... KArgs, typename... Args>
inline void timed_launch(const char* name, void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t shmem,
                         hipStream_t stream, Args... args) {
    hipEvent_t start = nullptr, stop = nullptr;
    if (g_timing_armed.load(std::memory_order_relaxed) && timing_claim(name, &start, &stop)) {
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, start, stop, 0, KArgs(args)...);
        return;
    }
    kernel<<<grid, block, shmem, stream>>>(KArgs(args)...);
}

}  // namespace ornith
