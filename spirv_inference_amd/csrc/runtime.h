// The context behind shp_ctx: one device, one stream, a split-K workspace and the
// per-launch event timers that replace KernelOutput.elapsed_ms (vulkan.rs:163-171).
#pragma once

#include <map>
#include <string>
#include <vector>

#include "common.h"

namespace shp {

struct Ctx {
    int device = -1;
    int cu_count = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    shp_run_info info{};
    // Split-K scratch of eager launches.  A graph captured from such a launch keeps the
    // pointer it saw, so a buffer outgrown later is retired (kept until the context is
    // destroyed) instead of freed.
    float* workspace = nullptr;
    size_t workspace_bytes = 0;
    std::vector<float*> retired;
    GemmTune tune;  // planner overrides of this context's dense launches (shp_tune)

    struct Timer {
        hipEvent_t a, b;
        std::string name;
    };
    bool timing = false;
    bool timing_before_capture = false;  // restored by shp_capture_end
    std::vector<Timer> timers;
    size_t timer_used = 0;
    std::map<std::string, std::pair<double, uint64_t>> timing_totals;
    // every timed launch in issue order since the last reset: (kernel name, ms)
    std::vector<std::pair<std::string, double>> timing_log;

    ~Ctx();
    int ensure_workspace(size_t bytes);
    int launch(const char* name, const void* in0, const void* in1, void* out,
               const int32_t* push, size_t n_push, uint64_t out_elems, const shp_epilogue* epi);
    int collect_timing();
};

// SHP_OK unless `stream` is being captured into a graph; then SHP_ERR_INVALID naming `what`.
// Entry points that allocate, copy, clear memory or wait for the stream call it first, so a
// call made between shp_capture_begin and shp_capture_end fails closed instead of recording
// a memset or copy node into the caller's graph or breaking the capture.
int refuse_while_capturing(hipStream_t stream, const char* what);

// Resolves, once per device and with that device current, the device address of the fixed
// split-K scratch array behind shp_launch_static (static_scratch.hip).
int static_scratch_attach(int device);

}  // namespace shp
