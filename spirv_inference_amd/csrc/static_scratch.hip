// shp_launch_static: a registry launch that allocates nothing.
//
// shp_launch_ex gives the dense kernels' split-K partials and per-tile arrival counters a
// context workspace that it hipMalloc's (and grows) on first need.  Callers that cannot
// allocate (code under stream capture, tight serving loops, harnesses that forbid
// hipMalloc) use this entry point instead: the same kernels and the same planner, with the
// partials and counters in `scratch`, a fixed device array of this file.  Each device that
// loads the library holds its own copy of the array until the process ends.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "common.h"
#include "gemm.h"
#include "runtime.h"

namespace shp {
// Largest split-K workspace one launch may use: counters (kSplitCounterBytes) + partials.
// The ResNet-50 b32 convolutions need at most 18.4 MiB, the BERT-base b8 s128 dots 36 MiB.
constexpr size_t kStaticScratchBytes = size_t(64) << 20;
}  // namespace shp

// The array itself.  In host code `scratch` names a host-side stand-in, never the device
// memory: host code uses the per-device address from hipGetSymbolAddress instead.
static __device__ __align__(256) float scratch[shp::kStaticScratchBytes / sizeof(float)];

namespace shp {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
float* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch`, per device
// Per device: the stream of the last eager (uncaptured) static launch and an event recorded
// after it, so a launch from another stream first waits for it instead of overwriting
// partials and counters that launch may still be using.
hipStream_t g_last_stream[kMaxDevices] = {};
hipEvent_t g_last_done[kMaxDevices] = {};

__global__ void zero_ints_kernel(int* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

}  // namespace

// Looks up (once per device, with `device` current) the address of `scratch` on `device`.
int static_scratch_attach(int device) {
    if (device < 0 || device >= kMaxDevices)
        return fail(SHP_ERR_INVALID, "static scratch: device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_scratch_ptr[device]) return SHP_OK;
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return fail(SHP_ERR_HIP, std::string("hipGetSymbolAddress(scratch) failed: ") +
                                     hipGetErrorString(e));
    g_scratch_ptr[device] = static_cast<float*>(ptr);
    return SHP_OK;
}

}  // namespace shp

using shp::Ctx;
using shp::fail;

extern "C" int shp_launch_static(shp_ctx* ctx, const char* kernel, const void* in0,
                                 const void* in1, void* out, const int32_t* push, size_t n_push,
                                 uint64_t out_elems, const shp_epilogue* epi) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_launch_static: null ctx");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    if (c->device < 0 || c->device >= shp::kMaxDevices)
        return fail(SHP_ERR_INVALID, "shp_launch_static: context has no device");
    SHP_HIP_CHECK(hipSetDevice(c->device));
    float* ws = nullptr;
    {
        std::lock_guard<std::mutex> lock(shp::g_mu);
        ws = shp::g_scratch_ptr[c->device];
    }
    if (!ws) {  // shp_create attaches it; a context from elsewhere attaches on first use
        int rc = shp::static_scratch_attach(c->device);
        if (rc) return rc;
        std::lock_guard<std::mutex> lock(shp::g_mu);
        ws = shp::g_scratch_ptr[c->device];
    }
    const size_t need =
        kernel ? shp::gemm_workspace_for_kernel(kernel, push, n_push, &c->tune) : 0;
    if (need > shp::kStaticScratchBytes)
        return fail(SHP_ERR_UNSUPPORTED,
                    std::string("shp_launch_static: ") + kernel + " needs " +
                        std::to_string(need) + " bytes of split-K scratch, more than the " +
                        std::to_string(shp::kStaticScratchBytes) +
                        "-byte static scratch; use shp_launch_ex");
    if (need == 0)  // no split-K scratch: nothing is shared
        return shp::launch_kernel(c->stream, kernel, in0, in1, out, push, n_push, out_elems, epi,
                                  ws, shp::kStaticScratchBytes, &c->tune);
    // One array per GPU serves every context and stream.  Launches on one stream are ordered
    // by it; a launch on another stream waits (on the device) for the last eager launch.  A
    // stream under capture cannot wait for work outside its graph, so there the call is
    // refused while that launch is still running.  Graph replays that overlap on one GPU
    // still race: the caller orders them.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    SHP_HIP_CHECK(hipStreamIsCapturing(c->stream, &cs));
    const bool capturing = cs != hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lock(shp::g_mu);
    hipEvent_t& done = shp::g_last_done[c->device];
    hipStream_t& last = shp::g_last_stream[c->device];
    if (last && last != c->stream) {
        if (capturing) {
            hipError_t q = hipEventQuery(done);
            if (q == hipErrorNotReady)
                return fail(SHP_ERR_UNSUPPORTED,
                            "shp_launch_static: a launch on another stream may still use the "
                            "static scratch; synchronise it before capturing");
            if (q != hipSuccess)
                return fail(SHP_ERR_HIP, std::string("shp_launch_static: ") + hipGetErrorString(q));
        } else {
            SHP_HIP_CHECK(hipStreamWaitEvent(c->stream, done, 0));
        }
    }
    // The array keeps the previous call's contents: start this launch's tile counters at
    // zero with a fill kernel (capturable, unlike a memset node).
    const int n = (int)(shp::kSplitCounterBytes / sizeof(int));
    hipLaunchKernelGGL(shp::zero_ints_kernel, dim3((n + 255) / 256), dim3(256), 0, c->stream,
                       reinterpret_cast<int*>(ws), n);
    SHP_HIP_CHECK(hipGetLastError());
    int rc = shp::launch_kernel(c->stream, kernel, in0, in1, out, push, n_push, out_elems, epi,
                                ws, shp::kStaticScratchBytes, &c->tune);
    if (rc || capturing) return rc;
    if (!done) SHP_HIP_CHECK(hipEventCreateWithFlags(&done, hipEventDisableTiming));
    SHP_HIP_CHECK(hipEventRecord(done, c->stream));
    last = c->stream;
    return SHP_OK;
}
