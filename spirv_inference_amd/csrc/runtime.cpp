// Context, resident memory, kernel registry and the dispatch entry points of the C ABI.
//
// Counterpart of tflite_loader::vulkan (source/tflite_loader/src/vulkan.rs:42-194): that
// module creates an instance, device, pipeline and host-visible buffers per dispatch and
// waits idle after each one.  Here the device and one stream live in the context, tensors
// are hipMalloc'd once and stay resident, and kernels are looked up by the reference's
// kernel names (kernels.rs:12-238).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"
#include "gemm.h"
#include "runtime.h"

namespace shp {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
    set_error(msg);
    return code;
}

namespace {

std::vector<const KernelEntry*>& registry() {
    static std::vector<const KernelEntry*> reg = [] {
        std::vector<const KernelEntry*> r;
        auto add = [&](const KernelEntry* t, int n) {
            for (int i = 0; i < n; ++i) r.push_back(&t[i]);
        };
        add(kElementwiseKernels, kElementwiseKernelCount);
        add(kReduceKernels, kReduceKernelCount);
        add(kGemmKernels, kGemmKernelCount);
        add(kSpatialKernels, kSpatialKernelCount);
        add(kDecodeKernels, kDecodeKernelCount);
        add(kHloOpKernels, kHloOpKernelCount);
        add(kBlockKernels, kBlockKernelCount);
        return r;
    }();
    return reg;
}

}  // namespace

const KernelEntry* find_kernel(const char* name) {
    if (!name) return nullptr;
    for (const KernelEntry* e : registry())
        if (std::strcmp(e->name, name) == 0) return e;
    return nullptr;
}

int launch_kernel(hipStream_t stream, const char* name, const void* in0, const void* in1,
                  void* out, const int32_t* push, size_t n_push, uint64_t out_elems,
                  const shp_epilogue* epi, float* workspace, size_t workspace_bytes,
                  const GemmTune* tune) {
    const KernelEntry* e = find_kernel(name);
    if (!e) return fail(SHP_ERR_UNKNOWN_KERNEL, std::string("unknown kernel '") +
                                                    (name ? name : "(null)") + "'");
    if ((int)n_push < e->n_push)
        return fail(SHP_ERR_PUSH, std::string(name) + ": push vector has " +
                                      std::to_string(n_push) + " entries, kernel needs " +
                                      std::to_string(e->n_push));
    if (n_push > 0 && !push) return fail(SHP_ERR_INVALID, std::string(name) + ": null push");
    static const shp_epilogue kNone = {nullptr, nullptr, SHP_ACT_NONE, 0.0f};
    if (epi && !e->epilogue_ok && (epi->bias || epi->residual || epi->act != SHP_ACT_NONE))
        return fail(SHP_ERR_UNSUPPORTED, std::string(name) + ": kernel has no fused epilogue");
    if (out_elems > 0 && !out) return fail(SHP_ERR_INVALID, std::string(name) + ": null output");
    Launch l{stream, in0, in1, out, push, n_push, out_elems, epi ? epi : &kNone, workspace,
             workspace_bytes, tune};
    return e->fn(l);
}

int refuse_while_capturing(hipStream_t stream, const char* what) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    SHP_HIP_CHECK(hipStreamIsCapturing(stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return fail(SHP_ERR_INVALID,
                    std::string(what) + ": refused while the context stream is being captured "
                                        "(the call allocates, copies, clears memory or waits "
                                        "for the stream)");
    return SHP_OK;
}

// ---- context ----------------------------------------------------------------------------
Ctx::~Ctx() {
    for (auto& t : timers) {
        (void)hipEventDestroy(t.a);
        (void)hipEventDestroy(t.b);
    }
    if (workspace) (void)hipFree(workspace);
    for (float* w : retired) (void)hipFree(w);
    if (own_stream) (void)hipStreamDestroy(own_stream);
}

int Ctx::ensure_workspace(size_t bytes) {
    if (bytes <= workspace_bytes) return SHP_OK;
    float* grown = nullptr;
    SHP_HIP_CHECK(hipMalloc((void**)&grown, bytes));
    // The old buffer may be baked into a captured hipGraph (a model's or the caller's):
    // keep it alive until the context goes away.
    if (workspace) retired.push_back(workspace);
    workspace = grown;
    workspace_bytes = bytes;
    // the split-K tile counters at its start must begin at zero (launches keep them zero)
    SHP_HIP_CHECK(hipMemset(workspace, 0, std::min(bytes, kSplitCounterBytes)));
    return SHP_OK;
}

int Ctx::launch(const char* name, const void* in0, const void* in1, void* out,
                const int32_t* push, size_t n_push, uint64_t out_elems, const shp_epilogue* epi) {
    if (device >= 0) SHP_HIP_CHECK(hipSetDevice(device));
    // A dense kernel's split-K partials live in the context workspace: grow it on the first
    // launch that asks for more, except while the stream is being captured into a graph
    // (no allocation there; such a launch runs without splitting K).  Model graphs size it
    // before they capture.
    const size_t need = name ? gemm_workspace_for_kernel(name, push, n_push, &tune) : 0;
    if (need > workspace_bytes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        SHP_HIP_CHECK(hipStreamIsCapturing(stream, &cs));
        if (cs == hipStreamCaptureStatusNone) {
            int rc = ensure_workspace(need);
            if (rc) return rc;
        }
    }
    Timer* t = nullptr;
    if (timing) {
        if (timer_used == timers.size()) {
            Timer nt;
            SHP_HIP_CHECK(hipEventCreate(&nt.a));
            SHP_HIP_CHECK(hipEventCreate(&nt.b));
            timers.push_back(nt);
        }
        t = &timers[timer_used++];
        t->name = name;
        SHP_HIP_CHECK(hipEventRecord(t->a, stream));
    }
    int rc = launch_kernel(stream, name, in0, in1, out, push, n_push, out_elems, epi, workspace,
                           workspace_bytes, &tune);
    if (t) {
        if (rc) {
            --timer_used;
        } else {
            SHP_HIP_CHECK(hipEventRecord(t->b, stream));
        }
    }
    return rc;
}

int Ctx::collect_timing() {
    if (timer_used == 0) return SHP_OK;
    SHP_HIP_CHECK(hipStreamSynchronize(stream));
    for (size_t i = 0; i < timer_used; ++i) {
        float ms = 0.0f;
        SHP_HIP_CHECK(hipEventElapsedTime(&ms, timers[i].a, timers[i].b));
        auto& acc = timing_totals[timers[i].name];
        acc.first += ms;
        acc.second += 1;
        timing_log.emplace_back(timers[i].name, (double)ms);
    }
    timer_used = 0;
    return SHP_OK;
}

}  // namespace shp

using shp::Ctx;
using shp::fail;

extern "C" {

const char* shp_last_error(void) { return shp::g_last_error.c_str(); }

int shp_create(const char* selector, shp_ctx** out) {
    if (!out) return fail(SHP_ERR_INVALID, "shp_create: null out");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0)
        return fail(SHP_ERR_NO_DEVICE, std::string("no HIP device: ") + hipGetErrorString(e));
    int dev = 0;
    std::string sel = selector ? selector : "any";
    if (sel == "any" || sel == "amd" || sel.empty()) {
        dev = 0;
    } else {
        char* end = nullptr;
        long v = std::strtol(sel.c_str(), &end, 10);
        if (!end || *end != '\0' || v < 0 || v >= count)
            return fail(SHP_ERR_NO_DEVICE, "device selector '" + sel + "' matched no device");
        dev = (int)v;
    }
    SHP_HIP_CHECK(hipSetDevice(dev));
    int arc = shp::static_scratch_attach(dev);
    if (arc) return arc;
    Ctx* c = new Ctx();
    c->device = dev;
    hipError_t se = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking);
    if (se != hipSuccess) {
        delete c;
        return fail(SHP_ERR_HIP, std::string("hipStreamCreate: ") + hipGetErrorString(se));
    }
    c->stream = c->own_stream;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess) {
        std::snprintf(c->info.device_name, sizeof(c->info.device_name), "%s (%s)", prop.name,
                      prop.gcnArchName);
        c->info.device_id = (uint32_t)prop.pciDeviceID;
        c->cu_count = prop.multiProcessorCount;
    }
    c->info.vendor_id = 0x1002;
    *out = reinterpret_cast<shp_ctx*>(c);
    return SHP_OK;
}

void shp_destroy(shp_ctx* ctx) {
    if (!ctx) return;
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    delete c;
}

int shp_device_info(shp_ctx* ctx, shp_run_info* info) {
    if (!ctx || !info) return fail(SHP_ERR_INVALID, "shp_device_info: null argument");
    *info = reinterpret_cast<Ctx*>(ctx)->info;
    return SHP_OK;
}

int shp_set_stream(shp_ctx* ctx, void* hip_stream) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_set_stream: null ctx");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    c->stream = hip_stream ? (hipStream_t)hip_stream : c->own_stream;
    return SHP_OK;
}

void* shp_get_stream(shp_ctx* ctx) {
    return ctx ? (void*)reinterpret_cast<Ctx*>(ctx)->stream : nullptr;
}

int shp_alloc(shp_ctx* ctx, size_t bytes, void** dptr) {
    if (!ctx || !dptr) return fail(SHP_ERR_INVALID, "shp_alloc: null argument");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    SHP_HIP_CHECK(hipSetDevice(c->device));
    *dptr = nullptr;
    SHP_HIP_CHECK(hipMalloc(dptr, bytes ? bytes : 4));
    return SHP_OK;
}

int shp_free(shp_ctx* ctx, void* dptr) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_free: null ctx");
    if (!dptr) return SHP_OK;
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    {
        int grc = shp::refuse_while_capturing(c->stream, "shp_free");
        if (grc) return grc;
    }
    SHP_HIP_CHECK(hipStreamSynchronize(c->stream));
    SHP_HIP_CHECK(hipFree(dptr));
    return SHP_OK;
}

int shp_upload(shp_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(SHP_ERR_INVALID, "shp_upload: null");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    {
        int grc = shp::refuse_while_capturing(c->stream, "shp_upload");
        if (grc) return grc;
    }
    if (!bytes) return SHP_OK;
    SHP_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
    SHP_HIP_CHECK(hipStreamSynchronize(c->stream));
    return SHP_OK;
}

int shp_download(shp_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(SHP_ERR_INVALID, "shp_download: null");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    {
        int grc = shp::refuse_while_capturing(c->stream, "shp_download");
        if (grc) return grc;
    }
    if (!bytes) return SHP_OK;
    SHP_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
    SHP_HIP_CHECK(hipStreamSynchronize(c->stream));
    return SHP_OK;
}

int shp_sync(shp_ctx* ctx) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_sync: null ctx");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    int rc = shp::refuse_while_capturing(c->stream, "shp_sync");
    if (rc) return rc;
    SHP_HIP_CHECK(hipStreamSynchronize(c->stream));
    return SHP_OK;
}

// Internal hooks for tests and experiments (not part of include/spirv_hip.h).
// Grow the context's split-K workspace so forced split counts are not clamped by it.
int shp_reserve_workspace(shp_ctx* ctx, uint64_t bytes) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_reserve_workspace: null ctx");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    int rc = shp::refuse_while_capturing(c->stream, "shp_reserve_workspace");
    return rc ? rc : c->ensure_workspace((size_t)bytes);
}

// Current split-K workspace of the context (its address and size), for lifetime checks.
int shp_workspace_info(shp_ctx* ctx, void** dptr, uint64_t* bytes) {
    if (!ctx || !dptr || !bytes) return fail(SHP_ERR_INVALID, "shp_workspace_info: null argument");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    *dptr = c->workspace;
    *bytes = c->workspace_bytes;
    return SHP_OK;
}

// Force parts of the planners' choices for launches on this context only (0 restores the
// automatic choice): gemm_tile, gemm_bk, gemm_splits, gemm_dma, gemm_pg, gemm_table, gemm_bl,
// gemm_sk, gemm_stem, gemm_group, dw_tile; the fused block's ir_th, ir_tw, ir_splits,
// ir_cout_splits and the model graphs' ir_fuse; conv_direct (-1: small-channel 3x3
// conv2d_nhwc on the implicit GEMM instead of the direct kernel); gemm_small (1x1 conv2d_nhwc
// on the small-product kernel: 1 wherever it fits, k >= 2 with k K-splits, -1 never); fc_mfma (-1:
// fully_connected with 2-16 rows on the wavefront-per-column or tiled kernels).
int shp_tune(shp_ctx* ctx, const char* key, int value) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_tune: null ctx");
    shp::GemmTune& t = reinterpret_cast<Ctx*>(ctx)->tune;
    std::string k = key ? key : "";
    if (k == "gemm_tile") t.tile = value;
    else if (k == "gemm_bk") t.bk = value;
    else if (k == "gemm_splits") t.splits = value;
    else if (k == "gemm_dma") t.dma = value;
    else if (k == "gemm_pg") t.pg = value;
    else if (k == "gemm_table") t.table = value;
    else if (k == "gemm_bl") t.bl = value;
    else if (k == "gemm_sk") t.sk = value;
    else if (k == "gemm_stem") t.stem = value;
    else if (k == "dw_tile") t.dw = value;
    else if (k == "gemm_group") t.group = value;
    else if (k == "ir_th") t.ir_th = value;
    else if (k == "ir_tw") t.ir_tw = value;
    else if (k == "ir_splits") t.ir_s = value;
    else if (k == "ir_cout_splits") t.ir_j = value;
    else if (k == "ir_fuse") t.ir_fuse = value;
    else if (k == "conv_direct") t.conv_direct = value;
    else if (k == "gemm_small") t.small = value;
    else if (k == "fc_mfma") t.fc = value;
    else return fail(SHP_ERR_INVALID, "shp_tune: unknown key '" + k + "'");
    return SHP_OK;
}

int shp_fill_random(shp_ctx* ctx, float* dptr, uint64_t n, uint64_t seed, uint64_t tensor_id,
                    int32_t kind, float lo, float hi) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_fill_random: null ctx");
    return shp::fill_random(reinterpret_cast<Ctx*>(ctx)->stream, dptr, n, seed, tensor_id, kind,
                            lo, hi);
}

int shp_kernel_count(void) { return (int)shp::registry().size(); }

const char* shp_kernel_name(int index) {
    auto& r = shp::registry();
    if (index < 0 || index >= (int)r.size()) return nullptr;
    return r[index]->name;
}

int shp_kernel_push_count(const char* kernel) {
    const shp::KernelEntry* e = shp::find_kernel(kernel);
    return e ? e->n_push : SHP_ERR_UNKNOWN_KERNEL;
}

int shp_launch(shp_ctx* ctx, const char* kernel, const void* in0, const void* in1, void* out,
               const int32_t* push, size_t n_push, uint64_t out_elems) {
    return shp_launch_ex(ctx, kernel, in0, in1, out, push, n_push, out_elems, nullptr);
}

int shp_launch_ex(shp_ctx* ctx, const char* kernel, const void* in0, const void* in1, void* out,
                  const int32_t* push, size_t n_push, uint64_t out_elems,
                  const shp_epilogue* epi) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_launch: null ctx");
    return reinterpret_cast<Ctx*>(ctx)->launch(kernel, in0, in1, out, push, n_push, out_elems,
                                               epi);
}

int shp_run_kernel(shp_ctx* ctx, const char* kernel, const float* in0, size_t n0,
                   const float* in1, size_t n1, float* out, size_t n_out, const int32_t* push,
                   size_t n_push, uint32_t grid_hint, shp_run_info* info) {
    (void)grid_hint;  // HIP picks its own grid; the reference's dispatch_x is advisory here
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_run_kernel: null ctx");
    if ((n0 && !in0) || (n1 && !in1) || (n_out && !out))
        return fail(SHP_ERR_INVALID, "shp_run_kernel: null buffer with non-zero size");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    {
        int grc = shp::refuse_while_capturing(c->stream, "shp_run_kernel");
        if (grc) return grc;
    }
    if (!shp::find_kernel(kernel))
        return fail(SHP_ERR_UNKNOWN_KERNEL,
                    std::string("unknown kernel '") + (kernel ? kernel : "(null)") + "'");
    SHP_HIP_CHECK(hipSetDevice(c->device));
    // Like vulkan.rs:109-112, every binding gets a buffer (>= 1 element) even if unused.
    void *d0 = nullptr, *d1 = nullptr, *d2 = nullptr;
    auto cleanup = [&] {
        if (d0) (void)hipFree(d0);
        if (d1) (void)hipFree(d1);
        if (d2) (void)hipFree(d2);
    };
    size_t b0 = (n0 ? n0 : 1) * 4, b1 = (n1 ? n1 : 1) * 4, b2 = (n_out ? n_out : 1) * 4;
    if (hipMalloc(&d0, b0) != hipSuccess || hipMalloc(&d1, b1) != hipSuccess ||
        hipMalloc(&d2, b2) != hipSuccess) {
        cleanup();
        return fail(SHP_ERR_HIP, "shp_run_kernel: device allocation failed");
    }
    int rc = SHP_OK;
    hipEvent_t ea = nullptr, eb = nullptr;
    do {
        if (hipMemsetAsync(d0, 0, b0, c->stream) != hipSuccess ||
            hipMemsetAsync(d1, 0, b1, c->stream) != hipSuccess ||
            hipMemsetAsync(d2, 0, b2, c->stream) != hipSuccess) {
            rc = fail(SHP_ERR_HIP, "shp_run_kernel: memset failed");
            break;
        }
        if (n0 && hipMemcpyAsync(d0, in0, n0 * 4, hipMemcpyHostToDevice, c->stream) != hipSuccess) {
            rc = fail(SHP_ERR_HIP, "shp_run_kernel: upload in0 failed");
            break;
        }
        if (n1 && hipMemcpyAsync(d1, in1, n1 * 4, hipMemcpyHostToDevice, c->stream) != hipSuccess) {
            rc = fail(SHP_ERR_HIP, "shp_run_kernel: upload in1 failed");
            break;
        }
        if (hipEventCreate(&ea) != hipSuccess || hipEventCreate(&eb) != hipSuccess) {
            rc = fail(SHP_ERR_HIP, "shp_run_kernel: event create failed");
            break;
        }
        (void)hipEventRecord(ea, c->stream);
        rc = c->launch(kernel, d0, d1, d2, push, n_push, n_out, nullptr);
        if (rc) break;
        (void)hipEventRecord(eb, c->stream);
        if (n_out &&
            hipMemcpyAsync(out, d2, n_out * 4, hipMemcpyDeviceToHost, c->stream) != hipSuccess) {
            rc = fail(SHP_ERR_HIP, "shp_run_kernel: download failed");
            break;
        }
        hipError_t se = hipStreamSynchronize(c->stream);
        if (se != hipSuccess) {
            rc = fail(SHP_ERR_HIP, std::string("shp_run_kernel: ") + hipGetErrorString(se));
            break;
        }
        if (info) {
            *info = c->info;
            float ms = 0.0f;
            (void)hipEventElapsedTime(&ms, ea, eb);
            info->elapsed_ms = ms;
        }
    } while (0);
    if (rc) (void)hipStreamSynchronize(c->stream);
    if (ea) (void)hipEventDestroy(ea);
    if (eb) (void)hipEventDestroy(eb);
    cleanup();
    return rc;
}

// ---- captured launch sequences (hipGraph) --------------------------------------------
// The reference re-records and resubmits a command buffer per dispatch (vulkan.rs:132-171);
// a caller that repeats one launch sequence records it once and replays it.
struct shp_graph {
    Ctx* ctx;
    hipStream_t stream;
    hipGraph_t graph;
    hipGraphExec_t exec;
};

int shp_capture_begin(shp_ctx* ctx) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_capture_begin: null ctx");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    SHP_HIP_CHECK(hipSetDevice(c->device));
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    SHP_HIP_CHECK(hipStreamIsCapturing(c->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return fail(SHP_ERR_INVALID, "shp_capture_begin: the context stream is already capturing");
    SHP_HIP_CHECK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->timing_before_capture = c->timing;
    c->timing = false;  // no event records inside the capture
    return SHP_OK;
}

int shp_capture_end(shp_ctx* ctx, shp_graph** out) {
    if (!ctx || !out) return fail(SHP_ERR_INVALID, "shp_capture_end: null argument");
    *out = nullptr;
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(c->stream, &g);
    c->timing = c->timing_before_capture;
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return fail(SHP_ERR_HIP, std::string("shp_capture_end: ") + hipGetErrorString(e));
    }
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return fail(SHP_ERR_HIP, std::string("shp_capture_end: instantiate: ") + hipGetErrorString(e));
    }
    *out = new shp_graph{c, c->stream, g, x};
    return SHP_OK;
}

int shp_graph_launch(shp_graph* g) {
    if (!g) return fail(SHP_ERR_INVALID, "shp_graph_launch: null graph");
    SHP_HIP_CHECK(hipGraphLaunch(g->exec, g->ctx->stream));
    return SHP_OK;
}

void shp_graph_destroy(shp_graph* g) {
    if (!g) return;
    (void)hipStreamSynchronize(g->ctx->stream);
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

int shp_timing_enable(shp_ctx* ctx, int enable) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_timing_enable: null ctx");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    c->timing = enable != 0;
    return SHP_OK;
}

int shp_timing_reset(shp_ctx* ctx) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_timing_reset: null ctx");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    {
        int grc = shp::refuse_while_capturing(c->stream, "shp_timing_reset");
        if (grc) return grc;
    }
    SHP_HIP_CHECK(hipStreamSynchronize(c->stream));
    c->timer_used = 0;
    c->timing_totals.clear();
    c->timing_log.clear();
    return SHP_OK;
}

int shp_timing_entry(shp_ctx* ctx, int index, char* name, size_t name_cap, double* total_ms,
                     uint64_t* count) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_timing_entry: null ctx");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    {
        int grc = shp::refuse_while_capturing(c->stream, "shp_timing_entry");
        if (grc) return grc;
    }
    int rc = c->collect_timing();
    if (rc) return rc;
    if (index < 0 || index >= (int)c->timing_totals.size())
        return fail(SHP_ERR_INVALID, "shp_timing_entry: index out of range");
    auto it = c->timing_totals.begin();
    std::advance(it, index);
    if (name && name_cap) {
        std::strncpy(name, it->first.c_str(), name_cap - 1);
        name[name_cap - 1] = '\0';
    }
    if (total_ms) *total_ms = it->second.first;
    if (count) *count = it->second.second;
    return SHP_OK;
}

int shp_timing_launch_count(shp_ctx* ctx, uint64_t* count) {
    if (!ctx || !count) return fail(SHP_ERR_INVALID, "shp_timing_launch_count: null argument");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    {
        int grc = shp::refuse_while_capturing(c->stream, "shp_timing_launch_count");
        if (grc) return grc;
    }
    int rc = c->collect_timing();
    if (rc) return rc;
    *count = c->timing_log.size();
    return SHP_OK;
}

int shp_timing_launch(shp_ctx* ctx, uint64_t index, char* name, size_t name_cap, double* ms) {
    if (!ctx) return fail(SHP_ERR_INVALID, "shp_timing_launch: null ctx");
    Ctx* c = reinterpret_cast<Ctx*>(ctx);
    {
        int grc = shp::refuse_while_capturing(c->stream, "shp_timing_launch");
        if (grc) return grc;
    }
    int rc = c->collect_timing();
    if (rc) return rc;
    if (index >= c->timing_log.size())
        return fail(SHP_ERR_INVALID, "shp_timing_launch: index out of range");
    const auto& e = c->timing_log[index];
    if (name && name_cap) {
        std::strncpy(name, e.first.c_str(), name_cap - 1);
        name[name_cap - 1] = '\0';
    }
    if (ms) *ms = e.second;
    return SHP_OK;
}

}  // extern "C"
