// Internal declarations shared by the kernel translation units and the runtime.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "spirv_hip.h"

namespace shp {

// Thread-local error message behind shp_last_error().
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

#define SHP_HIP_CHECK(expr)                                                           \
    do {                                                                              \
        hipError_t e__ = (expr);                                                      \
        if (e__ != hipSuccess)                                                        \
            return ::shp::fail(SHP_ERR_HIP, std::string(#expr " failed: ") +          \
                                                hipGetErrorString(e__));             \
    } while (0)

// Planner overrides of the dense kernels, held per context (all 0 = automatic choice):
// tile 1: 128x128, 2: 128x64, 3: 64x64; bk 16 or 32; splits: split-K count; dma 0 automatic,
// -1 never, 1: 128x128, 2: 128x64 pipelined kernel; pg: register prefetch depth 1 or 2;
// table: -1 ignores the measured per-shape plans (planner cost model only); dw: the NHWC
// depthwise convolution with (1) or without (-1) its LDS tile instead of the automatic choice;
// bl: the buffer-loaded GEMM kernel never (-1) or, where its operand forms allow it, always
// (1); with bl 1, tile 1/2/3 and bk 16/32/64 pick its tile; sk -1: never the persistent
// small-K kernel (K 64 row products), else wherever it applies; stem -1: never the 7x7
// 3-channel convolution kernel, else wherever it applies; group: see below.
struct GemmTune {
    int tile = 0, bk = 0, splits = 0, dma = 0, pg = 0, table = 0, dw = 0, bl = 0, sk = 0, stem = 0;
    int group = 0;  // tile-row band of the tile order: 0 automatic, -1 row major, k > 0 forced
    // inverted_residual_nhwc plan: output tile rows x columns, expanded-channel splits and
    // output-channel splits (0: the planner's choice)
    int ir_th = 0, ir_tw = 0, ir_s = 0, ir_j = 0;
    // model graphs: MBConv blocks as one inverted_residual_nhwc launch where it is expected
    // to pay (0), always (1), or as the three operators the TFLite scheduler dispatches (-1);
    // read when a model is built
    int ir_fuse = 0;
    // conv2d_nhwc with <= 4 input channels: the direct kernel where it fits (0) or the
    // implicit-GEMM kernels (-1)
    int conv_direct = 0;
    // 1x1 conv2d_nhwc: the small-product kernel where the 64x64 tiles would not fill the GPU
    // (0), wherever it takes the shape (1), with k >= 2 K-splits (k), never (-1)
    int small = 0;
    // fully_connected with 2-16 rows: the split-K MFMA kernel where it takes the shape (0) or
    // the wavefront-per-column and tiled kernels (-1)
    int fc = 0;
};

// Everything a launcher needs: the three bindings, the push vector and the epilogue.
struct Launch {
    hipStream_t stream;
    const void* in0;
    const void* in1;
    void* out;
    const int32_t* push;
    size_t n_push;
    uint64_t out_elems;
    const shp_epilogue* epi;  // never null inside launchers (zero epilogue if absent)
    float* workspace;         // context-owned scratch (split-K partials), may be null
    size_t workspace_bytes;
    const GemmTune* tune;     // the context's planner overrides (null: none)
};

using LaunchFn = int (*)(const Launch&);

struct KernelEntry {
    const char* name;
    int n_push;        // i32 count of the Params block
    bool epilogue_ok;  // accepts bias/residual/activation
    LaunchFn fn;
};

// Registry tables, one per translation unit; registry.cpp concatenates them.
extern KernelEntry kElementwiseKernels[];
extern const int kElementwiseKernelCount;
extern KernelEntry kReduceKernels[];
extern const int kReduceKernelCount;
extern KernelEntry kGemmKernels[];
extern const int kGemmKernelCount;
extern KernelEntry kSpatialKernels[];
extern const int kSpatialKernelCount;
extern KernelEntry kHloOpKernels[];
extern const int kHloOpKernelCount;
extern KernelEntry kDecodeKernels[];
extern const int kDecodeKernelCount;
extern KernelEntry kBlockKernels[];
extern const int kBlockKernelCount;

const KernelEntry* find_kernel(const char* name);

// Launch a registered kernel on a stream (used by the graph runtime and the models).
int launch_kernel(hipStream_t stream, const char* name, const void* in0, const void* in1,
                  void* out, const int32_t* push, size_t n_push, uint64_t out_elems,
                  const shp_epilogue* epi, float* workspace, size_t workspace_bytes,
                  const GemmTune* tune);

// Split-K workspace a dense kernel would ask for with this push vector (0 if none).
size_t gemm_workspace_for_kernel(const char* name, const int32_t* push, size_t n_push,
                                 const GemmTune* tune);
// The same for the fused block kernel inverted_residual_nhwc (kernels_block.hip).
size_t block_workspace_for_kernel(const int32_t* push, size_t n_push, const GemmTune* tune);
// Whether that kernel takes this push vector and is expected to beat the block's three
// operators (measured verdicts for the benchmark configs' blocks, a rule elsewhere).
bool block_fusion_pays(const int32_t* push, size_t n_push);
// conv2d_nhwc with at most 4 input channels (the 3-channel image stems) as a direct
// convolution (kernels_spatial.hip): SHP_ERR_UNSUPPORTED when the shape does not fit it.
int conv_nhwc_direct(const Launch& l);

// Counter-based RNG fill (kernels_elementwise.hip).
int fill_random(hipStream_t stream, float* p, uint64_t n, uint64_t seed, uint64_t tensor_id,
                int kind, float lo, float hi);

inline unsigned grid_1d(uint64_t n, unsigned block) {
    uint64_t g = (n + block - 1) / block;
    return g == 0 ? 1u : (unsigned)g;
}

// Shape check helper for launchers.
inline int check_total(const Launch& l, int64_t expect, const char* kernel) {
    if (expect < 0 || (uint64_t)expect != l.out_elems)
        return fail(SHP_ERR_SHAPE, std::string(kernel) + ": push-vector total " +
                                       std::to_string(expect) + " != output elements " +
                                       std::to_string(l.out_elems));
    return SHP_OK;
}

}  // namespace shp

// ---- device-side helpers --------------------------------------------------------
namespace shpd {

// erfc(z) as the XLA rational expansion the BERT fixture spells out op by op
// (source/xla_hlo/fixtures/bert_base.stablehlo.txt:59-144): a polynomial in z^2 for
// |z| <= 1, exp(-z^2)*P(1/z^2)/(min(|z|,10.06)*Q(1/z^2)) otherwise, reflected for z < 0.
__device__ __forceinline__ float erfc_xla(float z) {
    float az = fabsf(z);
    if (az > 1.0f) {
        float z2 = z * z;
        float e = expf(-z2);
        float q = 1.0f / z2;
        float p = ((0.102081165f * q + 0.429206669f) * q + 0.323790789f) * q + 0.053971976f;
        float d = ((((0.0172516778f * q + 0.391371638f) * q + 1.0f) * q + 0.621732414f) * q +
                   0.0956628621f);
        float r = e * (p / (fminf(az, 10.06f) * d));
        return z < 0.0f ? 2.0f - r : r;
    }
    float w = z * z;
    float s = ((((0.000561802299f * w - 0.00491381669f) * w + 0.0267075151f) * w -
                0.112800106f) * w + 0.376122952f) * w - 1.12837911f;
    return z * s + 1.0f;
}

__device__ __forceinline__ float apply_act(float x, int act, float alpha) {
    switch (act) {
        case SHP_ACT_RELU: return fmaxf(x, 0.0f);
        case SHP_ACT_RELU6: return fminf(fmaxf(x, 0.0f), 6.0f);
        case SHP_ACT_LEAKY: return fmaxf(alpha * x, x);
        case SHP_ACT_SIGMOID: return 1.0f / (1.0f + expf(-x));
        case SHP_ACT_TANH: {
            float c = fminf(fmaxf(x, -20.0f), 20.0f);
            float ep = expf(c), en = expf(-c);
            return (ep - en) / (ep + en);
        }
        case SHP_ACT_SILU: return x * (1.0f / (1.0f + expf(-x)));
        case SHP_ACT_GELU_ERF: return (0.5f * x) * erfc_xla(-x * 0.707106769f);
        default: return x;
    }
}

}  // namespace shpd
