// Model graphs of the benchmark configs and the C ABI of shp_model_*.
//
// The reference drives its kernels from two front-ends, one op at a time, with a host
// round trip per op: the TFLite scheduler (source/tflite_loader/src/scheduler.rs:29-1082)
// for MobileNetV2 / EfficientNet-Lite0, and the HLO interpreter
// (source/xla_hlo/src/compiler.rs:267-668) for ResNet-50 and BERT.  Here each config is
// built once as a resident graph of registry launches with the same kernel names and push
// vectors those front-ends produce, in NHWC, with the fused post-ops (bias, residual,
// ReLU/ReLU6/GELU) folded into the producing kernel's epilogue.
#include <cmath>
#include <cstring>

#include "model.h"

namespace shp {

Model::~Model() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    for (auto& t : tensors)
        if (t.kind != 3 && t.ptr) (void)hipFree(t.ptr);
}

int Model::tensor(uint64_t elems, int kind) {
    MTensor t;
    t.elems = elems;
    t.kind = kind;
    hipError_t e = hipMalloc((void**)&t.ptr, (elems ? elems : 1) * sizeof(float));
    if (e != hipSuccess) {
        if (!status) status = fail(SHP_ERR_HIP, std::string("model tensor hipMalloc: ") +
                                                    hipGetErrorString(e));
        t.ptr = nullptr;
    }
    tensors.push_back(t);
    return (int)tensors.size() - 1;
}

int Model::view(int parent, uint64_t offset, uint64_t elems) {
    MTensor t;
    const MTensor& p = tensors[parent];
    if (offset + elems > p.elems && !status)
        status = fail(SHP_ERR_SHAPE, "model view exceeds its parent tensor");
    t.ptr = p.ptr ? p.ptr + offset : nullptr;
    t.elems = elems;
    t.kind = 3;
    t.parent = parent;
    t.offset = offset;
    tensors.push_back(t);
    return (int)tensors.size() - 1;
}

void Model::fill_normal(int t, uint64_t offset, uint64_t elems, float stddev) {
    if (status || !tensors[t].ptr) return;
    int rc = fill_random(ctx->stream, tensors[t].ptr + offset, elems, seed, next_id++, 1, 0.0f,
                         stddev);
    if (rc && !status) status = rc;
}

int Model::weight_normal(uint64_t elems, float stddev, float mean) {
    int t = tensor(elems, 1);
    if (!status && tensors[t].ptr) {
        int rc = fill_random(ctx->stream, tensors[t].ptr, elems, seed, next_id++, 1, mean, stddev);
        if (rc && !status) status = rc;
    }
    weight_bytes += (double)elems * 4.0;
    return t;
}

int Model::weight_const(uint64_t elems, float value) {
    int t = tensor(elems, 1);
    if (!status && tensors[t].ptr) {
        int rc = fill_random(ctx->stream, tensors[t].ptr, elems, seed, next_id++, 0, value, value);
        if (rc && !status) status = rc;
    }
    weight_bytes += (double)elems * 4.0;
    return t;
}

int Model::op(const char* kernel, int in0, int in1, int out, std::vector<int32_t> push,
              int bias, int residual, int act, float alpha, const char* label) {
    MOp o;
    o.kernel = kernel;
    o.label = label;
    o.push = std::move(push);
    o.in0 = in0;
    o.in1 = in1;
    o.out = out;
    o.bias = bias;
    o.residual = residual;
    o.act = act;
    o.alpha = alpha;
    o.out_elems = tensors[out].elems;
    workspace_need = std::max(workspace_need,
                              gemm_workspace_for_kernel(kernel, o.push.data(), o.push.size(),
                                                        &ctx->tune));
    ops.push_back(std::move(o));
    return (int)ops.size() - 1;
}

int Model::finalize() {
    if (status) return status;
    if (workspace_need) {
        int rc = ctx->ensure_workspace(workspace_need);
        if (rc) return rc;
    }
    SHP_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    return SHP_OK;
}

int Model::run_eager() {
    for (const MOp& o : ops) {
        shp_epilogue epi{o.bias >= 0 ? tensors[o.bias].ptr : nullptr,
                         o.residual >= 0 ? tensors[o.residual].ptr : nullptr, o.act, o.alpha};
        int rc = ctx->launch(o.kernel.c_str(), o.in0 >= 0 ? tensors[o.in0].ptr : nullptr,
                             o.in1 >= 0 ? tensors[o.in1].ptr : nullptr, tensors[o.out].ptr,
                             o.push.data(), o.push.size(), o.out_elems, &epi);
        if (rc) return fail(rc, "op '" + o.label + "' (" + o.kernel + "): " + std::string(shp_last_error()));
    }
    return SHP_OK;
}

int Model::run() {
    if (!use_graph) return run_eager();
    if (exec && graph_stream != ctx->stream) {  // captured on another stream: recapture
        (void)hipGraphExecDestroy(exec);
        (void)hipGraphDestroy(graph);
        exec = nullptr;
        graph = nullptr;
    }
    if (!exec) {
        bool timing = ctx->timing;
        ctx->timing = false;  // no event records inside the capture
        SHP_HIP_CHECK(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
        int rc = run_eager();
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamEndCapture(ctx->stream, &g);
        ctx->timing = timing;
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) return fail(SHP_ERR_HIP, std::string("graph capture: ") + hipGetErrorString(e));
        graph = g;
        SHP_HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
        graph_stream = ctx->stream;
    }
    SHP_HIP_CHECK(hipGraphLaunch(exec, ctx->stream));
    return SHP_OK;
}

namespace {

inline int32_t f32_bits(float f) {
    int32_t b;
    std::memcpy(&b, &f, 4);
    return b;
}

// TF SAME padding offsets, source/tflite_loader/src/scheduler.rs:1597-1614.
void same_padding(int ih, int iw, int oh, int ow, int kh, int kw, int sh, int sw, int& pt,
                  int& pl) {
    int th = std::max((oh - 1) * sh + kh - ih, 0);
    int tw = std::max((ow - 1) * sw + kw - iw, 0);
    pt = th / 2;
    pl = tw / 2;
}

struct Act4 {  // an NHWC activation tensor
    int t, n, h, w, c;
};

// ---------------------------------------------------------------------------------------
// ResNet-50 v1.5 through the HLO path (compiler.rs vulkan_convolution :768-855): NHWC
// activations, HWIO weights, `convolution` + BiasAdd + folded batchnorm collapsed into
// one conv with a bias, ReLU / residual in the epilogue.  Stride sits on the 3x3 conv of
// each downsampling bottleneck (v1.5).  The pad ops in front of the stem conv and the max
// pool (resnet50.stablehlo.txt:31,64) are folded into those ops' pad_top/pad_left: the
// conv reads zeros outside the image exactly as the padded tensor holds them, and the
// pool's input is post-ReLU (>= 0) so skipping the zero taps leaves every maximum unchanged.
Act4 rn_conv(Model& m, Act4 x, int oc, int k, int s, int act, int residual, float wscale,
             const char* label) {
    int pad = (k - 1) / 2;
    int oh = (x.h + 2 * pad - k) / s + 1, ow = (x.w + 2 * pad - k) / s + 1;
    float std_he = std::sqrt(2.0f / (float)(k * k * x.c)) * wscale;
    int w = m.weight_normal((uint64_t)k * k * x.c * oc, std_he);
    int b = m.weight_normal(oc, 0.01f);
    int y = m.tensor((uint64_t)x.n * oh * ow * oc);
    int64_t total = (int64_t)x.n * oh * ow * oc;
    m.op("hlo_conv_nhwc_hwio", x.t, w, y,
         {x.n, x.h, x.w, x.c, k, k, oc, oh, ow, s, s, pad, pad, (int32_t)total}, b, residual, act,
         0.0f, label);
    m.flops += 2.0 * (double)x.n * oh * ow * oc * k * k * x.c;
    return Act4{y, x.n, oh, ow, oc};
}

}  // namespace

int build_resnet50(Model& m, int batch) {
    const int n = batch;
    int in = m.tensor((uint64_t)n * 224 * 224 * 3, 2);
    m.inputs.push_back(in);
    if (!m.status && m.tensors[in].ptr) {  // input N(0,1)
        int rc = fill_random(m.ctx->stream, m.tensors[in].ptr, m.tensors[in].elems, m.seed ^ 1, 0,
                             1, 0.0f, 1.0f);
        if (rc) return rc;
    }
    Act4 x{in, n, 224, 224, 3};
    x = rn_conv(m, x, 64, 7, 2, SHP_ACT_RELU, -1, 1.0f, "conv1");
    // max pool 3x3 s2 pad 1 -> [n,56,56,64] (hlo_reduce_window_rank4, kind max)
    int pool = m.tensor((uint64_t)n * 56 * 56 * 64);
    m.op("hlo_reduce_window_rank4", x.t, -1, pool,
         {n, 112, 112, 64, 56, 56, 3, 3, 2, 2, 1, 1, 1, n * 56 * 56 * 64}, -1, -1, 0, 0.0f,
         "pool1");
    x = Act4{pool, n, 56, 56, 64};
    const int blocks[4] = {3, 4, 6, 3};
    char label[64];
    for (int st = 0; st < 4; ++st) {
        int width = 64 << st;
        for (int b = 0; b < blocks[st]; ++b) {
            int s = (b == 0 && st > 0) ? 2 : 1;
            int shortcut = x.t;
            if (b == 0) {
                std::snprintf(label, sizeof label, "conv%d_block%d_0", st + 2, b + 1);
                shortcut = rn_conv(m, x, 4 * width, 1, s, SHP_ACT_NONE, -1, 1.0f, label).t;
            }
            std::snprintf(label, sizeof label, "conv%d_block%d_1", st + 2, b + 1);
            Act4 t1 = rn_conv(m, x, width, 1, 1, SHP_ACT_RELU, -1, 1.0f, label);
            std::snprintf(label, sizeof label, "conv%d_block%d_2", st + 2, b + 1);
            Act4 t2 = rn_conv(m, t1, width, 3, s, SHP_ACT_RELU, -1, 1.0f, label);
            // The branch's last folded BN starts at gamma = 0.2 (the zero-gamma init
            // practice, softened) so the residual stream keeps an O(1) scale over 16 blocks.
            std::snprintf(label, sizeof label, "conv%d_block%d_3", st + 2, b + 1);
            x = rn_conv(m, t2, 4 * width, 1, 1, SHP_ACT_RELU, shortcut, 0.2f, label);
        }
    }
    // global average pool -> [n, 2048]; dense 2048 -> 1000 (dot + BiasAdd); softmax rows
    int gap = m.tensor((uint64_t)n * 2048);
    m.op("global_avg_pool_nhwc", x.t, -1, gap, {n, 7, 7, 2048}, -1, -1, 0, 0.0f, "avg_pool");
    int fw = m.weight_normal(2048 * 1000, std::sqrt(2.0f / 2048.0f));
    int fb = m.weight_normal(1000, 0.01f);
    int logits = m.tensor((uint64_t)n * 1000);
    m.op("hlo_dot_rank2", gap, fw, logits, {n, 2048, 1000, n * 1000}, fb, -1, 0, 0.0f,
         "predictions");
    m.flops += 2.0 * n * 2048.0 * 1000.0;
    int probs = m.tensor((uint64_t)n * 1000);
    m.op("softmax_rows", logits, -1, probs, {n, 1000, f32_bits(1.0f)}, -1, -1, 0, 0.0f,
         "softmax");
    m.outputs.push_back(probs);
    m.outputs.push_back(logits);
    return m.finalize();
}

// ---------------------------------------------------------------------------------------
// TFLite path (scheduler.rs): Conv2D on NHWC with the model's OHWI weights + bias tail
// (conv2d_nhwc, push layout of conv2d.comp), DepthwiseConv2D with [KH,KW,C] + bias
// (depthwise_conv2d_nhwc, push of depthwise_conv2d.comp), fused ReLU6, residual Add fused
// into the projection conv, global AveragePool2D, FullyConnected + bias tail, Softmax.
namespace {

Act4 tfl_conv(Model& m, Act4 x, int oc, int k, int s, int act, int residual, const char* label) {
    int oh = (x.h + s - 1) / s, ow = (x.w + s - 1) / s;  // SAME
    int pt, pl;
    same_padding(x.h, x.w, oh, ow, k, k, s, s, pt, pl);
    uint64_t K = (uint64_t)k * k * x.c;
    int w = m.tensor(K * oc + oc, 1);
    m.fill_normal(w, 0, K * oc, std::sqrt(2.0f / (float)K));
    m.fill_normal(w, K * oc, oc, 0.01f);
    m.weight_bytes += (double)(K * oc + oc) * 4.0;
    int y = m.tensor((uint64_t)x.n * oh * ow * oc);
    int64_t total = (int64_t)x.n * oh * ow * oc;
    m.op("conv2d_nhwc", x.t, w, y, {x.n, x.c, x.h, x.w, oc, oh, ow, k, k, s, s, 1, pt, pl,
                                    (int32_t)total},
         -1, residual, act, 0.0f, label);
    m.flops += 2.0 * (double)total * K;
    return Act4{y, x.n, oh, ow, oc};
}

Act4 tfl_depthwise(Model& m, Act4 x, int k, int s, int act, const char* label) {
    int oh = (x.h + s - 1) / s, ow = (x.w + s - 1) / s;
    int pt, pl;
    same_padding(x.h, x.w, oh, ow, k, k, s, s, pt, pl);
    uint64_t kk = (uint64_t)k * k * x.c;
    int w = m.tensor(kk + x.c, 1);
    m.fill_normal(w, 0, kk, std::sqrt(2.0f / (float)(k * k)));
    m.fill_normal(w, kk, x.c, 0.01f);
    m.weight_bytes += (double)(kk + x.c) * 4.0;
    int y = m.tensor((uint64_t)x.n * oh * ow * x.c);
    int64_t total = (int64_t)x.n * oh * ow * x.c;
    m.op("depthwise_conv2d_nhwc", x.t, w, y,
         {x.n, x.c, x.h, x.w, oh, ow, k, k, s, s, 1, pt, pl, 1, 1, (int32_t)total}, -1, -1, act,
         0.0f, label);
    m.flops += 2.0 * (double)total * k * k;
    return Act4{y, x.n, oh, ow, x.c};
}

struct MBConv {
    int expand, k, s, c, n;
};

// The push vector of one MBConv block as a single inverted_residual_nhwc launch.
std::vector<int32_t> block_push(const Act4& x, int expand, int k, int s, int cout) {
    const int ce = expand != 1 ? x.c * expand : x.c;
    int oh = (x.h + s - 1) / s, ow = (x.w + s - 1) / s;
    int pt, pl;
    same_padding(x.h, x.w, oh, ow, k, k, s, s, pt, pl);
    return {x.n, x.c, x.h, x.w, ce, cout, oh, ow, k, s, pt, pl, expand != 1 ? 1 : 0,
            SHP_ACT_RELU6, SHP_ACT_RELU6, (int32_t)((int64_t)x.n * oh * ow * cout)};
}

// One MBConv block as a single inverted_residual_nhwc launch: the three operators' weight
// tensors packed back to back in one tensor and filled in the same order with the same
// distributions (so the weights equal those of the three-operator graph of the same seed).
Act4 tfl_block(Model& m, Act4 x, int expand, int k, int s, int cout, int residual,
               const char* label) {
    const int ce = expand != 1 ? x.c * expand : x.c;
    int oh = (x.h + s - 1) / s, ow = (x.w + s - 1) / s;
    const uint64_t ne = expand != 1 ? (uint64_t)ce * x.c + ce : 0;
    const uint64_t nd = (uint64_t)k * k * ce + ce, np = (uint64_t)cout * ce + cout;
    int w = m.tensor(ne + nd + np, 1);
    if (expand != 1) {
        m.fill_normal(w, 0, (uint64_t)ce * x.c, std::sqrt(2.0f / (float)x.c));
        m.fill_normal(w, (uint64_t)ce * x.c, ce, 0.01f);
    }
    m.fill_normal(w, ne, (uint64_t)k * k * ce, std::sqrt(2.0f / (float)(k * k)));
    m.fill_normal(w, ne + (uint64_t)k * k * ce, ce, 0.01f);
    m.fill_normal(w, ne + nd, (uint64_t)cout * ce, std::sqrt(2.0f / (float)ce));
    m.fill_normal(w, ne + nd + (uint64_t)cout * ce, cout, 0.01f);
    m.weight_bytes += (double)(ne + nd + np) * 4.0;
    int y = m.tensor((uint64_t)x.n * oh * ow * cout);
    const int64_t total = (int64_t)x.n * oh * ow * cout;
    m.op("inverted_residual_nhwc", x.t, w, y, block_push(x, expand, k, s, cout), -1, residual,
         SHP_ACT_NONE, 0.0f, label);
    if (expand != 1) m.flops += 2.0 * (double)x.n * x.h * x.w * x.c * ce;
    m.flops += 2.0 * (double)x.n * oh * ow * ce * k * k + 2.0 * (double)total * ce;
    return Act4{y, x.n, oh, ow, cout};
}

// The classifier head's 1x1 conv + ReLU6 + global average pool as one launch; returns the
// pooled [n][oc] tensor.
int tfl_head(Model& m, Act4 x, int oc, const char* label) {
    const uint64_t K = (uint64_t)x.c;
    int w = m.tensor(K * oc + oc, 1);
    m.fill_normal(w, 0, K * oc, std::sqrt(2.0f / (float)K));
    m.fill_normal(w, K * oc, oc, 0.01f);
    m.weight_bytes += (double)(K * oc + oc) * 4.0;
    int y = m.tensor((uint64_t)x.n * oc);
    m.op("conv1x1_gap_nhwc", x.t, w, y, {x.n, x.c, x.h, x.w, oc, x.n * oc}, -1, -1,
         SHP_ACT_RELU6, 0.0f, label);
    m.flops += 2.0 * (double)x.n * x.h * x.w * oc * K;
    return y;
}

int tfl_net(Model& m, int batch, const MBConv* cfg, int ncfg, int stem_c) {
    const int n = batch;
    int in = m.tensor((uint64_t)n * 224 * 224 * 3, 2);
    m.inputs.push_back(in);
    if (!m.status && m.tensors[in].ptr) {  // input U[-1, 1)
        int rc = fill_random(m.ctx->stream, m.tensors[in].ptr, m.tensors[in].elems, m.seed ^ 1, 0,
                             0, -1.0f, 1.0f);
        if (rc) return rc;
    }
    char label[64];
    Act4 x = tfl_conv(m, Act4{in, n, 224, 224, 3}, stem_c, 3, 2, SHP_ACT_RELU6, -1, "stem");
    int bi = 0;
    for (int i = 0; i < ncfg; ++i) {
        for (int r = 0; r < cfg[i].n; ++r, ++bi) {
            int s = r == 0 ? cfg[i].s : 1;
            const int fuse = m.ctx->tune.ir_fuse;
            const std::vector<int32_t> bp = block_push(x, cfg[i].expand, cfg[i].k, s, cfg[i].c);
            if (fuse > 0 || (fuse == 0 && block_fusion_pays(bp.data(), bp.size()))) {
                std::snprintf(label, sizeof label, "block%d_mbconv", bi);
                x = tfl_block(m, x, cfg[i].expand, cfg[i].k, s, cfg[i].c,
                              s == 1 && x.c == cfg[i].c ? x.t : -1, label);
                continue;
            }
            Act4 in_x = x;
            Act4 h = x;
            bool res = s == 1 && in_x.c == cfg[i].c;
            if (cfg[i].expand != 1) {
                std::snprintf(label, sizeof label, "block%d_expand", bi);
                h = tfl_conv(m, x, x.c * cfg[i].expand, 1, 1, SHP_ACT_RELU6, -1, label);
                // the depthwise and the projection as one launch where that pays (the
                // expanded tensor as the input; its weights fill as the two operators')
                const std::vector<int32_t> dp = block_push(h, 1, cfg[i].k, s, cfg[i].c);
                if (fuse == 0 && block_fusion_pays(dp.data(), dp.size())) {
                    std::snprintf(label, sizeof label, "block%d_dwproj", bi);
                    x = tfl_block(m, h, 1, cfg[i].k, s, cfg[i].c, res ? in_x.t : -1, label);
                    continue;
                }
            }
            std::snprintf(label, sizeof label, "block%d_depthwise", bi);
            h = tfl_depthwise(m, h, cfg[i].k, s, SHP_ACT_RELU6, label);
            std::snprintf(label, sizeof label, "block%d_project", bi);
            x = tfl_conv(m, h, cfg[i].c, 1, 1, SHP_ACT_NONE, res ? in_x.t : -1, label);
        }
    }
    int gap;
    if (m.ctx->tune.ir_fuse >= 0) {
        // the head's 1x1 conv + ReLU6 and the global average pool as one conv1x1_gap_nhwc
        // launch (weights filled as tfl_conv fills them, so they equal the two-operator
        // graph's of the same seed); the three-operator build keeps the reference's two
        gap = tfl_head(m, x, 1280, "head_conv_pool");
    } else {
        x = tfl_conv(m, x, 1280, 1, 1, SHP_ACT_RELU6, -1, "head_conv");
        gap = m.tensor((uint64_t)n * 1280);
        m.op("global_avg_pool_nhwc", x.t, -1, gap, {n, x.h, x.w, 1280}, -1, -1, 0, 0.0f,
             "avg_pool");
    }
    int fw = m.tensor(1280 * 1000 + 1000, 1);
    m.fill_normal(fw, 0, 1280 * 1000, std::sqrt(2.0f / 1280.0f));
    m.fill_normal(fw, 1280 * 1000, 1000, 0.01f);
    m.weight_bytes += (1280.0 * 1000 + 1000) * 4.0;
    int logits = m.tensor((uint64_t)n * 1000);
    m.op("fully_connected", gap, fw, logits, {n, 1280, 1000, n * 1000}, -1, -1, 0, 0.0f, "fc");
    m.flops += 2.0 * n * 1280.0 * 1000.0;
    // Softmax exactly as the reference dispatches it: softmax1000.comp over every element
    // of the output (classes = element_count, scheduler.rs:289), i.e. across the batch.
    int probs = m.tensor((uint64_t)n * 1000);
    m.op("softmax1000", logits, -1, probs, {n * 1000}, -1, -1, 0, 0.0f, "softmax");
    m.outputs.push_back(probs);
    m.outputs.push_back(logits);
    return m.finalize();
}

}  // namespace

int build_mobilenet_v2(Model& m, int batch) {
    // (expansion, kernel, stride, channels, repeats) — MobileNetV2-1.0
    static const MBConv cfg[] = {{1, 3, 1, 16, 1},  {6, 3, 2, 24, 2},  {6, 3, 2, 32, 3},
                                 {6, 3, 2, 64, 4},  {6, 3, 1, 96, 3},  {6, 3, 2, 160, 3},
                                 {6, 3, 1, 320, 1}};
    return tfl_net(m, batch, cfg, 7, 32);
}

int build_efficientnet_lite0(Model& m, int batch) {
    // EfficientNet-Lite0: MBConv without squeeze-excitation, ReLU6, 3x3/5x5 depthwise
    static const MBConv cfg[] = {{1, 3, 1, 16, 1},  {6, 3, 2, 24, 2},  {6, 5, 2, 40, 2},
                                 {6, 3, 2, 80, 3},  {6, 5, 1, 112, 3}, {6, 5, 2, 192, 4},
                                 {6, 3, 1, 320, 1}};
    return tfl_net(m, batch, cfg, 7, 32);
}

// ---------------------------------------------------------------------------------------
// BERT-base encoder through the HLO path: dot (hlo_dot_rank2) with bias/GELU/residual
// epilogues, attention as two dot_generals read in place from the fused QKV activation
// (no transposes, compiler.rs:1043-1058), row softmax with the 1/sqrt(64) scale
// (bert_base.stablehlo.txt:28-49), LayerNorm eps 1e-12.  At sequence 128 the three attention
// ops are one attention_fused launch (same math, Q/K/V read in place).
int build_bert_base(Model& m, int batch, int seq) {
    const int B = batch, S = seq, D = 768, H = 12, HD = 64, F = 3072, L = 12, V = 30522;
    const int M = B * S;
    if (S > 512 || S <= 0) return fail(SHP_ERR_SHAPE, "bert_base: seq_len must be in [1, 512]");
    int ids = m.tensor((uint64_t)M, 2);
    m.inputs.push_back(ids);
    if (!m.status && m.tensors[ids].ptr) {
        int rc = fill_random(m.ctx->stream, m.tensors[ids].ptr, M, m.seed ^ 3, 0, 2, 0.0f,
                             (float)V);
        if (rc) return rc;
    }
    int word = m.weight_normal((uint64_t)V * D, 0.02f);
    int pos = m.weight_normal(512ull * D, 0.02f);
    int type = m.weight_normal(2ull * D, 0.02f);
    int emb = m.tensor((uint64_t)M * D);
    m.op("gather_rows", ids, word, emb, {M, D, V}, -1, -1, 0, 0.0f, "word_embeddings");
    int e1 = m.tensor((uint64_t)M * D);
    // + position_embeddings[s]: broadcast over the batch (strides b:0, s:D, d:1)
    m.op("broadcast_binary", emb, pos, e1,
         {0, M * D, 1, B, S, D, 0, S * D, D, 1, 0, 0, D, 1}, -1, -1, 0, 0.0f, "add_position");
    int e2 = m.tensor((uint64_t)M * D);
    m.op("broadcast_binary", e1, type, e2, {0, M * D, 1, 1, M, D, 0, 0, D, 1, 0, 0, 0, 1}, -1,
         -1, 0, 0.0f, "add_token_type");
    auto ln_weights = [&]() {
        int t = m.tensor(2ull * D, 1);
        if (!m.status && m.tensors[t].ptr) {
            fill_random(m.ctx->stream, m.tensors[t].ptr, D, m.seed, m.next_id++, 0, 1.0f, 1.0f);
            fill_random(m.ctx->stream, m.tensors[t].ptr + D, D, m.seed, m.next_id++, 0, 0.0f, 0.0f);
        }
        m.weight_bytes += 2.0 * D * 4.0;
        return t;
    };
    const int32_t eps = f32_bits(1e-12f);
    int x = m.tensor((uint64_t)M * D);
    m.op("layernorm_rows", e2, ln_weights(), x, {M, D, eps}, -1, -1, 0, 0.0f, "embeddings_ln");
    int mask = m.weight_const(S, 0.0f);  // full attention mask: additive zeros
    char label[64];
    for (int l = 0; l < L; ++l) {
        int wqkv = m.weight_normal((uint64_t)D * 3 * D, 0.02f);
        int bqkv = m.weight_const(3 * D, 0.0f);
        int qkv = m.tensor((uint64_t)M * 3 * D);
        std::snprintf(label, sizeof label, "layer%d_qkv", l);
        m.op("hlo_dot_rank2", x, wqkv, qkv, {M, D, 3 * D, M * 3 * D}, bqkv, -1, 0, 0.0f, label);
        int ctxt = m.tensor((uint64_t)M * D);
        if (S == 128) {
            // the other branch's three ops in one launch (the fused kernel's sequence length)
            std::snprintf(label, sizeof label, "layer%d_attention", l);
            m.op("attention_fused", qkv, mask, ctxt,
                 {B, H, S, HD, 3 * D, 0, D, 2 * D, D, f32_bits(0.125f), M * D}, -1, -1, 0, 0.0f,
                 label);
        } else {
            int q = m.view(qkv, 0, (uint64_t)M * 3 * D);
            int k = m.view(qkv, D, (uint64_t)M * 3 * D - D);
            int v = m.view(qkv, 2 * D, (uint64_t)M * 3 * D - 2 * D);
            int scores = m.tensor((uint64_t)B * H * S * S);
            // scores[b,h,s,t] = sum_d Q[b,s,h,d] K[b,t,h,d]
            std::snprintf(label, sizeof label, "layer%d_scores", l);
            m.op("dot_general_strided", q, k, scores,
                 {B, H, S, S, HD, S * 3 * D, HD, 3 * D, 1, S * 3 * D, HD, 1, 3 * D, H * S * S, S * S,
                  S, 1},
                 -1, -1, 0, 0.0f, label);
            int probs = m.tensor((uint64_t)B * H * S * S);
            std::snprintf(label, sizeof label, "layer%d_softmax", l);
            m.op("softmax_rows", scores, mask, probs, {B * H * S, S, f32_bits(0.125f)}, -1, -1, 0,
                 0.0f, label);
            // ctx[b,s,h,d] = sum_t P[b,h,s,t] V[b,t,h,d]
            std::snprintf(label, sizeof label, "layer%d_context", l);
            m.op("dot_general_strided", probs, v, ctxt,
                 {B, H, S, HD, S, H * S * S, S * S, S, 1, S * 3 * D, HD, 3 * D, 1, S * D, HD, D, 1},
                 -1, -1, 0, 0.0f, label);
        }
        int wo = m.weight_normal((uint64_t)D * D, 0.02f);
        int bo = m.weight_const(D, 0.0f);
        int t1 = m.tensor((uint64_t)M * D);
        std::snprintf(label, sizeof label, "layer%d_attn_out", l);
        m.op("hlo_dot_rank2", ctxt, wo, t1, {M, D, D, M * D}, bo, x, 0, 0.0f, label);
        int x1 = m.tensor((uint64_t)M * D);
        std::snprintf(label, sizeof label, "layer%d_attn_ln", l);
        m.op("layernorm_rows", t1, ln_weights(), x1, {M, D, eps}, -1, -1, 0, 0.0f, label);
        int w1 = m.weight_normal((uint64_t)D * F, 0.02f);
        int b1 = m.weight_const(F, 0.0f);
        int hdn = m.tensor((uint64_t)M * F);
        std::snprintf(label, sizeof label, "layer%d_ffn1", l);
        m.op("hlo_dot_rank2", x1, w1, hdn, {M, D, F, M * F}, b1, -1, SHP_ACT_GELU_ERF, 0.0f, label);
        int w2 = m.weight_normal((uint64_t)F * D, 0.02f);
        int b2 = m.weight_const(D, 0.0f);
        int t2 = m.tensor((uint64_t)M * D);
        std::snprintf(label, sizeof label, "layer%d_ffn2", l);
        m.op("hlo_dot_rank2", hdn, w2, t2, {M, F, D, M * D}, b2, x1, 0, 0.0f, label);
        int x2 = m.tensor((uint64_t)M * D);
        std::snprintf(label, sizeof label, "layer%d_out_ln", l);
        m.op("layernorm_rows", t2, ln_weights(), x2, {M, D, eps}, -1, -1, 0, 0.0f, label);
        m.flops += 2.0 * M * D * 3.0 * D + 2.0 * 2.0 * B * H * S * S * HD + 2.0 * M * D * D +
                   2.0 * 2.0 * M * D * F;
        x = x2;
    }
    m.outputs.push_back(x);
    return m.finalize();
}

}  // namespace shp

using shp::fail;
using shp::Model;

extern "C" {

int shp_model_create(shp_ctx* ctx, const char* arch, int32_t batch, int32_t seq_len,
                     uint64_t seed, shp_model** out) {
    if (!ctx || !arch || !out) return fail(SHP_ERR_INVALID, "shp_model_create: null argument");
    {
        int grc = shp::refuse_while_capturing(reinterpret_cast<shp::Ctx*>(ctx)->stream,
                                              "shp_model_create");
        if (grc) return grc;
    }
    if (batch <= 0) return fail(SHP_ERR_SHAPE, "shp_model_create: batch must be > 0");
    *out = nullptr;
    Model* m = new Model();
    m->ctx = reinterpret_cast<shp::Ctx*>(ctx);
    m->arch = arch;
    m->seed = seed;
    (void)hipSetDevice(m->ctx->device);
    std::string a = arch;
    int rc;
    if (a == "resnet50_v1_5" || a == "resnet50") rc = shp::build_resnet50(*m, batch);
    else if (a == "mobilenet_v2") rc = shp::build_mobilenet_v2(*m, batch);
    else if (a == "efficientnet_lite0") rc = shp::build_efficientnet_lite0(*m, batch);
    else if (a == "bert_base") rc = shp::build_bert_base(*m, batch, seq_len > 0 ? seq_len : 128);
    else rc = fail(SHP_ERR_INVALID, "shp_model_create: unknown arch '" + a + "'");
    if (!rc) rc = m->status;
    if (rc) {
        delete m;
        return rc;
    }
    *out = reinterpret_cast<shp_model*>(m);
    return SHP_OK;
}

void shp_model_destroy(shp_model* model) {
    if (!model) return;
    Model* m = reinterpret_cast<Model*>(model);
    (void)hipStreamSynchronize(m->ctx->stream);
    delete m;
}

int shp_model_run(shp_model* model) {
    if (!model) return fail(SHP_ERR_INVALID, "shp_model_run: null model");
    Model* m = reinterpret_cast<Model*>(model);
    if (m->use_graph) {  // the model captures its own graph: no nesting in the caller's
        int rc = shp::refuse_while_capturing(m->ctx->stream, "shp_model_run with a graph");
        if (rc) return rc;
    }
    return m->run();
}

int shp_model_use_graph(shp_model* model, int enable) {
    if (!model) return fail(SHP_ERR_INVALID, "shp_model_use_graph: null model");
    Model* m = reinterpret_cast<Model*>(model);
    m->use_graph = enable != 0;
    if (!enable && m->exec) {  // a later enable captures again (with the current planner state)
        (void)hipStreamSynchronize(m->ctx->stream);
        (void)hipGraphExecDestroy(m->exec);
        (void)hipGraphDestroy(m->graph);
        m->exec = nullptr;
        m->graph = nullptr;
    }
    return SHP_OK;
}

static int io(shp_model* model, const std::vector<int>& which, int index, void** dptr,
              uint64_t* elems) {
    if (!model || !dptr || !elems) return fail(SHP_ERR_INVALID, "model io: null argument");
    Model* m = reinterpret_cast<Model*>(model);
    if (index < 0 || index >= (int)which.size()) return fail(SHP_ERR_INVALID, "model io: index");
    const shp::MTensor& t = m->tensors[which[index]];
    *dptr = t.ptr;
    *elems = t.elems;
    return SHP_OK;
}

int shp_model_input(shp_model* model, int index, void** dptr, uint64_t* elems) {
    return io(model, model ? reinterpret_cast<Model*>(model)->inputs : std::vector<int>{}, index,
              dptr, elems);
}

int shp_model_output(shp_model* model, int index, void** dptr, uint64_t* elems) {
    return io(model, model ? reinterpret_cast<Model*>(model)->outputs : std::vector<int>{}, index,
              dptr, elems);
}

int shp_model_work(shp_model* model, double* flops, double* weight_bytes) {
    if (!model) return fail(SHP_ERR_INVALID, "shp_model_work: null model");
    Model* m = reinterpret_cast<Model*>(model);
    if (flops) *flops = m->flops;
    if (weight_bytes) *weight_bytes = m->weight_bytes;
    return SHP_OK;
}

int shp_model_num_ops(shp_model* model) {
    return model ? (int)reinterpret_cast<Model*>(model)->ops.size() : 0;
}

int shp_model_op(shp_model* model, int index, shp_op_desc* d) {
    if (!model || !d) return fail(SHP_ERR_INVALID, "shp_model_op: null argument");
    Model* m = reinterpret_cast<Model*>(model);
    if (index < 0 || index >= (int)m->ops.size()) return fail(SHP_ERR_INVALID, "shp_model_op: index");
    const shp::MOp& o = m->ops[index];
    std::memset(d, 0, sizeof(*d));
    std::snprintf(d->kernel, sizeof d->kernel, "%s", o.kernel.c_str());
    std::snprintf(d->label, sizeof d->label, "%s", o.label.c_str());
    d->n_push = (int32_t)std::min<size_t>(o.push.size(), 40);
    for (int i = 0; i < d->n_push; ++i) d->push[i] = o.push[i];
    d->in0 = o.in0;
    d->in1 = o.in1;
    d->out = o.out;
    d->bias = o.bias;
    d->residual = o.residual;
    d->act = o.act;
    d->alpha = o.alpha;
    d->out_elems = o.out_elems;
    return SHP_OK;
}

int shp_model_num_tensors(shp_model* model) {
    return model ? (int)reinterpret_cast<Model*>(model)->tensors.size() : 0;
}

int shp_model_tensor(shp_model* model, int id, void** dptr, uint64_t* elems, int32_t* kind) {
    if (!model) return fail(SHP_ERR_INVALID, "shp_model_tensor: null model");
    Model* m = reinterpret_cast<Model*>(model);
    if (id < 0 || id >= (int)m->tensors.size()) return fail(SHP_ERR_INVALID, "shp_model_tensor: id");
    const shp::MTensor& t = m->tensors[id];
    if (dptr) *dptr = t.ptr;
    if (elems) *elems = t.elems;
    if (kind) *kind = t.kind;
    return SHP_OK;
}

int shp_model_tensor_parent(shp_model* model, int id, int32_t* parent, uint64_t* offset) {
    if (!model) return fail(SHP_ERR_INVALID, "shp_model_tensor_parent: null model");
    Model* m = reinterpret_cast<Model*>(model);
    if (id < 0 || id >= (int)m->tensors.size())
        return fail(SHP_ERR_INVALID, "shp_model_tensor_parent: id");
    if (parent) *parent = m->tensors[id].parent;
    if (offset) *offset = m->tensors[id].offset;
    return SHP_OK;
}

}  // extern "C"
