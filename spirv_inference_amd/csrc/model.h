// Resident op graphs: every tensor is hipMalloc'd once, ops are registry launches on the
// context stream, optionally captured once into a hipGraph and replayed.  This is the
// chained runtime of runtime/chained_graph_runtime/src/main.rs:260-590 (persistent buffers,
// one submission for the whole chain) generalised to whole models.
#pragma once

#include <string>
#include <vector>

#include "runtime.h"

namespace shp {

struct MTensor {
    float* ptr = nullptr;
    uint64_t elems = 0;
    int kind = 0;        // 0 activation, 1 weight/constant, 2 model input, 3 view
    int parent = -1;     // views: the tensor they alias
    uint64_t offset = 0; // views: element offset into the parent
};

struct MOp {
    std::string kernel, label;
    std::vector<int32_t> push;
    int in0 = -1, in1 = -1, out = -1, bias = -1, residual = -1;
    int act = SHP_ACT_NONE;
    float alpha = 0.0f;
    uint64_t out_elems = 0;
};

struct Model {
    Ctx* ctx = nullptr;
    std::string arch;
    uint64_t seed = 0;
    uint64_t next_id = 1;
    std::vector<MTensor> tensors;
    std::vector<MOp> ops;
    std::vector<int> inputs, outputs;
    double flops = 0.0, weight_bytes = 0.0;
    size_t workspace_need = 0;
    bool use_graph = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipStream_t graph_stream = nullptr;

    ~Model();
    int status = SHP_OK;  // first error hit while building

    int tensor(uint64_t elems, int kind = 0);
    int view(int parent, uint64_t offset, uint64_t elems);
    int weight_normal(uint64_t elems, float stddev, float mean = 0.0f);
    int weight_const(uint64_t elems, float value);
    // Fill [offset, offset+elems) of an existing tensor (packed weight + bias tails).
    void fill_normal(int t, uint64_t offset, uint64_t elems, float stddev);
    int op(const char* kernel, int in0, int in1, int out, std::vector<int32_t> push,
           int bias = -1, int residual = -1, int act = SHP_ACT_NONE, float alpha = 0.0f,
           const char* label = "");
    int finalize();  // size the split-K workspace
    int run();
    int run_eager();
};

int build_resnet50(Model& m, int batch);
int build_mobilenet_v2(Model& m, int batch);
int build_efficientnet_lite0(Model& m, int batch);
int build_bert_base(Model& m, int batch, int seq);

}  // namespace shp
