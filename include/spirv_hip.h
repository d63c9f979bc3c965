/*
 * spirv_hip.h — C ABI of the MI355X (gfx950) operator-kernel library.
 *
 * This is the drop-in boundary for the operator-dispatch layer of
 * agkdc1/SPIRV_INFERENCE.  The reference crosses the device boundary through
 *   tflite_loader::vulkan::run_kernel(device_selector, &KernelRun) -> KernelOutput
 *   (source/tflite_loader/src/vulkan.rs:27-44)
 * which creates a Vulkan device, uploads, dispatches one SPIR-V module chosen by
 * name (source/tflite_loader/src/kernels.rs:12-238), waits and reads back on every
 * call.  Here the kernel is still chosen by the reference's kernel name and driven by
 * the exact i32 push-constant vector of that kernel's `Params` block, but the device,
 * stream and tensors are created once and stay resident in HBM.
 *
 * Plain C: no HIP or torch types in any signature.  Every entry point returns
 * SHP_OK (0) or a negative SHP_ERR_* code; shp_last_error() gives a thread-local
 * message.  Unknown kernels, short push vectors and inconsistent sizes are errors,
 * never a silent fallback (mirrors the fail-closed `bail!` of
 * source/tflite_loader/src/scheduler.rs:1003-1007).
 *
 * One context = one HIP stream on one device.  A context is not thread-safe.
 * shp_launch* are asynchronous on the context stream; shp_run_kernel is synchronous.
 */
#ifndef SPIRV_HIP_H
#define SPIRV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------- */
#define SHP_OK 0
#define SHP_ERR_INVALID (-1)        /* null pointer / bad argument */
#define SHP_ERR_UNKNOWN_KERNEL (-2) /* name not in the registry */
#define SHP_ERR_PUSH (-3)           /* push vector shorter than the kernel's Params */
#define SHP_ERR_SHAPE (-4)          /* sizes inconsistent with the push vector */
#define SHP_ERR_HIP (-5)            /* HIP runtime error */
#define SHP_ERR_NO_DEVICE (-6)      /* selector matched no device */
#define SHP_ERR_UNSUPPORTED (-7)    /* configuration the kernel does not handle */

/* ---- types ----------------------------------------------------------------- */
typedef struct shp_ctx shp_ctx;

/* Replaces KernelOutput (source/tflite_loader/src/vulkan.rs:18-25).  The values
 * vector is written into the caller's `out` buffer instead of being returned. */
typedef struct shp_run_info {
    char device_name[256];
    uint32_t vendor_id; /* 0x1002 for AMD */
    uint32_t device_id;
    double elapsed_ms; /* hipEvent pair around the dispatch (kernel time only) */
} shp_run_info;

/* Fused activations applied in kernel epilogues.  The reference applies them as a
 * separate post-op dispatch (apply_activation, source/tflite_loader/src/scheduler.rs:1146-1197). */
enum {
    SHP_ACT_NONE = 0,
    SHP_ACT_RELU = 1,     /* relu.comp: max(x, 0) */
    SHP_ACT_RELU6 = 2,    /* relu6.comp: min(max(x, 0), 6) */
    SHP_ACT_LEAKY = 3,    /* leaky_relu.comp: max(alpha*x, x) */
    SHP_ACT_SIGMOID = 4,  /* sigmoid.comp: 1/(1+exp(-x)) */
    SHP_ACT_TANH = 5,     /* tanh.comp: clamp to +-20, (e^x-e^-x)/(e^x+e^-x) */
    SHP_ACT_SILU = 6,     /* x*sigmoid(x) (export_llama.py:298-299) */
    SHP_ACT_GELU_ERF = 7  /* 0.5*x*erfc(-x/sqrt(2)) (bert_base.stablehlo.txt:16-17) */
};

/* Epilogue of the dense and depthwise kernels: out = act(acc + bias[c] + residual).
 * `bias` is indexed by the output channel (last NHWC dim, the OC of NCHW, or the
 * column of a GEMM); `residual` has the layout of `out`.  Either may be NULL. */
typedef struct shp_epilogue {
    const float* bias;
    const float* residual;
    int32_t act;
    float alpha;
} shp_epilogue;

/* ---- context / device (device selection: vulkan.rs:204-231) ----------------- */

/* selector: "any", "amd", or a decimal device ordinal ("0").  Reports vendor 0x1002. */
int shp_create(const char* selector, shp_ctx** out);
void shp_destroy(shp_ctx* ctx);
const char* shp_last_error(void);
int shp_device_info(shp_ctx* ctx, shp_run_info* info);
/* Run the context's work on an external hipStream_t (NULL = the context's own). */
int shp_set_stream(shp_ctx* ctx, void* hip_stream);
void* shp_get_stream(shp_ctx* ctx);

/* ---- resident tensors (new: the reference re-uploads per op, vulkan.rs:109-112,172) */
int shp_alloc(shp_ctx* ctx, size_t bytes, void** dptr);
int shp_free(shp_ctx* ctx, void* dptr);
int shp_upload(shp_ctx* ctx, void* dst_dev, const void* src_host, size_t bytes);
int shp_download(shp_ctx* ctx, void* dst_host, const void* src_dev, size_t bytes);
int shp_sync(shp_ctx* ctx);

/* Deterministic counter-based fill used for the synthetic inputs and random-init
 * weights of the benchmark configs: value i of tensor `tensor_id` depends only on
 * (seed, tensor_id, i).  kind 0: uniform [lo, hi); kind 1: normal(mean=lo, std=hi);
 * kind 2: uniform integers in [lo, hi) written as int32 (token ids). */
int shp_fill_random(shp_ctx* ctx, float* dptr, uint64_t n, uint64_t seed, uint64_t tensor_id,
                    int32_t kind, float lo, float hi);

/* ---- kernel registry (source/tflite_loader/src/kernels.rs:12-257) ------------ */
int shp_kernel_count(void);
const char* shp_kernel_name(int index);
/* Number of i32 push constants of the kernel's Params block, or <0 if unknown. */
int shp_kernel_push_count(const char* kernel);

/* ---- dispatch ----------------------------------------------------------------- */

/* Device-pointer launch: the three-binding ABI of every .comp kernel
 * (binding 0 = in0, 1 = in1/weights, 2 = out) plus its i32 push vector.  Replaces the
 * KernelRun of vulkan.rs:27-36; `out_elems` is the KernelRun::output_elements. */
int shp_launch(shp_ctx* ctx, const char* kernel, const void* in0, const void* in1, void* out,
               const int32_t* push, size_t n_push, uint64_t out_elems);

/* As shp_launch, with a fused epilogue (bias / residual / activation). */
int shp_launch_ex(shp_ctx* ctx, const char* kernel, const void* in0, const void* in1, void* out,
                  const int32_t* push, size_t n_push, uint64_t out_elems,
                  const shp_epilogue* epi);

/* As shp_launch_ex, but allocates nothing.  No counterpart in the reference: it is for
 * callers that cannot call hipMalloc (code under stream capture, tight serving loops,
 * harnesses that forbid allocation).  The dense kernels' split-K partials and tile counters
 * live in one fixed 64 MiB device array per GPU (held until the process ends) instead of the
 * context workspace; a launch whose plan needs more returns SHP_ERR_UNSUPPORTED before
 * anything runs.  Every call on one GPU shares that array: calls that overlap on one GPU
 * (other streams, other contexts, other threads) race.  Per-launch timing does not apply. */
int shp_launch_static(shp_ctx* ctx, const char* kernel, const void* in0, const void* in1,
                      void* out, const int32_t* push, size_t n_push, uint64_t out_elems,
                      const shp_epilogue* epi);

/* Plan query of the fused MBConv kernel inverted_residual_nhwc (one launch for the three
 * operators scheduler.rs:321-548 dispatches for a MobileNetV2 / EfficientNet-Lite block:
 * 1x1 CONV_2D, DEPTHWISE_CONV_2D, 1x1 CONV_2D + residual ADD).  Host-only, no device needed.
 * out8 = {tile rows, tile columns, expanded-channel splits, output-channel splits, LDS bytes,
 * workgroups, projection blocks per wavefront, 1 if one launch is expected to beat the three
 * operators}.  Returns SHP_ERR_UNSUPPORTED for blocks the kernel does not take (a front end
 * then dispatches the three operators). */
int shp_block_plan(const int32_t* push, size_t n_push, int32_t* out8);

/* Host-to-host synchronous call with the semantics of
 * run_kernel(device_selector, &KernelRun) (source/tflite_loader/src/vulkan.rs:42-44):
 * upload in0[n0], in1[n1], dispatch, wait, download out[n_out].  grid_hint (the
 * reference's dispatch_x) is advisory.  `info` may be NULL. */
int shp_run_kernel(shp_ctx* ctx, const char* kernel, const float* in0, size_t n0,
                   const float* in1, size_t n1, float* out, size_t n_out, const int32_t* push,
                   size_t n_push, uint32_t grid_hint, shp_run_info* info);

/* ---- captured launch sequences (hipGraph) ------------------------------------
 * The reference records and submits a command buffer per dispatch
 * (source/tflite_loader/src/vulkan.rs:132-171).  A caller that repeats one sequence of
 * shp_launch* calls on a context records it once: between shp_capture_begin and
 * shp_capture_end nothing runs, the launches are recorded; shp_graph_launch replays them
 * on the context stream.  The recorded launches keep the device pointers they were given
 * (tensors, the context's split-K workspace): run the sequence once eagerly before
 * capturing so the workspace has its final size, and keep every tensor alive while the
 * graph can be replayed.  Per-launch timing is not recorded inside a capture. */
typedef struct shp_graph shp_graph;
int shp_capture_begin(shp_ctx* ctx);
int shp_capture_end(shp_ctx* ctx, shp_graph** out);
int shp_graph_launch(shp_graph* graph);
void shp_graph_destroy(shp_graph* graph);

/* ---- per-launch timing (the reference's KernelOutput.elapsed_ms, vulkan.rs:163-171) */
/* When enabled, every launch is bracketed by hipEvents on the context stream and
 * accumulated per kernel name. */
int shp_timing_enable(shp_ctx* ctx, int enable);
int shp_timing_reset(shp_ctx* ctx);
/* Fills name/total ms/count of entry `index` (synchronises first). */
int shp_timing_entry(shp_ctx* ctx, int index, char* name, size_t name_cap, double* total_ms,
                     uint64_t* count);
/* The timed launches one by one, in issue order since the last reset: the per-dispatch
 * `elapsed_ms` of the HLO runner's report (source/xla_hlo/src/compiler.rs:675-692
 * dispatch_record).  Both synchronise first. */
int shp_timing_launch_count(shp_ctx* ctx, uint64_t* count);
int shp_timing_launch(shp_ctx* ctx, uint64_t index, char* name, size_t name_cap, double* ms);

/* ---- resident op graphs: the chained runtime (runtime/chained_graph_runtime/src/main.rs:260-590)
 *      generalised, and the model drivers of the benchmark configs ---------------- */
typedef struct shp_model shp_model;

/* arch: "resnet50_v1_5" (HLO path, NHWC/HWIO, BN folded), "mobilenet_v2",
 * "efficientnet_lite0" (TFLite path), "bert_base".  seq_len only for bert_base.
 * Weights are filled with shp_fill_random(seed) per the config's init rule. */
int shp_model_create(shp_ctx* ctx, const char* arch, int32_t batch, int32_t seq_len,
                     uint64_t seed, shp_model** out);
void shp_model_destroy(shp_model* model);
/* Enqueue one forward pass of every op on the context stream. */
int shp_model_run(shp_model* model);
/* Capture the op list into a hipGraph once and replay it on later runs; disabling releases
 * the capture, so the next enable records the op list again. */
int shp_model_use_graph(shp_model* model, int enable);
int shp_model_input(shp_model* model, int index, void** dptr, uint64_t* elems);
int shp_model_output(shp_model* model, int index, void** dptr, uint64_t* elems);
/* Algorithmic work of one forward pass: 2*MAC of convs/GEMMs, and weight bytes. */
int shp_model_work(shp_model* model, double* flops, double* weight_bytes);

/* Op-list introspection: lets a checker replay every op on other hardware. */
typedef struct shp_op_desc {
    char kernel[64];
    int32_t push[40];
    int32_t n_push;
    int32_t in0, in1, out;   /* tensor ids (-1 = none) */
    int32_t bias, residual;  /* epilogue tensor ids (-1 = none) */
    int32_t act;
    float alpha;
    uint64_t out_elems;
    char label[64];
} shp_op_desc;
int shp_model_num_ops(shp_model* model);
int shp_model_op(shp_model* model, int index, shp_op_desc* desc);
int shp_model_num_tensors(shp_model* model);
/* kind: 0 activation, 1 weight/constant, 2 model input, 3 view into another tensor */
int shp_model_tensor(shp_model* model, int id, void** dptr, uint64_t* elems, int32_t* kind);
/* For a view: the tensor it aliases and its element offset (parent -1 otherwise). */
int shp_model_tensor_parent(shp_model* model, int id, int32_t* parent, uint64_t* offset);

/* ---- TinyLlama-shaped greedy decode with a KV cache (export_llama.py:269-375 math,
 *      run_llama_spirv.py:194-295 loop, without the full S=64 recompute) ----------- */
typedef struct shp_llama shp_llama;
typedef struct shp_llama_config {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_seq;
    float rms_eps, rope_theta;
} shp_llama_config;

int shp_llama_create(shp_ctx* ctx, const shp_llama_config* cfg, uint64_t seed,
                     shp_llama** out);
void shp_llama_destroy(shp_llama* lm);
/* Clears the KV cache and the position counter.  Like every call below that copies,
 * clears memory or synchronises, it returns SHP_ERR_INVALID while the context stream is
 * being captured (between shp_capture_begin and shp_capture_end). */
int shp_llama_reset(shp_llama* lm);
/* Runs one token at the current position (KV cache append), writes logits to the
 * device logits buffer and the greedy argmax (lowest index on ties) to the device
 * token slot; advances the position. Asynchronous. */
int shp_llama_step(shp_llama* lm, int32_t token);
/* Runs n_steps tokens, each fed by the previous step's on-device argmax (no host round
 * trip between tokens).  Asynchronous. */
int shp_llama_decode(shp_llama* lm, int32_t n_steps);
/* Synchronises and copies the argmax of every step so far (one per step, in order). */
int shp_llama_tokens(shp_llama* lm, int32_t* out, int32_t cap, int32_t* n_out);
/* Feeds prompt[0..n_prompt) then generates n_new greedy tokens into out_tokens
 * (synchronous).  Stops early at token 2 (EOS) or 0 (PAD) like run_llama_spirv.py:292-294;
 * returns the number written through *n_out. */
int shp_llama_generate(shp_llama* lm, const int32_t* prompt, int32_t n_prompt, int32_t n_new,
                       int32_t* out_tokens, int32_t* n_out);
int shp_llama_use_graph(shp_llama* lm, int enable);
/* Decode engines.  All three compute the same math on the same device state, so they can be
 * switched between calls.
 *   SHP_LLAMA_KERNELS     one launch per op (5 per layer + lm_head + argmax), eager;
 *   SHP_LLAMA_GRAPH       the same launches replayed from a hipGraph per token;
 *   SHP_LLAMA_PERSISTENT  one cooperative launch per step/decode call: a workgroup per CU
 *                         streams its share of every layer, phases separated by grid
 *                         barriers (default where the device and shape allow it).
 * use_graph(1/0) selects GRAPH/KERNELS.  Selecting PERSISTENT where it is unavailable
 * returns SHP_ERR_UNSUPPORTED with the reason. */
enum { SHP_LLAMA_KERNELS = 0, SHP_LLAMA_GRAPH = 1, SHP_LLAMA_PERSISTENT = 2 };
int shp_llama_set_engine(shp_llama* lm, int engine);
int shp_llama_engine(shp_llama* lm, int* engine);
/* Bound of the persistent engine's grid waits, in polls (default 2^22, about seconds; a
 * negative value restores it).  A wait that gives up makes every workgroup exit; the call
 * then returns SHP_ERR_HIP and the decode state is undefined until shp_llama_reset, as
 * run_llama_spirv.py:76-81,237-246 aborts on a non-zero status.  A small limit forces that
 * path from the host (tests of the recovery).  No counterpart in the reference, whose
 * dispatches never wait on each other inside a launch. */
int shp_llama_set_wait_limit(shp_llama* lm, int64_t polls);
int shp_llama_logits(shp_llama* lm, void** dptr, uint64_t* elems);
/* Weight tensors for checkers: which = "embed" [vocab,hidden], "final_norm", "lm_head"
 * [vocab,hidden], or per layer "attn_norm", "wqkv" (rows q | k | v), "wo", "ffn_norm",
 * "w_gate_up" (rows interleaved: 2n = gate n, 2n+1 = up n), "w_down", and the layer's KV
 * cache "k_cache" / "v_cache" [n_kv_heads][max_seq][head_dim] (rows < the current position
 * are valid).
 * Projection matrices are stored row-major [out,in], the transpose of export_llama.py's
 * [in,out] (`.T` at :203-217,238): one output's weights are contiguous for the GEMV. */
int shp_llama_weight(shp_llama* lm, int32_t layer, const char* which, void** dptr,
                     uint64_t* elems);
int shp_llama_weight_bytes(shp_llama* lm, double* bytes);

#ifdef __cplusplus
}
#endif

#endif /* SPIRV_HIP_H */
