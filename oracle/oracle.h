/*
 * oracle.h — CPU restatement of agkdc1/SPIRV_INFERENCE's operator kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP kernels of
 * spirv_inference_amd: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load it.  The product library never links, loads or falls back to it.
 *
 * Every kernel follows the loop order and arithmetic of the reference GLSL source it
 * cites (one output element per iteration, the reference's serial inner loops, fp32
 * accumulation).  The library is compiled with -ffp-contract=off so that mul+add pairs
 * are not fused, which lets it reproduce the reference's golden vectors bit for bit.
 * Output elements are independent, so the outer loops are spread over OpenMP threads
 * without changing any result.
 */
#ifndef SPIRV_ORACLE_H
#define SPIRV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Runs `name` with the reference's push vector on host buffers.  The epilogue (bias
 * indexed by output channel, residual with the output's layout, activation code as in
 * spirv_hip.h) is applied after the base kernel exactly as the HIP kernels define it;
 * kernels with a packed bias tail (conv2d, conv2d_nhwc, depthwise_*, fully_connected)
 * ignore `bias`.  Returns 0, or a negative code with orc_last_error() set. */
int orc_run_kernel(const char* name, const float* in0, size_t n0, const float* in1, size_t n1,
                   float* out, size_t n_out, const int32_t* push, size_t n_push,
                   const float* bias, const float* residual, int32_t act, float alpha);
const char* orc_last_error(void);
int orc_kernel_count(void);
const char* orc_kernel_name(int index);
void orc_set_threads(int n);

/* Host-side helpers of the TFLite scheduler (source/tflite_loader/src/scheduler.rs). */
void orc_same_padding(int same, int ih, int iw, int oh, int ow, int kh, int kw, int sh, int sw,
                      int32_t* pad_top, int32_t* pad_left);                    /* :1597-1614 */
void orc_pack_conv_weight(const float* ohwi, const float* bias, int oc, int kh, int kw, int ic,
                          float* out);                                         /* :1327-1362 */
void orc_pack_depthwise_weight(const float* hwc, const float* bias, int kh, int kw, int c,
                               float* out);                                    /* :1364-1400 */
void orc_pack_fc_weight(const float* w, const float* bias, int out_size, int in_size,
                        float* out);                                           /* :1402-1436 */
/* top1 of scheduler.rs:1637-1648: max_by(total_cmp) keeps the LAST maximum; a 1001-class
 * head is offset by one (imagenet_class_offset :1671-1677).  Returns the class. */
int orc_top1_reference(const float* v, size_t n, float* confidence);
/* numpy argmax semantics (run_llama_spirv.py:252-254): FIRST maximum. */
int orc_argmax_first(const float* v, size_t n);
/* tensor::compare (source/tflite_loader/src/tensor.rs:28-54). */
void orc_compare(const float* actual, size_t na, const float* expected, size_t ne, float eps,
                 uint64_t* mismatch, float* max_abs, float* max_rel);

/* Closed-form generators of the reference's own fixtures. */
/* tests/parity_test/generate_fixtures.py:67-82 — which: 0 relu_input(4096), 1 softmax_input(128),
 * 2 batchnorm_input(256), 3 batchnorm_params(5), 4 conv1d_input(1024), 5 conv1d_filter(6144) */
int orc_parity_fixture(int which, float* out, size_t n);
/* source/inference_poc/src/fixture.rs:28-72 — which: 0 input(64), 1 conv_weight(12),
 * 2 bn_param(16), 3 fc_param(250) */
int orc_poc_fixture(int which, float* out, size_t n);

/* TinyLlama-shaped decoder (export_llama.py:269-375) for one sequence.
 * Weight layout: wqkv rows = [q (nh*64) | k (nkv*64) | v (nkv*64)] x hidden;
 * wo [hidden][nh*64]; w_gu rows interleaved (2n = gate n, 2n+1 = up n) x hidden;
 * w_down [hidden][ffn]; lm_head [vocab][hidden]; embed [vocab][hidden].
 * layers[l*6 + {0..5}] = {attn_norm, wqkv, wo, ffn_norm, w_gu, w_down}. */
typedef struct orc_llama_cfg {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_seq;
    float rms_eps, rope_theta;
} orc_llama_cfg;

/* One token at position `pos` with a KV cache ([layer][kv][max_seq][64] each);
 * writes logits[vocab]. */
int orc_llama_step(const orc_llama_cfg* cfg, const float* const* layers, const float* embed,
                   const float* final_norm, const float* lm_head, float* k_cache,
                   float* v_cache, int32_t pos, int32_t token, float* logits);
/* Full recompute of S positions with the causal mask (the reference's algorithm:
 * run_llama_spirv.py:198-206 + export_llama.py); writes logits[S][vocab]. */
int orc_llama_full(const orc_llama_cfg* cfg, const float* const* layers, const float* embed,
                   const float* final_norm, const float* lm_head, const int32_t* tokens,
                   int32_t S, float* logits);

#ifdef __cplusplus
}
#endif

#endif
