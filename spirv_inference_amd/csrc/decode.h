// Batch-1 decode kernels used by the TinyLlama-shaped engine (llama.cpp) and exposed in
// part through the registry (gemv_nt, argmax_rows).
#pragma once

#include "common.h"

namespace shp {

// Device-resident decode state: the token to feed, its position, and the generated ids.
struct DecodeState {
    int32_t token;
    int32_t pos;
    int32_t step;      // number of argmax results written to out_tokens
    int32_t pad;
    int32_t out_tokens[4096];
};

enum GemvMode {
    GEMV_PLAIN = 0,     // y[n] = dot(v, W[n])              (+ residual[n])
    GEMV_SWIGLU = 1,    // rows 2n, 2n+1: y[n] = silu(dot(v,W[2n])) * dot(v,W[2n+1])
};

// y = W v with W row-major [rows][K]; v = x, or rmsnorm(x) * norm_w when norm_w != null.
// `residual` (may alias y) is added per output row.  Work is spread over at most
// `max_groups` workgroups of four wavefronts.
int gemv_launch(hipStream_t s, const float* x, const float* norm_w, float eps, const float* w,
                int rows, int K, int mode, float* y, const float* residual);

// Copies embed[state.token] into x.
int embed_launch(hipStream_t s, const float* embed, int hidden, const DecodeState* st, float* x);

// RoPE on q and k at state.pos, appends k and v to the caches, and writes the attention
// output for every query head (causal over positions 0..pos).
int attention_decode_launch(hipStream_t s, const float* qkv, float* k_cache, float* v_cache,
                            int n_heads, int n_kv, int head_dim, int max_seq, float theta,
                            const DecodeState* st, float* out);

// state.token = token (a kernel argument, so no host buffer is involved).
int set_token_launch(hipStream_t s, DecodeState* st, int32_t token);

// Greedy argmax of logits (lowest index on ties) into state.token and
// state.out_tokens[state.step]; advances pos and step.
int argmax_advance_launch(hipStream_t s, const float* logits, int n, DecodeState* st);

}  // namespace shp
