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

// ---- persistent decode: every token of a decode call in one cooperative launch ----------
struct PersistLayer {
    const float *attn_norm, *wqkv, *wo, *ffn_norm, *w_gu, *w_down;
};

struct ArgmaxCand {
    float value;
    int32_t index;
};

struct PersistArgs {
    const PersistLayer* layers;  // device array [n_layers]
    const float* embed;
    const float* final_norm;
    const float* lm_head;
    float* k_cache;
    float* v_cache;
    float* x;       // [hidden] residual stream
    float* qkv;     // [(n_heads + 2 n_kv) * 64]
    // [(n_heads + 2 n_kv) * 64] the qkv rows as tagged words, (phase epoch << 32) | float bits:
    // attention waits for its head's words instead of a grid barrier
    unsigned long long* qkv_tag;
    unsigned long long* x_tag;  // [hidden] x as tagged words (the phases that write x tag it)
    float* att;     // [n_heads * 64] attention output
    float* act;     // [ffn] silu(gate) * up
    float* logits;  // [vocab]
    ArgmaxCand* cand;  // [grid] per-workgroup argmax of its logits rows
    const float* zero_row;  // >= max(hidden, n_heads * 64, ffn) zeros (padding-row loads)
    DecodeState* st;
    unsigned long long* flags;  // barrier epoch flag of workgroup b at flags[8 * b] (monotonic)
    int* abort_flag;            // set when a barrier wait exceeds spin_limit
    unsigned long long bar_base;  // barriers completed before this launch (epoch base)
    long long spin_limit;         // polls of the counter before a wait gives up
    long long spin_start;         // poll count a wait starts from (0, or 127: check at once)
    int n_layers, hidden, n_heads, n_kv, ffn, vocab, max_seq;
    float eps, theta;
    int n_tokens;      // tokens decoded by this launch
    int forced_token;  // >= 0: the first token fed (a prompt id); < 0: state.token
    // Optional phase timestamps (100 MHz wall clock), null when not profiling:
    // prof[((token * barriers_per_token + k) * 16 + slot) * grid + workgroup], slot 0 arrival
    // at barrier k, 1 its pass; in the attention phase 2 = first tile staged; in the gate/up
    // phase 3 = vector normalised, 4 + c = chunk c done.
    unsigned long long* prof;
};

// Grid barriers one token costs: five per layer and one before the global argmax.
inline int persist_barriers_per_token(int n_layers) { return 5 * n_layers + 1; }
// unsigned long long slots of the barrier flags of a grid of `grid` workgroups.
inline int persist_flag_slots(int grid) { return 8 * grid; }

// Checks that the persistent kernel supports this shape and that the device can keep one
// workgroup per CU resident.  On success *grid > 0 and *lds is the dynamic LDS size;
// otherwise *grid = 0 and *why gives the reason.
int persist_plan(int device, PersistArgs* a, int* grid, size_t* lds, std::string* why);

// One cooperative launch decoding a.n_tokens tokens.
int persist_launch(hipStream_t s, const PersistArgs& a, int grid, size_t lds);

}  // namespace shp
