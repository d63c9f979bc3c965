// TinyLlama-shaped greedy decode with a KV cache: the C ABI of shp_llama_*.
//
// The reference decodes by re-running the whole S=64 HLO graph per token in a fresh
// process (source/xla_hlo/tools/run_llama_spirv.py:194-295): every step re-reads all
// 4.1 GB of weights from disk and recomputes all 64 positions.  Here the weights are
// generated once in HBM, keys and values are cached, and a step is 5 launches per layer —
// fused RMSNorm+QKV GEMV, RoPE+KV-append+attention, Wo GEMV with the residual add, fused
// RMSNorm+gate/up GEMV with SiLU*up, down GEMV with the residual add — plus the final
// RMSNorm+lm_head GEMV and an on-device argmax that feeds the next step.  That step can run
// eagerly or replayed from a hipGraph; the default engine instead runs a whole step or
// decode call as one cooperative launch (kernels_decode_persist.hip).  Nothing returns to
// the host between tokens in either form.
#include <cmath>
#include <vector>

#include "decode.h"
#include "runtime.h"

namespace shp {

struct Llama {
    static constexpr long long kDefaultSpinLimit = 1ll << 22;
    Ctx* ctx = nullptr;
    shp_llama_config cfg{};
    uint64_t seed = 0;
    uint64_t next_id = 1;
    struct Layer {
        float *attn_norm, *wqkv, *wo, *ffn_norm, *w_gu, *w_down;
    };
    std::vector<Layer> layers;
    float *embed = nullptr, *final_norm = nullptr, *lm_head = nullptr;
    float *k_cache = nullptr, *v_cache = nullptr;
    float *x = nullptr, *qkv = nullptr, *att = nullptr, *act = nullptr, *logits = nullptr;
    DecodeState* st = nullptr;
    std::vector<void*> allocs;
    double weight_bytes = 0.0;
    int host_pos = 0;
    int engine = SHP_LLAMA_GRAPH;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipStream_t graph_stream = nullptr;

    // persistent engine
    PersistArgs pa{};
    int p_grid = 0;
    size_t p_lds = 0;
    std::string p_why;
    unsigned long long* bar = nullptr;  // barrier flags
    int* abort_flag = nullptr;
    unsigned long long bar_top = 0;  // barriers completed by all launches so far

    ~Llama() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        for (void* p : allocs) (void)hipFree(p);
    }

    int alloc(float** p, uint64_t elems) {
        SHP_HIP_CHECK(hipMalloc((void**)p, elems * sizeof(float)));
        allocs.push_back(*p);
        return SHP_OK;
    }
    int weight(float** p, uint64_t elems, int kind, float a, float b) {
        int rc = alloc(p, elems);
        if (rc) return rc;
        weight_bytes += (double)elems * 4.0;
        return fill_random(ctx->stream, *p, elems, seed, next_id++, kind, a, b);
    }

    int qkv_rows() const { return (cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim; }

    int enqueue_step() {
        const int H = cfg.hidden, F = cfg.ffn, qd = cfg.n_heads * cfg.head_dim;
        const uint64_t cache_layer = (uint64_t)cfg.n_kv_heads * cfg.max_seq * cfg.head_dim;
        hipStream_t s = ctx->stream;
        int rc = embed_launch(s, embed, H, st, x);
        for (int l = 0; l < cfg.n_layers && !rc; ++l) {
            const Layer& L = layers[l];
            rc = gemv_launch(s, x, L.attn_norm, cfg.rms_eps, L.wqkv, qkv_rows(), H, GEMV_PLAIN,
                             qkv, nullptr);
            if (!rc)
                rc = attention_decode_launch(s, qkv, k_cache + l * cache_layer,
                                             v_cache + l * cache_layer, cfg.n_heads,
                                             cfg.n_kv_heads, cfg.head_dim, cfg.max_seq,
                                             cfg.rope_theta, st, att);
            if (!rc) rc = gemv_launch(s, att, nullptr, 0.0f, L.wo, H, qd, GEMV_PLAIN, x, x);
            if (!rc)
                rc = gemv_launch(s, x, L.ffn_norm, cfg.rms_eps, L.w_gu, 2 * F, H, GEMV_SWIGLU, act,
                                 nullptr);
            if (!rc) rc = gemv_launch(s, act, nullptr, 0.0f, L.w_down, H, F, GEMV_PLAIN, x, x);
        }
        if (!rc)
            rc = gemv_launch(s, x, final_norm, cfg.rms_eps, lm_head, cfg.vocab, H, GEMV_PLAIN,
                             logits, nullptr);
        if (!rc) rc = argmax_advance_launch(s, logits, cfg.vocab, st);
        return rc;
    }

    int check_room(int n) {
        if (host_pos + n > cfg.max_seq)
            return fail(SHP_ERR_SHAPE, "llama: KV cache full (position " +
                                           std::to_string(host_pos + n - 1) + " >= max_seq)");
        if (host_pos + n > 4096) return fail(SHP_ERR_SHAPE, "llama: token log full");
        return SHP_OK;
    }

    // n tokens in one cooperative launch; forced >= 0 feeds that id as the first token.
    // `prof` (optional) receives the phase timestamps (see PersistArgs::prof).
    int persist_run(int n, int forced, unsigned long long* prof = nullptr) {
        int rc = check_room(n);
        if (rc) return rc;
        PersistArgs a = pa;
        a.bar_base = bar_top;
        a.n_tokens = n;
        a.forced_token = forced;
        a.prof = prof;
        rc = persist_launch(ctx->stream, a, p_grid, p_lds);
        if (rc) return rc;
        bar_top += (unsigned long long)n * persist_barriers_per_token(cfg.n_layers);
        // a barrier wait that gave up makes every workgroup exit; report it and re-arm
        int aborted = 0;
        SHP_HIP_CHECK(hipMemcpyAsync(&aborted, abort_flag, sizeof(int), hipMemcpyDeviceToHost,
                                     ctx->stream));
        SHP_HIP_CHECK(hipStreamSynchronize(ctx->stream));
        if (aborted) {
            SHP_HIP_CHECK(hipMemsetAsync(bar, 0,
                                         persist_flag_slots(p_grid) * sizeof(unsigned long long),
                                         ctx->stream));
            SHP_HIP_CHECK(hipMemsetAsync(abort_flag, 0, sizeof(int), ctx->stream));
            // epochs restart at 0: tags written before the abort must not match them
            SHP_HIP_CHECK(hipMemsetAsync(pa.qkv_tag, 0,
                                         (size_t)qkv_rows() * sizeof(unsigned long long),
                                         ctx->stream));
            SHP_HIP_CHECK(hipMemsetAsync(pa.x_tag, 0,
                                         (size_t)cfg.hidden * sizeof(unsigned long long),
                                         ctx->stream));
            SHP_HIP_CHECK(hipStreamSynchronize(ctx->stream));
            bar_top = 0;
            return fail(SHP_ERR_HIP, "llama: persistent decode grid barrier timed out; state "
                                     "is undefined until reset");
        }
        host_pos += n;
        return SHP_OK;
    }

    int step() {
        int rc = check_room(1);
        if (rc) return rc;
        if (engine == SHP_LLAMA_PERSISTENT) return persist_run(1, -1);
        if (engine == SHP_LLAMA_KERNELS) {
            rc = enqueue_step();
        } else {
            if (exec && graph_stream != ctx->stream) {
                (void)hipGraphExecDestroy(exec);
                (void)hipGraphDestroy(graph);
                exec = nullptr;
                graph = nullptr;
            }
            if (!exec) {
                SHP_HIP_CHECK(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
                rc = enqueue_step();
                hipGraph_t g = nullptr;
                hipError_t e = hipStreamEndCapture(ctx->stream, &g);
                if (rc) {
                    if (g) (void)hipGraphDestroy(g);
                    return rc;
                }
                if (e != hipSuccess)
                    return fail(SHP_ERR_HIP, std::string("llama capture: ") + hipGetErrorString(e));
                graph = g;
                SHP_HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
                graph_stream = ctx->stream;
            }
            SHP_HIP_CHECK(hipGraphLaunch(exec, ctx->stream));
            rc = SHP_OK;
        }
        if (!rc) ++host_pos;
        return rc;
    }

    int setup_persistent() {
        pa = PersistArgs{};
        std::vector<PersistLayer> hl;
        for (const Layer& L : layers)
            hl.push_back(PersistLayer{L.attn_norm, L.wqkv, L.wo, L.ffn_norm, L.w_gu, L.w_down});
        PersistLayer* dl = nullptr;
        SHP_HIP_CHECK(hipMalloc((void**)&dl, hl.size() * sizeof(PersistLayer)));
        allocs.push_back(dl);
        SHP_HIP_CHECK(hipMemcpy(dl, hl.data(), hl.size() * sizeof(PersistLayer),
                                hipMemcpyHostToDevice));
        const int qd = cfg.n_heads * cfg.head_dim;
        const uint64_t zrow = (uint64_t)std::max(std::max(cfg.hidden, qd), cfg.ffn);
        float* zero = nullptr;
        int rc = alloc(&zero, zrow);
        if (rc) return rc;
        SHP_HIP_CHECK(hipMemset(zero, 0, zrow * sizeof(float)));
        SHP_HIP_CHECK(hipMalloc((void**)&abort_flag, sizeof(int)));
        allocs.push_back(abort_flag);
        SHP_HIP_CHECK(hipMemset(abort_flag, 0, sizeof(int)));
        pa.layers = dl;
        pa.embed = embed;
        pa.final_norm = final_norm;
        pa.lm_head = lm_head;
        pa.k_cache = k_cache;
        pa.v_cache = v_cache;
        pa.x = x;
        pa.qkv = qkv;
        pa.att = att;
        pa.act = act;
        pa.logits = logits;
        pa.zero_row = zero;
        pa.st = st;
        pa.abort_flag = abort_flag;
        pa.spin_limit = kDefaultSpinLimit;  // ~1 us per poll: a wait gives up after seconds
        pa.spin_start = 0;
        pa.n_layers = cfg.n_layers;
        pa.hidden = cfg.hidden;
        pa.n_heads = cfg.n_heads;
        pa.n_kv = cfg.n_kv_heads;
        pa.ffn = cfg.ffn;
        pa.vocab = cfg.vocab;
        pa.max_seq = cfg.max_seq;
        pa.eps = cfg.rms_eps;
        pa.theta = cfg.rope_theta;
        rc = persist_plan(ctx->device, &pa, &p_grid, &p_lds, &p_why);
        if (rc) return rc;
        if (p_grid <= 0) return SHP_OK;  // unsupported: p_why says why
        ArgmaxCand* cand = nullptr;
        SHP_HIP_CHECK(hipMalloc((void**)&cand, (size_t)p_grid * sizeof(ArgmaxCand)));
        allocs.push_back(cand);
        pa.cand = cand;
        unsigned long long* tag = nullptr;
        const size_t tbytes = (size_t)qkv_rows() * sizeof(unsigned long long);
        SHP_HIP_CHECK(hipMalloc((void**)&tag, tbytes));
        allocs.push_back(tag);
        SHP_HIP_CHECK(hipMemset(tag, 0, tbytes));  // epoch 0: never a live phase's
        pa.qkv_tag = tag;
        unsigned long long* xtag = nullptr;
        const size_t xbytes = (size_t)cfg.hidden * sizeof(unsigned long long);
        SHP_HIP_CHECK(hipMalloc((void**)&xtag, xbytes));
        allocs.push_back(xtag);
        SHP_HIP_CHECK(hipMemset(xtag, 0, xbytes));
        pa.x_tag = xtag;
        const size_t fbytes = persist_flag_slots(p_grid) * sizeof(unsigned long long);
        SHP_HIP_CHECK(hipMalloc((void**)&bar, fbytes));
        allocs.push_back(bar);
        SHP_HIP_CHECK(hipMemset(bar, 0, fbytes));
        pa.flags = bar;
        return SHP_OK;
    }

    int reset() {
        SHP_HIP_CHECK(hipMemsetAsync(st, 0, sizeof(DecodeState), ctx->stream));
        host_pos = 0;
        return SHP_OK;
    }
};

}  // namespace shp

using shp::fail;
using shp::Llama;

extern "C" {

int shp_llama_create(shp_ctx* ctx, const shp_llama_config* cfg, uint64_t seed, shp_llama** out) {
    if (!ctx || !cfg || !out) return fail(SHP_ERR_INVALID, "shp_llama_create: null argument");
    {
        int grc = shp::refuse_while_capturing(reinterpret_cast<shp::Ctx*>(ctx)->stream, "shp_llama_create");
        if (grc) return grc;
    }
    *out = nullptr;
    const shp_llama_config& c = *cfg;
    if (c.n_layers <= 0 || c.hidden <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 ||
        c.head_dim != 64 || c.n_heads % c.n_kv_heads != 0 || c.ffn <= 0 || c.vocab <= 0 ||
        c.max_seq <= 0 || c.max_seq > 4096 || c.hidden % 4 != 0 || c.ffn % 4 != 0 ||
        c.n_heads * c.head_dim % 4 != 0)
        return fail(SHP_ERR_UNSUPPORTED,
                    "shp_llama_create: needs head_dim 64, n_heads % n_kv == 0, hidden/ffn % 4 == 0, "
                    "max_seq <= 4096");
    if ((size_t)std::max(c.hidden, c.ffn) * 4 > 64 * 1024)
        return fail(SHP_ERR_UNSUPPORTED, "shp_llama_create: hidden/ffn too large for LDS staging");
    Llama* lm = new Llama();
    lm->ctx = reinterpret_cast<shp::Ctx*>(ctx);
    lm->cfg = c;
    lm->seed = seed;
    (void)hipSetDevice(lm->ctx->device);
    const uint64_t H = c.hidden, F = c.ffn, qd = (uint64_t)c.n_heads * 64;
    int rc = SHP_OK;
    // random-init weights: matrices and embedding N(0, 0.02); RMSNorm weights 1
    rc = lm->weight(&lm->embed, (uint64_t)c.vocab * H, 1, 0.0f, 0.02f);
    for (int l = 0; l < c.n_layers && !rc; ++l) {
        Llama::Layer L{};
        rc = lm->weight(&L.attn_norm, H, 0, 1.0f, 1.0f);
        if (!rc) rc = lm->weight(&L.wqkv, (uint64_t)lm->qkv_rows() * H, 1, 0.0f, 0.02f);
        if (!rc) rc = lm->weight(&L.wo, H * qd, 1, 0.0f, 0.02f);
        if (!rc) rc = lm->weight(&L.ffn_norm, H, 0, 1.0f, 1.0f);
        if (!rc) rc = lm->weight(&L.w_gu, 2 * F * H, 1, 0.0f, 0.02f);
        if (!rc) rc = lm->weight(&L.w_down, H * F, 1, 0.0f, 0.02f);
        lm->layers.push_back(L);
    }
    if (!rc) rc = lm->weight(&lm->final_norm, H, 0, 1.0f, 1.0f);
    if (!rc) rc = lm->weight(&lm->lm_head, (uint64_t)c.vocab * H, 1, 0.0f, 0.02f);
    const uint64_t cache = (uint64_t)c.n_layers * c.n_kv_heads * c.max_seq * 64;
    if (!rc) rc = lm->alloc(&lm->k_cache, cache);
    if (!rc) rc = lm->alloc(&lm->v_cache, cache);
    if (!rc) rc = lm->alloc(&lm->x, H);
    if (!rc) rc = lm->alloc(&lm->qkv, (uint64_t)lm->qkv_rows());
    if (!rc) rc = lm->alloc(&lm->att, qd);
    if (!rc) rc = lm->alloc(&lm->act, F);
    if (!rc) rc = lm->alloc(&lm->logits, (uint64_t)c.vocab);
    if (!rc) {
        hipError_t e = hipMalloc((void**)&lm->st, sizeof(shp::DecodeState));
        if (e != hipSuccess) rc = fail(SHP_ERR_HIP, "llama state hipMalloc failed");
        else lm->allocs.push_back(lm->st);
    }
    if (!rc) rc = lm->reset();
    if (!rc) rc = lm->setup_persistent();
    if (!rc && lm->p_grid > 0) lm->engine = SHP_LLAMA_PERSISTENT;
    if (!rc) {
        hipError_t e = hipStreamSynchronize(lm->ctx->stream);
        if (e != hipSuccess) rc = fail(SHP_ERR_HIP, hipGetErrorString(e));
    }
    if (rc) {
        delete lm;
        return rc;
    }
    *out = reinterpret_cast<shp_llama*>(lm);
    return SHP_OK;
}

void shp_llama_destroy(shp_llama* p) {
    if (!p) return;
    Llama* lm = reinterpret_cast<Llama*>(p);
    (void)hipStreamSynchronize(lm->ctx->stream);
    delete lm;
}

int shp_llama_reset(shp_llama* p) {
    if (!p) return fail(SHP_ERR_INVALID, "shp_llama_reset: null");
    {
        int grc = shp::refuse_while_capturing(reinterpret_cast<Llama*>(p)->ctx->stream, "shp_llama_reset");
        if (grc) return grc;
    }
    return reinterpret_cast<Llama*>(p)->reset();
}

int shp_llama_step(shp_llama* p, int32_t token) {
    if (!p) return fail(SHP_ERR_INVALID, "shp_llama_step: null");
    {
        int grc = shp::refuse_while_capturing(reinterpret_cast<Llama*>(p)->ctx->stream, "shp_llama_step");
        if (grc) return grc;
    }
    Llama* lm = reinterpret_cast<Llama*>(p);
    if (token < 0 || token >= lm->cfg.vocab) return fail(SHP_ERR_SHAPE, "shp_llama_step: token id");
    if (lm->engine == SHP_LLAMA_PERSISTENT) return lm->persist_run(1, token);
    int rc = shp::set_token_launch(lm->ctx->stream, lm->st, token);
    return rc ? rc : lm->step();
}

int shp_llama_decode(shp_llama* p, int32_t n_steps) {
    if (!p) return fail(SHP_ERR_INVALID, "shp_llama_decode: null");
    {
        int grc = shp::refuse_while_capturing(reinterpret_cast<Llama*>(p)->ctx->stream, "shp_llama_decode");
        if (grc) return grc;
    }
    Llama* lm = reinterpret_cast<Llama*>(p);
    if (n_steps < 0) return fail(SHP_ERR_INVALID, "shp_llama_decode: n_steps < 0");
    if (n_steps == 0) return SHP_OK;
    if (lm->engine == SHP_LLAMA_PERSISTENT) return lm->persist_run(n_steps, -1);
    for (int i = 0; i < n_steps; ++i) {
        int rc = lm->step();
        if (rc) return rc;
    }
    return SHP_OK;
}

int shp_llama_tokens(shp_llama* p, int32_t* out, int32_t cap, int32_t* n_out) {
    if (!p || !n_out) return fail(SHP_ERR_INVALID, "shp_llama_tokens: null");
    {
        int grc = shp::refuse_while_capturing(reinterpret_cast<Llama*>(p)->ctx->stream, "shp_llama_tokens");
        if (grc) return grc;
    }
    Llama* lm = reinterpret_cast<Llama*>(p);
    shp::DecodeState h;
    SHP_HIP_CHECK(hipMemcpyAsync(&h, lm->st, sizeof(h), hipMemcpyDeviceToHost, lm->ctx->stream));
    SHP_HIP_CHECK(hipStreamSynchronize(lm->ctx->stream));
    int n = std::min<int>(h.step, std::min(cap, 4096));
    if (out)
        for (int i = 0; i < n; ++i) out[i] = h.out_tokens[i];
    *n_out = n;
    return SHP_OK;
}

int shp_llama_generate(shp_llama* p, const int32_t* prompt, int32_t n_prompt, int32_t n_new,
                       int32_t* out_tokens, int32_t* n_out) {
    if (!p || (!prompt && n_prompt) || n_prompt <= 0 || n_new < 0 || !n_out)
        return fail(SHP_ERR_INVALID, "shp_llama_generate: bad arguments");
    {
        int grc = shp::refuse_while_capturing(reinterpret_cast<Llama*>(p)->ctx->stream, "shp_llama_generate");
        if (grc) return grc;
    }
    Llama* lm = reinterpret_cast<Llama*>(p);
    if (n_prompt + n_new - 1 > lm->cfg.max_seq)
        return fail(SHP_ERR_SHAPE, "shp_llama_generate: prompt + new tokens exceed max_seq");
    int rc = lm->reset();
    for (int i = 0; i < n_prompt && !rc; ++i) rc = shp_llama_step(p, prompt[i]);
    if (!rc && n_new > 1) rc = shp_llama_decode(p, n_new - 1);
    if (rc) return rc;
    std::vector<int32_t> all(4096);
    int32_t n = 0;
    rc = shp_llama_tokens(p, all.data(), 4096, &n);
    if (rc) return rc;
    // generated token t is the argmax after position n_prompt - 1 + t; like
    // run_llama_spirv.py:292-294 the loop ends at EOS (2) or PAD (0), which is not kept
    int w = 0;
    for (int t = 0; t < n_new && n_prompt - 1 + t < n; ++t) {
        int tok = all[n_prompt - 1 + t];
        if (tok == 2 || tok == 0) break;
        if (out_tokens) out_tokens[w] = tok;
        ++w;
    }
    *n_out = w;
    return SHP_OK;
}

int shp_llama_use_graph(shp_llama* p, int enable) {
    if (!p) return fail(SHP_ERR_INVALID, "shp_llama_use_graph: null");
    reinterpret_cast<Llama*>(p)->engine = enable ? SHP_LLAMA_GRAPH : SHP_LLAMA_KERNELS;
    return SHP_OK;
}

int shp_llama_set_engine(shp_llama* p, int engine) {
    if (!p) return fail(SHP_ERR_INVALID, "shp_llama_set_engine: null");
    Llama* lm = reinterpret_cast<Llama*>(p);
    if (engine != SHP_LLAMA_KERNELS && engine != SHP_LLAMA_GRAPH && engine != SHP_LLAMA_PERSISTENT)
        return fail(SHP_ERR_INVALID, "shp_llama_set_engine: unknown engine");
    if (engine == SHP_LLAMA_PERSISTENT && lm->p_grid <= 0)
        return fail(SHP_ERR_UNSUPPORTED, "shp_llama_set_engine: persistent engine unavailable: " +
                                             lm->p_why);
    lm->engine = engine;
    return SHP_OK;
}

// Internal profiling hook (not part of include/spirv_hip.h): decodes n tokens with the
// persistent engine and copies the phase timestamps to host_out, which must hold
// n * (5 * n_layers + 1) * 16 * grid values; *grid receives the workgroup count.
int shp_llama_profile_persistent(shp_llama* p, int32_t n, unsigned long long* host_out,
                                 uint64_t cap, int32_t* grid) {
    if (!p || !host_out || !grid || n <= 0)
        return fail(SHP_ERR_INVALID, "shp_llama_profile_persistent: bad arguments");
    {
        int grc = shp::refuse_while_capturing(reinterpret_cast<Llama*>(p)->ctx->stream, "shp_llama_profile_persistent");
        if (grc) return grc;
    }
    Llama* lm = reinterpret_cast<Llama*>(p);
    if (lm->p_grid <= 0) return fail(SHP_ERR_UNSUPPORTED, "persistent engine unavailable");
    const uint64_t need = (uint64_t)n * shp::persist_barriers_per_token(lm->cfg.n_layers) * 16 *
                          (uint64_t)lm->p_grid;
    if (cap < need) return fail(SHP_ERR_INVALID, "shp_llama_profile_persistent: buffer too small");
    unsigned long long* d = nullptr;
    SHP_HIP_CHECK(hipMalloc((void**)&d, need * sizeof(unsigned long long)));
    int rc = lm->persist_run(n, -1, d);
    if (!rc) {
        hipError_t e = hipMemcpy(host_out, d, need * sizeof(unsigned long long),
                                 hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = fail(SHP_ERR_HIP, hipGetErrorString(e));
    }
    (void)hipFree(d);
    *grid = lm->p_grid;
    return rc;
}

int shp_llama_set_wait_limit(shp_llama* p, int64_t polls) {
    if (!p) return fail(SHP_ERR_INVALID, "shp_llama_set_wait_limit: null");
    Llama* lm = reinterpret_cast<Llama*>(p);
    if (polls < 0) polls = shp::Llama::kDefaultSpinLimit;
    lm->pa.spin_limit = polls;
    // below one check interval the first missed poll already checks, so the limit holds
    lm->pa.spin_start = polls < 128 ? 127 : 0;
    return SHP_OK;
}

int shp_llama_engine(shp_llama* p, int* engine) {
    if (!p || !engine) return fail(SHP_ERR_INVALID, "shp_llama_engine: null");
    *engine = reinterpret_cast<Llama*>(p)->engine;
    return SHP_OK;
}

int shp_llama_logits(shp_llama* p, void** dptr, uint64_t* elems) {
    if (!p || !dptr || !elems) return fail(SHP_ERR_INVALID, "shp_llama_logits: null");
    Llama* lm = reinterpret_cast<Llama*>(p);
    *dptr = lm->logits;
    *elems = (uint64_t)lm->cfg.vocab;
    return SHP_OK;
}

int shp_llama_weight(shp_llama* p, int32_t layer, const char* which, void** dptr,
                     uint64_t* elems) {
    if (!p || !which || !dptr || !elems) return fail(SHP_ERR_INVALID, "shp_llama_weight: null");
    Llama* lm = reinterpret_cast<Llama*>(p);
    const shp_llama_config& c = lm->cfg;
    const uint64_t H = c.hidden, F = c.ffn, qd = (uint64_t)c.n_heads * 64;
    std::string w = which;
    if (w == "embed") { *dptr = lm->embed; *elems = (uint64_t)c.vocab * H; return SHP_OK; }
    if (w == "final_norm") { *dptr = lm->final_norm; *elems = H; return SHP_OK; }
    if (w == "lm_head") { *dptr = lm->lm_head; *elems = (uint64_t)c.vocab * H; return SHP_OK; }
    if (layer < 0 || layer >= c.n_layers) return fail(SHP_ERR_INVALID, "shp_llama_weight: layer");
    const Llama::Layer& L = lm->layers[layer];
    if (w == "attn_norm") { *dptr = L.attn_norm; *elems = H; return SHP_OK; }
    if (w == "wqkv") { *dptr = L.wqkv; *elems = (uint64_t)lm->qkv_rows() * H; return SHP_OK; }
    if (w == "wo") { *dptr = L.wo; *elems = H * qd; return SHP_OK; }
    if (w == "ffn_norm") { *dptr = L.ffn_norm; *elems = H; return SHP_OK; }
    if (w == "w_gate_up") { *dptr = L.w_gu; *elems = 2 * F * H; return SHP_OK; }
    if (w == "w_down") { *dptr = L.w_down; *elems = H * F; return SHP_OK; }
    const uint64_t cache_layer = (uint64_t)c.n_kv_heads * c.max_seq * c.head_dim;
    if (w == "k_cache") { *dptr = lm->k_cache + layer * cache_layer; *elems = cache_layer; return SHP_OK; }
    if (w == "v_cache") { *dptr = lm->v_cache + layer * cache_layer; *elems = cache_layer; return SHP_OK; }
    return fail(SHP_ERR_INVALID, "shp_llama_weight: unknown tensor '" + w + "'");
}

int shp_llama_weight_bytes(shp_llama* p, double* bytes) {
    if (!p || !bytes) return fail(SHP_ERR_INVALID, "shp_llama_weight_bytes: null");
    *bytes = reinterpret_cast<Llama*>(p)->weight_bytes;
    return SHP_OK;
}

}  // extern "C"
