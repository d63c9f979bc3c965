/*
 * oracle.c — CPU restatement of the reference's operator kernels (TEST INFRASTRUCTURE).
 *
 * Each function cites the GLSL kernel (kernels/<op>/glsl/<op>.comp) or host routine it
 * restates.  Per output element the arithmetic and summation order are the reference's;
 * where a loop nest is reordered for speed (conv, dot, fully_connected), only independent
 * outputs are interleaved — every accumulator still sees its terms in the reference order,
 * so results are identical to the naive per-output loop.
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static __thread char g_err[256];

static int orc_fail(int code, const char* msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return code;
}

const char* orc_last_error(void) { return g_err; }

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

enum { ACT_NONE = 0, ACT_RELU, ACT_RELU6, ACT_LEAKY, ACT_SIGMOID, ACT_TANH, ACT_SILU, ACT_GELU };

/* erfc as the XLA expansion spelled out in source/xla_hlo/fixtures/bert_base.stablehlo.txt:59-144 */
static float erfc_xla(float z) {
    float az = fabsf(z);
    if (az > 1.0f) {
        float z2 = z * z;
        float e = expf(-z2);
        float q = 1.0f / z2;
        float p = 0.102081165f * q;
        p = p + 0.429206669f;
        p = p * q;
        p = p + 0.323790789f;
        p = p * q;
        p = p + 0.053971976f;
        float d = 0.0172516778f * q;
        d = d + 0.391371638f;
        d = d * q;
        d = d + 1.0f;
        d = d * q;
        d = d + 0.621732414f;
        d = d * q;
        d = d + 0.0956628621f;
        float den = fminf(az, 10.06f) * d;
        float r = e * (p / den);
        return z < 0.0f ? 2.0f - r : r;
    }
    float w = z * z;
    float s = 0.000561802299f * w;
    s = s + -0.00491381669f;
    s = s * w;
    s = s + 0.0267075151f;
    s = s * w;
    s = s + -0.112800106f;
    s = s * w;
    s = s + 0.376122952f;
    s = s * w;
    s = s + -1.12837911f;
    return z * s + 1.0f;
}

static float act_f(float x, int act, float alpha) {
    switch (act) {
        case ACT_RELU: return x > 0.0f ? x : 0.0f;                 /* relu.comp: max(x, 0) */
        case ACT_RELU6: return fminf(fmaxf(x, 0.0f), 6.0f);        /* relu6.comp */
        case ACT_LEAKY: return fmaxf(alpha * x, x);                /* leaky_relu.comp:17 */
        case ACT_SIGMOID: return 1.0f / (1.0f + expf(-x));         /* sigmoid.comp */
        case ACT_TANH: {                                           /* tanh.comp:15-18 */
            float c = fminf(fmaxf(x, -20.0f), 20.0f);
            float ep = expf(c), en = expf(-c);
            return (ep - en) / (ep + en);
        }
        case ACT_SILU: return x * (1.0f / (1.0f + expf(-x)));      /* export_llama.py:298-299 */
        case ACT_GELU: {                                           /* bert_base.stablehlo.txt */
            float hx = 0.5f * x;
            return hx * erfc_xla(-x * 0.707106769f);
        }
        default: return x;
    }
}

/* out[i] = act(out[i] + bias[chan(i)] + residual[i]) */
static void epilogue(float* out, size_t n, size_t channels, const float* bias,
                     const float* residual, int act, float alpha) {
    if (!bias && !residual && act == ACT_NONE) return;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        float v = out[i];
        if (bias) v = v + bias[channels ? i % channels : i];
        if (residual) v = v + residual[i];
        out[i] = act_f(v, act, alpha);
    }
}

static float bits_to_f32(int32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}

#define NEED(n)                                                          \
    do {                                                                 \
        if ((int)n_push < (n)) return orc_fail(-3, "push vector too short"); \
    } while (0)
#define TOTAL(t)                                                                     \
    do {                                                                             \
        if ((int64_t)(t) != (int64_t)n_out) return orc_fail(-4, "total != n_out");    \
    } while (0)

/* ---- elementwise: kernels/<op>/glsl/<op>.comp (one output per invocation) ------------- */
static float un_op(const char* name, float x, float alpha, int* ok) {
    *ok = 1;
    if (!strcmp(name, "abs")) return fabsf(x);
    if (!strcmp(name, "exp")) return expf(x);
    if (!strcmp(name, "log")) return logf(x);
    if (!strcmp(name, "neg")) return -x;
    if (!strcmp(name, "sqrt")) return sqrtf(x);
    if (!strcmp(name, "rsqrt")) return 1.0f / sqrtf(x);  /* inversesqrt; engine.rs:64-68 */
    if (!strcmp(name, "sigmoid") || !strcmp(name, "logistic")) return act_f(x, ACT_SIGMOID, 0);
    if (!strcmp(name, "tanh")) return act_f(x, ACT_TANH, 0);
    if (!strcmp(name, "relu")) return act_f(x, ACT_RELU, 0);
    if (!strcmp(name, "relu6")) return act_f(x, ACT_RELU6, 0);
    if (!strcmp(name, "sine")) return sinf(x);
    if (!strcmp(name, "reshape")) return x;
    if (!strcmp(name, "leaky_relu")) return fmaxf(alpha * x, x);
    if (!strcmp(name, "silu")) return act_f(x, ACT_SILU, 0);
    if (!strcmp(name, "gelu_erf")) return act_f(x, ACT_GELU, 0);
    if (!strcmp(name, "cosine")) return cosf(x);
    if (!strcmp(name, "floor")) return floorf(x);
    if (!strcmp(name, "ceil")) return ceilf(x);
    *ok = 0;
    return 0.0f;
}

static int bin_code(const char* name) {
    static const char* names[] = {"add", "sub", "mul", "div", "pow", "min", "max"};
    for (int i = 0; i < 7; ++i)
        if (!strcmp(name, names[i])) return i;
    return -1;
}

static float bin_op(int op, float a, float b) {
    switch (op) {
        case 0: return a + b;
        case 1: return a - b;
        case 2: return a * b;
        case 3: return a / b;
        case 4: return powf(a, b);
        case 5: return fminf(a, b);
        case 6: return fmaxf(a, b);
        default: return fmodf(a, b);
    }
}

/* ---- hlo_conv_nhwc_hwio.comp:25-49 — acc = 0; ky -> kx -> ic ---------------------------- */
static int k_hlo_conv(const float* in, const float* w, float* out, const int32_t* q) {
    int n = q[0], ih = q[1], iw = q[2], ic = q[3], kh = q[4], kw = q[5], oc = q[6], oh = q[7],
        ow = q[8], sh = q[9], sw = q[10], pt = q[11], pl = q[12];
    int64_t pixels = (int64_t)n * oh * ow;
#pragma omp parallel
    {
        float* acc = (float*)malloc(sizeof(float) * (size_t)oc);
#pragma omp for schedule(static)
        for (int64_t p = 0; p < pixels; ++p) {
            int x = (int)(p % ow), y = (int)((p / ow) % oh), b = (int)(p / ((int64_t)ow * oh));
            for (int c = 0; c < oc; ++c) acc[c] = 0.0f;
            for (int ky = 0; ky < kh; ++ky) {
                int iy = y * sh + ky - pt;
                if (iy < 0 || iy >= ih) continue;
                for (int kx = 0; kx < kw; ++kx) {
                    int ix = x * sw + kx - pl;
                    if (ix < 0 || ix >= iw) continue;
                    const float* ip = in + (((int64_t)b * ih + iy) * iw + ix) * ic;
                    const float* wp = w + ((int64_t)ky * kw + kx) * ic * oc;
                    for (int c = 0; c < ic; ++c) {
                        float v = ip[c];
                        const float* wr = wp + (int64_t)c * oc;
                        for (int o = 0; o < oc; ++o) acc[o] = acc[o] + v * wr[o];
                    }
                }
            }
            memcpy(out + p * oc, acc, sizeof(float) * (size_t)oc);
        }
        free(acc);
    }
    return 0;
}

/* ---- conv2d.comp:26-50 — acc = bias; ic -> kh -> kw; NCHW in/out, OIHW + bias tail.
 * nhwc=1 restates the same loop on NHWC activations with OHWI weights (conv2d_nhwc). ---- */
static int k_conv2d(const float* in, const float* w, float* out, const int32_t* q, int nhwc) {
    int n = q[0], ic = q[1], ih = q[2], iw = q[3], oc = q[4], oh = q[5], ow = q[6], kh = q[7],
        kw = q[8], sh = q[9], sw = q[10], pt = q[12], pl = q[13];
    int64_t K = (int64_t)ic * kh * kw;
    const float* bias = w + (int64_t)oc * K;
    /* weights transposed to [ic][kh][kw][oc] so the oc loop is contiguous */
    float* wt = (float*)malloc(sizeof(float) * (size_t)(K * oc));
    for (int o = 0; o < oc; ++o)
        for (int c = 0; c < ic; ++c)
            for (int y = 0; y < kh; ++y)
                for (int x = 0; x < kw; ++x) {
                    int64_t src = nhwc ? (((int64_t)o * kh + y) * kw + x) * ic + c
                                       : (((int64_t)o * ic + c) * kh + y) * kw + x;
                    wt[(((int64_t)c * kh + y) * kw + x) * oc + o] = w[src];
                }
    int64_t pixels = (int64_t)n * oh * ow;
#pragma omp parallel
    {
        float* acc = (float*)malloc(sizeof(float) * (size_t)oc);
#pragma omp for schedule(static)
        for (int64_t p = 0; p < pixels; ++p) {
            int x = (int)(p % ow), y = (int)((p / ow) % oh), b = (int)(p / ((int64_t)ow * oh));
            for (int o = 0; o < oc; ++o) acc[o] = bias[o];
            for (int c = 0; c < ic; ++c)
                for (int ky = 0; ky < kh; ++ky) {
                    int iy = y * sh + ky - pt;
                    if (iy < 0 || iy >= ih) continue;
                    for (int kx = 0; kx < kw; ++kx) {
                        int ix = x * sw + kx - pl;
                        if (ix < 0 || ix >= iw) continue;
                        float v = nhwc ? in[(((int64_t)b * ih + iy) * iw + ix) * ic + c]
                                       : in[(((int64_t)b * ic + c) * ih + iy) * iw + ix];
                        const float* wr = wt + (((int64_t)c * kh + ky) * kw + kx) * oc;
                        for (int o = 0; o < oc; ++o) acc[o] = acc[o] + v * wr[o];
                    }
                }
            for (int o = 0; o < oc; ++o) {
                if (nhwc)
                    out[p * oc + o] = acc[o];
                else
                    out[(((int64_t)b * oc + o) * oh + y) * ow + x] = acc[o];
            }
        }
        free(acc);
    }
    free(wt);
    return 0;
}

/* ---- depthwise_conv2d.comp:27-49 — acc = bias[c]; kh -> kw (NCHW, [C,KH,KW] + bias).
 * nhwc=1: the same loop on NHWC activations with TFLite's [KH,KW,C] + bias layout. ---- */
static int k_depthwise(const float* in, const float* w, float* out, const int32_t* q, int nhwc) {
    int n = q[0], c = q[1], ih = q[2], iw = q[3], oh = q[4], ow = q[5], kh = q[6], kw = q[7],
        sh = q[8], sw = q[9], pt = q[11], pl = q[12], dh = q[13], dw = q[14];
    int64_t total = (int64_t)n * c * oh * ow;
    const float* bias = w + (int64_t)c * kh * kw;
#pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        int x, y, ch, b;
        if (nhwc) {
            ch = (int)(idx % c);
            x = (int)((idx / c) % ow);
            y = (int)((idx / ((int64_t)c * ow)) % oh);
            b = (int)(idx / ((int64_t)c * ow * oh));
        } else {
            x = (int)(idx % ow);
            y = (int)((idx / ow) % oh);
            ch = (int)((idx / ((int64_t)ow * oh)) % c);
            b = (int)(idx / ((int64_t)ow * oh * c));
        }
        float acc = bias[ch];
        for (int ky = 0; ky < kh; ++ky) {
            int iy = y * sh + ky * dh - pt;
            if (iy < 0 || iy >= ih) continue;
            for (int kx = 0; kx < kw; ++kx) {
                int ix = x * sw + kx * dw - pl;
                if (ix < 0 || ix >= iw) continue;
                float v, wv;
                if (nhwc) {
                    v = in[(((int64_t)b * ih + iy) * iw + ix) * c + ch];
                    wv = w[((int64_t)ky * kw + kx) * c + ch];
                } else {
                    v = in[(((int64_t)b * c + ch) * ih + iy) * iw + ix];
                    wv = w[((int64_t)ch * kh + ky) * kw + kx];
                }
                acc = acc + v * wv;
            }
        }
        out[idx] = acc;
    }
    return 0;
}

/* ---- fully_connected.comp:15-28 — acc = bias[o]; i ascending; W [out][in] + bias ---- */
static int k_fully_connected(const float* in, const float* w, float* out, const int32_t* q) {
    int batches = q[0], K = q[1], N = q[2];
    const float* bias = w + (int64_t)N * K;
    float* wt = (float*)malloc(sizeof(float) * (size_t)K * N);
    for (int o = 0; o < N; ++o)
        for (int i = 0; i < K; ++i) wt[(int64_t)i * N + o] = w[(int64_t)o * K + i];
#pragma omp parallel for schedule(static)
    for (int b = 0; b < batches; ++b) {
        float* acc = out + (int64_t)b * N;
        for (int o = 0; o < N; ++o) acc[o] = bias[o];
        for (int i = 0; i < K; ++i) {
            float v = in[(int64_t)b * K + i];
            const float* wr = wt + (int64_t)i * N;
            for (int o = 0; o < N; ++o) acc[o] = acc[o] + v * wr[o];
        }
    }
    free(wt);
    return 0;
}

/* ---- dot with one contracting dim and strided batch (compiler.rs dot_general
 * :1829-1877; hlo_dot_batched.comp:19-38 and hlo_dot_rank2.comp:15-26 are special
 * cases): acc = 0; k ascending. ---------------------------------------------------------- */
static void dot_strided(int bo_n, int bi_n, int M, int N, int K, const float* A, int64_t sao,
                        int64_t sai, int64_t sam, int64_t sak, const float* B, int64_t sbo,
                        int64_t sbi, int64_t sbk, int64_t sbn, float* C, int64_t sco, int64_t sci,
                        int64_t scm, int64_t scn, const float* bias, const float* residual,
                        int act, float alpha) {
    int64_t rows = (int64_t)bo_n * bi_n * M;
#pragma omp parallel
    {
        float* acc = (float*)malloc(sizeof(float) * (size_t)N);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            int m = (int)(r % M);
            int64_t bz = r / M;
            int bo = (int)(bz / bi_n), bi = (int)(bz % bi_n);
            const float* a = A + bo * sao + bi * sai + m * sam;
            const float* b = B + bo * sbo + bi * sbi;
            for (int n = 0; n < N; ++n) acc[n] = 0.0f;
            for (int k = 0; k < K; ++k) {
                float av = a[k * sak];
                const float* br = b + k * sbk;
                if (sbn == 1)
                    for (int n = 0; n < N; ++n) acc[n] = acc[n] + av * br[n];
                else
                    for (int n = 0; n < N; ++n) acc[n] = acc[n] + av * br[n * sbn];
            }
            float* c = C + bo * sco + bi * sci + m * scm;
            for (int n = 0; n < N; ++n) {
                float v = acc[n];
                if (bias) v = v + bias[n];
                if (residual) v = v + residual[(c - C) + n * scn];
                c[n * scn] = act_f(v, act, alpha);
            }
        }
        free(acc);
    }
}

/* ---- hlo_reduce_rank4.comp:44-79 ----------------------------------------------------- */
static int k_reduce_rank4(const float* in, float* out, const int32_t* q, size_t n_out) {
    int rank = q[0];
    int d[4] = {q[1], q[2], q[3], q[4]}, od[4] = {q[5], q[6], q[7], q[8]};
    int r[4] = {q[9], q[10], q[11], q[12]};
    int kind = q[13];
#pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < (int64_t)n_out; ++idx) {
        int oc[4] = {0, 0, 0, 0};
        int64_t tmp = idx;
        for (int a = rank - 1; a >= 0; --a) {
            if (r[a] == 0) {
                int dim = od[a] > 1 ? od[a] : 1;
                oc[a] = (int)(tmp % dim);
                tmp /= dim;
            }
        }
        float acc = kind == 1 ? -3.4028234663852886e+38f : 0.0f;
        for (int a0 = 0; a0 < (r[0] ? d[0] : 1); ++a0)
            for (int a1 = 0; a1 < (r[1] ? d[1] : 1); ++a1)
                for (int a2 = 0; a2 < (r[2] ? d[2] : 1); ++a2)
                    for (int a3 = 0; a3 < (r[3] ? d[3] : 1); ++a3) {
                        int c0 = r[0] ? a0 : oc[0], c1 = r[1] ? a1 : oc[1];
                        int c2 = r[2] ? a2 : oc[2], c3 = r[3] ? a3 : oc[3];
                        float v = in[(((int64_t)c0 * d[1] + c1) * d[2] + c2) * d[3] + c3];
                        acc = kind == 1 ? fmaxf(acc, v) : acc + v;
                    }
        out[idx] = acc;
    }
    return 0;
}

/* ---- hlo_reduce_window_rank4.comp:25-49 (NHWC) ------------------------------------------ */
static int k_reduce_window(const float* in, float* out, const int32_t* q, size_t n_out) {
    int ih = q[1], iw = q[2], c = q[3], oh = q[4], ow = q[5], wh = q[6], ww = q[7], sh = q[8],
        sw = q[9], pt = q[10], pl = q[11], kind = q[12];
#pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < (int64_t)n_out; ++idx) {
        int ch = (int)(idx % c), ox = (int)((idx / c) % ow), oy = (int)((idx / ((int64_t)c * ow)) % oh);
        int b = (int)(idx / ((int64_t)c * ow * oh));
        float acc = kind == 1 ? -3.4028234663852886e+38f : 0.0f;
        for (int ky = 0; ky < wh; ++ky) {
            int iy = oy * sh + ky - pt;
            if (iy < 0 || iy >= ih) continue;
            for (int kx = 0; kx < ww; ++kx) {
                int ix = ox * sw + kx - pl;
                if (ix < 0 || ix >= iw) continue;
                float v = in[(((int64_t)b * ih + iy) * iw + ix) * c + ch];
                acc = kind == 1 ? fmaxf(acc, v) : acc + v;
            }
        }
        out[idx] = acc;
    }
    return 0;
}

/* ---- max_pool2d.comp:25-44 (NCHW) ---------------------------------------------------- */
static int k_max_pool(const float* in, float* out, const int32_t* q, size_t n_out) {
    int c = q[1], ih = q[2], iw = q[3], oh = q[4], ow = q[5], kh = q[6], kw = q[7], sh = q[8],
        sw = q[9], pt = q[11], pl = q[12];
#pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < (int64_t)n_out; ++idx) {
        int x = (int)(idx % ow), y = (int)((idx / ow) % oh), ch = (int)((idx / ((int64_t)ow * oh)) % c);
        int b = (int)(idx / ((int64_t)ow * oh * c));
        float best = -3.402823466e+38f;
        for (int ky = 0; ky < kh; ++ky) {
            int iy = y * sh + ky - pt;
            if (iy < 0 || iy >= ih) continue;
            for (int kx = 0; kx < kw; ++kx) {
                int ix = x * sw + kx - pl;
                if (ix < 0 || ix >= iw) continue;
                best = fmaxf(best, in[(((int64_t)b * c + ch) * ih + iy) * iw + ix]);
            }
        }
        out[idx] = best;
    }
    return 0;
}

/* ---- softmax10.comp:8-20 / softmax1000.comp:10-22: softmax over the whole tensor ----- */
static void softmax_whole(const float* in, float* out, int n) {
    float m = in[0];
    for (int j = 1; j < n; ++j) m = fmaxf(m, in[j]);
    float sum = 0.0f;
    for (int j = 0; j < n; ++j) sum = sum + expf(in[j] - m);
    for (int i = 0; i < n; ++i) out[i] = expf(in[i] - m) / sum;
}

/* ---- resize_bilinear.comp:20-55 (NCHW) ------------------------------------------------ */
static float src_coord(int o, int in_size, int out_size, int ac, int hp) {
    if (ac != 0 && out_size > 1) return (float)o * (float)(in_size - 1) / (float)(out_size - 1);
    if (hp != 0) return ((float)o + 0.5f) * (float)in_size / (float)out_size - 0.5f;
    return (float)o * (float)in_size / (float)out_size;
}

static int k_resize(const float* in, float* out, const int32_t* q, size_t n_out) {
    int c = q[1], ih = q[2], iw = q[3], oh = q[4], ow = q[5], ac = q[6], hp = q[7];
#pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < (int64_t)n_out; ++idx) {
        int x = (int)(idx % ow), y = (int)((idx / ow) % oh), ch = (int)((idx / ((int64_t)ow * oh)) % c);
        int b = (int)(idx / ((int64_t)ow * oh * c));
        float in_y = fminf(fmaxf(src_coord(y, ih, oh, ac, hp), 0.0f), (float)(ih - 1));
        float in_x = fminf(fmaxf(src_coord(x, iw, ow, ac, hp), 0.0f), (float)(iw - 1));
        int y0 = (int)floorf(in_y), x0 = (int)floorf(in_x);
        int y1 = y0 + 1 < ih - 1 ? y0 + 1 : ih - 1, x1 = x0 + 1 < iw - 1 ? x0 + 1 : iw - 1;
        float yl = in_y - (float)y0, xl = in_x - (float)x0;
        const float* p = in + ((int64_t)b * c + ch) * ih * iw;
        float top = p[y0 * iw + x0] * (1.0f - xl) + p[y0 * iw + x1] * xl;
        float bot = p[y1 * iw + x0] * (1.0f - xl) + p[y1 * iw + x1] * xl;
        out[idx] = top * (1.0f - yl) + bot * yl;
    }
    return 0;
}

/* ---- pad.comp:15-45 ------------------------------------------------------------------- */
static int k_pad(const float* in, const float* pv, float* out, const int32_t* q, size_t n_out) {
    const int* od = q;
    const int* id = q + 4;
    const int* pl = q + 8;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n_out; ++i) {
        int64_t os1 = (int64_t)od[2] * od[3], os0 = od[1] * os1;
        int c0 = (int)(i / os0), c1 = (int)((i / os1) % od[1]), c2 = (int)((i / od[3]) % od[2]),
            c3 = (int)(i % od[3]);
        int s0 = c0 - pl[0], s1 = c1 - pl[1], s2 = c2 - pl[2], s3 = c3 - pl[3];
        if (s0 >= 0 && s0 < id[0] && s1 >= 0 && s1 < id[1] && s2 >= 0 && s2 < id[2] && s3 >= 0 &&
            s3 < id[3])
            out[i] = in[(int64_t)s0 * id[1] * id[2] * id[3] + (int64_t)s1 * id[2] * id[3] +
                        (int64_t)s2 * id[3] + s3];
        else
            out[i] = pv[0];
    }
    return 0;
}

/* ---- transpose.comp:31-52 ------------------------------------------------------------- */
static int k_transpose(const float* in, float* out, const int32_t* q, size_t n_out) {
    const int* ind = q;
    const int* outd = q + 4;
    const int* perm = q + 8;
#pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < (int64_t)n_out; ++idx) {
        int o3 = (int)(idx % outd[3]), o2 = (int)((idx / outd[3]) % outd[2]);
        int o1 = (int)((idx / ((int64_t)outd[3] * outd[2])) % outd[1]);
        int o0 = (int)(idx / ((int64_t)outd[3] * outd[2] * outd[1]));
        int vals[4] = {o0, o1, o2, o3}, i_[4] = {0, 0, 0, 0};
        for (int k = 0; k < 4; ++k) i_[perm[k]] = vals[k];
        out[idx] = in[(((int64_t)i_[0] * ind[1] + i_[1]) * ind[2] + i_[2]) * ind[3] + i_[3]];
    }
    return 0;
}

/* ---- fused attention: the scores dot_general, the row softmax and the context dot_general
 * of one encoder layer (bert_base.stablehlo.txt:28-49), in their arithmetic and order:
 * scores[t] = sum_d Q[s][d] K[t][d] (d ascending), v = scores * scale + mask[t], the softmax of
 * softmax_rows, ctx[d] = sum_t P[t] V[t][d] (t ascending); float throughout.  Q, K and V of
 * head h are the columns q_off/k_off/v_off + h*HD of rows of ld_in floats (one fused QKV
 * activation); ctx row (b, s) holds head h at columns h*HD of ld_out floats. */
static void attention_fused(const float* in, const float* mask, float* out, int B, int H, int S,
                            int HD, int64_t ld_in, int q_off, int k_off, int v_off, int64_t ld_out,
                            float scale) {
#pragma omp parallel
    {
        float* p = (float*)malloc(sizeof(float) * (size_t)S);
        float* acc = (float*)malloc(sizeof(float) * (size_t)HD);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < (int64_t)B * H * S; ++r) {
            const int s = (int)(r % S), h = (int)((r / S) % H), b = (int)(r / ((int64_t)S * H));
            const float* rows = in + (int64_t)b * S * ld_in + (int64_t)h * HD;
            const float* q = rows + (int64_t)s * ld_in + q_off;
            float m = -INFINITY;
            for (int t = 0; t < S; ++t) {
                const float* k = rows + (int64_t)t * ld_in + k_off;
                float sc = 0.0f;
                for (int d = 0; d < HD; ++d) sc = sc + q[d] * k[d];
                p[t] = sc;
                float v = sc * scale + (mask ? mask[t] : 0.0f);
                m = fmaxf(m, v);
            }
            float sum = 0.0f;
            for (int t = 0; t < S; ++t) {
                float v = p[t] * scale + (mask ? mask[t] : 0.0f);
                p[t] = expf(v - m);
                sum = sum + p[t];
            }
            for (int t = 0; t < S; ++t) p[t] = p[t] / sum;
            for (int d = 0; d < HD; ++d) acc[d] = 0.0f;
            for (int t = 0; t < S; ++t) {
                const float* v = rows + (int64_t)t * ld_in + v_off;
                for (int d = 0; d < HD; ++d) acc[d] = acc[d] + p[t] * v[d];
            }
            float* o = out + ((int64_t)b * S + s) * ld_out + (int64_t)h * HD;
            for (int d = 0; d < HD; ++d) o[d] = acc[d];
        }
        free(p);
        free(acc);
    }
}

/* ---- row normalisations / softmax as the HLO op chains ------------------------------- */
/* softmax over each row of (x*scale + mask): reduce(max) -> subtract -> exponential ->
 * reduce(sum) -> divide (bert_base.stablehlo.txt:33-49, resnet50.stablehlo.txt:1714) */
static void softmax_rows(const float* in, const float* mask, float* out, int rows, int cols,
                         float scale) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* x = in + (int64_t)r * cols;
        float* y = out + (int64_t)r * cols;
        float m = -INFINITY;
        for (int c = 0; c < cols; ++c) {
            float v = x[c] * scale + (mask ? mask[c] : 0.0f);
            m = fmaxf(m, v);
        }
        float s = 0.0f;
        for (int c = 0; c < cols; ++c) {
            float v = x[c] * scale + (mask ? mask[c] : 0.0f);
            y[c] = expf(v - m);
            s = s + y[c];
        }
        for (int c = 0; c < cols; ++c) y[c] = y[c] / s;
    }
}

/* layernorm (TF: mean, mean((x-mean)^2), (x-mean)*rsqrt(var+eps)*gamma+beta) and
 * rms_norm (export_llama.py:284-286: x * rsqrt(mean(x^2) + eps) * w) */
static void rownorm(const float* in, const float* w, float* out, int rows, int cols, float eps,
                    int rms) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* x = in + (int64_t)r * cols;
        float* y = out + (int64_t)r * cols;
        float mean = 0.0f;
        if (!rms) {
            float s = 0.0f;
            for (int c = 0; c < cols; ++c) s = s + x[c];
            mean = s / (float)cols;
        }
        float ss = 0.0f;
        for (int c = 0; c < cols; ++c) {
            float d = x[c] - mean;
            ss = ss + d * d;
        }
        float inv = 1.0f / sqrtf(ss / (float)cols + eps);
        for (int c = 0; c < cols; ++c) {
            float v = (x[c] - mean) * inv;
            y[c] = rms ? v * w[c] : v * w[c] + w[cols + c];
        }
    }
}

/* ---- HLO host shape ops (source/xla_hlo/src/compiler.rs), restated the way the Rust
 * helpers run them: per element, unravel the index (unravel :1299-1307), map the
 * coordinate, ravel it (ravel :1309-1315). */
#define HMAX 8
static int64_t h_elems(const int32_t* d, int r) {
    int64_t n = 1;
    for (int k = 0; k < r; ++k) n *= d[k];
    return n;
}
static void h_unravel(int64_t idx, const int32_t* shape, int r, int64_t* c) {
    int64_t st[HMAX], s = 1;
    for (int k = r - 1; k >= 0; --k) {
        st[k] = s;
        s *= shape[k];
    }
    for (int k = 0; k < r; ++k) {
        c[k] = idx / st[k];
        idx %= st[k];
    }
}
static int64_t h_ravel(const int64_t* c, const int32_t* shape, int r) {
    int64_t s = 1, idx = 0;
    for (int k = r - 1; k >= 0; --k) {
        idx += c[k] * s;
        s *= shape[k];
    }
    return idx;
}
static int h_dims_ok(const int32_t* d, int r) {
    if (r < 0 || r > HMAX) return 0;
    for (int k = 0; k < r; ++k)
        if (d[k] <= 0) return 0;
    return 1;
}

/* broadcast_tensor :1361-1393 with explicit `dimensions` (map[a] = output axis of a) */
static int h_broadcast(const float* src, const int32_t* sd, int rs, const int32_t* map,
                       float* out, const int32_t* od, int ro) {
    int64_t n_out = h_elems(od, ro), n_src = h_elems(sd, rs);
    int same = rs == ro;
    for (int k = 0; same && k < rs; ++k) same = sd[k] == od[k];
    if (n_src == n_out && same) {
        memcpy(out, src, (size_t)n_out * sizeof(float));
        return 0;
    }
    if (n_src == 1) {
        for (int64_t i = 0; i < n_out; ++i) out[i] = src[0];
        return 0;
    }
    for (int a = 0; a < rs; ++a)
        if (map[a] < 0 || map[a] >= ro || (sd[a] != 1 && sd[a] != od[map[a]])) return -1;
    for (int64_t idx = 0; idx < n_out; ++idx) {
        int64_t oc[HMAX], sc[HMAX];
        h_unravel(idx, od, ro, oc);
        for (int a = 0; a < rs; ++a) sc[a] = sd[a] == 1 ? 0 : oc[map[a]];
        out[idx] = src[h_ravel(sc, sd, rs)];
    }
    return 0;
}

/* binary_tensor :1521-1564 operand rule: as many values as the output -> used flat, else
 * broadcast_tensor with infer_broadcast_dims :1566-1572 (trailing alignment). */
static int h_operand(const float* src, const int32_t* sd, int rs, float* out, const int32_t* od,
                     int ro) {
    int64_t n_out = h_elems(od, ro);
    if (h_elems(sd, rs) == n_out) {
        memcpy(out, src, (size_t)n_out * sizeof(float));
        return 0;
    }
    if (rs > ro) return h_elems(sd, rs) == 1 ? h_broadcast(src, sd, rs, NULL, out, od, ro) : -1;
    int32_t map[HMAX];
    for (int a = 0; a < rs; ++a) map[a] = a + (ro - rs);
    return h_broadcast(src, sd, rs, map, out, od, ro);
}

/* reduce_tensor :1730-1759: walk the source in index order, fold into the kept coordinate */
static void h_reduce(const float* src, const int32_t* sd, int r, const int32_t* red, int kind,
                     float init, float* out, int64_t n_out) {
    for (int64_t i = 0; i < n_out; ++i) out[i] = init;
    int32_t od[HMAX];
    int ro = 0;
    for (int k = 0; k < r; ++k)
        if (!red[k]) od[ro++] = sd[k];
    int64_t n = h_elems(sd, r);
    for (int64_t idx = 0; idx < n; ++idx) {
        int64_t c[HMAX], oc[HMAX];
        h_unravel(idx, sd, r, c);
        int j = 0;
        for (int k = 0; k < r; ++k)
            if (!red[k]) oc[j++] = c[k];
        int64_t o = ro ? h_ravel(oc, od, ro) : 0;
        out[o] = kind ? fmaxf(out[o], src[idx]) : out[o] + src[idx];
    }
}

static const char* kNames[] = {
    "abs", "exp", "log", "neg", "sqrt", "rsqrt", "sigmoid", "logistic", "tanh", "relu", "relu6",
    "sine", "reshape", "leaky_relu", "add", "sub", "mul", "div", "pow", "min", "max", "concat",
    "pad", "transpose", "l2norm", "silu", "gelu_erf", "cosine", "floor", "ceil",
    "l2_normalization", "broadcast_binary", "bias_act", "hlo_reduce_rank4",
    "hlo_reduce_window_rank4", "max_pool2d", "global_avg_pool_sum", "global_avg_pool_finalize",
    "softmax10", "softmax1000", "global_avg_pool_nhwc", "softmax_rows", "layernorm_rows",
    "rmsnorm_rows", "hlo_conv_nhwc_hwio", "conv2d", "fully_connected", "hlo_dot_batched",
    "hlo_dot_rank2", "conv2d_nhwc", "dot_general_strided", "depthwise_conv2d",
    "resize_bilinear", "depthwise_conv2d_nhwc", "gemv_nt", "argmax_rows", "gather_rows", "hlo_broadcast",
    "hlo_transpose", "hlo_slice", "hlo_concatenate_into", "hlo_compare", "hlo_select",
    "hlo_reduce", "hlo_strided_copy", "attention_fused", "nan_count", "inverted_residual_nhwc",
    "conv1x1_gap_nhwc"};

int orc_kernel_count(void) { return (int)(sizeof kNames / sizeof kNames[0]); }
const char* orc_kernel_name(int i) {
    return (i >= 0 && i < orc_kernel_count()) ? kNames[i] : NULL;
}

int orc_run_kernel(const char* name, const float* in0, size_t n0, const float* in1, size_t n1,
                   float* out, size_t n_out, const int32_t* push, size_t n_push,
                   const float* bias, const float* residual, int32_t act, float alpha) {
    (void)n0;
    (void)n1;
    if (!name) return orc_fail(-1, "null kernel name");
    int ok = 0;
    float la = 0.0f;
    if (!strcmp(name, "leaky_relu")) {
        NEED(2);
        la = bits_to_f32(push[1]);
    }
    un_op(name, 0.0f, 0.0f, &ok);
    if (ok) { /* unary: push {total} */
        NEED(1);
        TOTAL(push[0]);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < (int64_t)n_out; ++i) {
            int k;
            out[i] = un_op(name, in0[i], la, &k);
        }
        return 0;
    }
    int bc = bin_code(name);
    if (bc >= 0) { /* binary: push {total} */
        NEED(1);
        TOTAL(push[0]);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < (int64_t)n_out; ++i) out[i] = bin_op(bc, in0[i], in1[i]);
        return 0;
    }
    if (!strcmp(name, "concat")) { /* concat.comp:13-17 */
        NEED(2);
        TOTAL(push[1]);
        for (int64_t i = 0; i < (int64_t)n_out; ++i)
            out[i] = i < push[0] ? in0[i] : in1[i - push[0]];
        return 0;
    }
    if (!strcmp(name, "pad")) {
        NEED(13);
        TOTAL(push[12]);
        return k_pad(in0, in1, out, push, n_out);
    }
    if (!strcmp(name, "transpose")) {
        NEED(13);
        TOTAL(push[12]);
        return k_transpose(in0, out, push, n_out);
    }
    if (!strcmp(name, "l2norm")) { /* l2norm.comp:13-18 */
        NEED(2);
        TOTAL(push[0]);
        float norm = bits_to_f32(push[1]);
        float d = fmaxf(norm, 1.0e-12f);
        for (size_t i = 0; i < n_out; ++i) out[i] = in0[i] / d;
        return 0;
    }
    if (!strcmp(name, "l2_normalization")) { /* scheduler.rs:816 norm, then l2norm.comp */
        NEED(1);
        TOTAL(push[0]);
        float s = 0.0f;
        for (size_t i = 0; i < n_out; ++i) s = s + in0[i] * in0[i];
        float d = fmaxf(sqrtf(s), 1.0e-12f);
        for (size_t i = 0; i < n_out; ++i) out[i] = in0[i] / d;
        return 0;
    }
    if (!strcmp(name, "broadcast_binary")) { /* compiler.rs:705-729 + :1361-1393 */
        NEED(14);
        TOTAL(push[1]);
        int op = push[0];
        const int32_t* d = push + 2;
        const int32_t* as = push + 6;
        const int32_t* bs = push + 10;
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < (int64_t)n_out; ++i) {
            int64_t r = i, ai = 0, bi = 0;
            for (int k = 3; k >= 0; --k) {
                int c = (int)(r % d[k]);
                r /= d[k];
                ai += (int64_t)c * as[k];
                bi += (int64_t)c * bs[k];
            }
            out[i] = bin_op(op, in0[ai], in1[bi]);
        }
        return 0;
    }
    if (!strcmp(name, "bias_act")) {
        NEED(2);
        TOTAL(push[0]);
        memcpy(out, in0, n_out * sizeof(float));
        epilogue(out, n_out, (size_t)push[1], bias, residual, act, alpha);
        return 0;
    }
    if (!strcmp(name, "hlo_reduce_rank4")) {
        NEED(15);
        TOTAL(push[14]);
        return k_reduce_rank4(in0, out, push, n_out);
    }
    if (!strcmp(name, "hlo_reduce_window_rank4")) {
        NEED(14);
        TOTAL(push[13]);
        return k_reduce_window(in0, out, push, n_out);
    }
    if (!strcmp(name, "max_pool2d")) {
        NEED(14);
        TOTAL(push[13]);
        return k_max_pool(in0, out, push, n_out);
    }
    if (!strcmp(name, "global_avg_pool_sum")) { /* global_avg_pool_sum.comp:15-28 */
        NEED(4);
        TOTAL((int64_t)push[0] * push[1]);
        int hw = push[2] * push[3];
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < (int64_t)n_out; ++i) {
            float acc = 0.0f;
            for (int j = 0; j < hw; ++j) acc = acc + in0[i * hw + j];
            out[i] = acc;
        }
        return 0;
    }
    if (!strcmp(name, "global_avg_pool_finalize")) { /* global_avg_pool_finalize.comp:15-19 */
        NEED(4);
        TOTAL((int64_t)push[0] * push[1]);
        float hw = (float)(push[2] * push[3]);
        for (size_t i = 0; i < n_out; ++i) out[i] = in0[i] / hw;
        return 0;
    }
    if (!strcmp(name, "global_avg_pool_nhwc")) { /* sum then / (h*w), per (n, c) */
        NEED(4);
        TOTAL((int64_t)push[0] * push[3]);
        int hw = push[1] * push[2], c = push[3];
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < (int64_t)n_out; ++i) {
            int64_t b = i / c;
            int ch = (int)(i % c);
            float acc = 0.0f;
            for (int j = 0; j < hw; ++j) acc = acc + in0[(b * hw + j) * c + ch];
            out[i] = acc / (float)hw;
        }
        return 0;
    }
    if (!strcmp(name, "softmax10")) {
        if (n_out != 10) return orc_fail(-4, "softmax10 is fixed at 10 classes");
        softmax_whole(in0, out, 10);
        return 0;
    }
    if (!strcmp(name, "softmax1000")) {
        NEED(1);
        TOTAL(push[0]);
        softmax_whole(in0, out, push[0]);
        return 0;
    }
    if (!strcmp(name, "softmax_rows")) {
        NEED(3);
        TOTAL((int64_t)push[0] * push[1]);
        softmax_rows(in0, in1, out, push[0], push[1], bits_to_f32(push[2]));
        return 0;
    }
    if (!strcmp(name, "layernorm_rows") || !strcmp(name, "rmsnorm_rows")) {
        NEED(3);
        TOTAL((int64_t)push[0] * push[1]);
        rownorm(in0, in1, out, push[0], push[1], bits_to_f32(push[2]),
                !strcmp(name, "rmsnorm_rows"));
        return 0;
    }
    if (!strcmp(name, "hlo_conv_nhwc_hwio")) {
        NEED(14);
        TOTAL((int64_t)push[0] * push[7] * push[8] * push[6]);
        k_hlo_conv(in0, in1, out, push);
        epilogue(out, n_out, (size_t)push[6], bias, residual, act, alpha);
        return 0;
    }
    if (!strcmp(name, "conv2d") || !strcmp(name, "conv2d_nhwc")) {
        NEED(15);
        TOTAL((int64_t)push[0] * push[4] * push[5] * push[6]);
        int nhwc = !strcmp(name, "conv2d_nhwc");
        k_conv2d(in0, in1, out, push, nhwc);
        epilogue(out, n_out, 0, NULL, residual, act, alpha);
        return 0;
    }
    if (!strcmp(name, "inverted_residual_nhwc")) {
        /* An MBConv block as the TFLite scheduler dispatches it, three operators in order
         * (scheduler.rs:321-427 CONV_2D, :429-548 DEPTHWISE_CONV_2D, then the projection
         * CONV_2D and the residual ADD): the loops of conv2d_nhwc (1x1) and
         * depthwise_conv2d_nhwc above on the operators' own weight tensors, which the packed
         * in1 holds back to back.  push {n, cin, h, w, ce, cout, oh, ow, k, s, pt, pl,
         * expand, act_e, act_d, total}; residual and act apply to the projection. */
        NEED(16);
        const int n = push[0], cin = push[1], h = push[2], w = push[3], ce = push[4],
                  cout = push[5], oh = push[6], ow = push[7], k = push[8], st = push[9],
                  pt = push[10], pl = push[11], expand = push[12], act_e = push[13],
                  act_d = push[14];
        TOTAL((int64_t)n * oh * ow * cout);
        if (!expand && ce != cin) return orc_fail(-4, "inverted_residual_nhwc: ce != cin");
        const float* wp = in1;
        const float* e = in0;
        float* ebuf = NULL;
        if (expand) {
            const size_t ne = (size_t)n * h * w * ce;
            ebuf = (float*)malloc(sizeof(float) * ne);
            const int32_t qe[15] = {n, cin, h, w, ce, h, w, 1, 1, 1, 1, 1, 0, 0, (int32_t)ne};
            k_conv2d(in0, wp, ebuf, qe, 1);
            epilogue(ebuf, ne, 0, NULL, NULL, act_e, alpha);
            e = ebuf;
            wp += (size_t)ce * cin + ce;
        }
        const size_t nd = (size_t)n * oh * ow * ce;
        float* dbuf = (float*)malloc(sizeof(float) * nd);
        const int32_t qd[16] = {n, ce, h, w, oh, ow, k, k, st, st, 1, pt, pl, 1, 1, (int32_t)nd};
        k_depthwise(e, wp, dbuf, qd, 1);
        epilogue(dbuf, nd, 0, NULL, NULL, act_d, alpha);
        wp += (size_t)k * k * ce + ce;
        const int32_t qp[15] = {n, ce, oh, ow, cout, oh, ow, 1, 1, 1, 1, 1, 0, 0, (int32_t)n_out};
        k_conv2d(dbuf, wp, out, qp, 1);
        epilogue(out, n_out, 0, NULL, residual, act, alpha);
        free(ebuf);
        free(dbuf);
        return 0;
    }
    if (!strcmp(name, "conv1x1_gap_nhwc")) {
        /* The classifier head as the TFLite scheduler dispatches it: CONV_2D 1x1 with its fused
         * activation (scheduler.rs:321-427), then MEAN over H and W (:549-613) -- the loops of
         * conv2d_nhwc and global_avg_pool_nhwc above.  push {n, cin, h, w, cout, total}. */
        NEED(6);
        const int n = push[0], cin = push[1], h = push[2], w = push[3], cout = push[4];
        TOTAL((int64_t)n * cout);
        if (residual) return orc_fail(-4, "conv1x1_gap_nhwc: no residual");
        const size_t nc = (size_t)n * h * w * cout;
        float* cbuf = (float*)malloc(sizeof(float) * nc);
        const int32_t qc[15] = {n, cin, h, w, cout, h, w, 1, 1, 1, 1, 1, 0, 0, (int32_t)nc};
        k_conv2d(in0, in1, cbuf, qc, 1);
        epilogue(cbuf, nc, 0, NULL, NULL, act, alpha);
        const int hw = h * w;
        for (int64_t i = 0; i < (int64_t)n_out; ++i) {
            const int64_t b = i / cout;
            const int ch = (int)(i % cout);
            float acc = 0.0f;
            for (int j = 0; j < hw; ++j) acc = acc + cbuf[(b * hw + j) * cout + ch];
            out[i] = acc / (float)hw;
        }
        free(cbuf);
        return 0;
    }
    if (!strcmp(name, "depthwise_conv2d") || !strcmp(name, "depthwise_conv2d_nhwc")) {
        NEED(16);
        TOTAL((int64_t)push[0] * push[1] * push[4] * push[5]);
        k_depthwise(in0, in1, out, push, !strcmp(name, "depthwise_conv2d_nhwc"));
        epilogue(out, n_out, 0, NULL, residual, act, alpha);
        return 0;
    }
    if (!strcmp(name, "fully_connected")) {
        NEED(4);
        TOTAL((int64_t)push[0] * push[2]);
        k_fully_connected(in0, in1, out, push);
        epilogue(out, n_out, 0, NULL, residual, act, alpha);
        return 0;
    }
    if (!strcmp(name, "hlo_dot_batched")) { /* hlo_dot_batched.comp:19-38 */
        NEED(5);
        int B = push[0], M = push[1], K = push[2], N = push[3];
        TOTAL((int64_t)B * M * N);
        dot_strided(B, 1, M, N, K, in0, (int64_t)M * K, 0, K, 1, in1, (int64_t)K * N, 0, N, 1,
                    out, (int64_t)M * N, 0, N, 1, bias, residual, act, alpha);
        return 0;
    }
    if (!strcmp(name, "hlo_dot_rank2")) { /* hlo_dot_rank2.comp:15-26 */
        NEED(4);
        int M = push[0], K = push[1], N = push[2];
        TOTAL((int64_t)M * N);
        dot_strided(1, 1, M, N, K, in0, 0, 0, K, 1, in1, 0, 0, N, 1, out, 0, 0, N, 1, bias,
                    residual, act, alpha);
        return 0;
    }
    if (!strcmp(name, "dot_general_strided")) {
        NEED(17);
        const int32_t* q = push;
        TOTAL((int64_t)q[0] * q[1] * q[2] * q[3]);
        dot_strided(q[0], q[1], q[2], q[3], q[4], in0, q[5], q[6], q[7], q[8], in1, q[9], q[10],
                    q[11], q[12], out, q[13], q[14], q[15], q[16], bias, residual, act, alpha);
        return 0;
    }
    if (!strcmp(name, "attention_fused")) {
        /* {B, H, S, HD, ld_in, q_off, k_off, v_off, ld_out, scale_bits, total = B*S*ld_out} */
        NEED(11);
        const int32_t* q = push;
        if (q[0] <= 0 || q[1] <= 0 || q[2] <= 0 || q[3] <= 0)
            return orc_fail(-4, "attention_fused: dims");
        TOTAL((int64_t)q[0] * q[2] * q[8]);
        if (q[10] != (int32_t)n_out) return orc_fail(-4, "attention_fused: total");
        attention_fused(in0, in1, out, q[0], q[1], q[2], q[3], q[4], q[5], q[6], q[7], q[8],
                        bits_to_f32(q[9]));
        return 0;
    }
    if (!strcmp(name, "resize_bilinear")) {
        NEED(9);
        TOTAL((int64_t)push[0] * push[1] * push[4] * push[5]);
        return k_resize(in0, out, push, n_out);
    }
    if (!strcmp(name, "gemv_nt")) { /* y[n] = sum_k x[k] W[n][k] (k ascending) + bias + res */
        NEED(2);
        int N = push[0], K = push[1];
        TOTAL(N);
#pragma omp parallel for schedule(static)
        for (int n = 0; n < N; ++n) {
            float acc = 0.0f;
            const float* w = in1 + (int64_t)n * K;
            for (int k = 0; k < K; ++k) acc = acc + in0[k] * w[k];
            out[n] = acc;
        }
        epilogue(out, n_out, 0, bias, residual, act, alpha);
        return 0;
    }
    if (!strcmp(name, "nan_count")) {
        /* compiler.rs:613-623 NaN trace: count of NaN values and the first one's index
         * (-1 when none), stored as uint32 / int32 bits in out[0], out[1] */
        NEED(1);
        TOTAL(2);
        uint32_t cnt = 0;
        int32_t first = -1;
        for (int64_t i = 0; i < (int64_t)push[0]; ++i)
            if (isnan(in0[i])) {
                if (first < 0) first = (int32_t)i;
                ++cnt;
            }
        memcpy(&out[0], &cnt, 4);
        memcpy(&out[1], &first, 4);
        return 0;
    }
    if (!strcmp(name, "gather_rows")) { /* embed_table[ids] (run_llama_spirv.py:203) */
        NEED(3);
        int nid = push[0], len = push[1], rows = push[2];
        TOTAL((int64_t)nid * len);
        for (int r = 0; r < nid; ++r) {
            int32_t id;
            memcpy(&id, &in0[r], 4);
            for (int c = 0; c < len; ++c)
                out[(int64_t)r * len + c] =
                    (id >= 0 && id < rows) ? in1[(int64_t)id * len + c] : 0.0f;
        }
        return 0;
    }
    if (!strcmp(name, "argmax_rows")) { /* numpy argmax: first maximum; stored as int32 */
        NEED(2);
        TOTAL(push[0]);
        int cols = push[1];
        for (int r = 0; r < push[0]; ++r) {
            int32_t idx = orc_argmax_first(in0 + (int64_t)r * cols, (size_t)cols);
            memcpy(&out[r], &idx, 4);
        }
        return 0;
    }
    if (!strcmp(name, "hlo_broadcast")) { /* compiler.rs:336-347 */
        NEED(3);
        int rs = push[0], ro = push[1];
        if (rs < 0 || rs > HMAX || ro < 1 || ro > HMAX) return orc_fail(-4, "hlo_broadcast: rank");
        NEED(3 + 2 * rs + ro);
        const int32_t *sd = push + 3, *od = push + 3 + rs, *map = push + 3 + rs + ro;
        if (!h_dims_ok(sd, rs) || !h_dims_ok(od, ro) || h_elems(od, ro) != push[2])
            return orc_fail(-4, "hlo_broadcast: dims");
        TOTAL(push[2]);
        if (h_broadcast(in0, sd, rs, map, out, od, ro)) return orc_fail(-4, "hlo_broadcast: dimensions");
        return 0;
    }
    if (!strcmp(name, "hlo_transpose")) { /* compiler.rs:374-386, transpose_tensor :1395-1418 */
        NEED(2);
        int r = push[0];
        if (r < 1 || r > HMAX) return orc_fail(-4, "hlo_transpose: rank");
        NEED(2 + 2 * r);
        const int32_t *sd = push + 2, *perm = push + 2 + r;
        if (!h_dims_ok(sd, r) || h_elems(sd, r) != push[1]) return orc_fail(-4, "hlo_transpose: dims");
        TOTAL(push[1]);
        int32_t od[HMAX];
        int seen = 0, ident = 1;
        for (int i = 0; i < r; ++i) {
            if (perm[i] < 0 || perm[i] >= r || ((seen >> perm[i]) & 1)) return orc_fail(-4, "hlo_transpose: perm");
            seen |= 1 << perm[i];
            ident &= perm[i] == i;
            od[i] = sd[perm[i]];
        }
        if (ident) {
            memcpy(out, in0, n_out * sizeof(float));
            return 0;
        }
        for (int64_t idx = 0; idx < (int64_t)n_out; ++idx) {
            int64_t oc[HMAX], sc[HMAX];
            h_unravel(idx, od, r, oc);
            for (int i = 0; i < r; ++i) sc[perm[i]] = oc[i];
            out[idx] = in0[h_ravel(sc, sd, r)];
        }
        return 0;
    }
    if (!strcmp(name, "hlo_strided_copy")) { /* no reference counterpart: a view of the
                                                 compiled HLO program made contiguous */
        NEED(2);
        int r = push[0];
        if (r < 1 || r > HMAX) return orc_fail(-4, "hlo_strided_copy: rank");
        NEED(2 + 2 * r);
        const int32_t *od = push + 2, *st = push + 2 + r;
        if (!h_dims_ok(od, r) || h_elems(od, r) != push[1]) return orc_fail(-4, "hlo_strided_copy: dims");
        TOTAL(push[1]);
        int64_t extent = 1;
        for (int k = 0; k < r; ++k) {
            if (st[k] < 0) return orc_fail(-4, "hlo_strided_copy: negative stride");
            extent += (int64_t)(od[k] - 1) * st[k];
        }
        if (n0 > 0 && extent > (int64_t)n0) return orc_fail(-4, "hlo_strided_copy: view exceeds in0");
        for (int64_t idx = 0; idx < (int64_t)n_out; ++idx) {
            int64_t oc[HMAX], off = 0;
            h_unravel(idx, od, r, oc);
            for (int k = 0; k < r; ++k) off += oc[k] * st[k];
            out[idx] = in0[off];
        }
        return 0;
    }
    if (!strcmp(name, "hlo_slice")) { /* compiler.rs:570-582, cpu_slice :1931-1952 */
        NEED(2);
        int r = push[0];
        if (r < 1 || r > HMAX) return orc_fail(-4, "hlo_slice: rank");
        NEED(2 + 4 * r);
        const int32_t *sd = push + 2, *st = push + 2 + r, *lim = push + 2 + 2 * r, *sp = push + 2 + 3 * r;
        if (!h_dims_ok(sd, r)) return orc_fail(-4, "hlo_slice: dims");
        int32_t od[HMAX];
        for (int k = 0; k < r; ++k) {
            if (st[k] < 0 || sp[k] < 1 || lim[k] <= st[k]) return orc_fail(-4, "hlo_slice: spec");
            od[k] = (lim[k] - st[k] + sp[k] - 1) / sp[k];
        }
        if (h_elems(od, r) != push[1]) return orc_fail(-4, "hlo_slice: total");
        TOTAL(push[1]);
        for (int64_t idx = 0; idx < (int64_t)n_out; ++idx) {
            int64_t oc[HMAX], sc[HMAX];
            int in = 1;
            h_unravel(idx, od, r, oc);
            for (int k = 0; k < r; ++k) {
                sc[k] = st[k] + oc[k] * sp[k];
                in &= sc[k] < sd[k];
            }
            out[idx] = in ? in0[h_ravel(sc, sd, r)] : 0.0f;
        }
        return 0;
    }
    if (!strcmp(name, "hlo_concatenate_into")) { /* compiler.rs:554-569, cpu_concatenate :1879-1895 */
        NEED(3);
        int r = push[0], dim = push[1], offset = push[2];
        if (r < 1 || r > HMAX || dim < 0 || dim >= r || offset < 0) return orc_fail(-4, "hlo_concatenate_into: rank/dim");
        NEED(3 + 2 * r);
        const int32_t *od = push + 3, *id = push + 3 + r;
        if (!h_dims_ok(od, r) || !h_dims_ok(id, r)) return orc_fail(-4, "hlo_concatenate_into: dims");
        TOTAL(h_elems(od, r));
        int64_t n = h_elems(id, r);
        for (int64_t idx = 0; idx < n; ++idx) {
            int64_t c[HMAX];
            int in = 1;
            h_unravel(idx, id, r, c);
            c[dim] += offset;
            for (int k = 0; k < r; ++k) in &= c[k] < od[k];
            if (in) out[h_ravel(c, od, r)] = in0[idx];
        }
        return 0;
    }
    if (!strcmp(name, "hlo_compare") || !strcmp(name, "hlo_select")) {
        /* compare: compiler.rs:511-537 over binary_tensor; select: select_tensor :1574-1620
         * with on_false already in `out` */
        int sel = !strcmp(name, "hlo_select");
#define Q(k) push[(k) - sel] /* field k of the compare layout; select lacks field 0 */
        NEED(5 - sel);
        int ro = Q(2), ra = Q(3), rb = Q(4);
        if (ro < 1 || ro > HMAX || ra < 0 || ra > HMAX || rb < 0 || rb > HMAX) return orc_fail(-4, "compare/select: rank");
        NEED(5 - sel + ro + ra + rb);
        const int32_t *od = push + 5 - sel, *ad = od + ro, *bd = od + ro + ra;
        if (!h_dims_ok(od, ro) || !h_dims_ok(ad, ra) || !h_dims_ok(bd, rb) || h_elems(od, ro) != Q(1))
            return orc_fail(-4, "compare/select: dims");
        TOTAL(Q(1));
        int dir = sel ? 0 : Q(0);
#undef Q
        float* a = (float*)malloc(n_out * sizeof(float));
        float* b = (float*)malloc(n_out * sizeof(float));
        int bad = !a || !b || h_operand(in0, ad, ra, a, od, ro) || h_operand(in1, bd, rb, b, od, ro);
        if (!bad) {
            for (size_t i = 0; i < n_out; ++i) {
                if (sel) {
                    if (a[i] != 0.0f) out[i] = b[i];
                    continue;
                }
                int t;
                switch (dir) {
                    case 0: t = a[i] < b[i]; break;
                    case 1: t = a[i] <= b[i]; break;
                    case 2: t = a[i] == b[i]; break;
                    case 3: t = a[i] != b[i]; break;
                    case 4: t = a[i] >= b[i]; break;
                    default: t = a[i] > b[i]; break;
                }
                out[i] = t ? 1.0f : 0.0f;
            }
        }
        free(a);
        free(b);
        return bad ? orc_fail(-4, "compare/select: operand does not broadcast") : 0;
    }
    if (!strcmp(name, "hlo_reduce")) { /* compiler.rs:939-1007 rank > 4 path: reduce_tensor */
        NEED(4);
        int r = push[1];
        if (r < 1 || r > HMAX || (push[0] != 0 && push[0] != 1)) return orc_fail(-4, "hlo_reduce: rank/kind");
        NEED(4 + 2 * r);
        const int32_t *sd = push + 4, *red = push + 4 + r;
        if (!h_dims_ok(sd, r)) return orc_fail(-4, "hlo_reduce: dims");
        int64_t kept = 1;
        for (int k = 0; k < r; ++k)
            if (!red[k]) kept *= sd[k];
        if (kept != push[2]) return orc_fail(-4, "hlo_reduce: total");
        TOTAL(push[2]);
        h_reduce(in0, sd, r, red, push[0], bits_to_f32(push[3]), out, (int64_t)n_out);
        return 0;
    }
    char msg[128];
    snprintf(msg, sizeof msg, "oracle: unknown kernel '%s'", name);
    return orc_fail(-2, msg);
}

/* ---- host helpers ------------------------------------------------------------------------ */
void orc_same_padding(int same, int ih, int iw, int oh, int ow, int kh, int kw, int sh, int sw,
                      int32_t* pad_top, int32_t* pad_left) {
    if (!same) {
        *pad_top = 0;
        *pad_left = 0;
        return;
    }
    int th = (oh - 1) * sh + kh - ih, tw = (ow - 1) * sw + kw - iw;
    if (th < 0) th = 0;
    if (tw < 0) tw = 0;
    *pad_top = th / 2;
    *pad_left = tw / 2;
}

void orc_pack_conv_weight(const float* src, const float* bias, int oc, int kh, int kw, int ic,
                          float* out) {
    for (int o = 0; o < oc; ++o) {
        for (int i = 0; i < ic; ++i)
            for (int y = 0; y < kh; ++y)
                for (int x = 0; x < kw; ++x)
                    out[(((int64_t)o * ic + i) * kh + y) * kw + x] =
                        src[(((int64_t)o * kh + y) * kw + x) * ic + i];
        out[(int64_t)oc * ic * kh * kw + o] = bias[o];
    }
}

void orc_pack_depthwise_weight(const float* src, const float* bias, int kh, int kw, int c,
                               float* out) {
    for (int ch = 0; ch < c; ++ch) {
        for (int y = 0; y < kh; ++y)
            for (int x = 0; x < kw; ++x)
                out[((int64_t)ch * kh + y) * kw + x] = src[((int64_t)y * kw + x) * c + ch];
        out[(int64_t)c * kh * kw + ch] = bias[ch];
    }
}

void orc_pack_fc_weight(const float* w, const float* bias, int out_size, int in_size, float* out) {
    memcpy(out, w, sizeof(float) * (size_t)out_size * in_size);
    memcpy(out + (int64_t)out_size * in_size, bias, sizeof(float) * (size_t)out_size);
}

int orc_top1_reference(const float* v, size_t n, float* confidence) {
    size_t offset = n == 1001 ? 1 : 0;
    size_t best = offset;
    if (n <= offset) {
        if (confidence) *confidence = 0.0f;
        return 0;
    }
    for (size_t i = offset + 1; i < n; ++i)
        if (!(v[i] < v[best])) best = i; /* max_by keeps the last of equal maxima */
    if (confidence) *confidence = v[best];
    return (int)(best - offset);
}

int orc_argmax_first(const float* v, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; ++i)
        if (v[i] > v[best]) best = i;
    return (int)best;
}

void orc_compare(const float* a, size_t na, const float* e, size_t ne, float eps,
                 uint64_t* mismatch, float* max_abs, float* max_rel) {
    uint64_t mm = 0;
    float ma = 0.0f, mr = 0.0f;
    size_t n = na < ne ? na : ne;
    for (size_t i = 0; i < n; ++i) {
        float d = fabsf(a[i] - e[i]);
        float r = d / fmaxf(fabsf(e[i]), 1.0e-30f);
        ma = fmaxf(ma, d);
        mr = fmaxf(mr, r);
        if (d > eps) ++mm;
    }
    mm += na > ne ? na - ne : ne - na;
    *mismatch = mm;
    *max_abs = ma;
    *max_rel = mr;
}

/* ---- closed-form fixtures -------------------------------------------------------------- */
int orc_parity_fixture(int which, float* out, size_t n) {
    /* generate_fixtures.py:67-82 (values rounded to f32 by struct.pack) */
    static const size_t sizes[] = {4096, 128, 256, 5, 16 * 64, 3 * 64 * 32};
    if (which < 0 || which > 5 || n != sizes[which]) return orc_fail(-4, "fixture size");
    for (size_t i = 0; i < n; ++i) {
        double v = 0.0;
        switch (which) {
            case 0:
                if (i == 0) v = -0.0;
                else if (i == 1) v = 0.0;
                else if (i % 17 == 0) v = ((double)((long)(i % 31) - 15)) * 1.0e-7;
                else v = ((double)((long)((i * 37) % 211) - 105)) * 0.03125;
                break;
            case 1: v = ((double)((long)((i * 13) % 37) - 18)) * 0.0625; break;
            case 2: v = ((double)((long)((i * 19) % 127) - 63)) * 0.015625; break;
            case 3: {
                static const double p[5] = {0.125, 1.0, 1.0, 0.0, 0.0};
                v = p[i];
                break;
            }
            case 4: v = ((double)((long)((i * 17) % 97) - 48)) * 0.00390625; break;
            case 5: v = ((double)((long)((i * 11) % 53) - 26)) * 0.001953125; break;
        }
        out[i] = (float)v;
    }
    return 0;
}

int orc_poc_fixture(int which, float* out, size_t n) {
    /* source/inference_poc/src/fixture.rs:28-50 (f32 arithmetic as in Rust) */
    static const size_t sizes[] = {64, 12, 16, 250};
    if (which < 0 || which > 3 || n != sizes[which]) return orc_fail(-4, "fixture size");
    if (which == 0)
        for (size_t i = 0; i < 64; ++i) out[i] = ((float)((i * 17) % 101) - 50.0f) * 0.015625f;
    if (which == 1)
        for (size_t i = 0; i < 12; ++i) out[i] = ((float)((i * 11) % 31) - 15.0f) * 0.03125f;
    if (which == 2)
        for (int c = 0; c < 4; ++c) {
            out[c * 4 + 0] = 0.85f + (float)c * 0.05f;
            out[c * 4 + 1] = -0.10f + (float)c * 0.04f;
            out[c * 4 + 2] = -0.05f + (float)c * 0.025f;
            out[c * 4 + 3] = 0.70f + (float)c * 0.08f;
        }
    if (which == 3) {
        for (size_t i = 0; i < 240; ++i) out[i] = ((float)((i * 7) % 43) - 21.0f) * 0.0078125f;
        for (size_t i = 0; i < 10; ++i) out[240 + i] = ((float)i - 4.5f) * 0.015625f;
    }
    return 0;
}

/* ---- TinyLlama-shaped decoder (export_llama.py:269-375) ------------------------------ */
static void rms_norm_vec(const float* x, const float* w, float* y, int n, float eps) {
    /* variance = reduce_mean(square(x)); x * rsqrt(variance + eps) * w */
    float ss = 0.0f;
    for (int i = 0; i < n; ++i) ss = ss + x[i] * x[i];
    float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; ++i) y[i] = (x[i] * inv) * w[i];
}

/* y[r] = sum_k v[k] * W[r*row_stride][k], k ascending (matmul(h, W_in_out)) */
static void matvec(const float* v, const float* W, int rows, int K, int64_t row_stride,
                   float* y) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* w = W + (int64_t)r * row_stride * K;
        float acc = 0.0f;
        for (int k = 0; k < K; ++k) acc = acc + v[k] * w[k];
        y[r] = acc;
    }
}

/* RoPE rotate-half with numpy-float32 tables (run_llama_spirv.py:87-97):
 * inv_freq[j] = 1 / theta^(2j/64); angle = pos * inv_freq[i % 32] */
static void rope(float* x, int pos, float theta) {
    float tmp[64];
    for (int i = 0; i < 64; ++i) {
        int j = i % 32;
        float inv = 1.0f / powf(theta, (float)(2 * j) / 64.0f);
        float ang = (float)pos * inv;
        float rh = i < 32 ? -x[i + 32] : x[i - 32];
        tmp[i] = x[i] * cosf(ang) + rh * sinf(ang);
    }
    memcpy(x, tmp, sizeof tmp);
}

static int llama_check(const orc_llama_cfg* c) {
    if (c->head_dim != 64 || c->n_kv_heads <= 0 || c->n_heads % c->n_kv_heads != 0)
        return orc_fail(-7, "llama oracle: head_dim must be 64 and heads divisible by kv heads");
    return 0;
}

int orc_llama_step(const orc_llama_cfg* c, const float* const* layers, const float* embed,
                   const float* final_norm, const float* lm_head, float* k_cache,
                   float* v_cache, int32_t pos, int32_t token, float* logits) {
    if (llama_check(c)) return -7;
    if (pos < 0 || pos >= c->max_seq) return orc_fail(-4, "llama oracle: pos out of range");
    int H = c->hidden, nh = c->n_heads, nkv = c->n_kv_heads, F = c->ffn;
    int qd = nh * 64, kd = nkv * 64, group = nh / nkv;
    float* x = (float*)malloc(sizeof(float) * H);
    float* h = (float*)malloc(sizeof(float) * H);
    float* qkv = (float*)malloc(sizeof(float) * (size_t)(qd + 2 * kd));
    float* att = (float*)malloc(sizeof(float) * qd);
    float* tmp = (float*)malloc(sizeof(float) * (size_t)(H > 2 * F ? H : 2 * F));
    float* act = (float*)malloc(sizeof(float) * F);
    float* sc = (float*)malloc(sizeof(float) * (size_t)c->max_seq);
    memcpy(x, embed + (int64_t)token * H, sizeof(float) * H);
    for (int l = 0; l < c->n_layers; ++l) {
        const float* const* L = layers + (size_t)l * 6;
        float* kc = k_cache + (int64_t)l * nkv * c->max_seq * 64;
        float* vc = v_cache + (int64_t)l * nkv * c->max_seq * 64;
        rms_norm_vec(x, L[0], h, H, c->rms_eps);
        matvec(h, L[1], qd + 2 * kd, H, 1, qkv);
        for (int hh = 0; hh < nh; ++hh) rope(qkv + hh * 64, pos, c->rope_theta);
        for (int g = 0; g < nkv; ++g) {
            rope(qkv + qd + g * 64, pos, c->rope_theta);
            memcpy(kc + ((int64_t)g * c->max_seq + pos) * 64, qkv + qd + g * 64, 64 * 4);
            memcpy(vc + ((int64_t)g * c->max_seq + pos) * 64, qkv + qd + kd + g * 64, 64 * 4);
        }
        for (int hh = 0; hh < nh; ++hh) {
            int g = hh / group;
            const float* q = qkv + hh * 64;
            float m = -INFINITY;
            for (int t = 0; t <= pos; ++t) {
                const float* kt = kc + ((int64_t)g * c->max_seq + t) * 64;
                float d = 0.0f;
                for (int i = 0; i < 64; ++i) d = d + q[i] * kt[i];
                sc[t] = d * 0.125f; /* * rsqrt(64) */
                m = fmaxf(m, sc[t]);
            }
            float s = 0.0f;
            for (int t = 0; t <= pos; ++t) {
                sc[t] = expf(sc[t] - m);
                s = s + sc[t];
            }
            for (int i = 0; i < 64; ++i) {
                float o = 0.0f;
                for (int t = 0; t <= pos; ++t)
                    o = o + (sc[t] / s) * vc[((int64_t)g * c->max_seq + t) * 64 + i];
                att[hh * 64 + i] = o;
            }
        }
        matvec(att, L[2], H, qd, 1, tmp);
        for (int i = 0; i < H; ++i) x[i] = x[i] + tmp[i];
        rms_norm_vec(x, L[3], h, H, c->rms_eps);
        matvec(h, L[4], 2 * F, H, 1, tmp);
        for (int i = 0; i < F; ++i) {
            float g = tmp[2 * i], u = tmp[2 * i + 1];
            act[i] = (g * (1.0f / (1.0f + expf(-g)))) * u;
        }
        matvec(act, L[5], H, F, 1, tmp);
        for (int i = 0; i < H; ++i) x[i] = x[i] + tmp[i];
    }
    rms_norm_vec(x, final_norm, h, H, c->rms_eps);
    matvec(h, lm_head, c->vocab, H, 1, logits);
    free(x); free(h); free(qkv); free(att); free(tmp); free(act); free(sc);
    return 0;
}

int orc_llama_full(const orc_llama_cfg* c, const float* const* layers, const float* embed,
                   const float* final_norm, const float* lm_head, const int32_t* tokens,
                   int32_t S, float* logits) {
    /* Full recompute: every position attends to positions <= itself; masked scores get
     * -1e9 before the softmax (build_causal_mask, run_llama_spirv.py:100-107). */
    if (llama_check(c)) return -7;
    int H = c->hidden, nh = c->n_heads, nkv = c->n_kv_heads, F = c->ffn;
    int qd = nh * 64, kd = nkv * 64, group = nh / nkv;
    float* X = (float*)malloc(sizeof(float) * (size_t)S * H);
    float* Hn = (float*)malloc(sizeof(float) * (size_t)S * H);
    float* QKV = (float*)malloc(sizeof(float) * (size_t)S * (qd + 2 * kd));
    float* ATT = (float*)malloc(sizeof(float) * (size_t)S * qd);
    float* T = (float*)malloc(sizeof(float) * (size_t)S * (H > 2 * F ? H : 2 * F));
    float* A = (float*)malloc(sizeof(float) * (size_t)S * F);
    float* sc = (float*)malloc(sizeof(float) * (size_t)S);
    for (int s = 0; s < S; ++s) memcpy(X + (int64_t)s * H, embed + (int64_t)tokens[s] * H, H * 4);
    int W3 = qd + 2 * kd;
    for (int l = 0; l < c->n_layers; ++l) {
        const float* const* L = layers + (size_t)l * 6;
        for (int s = 0; s < S; ++s) {
            rms_norm_vec(X + (int64_t)s * H, L[0], Hn + (int64_t)s * H, H, c->rms_eps);
            matvec(Hn + (int64_t)s * H, L[1], W3, H, 1, QKV + (int64_t)s * W3);
            for (int hh = 0; hh < nh; ++hh) rope(QKV + (int64_t)s * W3 + hh * 64, s, c->rope_theta);
            for (int g = 0; g < nkv; ++g) rope(QKV + (int64_t)s * W3 + qd + g * 64, s, c->rope_theta);
        }
        for (int s = 0; s < S; ++s)
            for (int hh = 0; hh < nh; ++hh) {
                int g = hh / group;
                const float* q = QKV + (int64_t)s * W3 + hh * 64;
                float m = -INFINITY;
                for (int t = 0; t < S; ++t) {
                    const float* kt = QKV + (int64_t)t * W3 + qd + g * 64;
                    float d = 0.0f;
                    for (int i = 0; i < 64; ++i) d = d + q[i] * kt[i];
                    float mask = t > s ? -1e9f : 0.0f;
                    sc[t] = d * 0.125f + mask;
                    m = fmaxf(m, sc[t]);
                }
                float sum = 0.0f;
                for (int t = 0; t < S; ++t) {
                    sc[t] = expf(sc[t] - m);
                    sum = sum + sc[t];
                }
                for (int i = 0; i < 64; ++i) {
                    float o = 0.0f;
                    for (int t = 0; t < S; ++t)
                        o = o + (sc[t] / sum) * QKV[(int64_t)t * W3 + qd + kd + g * 64 + i];
                    ATT[(int64_t)s * qd + hh * 64 + i] = o;
                }
            }
        for (int s = 0; s < S; ++s) {
            matvec(ATT + (int64_t)s * qd, L[2], H, qd, 1, T);
            for (int i = 0; i < H; ++i) X[(int64_t)s * H + i] = X[(int64_t)s * H + i] + T[i];
            rms_norm_vec(X + (int64_t)s * H, L[3], Hn, H, c->rms_eps);
            matvec(Hn, L[4], 2 * F, H, 1, T);
            for (int i = 0; i < F; ++i) {
                float g = T[2 * i], u = T[2 * i + 1];
                A[i] = (g * (1.0f / (1.0f + expf(-g)))) * u;
            }
            matvec(A, L[5], H, F, 1, T);
            for (int i = 0; i < H; ++i) X[(int64_t)s * H + i] = X[(int64_t)s * H + i] + T[i];
        }
    }
    for (int s = 0; s < S; ++s) {
        rms_norm_vec(X + (int64_t)s * H, final_norm, Hn, H, c->rms_eps);
        matvec(Hn, lm_head, c->vocab, H, 1, logits + (int64_t)s * c->vocab);
    }
    free(X); free(Hn); free(QKV); free(ATT); free(T); free(A); free(sc);
    return 0;
}
