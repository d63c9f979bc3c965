// Batch-1 decode kernels: HBM-bound GEMV with fused RMSNorm / SwiGLU / residual, RoPE +
// KV-cache attention, embedding gather and greedy argmax.
//
// The reference has no decode kernel: TinyLlama runs as a full S=64 recompute of the HLO
// graph per token (source/xla_hlo/tools/run_llama_spirv.py:194-295), i.e. M=64 GEMMs over
// weights re-read from disk.  The math restated here is export_llama.py:284-375:
//   rms_norm(x, w) = x * rsqrt(mean(x^2) + eps) * w                  (:284-286)
//   q,k,v = h @ Wq, h @ Wk, h @ Wv; RoPE rotate-half on q and k      (:288-296, 319-331)
//   GQA: each KV head serves n_heads/n_kv query heads                (:333-343)
//   scores = (q . k) * rsqrt(64) + mask; softmax; @ v                (:346-350)
//   x += att @ Wo; x += (silu(h @ Wg) * (h @ Wu)) @ Wd                (:355-372)
// with a KV cache instead of the recompute, so one token reads every weight once.
#include "decode.h"

namespace {

using shp::DecodeState;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

typedef float nfloat4 __attribute__((ext_vector_type(4)));

// Streaming 16-byte load: weights are read exactly once per token, so keep them from
// displacing the staged vectors and KV cache in the caches.
__device__ __forceinline__ float4 ld_stream4(const float* p) {
    nfloat4 v = __builtin_nontemporal_load(reinterpret_cast<const nfloat4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// Dot product of one weight row (K floats, 16-byte aligned, K % 4 == 0) with the staged
// vector in LDS.  Eight 16-byte loads are issued before they are consumed so a wavefront
// keeps 8 KiB in flight.
__device__ __forceinline__ float row_dot(const float* __restrict__ row, const float* vs, int K,
                                         int lane) {
    float acc = 0.0f;
    int k = lane * 4;
    for (; k + 7 * 256 < K; k += 8 * 256) {
        float4 w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) w[u] = ld_stream4(row + k + u * 256);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            float4 v = *reinterpret_cast<const float4*>(vs + k + u * 256);
            acc += w[u].x * v.x + w[u].y * v.y + w[u].z * v.z + w[u].w * v.w;
        }
    }
    for (; k < K; k += 256) {
        float4 w = ld_stream4(row + k);
        float4 v = *reinterpret_cast<const float4*>(vs + k);
        acc += w.x * v.x + w.y * v.y + w.z * v.z + w.w * v.w;
    }
    return wave_sum(acc);
}

template <int MODE, bool NORM>
__global__ __launch_bounds__(256) void gemv_kernel(const float* __restrict__ x,
                                                   const float* __restrict__ norm_w, float eps,
                                                   const float* __restrict__ W, int rows_out,
                                                   int K, float* y, const float* residual) {
    extern __shared__ __attribute__((aligned(16))) float vs[];
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if constexpr (NORM) {
        float ss = 0.0f;
        for (int k = tid; k < K; k += 256) ss += x[k] * x[k];
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float tot = red[0] + red[1] + red[2] + red[3];
        float inv = 1.0f / sqrtf(tot / (float)K + eps);
        for (int k = tid; k < K; k += 256) vs[k] = (x[k] * inv) * norm_w[k];
    } else {
        for (int k = tid; k < K; k += 256) vs[k] = x[k];
    }
    __syncthreads();
    const int nw = gridDim.x * 4;
    for (int r = blockIdx.x * 4 + wave; r < rows_out; r += nw) {
        if constexpr (MODE == shp::GEMV_SWIGLU) {
            float g = row_dot(W + (int64_t)(2 * r) * K, vs, K, lane);
            float u = row_dot(W + (int64_t)(2 * r + 1) * K, vs, K, lane);
            if (lane == 0) y[r] = (g * (1.0f / (1.0f + expf(-g)))) * u;
        } else {
            float d = row_dot(W + (int64_t)r * K, vs, K, lane);
            if (lane == 0) y[r] = residual ? residual[r] + d : d;
        }
    }
}

__global__ void embed_kernel(const float* __restrict__ embed, int hidden,
                             const DecodeState* __restrict__ st, float* __restrict__ x) {
    const float* row = embed + (int64_t)st->token * hidden;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
        x[i] = row[i];
}

// One wavefront per query head; head_dim must be 64 (one element per lane).
__global__ __launch_bounds__(64) void attention_decode_kernel(
    const float* __restrict__ qkv, float* __restrict__ k_cache, float* __restrict__ v_cache,
    int n_heads, int n_kv, int max_seq, float theta, const DecodeState* __restrict__ st,
    float* __restrict__ out) {
    extern __shared__ float ps[];  // [max_seq] probabilities
    __shared__ float qs[64], ks[64];
    const int h = blockIdx.x, lane = threadIdx.x;
    const int group = n_heads / n_kv;
    const int g = h / group;
    const int pos = st->pos;
    // RoPE (rotate-half): out = x*cos + rotate_half(x)*sin, angle = pos * theta^(-2j/64)
    const int j = lane & 31;
    const float inv_freq = 1.0f / powf(theta, (float)(2 * j) / 64.0f);
    const float ang = (float)pos * inv_freq;
    const float c = cosf(ang), s = sinf(ang);
    float q = qkv[h * 64 + lane];
    float qp = __shfl_xor(q, 32);
    float qr = q * c + (lane < 32 ? -qp : qp) * s;
    float k = qkv[n_heads * 64 + g * 64 + lane];
    float kp = __shfl_xor(k, 32);
    float kr = k * c + (lane < 32 ? -kp : kp) * s;
    float v = qkv[(n_heads + n_kv) * 64 + g * 64 + lane];
    qs[lane] = qr;
    ks[lane] = kr;
    float* kc = k_cache + (int64_t)g * max_seq * 64;
    float* vc = v_cache + (int64_t)g * max_seq * 64;
    if (h % group == 0) {
        kc[(int64_t)pos * 64 + lane] = kr;
        vc[(int64_t)pos * 64 + lane] = v;
    }
    __syncthreads();
    // scores: lane t handles keys t, t+64, ...
    float m = -3.4028234663852886e+38f;
    for (int t = lane; t <= pos; t += 64) {
        const float* kr_t = (t == pos) ? ks : kc + (int64_t)t * 64;
        float d = 0.0f;
#pragma unroll 16
        for (int i = 0; i < 64; ++i) d += qs[i] * kr_t[i];
        d *= 0.125f;
        ps[t] = d;
        m = fmaxf(m, d);
    }
    m = wave_max(m);
    float sum = 0.0f;
    for (int t = lane; t <= pos; t += 64) {
        float e = expf(ps[t] - m);
        ps[t] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    __syncthreads();
    float o = 0.0f;
    for (int t = 0; t <= pos; ++t) {
        float vt = (t == pos) ? v : vc[(int64_t)t * 64 + lane];
        o += (ps[t] / sum) * vt;
    }
    out[h * 64 + lane] = o;
}

__global__ __launch_bounds__(1024) void argmax_advance_kernel(const float* __restrict__ logits,
                                                              int n, DecodeState* st) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    float best = -3.4028234663852886e+38f;
    int idx = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += 1024) {
        float v = logits[i];
        if (v > best) { best = v; idx = i; }
    }
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(best, o);
        int oi = __shfl_xor(idx, o);
        if (ov > best || (ov == best && oi < idx)) { best = ov; idx = oi; }
    }
    if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = best; bi[threadIdx.x >> 6] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w)
            if (bv[w] > best || (bv[w] == best && bi[w] < idx)) { best = bv[w]; idx = bi[w]; }
        if (idx == 0x7fffffff) idx = 0;
        st->token = idx;
        if (st->step < 4096) st->out_tokens[st->step] = idx;
        st->step += 1;
        st->pos += 1;
    }
}

// argmax_rows (registry): out[r] = lowest index of the row maximum, stored as int32.
__global__ __launch_bounds__(256) void argmax_rows_kernel(const float* __restrict__ x,
                                                          int32_t* __restrict__ out, int rows,
                                                          int cols) {
    int lane = threadIdx.x & 63;
    for (int r = blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += gridDim.x * 4) {
        const float* xr = x + (int64_t)r * cols;
        float best = -3.4028234663852886e+38f;
        int idx = 0x7fffffff;
        for (int i = lane; i < cols; i += 64) {
            float v = xr[i];
            if (v > best) { best = v; idx = i; }
        }
        for (int o = 32; o > 0; o >>= 1) {
            float ov = __shfl_xor(best, o);
            int oi = __shfl_xor(idx, o);
            if (ov > best || (ov == best && oi < idx)) { best = ov; idx = oi; }
        }
        if (lane == 0) out[r] = idx == 0x7fffffff ? 0 : idx;
    }
}

// gemv_nt (registry): y[n] = act(sum_k x[k] W[n][k] + bias[n] + residual[n])
__global__ __launch_bounds__(256) void gemv_nt_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ W, int N, int K,
                                                      float* __restrict__ y,
                                                      const float* __restrict__ bias,
                                                      const float* __restrict__ residual,
                                                      int act, float alpha) {
    int lane = threadIdx.x & 63;
    for (int r = blockIdx.x * 4 + (threadIdx.x >> 6); r < N; r += gridDim.x * 4) {
        const float* row = W + (int64_t)r * K;
        float acc = 0.0f;
        for (int k = lane; k < K; k += 64) acc += row[k] * x[k];
        acc = wave_sum(acc);
        if (lane == 0) {
            float v = acc + (bias ? bias[r] : 0.0f) + (residual ? residual[r] : 0.0f);
            y[r] = shpd::apply_act(v, act, alpha);
        }
    }
}

int launch_gemv_nt(const shp::Launch& l) {
    if (l.n_push < 2) return shp::fail(SHP_ERR_PUSH, "gemv_nt needs push {N, K}");
    int N = l.push[0], K = l.push[1];
    if (N <= 0 || K < 0) return shp::fail(SHP_ERR_SHAPE, "gemv_nt: dims");
    int rc = shp::check_total(l, N, "gemv_nt");
    if (rc) return rc;
    bool fast = K % 4 == 0 && K > 0 && ((uintptr_t)l.in0 & 15) == 0 &&
                ((uintptr_t)l.in1 & 15) == 0 && !l.epi->bias && l.epi->act == SHP_ACT_NONE &&
                (size_t)K * 4 <= 64 * 1024;
    if (fast)
        return shp::gemv_launch(l.stream, (const float*)l.in0, nullptr, 0.0f,
                                (const float*)l.in1, N, K, shp::GEMV_PLAIN, (float*)l.out,
                                l.epi->residual);
    unsigned g = (unsigned)std::min(1024, (N + 3) / 4);
    hipLaunchKernelGGL(gemv_nt_kernel, dim3(g), dim3(256), 0, l.stream, (const float*)l.in0,
                       (const float*)l.in1, N, K, (float*)l.out, l.epi->bias, l.epi->residual,
                       l.epi->act, l.epi->alpha);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

int launch_argmax_rows(const shp::Launch& l) {
    if (l.n_push < 2) return shp::fail(SHP_ERR_PUSH, "argmax_rows needs push {rows, cols}");
    int rows = l.push[0], cols = l.push[1];
    if (rows <= 0 || cols <= 0) return shp::fail(SHP_ERR_SHAPE, "argmax_rows: dims");
    int rc = shp::check_total(l, rows, "argmax_rows");
    if (rc) return rc;
    unsigned g = (unsigned)std::min(4096, (rows + 3) / 4);
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(g), dim3(256), 0, l.stream, (const float*)l.in0,
                       (int32_t*)l.out, rows, cols);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

}  // namespace

namespace shp {

int gemv_launch(hipStream_t s, const float* x, const float* norm_w, float eps, const float* w,
                int rows, int K, int mode, float* y, const float* residual) {
    if (rows <= 0 || K <= 0 || K % 4 != 0)
        return fail(SHP_ERR_SHAPE, "gemv: rows > 0 and K % 4 == 0 required");
    if (((uintptr_t)w & 15) != 0) return fail(SHP_ERR_INVALID, "gemv: weights not 16B aligned");
    size_t lds = (size_t)K * sizeof(float);
    if (lds > 64 * 1024) return fail(SHP_ERR_UNSUPPORTED, "gemv: K too large for LDS staging");
    int rows_out = mode == GEMV_SWIGLU ? rows / 2 : rows;
    unsigned g = (unsigned)std::min(1024, (rows_out + 3) / 4);
    if (mode == GEMV_SWIGLU) {
        if (norm_w)
            hipLaunchKernelGGL((gemv_kernel<GEMV_SWIGLU, true>), dim3(g), dim3(256), lds, s, x,
                               norm_w, eps, w, rows_out, K, y, residual);
        else
            hipLaunchKernelGGL((gemv_kernel<GEMV_SWIGLU, false>), dim3(g), dim3(256), lds, s, x,
                               norm_w, eps, w, rows_out, K, y, residual);
    } else {
        if (norm_w)
            hipLaunchKernelGGL((gemv_kernel<GEMV_PLAIN, true>), dim3(g), dim3(256), lds, s, x,
                               norm_w, eps, w, rows_out, K, y, residual);
        else
            hipLaunchKernelGGL((gemv_kernel<GEMV_PLAIN, false>), dim3(g), dim3(256), lds, s, x,
                               norm_w, eps, w, rows_out, K, y, residual);
    }
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

int embed_launch(hipStream_t s, const float* embed, int hidden, const DecodeState* st, float* x) {
    hipLaunchKernelGGL(embed_kernel, dim3((hidden + 255) / 256), dim3(256), 0, s, embed, hidden, st,
                       x);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

int attention_decode_launch(hipStream_t s, const float* qkv, float* k_cache, float* v_cache,
                            int n_heads, int n_kv, int head_dim, int max_seq, float theta,
                            const DecodeState* st, float* out) {
    if (head_dim != 64) return fail(SHP_ERR_UNSUPPORTED, "attention_decode: head_dim must be 64");
    if (n_kv <= 0 || n_heads % n_kv != 0) return fail(SHP_ERR_SHAPE, "attention_decode: heads");
    size_t lds = (size_t)max_seq * sizeof(float);
    hipLaunchKernelGGL(attention_decode_kernel, dim3(n_heads), dim3(64), lds, s, qkv, k_cache,
                       v_cache, n_heads, n_kv, max_seq, theta, st, out);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

__global__ void set_token_kernel(DecodeState* st, int32_t token) { st->token = token; }

int set_token_launch(hipStream_t s, DecodeState* st, int32_t token) {
    hipLaunchKernelGGL(set_token_kernel, dim3(1), dim3(1), 0, s, st, token);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

int argmax_advance_launch(hipStream_t s, const float* logits, int n, DecodeState* st) {
    hipLaunchKernelGGL(argmax_advance_kernel, dim3(1), dim3(1024), 0, s, logits, n, st);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

KernelEntry kDecodeKernels[] = {
    {"gemv_nt", 2, true, launch_gemv_nt},
    {"argmax_rows", 2, false, launch_argmax_rows},
};
const int kDecodeKernelCount = sizeof(kDecodeKernels) / sizeof(kDecodeKernels[0]);

}  // namespace shp
