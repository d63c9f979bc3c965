// Elementwise, data-movement and fill kernels.
//
// Reference kernels restated here (semantics and push layouts unchanged):
//   unary   kernels/{abs,exp,log,neg,sqrt,rsqrt,sigmoid,tanh,relu,relu6,sine,reshape}/glsl/*.comp
//   leaky   kernels/leaky_relu/glsl/leaky_relu.comp:17 (max(alpha*x, x), alpha as f32 bits)
//   binary  kernels/{add,sub,mul,div,pow,min,max}/glsl/*.comp (push: total)
//   concat  kernels/concat/glsl/concat.comp:13-17 (push: a_total, total)
//   pad     kernels/pad/glsl/pad.comp:15-45 (13 i32, pad value = in1[0])
//   transpose kernels/transpose/glsl/transpose.comp:31-52 (13 i32)
//   l2norm  kernels/l2norm/glsl/l2norm.comp:13-18 (norm passed as f32 bits)
// The reference runs one invocation per element with 128-wide groups; here each thread
// handles 4 consecutive elements with 16-byte loads where the buffers allow it, in a
// grid-stride loop sized for 256 CUs.
#include "common.h"

namespace {

enum UnaryOp {
    U_ABS, U_EXP, U_LOG, U_NEG, U_SQRT, U_RSQRT, U_SIGMOID, U_TANH, U_RELU, U_RELU6,
    U_SINE, U_COPY, U_LEAKY, U_SILU, U_GELU, U_COS, U_FLOOR, U_CEIL
};
enum BinaryOp { B_ADD, B_SUB, B_MUL, B_DIV, B_POW, B_MIN, B_MAX, B_REM };

template <int OP>
__device__ __forceinline__ float unary_op(float x, float alpha) {
    if constexpr (OP == U_ABS) return fabsf(x);
    if constexpr (OP == U_EXP) return expf(x);
    if constexpr (OP == U_LOG) return logf(x);
    if constexpr (OP == U_NEG) return -x;
    if constexpr (OP == U_SQRT) return sqrtf(x);
    if constexpr (OP == U_RSQRT) return 1.0f / sqrtf(x);
    if constexpr (OP == U_SIGMOID) return 1.0f / (1.0f + expf(-x));
    if constexpr (OP == U_TANH) return shpd::apply_act(x, SHP_ACT_TANH, 0.0f);
    if constexpr (OP == U_RELU) return fmaxf(x, 0.0f);
    if constexpr (OP == U_RELU6) return fminf(fmaxf(x, 0.0f), 6.0f);
    if constexpr (OP == U_SINE) return sinf(x);
    if constexpr (OP == U_COPY) return x;
    if constexpr (OP == U_LEAKY) return fmaxf(alpha * x, x);
    if constexpr (OP == U_SILU) return x * (1.0f / (1.0f + expf(-x)));
    if constexpr (OP == U_GELU) return shpd::apply_act(x, SHP_ACT_GELU_ERF, 0.0f);
    if constexpr (OP == U_COS) return cosf(x);
    if constexpr (OP == U_FLOOR) return floorf(x);
    if constexpr (OP == U_CEIL) return ceilf(x);
    return x;
}

template <int OP>
__device__ __forceinline__ float binary_op(float a, float b) {
    if constexpr (OP == B_ADD) return a + b;
    if constexpr (OP == B_SUB) return a - b;
    if constexpr (OP == B_MUL) return a * b;
    if constexpr (OP == B_DIV) return a / b;
    if constexpr (OP == B_POW) return powf(a, b);
    if constexpr (OP == B_MIN) return fminf(a, b);
    if constexpr (OP == B_MAX) return fmaxf(a, b);
    if constexpr (OP == B_REM) return fmodf(a, b);
    return a;
}

constexpr int kBlock = 256;

inline unsigned ew_grid(uint64_t n4) {
    // Enough groups to cover the vectorised range, capped to a few waves per CU.
    uint64_t g = (n4 + kBlock - 1) / kBlock;
    if (g > 256 * 16) g = 256 * 16;
    return g == 0 ? 1u : (unsigned)g;
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The vectorised streams: every thread moves kUnroll float4 per iteration, all loads issued
// before the first store, so a wavefront keeps kUnroll 1 KiB requests in flight.  Streams of at
// least kNtElems elements per operand use non-temporal loads and stores (they do not fit the
// caches the next op would read them from).  On MI355X: 6.3-6.5 TB/s for a 256 MiB copy or add
// against 5.0-5.2 with one float4 per iteration.
constexpr int kUnroll = 4;
constexpr uint64_t kNtElems = 8ull << 20;  // 32 MiB of floats
typedef float ew4 __attribute__((ext_vector_type(4)));

inline unsigned ew_grid_vec(uint64_t n4) {
    uint64_t g = (n4 + kBlock * kUnroll - 1) / (kBlock * kUnroll);
    if (g > 256 * 32) g = 256 * 32;
    return g == 0 ? 1u : (unsigned)g;
}

template <bool NT>
__device__ __forceinline__ ew4 ew_load(const ew4* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}
template <bool NT>
__device__ __forceinline__ void ew_store(ew4 v, ew4* p) {
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

template <int OP, bool VEC, bool NT = false>
__global__ __launch_bounds__(kBlock) void unary_kernel(const float* __restrict__ x,
                                                       float* __restrict__ y, uint64_t n,
                                                       float alpha) {
    uint64_t tid = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    uint64_t stride = (uint64_t)gridDim.x * kBlock;
    if constexpr (VEC) {
        uint64_t n4 = n >> 2;
        const ew4* x4 = reinterpret_cast<const ew4*>(x);
        ew4* y4 = reinterpret_cast<ew4*>(y);
        for (uint64_t b0 = (uint64_t)blockIdx.x * kBlock * kUnroll + threadIdx.x; b0 < n4;
             b0 += stride * kUnroll) {
            ew4 v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
                if (b0 + u * kBlock < n4) v[u] = ew_load<NT>(x4 + b0 + u * kBlock);
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                if (b0 + u * kBlock >= n4) continue;
                ew4 r;
#pragma unroll
                for (int c = 0; c < 4; ++c) r[c] = unary_op<OP>(v[u][c], alpha);
                ew_store<NT>(r, y4 + b0 + u * kBlock);
            }
        }
        for (uint64_t i = (n4 << 2) + tid; i < n; i += stride) y[i] = unary_op<OP>(x[i], alpha);
    } else {
        for (uint64_t i = tid; i < n; i += stride) y[i] = unary_op<OP>(x[i], alpha);
    }
}

template <int OP, bool VEC, bool NT = false>
__global__ __launch_bounds__(kBlock) void binary_kernel(const float* __restrict__ a,
                                                        const float* __restrict__ b,
                                                        float* __restrict__ y, uint64_t n) {
    uint64_t tid = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    uint64_t stride = (uint64_t)gridDim.x * kBlock;
    if constexpr (VEC) {
        uint64_t n4 = n >> 2;
        const ew4* a4 = reinterpret_cast<const ew4*>(a);
        const ew4* b4 = reinterpret_cast<const ew4*>(b);
        ew4* y4 = reinterpret_cast<ew4*>(y);
        for (uint64_t b0 = (uint64_t)blockIdx.x * kBlock * kUnroll + threadIdx.x; b0 < n4;
             b0 += stride * kUnroll) {
            ew4 u4[kUnroll], v4[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
                if (b0 + u * kBlock < n4) {
                    u4[u] = ew_load<NT>(a4 + b0 + u * kBlock);
                    v4[u] = ew_load<NT>(b4 + b0 + u * kBlock);
                }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                if (b0 + u * kBlock >= n4) continue;
                ew4 r;
#pragma unroll
                for (int c = 0; c < 4; ++c) r[c] = binary_op<OP>(u4[u][c], v4[u][c]);
                ew_store<NT>(r, y4 + b0 + u * kBlock);
            }
        }
        for (uint64_t i = (n4 << 2) + tid; i < n; i += stride) y[i] = binary_op<OP>(a[i], b[i]);
    } else {
        for (uint64_t i = tid; i < n; i += stride) y[i] = binary_op<OP>(a[i], b[i]);
    }
}

template <int OP>
int launch_unary_n(hipStream_t s, const float* x, float* y, uint64_t n, float alpha) {
    bool vec = aligned16(x) && aligned16(y);
    if (vec && n >= kNtElems)
        hipLaunchKernelGGL((unary_kernel<OP, true, true>), dim3(ew_grid_vec(n / 4)), dim3(kBlock),
                           0, s, x, y, n, alpha);
    else if (vec)
        hipLaunchKernelGGL((unary_kernel<OP, true>), dim3(ew_grid_vec(n / 4)), dim3(kBlock), 0,
                           s, x, y, n, alpha);
    else
        hipLaunchKernelGGL((unary_kernel<OP, false>), dim3(ew_grid(n)), dim3(kBlock), 0, s, x, y,
                           n, alpha);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

template <int OP>
int launch_unary(const shp::Launch& l) {
    if (l.n_push < 1) return shp::fail(SHP_ERR_PUSH, "unary kernel needs push[0]=total");
    int rc = shp::check_total(l, l.push[0], "unary");
    if (rc) return rc;
    float alpha = 0.0f;
    if constexpr (OP == U_LEAKY) {
        if (l.n_push < 2) return shp::fail(SHP_ERR_PUSH, "leaky_relu needs push[1]=alpha_bits");
        int32_t bits = l.push[1];
        memcpy(&alpha, &bits, 4);
    }
    return launch_unary_n<OP>(l.stream, (const float*)l.in0, (float*)l.out, l.out_elems, alpha);
}

template <int OP>
int launch_binary(const shp::Launch& l) {
    if (l.n_push < 1) return shp::fail(SHP_ERR_PUSH, "binary kernel needs push[0]=total");
    int rc = shp::check_total(l, l.push[0], "binary");
    if (rc) return rc;
    const float* a = (const float*)l.in0;
    const float* b = (const float*)l.in1;
    float* y = (float*)l.out;
    uint64_t n = l.out_elems;
    const bool vec = aligned16(a) && aligned16(b) && aligned16(y);
    if (vec && n >= kNtElems)
        hipLaunchKernelGGL((binary_kernel<OP, true, true>), dim3(ew_grid_vec(n / 4)), dim3(kBlock),
                           0, l.stream, a, b, y, n);
    else if (vec)
        hipLaunchKernelGGL((binary_kernel<OP, true>), dim3(ew_grid_vec(n / 4)), dim3(kBlock), 0,
                           l.stream, a, b, y, n);
    else
        hipLaunchKernelGGL((binary_kernel<OP, false>), dim3(ew_grid(n)), dim3(kBlock), 0,
                           l.stream, a, b, y, n);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- concat (concat.comp:13-17): flat A||B ------------------------------------------
__global__ __launch_bounds__(kBlock) void concat_kernel(const float* __restrict__ a,
                                                        const float* __restrict__ b,
                                                        float* __restrict__ y, uint64_t a_total,
                                                        uint64_t total) {
    uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += stride)
        y[i] = i < a_total ? a[i] : b[i - a_total];
}

int launch_concat(const shp::Launch& l) {
    if (l.n_push < 2) return shp::fail(SHP_ERR_PUSH, "concat needs push {a_total, total}");
    int rc = shp::check_total(l, l.push[1], "concat");
    if (rc) return rc;
    if (l.push[0] < 0 || l.push[0] > l.push[1])
        return shp::fail(SHP_ERR_SHAPE, "concat: a_total outside [0, total]");
    hipLaunchKernelGGL(concat_kernel, dim3(ew_grid(l.out_elems)), dim3(kBlock), 0, l.stream,
                       (const float*)l.in0, (const float*)l.in1, (float*)l.out,
                       (uint64_t)l.push[0], l.out_elems);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- pad (pad.comp:15-45): rank<=4 constant pad, low pads only, value = in1[0] -------
struct Pad4 {
    int od[4], id[4], pl[4];
};

__global__ __launch_bounds__(kBlock) void pad_kernel(const float* __restrict__ x,
                                                     const float* __restrict__ pad_value,
                                                     float* __restrict__ y, Pad4 p,
                                                     uint64_t total) {
    uint64_t stride = (uint64_t)gridDim.x * kBlock;
    float pv = pad_value[0];
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += stride) {
        uint64_t r = i;
        int c3 = (int)(r % p.od[3]); r /= p.od[3];
        int c2 = (int)(r % p.od[2]); r /= p.od[2];
        int c1 = (int)(r % p.od[1]); r /= p.od[1];
        int c0 = (int)r;
        int s0 = c0 - p.pl[0], s1 = c1 - p.pl[1], s2 = c2 - p.pl[2], s3 = c3 - p.pl[3];
        float v = pv;
        if (s0 >= 0 && s0 < p.id[0] && s1 >= 0 && s1 < p.id[1] && s2 >= 0 && s2 < p.id[2] &&
            s3 >= 0 && s3 < p.id[3])
            v = x[(((uint64_t)s0 * p.id[1] + s1) * p.id[2] + s2) * p.id[3] + s3];
        y[i] = v;
    }
}

int launch_pad(const shp::Launch& l) {
    if (l.n_push < 13) return shp::fail(SHP_ERR_PUSH, "pad needs 13 push constants");
    int rc = shp::check_total(l, l.push[12], "pad");
    if (rc) return rc;
    Pad4 p;
    int64_t prod = 1;
    for (int i = 0; i < 4; ++i) {
        p.od[i] = l.push[i];
        p.id[i] = l.push[4 + i];
        p.pl[i] = l.push[8 + i];
        if (p.od[i] <= 0 || p.id[i] <= 0) return shp::fail(SHP_ERR_SHAPE, "pad: non-positive dim");
        prod *= p.od[i];
    }
    if (prod != l.push[12]) return shp::fail(SHP_ERR_SHAPE, "pad: total != prod(out dims)");
    hipLaunchKernelGGL(pad_kernel, dim3(ew_grid(l.out_elems)), dim3(kBlock), 0, l.stream,
                       (const float*)l.in0, (const float*)l.in1, (float*)l.out, p, l.out_elems);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- transpose (transpose.comp:31-52): out coordinate o_k feeds input axis perm[k] ---
struct Tr4 {
    int in[4], out[4], perm[4];
};

__global__ __launch_bounds__(kBlock) void transpose_kernel(const float* __restrict__ x,
                                                           float* __restrict__ y, Tr4 t,
                                                           uint64_t total) {
    uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += stride) {
        uint64_t r = i;
        int o[4];
        o[3] = (int)(r % t.out[3]); r /= t.out[3];
        o[2] = (int)(r % t.out[2]); r /= t.out[2];
        o[1] = (int)(r % t.out[1]); r /= t.out[1];
        o[0] = (int)r;
        int c[4] = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            int a = t.perm[k];
            if (a == 0) c[0] = o[k];
            if (a == 1) c[1] = o[k];
            if (a == 2) c[2] = o[k];
            if (a == 3) c[3] = o[k];
        }
        y[i] = x[(((uint64_t)c[0] * t.in[1] + c[1]) * t.in[2] + c[2]) * t.in[3] + c[3]];
    }
}

// Tiled path for the common "swap the last two axes" / NCHW<->NHWC permutations: a
// 64x64 tile through LDS so both the read and the write are coalesced.
__global__ __launch_bounds__(256) void transpose_last2_kernel(const float* __restrict__ x,
                                                              float* __restrict__ y, int rows,
                                                              int cols, int batch) {
    __shared__ float tile[64][65];
    int b = blockIdx.z;
    int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    const float* xb = x + (uint64_t)b * rows * cols;
    float* yb = y + (uint64_t)b * rows * cols;
    int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        int r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) tile[i][tx] = xb[(uint64_t)r * cols + c];
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        int c = c0 + i, r = r0 + tx;
        if (r < rows && c < cols) yb[(uint64_t)c * rows + r] = tile[tx][i];
    }
}

int launch_transpose(const shp::Launch& l) {
    if (l.n_push < 13) return shp::fail(SHP_ERR_PUSH, "transpose needs 13 push constants");
    int rc = shp::check_total(l, l.push[12], "transpose");
    if (rc) return rc;
    Tr4 t;
    int64_t pin = 1, pout = 1;
    int seen = 0;
    for (int i = 0; i < 4; ++i) {
        t.in[i] = l.push[i];
        t.out[i] = l.push[4 + i];
        t.perm[i] = l.push[8 + i];
        if (t.in[i] <= 0 || t.out[i] <= 0 || t.perm[i] < 0 || t.perm[i] > 3)
            return shp::fail(SHP_ERR_SHAPE, "transpose: bad dims or permutation");
        seen |= 1 << t.perm[i];
        pin *= t.in[i];
        pout *= t.out[i];
    }
    if (seen != 15 || pin != pout || pout != l.push[12])
        return shp::fail(SHP_ERR_SHAPE, "transpose: permutation/dims inconsistent");
    for (int k = 0; k < 4; ++k)
        if (t.out[k] != t.in[t.perm[k]])
            return shp::fail(SHP_ERR_SHAPE, "transpose: out dims != permuted in dims");
    // Collapse to batch x (rows x cols) -> (cols x rows) when the permutation swaps two
    // trailing groups of axes while keeping a leading group in place.
    int p0 = t.perm[0], p1 = t.perm[1], p2 = t.perm[2], p3 = t.perm[3];
    int batch = 0, rows = 0, cols = 0;
    if (p0 == 0 && p1 == 1 && p2 == 3 && p3 == 2) {
        batch = t.in[0] * t.in[1]; rows = t.in[2]; cols = t.in[3];
    } else if (p0 == 0 && p1 == 2 && p2 == 3 && p3 == 1) {  // NCHW -> NHWC
        batch = t.in[0]; rows = t.in[1]; cols = t.in[2] * t.in[3];
    } else if (p0 == 0 && p1 == 3 && p2 == 1 && p3 == 2) {  // NHWC -> NCHW
        batch = t.in[0]; rows = t.in[1] * t.in[2]; cols = t.in[3];
    } else if (p0 == 1 && p1 == 0 && p2 == 2 && p3 == 3 && t.in[2] * t.in[3] == 1) {
        batch = 1; rows = t.in[0]; cols = t.in[1];
    }
    if (batch > 0 && batch < 65536) {
        dim3 grid((cols + 63) / 64, (rows + 63) / 64, batch);
        hipLaunchKernelGGL(transpose_last2_kernel, grid, dim3(256), 0, l.stream,
                           (const float*)l.in0, (float*)l.out, rows, cols, batch);
    } else {
        hipLaunchKernelGGL(transpose_kernel, dim3(ew_grid(l.out_elems)), dim3(kBlock), 0,
                           l.stream, (const float*)l.in0, (float*)l.out, t, l.out_elems);
    }
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- l2norm (l2norm.comp:13-18): out = x / max(norm, 1e-12), norm from push bits ----
__global__ __launch_bounds__(kBlock) void l2norm_scale_kernel(const float* __restrict__ x,
                                                              float* __restrict__ y, uint64_t n,
                                                              float norm) {
    uint64_t stride = (uint64_t)gridDim.x * kBlock;
    float d = fmaxf(norm, 1.0e-12f);
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        y[i] = x[i] / d;
}

int launch_l2norm(const shp::Launch& l) {
    if (l.n_push < 2) return shp::fail(SHP_ERR_PUSH, "l2norm needs push {total, norm_bits}");
    int rc = shp::check_total(l, l.push[0], "l2norm");
    if (rc) return rc;
    float norm;
    int32_t bits = l.push[1];
    memcpy(&norm, &bits, 4);
    hipLaunchKernelGGL(l2norm_scale_kernel, dim3(ew_grid(l.out_elems)), dim3(kBlock), 0,
                       l.stream, (const float*)l.in0, (float*)l.out, l.out_elems, norm);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- l2_normalization (native): the reference computes ||x|| on the CPU
// (scheduler.rs:816) and passes it as push bits; here one 1024-thread group reduces the
// sum of squares in fp32 and scales in the same launch.  push: {total}.
__global__ __launch_bounds__(1024) void l2_normalization_kernel(const float* __restrict__ x,
                                                                float* __restrict__ y,
                                                                uint64_t n) {
    __shared__ float red[16];
    float acc = 0.0f;
    for (uint64_t i = threadIdx.x; i < n; i += 1024) acc += x[i] * x[i];
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x < 64) {
        float v = threadIdx.x < 16 ? red[threadIdx.x] : 0.0f;
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
        if (threadIdx.x == 0) red[0] = v;
    }
    __syncthreads();
    float d = fmaxf(sqrtf(red[0]), 1.0e-12f);
    for (uint64_t i = threadIdx.x; i < n; i += 1024) y[i] = x[i] / d;
}

int launch_l2_normalization(const shp::Launch& l) {
    if (l.n_push < 1) return shp::fail(SHP_ERR_PUSH, "l2_normalization needs push {total}");
    int rc = shp::check_total(l, l.push[0], "l2_normalization");
    if (rc) return rc;
    hipLaunchKernelGGL(l2_normalization_kernel, dim3(1), dim3(1024), 0, l.stream,
                       (const float*)l.in0, (float*)l.out, l.out_elems);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- broadcast_binary (native): c = a op b with stride-0 broadcast over rank<=4.
// Replaces the CPU broadcast_tensor + equal-size dispatch of compiler.rs:705-729,1361-1393.
// push: {op, total, d0,d1,d2,d3, as0,as1,as2,as3, bs0,bs1,bs2,bs3} (element strides).
struct Bcast {
    int op;
    int d[4];
    int64_t as[4], bs[4];
};

__global__ __launch_bounds__(kBlock) void broadcast_binary_kernel(const float* __restrict__ a,
                                                                  const float* __restrict__ b,
                                                                  float* __restrict__ y, Bcast p,
                                                                  uint64_t total) {
    uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += stride) {
        uint64_t r = i;
        int64_t ai = 0, bi = 0;
#pragma unroll
        for (int k = 3; k >= 0; --k) {
            int c = (int)(r % p.d[k]);
            r /= p.d[k];
            ai += c * p.as[k];
            bi += c * p.bs[k];
        }
        float u = a[ai], v = b[bi], o;
        switch (p.op) {
            case B_ADD: o = u + v; break;
            case B_SUB: o = u - v; break;
            case B_MUL: o = u * v; break;
            case B_DIV: o = u / v; break;
            case B_POW: o = powf(u, v); break;
            case B_MIN: o = fminf(u, v); break;
            case B_MAX: o = fmaxf(u, v); break;
            default: o = fmodf(u, v); break;
        }
        y[i] = o;
    }
}

int launch_broadcast_binary(const shp::Launch& l) {
    if (l.n_push < 14) return shp::fail(SHP_ERR_PUSH, "broadcast_binary needs 14 push constants");
    int rc = shp::check_total(l, l.push[1], "broadcast_binary");
    if (rc) return rc;
    Bcast p;
    p.op = l.push[0];
    if (p.op < B_ADD || p.op > B_REM) return shp::fail(SHP_ERR_INVALID, "broadcast_binary: op");
    int64_t prod = 1;
    for (int k = 0; k < 4; ++k) {
        p.d[k] = l.push[2 + k];
        p.as[k] = l.push[6 + k];
        p.bs[k] = l.push[10 + k];
        if (p.d[k] <= 0 || p.as[k] < 0 || p.bs[k] < 0)
            return shp::fail(SHP_ERR_SHAPE, "broadcast_binary: bad dims/strides");
        prod *= p.d[k];
    }
    if (prod != l.push[1]) return shp::fail(SHP_ERR_SHAPE, "broadcast_binary: total mismatch");
    hipLaunchKernelGGL(broadcast_binary_kernel, dim3(ew_grid(l.out_elems)), dim3(kBlock), 0,
                       l.stream, (const float*)l.in0, (const float*)l.in1, (float*)l.out, p,
                       l.out_elems);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- bias_act (native epilogue as a standalone op): y = act(x + bias[i % C] + res).
// push: {total, channels}; bias via the epilogue, residual via the epilogue.
__global__ __launch_bounds__(kBlock) void bias_act_kernel(const float* __restrict__ x,
                                                          float* __restrict__ y, uint64_t n,
                                                          int channels,
                                                          const float* __restrict__ bias,
                                                          const float* __restrict__ res, int act,
                                                          float alpha) {
    uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        float v = x[i];
        if (bias) v += bias[i % (uint64_t)channels];
        if (res) v += res[i];
        y[i] = shpd::apply_act(v, act, alpha);
    }
}

int launch_bias_act(const shp::Launch& l) {
    if (l.n_push < 2) return shp::fail(SHP_ERR_PUSH, "bias_act needs push {total, channels}");
    int rc = shp::check_total(l, l.push[0], "bias_act");
    if (rc) return rc;
    if (l.push[1] <= 0) return shp::fail(SHP_ERR_SHAPE, "bias_act: channels <= 0");
    hipLaunchKernelGGL(bias_act_kernel, dim3(ew_grid(l.out_elems)), dim3(kBlock), 0, l.stream,
                       (const float*)l.in0, (float*)l.out, l.out_elems, l.push[1], l.epi->bias,
                       l.epi->residual, l.epi->act, l.epi->alpha);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- gather_rows (native): out[i][:] = table[ids[i]][:] — the embedding lookup the
// reference does in numpy (run_llama_spirv.py:203).  push {n_ids, row_len, n_rows};
// in0 = int32 ids, in1 = table.  An id outside [0, n_rows) yields a zero row (no read).
__global__ __launch_bounds__(kBlock) void gather_rows_kernel(const int32_t* __restrict__ ids,
                                                             const float* __restrict__ table,
                                                             float* __restrict__ y, int n_ids,
                                                             int row_len, int n_rows) {
    uint64_t total = (uint64_t)n_ids * row_len;
    uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += stride) {
        int r = (int)(i / row_len), c = (int)(i % row_len);
        int id = ids[r];
        y[i] = (id >= 0 && id < n_rows) ? table[(uint64_t)id * row_len + c] : 0.0f;
    }
}

int launch_gather_rows(const shp::Launch& l) {
    if (l.n_push < 3) return shp::fail(SHP_ERR_PUSH, "gather_rows needs {n_ids, row_len, n_rows}");
    if (l.push[0] <= 0 || l.push[1] <= 0 || l.push[2] <= 0)
        return shp::fail(SHP_ERR_SHAPE, "gather_rows: dims");
    int rc = shp::check_total(l, (int64_t)l.push[0] * l.push[1], "gather_rows");
    if (rc) return rc;
    hipLaunchKernelGGL(gather_rows_kernel, dim3(ew_grid(l.out_elems)), dim3(kBlock), 0, l.stream,
                       (const int32_t*)l.in0, (const float*)l.in1, (float*)l.out, l.push[0],
                       l.push[1], l.push[2]);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- counter-based RNG fill ----------------------------------------------------------
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(kBlock) void fill_random_kernel(float* __restrict__ p, uint64_t n,
                                                             uint64_t key, int kind, float lo,
                                                             float hi) {
    uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        uint64_t h = mix64(key + i);
        if (kind == 0) {
            float u = (float)(h >> 40) * (1.0f / 16777216.0f);
            p[i] = lo + (hi - lo) * u;
        } else if (kind == 2) {  // uniform integers in [lo, hi) stored as int32
            int64_t span = (int64_t)hi - (int64_t)lo;
            int32_t v = (int32_t)((int64_t)lo + (int64_t)((h >> 11) % (uint64_t)span));
            reinterpret_cast<int32_t*>(p)[i] = v;
        } else {
            float u1 = (float)((h >> 40) + 1) * (1.0f / 16777216.0f);        // (0, 1]
            float u2 = (float)((h >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);  // [0, 1)
            float r = sqrtf(-2.0f * logf(u1));
            p[i] = lo + hi * (r * cosf(6.2831853071795865f * u2));
        }
    }
}

}  // namespace

namespace shp {

int fill_random(hipStream_t stream, float* p, uint64_t n, uint64_t seed, uint64_t tensor_id,
                int kind, float lo, float hi) {
    if (!p && n) return fail(SHP_ERR_INVALID, "fill_random: null pointer");
    if (kind < 0 || kind > 2) return fail(SHP_ERR_INVALID, "fill_random: kind must be 0, 1 or 2");
    if (kind == 2 && !(hi > lo)) return fail(SHP_ERR_INVALID, "fill_random: empty int range");
    if (n == 0) return SHP_OK;
    // Host-side mirror of mix64 for the per-tensor key.
    auto hmix = [](uint64_t z) {
        z += 0x9E3779B97F4A7C15ull;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    };
    uint64_t key = hmix(seed ^ hmix(tensor_id * 0xD1B54A32D192ED03ull + 1));
    hipLaunchKernelGGL(fill_random_kernel, dim3(ew_grid(n)), dim3(kBlock), 0, stream, p, n, key,
                       kind, lo, hi);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

KernelEntry kElementwiseKernels[] = {
    {"abs", 1, false, launch_unary<U_ABS>},
    {"exp", 1, false, launch_unary<U_EXP>},
    {"log", 1, false, launch_unary<U_LOG>},
    {"neg", 1, false, launch_unary<U_NEG>},
    {"sqrt", 1, false, launch_unary<U_SQRT>},
    {"rsqrt", 1, false, launch_unary<U_RSQRT>},
    {"sigmoid", 1, false, launch_unary<U_SIGMOID>},
    {"logistic", 1, false, launch_unary<U_SIGMOID>},
    {"tanh", 1, false, launch_unary<U_TANH>},
    {"relu", 1, false, launch_unary<U_RELU>},
    {"relu6", 1, false, launch_unary<U_RELU6>},
    {"sine", 1, false, launch_unary<U_SINE>},
    {"reshape", 1, false, launch_unary<U_COPY>},
    {"leaky_relu", 2, false, launch_unary<U_LEAKY>},
    {"add", 1, false, launch_binary<B_ADD>},
    {"sub", 1, false, launch_binary<B_SUB>},
    {"mul", 1, false, launch_binary<B_MUL>},
    {"div", 1, false, launch_binary<B_DIV>},
    {"pow", 1, false, launch_binary<B_POW>},
    {"min", 1, false, launch_binary<B_MIN>},
    {"max", 1, false, launch_binary<B_MAX>},
    {"concat", 2, false, launch_concat},
    {"pad", 13, false, launch_pad},
    {"transpose", 13, false, launch_transpose},
    {"l2norm", 2, false, launch_l2norm},
    // native extensions (no reference counterpart kernel)
    {"silu", 1, false, launch_unary<U_SILU>},
    {"gelu_erf", 1, false, launch_unary<U_GELU>},
    {"cosine", 1, false, launch_unary<U_COS>},
    {"floor", 1, false, launch_unary<U_FLOOR>},
    {"ceil", 1, false, launch_unary<U_CEIL>},
    {"l2_normalization", 1, false, launch_l2_normalization},
    {"broadcast_binary", 14, false, launch_broadcast_binary},
    {"bias_act", 2, true, launch_bias_act},
    {"gather_rows", 3, false, launch_gather_rows},
};
const int kElementwiseKernelCount = sizeof(kElementwiseKernels) / sizeof(kElementwiseKernels[0]);

}  // namespace shp
