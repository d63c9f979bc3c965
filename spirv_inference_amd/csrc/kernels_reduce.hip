// Reductions, pooling, softmax and row normalisations.
//
// Reference kernels restated here (semantics and push layouts unchanged):
//   hlo_reduce_rank4        kernels/hlo_reduce_rank4/glsl/hlo_reduce_rank4.comp:44-79 (15 i32)
//   hlo_reduce_window_rank4 kernels/hlo_reduce_window_rank4/glsl/...comp:25-49 (14 i32, NHWC)
//   max_pool2d              kernels/max_pool2d/glsl/max_pool2d.comp:25-44 (14 i32, NCHW)
//   global_avg_pool_sum     kernels/global_avg_pool/glsl/global_avg_pool_sum.comp:15-28
//   global_avg_pool_finalize kernels/global_avg_pool/glsl/global_avg_pool_finalize.comp:15-19
//   softmax10 / softmax1000 kernels/softmax/glsl/softmax10.comp:8-20,
//                           kernels/softmax1000/glsl/softmax1000.comp:10-22 — the softmax
//                           runs over the WHOLE tensor (every element of every row), which
//                           is what the reference computes at batch > 1.
// The reference assigns one invocation per output with a serial loop; here the mapping
// follows the memory layout: when the reduced axis is the contiguous one a wavefront
// shares each output (DPP/shuffle tree), otherwise a thread owns an output and adjacent
// threads read adjacent addresses.
#include "common.h"

namespace {

constexpr float kNegMax = -3.4028234663852886e+38f;

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

// Block-wide reductions for blocks of up to 1024 threads (16 wavefronts).
__device__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = (threadIdx.x & 63) < nw ? red[threadIdx.x & 63] : 0.0f;
    return wave_sum(r);
}
__device__ float block_max(float v, float* red) {
    v = wave_max(v);
    int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = (threadIdx.x & 63) < nw ? red[threadIdx.x & 63] : kNegMax;
    return wave_max(r);
}

inline unsigned cap_grid(uint64_t n, unsigned block) {
    uint64_t g = (n + block - 1) / block;
    if (g > 65536) g = 65536;
    return g == 0 ? 1u : (unsigned)g;
}

// ---- hlo_reduce_rank4 --------------------------------------------------------------
struct Red4 {
    int rank;
    int d[4];
    int od[4];
    int r[4];
    int kind;  // 1 = max, else sum
};

// Thread per output: adjacent outputs are adjacent along the innermost kept axis.
__global__ __launch_bounds__(256) void reduce_rank4_thread_kernel(const float* __restrict__ x,
                                                                  float* __restrict__ y, Red4 p,
                                                                  uint64_t total) {
    uint64_t stride = (uint64_t)gridDim.x * 256;
    int64_t st[4] = {(int64_t)p.d[1] * p.d[2] * p.d[3], (int64_t)p.d[2] * p.d[3], p.d[3], 1};
    for (uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += stride) {
        int oc[4] = {0, 0, 0, 0};
        uint64_t t = idx;
        for (int a = p.rank - 1; a >= 0; --a) {
            if (p.r[a] == 0) {
                int dim = p.od[a] > 1 ? p.od[a] : 1;
                oc[a] = (int)(t % dim);
                t /= dim;
            }
        }
        float acc = p.kind == 1 ? kNegMax : 0.0f;
        int e0 = p.r[0] ? p.d[0] : 1, e1 = p.r[1] ? p.d[1] : 1;
        int e2 = p.r[2] ? p.d[2] : 1, e3 = p.r[3] ? p.d[3] : 1;
        for (int a0 = 0; a0 < e0; ++a0)
            for (int a1 = 0; a1 < e1; ++a1)
                for (int a2 = 0; a2 < e2; ++a2)
                    for (int a3 = 0; a3 < e3; ++a3) {
                        int c0 = p.r[0] ? a0 : oc[0], c1 = p.r[1] ? a1 : oc[1];
                        int c2 = p.r[2] ? a2 : oc[2], c3 = p.r[3] ? a3 : oc[3];
                        float v = x[c0 * st[0] + c1 * st[1] + c2 * st[2] + c3];
                        acc = p.kind == 1 ? fmaxf(acc, v) : acc + v;
                    }
        y[idx] = acc;
    }
}

// Wavefront per output when the innermost axis is reduced (contiguous reads per lane).
__global__ __launch_bounds__(256) void reduce_rank4_wave_kernel(const float* __restrict__ x,
                                                                float* __restrict__ y, Red4 p,
                                                                uint64_t total) {
    int lane = threadIdx.x & 63;
    uint64_t wave = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    uint64_t nwaves = (uint64_t)gridDim.x * 4;
    int64_t st[4] = {(int64_t)p.d[1] * p.d[2] * p.d[3], (int64_t)p.d[2] * p.d[3], p.d[3], 1};
    int e[4];
    int64_t rlen = 1;
    for (int a = 0; a < 4; ++a) {
        e[a] = p.r[a] ? p.d[a] : 1;
        rlen *= e[a];
    }
    for (uint64_t idx = wave; idx < total; idx += nwaves) {
        int oc[4] = {0, 0, 0, 0};
        uint64_t t = idx;
        for (int a = p.rank - 1; a >= 0; --a) {
            if (p.r[a] == 0) {
                int dim = p.od[a] > 1 ? p.od[a] : 1;
                oc[a] = (int)(t % dim);
                t /= dim;
            }
        }
        int64_t base = 0;
        for (int a = 0; a < 4; ++a)
            if (!p.r[a]) base += oc[a] * st[a];
        float acc = p.kind == 1 ? kNegMax : 0.0f;
        for (int64_t j = lane; j < rlen; j += 64) {
            int64_t u = j, off = base;
            for (int a = 3; a >= 0; --a) {
                if (p.r[a]) {
                    off += (u % e[a]) * st[a];
                    u /= e[a];
                }
            }
            float v = x[off];
            acc = p.kind == 1 ? fmaxf(acc, v) : acc + v;
        }
        acc = p.kind == 1 ? wave_max(acc) : wave_sum(acc);
        if (lane == 0) y[idx] = acc;
    }
}

int launch_reduce_rank4(const shp::Launch& l) {
    if (l.n_push < 15) return shp::fail(SHP_ERR_PUSH, "hlo_reduce_rank4 needs 15 push constants");
    int rc = shp::check_total(l, l.push[14], "hlo_reduce_rank4");
    if (rc) return rc;
    Red4 p;
    p.rank = l.push[0];
    if (p.rank < 1 || p.rank > 4) return shp::fail(SHP_ERR_SHAPE, "hlo_reduce_rank4: rank");
    int64_t outp = 1;
    for (int i = 0; i < 4; ++i) {
        p.d[i] = l.push[1 + i];
        p.od[i] = l.push[5 + i];
        p.r[i] = l.push[9 + i];
        if (p.d[i] <= 0) return shp::fail(SHP_ERR_SHAPE, "hlo_reduce_rank4: dims must be > 0");
        if (i >= p.rank && (p.d[i] != 1 || p.r[i]))
            return shp::fail(SHP_ERR_SHAPE, "hlo_reduce_rank4: axes beyond rank must be 1");
        if (!p.r[i] && i < p.rank) {
            if (p.od[i] != p.d[i]) return shp::fail(SHP_ERR_SHAPE, "hlo_reduce_rank4: out dim");
            outp *= p.od[i];
        }
    }
    if (outp != l.push[14]) return shp::fail(SHP_ERR_SHAPE, "hlo_reduce_rank4: total");
    p.kind = l.push[13];
    bool inner_reduced = p.r[p.rank - 1] != 0;
    if (inner_reduced) {
        hipLaunchKernelGGL(reduce_rank4_wave_kernel, dim3(cap_grid(l.out_elems, 4)), dim3(256), 0,
                           l.stream, (const float*)l.in0, (float*)l.out, p, l.out_elems);
    } else {
        hipLaunchKernelGGL(reduce_rank4_thread_kernel, dim3(cap_grid(l.out_elems, 256)),
                           dim3(256), 0, l.stream, (const float*)l.in0, (float*)l.out, p,
                           l.out_elems);
    }
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- hlo_reduce_window_rank4 (NHWC windows; out-of-range taps skipped) ---------------
struct Win {
    int n, ih, iw, c, oh, ow, wh, ww, sh, sw, pt, pl, kind;
};

__global__ __launch_bounds__(256) void reduce_window_kernel(const float* __restrict__ x,
                                                            float* __restrict__ y, Win p,
                                                            uint64_t total) {
    uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += stride) {
        uint64_t t = idx;
        int ch = (int)(t % p.c); t /= p.c;
        int ox = (int)(t % p.ow); t /= p.ow;
        int oy = (int)(t % p.oh); t /= p.oh;
        int b = (int)t;
        float acc = p.kind == 1 ? kNegMax : 0.0f;
        for (int ky = 0; ky < p.wh; ++ky) {
            int iy = oy * p.sh + ky - p.pt;
            if (iy < 0 || iy >= p.ih) continue;
            for (int kx = 0; kx < p.ww; ++kx) {
                int ix = ox * p.sw + kx - p.pl;
                if (ix < 0 || ix >= p.iw) continue;
                float v = x[(((uint64_t)b * p.ih + iy) * p.iw + ix) * p.c + ch];
                acc = p.kind == 1 ? fmaxf(acc, v) : acc + v;
            }
        }
        y[idx] = acc;
    }
}

// Four channels per thread (NHWC, C % 4 == 0, 16-byte aligned): 16-byte loads and a quarter
// of the index arithmetic.  Each channel still folds its window in (ky, kx) order, so the
// result equals reduce_window_kernel's bit for bit.
__global__ __launch_bounds__(256) void reduce_window4_kernel(const float4* __restrict__ x,
                                                             float4* __restrict__ y, Win p,
                                                             unsigned total4) {
    const int c4 = p.c / 4;
    for (unsigned idx = blockIdx.x * 256u + threadIdx.x; idx < total4; idx += gridDim.x * 256u) {
        unsigned t = idx;
        const int ch = (int)(t % (unsigned)c4); t /= (unsigned)c4;
        const int ox = (int)(t % (unsigned)p.ow); t /= (unsigned)p.ow;
        const int oy = (int)(t % (unsigned)p.oh);
        const int b = (int)(t / (unsigned)p.oh);
        const float init = p.kind == 1 ? kNegMax : 0.0f;
        float4 acc = make_float4(init, init, init, init);
        for (int ky = 0; ky < p.wh; ++ky) {
            const int iy = oy * p.sh + ky - p.pt;
            if (iy < 0 || iy >= p.ih) continue;
            for (int kx = 0; kx < p.ww; ++kx) {
                const int ix = ox * p.sw + kx - p.pl;
                if (ix < 0 || ix >= p.iw) continue;
                const float4 v = x[((size_t)(b * p.ih + iy) * p.iw + ix) * c4 + ch];
                if (p.kind == 1) {
                    acc.x = fmaxf(acc.x, v.x); acc.y = fmaxf(acc.y, v.y);
                    acc.z = fmaxf(acc.z, v.z); acc.w = fmaxf(acc.w, v.w);
                } else {
                    acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
                }
            }
        }
        y[idx] = acc;
    }
}

int launch_reduce_window(const shp::Launch& l) {
    if (l.n_push < 14)
        return shp::fail(SHP_ERR_PUSH, "hlo_reduce_window_rank4 needs 14 push constants");
    int rc = shp::check_total(l, l.push[13], "hlo_reduce_window_rank4");
    if (rc) return rc;
    Win p{l.push[0], l.push[1], l.push[2], l.push[3], l.push[4], l.push[5], l.push[6],
          l.push[7], l.push[8], l.push[9], l.push[10], l.push[11], l.push[12]};
    if (p.n <= 0 || p.ih <= 0 || p.iw <= 0 || p.c <= 0 || p.oh <= 0 || p.ow <= 0 || p.wh <= 0 ||
        p.ww <= 0 || p.sh <= 0 || p.sw <= 0)
        return shp::fail(SHP_ERR_SHAPE, "hlo_reduce_window_rank4: non-positive dim");
    if ((int64_t)p.n * p.oh * p.ow * p.c != l.push[13])
        return shp::fail(SHP_ERR_SHAPE, "hlo_reduce_window_rank4: total");
    const bool vec = p.c % 4 == 0 && ((uintptr_t)l.in0 & 15) == 0 && ((uintptr_t)l.out & 15) == 0 &&
                     l.out_elems / 4 < 0xffffffffull &&
                     (uint64_t)p.n * p.ih * p.iw * p.c / 4 < 0xffffffffull;
    if (vec)
        hipLaunchKernelGGL(reduce_window4_kernel, dim3(cap_grid(l.out_elems / 4, 256)), dim3(256),
                           0, l.stream, (const float4*)l.in0, (float4*)l.out, p,
                           (unsigned)(l.out_elems / 4));
    else
        hipLaunchKernelGGL(reduce_window_kernel, dim3(cap_grid(l.out_elems, 256)), dim3(256), 0,
                           l.stream, (const float*)l.in0, (float*)l.out, p, l.out_elems);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- max_pool2d (NCHW) ------------------------------------------------------------------
struct Pool {
    int n, c, ih, iw, oh, ow, kh, kw, sh, sw, same, pt, pl;
};

__global__ __launch_bounds__(256) void max_pool_nchw_kernel(const float* __restrict__ x,
                                                            float* __restrict__ y, Pool p,
                                                            uint64_t total) {
    uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += stride) {
        uint64_t t = idx;
        int ow = (int)(t % p.ow); t /= p.ow;
        int oh = (int)(t % p.oh); t /= p.oh;
        int c = (int)(t % p.c); t /= p.c;
        int n = (int)t;
        float best = kNegMax;
        const float* xp = x + ((uint64_t)n * p.c + c) * p.ih * p.iw;
        for (int kh = 0; kh < p.kh; ++kh) {
            int ih = oh * p.sh + kh - p.pt;
            if (ih < 0 || ih >= p.ih) continue;
            for (int kw = 0; kw < p.kw; ++kw) {
                int iw = ow * p.sw + kw - p.pl;
                if (iw < 0 || iw >= p.iw) continue;
                best = fmaxf(best, xp[ih * p.iw + iw]);
            }
        }
        y[idx] = best;
    }
}

int launch_max_pool2d(const shp::Launch& l) {
    if (l.n_push < 14) return shp::fail(SHP_ERR_PUSH, "max_pool2d needs 14 push constants");
    int rc = shp::check_total(l, l.push[13], "max_pool2d");
    if (rc) return rc;
    Pool p{l.push[0], l.push[1], l.push[2], l.push[3], l.push[4], l.push[5], l.push[6],
           l.push[7], l.push[8], l.push[9], l.push[10], l.push[11], l.push[12]};
    if (p.n <= 0 || p.c <= 0 || p.ih <= 0 || p.iw <= 0 || p.oh <= 0 || p.ow <= 0 || p.kh <= 0 ||
        p.kw <= 0 || p.sh <= 0 || p.sw <= 0)
        return shp::fail(SHP_ERR_SHAPE, "max_pool2d: non-positive dim");
    if ((int64_t)p.n * p.c * p.oh * p.ow != l.push[13])
        return shp::fail(SHP_ERR_SHAPE, "max_pool2d: total");
    hipLaunchKernelGGL(max_pool_nchw_kernel, dim3(cap_grid(l.out_elems, 256)), dim3(256), 0,
                       l.stream, (const float*)l.in0, (float*)l.out, p, l.out_elems);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- global_avg_pool_sum / _finalize (NCHW, push {n,c,h,w}) -----------------------------
__global__ __launch_bounds__(256) void gap_sum_nchw_kernel(const float* __restrict__ x,
                                                           float* __restrict__ y, uint64_t nc,
                                                           int hw) {
    int lane = threadIdx.x & 63;
    uint64_t wave = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    uint64_t nwaves = (uint64_t)gridDim.x * 4;
    for (uint64_t o = wave; o < nc; o += nwaves) {
        const float* xp = x + o * hw;
        float acc = 0.0f;
        for (int j = lane; j < hw; j += 64) acc += xp[j];
        acc = wave_sum(acc);
        if (lane == 0) y[o] = acc;
    }
}

__global__ __launch_bounds__(256) void gap_finalize_kernel(const float* __restrict__ x,
                                                           float* __restrict__ y, uint64_t nc,
                                                           float hw) {
    uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < nc; i += stride)
        y[i] = x[i] / hw;
}

int gap_check(const shp::Launch& l, const char* name) {
    if (l.n_push < 4) return shp::fail(SHP_ERR_PUSH, std::string(name) + " needs {n,c,h,w}");
    for (int i = 0; i < 4; ++i)
        if (l.push[i] <= 0) return shp::fail(SHP_ERR_SHAPE, std::string(name) + ": dims");
    return shp::check_total(l, (int64_t)l.push[0] * l.push[1], name);
}

int launch_gap_sum(const shp::Launch& l) {
    int rc = gap_check(l, "global_avg_pool_sum");
    if (rc) return rc;
    hipLaunchKernelGGL(gap_sum_nchw_kernel, dim3(cap_grid(l.out_elems, 4)), dim3(256), 0,
                       l.stream, (const float*)l.in0, (float*)l.out, l.out_elems,
                       l.push[2] * l.push[3]);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

int launch_gap_finalize(const shp::Launch& l) {
    int rc = gap_check(l, "global_avg_pool_finalize");
    if (rc) return rc;
    hipLaunchKernelGGL(gap_finalize_kernel, dim3(cap_grid(l.out_elems, 256)), dim3(256), 0,
                       l.stream, (const float*)l.in0, (float*)l.out, l.out_elems,
                       (float)(l.push[2] * l.push[3]));
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- global_avg_pool_nhwc (native): out[n,c] = sum_{h,w} x[n,h,w,c] / (h*w), one pass.
// push {n, h, w, c}.  Thread per (n, c): adjacent threads read adjacent channels.
__global__ __launch_bounds__(256) void gap_nhwc_kernel(const float* __restrict__ x,
                                                       float* __restrict__ y, int n, int hw,
                                                       int c) {
    uint64_t total = (uint64_t)n * c;
    uint64_t stride = (uint64_t)gridDim.x * 256;
    float inv = (float)hw;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
        int ch = (int)(i % c);
        uint64_t b = i / c;
        const float* xp = x + b * hw * c + ch;
        float acc = 0.0f;
        // loads in groups of 8 so they are in flight together; the sum stays in pixel order
        int j = 0;
        for (; j + 8 <= hw; j += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = xp[(uint64_t)(j + u) * c];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc += v[u];
        }
        for (; j < hw; ++j) acc += xp[(uint64_t)j * c];
        y[i] = acc / inv;
    }
}

int launch_gap_nhwc(const shp::Launch& l) {
    if (l.n_push < 4) return shp::fail(SHP_ERR_PUSH, "global_avg_pool_nhwc needs {n,h,w,c}");
    for (int i = 0; i < 4; ++i)
        if (l.push[i] <= 0) return shp::fail(SHP_ERR_SHAPE, "global_avg_pool_nhwc: dims");
    int rc = shp::check_total(l, (int64_t)l.push[0] * l.push[3], "global_avg_pool_nhwc");
    if (rc) return rc;
    hipLaunchKernelGGL(gap_nhwc_kernel, dim3(cap_grid(l.out_elems, 256)), dim3(256), 0, l.stream,
                       (const float*)l.in0, (float*)l.out, l.push[0], l.push[1] * l.push[2],
                       l.push[3]);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- softmax10 / softmax1000: whole-tensor softmax ------------------------------------
__global__ __launch_bounds__(1024) void softmax_whole_kernel(const float* __restrict__ x,
                                                             float* __restrict__ y, int n) {
    __shared__ float red[16];
    float m = kNegMax;
    for (int i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, x[i]);
    m = block_max(m, red);
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s += expf(x[i] - m);
    s = block_sum(s, red);
    for (int i = threadIdx.x; i < n; i += blockDim.x) y[i] = expf(x[i] - m) / s;
}

// The same softmax for n <= 1024 * R in one pass over memory: each thread loads its R
// elements at once and keeps them and their exponentials in registers.  The per-thread sums
// run in the same element order and the reductions are the same, so the results equal the
// three-pass kernel's bit for bit.
template <int R>
__global__ __launch_bounds__(1024) void softmax_whole_reg_kernel(const float* __restrict__ x,
                                                                 float* __restrict__ y, int n) {
    __shared__ float red[16];
    float v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x + r * 1024;
        v[r] = i < n ? x[i] : kNegMax;
    }
    float m = kNegMax;
#pragma unroll
    for (int r = 0; r < R; ++r) m = fmaxf(m, v[r]);
    m = block_max(m, red);
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x + r * 1024;
        v[r] = expf(v[r] - m);
        if (i < n) s += v[r];
    }
    s = block_sum(s, red);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x + r * 1024;
        if (i < n) y[i] = v[r] / s;
    }
}

int launch_softmax10(const shp::Launch& l) {
    if (l.out_elems != 10)
        return shp::fail(SHP_ERR_SHAPE, "softmax10: the reference kernel is fixed at 10 classes");
    hipLaunchKernelGGL(softmax_whole_kernel, dim3(1), dim3(64), 0, l.stream, (const float*)l.in0,
                       (float*)l.out, 10);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

int launch_softmax1000(const shp::Launch& l) {
    if (l.n_push < 1) return shp::fail(SHP_ERR_PUSH, "softmax1000 needs push {class_count}");
    int rc = shp::check_total(l, l.push[0], "softmax1000");
    if (rc) return rc;
    if (l.push[0] <= 0) return shp::fail(SHP_ERR_SHAPE, "softmax1000: class_count <= 0");
    const int n = l.push[0];
    const float* x = (const float*)l.in0;
    float* y = (float*)l.out;
    if (n <= 1024)
        hipLaunchKernelGGL((softmax_whole_reg_kernel<1>), dim3(1), dim3(1024), 0, l.stream, x, y, n);
    else if (n <= 2048)
        hipLaunchKernelGGL((softmax_whole_reg_kernel<2>), dim3(1), dim3(1024), 0, l.stream, x, y, n);
    else if (n <= 8192)
        hipLaunchKernelGGL((softmax_whole_reg_kernel<8>), dim3(1), dim3(1024), 0, l.stream, x, y, n);
    else
        hipLaunchKernelGGL(softmax_whole_kernel, dim3(1), dim3(1024), 0, l.stream, x, y, n);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- softmax_rows (native): per-row softmax of (x * scale + mask[col]).
// push {rows, cols, scale_bits}; in1 = optional additive mask of length cols (or NULL).
// The HLO graphs spell this as reduce(max) -> subtract -> exp -> reduce(sum) -> divide
// with CPU broadcasts in between (resnet50.stablehlo.txt:1714, bert_base.stablehlo.txt:36-49).
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ mask,
                                                           float* __restrict__ y, int rows,
                                                           int cols, float scale) {
    __shared__ float red[16];
    for (int r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = x + (uint64_t)r * cols;
        float* yr = y + (uint64_t)r * cols;
        float m = kNegMax;
        for (int i = threadIdx.x; i < cols; i += blockDim.x) {
            float v = xr[i] * scale + (mask ? mask[i] : 0.0f);
            m = fmaxf(m, v);
        }
        m = block_max(m, red);
        float s = 0.0f;
        for (int i = threadIdx.x; i < cols; i += blockDim.x) {
            float v = xr[i] * scale + (mask ? mask[i] : 0.0f);
            s += expf(v - m);
        }
        s = block_sum(s, red);
        for (int i = threadIdx.x; i < cols; i += blockDim.x) {
            float v = xr[i] * scale + (mask ? mask[i] : 0.0f);
            yr[i] = expf(v - m) / s;
        }
    }
}

// One wavefront per row for short rows (attention scores of length <= 1024).
__global__ __launch_bounds__(256) void softmax_rows_wave_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ mask,
                                                                float* __restrict__ y, int rows,
                                                                int cols, float scale) {
    int lane = threadIdx.x & 63;
    int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    int nwaves = gridDim.x * 4;
    constexpr int kMaxPer = 16;
    for (int r = wave; r < rows; r += nwaves) {
        const float* xr = x + (uint64_t)r * cols;
        float* yr = y + (uint64_t)r * cols;
        float v[kMaxPer];
        float m = kNegMax;
#pragma unroll
        for (int j = 0; j < kMaxPer; ++j) {
            int i = lane + j * 64;
            v[j] = i < cols ? xr[i] * scale + (mask ? mask[i] : 0.0f) : kNegMax;
            m = fmaxf(m, v[j]);
        }
        m = wave_max(m);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxPer; ++j) {
            int i = lane + j * 64;
            v[j] = i < cols ? expf(v[j] - m) : 0.0f;
            s += v[j];
        }
        s = wave_sum(s);
#pragma unroll
        for (int j = 0; j < kMaxPer; ++j) {
            int i = lane + j * 64;
            if (i < cols) yr[i] = v[j] / s;
        }
    }
}

int launch_softmax_rows(const shp::Launch& l) {
    if (l.n_push < 3) return shp::fail(SHP_ERR_PUSH, "softmax_rows needs {rows, cols, scale_bits}");
    int rows = l.push[0], cols = l.push[1];
    if (rows <= 0 || cols <= 0) return shp::fail(SHP_ERR_SHAPE, "softmax_rows: dims");
    int rc = shp::check_total(l, (int64_t)rows * cols, "softmax_rows");
    if (rc) return rc;
    float scale;
    int32_t bits = l.push[2];
    memcpy(&scale, &bits, 4);
    if (cols <= 1024) {
        hipLaunchKernelGGL(softmax_rows_wave_kernel, dim3(cap_grid(rows, 4)), dim3(256), 0,
                           l.stream, (const float*)l.in0, (const float*)l.in1, (float*)l.out,
                           rows, cols, scale);
    } else {
        unsigned g = rows < 65536 ? rows : 65536;
        hipLaunchKernelGGL(softmax_rows_kernel, dim3(g), dim3(256), 0, l.stream,
                           (const float*)l.in0, (const float*)l.in1, (float*)l.out, rows, cols,
                           scale);
    }
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- layernorm_rows / rmsnorm_rows (native) -----------------------------------------
// layernorm: y = (x - mean) * rsqrt(var + eps) * gamma + beta, var = mean((x-mean)^2);
//            in1 = [gamma(cols) | beta(cols)]  (BERT, eps 1e-12)
// rmsnorm:   y = x * rsqrt(mean(x^2) + eps) * w; in1 = w(cols)   (export_llama.py:284-286)
// push {rows, cols, eps_bits}.  One 256-thread group per row, fp32 accumulation.
template <bool RMS>
__global__ __launch_bounds__(256) void rownorm_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ w,
                                                      float* __restrict__ y, int rows, int cols,
                                                      float eps) {
    __shared__ float red[16];
    for (int r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = x + (uint64_t)r * cols;
        float* yr = y + (uint64_t)r * cols;
        float mean = 0.0f;
        if (!RMS) {
            float s = 0.0f;
            for (int i = threadIdx.x; i < cols; i += blockDim.x) s += xr[i];
            mean = block_sum(s, red) / (float)cols;
        }
        float ss = 0.0f;
        for (int i = threadIdx.x; i < cols; i += blockDim.x) {
            float d = xr[i] - mean;
            ss += d * d;
        }
        float var = block_sum(ss, red) / (float)cols;
        float inv = 1.0f / sqrtf(var + eps);
        for (int i = threadIdx.x; i < cols; i += blockDim.x) {
            float v = (xr[i] - mean) * inv;
            yr[i] = RMS ? v * w[i] : v * w[i] + w[cols + i];
        }
    }
}

template <bool RMS>
int launch_rownorm(const shp::Launch& l) {
    if (l.n_push < 3) return shp::fail(SHP_ERR_PUSH, "row norm needs {rows, cols, eps_bits}");
    int rows = l.push[0], cols = l.push[1];
    if (rows <= 0 || cols <= 0) return shp::fail(SHP_ERR_SHAPE, "row norm: dims");
    int rc = shp::check_total(l, (int64_t)rows * cols, RMS ? "rmsnorm_rows" : "layernorm_rows");
    if (rc) return rc;
    if (!l.in1) return shp::fail(SHP_ERR_INVALID, "row norm: weights (in1) required");
    float eps;
    int32_t bits = l.push[2];
    memcpy(&eps, &bits, 4);
    unsigned g = rows < 65536 ? rows : 65536;
    hipLaunchKernelGGL((rownorm_kernel<RMS>), dim3(g), dim3(256), 0, l.stream,
                       (const float*)l.in0, (const float*)l.in1, (float*)l.out, rows, cols, eps);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- nan_count: the NaN trace of the HLO runner (compiler.rs:613-623), on the device -------
// out[0] = number of NaN values among x[0, n) (uint32 bits), out[1] = index of the first one
// (int32 bits, -1 when there is none).  The first kernel sets out to {0, 0xFFFFFFFF} (a
// kernel, not a memset, so the pair can sit inside a captured graph); the second folds a
// grid-stride count and the smallest index per wavefront and merges them with atomics.
__global__ void nan_count_init_kernel(uint32_t* out) {
    out[0] = 0u;
    out[1] = 0xFFFFFFFFu;
}

__global__ __launch_bounds__(256) void nan_count_kernel(const float* __restrict__ x,
                                                        uint32_t* out, uint32_t n) {
    uint32_t cnt = 0, first = 0xFFFFFFFFu;
    const uint32_t stride = gridDim.x * 256u;
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += stride) {
        if (__builtin_isnan(x[i])) {
            ++cnt;
            first = first < i ? first : i;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        cnt += __shfl_xor(cnt, o);
        uint32_t f = __shfl_xor(first, o);
        first = first < f ? first : f;
    }
    if ((threadIdx.x & 63) == 0 && cnt) {
        atomicAdd(&out[0], cnt);
        atomicMin(&out[1], first);
    }
}

int launch_nan_count(const shp::Launch& l) {
    if (l.n_push < 1) return shp::fail(SHP_ERR_PUSH, "nan_count needs {n}");
    int64_t n = l.push[0];
    if (n < 0) return shp::fail(SHP_ERR_SHAPE, "nan_count: n < 0");
    int rc = shp::check_total(l, 2, "nan_count");
    if (rc) return rc;
    if (n > 0 && !l.in0) return shp::fail(SHP_ERR_INVALID, "nan_count: input (in0) required");
    hipLaunchKernelGGL(nan_count_init_kernel, dim3(1), dim3(1), 0, l.stream, (uint32_t*)l.out);
    SHP_HIP_CHECK(hipGetLastError());
    if (n > 0) {
        unsigned g = cap_grid((uint64_t)n, 256);
        if (g > 2048) g = 2048;
        hipLaunchKernelGGL(nan_count_kernel, dim3(g), dim3(256), 0, l.stream,
                           (const float*)l.in0, (uint32_t*)l.out, (uint32_t)n);
        SHP_HIP_CHECK(hipGetLastError());
    }
    return SHP_OK;
}

}  // namespace

namespace shp {

KernelEntry kReduceKernels[] = {
    {"hlo_reduce_rank4", 15, false, launch_reduce_rank4},
    {"hlo_reduce_window_rank4", 14, false, launch_reduce_window},
    {"max_pool2d", 14, false, launch_max_pool2d},
    {"global_avg_pool_sum", 4, false, launch_gap_sum},
    {"global_avg_pool_finalize", 4, false, launch_gap_finalize},
    {"softmax10", 0, false, launch_softmax10},
    {"softmax1000", 1, false, launch_softmax1000},
    // native extensions
    {"global_avg_pool_nhwc", 4, false, launch_gap_nhwc},
    {"softmax_rows", 3, false, launch_softmax_rows},
    {"layernorm_rows", 3, false, launch_rownorm<false>},
    {"rmsnorm_rows", 3, false, launch_rownorm<true>},
    {"nan_count", 1, false, launch_nan_count},
};
const int kReduceKernelCount = sizeof(kReduceKernels) / sizeof(kReduceKernels[0]);

}  // namespace shp
