// Depthwise convolution and bilinear resize.
//
//   depthwise_conv2d  kernels/depthwise_conv2d/glsl/depthwise_conv2d.comp:27-49
//                     (NCHW, weights [C,KH,KW] + bias tail: scheduler.rs:1364-1400;
//                      push {n,c,ih,iw,oh,ow,kh,kw,sh,sw,same,pt,pl,dh,dw,total})
//   resize_bilinear   kernels/resize_bilinear/glsl/resize_bilinear.comp:20-55 (NCHW)
// Native: depthwise_conv2d_nhwc reads TFLite's own [1,KH,KW,C] weight layout + bias tail on
// NHWC activations; each thread produces four adjacent channels of one output pixel with
// 16-byte loads, so a wavefront reads 256 contiguous channels per tap.
#include "common.h"

namespace {

struct Dw {
    int n, c, ih, iw, oh, ow, kh, kw, sh, sw, same, pt, pl, dh, dw;
};

int dw_parse(const shp::Launch& l, Dw& d, const char* name) {
    if (l.n_push < 16) return shp::fail(SHP_ERR_PUSH, std::string(name) + " needs 16 push constants");
    const int32_t* q = l.push;
    d = Dw{q[0], q[1], q[2], q[3], q[4], q[5], q[6], q[7], q[8], q[9], q[10], q[11], q[12], q[13],
           q[14]};
    if (d.n <= 0 || d.c <= 0 || d.ih <= 0 || d.iw <= 0 || d.oh <= 0 || d.ow <= 0 || d.kh <= 0 ||
        d.kw <= 0 || d.sh <= 0 || d.sw <= 0 || d.dh <= 0 || d.dw <= 0)
        return shp::fail(SHP_ERR_SHAPE, std::string(name) + ": non-positive dim");
    int64_t total = (int64_t)d.n * d.c * d.oh * d.ow;
    if (q[15] != total) return shp::fail(SHP_ERR_SHAPE, std::string(name) + ": total");
    return shp::check_total(l, total, name);
}

__global__ __launch_bounds__(256) void dw_nchw_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ w,
                                                      float* __restrict__ y, Dw d,
                                                      uint64_t total, const float* residual,
                                                      int act, float alpha) {
    uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += stride) {
        uint64_t t = idx;
        int ow = (int)(t % d.ow); t /= d.ow;
        int oh = (int)(t % d.oh); t /= d.oh;
        int c = (int)(t % d.c); t /= d.c;
        int n = (int)t;
        float acc = w[(int64_t)d.c * d.kh * d.kw + c];
        const float* xp = x + ((uint64_t)n * d.c + c) * d.ih * d.iw;
        const float* wp = w + (int64_t)c * d.kh * d.kw;
        for (int kh = 0; kh < d.kh; ++kh) {
            int ih = oh * d.sh + kh * d.dh - d.pt;
            if (ih < 0 || ih >= d.ih) continue;
            for (int kw = 0; kw < d.kw; ++kw) {
                int iw = ow * d.sw + kw * d.dw - d.pl;
                if (iw < 0 || iw >= d.iw) continue;
                acc += xp[ih * d.iw + iw] * wp[kh * d.kw + kw];
            }
        }
        if (residual) acc += residual[idx];
        y[idx] = shpd::apply_act(acc, act, alpha);
    }
}

int launch_dw_nchw(const shp::Launch& l) {
    Dw d;
    int rc = dw_parse(l, d, "depthwise_conv2d");
    if (rc) return rc;
    uint64_t g = (l.out_elems + 255) / 256;
    if (g > 65536) g = 65536;
    hipLaunchKernelGGL(dw_nchw_kernel, dim3((unsigned)g), dim3(256), 0, l.stream,
                       (const float*)l.in0, (const float*)l.in1, (float*)l.out, d, l.out_elems,
                       l.epi->residual, l.epi->act, l.epi->alpha);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// NHWC, weights [KH][KW][C] + bias[C]; 4 channels per thread.
template <bool VEC>
__global__ __launch_bounds__(256) void dw_nhwc_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ w,
                                                      float* __restrict__ y, Dw d,
                                                      uint64_t groups, const float* residual,
                                                      int act, float alpha) {
    const int cg = (d.c + 3) / 4;  // channel groups of 4
    const float* bias = w + (int64_t)d.kh * d.kw * d.c;
    uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t g = (uint64_t)blockIdx.x * 256 + threadIdx.x; g < groups; g += stride) {
        int c4 = (int)(g % cg);
        uint64_t pix = g / cg;
        int ox = (int)(pix % d.ow);
        uint64_t t = pix / d.ow;
        int oy = (int)(t % d.oh);
        int n = (int)(t / d.oh);
        int c = c4 * 4;
        float acc[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] = (c + q < d.c) ? bias[c + q] : 0.0f;
        const float* xb = x + (uint64_t)n * d.ih * d.iw * d.c;
        for (int ky = 0; ky < d.kh; ++ky) {
            int iy = oy * d.sh + ky * d.dh - d.pt;
            if (iy < 0 || iy >= d.ih) continue;
            for (int kx = 0; kx < d.kw; ++kx) {
                int ix = ox * d.sw + kx * d.dw - d.pl;
                if (ix < 0 || ix >= d.iw) continue;
                const float* xp = xb + ((uint64_t)iy * d.iw + ix) * d.c + c;
                const float* wp = w + ((int64_t)ky * d.kw + kx) * d.c + c;
                if constexpr (VEC) {
                    float4 xv = *reinterpret_cast<const float4*>(xp);
                    float4 wv = *reinterpret_cast<const float4*>(wp);
                    acc[0] += xv.x * wv.x;
                    acc[1] += xv.y * wv.y;
                    acc[2] += xv.z * wv.z;
                    acc[3] += xv.w * wv.w;
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (c + q < d.c) acc[q] += xp[q] * wp[q];
                }
            }
        }
        float* yp = y + pix * d.c + c;
        const float* rp = residual ? residual + pix * d.c + c : nullptr;
        if constexpr (VEC) {
            float4 o;
            o.x = shpd::apply_act(acc[0] + (rp ? rp[0] : 0.f), act, alpha);
            o.y = shpd::apply_act(acc[1] + (rp ? rp[1] : 0.f), act, alpha);
            o.z = shpd::apply_act(acc[2] + (rp ? rp[2] : 0.f), act, alpha);
            o.w = shpd::apply_act(acc[3] + (rp ? rp[3] : 0.f), act, alpha);
            *reinterpret_cast<float4*>(yp) = o;
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (c + q < d.c) yp[q] = shpd::apply_act(acc[q] + (rp ? rp[q] : 0.f), act, alpha);
        }
    }
}

int launch_dw_nhwc(const shp::Launch& l) {
    Dw d;
    int rc = dw_parse(l, d, "depthwise_conv2d_nhwc");
    if (rc) return rc;
    uint64_t groups = (uint64_t)d.n * d.oh * d.ow * ((d.c + 3) / 4);
    uint64_t g = (groups + 255) / 256;
    if (g > 65536) g = 65536;
    bool vec = d.c % 4 == 0 && ((uintptr_t)l.in0 & 15) == 0 && ((uintptr_t)l.in1 & 15) == 0 &&
               ((uintptr_t)l.out & 15) == 0;
    if (vec)
        hipLaunchKernelGGL((dw_nhwc_kernel<true>), dim3((unsigned)g), dim3(256), 0, l.stream,
                           (const float*)l.in0, (const float*)l.in1, (float*)l.out, d, groups,
                           l.epi->residual, l.epi->act, l.epi->alpha);
    else
        hipLaunchKernelGGL((dw_nhwc_kernel<false>), dim3((unsigned)g), dim3(256), 0, l.stream,
                           (const float*)l.in0, (const float*)l.in1, (float*)l.out, d, groups,
                           l.epi->residual, l.epi->act, l.epi->alpha);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- resize_bilinear (NCHW): push {n, c, ih, iw, oh, ow, align_corners, half_pixel, total}
struct Rz {
    int n, c, ih, iw, oh, ow, ac, hp;
};

__device__ __forceinline__ float src_coord(int o, int in_size, int out_size, int ac, int hp) {
    if (ac != 0 && out_size > 1) return (float)o * (float)(in_size - 1) / (float)(out_size - 1);
    if (hp != 0) return ((float)o + 0.5f) * (float)in_size / (float)out_size - 0.5f;
    return (float)o * (float)in_size / (float)out_size;
}

__global__ __launch_bounds__(256) void resize_bilinear_kernel(const float* __restrict__ x,
                                                              float* __restrict__ y, Rz r,
                                                              uint64_t total) {
    uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += stride) {
        uint64_t t = idx;
        int ow = (int)(t % r.ow); t /= r.ow;
        int oh = (int)(t % r.oh); t /= r.oh;
        int c = (int)(t % r.c); t /= r.c;
        int n = (int)t;
        float in_y = fminf(fmaxf(src_coord(oh, r.ih, r.oh, r.ac, r.hp), 0.0f), (float)(r.ih - 1));
        float in_x = fminf(fmaxf(src_coord(ow, r.iw, r.ow, r.ac, r.hp), 0.0f), (float)(r.iw - 1));
        int y0 = (int)floorf(in_y), x0 = (int)floorf(in_x);
        int y1 = min(y0 + 1, r.ih - 1), x1 = min(x0 + 1, r.iw - 1);
        float yl = in_y - (float)y0, xl = in_x - (float)x0;
        const float* xp = x + ((uint64_t)n * r.c + c) * r.ih * r.iw;
        float v00 = xp[y0 * r.iw + x0], v01 = xp[y0 * r.iw + x1];
        float v10 = xp[y1 * r.iw + x0], v11 = xp[y1 * r.iw + x1];
        // GLSL mix(a, b, t) = a * (1 - t) + b * t
        float top = v00 * (1.0f - xl) + v01 * xl;
        float bot = v10 * (1.0f - xl) + v11 * xl;
        y[idx] = top * (1.0f - yl) + bot * yl;
    }
}

int launch_resize_bilinear(const shp::Launch& l) {
    if (l.n_push < 9) return shp::fail(SHP_ERR_PUSH, "resize_bilinear needs 9 push constants");
    const int32_t* q = l.push;
    Rz r{q[0], q[1], q[2], q[3], q[4], q[5], q[6], q[7]};
    if (r.n <= 0 || r.c <= 0 || r.ih <= 0 || r.iw <= 0 || r.oh <= 0 || r.ow <= 0)
        return shp::fail(SHP_ERR_SHAPE, "resize_bilinear: non-positive dim");
    int64_t total = (int64_t)r.n * r.c * r.oh * r.ow;
    if (q[8] != total) return shp::fail(SHP_ERR_SHAPE, "resize_bilinear: total");
    int rc = shp::check_total(l, total, "resize_bilinear");
    if (rc) return rc;
    uint64_t g = (l.out_elems + 255) / 256;
    if (g > 65536) g = 65536;
    hipLaunchKernelGGL(resize_bilinear_kernel, dim3((unsigned)g), dim3(256), 0, l.stream,
                       (const float*)l.in0, (float*)l.out, r, l.out_elems);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

}  // namespace

namespace shp {

KernelEntry kSpatialKernels[] = {
    {"depthwise_conv2d", 16, true, launch_dw_nchw},
    {"resize_bilinear", 9, false, launch_resize_bilinear},
    // native extensions
    {"depthwise_conv2d_nhwc", 16, true, launch_dw_nhwc},
};
const int kSpatialKernelCount = sizeof(kSpatialKernels) / sizeof(kSpatialKernels[0]);

}  // namespace shp
