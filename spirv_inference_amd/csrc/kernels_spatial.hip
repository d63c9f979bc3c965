// Depthwise convolution and bilinear resize.
//
//   depthwise_conv2d  kernels/depthwise_conv2d/glsl/depthwise_conv2d.comp:27-49
//                     (NCHW, weights [C,KH,KW] + bias tail: scheduler.rs:1364-1400;
//                      push {n,c,ih,iw,oh,ow,kh,kw,sh,sw,same,pt,pl,dh,dw,total})
//   resize_bilinear   kernels/resize_bilinear/glsl/resize_bilinear.comp:20-55 (NCHW)
// Native: depthwise_conv2d_nhwc reads TFLite's own [1,KH,KW,C] weight layout + bias tail on
// NHWC activations.  A workgroup owns an 8x8-pixel x 32-channel output tile: it stages the
// input patch the tile's windows cover (the halo included) and the tile's weights in LDS with
// 16-byte loads, so every input element crosses HBM/L2 once per tile instead of once per tap;
// each thread then produces four adjacent channels of two output pixels from LDS.  The taps
// are summed in the reference loop order, skipping the padding taps.
#include "common.h"
#include "coherent.h"

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

constexpr int DT_H = 8, DT_W = 8, DT_C = 32;  // output tile of the LDS kernel

__global__ __launch_bounds__(256) void dw_nhwc_tile_kernel(
    const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y, Dw d,
    int tiles_x, int tiles_y, int ctiles, int PH, int PW, const float* residual, int act,
    float alpha) {
    extern __shared__ __attribute__((aligned(16))) float sm[];
    float* const patch = sm;                       // [PH][PW][DT_C]
    float* const ws = sm + PH * PW * DT_C;         // [kh*kw + 1][DT_C] (bias last)
    int b = blockIdx.x;
    const int ct = b % ctiles;
    b /= ctiles;
    const int tx = b % tiles_x;
    b /= tiles_x;
    const int ty = b % tiles_y;
    const int n = b / tiles_y;
    const int c0 = ct * DT_C, oy0 = ty * DT_H, ox0 = tx * DT_W;
    const int iy0 = oy0 * d.sh - d.pt, ix0 = ox0 * d.sw - d.pl;
    const int tid = threadIdx.x, cg = tid & 7;
    const float* xb = x + (uint64_t)n * d.ih * d.iw * d.c;
    for (int i = tid; i < PH * PW * 8; i += 256) {
        const int pix = i >> 3, g = i & 7;
        const int py = pix / PW, px = pix - py * PW;
        const int iy = iy0 + py, ix = ix0 + px;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if ((unsigned)iy < (unsigned)d.ih && (unsigned)ix < (unsigned)d.iw && c0 + g * 4 < d.c)
            v = *reinterpret_cast<const float4*>(xb + ((uint64_t)iy * d.iw + ix) * d.c + c0 + g * 4);
        *reinterpret_cast<float4*>(patch + pix * DT_C + g * 4) = v;
    }
    const int taps = d.kh * d.kw;
    for (int i = tid; i < (taps + 1) * 8; i += 256) {  // row `taps` of w is the bias tail
        const int tp = i >> 3, g = i & 7;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c0 + g * 4 < d.c) v = *reinterpret_cast<const float4*>(w + (int64_t)tp * d.c + c0 + g * 4);
        *reinterpret_cast<float4*>(ws + tp * DT_C + g * 4) = v;
    }
    __syncthreads();
    if (c0 + cg * 4 >= d.c) return;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int pl = (tid >> 3) + 32 * k;
        const int py = pl >> 3, px = pl & 7;
        const int oy = oy0 + py, ox = ox0 + px;
        if (oy >= d.oh || ox >= d.ow) continue;
        const float4 bv = *reinterpret_cast<const float4*>(ws + taps * DT_C + cg * 4);
        float acc[4] = {bv.x, bv.y, bv.z, bv.w};
        for (int ky = 0; ky < d.kh; ++ky) {
            const int iy = oy * d.sh + ky * d.dh - d.pt;
            if (iy < 0 || iy >= d.ih) continue;
            const int ly = py * d.sh + ky * d.dh;
            for (int kx = 0; kx < d.kw; ++kx) {
                const int ix = ox * d.sw + kx * d.dw - d.pl;
                if (ix < 0 || ix >= d.iw) continue;
                const int lx = px * d.sw + kx * d.dw;
                const float4 xv = *reinterpret_cast<const float4*>(patch + (ly * PW + lx) * DT_C + cg * 4);
                const float4 wv = *reinterpret_cast<const float4*>(ws + (ky * d.kw + kx) * DT_C + cg * 4);
                acc[0] += xv.x * wv.x;
                acc[1] += xv.y * wv.y;
                acc[2] += xv.z * wv.z;
                acc[3] += xv.w * wv.w;
            }
        }
        const uint64_t o = (((uint64_t)n * d.oh + oy) * d.ow + ox) * d.c + c0 + cg * 4;
        const float* rp = residual ? residual + o : nullptr;
        float4 v;
        v.x = shpd::apply_act(acc[0] + (rp ? rp[0] : 0.f), act, alpha);
        v.y = shpd::apply_act(acc[1] + (rp ? rp[1] : 0.f), act, alpha);
        v.z = shpd::apply_act(acc[2] + (rp ? rp[2] : 0.f), act, alpha);
        v.w = shpd::apply_act(acc[3] + (rp ? rp[3] : 0.f), act, alpha);
        *reinterpret_cast<float4*>(y + o) = v;
    }
}

// The same with the kernel size fixed (3x3 or 5x5): every tap's operands are loaded
// unconditionally from clamped coordinates and a padding tap's operand is replaced by zero, so the
// fully unrolled taps issue all their loads before the first FMA.  The runtime-size loop
// above waits for each tap's loads in turn (its `continue`s are branches), one L2 round trip
// per tap: 11-13 us for the 5x5 layers of EfficientNet-Lite0 b8 whatever their size.
template <int KH, int KW>
__global__ __launch_bounds__(256) void dw_nhwc_fixed_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            float* __restrict__ y, Dw d,
                                                            uint64_t groups,
                                                            const float* residual, int act,
                                                            float alpha) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int cg = d.c / 4;
    const float* bias = w + (int64_t)KH * KW * d.c;
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t g = (uint64_t)blockIdx.x * 256 + threadIdx.x; g < groups; g += stride) {
        const int c = (int)(g % cg) * 4;
        const uint64_t pix = g / cg;
        const int ox = (int)(pix % d.ow);
        const uint64_t t = pix / d.ow;
        const int oy = (int)(t % d.oh), n = (int)(t / d.oh);
        const float* xb = x + (uint64_t)n * d.ih * d.iw * d.c + c;
        f4 xv[KH][KW], wv[KH][KW];
        bool ok[KH][KW];
#pragma unroll
        for (int ky = 0; ky < KH; ++ky) {
            const int iy = oy * d.sh + ky * d.dh - d.pt;
            const int cy = min(max(iy, 0), d.ih - 1);
#pragma unroll
            for (int kx = 0; kx < KW; ++kx) {
                const int ix = ox * d.sw + kx * d.dw - d.pl;
                const int cx = min(max(ix, 0), d.iw - 1);
                ok[ky][kx] = (unsigned)iy < (unsigned)d.ih && (unsigned)ix < (unsigned)d.iw;
                xv[ky][kx] = *reinterpret_cast<const f4*>(xb + ((uint64_t)cy * d.iw + cx) * d.c);
                wv[ky][kx] = *reinterpret_cast<const f4*>(w + (ky * KW + kx) * d.c + c);
            }
        }
        f4 acc = *reinterpret_cast<const f4*>(bias + c);
#pragma unroll
        for (int ky = 0; ky < KH; ++ky)
#pragma unroll
            for (int kx = 0; kx < KW; ++kx)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    acc[q] += (ok[ky][kx] ? xv[ky][kx][q] : 0.0f) * wv[ky][kx][q];
        const uint64_t o = pix * d.c + c;
        f4 r = residual ? *reinterpret_cast<const f4*>(residual + o) : f4{0.f, 0.f, 0.f, 0.f};
        f4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = shpd::apply_act(acc[q] + r[q], act, alpha);
        *reinterpret_cast<f4*>(y + o) = v;
    }
}

// W-blocked variant of dw_nhwc_fixed_kernel (horizontal dilation 1, stride SW 1 or 2): a
// thread computes OB = 4 adjacent outputs along W for 4 channels.  Per kernel row it loads the
// (OB - 1) * SW + KW input columns those outputs share and the row's KW weights once, instead
// of KW columns and KW weights per output (for 5x5 stride 1: 8 + 5 loads per row instead of
// 40).  Each output accumulates exactly as in dw_nhwc_fixed_kernel (bias, then the taps in
// (ky, kx) order, padding operands replaced by zero), so the results are bit for bit the same.
template <int KH, int KW, int SW>
__global__ __launch_bounds__(256) void dw_nhwc_wblk_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           float* __restrict__ y, Dw d,
                                                           uint64_t groups,
                                                           const float* residual, int act,
                                                           float alpha) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int OB = 4;
    constexpr int NCOL = (OB - 1) * SW + KW;
    const int cg = d.c / 4;
    const int owb = (d.ow + OB - 1) / OB;
    const float* bias = w + (int64_t)KH * KW * d.c;
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t g = (uint64_t)blockIdx.x * 256 + threadIdx.x; g < groups; g += stride) {
        const int c = (int)(g % cg) * 4;
        const uint64_t pix = g / cg;
        const int ox0 = (int)(pix % owb) * OB;
        const uint64_t t = pix / owb;
        const int oy = (int)(t % d.oh), n = (int)(t / d.oh);
        const float* xb = x + (uint64_t)n * d.ih * d.iw * d.c + c;
        const f4 b = *reinterpret_cast<const f4*>(bias + c);
        f4 acc[OB];
#pragma unroll
        for (int o = 0; o < OB; ++o) acc[o] = b;
        // 3x3: all rows unrolled (all loads issued before the first FMA); 5x5: one row's
        // columns live at a time, which keeps the VGPRs (and the occupancy) of the 3x3 case
        constexpr int KU = KH == 3 ? KH : 1;
#pragma unroll KU
        for (int ky = 0; ky < KH; ++ky) {
            const int iy = oy * d.sh + ky * d.dh - d.pt;
            const int cy = min(max(iy, 0), d.ih - 1);
            const bool oky = (unsigned)iy < (unsigned)d.ih;
            f4 xv[NCOL];
            bool ok[NCOL];
#pragma unroll
            for (int j = 0; j < NCOL; ++j) {
                const int ix = ox0 * SW - d.pl + j;
                const int cx = min(max(ix, 0), d.iw - 1);
                ok[j] = oky && (unsigned)ix < (unsigned)d.iw;
                xv[j] = *reinterpret_cast<const f4*>(xb + ((uint64_t)cy * d.iw + cx) * d.c);
            }
#pragma unroll
            for (int kx = 0; kx < KW; ++kx) {
                const f4 wv = *reinterpret_cast<const f4*>(w + (ky * KW + kx) * d.c + c);
#pragma unroll
                for (int o = 0; o < OB; ++o)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        acc[o][q] += (ok[o * SW + kx] ? xv[o * SW + kx][q] : 0.0f) * wv[q];
            }
        }
#pragma unroll
        for (int o = 0; o < OB; ++o) {
            if (ox0 + o >= d.ow) break;
            const uint64_t off = ((((uint64_t)n * d.oh + oy) * d.ow) + ox0 + o) * d.c + c;
            f4 r = residual ? *reinterpret_cast<const f4*>(residual + off) : f4{0.f, 0.f, 0.f, 0.f};
            f4 v;
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = shpd::apply_act(acc[o][q] + r[q], act, alpha);
            *reinterpret_cast<f4*>(y + off) = v;
        }
    }
}

template <int KH, int KW>
void launch_dw_wblk(const shp::Launch& l, const Dw& d) {
    const uint64_t groups = (uint64_t)d.n * d.oh * ((d.ow + 3) / 4) * (d.c / 4);
    uint64_t g = (groups + 255) / 256;
    if (g > 65536) g = 65536;
    if (d.sw == 1)
        hipLaunchKernelGGL((dw_nhwc_wblk_kernel<KH, KW, 1>), dim3((unsigned)g), dim3(256), 0,
                           l.stream, (const float*)l.in0, (const float*)l.in1, (float*)l.out, d,
                           groups, l.epi->residual, l.epi->act, l.epi->alpha);
    else
        hipLaunchKernelGGL((dw_nhwc_wblk_kernel<KH, KW, 2>), dim3((unsigned)g), dim3(256), 0,
                           l.stream, (const float*)l.in0, (const float*)l.in1, (float*)l.out, d,
                           groups, l.epi->residual, l.epi->act, l.epi->alpha);
}

int launch_dw_nhwc(const shp::Launch& l) {
    Dw d;
    int rc = dw_parse(l, d, "depthwise_conv2d_nhwc");
    if (rc) return rc;
    uint64_t groups = (uint64_t)d.n * d.oh * d.ow * ((d.c + 3) / 4);
    uint64_t g = (groups + 255) / 256;
    if (g > 65536) g = 65536;
    bool vec = d.c % 4 == 0 && ((uintptr_t)l.in0 & 15) == 0 && ((uintptr_t)l.in1 & 15) == 0 &&
               ((uintptr_t)l.out & 15) == 0 &&
               (!l.epi->residual || ((uintptr_t)l.epi->residual & 15) == 0);
    const int PH = (DT_H - 1) * d.sh + (d.kh - 1) * d.dh + 1;
    const int PW = (DT_W - 1) * d.sw + (d.kw - 1) * d.dw + 1;
    const size_t lds = ((size_t)PH * PW + d.kh * d.kw + 1) * DT_C * sizeof(float);
    const int tiles_y = (d.oh + DT_H - 1) / DT_H, tiles_x = (d.ow + DT_W - 1) / DT_W;
    const int ctiles = (d.c + DT_C - 1) / DT_C;
    const int64_t wgs = (int64_t)d.n * tiles_y * tiles_x * ctiles;
    // The tile pays off at stride 1 with enough tiles to fill the CUs (MI355X per-layer
    // A/B over the EfficientNet-Lite0 b8 / MobileNetV2 b1 layers: 14-21 % faster there;
    // stride 2 stages a 4x larger patch per output and loses, as do small grids).
    const bool tile = vec && lds <= 64 * 1024 && d.sh == 1 && d.sw == 1 &&
                      wgs >= (d.kh * d.kw >= 25 ? 512 : 1024) && wgs <= 0x7fffffff;
    bool use_tile = tile;
    const bool wblk_ok = vec && d.dw == 1 && (d.sw == 1 || d.sw == 2) &&
                         ((d.kh == 3 && d.kw == 3) || (d.kh == 5 && d.kw == 5));
    // The W-blocked kernel wins on the 5x5 layers with output rows of >= 14 (MI355X per-layer
    // A/B over the EfficientNet-Lite0 b8 layers: 11-17 % faster than the tiled or fixed kernel,
    // bit for bit the same results); with 4x fewer threads it loses on smaller outputs and on
    // every 3x3 layer there.
    bool use_wblk = wblk_ok && d.kh == 5 && d.ow >= 14;
    if (use_wblk) use_tile = false;
    if (l.tune && l.tune->dw != 0) use_wblk = false;
    if (l.tune && l.tune->dw < 0) use_tile = false;  // overrides: -1 untiled, 1 tiled, 2 W-blocked
    if (l.tune && l.tune->dw == 1 && vec && lds <= 64 * 1024 && wgs <= 0x7fffffff) use_tile = true;
    if (l.tune && l.tune->dw == 2 && wblk_ok) {
        use_tile = false;
        use_wblk = true;
    }
    if (use_wblk) {
        if (d.kh == 3) launch_dw_wblk<3, 3>(l, d);
        else launch_dw_wblk<5, 5>(l, d);
    } else if (use_tile) {
        hipLaunchKernelGGL(dw_nhwc_tile_kernel, dim3((unsigned)wgs), dim3(256), lds, l.stream,
                           (const float*)l.in0, (const float*)l.in1, (float*)l.out, d, tiles_x,
                           tiles_y, ctiles, PH, PW, l.epi->residual, l.epi->act, l.epi->alpha);
    } else if (vec && d.kh == 3 && d.kw == 3)
        hipLaunchKernelGGL((dw_nhwc_fixed_kernel<3, 3>), dim3((unsigned)g), dim3(256), 0, l.stream,
                           (const float*)l.in0, (const float*)l.in1, (float*)l.out, d, groups,
                           l.epi->residual, l.epi->act, l.epi->alpha);
    else if (vec && d.kh == 5 && d.kw == 5)
        hipLaunchKernelGGL((dw_nhwc_fixed_kernel<5, 5>), dim3((unsigned)g), dim3(256), 0, l.stream,
                           (const float*)l.in0, (const float*)l.in1, (float*)l.out, d, groups,
                           l.epi->residual, l.epi->act, l.epi->alpha);
    else if (vec)
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

// ---- conv2d_nhwc 3x3 with 1-4 input channels (the 3-channel image stems) ------------------
// An implicit GEMM would run K = KH*KW*CI (27 for a 3x3 stem) through tiles built for deep K.
// Here one thread makes 8 adjacent output channels of one pixel: it loads the pixel's
// KH*KW*CI input values once (buffer loads; taps in the padding read zeros), then sums them
// against the workgroup's weights, staged in LDS as [k][oc] so the 8 weights of one tap are
// two 16-byte reads that every thread of a pixel group shares.  Sums start at the bias and
// run channel, kernel row, kernel column, as the reference loops (scheduler.rs:321-427).
struct ConvD {
    int h, w, oc, oh, ow, kh, kw, sh, sw, pt, pl, ocg, total;
    unsigned m_ocg, m_ow, m_oh;  // floor((2^32 - 1) / d): n / d = umulhi(n + 1, m)
};

__device__ __forceinline__ int udiv_mh(int n, unsigned m) {
    return (int)__umulhi((unsigned)n + 1u, m);
}

template <int CI, int KH, int KW>
__global__ __launch_bounds__(256) void conv_direct_nhwc_kernel(const float* __restrict__ x,
                                                               const float* __restrict__ w,
                                                               float* __restrict__ y, ConvD d,
                                                               const float* __restrict__ res,
                                                               int act, float alpha) {
    extern __shared__ __attribute__((aligned(16))) float cw[];  // [K][oc] weights, oc biases
    constexpr int KK = KH * KW;
    constexpr int K = KK * CI;
    const int tid = threadIdx.x;
    // this thread's inputs load first, so their round trip overlaps the weight staging's
    const int idx = blockIdx.x * 256 + tid;
    const bool live = idx < d.total;
    const int pix = udiv_mh(live ? idx : 0, d.m_ocg), g = (live ? idx : 0) - pix * d.ocg;
    const int q = udiv_mh(pix, d.m_ow), ox = pix - q * d.ow;
    const int img = udiv_mh(q, d.m_oh), oy = q - img * d.oh;
    const int iy0 = oy * d.sh - d.pt, ix0 = ox * d.sw - d.pl;
    const __amdgpu_buffer_rsrc_t xr =
        buffer_rsrc(x + (int64_t)img * d.h * d.w * CI, (int64_t)d.h * d.w * CI);
    float v[K];
#pragma unroll
    for (int t = 0; t < KK; ++t) {
        const int ky = t / KW, kx = t % KW;
        const int iy = iy0 + ky, ix = ix0 + kx;
        const bool ok = ((unsigned)iy < (unsigned)d.h) & ((unsigned)ix < (unsigned)d.w);
        const unsigned off = ok ? (unsigned)((iy * d.w + ix) * CI) * 4u : 0x80000000u;
#pragma unroll
        for (int c = 0; c < CI; ++c)
            v[t * CI + c] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(xr, off + 4u * c, 0u, 0));
    }
    for (int e = tid; e < K * d.oc; e += 256) {  // OHWI -> [k][oc]
        const int o = e / K, k = e - o * K;
        cw[k * d.oc + o] = w[e];
    }
    for (int e = tid; e < d.oc; e += 256) cw[K * d.oc + e] = w[K * d.oc + e];
    __syncthreads();
    if (!live) return;
    const float* wg = cw + 8 * g;
    f4v a0 = *reinterpret_cast<const f4v*>(wg + K * d.oc);
    f4v a1 = *reinterpret_cast<const f4v*>(wg + K * d.oc + 4);
#pragma unroll
    for (int c = 0; c < CI; ++c) {
#pragma unroll
        for (int t = 0; t < KK; ++t) {
            const float* wk = wg + (t * CI + c) * d.oc;
            const f4v w0 = *reinterpret_cast<const f4v*>(wk);
            const f4v w1 = *reinterpret_cast<const f4v*>(wk + 4);
            const float xv = v[t * CI + c];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                a0[j] = fmaf(xv, w0[j], a0[j]);
                a1[j] = fmaf(xv, w1[j], a1[j]);
            }
        }
    }
    const int64_t o = (int64_t)pix * d.oc + 8 * g;
    if (res) {
        a0 += *reinterpret_cast<const f4v*>(res + o);
        a1 += *reinterpret_cast<const f4v*>(res + o + 4);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        a0[j] = shpd::apply_act(a0[j], act, alpha);
        a1[j] = shpd::apply_act(a1[j], act, alpha);
    }
    *reinterpret_cast<f4v*>(y + o) = a0;
    *reinterpret_cast<f4v*>(y + o + 4) = a1;
}

}  // namespace

namespace shp {

int conv_nhwc_direct(const Launch& l) {
    // push {n, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, same, pt, pl, total}, checked by the
    // caller (positive dims, total)
    const int32_t* q = l.push;
    const int n = q[0], ci = q[1], oc = q[4], kh = q[7], kw = q[8];
    const int64_t K = (int64_t)kh * kw * ci;
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (ci > 4 || kh != 3 || kw != 3 || oc % 8 || (K + 1) * oc * 4 > 65536 || !al16(l.out) ||
        (l.epi->residual && !al16(l.epi->residual)))
        return SHP_ERR_UNSUPPORTED;
    ConvD d;
    d.h = q[2]; d.w = q[3]; d.oc = oc; d.oh = q[5]; d.ow = q[6]; d.kh = kh; d.kw = kw;
    d.sh = q[9]; d.sw = q[10]; d.pt = q[12]; d.pl = q[13]; d.ocg = oc / 8;
    const int64_t total = (int64_t)n * d.oh * d.ow * d.ocg;
    const int64_t dmax = std::max<int64_t>(d.ocg, std::max(d.ow, d.oh));
    // one image's input within the buffer loads' 32-bit byte offsets; the multiply-high
    // divisions exact for every thread index
    if ((int64_t)d.h * d.w * ci * 4 >= (1ll << 31) || total >= (1ll << 31) ||
        (total + 1) * dmax > (1ll << 32))
        return SHP_ERR_UNSUPPORTED;
    d.total = (int)total;
    d.m_ocg = (unsigned)(0xFFFFFFFFull / (uint64_t)d.ocg);
    d.m_ow = (unsigned)(0xFFFFFFFFull / (uint64_t)d.ow);
    d.m_oh = (unsigned)(0xFFFFFFFFull / (uint64_t)d.oh);
    const dim3 grid(grid_1d((uint64_t)total, 256));
    const size_t lds = (size_t)(K + 1) * oc * 4;
    const float* x = (const float*)l.in0;
    const float* w = (const float*)l.in1;
    float* y = (float*)l.out;
    const float* res = l.epi->residual;
    switch (ci) {
        case 1: hipLaunchKernelGGL((conv_direct_nhwc_kernel<1, 3, 3>), grid, dim3(256), lds, l.stream, x, w, y, d, res, l.epi->act, l.epi->alpha); break;
        case 2: hipLaunchKernelGGL((conv_direct_nhwc_kernel<2, 3, 3>), grid, dim3(256), lds, l.stream, x, w, y, d, res, l.epi->act, l.epi->alpha); break;
        case 3: hipLaunchKernelGGL((conv_direct_nhwc_kernel<3, 3, 3>), grid, dim3(256), lds, l.stream, x, w, y, d, res, l.epi->act, l.epi->alpha); break;
        default: hipLaunchKernelGGL((conv_direct_nhwc_kernel<4, 3, 3>), grid, dim3(256), lds, l.stream, x, w, y, d, res, l.epi->act, l.epi->alpha); break;
    }
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

KernelEntry kSpatialKernels[] = {
    {"depthwise_conv2d", 16, true, launch_dw_nchw},
    {"resize_bilinear", 9, false, launch_resize_bilinear},
    // native extensions
    {"depthwise_conv2d_nhwc", 16, true, launch_dw_nhwc},
};
const int kSpatialKernelCount = sizeof(kSpatialKernels) / sizeof(kSpatialKernels[0]);

}  // namespace shp
