// inverted_residual_nhwc: a MobileNetV2 / EfficientNet-Lite inverted-residual (MBConv) block
// in one launch.
//
// The reference runs the block as three TFLite operators, one dispatch and one host round
// trip each (source/tflite_loader/src/scheduler.rs:321-427 CONV_2D, :429-548
// DEPTHWISE_CONV_2D, then the projection CONV_2D with the residual ADD):
//   E = act_e(x . We + be)               1x1 expand    (kernels/conv2d/glsl/conv2d.comp:26-50)
//   D = act_d(depthwise_k,s(E) + bd)     depthwise     (depthwise_conv2d.comp:27-49, SAME pad)
//   y = act_o(D . Wp + bp [+ x])         1x1 project + residual
// A workgroup here owns an output tile of TH x TW pixels of one image and a slice of the
// output channels.  It stages the input patch that the tile's depthwise windows cover (the
// halo) in LDS once, then walks the expanded channels 16 at a time:
//   1. expand: the halo patch times 16 columns of We on the fp32 matrix cores
//      (v_mfma_f32_16x16x4_f32, operands from LDS), + bias, activation, and zero where the
//      halo pixel lies outside the image (the depthwise's SAME padding of E);
//   2. depthwise: the k x k taps of those 16 channels from LDS, + bias, activation;
//   3. project: those 16 channels times their 16 rows of Wp, accumulated in MFMA registers.
// E and D never leave the CU: the block reads x and the weights and writes y, where the
// three-operator form also writes and reads back the expanded tensor (the block's largest)
// and the depthwise output, and pays two more launches.
//
// Where the tiles alone cannot fill the GPU (7x7 and 14x14 maps at batch 1) the expanded
// channels are split over S workgroups per tile (each projects its own channel range) and
// the output channels over J.  The S partial projections of a tile go to the context
// workspace with device-coherent stores; the workgroup that completes the tile last sums
// them in split order (so the result does not depend on arrival order), applies bias,
// residual and activation, and resets the tile's arrival counter to zero.
//
// Packed weights (in1), the three operators' own tensors back to back:
//   [We: ce x cin (OHWI 1x1) | be: ce]  (only with expand = 1)
//   [Wd: k x k x ce ([KH][KW][C]) | bd: ce] [Wp: cout x ce (OHWI 1x1) | bp: cout]
// push {n, cin, h, w, ce, cout, oh, ow, k, s, pt, pl, expand, act_e, act_d, total};
// the epilogue's residual and activation apply to y (its bias slot must be empty).
#include <map>
#include <mutex>
#include <tuple>

#include "coherent.h"
#include "common.h"
#include "gemm.h"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int CC = 32;       // expanded channels per chunk (two 16-column MFMA blocks)
constexpr int ES = CC + 1;   // LDS row stride (floats) of the expanded chunk
constexpr int DS = CC + 4;   // of the depthwise chunk: 16-byte rows, 4 banks apart
constexpr int WPS = CC + 4;  // of the projection weight chunk
constexpr int NPF = 12;      // float4 weight loads per thread and chunk, at most
constexpr int NPF_DP = 6;    // the same without expand, where two chunks' sets are in flight
constexpr int kMaxLds = 160 * 1024;

// LDS layout (float offsets) of one workgroup, shared by the host plan and the kernel:
// halo patch | We chunk | be | Wd taps | bd | E | D | Wp chunk | halo-row validity | flag.
// Without an expand there is no halo patch or We: E holds the chunk's 32 input channels of
// the halo, staged from x chunk by chunk.
struct IrLds {
    int x, w, be, wd, bd, e, d, wp, hv, flag, total;
};
__host__ __device__ inline IrLds ir_lds(int hpb, int xs, int expand, int k, int pb, int ob) {
    IrLds l;
    int o = 0;
    l.x = o;    o += expand ? hpb * 16 * xs : 0;
    l.w = o;    o += expand ? CC * xs : 0;
    l.be = o;   o += CC;
    l.wd = o;   o += k * k * CC;
    l.bd = o;   o += CC;
    l.e = o;    o += hpb * 16 * ES;  // without expand: the chunk's 32 channels of the halo
    l.d = o;    o += pb * 16 * DS;
    l.wp = o;   o += ob * 16 * WPS;
    l.hv = o;   o += hpb * 16;
    l.flag = o; o += 4;
    l.total = o;
    return l;
}

struct IrArgs {
    const float* x;
    const float* w;
    float* y;
    const float* res;
    float* partial;
    int* counters;
    int n, h, w_, cin, ce, cout, oh, ow, pt, pl;
    int expand, act_e, act_d, act_o;
    float alpha;
    int th, tw, tiles_y, tiles_x;  // output tile and the tile grid of one image
    int hw, hp, hpb;               // halo columns, halo pixels, 16-row blocks of them
    int cin16, xs;                 // cin rounded up to 16; LDS row stride of x and We
    int nchunk, cpw, S;            // 32-channel chunks of ce (the last may hold 16),
                                   // chunks per split, splits
    int J, coj, ob, pb;            // output-channel splits, channels per split (16 * ob),
                                   // 16-row blocks of the output tile
    int w_wd;  // packed-weight offset of the depthwise taps (ce * (cin + 1) with expand, else 0)
    // floor((2^32 - 1) / d) for the divisors cin / 4, cin16 / 4, hw, tw, S, J, tiles_x and
    // tiles_y: n / d = umulhi(n + 1, m) exactly for (n + 1) * d <= 2^32, d = 1 included
    unsigned m_cin4, m_c4n, m_hw, m_tw, m_S, m_J, m_tx, m_ty;
};

// 16-byte buffer load; a byte offset at or past the range (kOob) reads zeros without a
// memory access, so masked loads need no branch.
constexpr unsigned kOob = 0x80000000u;
__device__ __forceinline__ f4v ld16(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
    return __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

// One add and one multiply-high, no select on the divisor (a select split the kernel-argument
// loads into three dependent scalar-load round trips).
__device__ __forceinline__ int udiv(int n, unsigned m) {
    return (int)__umulhi((unsigned)n + 1u, m);
}

// The idx-th float4 of one chunk's weights: the We rows (cin wide), then rows of 32 channels
// (8 float4): be (with expand), the k*k Wd taps, bd, the Wp rows of this output-channel
// slice.  In the packed buffer be, the taps and bd sit ce apart from w_be (= w_wd - ce
// without expand) and the Wp rows follow; in LDS be, the taps and bd are 32 apart from o_be
// and the Wp rows WPS apart from o_wp, so a slot is a few selects, not a chain of branches.
// goff: packed-weight offset at chunk 0; meta: LDS offset | channel within the chunk << 16
// | 1 << 24 for the We rows (which advance 32 rows per chunk; the rest 32 channels).
template <int K>
__device__ __forceinline__ void weight_slot(const IrArgs& a, const IrLds& L, int j, int idx,
                                            int& goff, int& meta) {
    const int nwe = a.expand ? CC * (a.cin >> 2) : 0;
    // We rows (at the start of the packed buffer)
    const int r = udiv(idx, a.m_cin4), q = idx - r * (a.cin >> 2);
    const int g_we = 4 * idx, l_we = L.w + r * a.xs + 4 * q;
    // 32-channel rows: row 0 = be (a virtual row before the taps without expand)
    const int i8 = idx - nwe;
    const int row = (i8 >> 3) + (a.expand ? 0 : 1), q8 = i8 & 7;
    const bool wp = row >= K * K + 2;
    const int rp = row - (K * K + 2);
    const int base = a.w_wd - a.ce;  // be's offset (w_be with expand)
    const int g_row = base + (row + (wp ? j * a.coj : 0)) * a.ce + 4 * q8;
    const int l_row = wp ? L.wp + rp * WPS + 4 * q8 : L.be + row * CC + 4 * q8;
    const bool we = idx < nwe;
    goff = we ? g_we : g_row;
    meta = we ? (l_we | (r << 16) | (1 << 24)) : (l_row | ((4 * q8) << 16));
}

// Loads (fetch) and LDS stores (put) of this thread's float4s of one chunk's weights,
// unrolled by recursion so the staging registers stay registers.  Channels past ce (the
// second half of a 16-channel last chunk) read as zeros.
template <int U, int N>
__device__ __forceinline__ void fetch_weights(f4v (&pf)[N], const IrArgs& a,
                                              __amdgpu_buffer_rsrc_t wr, const int (&goff)[NPF],
                                              const int (&meta)[NPF], int tid, int nf, int ch) {
    if constexpr (U < N) {
        const bool ok = (tid + 256 * U < nf) & (ch * CC + ((meta[U] >> 16) & 255) < a.ce);
        const int stp = (meta[U] >> 24) ? CC * a.cin : CC;
        pf[U] = ld16(wr, ok ? (unsigned)(goff[U] + stp * ch) * 4u : kOob);
        fetch_weights<U + 1, N>(pf, a, wr, goff, meta, tid, nf, ch);
    }
}
template <int U, int N>
__device__ __forceinline__ void put_weights(const f4v (&pf)[N], float* lds,
                                            const int (&meta)[NPF], int tid, int nf) {
    if constexpr (U < N) {
        if (tid + 256 * U < nf) *reinterpret_cast<f4v*>(lds + (meta[U] & 0xFFFF)) = pf[U];
        put_weights<U + 1, N>(pf, lds, meta, tid, nf);
    }
}

// The expand and depthwise activations: none, ReLU or ReLU6 as one clamp (the host refuses
// the others), so the per-element code has no branches.
struct ActClamp {
    float lo, hi;
    bool on;
    __device__ explicit ActClamp(int act)
        : lo(0.f), hi(act == SHP_ACT_RELU6 ? 6.f : __builtin_huge_valf()), on(act != SHP_ACT_NONE) {}
    __device__ float operator()(float v) const { return on ? fminf(fmaxf(v, lo), hi) : v; }
};

__device__ __forceinline__ floatx4 mfma4(f4v a, f4v b, floatx4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, c, 0, 0, 0);
}

// K, ST: depthwise kernel size and stride; NBW: projection blocks (16 pixels x 16 output
// channels) per wavefront, at most; EXP: the block has an expand (a.expand, as a constant).
// Without one the input already has the expanded channels: each chunk's 32 of them are staged
// over the halo from x (UH float4 per thread, loaded two chunks ahead with the chunk's weights,
// in two register sets), so the LDS never holds all channels and the depthwise reads them as it
// reads E.
constexpr int UH = 5;  // halo float4 per thread per chunk without expand: 8 * hpb * 16 <= 256 * UH
template <int K, int ST, int NBW, bool EXP>
__global__ __launch_bounds__(256) void ir_kernel(IrArgs a) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, li = lane & 15;
    const int id = blockIdx.x;
    const int q_s = udiv(id, a.m_S), si = id - q_s * a.S;
    const int tile = udiv(q_s, a.m_J), j = q_s - tile * a.J;  // tile: (img, ty, tx) row-major
    const int q_x = udiv(tile, a.m_tx), tx = tile - q_x * a.tiles_x;
    const int img = udiv(q_x, a.m_ty), ty = q_x - img * a.tiles_y;
    const int oy0 = ty * a.th, ox0 = tx * a.tw;
    const int iy0 = oy0 * ST - a.pt, ix0 = ox0 * ST - a.pl;
    const int c_begin = si * a.cpw;
    const int c_end = min(a.nchunk, c_begin + a.cpw);
    const int cv = min(a.coj, a.cout - j * a.coj);  // output channels of this slice
    const int nf = (EXP ? CC * (a.cin >> 2) + 8 : 0) + 8 * K * K + 8 + 8 * cv;
    const int P = a.th * a.tw;
    const int nblk = a.pb * a.ob;
    const int hrows = a.hpb * 16;

    const IrLds L = ir_lds(a.hpb, a.xs, EXP, K, a.pb, a.ob);
    float* Xs = lds + L.x;
    float* Ws = lds + L.w;
    const float* Bes = lds + L.be;
    const float* Wds = lds + L.wd;
    const float* Bds = lds + L.bd;
    float* Es = lds + L.e;
    float* Ds = lds + L.d;
    float* Wps = lds + L.wp;
    int* hvalid = reinterpret_cast<int*>(lds + L.hv);  // halo row inside the image

    // halo patch of x: hrows rows (halo pixels, row-major) of cin16 floats; zero outside
    // the image, in the padding columns and in the rows past the patch.  8 float4 loads per
    // thread per batch; the first batch is issued before the weight slots are set up and
    // stored after the first chunk's weight loads are issued, so the two overlap.
    const int c4n = a.cin16 >> 2;
    const int xtotal = hrows * c4n;
    f4v xv[8];
    int xd[8];
    // (branch-free: a float4 outside the image is a buffer load past the range, so zeros)
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.x + (int64_t)img * a.h * a.w_ * a.cin,
                                                  (int64_t)a.h * a.w_ * a.cin);
    auto load_x = [&](int e0) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int e = e0 + 256 * t;
            const int r = udiv(e, a.m_c4n), q = e - r * c4n;
            const int hy = udiv(r, a.m_hw), hx = r - hy * a.hw;
            const int iy = iy0 + hy, ix = ix0 + hx;
            const bool in = (e < xtotal) & (r < a.hp) & (4 * q < a.cin) &
                            ((unsigned)iy < (unsigned)a.h) & ((unsigned)ix < (unsigned)a.w_);
            xv[t] = ld16(xr, in ? (unsigned)((iy * a.w_ + ix) * a.cin + 4 * q) * 4u : kOob);
            xd[t] = e < xtotal ? r * a.xs + 4 * q : -1;
        }
    };
    auto store_x = [&]() {
#pragma unroll
        for (int t = 0; t < 8; ++t)
            if (xd[t] >= 0) *reinterpret_cast<f4v*>(Xs + xd[t]) = xv[t];
    };
    // without expand: the chunk's 32 channels of the halo, 8 float4 per halo row
    f4v hq[UH], hq2[UH];
    auto load_h = [&](f4v (&hh)[UH], int ch) {
#pragma unroll
        for (int u = 0; u < UH; ++u) {
            const int e = tid + 256 * u;
            const int r = e >> 3, c = ch * CC + 4 * (e & 7);
            const int hy = udiv(r, a.m_hw), hx = r - hy * a.hw;
            const int iy = iy0 + hy, ix = ix0 + hx;
            const bool in = (r < a.hp) & (c < a.cin) & ((unsigned)iy < (unsigned)a.h) &
                            ((unsigned)ix < (unsigned)a.w_);
            hh[u] = ld16(xr, in ? (unsigned)((iy * a.w_ + ix) * a.cin + c) * 4u : kOob);
        }
    };
    auto store_h = [&](const f4v (&hh)[UH]) {
#pragma unroll
        for (int u = 0; u < UH; ++u) {
            const int e = tid + 256 * u;
            if (e < hrows * 8) {
                float* d = Es + (e >> 3) * ES + 4 * (e & 7);  // rows 33 floats apart
#pragma unroll
                for (int i = 0; i < 4; ++i) d[i] = hh[u][i];
            }
        }
    };
    // Without expand every chunk load is issued unconditionally, so the wait counts do not
    // depend on the path: a chunk past this split's end is asked for as chunk nchunk, which
    // lies past ce and reads zeros without a memory access.
    const int c_none = a.nchunk;
    if (EXP)
        load_x(tid);
    else
        load_h(hq, c_begin < c_end ? c_begin : c_none);

    // this thread's share of every chunk's weights, and the first chunk's loads
    int goff[NPF], meta[NPF];
#pragma unroll
    for (int u = 0; u < NPF; ++u) {
        goff[u] = meta[u] = 0;
        if (tid + 256 * u < nf) weight_slot<K>(a, L, j, tid + 256 * u, goff[u], meta[u]);
    }
    // (native vectors: HIP's float4 struct copies would pin them to scratch)
    f4v pf[EXP ? NPF : NPF_DP];
    const __amdgpu_buffer_rsrc_t wr =
        buffer_rsrc(a.w, a.w_wd + (int64_t)(K * K + 1 + a.cout) * a.ce + a.cout);
    fetch_weights<0>(pf, a, wr, goff, meta, tid, nf, c_begin < c_end ? c_begin : 0);
    // without expand the next chunk's halo and weights load too (a second register set): each
    // chunk's loads go out two chunks ahead of its use
    f4v pf2[EXP ? 1 : NPF_DP];
    if (!EXP) {
        const int c1 = c_begin + 1 < c_end ? c_begin + 1 : c_none;
        load_h(hq2, c1);
        fetch_weights<0>(pf2, a, wr, goff, meta, tid, nf, c1);
    }

    if (EXP) {
        store_x();
        for (int e0 = tid + 2048; e0 < xtotal; e0 += 2048) {  // patches of more than 2048 float4
            load_x(e0);
            store_x();
        }
        for (int r = tid; r < hrows; r += 256) {
            const int hy = udiv(r, a.m_hw), hx = r - hy * a.hw;
            const int iy = iy0 + hy, ix = ix0 + hx;
            hvalid[r] = r < a.hp && iy >= 0 && iy < a.h && ix >= 0 && ix < a.w_;
        }
    }
    // never written by the chunk staging: We padding columns, Wp rows past this slice and
    // the depthwise rows past the tile's pixels (read by the projection as zeros)
    if (EXP && a.cin16 > a.cin) {
        const int pc = a.cin16 - a.cin;
        for (int e = tid; e < CC * pc; e += 256) Ws[(e / pc) * a.xs + a.cin + e % pc] = 0.f;
    }
    for (int e = tid; e < (a.ob * 16 - cv) * CC; e += 256)
        Wps[(cv + e / CC) * WPS + e % CC] = 0.f;
    for (int e = tid; e < (a.pb * 16 - P) * CC; e += 256) Ds[(P + e / CC) * DS + e % CC] = 0.f;

    floatx4 acc[NBW];
#pragma unroll
    for (int i = 0; i < NBW; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int dc = tid & 31, dy = tid >> 5;  // depthwise: channel and output row of the tile
    auto body = [&](int ch) {  // one staged chunk: expand, depthwise, projection
        const int c0 = ch * CC;
        const bool half = c0 + 16 >= a.ce;  // a 16-channel last chunk: one column block
        if (EXP) {
            // E[halo pixel][32 channels]: lane group g sums the K quarter [g*Q, g*Q + Q) of
            // cin16, so each lane reads 16 contiguous bytes of its row per 4 MFMA steps; the
            // row block's x reads serve both column blocks, and the next step's operands are
            // read before this step's products issue
            const int Q = a.cin16 >> 2;
            const ActClamp act_e(a.act_e);
            const float be0 = Bes[li], be1 = Bes[16 + li];
            const float* wb0 = Ws + li * a.xs + g * Q;
            const float* wb1 = wb0 + 16 * a.xs;
            for (int hb = wave; hb < a.hpb; hb += 8) {  // row blocks hb and hb + 4
                const bool two = hb + 4 < a.hpb;
                const float* xa0 = Xs + (hb * 16 + li) * a.xs + g * Q;
                const float* xa1 = two ? xa0 + 64 * a.xs : xa0;
                // validity of this lane's 4 accumulator rows (one 16-byte read each, issued
                // ahead of the products instead of one dependent read per row after them)
                const int4 in0 = *reinterpret_cast<const int4*>(hvalid + hb * 16 + 4 * g);
                const int4 in1 = *reinterpret_cast<const int4*>(hvalid + (two ? hb + 4 : hb) * 16 + 4 * g);
                floatx4 e00 = {0.f, 0.f, 0.f, 0.f}, e01 = e00, e10 = e00, e11 = e00;
                f4v x0 = *reinterpret_cast<const f4v*>(xa0);
                f4v x1 = *reinterpret_cast<const f4v*>(xa1);
                f4v b0 = *reinterpret_cast<const f4v*>(wb0);
                f4v b1 = *reinterpret_cast<const f4v*>(wb1);
                for (int u = 4; u <= Q; u += 4) {
                    // (at u = Q the reads land in the rows' padding, 4 Q = cin16 < xs, unused)
                    const f4v nx0 = *reinterpret_cast<const f4v*>(xa0 + u);
                    const f4v nx1 = *reinterpret_cast<const f4v*>(xa1 + u);
                    const f4v nb0 = *reinterpret_cast<const f4v*>(wb0 + u);
                    const f4v nb1 = *reinterpret_cast<const f4v*>(wb1 + u);
                    // zero weights past ce (a 16-channel last chunk) in the second column block
                    e00 = mfma4(x0, b0, e00);
                    e01 = mfma4(x0, b1, e01);
                    if (two) {
                        e10 = mfma4(x1, b0, e10);
                        e11 = mfma4(x1, b1, e11);
                    }
                    x0 = nx0;
                    x1 = nx1;
                    b0 = nb0;
                    b1 = nb1;
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {  // accumulator r: row 4g + r, column li
                    const int row = hb * 16 + 4 * g + r;
                    const bool in = (&in0.x)[r];
                    Es[row * ES + li] = in ? act_e(e00[r] + be0) : 0.f;
                    Es[row * ES + 16 + li] = in && !half ? act_e(e01[r] + be1) : 0.f;
                    if (two) {
                        const bool in1r = (&in1.x)[r];
                        Es[(row + 64) * ES + li] = in1r ? act_e(e10[r] + be0) : 0.f;
                        Es[(row + 64) * ES + 16 + li] = in1r && !half ? act_e(e11[r] + be1) : 0.f;
                    }
                }
            }
            __syncthreads();
        }
        if (dy < a.th) {
            // depthwise, one output row of the tile per thread: the K x K window slides
            // along the row in registers (ST new columns per pixel); taps bias first, then
            // row by row as the reference sums them
            const float* src = Es + dc;
            const int rs = ES;
            const ActClamp act_d(a.act_d);
            float wk[K * K];
#pragma unroll
            for (int t = 0; t < K * K; ++t) wk[t] = Wds[t * CC + dc];
            const float bd = Bds[dc];
            float win[K][K];
            const int r0 = dy * ST * a.hw;
#pragma unroll
            for (int ky = 0; ky < K; ++ky)
#pragma unroll
                for (int kx = 0; kx < K; ++kx) win[ky][kx] = src[(r0 + ky * a.hw + kx) * rs];
#pragma unroll
            for (int px = 0; px < 8; ++px) {  // tw <= 8
                if (px >= a.tw) break;
                if (px > 0) {
                    const int c1 = px * ST;
#pragma unroll
                    for (int ky = 0; ky < K; ++ky) {
#pragma unroll
                        for (int kx = 0; kx < K - ST; ++kx) win[ky][kx] = win[ky][kx + ST];
#pragma unroll
                        for (int kx = K - ST; kx < K; ++kx)
                            win[ky][kx] = src[(r0 + ky * a.hw + c1 + kx) * rs];
                    }
                }
                float sacc = bd;
#pragma unroll
                for (int ky = 0; ky < K; ++ky)
#pragma unroll
                    for (int kx = 0; kx < K; ++kx) sacc = fmaf(win[ky][kx], wk[ky * K + kx], sacc);
                Ds[(dy * a.tw + px) * DS + dc] = act_d(sacc);
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NBW; ++i) {  // project the chunk's 32 channels
            const int b = wave + 4 * i;
            if (b < nblk) {
                const int pbi = b / a.ob, obi = b - pbi * a.ob;
                const float* da = Ds + (pbi * 16 + li) * DS + 8 * g;
                const float* wp = Wps + (obi * 16 + li) * WPS + 8 * g;
                acc[i] = mfma4(*reinterpret_cast<const f4v*>(da), *reinterpret_cast<const f4v*>(wp),
                               acc[i]);
                acc[i] = mfma4(*reinterpret_cast<const f4v*>(da + 4),
                               *reinterpret_cast<const f4v*>(wp + 4), acc[i]);
            }
        }
    };
    if constexpr (EXP) {
        for (int ch = c_begin; ch < c_end; ++ch) {
            __syncthreads();  // the previous chunk's readers are done with its weights, E and D
            put_weights<0>(pf, lds, meta, tid, nf);
            if (ch + 1 < c_end)  // the next chunk's weights load while this one computes
                fetch_weights<0>(pf, a, wr, goff, meta, tid, nf, ch + 1);
            __syncthreads();
            body(ch);
        }
    } else {
        // chunks in pairs, the first of a pair from set 1 (pf, hq) and the second from set 2
        // (pf2, hq2); a set, once stored, loads the chunk two ahead
        auto step = [&](f4v (&hh)[UH], f4v (&pp)[NPF_DP], int ch) {
            __syncthreads();  // the previous chunk's readers are done with its weights and D
            put_weights<0>(pp, lds, meta, tid, nf);
            store_h(hh);
            const int cn = ch + 2 < c_end ? ch + 2 : c_none;
            load_h(hh, cn);
            fetch_weights<0>(pp, a, wr, goff, meta, tid, nf, cn);
            __syncthreads();
            body(ch);
        };
        int ch = c_begin;
        for (; ch + 1 < c_end; ch += 2) {
            step(hq, pf, ch);
            step(hq2, pf2, ch + 1);
        }
        if (ch < c_end) step(hq, pf, ch);
    }

    // Output position (projection block b, lane l): 4 pixels of one output channel.  Its
    // bias and residuals load first (pre), ahead of the split sums, and the sums then store
    // with them (store); idx < 0 marks pixels outside the map.
    struct Out {
        int64_t idx[4];
        float bias;
        f4v res;
    };
    auto pre = [&](int b, int l) {
        Out u;
        const int pbi = b / a.ob, obi = b - pbi * a.ob;
        const int oo = obi * 16 + (l & 15);
        const int o = j * a.coj + oo;
        u.bias = 0.f;
        u.res = f4v{0.f, 0.f, 0.f, 0.f};
        if (oo < cv) u.bias = a.w[a.w_wd + (K * K + 1 + a.cout) * a.ce + o];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int p = pbi * 16 + 4 * (l >> 4) + r;
            const int py = udiv(p, a.m_tw), px = p - py * a.tw;
            const int oy = oy0 + py, ox = ox0 + px;
            const bool ok = oo < cv && p < P && oy < a.oh && ox < a.ow;
            u.idx[r] = ok ? (((int64_t)img * a.oh + oy) * a.ow + ox) * a.cout + o : -1;
            if (ok && a.res) u.res[r] = a.res[u.idx[r]];
        }
        return u;
    };
    auto store = [&](const Out& u, floatx4 v) {  // bias, residual, activation of 4 outputs
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (u.idx[r] >= 0)
                a.y[u.idx[r]] = shpd::apply_act(v[r] + u.bias + u.res[r], a.act_o, a.alpha);
    };

    if (a.S == 1) {
#pragma unroll
        for (int i = 0; i < NBW; ++i)
            if (wave + 4 * i < nblk) store(pre(wave + 4 * i, lane), acc[i]);
        return;
    }
    // split expanded channels: partials, then the last arrival sums them
    const int slot = tile * a.J + j;
    const int W = nblk * 64;  // float4 positions of one split's partial (block, lane)
    const __amdgpu_buffer_rsrc_t prs =
        buffer_rsrc(a.partial + (int64_t)slot * a.S * W * 4, (int64_t)a.S * W * 4);
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
        const int b = wave + 4 * i;
        if (b < nblk)
            st_coh16(prs, (unsigned)((si * W + b * 64 + lane) * 16),
                     make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]));
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partials are stored
    __syncthreads();
    int* flag = reinterpret_cast<int*>(lds + L.flag);
    int* cnt = a.counters + slot;
    if (tid == 0)
        *flag = __hip_atomic_fetch_add((SHP_GLOBAL int*)cnt, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == a.S - 1;
    __syncthreads();
    if (!*flag) return;
    // the last arrival: every thread sums its positions over the splits, in split order, and
    // stores their outputs; one position with up to 16 splits of loads in flight where the
    // tile fits one pass, else 2 positions x 8 splits
    if (W <= 256) {
        if (tid < W) {
            float4 q[16];
            f4v t = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < 16; ++u)
                if (u < a.S) q[u] = ld_coh16(prs, (unsigned)((u * W + tid) * 16), 0);
            const Out op = pre(tid >> 6, tid & 63);  // its loads go out behind the partials
#pragma unroll
            for (int u = 0; u < 16; ++u)
                if (u < a.S) t += f4v{q[u].x, q[u].y, q[u].z, q[u].w};
            for (int s0 = 16; s0 < a.S; s0 += 16) {
#pragma unroll
                for (int u = 0; u < 16; ++u)
                    if (s0 + u < a.S)
                        q[u] = ld_coh16(prs, (unsigned)(((s0 + u) * W + tid) * 16), 0);
#pragma unroll
                for (int u = 0; u < 16; ++u)
                    if (s0 + u < a.S) t += f4v{q[u].x, q[u].y, q[u].z, q[u].w};
            }
            store(op, floatx4{t.x, t.y, t.z, t.w});
        }
    } else
    for (int f0 = tid; f0 < W; f0 += 512) {
        float4 q[2][8];
        f4v t[2];
        Out op[2];
        for (int s0 = 0; s0 < a.S; s0 += 8) {
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (f0 + 256 * m < W && s0 + u < a.S)
                        q[m][u] = ld_coh16(prs, (unsigned)(((s0 + u) * W + f0 + 256 * m) * 16), 0);
            if (s0 == 0) {
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    const int f = min(f0 + 256 * m, W - 1);
                    op[m] = pre(f >> 6, f & 63);
                    t[m] = f4v{0.f, 0.f, 0.f, 0.f};
                }
            }
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (f0 + 256 * m < W && s0 + u < a.S)
                        t[m] += f4v{q[m][u].x, q[m][u].y, q[m][u].z, q[m][u].w};
        }
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int f = f0 + 256 * m;
            if (f < W) store(op[m], floatx4{t[m].x, t[m].y, t[m].z, t[m].w});
        }
    }
    if (tid == 0)
        __hip_atomic_store((SHP_GLOBAL int*)cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- host: shape, plan, launch ------------------------------------------------------------

struct IrShape {
    int n, cin, h, w, ce, cout, oh, ow, k, s, pt, pl, expand, act_e, act_d;
};

struct IrPlan {
    int th = 0, tw = 0, S = 1, J = 1;
    double cost = 1e30;
};

int ceil_div(int a, int b) { return (a + b - 1) / b; }

// LDS row stride for rows of c16 floats: congruent to 4 modulo 32, so the 16 rows one
// 16-byte MFMA operand read touches start 4 banks apart
int row_stride(int c16) { return c16 + (36 - c16 % 32) % 32; }

// Derived sizes of one plan (everything the kernel arguments need except pointers).
struct IrGeom {
    int tiles_y, tiles_x, tiles, hh, hw, hp, hpb, cin16, xs, nchunk, cpw, S, J, coj, ob, pb;
    int nblk, nbw, nf_max, lds_floats;
    bool expand;
};

IrGeom geometry(const IrShape& sh, int th, int tw, int S, int J) {
    IrGeom g{};
    g.tiles_y = ceil_div(sh.oh, th);
    g.tiles_x = ceil_div(sh.ow, tw);
    g.tiles = sh.n * g.tiles_y * g.tiles_x;
    g.hh = (th - 1) * sh.s + sh.k;
    g.hw = (tw - 1) * sh.s + sh.k;
    g.hp = g.hh * g.hw;
    g.hpb = ceil_div(g.hp, 16);
    g.cin16 = ceil_div(sh.cin, 16) * 16;
    g.xs = row_stride(g.cin16);
    g.nchunk = ceil_div(sh.ce, CC);
    g.cpw = ceil_div(g.nchunk, std::max(1, std::min(S, g.nchunk)));
    g.S = ceil_div(g.nchunk, g.cpw);  // no empty split
    const int ob_all = ceil_div(sh.cout, 16);
    g.ob = ceil_div(ob_all, std::max(1, std::min(J, ob_all)));
    g.coj = 16 * g.ob;
    g.J = ceil_div(sh.cout, g.coj);
    g.pb = ceil_div(th * tw, 16);
    g.nblk = g.pb * g.ob;
    g.nbw = ceil_div(g.nblk, 4);
    g.nf_max = (sh.expand ? CC * (sh.cin / 4) + 8 : 0) + 8 * sh.k * sh.k + 8 + 8 * g.coj;
    g.lds_floats = ir_lds(g.hpb, g.xs, sh.expand, sh.k, g.pb, g.ob).total;
    g.expand = sh.expand != 0;
    return g;
}

bool geometry_ok(const IrGeom& g) {
    return g.lds_floats * 4 <= kMaxLds && g.nbw <= 20 &&
           g.nf_max <= 256 * (g.expand ? NPF : NPF_DP) &&
           (g.expand || g.hpb * 16 * 8 <= 256 * UH) &&  // the halo chunk's float4 per thread
           (int64_t)g.S * g.nblk * 1024 < (1ll << 31) &&
           // the kernel's multiply-high divisions of the workgroup id stay exact
           (int64_t)g.tiles * g.J * g.S *
                   std::max(std::max(g.S, g.J), std::max(g.tiles_x, g.tiles_y)) < (1ll << 31) &&
           (g.S == 1 || (int64_t)g.tiles * g.J <= (int64_t)(shp::kSplitCounterBytes / sizeof(int))) &&
           (int64_t)g.tiles * g.J * g.S < (1ll << 31);
}

size_t workspace_bytes(const IrGeom& g) {
    if (g.S <= 1) return 0;
    return shp::kSplitCounterBytes + (size_t)g.tiles * g.J * g.S * g.nblk * 256 * sizeof(float);
}

// Estimated time of a plan in CU cycles (constants from MI355X phase timings of the
// kernel): the workgroups run in rounds of 256 (or 512 where two fit in a CU, each then
// ~1.6x slower); a workgroup pays the halo load, per 32-channel chunk the expand MFMAs of
// its busiest wavefront, the depthwise window loads and taps, the projection MFMAs and the
// chunk's barriers and weight staging, and with split channels the partial stores, the
// arrival count and, for the last arrival, the split-ordered sum in rounds of loads.
double plan_cost(const IrShape& sh, const IrGeom& g) {
    const double expand = sh.expand ? ceil_div(g.hpb, 4) * g.cin16 * 16.0 : 0.0;
    const double dw = g.hw * sh.k * 24.0 + (ceil_div(g.hp, g.hw) / sh.s) * 0.0 +
                      (g.hw / sh.s) * sh.k * sh.k * 4.0;
    const double proj = g.nbw * 8.0 * 32.0;
    const double chunk = expand + dw + proj + 1500.0;
    double wg = 7000.0 + g.cpw * chunk + 1000.0;
    if (g.S > 1)
        wg += 5000.0 + ceil_div(g.S, 8) * ceil_div(g.nblk * 64, 512) * 4000.0 + 2000.0;
    const int occ = std::max(1, std::min(2, kMaxLds / std::max(1, g.lds_floats * 4)));
    const double wgs = (double)g.tiles * g.J * g.S;
    const double rounds = std::ceil(wgs / (256.0 * occ));
    return rounds * wg * (occ > 1 && wgs > 256.0 ? 1.6 : 1.0);
}

// Plans measured best on MI355X for the MBConv blocks of the benchmark configs (every tile,
// split and output-channel slice per block, each timed as 20 launches of the block replayed
// from a hipGraph, beside the three operators conv2d_nhwc, depthwise_conv2d_nhwc, conv2d_nhwc
// timed the same way), and whether one launch beat the three operators; where the two were
// close the whole model's graph replay decided.  The cost model and the rule of fusion_pays
// cover every other shape.
struct TunedBlock {
    int n, cin, h, w, ce, cout, k, s, expand;
    int th, tw, S, J;
    bool fuse;
};
const TunedBlock kTunedBlocks[] = {
    // MobileNetV2-1.0 batch 1 (us per launch: one launch / three launches)
    {1, 32, 112, 112, 32, 16, 3, 1, 0, 7, 7, 1, 1, true},     // block0: 7.4 / 10.3
    {1, 16, 112, 112, 96, 24, 3, 2, 1, 8, 4, 3, 1, true},     // block1: 11.9 / 19.6
    {1, 24, 56, 56, 144, 24, 3, 1, 1, 8, 4, 4, 1, true},      // block2: 13.4 / 20.4
    {1, 24, 56, 56, 144, 32, 3, 2, 1, 4, 2, 3, 1, true},      // block3: 12.7 / 18.8
    {1, 32, 28, 28, 192, 32, 3, 1, 1, 8, 4, 6, 1, true},      // block4-5: 10.5 / 18.6
    {1, 32, 28, 28, 192, 64, 3, 2, 1, 7, 1, 6, 1, true},      // block6: 10.3 / 17.9
    {1, 64, 14, 14, 384, 64, 3, 1, 1, 8, 2, 12, 1, true},     // block7-9: 11.7 / 18.5
    {1, 64, 14, 14, 384, 96, 3, 1, 1, 8, 4, 12, 4, true},     // block10: 12.2 / 18.0
    {1, 96, 14, 14, 576, 96, 3, 1, 1, 8, 2, 16, 2, true},     // block11-12: 14.6 / 19.9
    {1, 96, 14, 14, 576, 160, 3, 2, 1, 7, 1, 16, 4, true},    // block13: 14.6 / 19.9
    {1, 160, 7, 7, 960, 160, 3, 1, 1, 4, 4, 16, 3, true},     // block14-15: 16.8 / 21.7
    {1, 160, 7, 7, 960, 320, 3, 1, 1, 7, 2, 16, 3, false},    // block16: 18.7 / 16.3
    // EfficientNet-Lite0 batch 8
    {8, 32, 112, 112, 32, 16, 3, 1, 0, 8, 7, 1, 1, true},     // block0: 24.6 / 29.5
    {8, 16, 112, 112, 96, 24, 3, 2, 1, 7, 4, 1, 1, true},     // block1: 32.5 / 42.7
    {8, 24, 56, 56, 144, 24, 3, 1, 1, 8, 7, 1, 1, true},      // block2: 27.2 / 43.5
    {8, 24, 56, 56, 144, 40, 5, 2, 1, 7, 2, 1, 1, true},      // block3: 24.6 / 41.6
    {8, 40, 28, 28, 240, 40, 5, 1, 1, 7, 7, 4, 1, false},     // block4: 24.0 / 28.2
    {8, 40, 28, 28, 240, 80, 3, 2, 1, 8, 2, 4, 1, true},      // block5: 17.4 / 27.5
    {8, 80, 14, 14, 480, 80, 3, 1, 1, 7, 4, 8, 1, false},     // block6-7: 22.6 / 25.6
    {8, 80, 14, 14, 480, 112, 5, 1, 1, 4, 4, 4, 1, false},    // block8: 26.3 / 29.5
    {8, 112, 14, 14, 672, 112, 5, 1, 1, 4, 4, 4, 1, false},   // block9-10: 38.5 / 36.5
    {8, 112, 14, 14, 672, 192, 5, 2, 1, 7, 2, 8, 1, false},   // block11: 28.0 / 28.8
    {8, 192, 7, 7, 1152, 192, 5, 1, 1, 7, 4, 8, 2, false},    // block12-14: 45.6 / 29.7
    {8, 192, 7, 7, 1152, 320, 3, 1, 1, 7, 4, 8, 2, false},    // block15: 42.7 / 27.8
    // EfficientNet-Lite0 batch 8, the blocks above that do not fuse whole: depthwise +
    // projection as one launch after the expand GEMM (us: one launch / two launches)
    {8, 240, 28, 28, 240, 40, 5, 1, 0, 8, 4, 2, 1, true},     // block4: 16.2 / 21.0
    {8, 480, 14, 14, 480, 80, 3, 1, 0, 7, 2, 4, 1, true},     // block6-7: 15.6 / 16.5
    {8, 480, 14, 14, 480, 112, 5, 1, 0, 8, 2, 4, 1, true},    // block8: 16.7 / 19.8
    {8, 672, 14, 14, 672, 112, 5, 1, 0, 8, 2, 4, 1, true},    // block9-10: 20.7 / 22.9
    {8, 672, 14, 14, 672, 192, 5, 2, 0, 7, 2, 8, 2, false},   // block11: 16.0 / 15.4
    {8, 1152, 7, 7, 1152, 192, 5, 1, 0, 7, 2, 8, 2, true},    // block12-14: 19.0 / 19.6
    {8, 1152, 7, 7, 1152, 320, 3, 1, 0, 7, 4, 8, 4, false},   // block15: 23.5 / 17.9
};

const TunedBlock* tuned_block(const IrShape& sh) {
    for (const TunedBlock& t : kTunedBlocks)
        if (t.n == sh.n && t.cin == sh.cin && t.h == sh.h && t.w == sh.w && t.ce == sh.ce &&
            t.cout == sh.cout && t.k == sh.k && t.s == sh.s && t.expand == sh.expand)
            return &t;
    return nullptr;
}

// Whether one launch is expected to beat the three-operator form: the measured verdict for
// the blocks above; elsewhere, for blocks with an expand, where the separate launches are
// latency-bound (at most 1024 output pixels in the batch) or the expand is a thin,
// memory-bound product (cin <= 48) whose output the fused form never writes.
bool fusion_pays(const IrShape& sh) {
    if (const TunedBlock* t = tuned_block(sh)) return t->fuse;
    return sh.expand && ((int64_t)sh.n * sh.oh * sh.ow <= 1024 || sh.cin <= 48);
}

IrPlan choose_plan(const IrShape& sh, const shp::GemmTune& tn, bool allow_split) {
    static std::mutex mu;
    static std::map<std::tuple<std::vector<int>, bool>, IrPlan> cache;
    const std::vector<int> key{sh.n, sh.cin, sh.h, sh.w, sh.ce, sh.cout, sh.oh, sh.ow, sh.k,
                               sh.s, sh.pt, sh.pl, sh.expand, tn.ir_th, tn.ir_tw, tn.ir_s,
                               tn.ir_j};
    {
        std::lock_guard<std::mutex> lk(mu);
        auto it = cache.find({key, allow_split});
        if (it != cache.end()) return it->second;
    }
    IrPlan best;
    const TunedBlock* tb = tuned_block(sh);
    if (tb && !tn.ir_th && !tn.ir_tw && !tn.ir_s && !tn.ir_j && (tb->S == 1 || allow_split)) {
        const IrGeom g = geometry(sh, tb->th, tb->tw, tb->S, tb->J);
        if (geometry_ok(g)) best = IrPlan{tb->th, tb->tw, g.S, g.J, plan_cost(sh, g)};
    }
    const int nchunk = ceil_div(sh.ce, CC);
    const int ob_all = ceil_div(sh.cout, 16);
    const int force_s = std::min(tn.ir_s, nchunk), force_j = std::min(tn.ir_j, ob_all);
    static const int kEdge[] = {8, 7, 4, 2, 1};
    if (best.th) {
        std::lock_guard<std::mutex> lk(mu);
        cache[{key, allow_split}] = best;
        return best;
    }
    static const int kSplit[] = {1, 2, 3, 4, 5, 6, 8, 10, 12, 15, 16, 20, 24, 30, 36, 40, 48, 60, 72};
    for (int th0 : kEdge) {
        const int th = std::min(th0, sh.oh);
        if (tn.ir_th && th != std::min(tn.ir_th, sh.oh)) continue;
        for (int tw0 : kEdge) {
            const int tw = std::min(tw0, sh.ow);
            if (tn.ir_tw && tw != std::min(tn.ir_tw, sh.ow)) continue;
            if (th * tw > 64) continue;
            std::vector<int> splits(std::begin(kSplit), std::end(kSplit));
            if (force_s > 0) splits.assign(1, force_s);
            for (int S : splits) {
                if (S > nchunk || (S > 1 && !allow_split)) continue;
                for (int J = 1; J <= ob_all && J <= 8; ++J) {
                    if (force_j > 0 && J != force_j) continue;
                    const IrGeom g = geometry(sh, th, tw, S, J);
                    if (g.S != S && force_s <= 0) continue;  // duplicate of a smaller S
                    if (g.J != J && force_j <= 0) continue;
                    if (!geometry_ok(g)) continue;
                    const double c = plan_cost(sh, g);
                    if (c < best.cost * 0.999) best = IrPlan{th, tw, g.S, g.J, c};
                }
            }
        }
    }
    std::lock_guard<std::mutex> lk(mu);
    cache[{key, allow_split}] = best;
    return best;
}

int parse(const int32_t* q, size_t n, IrShape& sh) {
    if (n < 16)
        return shp::fail(SHP_ERR_PUSH, "inverted_residual_nhwc needs 16 push constants");
    sh = IrShape{q[0], q[1], q[2], q[3], q[4], q[5], q[6], q[7], q[8], q[9], q[10], q[11],
                 q[12], q[13], q[14]};
    if (sh.n <= 0 || sh.cin <= 0 || sh.h <= 0 || sh.w <= 0 || sh.ce <= 0 || sh.cout <= 0 ||
        sh.oh <= 0 || sh.ow <= 0 || sh.k <= 0 || sh.s <= 0)
        return shp::fail(SHP_ERR_SHAPE, "inverted_residual_nhwc: non-positive dim");
    if ((sh.k != 3 && sh.k != 5) || sh.s > 2 || sh.pt < 0 || sh.pl < 0 || sh.pt >= sh.k ||
        sh.pl >= sh.k)
        return shp::fail(SHP_ERR_UNSUPPORTED,
                         "inverted_residual_nhwc: kernel 3 or 5, stride 1 or 2, padding < kernel");
    if (sh.cin % 4 || sh.ce % 16)
        return shp::fail(SHP_ERR_UNSUPPORTED,
                         "inverted_residual_nhwc: cin must be a multiple of 4, ce of 16");
    auto clamp_act = [](int act) {
        return act == SHP_ACT_NONE || act == SHP_ACT_RELU || act == SHP_ACT_RELU6;
    };
    if (!clamp_act(sh.act_e) || !clamp_act(sh.act_d))
        return shp::fail(SHP_ERR_UNSUPPORTED,
                         "inverted_residual_nhwc: expand/depthwise activation must be none, "
                         "relu or relu6");
    if (sh.expand != 0 && sh.expand != 1)
        return shp::fail(SHP_ERR_SHAPE, "inverted_residual_nhwc: expand must be 0 or 1");
    if (!sh.expand && sh.ce != sh.cin)
        return shp::fail(SHP_ERR_SHAPE, "inverted_residual_nhwc: ce != cin without expand");
    if ((int64_t)(sh.oh - 1) * sh.s - sh.pt >= sh.h || (int64_t)(sh.ow - 1) * sh.s - sh.pl >= sh.w)
        return shp::fail(SHP_ERR_SHAPE, "inverted_residual_nhwc: output window outside input");
    if ((int64_t)q[15] != (int64_t)sh.n * sh.oh * sh.ow * sh.cout)
        return shp::fail(SHP_ERR_SHAPE, "inverted_residual_nhwc: total != n*oh*ow*cout");
    const int64_t wn = (sh.expand ? (int64_t)sh.ce * sh.cin + sh.ce : 0) +
                       (int64_t)sh.k * sh.k * sh.ce + sh.ce + (int64_t)sh.cout * sh.ce + sh.cout;
    // the halo and weight loads are buffer loads with 32-bit byte offsets over one image of x
    // and over the packed weights
    if (wn * 4 >= (1ll << 31) || (int64_t)sh.h * sh.w * sh.cin * 4 >= (1ll << 31) ||
        (int64_t)sh.n * sh.h * sh.w * sh.cin >= (1ll << 40))
        return shp::fail(SHP_ERR_SHAPE, "inverted_residual_nhwc: tensors too large");
    return SHP_OK;
}

template <int K, int ST, int NBW, bool EXP>
int launch_variant(hipStream_t stream, const IrArgs& a, unsigned grid, size_t lds) {
    if (lds > 64 * 1024)
        SHP_HIP_CHECK(hipFuncSetAttribute((const void*)ir_kernel<K, ST, NBW, EXP>,
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL((ir_kernel<K, ST, NBW, EXP>), dim3(grid), dim3(256), lds, stream, a);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

template <int K, int ST, bool EXP>
int launch_nbw_e(hipStream_t stream, const IrArgs& a, int nbw, unsigned grid, size_t lds) {
    if (nbw <= 2) return launch_variant<K, ST, 2, EXP>(stream, a, grid, lds);
    if (nbw <= 4) return launch_variant<K, ST, 4, EXP>(stream, a, grid, lds);
    if (nbw <= 8) return launch_variant<K, ST, 8, EXP>(stream, a, grid, lds);
    return launch_variant<K, ST, 20, EXP>(stream, a, grid, lds);
}
template <int K, int ST>
int launch_nbw(hipStream_t stream, const IrArgs& a, int nbw, unsigned grid, size_t lds) {
    return a.expand ? launch_nbw_e<K, ST, true>(stream, a, nbw, grid, lds)
                    : launch_nbw_e<K, ST, false>(stream, a, nbw, grid, lds);
}

int launch_ir(const shp::Launch& l) {
    IrShape sh;
    int rc = parse(l.push, l.n_push, sh);
    if (rc) return rc;
    rc = shp::check_total(l, (int64_t)sh.n * sh.oh * sh.ow * sh.cout, "inverted_residual_nhwc");
    if (rc) return rc;
    if (l.epi->bias)
        return shp::fail(SHP_ERR_INVALID,
                         "inverted_residual_nhwc: the biases are part of the packed weights");
    auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (!l.in0 || !l.in1 || !l.out || !a16(l.in0) || !a16(l.in1))
        return shp::fail(SHP_ERR_UNSUPPORTED,
                         "inverted_residual_nhwc: x and the weights must be 16-byte aligned");
    static const shp::GemmTune kAuto;
    const shp::GemmTune& tn = l.tune ? *l.tune : kAuto;
    IrPlan pl = choose_plan(sh, tn, true);
    IrGeom g = pl.th ? geometry(sh, pl.th, pl.tw, pl.S, pl.J) : IrGeom{};
    if (pl.th && g.S > 1 && (l.workspace == nullptr || l.workspace_bytes < workspace_bytes(g))) {
        pl = choose_plan(sh, tn, false);  // no room for partials: one split per tile
        if (pl.th) g = geometry(sh, pl.th, pl.tw, pl.S, pl.J);
    }
    if (!pl.th)
        return shp::fail(SHP_ERR_UNSUPPORTED,
                         "inverted_residual_nhwc: no tile of this block fits the LDS");
    IrArgs a{};
    a.x = (const float*)l.in0;
    a.w = (const float*)l.in1;
    a.y = (float*)l.out;
    a.res = l.epi->residual;
    a.partial = g.S > 1 ? l.workspace + shp::kSplitCounterBytes / sizeof(float) : nullptr;
    a.counters = g.S > 1 ? reinterpret_cast<int*>(l.workspace) : nullptr;
    a.n = sh.n; a.h = sh.h; a.w_ = sh.w; a.cin = sh.cin; a.ce = sh.ce; a.cout = sh.cout;
    a.oh = sh.oh; a.ow = sh.ow; a.pt = sh.pt; a.pl = sh.pl;
    a.expand = sh.expand; a.act_e = sh.act_e; a.act_d = sh.act_d; a.act_o = l.epi->act;
    a.alpha = l.epi->alpha;
    a.th = pl.th; a.tw = pl.tw; a.tiles_y = g.tiles_y; a.tiles_x = g.tiles_x;
    a.hw = g.hw; a.hp = g.hp; a.hpb = g.hpb;
    a.cin16 = g.cin16; a.xs = g.xs;
    a.nchunk = g.nchunk; a.cpw = g.cpw; a.S = g.S;
    a.J = g.J; a.coj = g.coj; a.ob = g.ob; a.pb = g.pb;
    auto magic = [](int d) { return (unsigned)(0xFFFFFFFFull / (uint64_t)d); };
    a.m_cin4 = magic(sh.cin / 4);
    a.m_c4n = magic(g.cin16 / 4);
    a.m_hw = magic(g.hw);
    a.m_tw = magic(pl.tw);
    a.m_S = magic(g.S);
    a.m_J = magic(g.J);
    a.m_tx = magic(g.tiles_x);
    a.m_ty = magic(g.tiles_y);
    a.w_wd = sh.expand ? sh.ce * (sh.cin + 1) : 0;
    const unsigned grid = (unsigned)((int64_t)g.tiles * g.J * g.S);
    const size_t lds = (size_t)g.lds_floats * sizeof(float);
    if (sh.k == 3)
        return sh.s == 1 ? launch_nbw<3, 1>(l.stream, a, g.nbw, grid, lds)
                         : launch_nbw<3, 2>(l.stream, a, g.nbw, grid, lds);
    return sh.s == 1 ? launch_nbw<5, 1>(l.stream, a, g.nbw, grid, lds)
                     : launch_nbw<5, 2>(l.stream, a, g.nbw, grid, lds);
}

}  // namespace

namespace shp {

bool block_fusion_pays(const int32_t* push, size_t n_push) {
    IrShape sh;
    if (!push || parse(push, n_push, sh) != SHP_OK) {
        set_error("");
        return false;
    }
    static const GemmTune kAuto;
    return fusion_pays(sh) && choose_plan(sh, kAuto, true).th > 0;
}

size_t block_workspace_for_kernel(const int32_t* push, size_t n_push, const GemmTune* tune) {
    IrShape sh;
    if (!push || parse(push, n_push, sh) != SHP_OK) {
        set_error("");
        return 0;
    }
    static const GemmTune kAuto;
    const IrPlan pl = choose_plan(sh, tune ? *tune : kAuto, true);
    if (!pl.th) return 0;
    return workspace_bytes(geometry(sh, pl.th, pl.tw, pl.S, pl.J));
}

}  // namespace shp

// The plan the launcher picks for this push vector (default tune, workspace large enough)
// and whether one launch is expected to beat the three operators:
// {th, tw, S, J, LDS bytes, workgroups, projection blocks per wavefront, fusion pays}.
extern "C" int shp_block_plan(const int32_t* push, size_t n_push, int32_t* out8) {
    IrShape sh;
    if (!push || !out8) return shp::fail(SHP_ERR_INVALID, "shp_block_plan: null argument");
    int rc = parse(push, n_push, sh);
    if (rc) return rc;
    static const shp::GemmTune kAuto;
    const IrPlan pl = choose_plan(sh, kAuto, true);
    if (!pl.th) return shp::fail(SHP_ERR_UNSUPPORTED, "shp_block_plan: no plan");
    const IrGeom g = geometry(sh, pl.th, pl.tw, pl.S, pl.J);
    const int32_t v[8] = {pl.th, pl.tw, g.S, g.J, g.lds_floats * 4, g.tiles * g.J * g.S, g.nbw,
                          fusion_pays(sh) ? 1 : 0};
    std::memcpy(out8, v, sizeof v);
    return SHP_OK;
}

namespace {

// ---- conv1x1_gap_nhwc: the classifier head's 1x1 convolution, its activation and the global
// average pool in one launch (the TFLite graph's CONV_2D + MEAN, scheduler.rs:321-427 and
// :549-613).  push {n, cin, h, w, cout, total = n * cout}; in1 = [cout][cin] weights + bias
// tail; the epilogue's activation applies per pixel, before the mean.  A workgroup owns one
// image and 16 output channels: each wavefront takes 16-pixel row blocks and runs the
// product on v_mfma_f32_16x16x4_f32 (lane group g reads the K quarter [4g, 4g + 4) of every
// 16-wide K step, 16 contiguous bytes, for x and the weights alike), two accumulators on
// alternate K steps, operands loaded eight K steps at a time one group ahead; the activated
// pixels are summed per lane, across the lane groups and across the wavefronts in LDS, and
// divided by h * w as the reference pool does.  The convolution's output never reaches
// memory.
__global__ __launch_bounds__(256) void conv1x1_gap_kernel(const float* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          float* __restrict__ y, int cin,
                                                          int hw, int cout, int cblk, int act,
                                                          float alpha) {
    __shared__ float part[4][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, li = lane & 15;
    const int img = blockIdx.x / cblk, c0 = (blockIdx.x - img * cblk) * 16;
    const int col = c0 + li;
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(x + (int64_t)img * hw * cin, (int64_t)hw * cin);
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(w, (int64_t)cout * cin + cout);
    const bool col_ok = col < cout;
    const unsigned wrow = (unsigned)(col * cin) * 4u;
    const float bias = col_ok ? w[(int64_t)cout * cin + col] : 0.f;
    const int nrb = (hw + 15) >> 4;
    float sum = 0.f;
    constexpr int G = 8;  // 16-wide K steps per load group (K 128)
    for (int rb = wave; rb < nrb; rb += 4) {
        const int px = rb * 16 + li;
        const bool px_ok = px < hw;
        const unsigned xrow = (unsigned)(px * cin) * 4u;
        floatx4 e0 = {0.f, 0.f, 0.f, 0.f}, e1 = e0;
        // a group's 2 x G loads go out together, and the next group's before this group's
        // products, so the L2 round trips overlap instead of one per K step
        f4v xa[G], wb[G];
        auto load = [&](f4v (&xv)[G], f4v (&wv)[G], int k0) {
#pragma unroll
            for (int c = 0; c < G; ++c) {
                const int k = k0 + 16 * c + 4 * g;
                xv[c] = ld16(xr, px_ok && k < cin ? xrow + 4u * k : kOob);
                wv[c] = ld16(wr, col_ok && k < cin ? wrow + 4u * k : kOob);
            }
        };
        load(xa, wb, 0);
        for (int k0 = 0; k0 < cin; k0 += 16 * G) {
            f4v xn[G], wn[G];
            if (k0 + 16 * G < cin) load(xn, wn, k0 + 16 * G);
#pragma unroll
            for (int c = 0; c < G; c += 2) {
                e0 = mfma4(xa[c], wb[c], e0);
                e1 = mfma4(xa[c + 1], wb[c + 1], e1);
            }
#pragma unroll
            for (int c = 0; c < G; ++c) {
                xa[c] = xn[c];
                wb[c] = wn[c];
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // accumulator r: pixel rb * 16 + 4g + r, channel li
            const float v = shpd::apply_act(e0[r] + e1[r] + bias, act, alpha);
            sum += rb * 16 + 4 * g + r < hw ? v : 0.f;
        }
    }
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
    if (g == 0) part[wave][li] = sum;
    __syncthreads();
    if (tid < 16 && c0 + tid < cout)
        y[(int64_t)img * cout + c0 + tid] =
            (part[0][tid] + part[1][tid] + part[2][tid] + part[3][tid]) / (float)hw;
}

// The same head for maps of at most 64 pixels and at most 512 input channels (the 7x7
// heads), with the K steps split over the NWV wavefronts instead of the row blocks: wavefront w
// takes the 16-wide K steps w, w + NWV, ... for all four row blocks and CB column blocks, and
// issues every operand load of its share at once (one round trip to L2 / HBM instead of one
// per load group); the partial products meet in LDS, summed in wavefront order, and
// wavefront r < 4 then finishes row block r as the kernel above does.  Eight wavefronts (half
// the K steps each, twice the loads in flight per CU) against four: MobileNetV2 b1 forward
// 0.2366 -> 0.2349 ms, EfficientNet-Lite0 b8 0.4148 -> 0.4141 ms.
template <int CB, int NWV = 4>
__global__ __launch_bounds__(64 * NWV) void conv1x1_gap_small_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ w,
                                                                float* __restrict__ y, int cin,
                                                                int hw, int cout, int cblk,
                                                                int act, float alpha) {
    constexpr int NK = 32 / NWV;  // K steps per wavefront: cin <= 512
    __shared__ f4v red[NWV][4][CB][64];
    __shared__ float part[4][16 * CB];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, li = lane & 15;
    const int img = blockIdx.x / cblk, c0 = (blockIdx.x - img * cblk) * 16 * CB;
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(x + (int64_t)img * hw * cin, (int64_t)hw * cin);
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(w, (int64_t)cout * cin + cout);
    const int nch = (cin + 15) >> 4;
    float biasv[CB];  // the epilogue's biases load with the operands
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        const int col = c0 + cb * 16 + li;
        biasv[cb] = col < cout ? w[(int64_t)cout * cin + col] : 0.f;
    }
    f4v xa[NK][4], wb[NK][CB];
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        const int k = 16 * (wave + NWV * i) + 4 * g;
        const bool kok = k < cin;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const int px = rb * 16 + li;
            xa[i][rb] = ld16(xr, kok && px < hw ? (unsigned)(px * cin + k) * 4u : kOob);
        }
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const int col = c0 + cb * 16 + li;
            wb[i][cb] = ld16(wr, kok && col < cout ? (unsigned)(col * cin + k) * 4u : kOob);
        }
    }
    floatx4 acc[4][CB];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        if (wave + NWV * i < nch) {
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = mfma4(xa[i][rb], wb[i][cb], acc[rb][cb]);
        }
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
            red[wave][rb][cb][lane] = f4v{acc[rb][cb][0], acc[rb][cb][1], acc[rb][cb][2], acc[rb][cb][3]};
    __syncthreads();
    const int rb = wave;
    if (rb < 4) {
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        const float bias = biasv[cb];
        f4v v = red[0][rb][cb][lane];
#pragma unroll
        for (int u = 1; u < NWV; ++u) v += red[u][rb][cb][lane];
        float sum = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // pixel rb * 16 + 4g + r, channel li of block cb
            const float a = shpd::apply_act(v[r] + bias, act, alpha);
            sum += rb * 16 + 4 * g + r < hw ? a : 0.f;
        }
        sum += __shfl_xor(sum, 16);
        sum += __shfl_xor(sum, 32);
        if (g == 0) part[rb][cb * 16 + li] = sum;
    }
    }
    __syncthreads();
    if (tid < 16 * CB && c0 + tid < cout)
        y[(int64_t)img * cout + c0 + tid] =
            (part[0][tid] + part[1][tid] + part[2][tid] + part[3][tid]) / (float)hw;
}

int launch_conv1x1_gap(const shp::Launch& l) {
    if (l.n_push < 6) return shp::fail(SHP_ERR_PUSH, "conv1x1_gap_nhwc needs 6 push constants");
    const int32_t* q = l.push;
    const int n = q[0], cin = q[1], h = q[2], wd = q[3], cout = q[4];
    if (n <= 0 || cin <= 0 || h <= 0 || wd <= 0 || cout <= 0)
        return shp::fail(SHP_ERR_SHAPE, "conv1x1_gap_nhwc: non-positive dim");
    if ((int64_t)q[5] != (int64_t)n * cout)
        return shp::fail(SHP_ERR_SHAPE, "conv1x1_gap_nhwc: total != n*cout");
    int rc = shp::check_total(l, (int64_t)n * cout, "conv1x1_gap_nhwc");
    if (rc) return rc;
    if (l.epi->bias || l.epi->residual)
        return shp::fail(SHP_ERR_INVALID,
                         "conv1x1_gap_nhwc: the bias is the weights' tail; no residual");
    auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (cin % 4 || !l.in0 || !l.in1 || !a16(l.in0) || !a16(l.in1))
        return shp::fail(SHP_ERR_UNSUPPORTED,
                         "conv1x1_gap_nhwc: cin must be a multiple of 4, x and weights 16-byte "
                         "aligned");
    // buffer loads with 32-bit byte offsets over one image of x and over the weights
    const int64_t hw = (int64_t)h * wd;
    if (hw * cin * 4 >= (1ll << 31) || ((int64_t)cout * cin + cout) * 4 >= (1ll << 31))
        return shp::fail(SHP_ERR_SHAPE, "conv1x1_gap_nhwc: tensors too large");
    const int cblk = (cout + 15) / 16;
    if ((int64_t)n * cblk >= (1ll << 31))
        return shp::fail(SHP_ERR_SHAPE, "conv1x1_gap_nhwc: grid too large");
    if (hw <= 64 && cin <= 512) {
        // two column blocks per workgroup once that still leaves >= 256 workgroups
        const int cb2 = (cout + 31) / 32;
        if ((int64_t)n * cb2 >= 256) {
            hipLaunchKernelGGL((conv1x1_gap_small_kernel<2, 8>), dim3((unsigned)(n * cb2)), dim3(512),
                               0, l.stream, (const float*)l.in0, (const float*)l.in1,
                               (float*)l.out, cin, (int)hw, cout, cb2, l.epi->act, l.epi->alpha);
        } else {
            hipLaunchKernelGGL((conv1x1_gap_small_kernel<1, 8>), dim3((unsigned)(n * cblk)), dim3(512),
                               0, l.stream, (const float*)l.in0, (const float*)l.in1,
                               (float*)l.out, cin, (int)hw, cout, cblk, l.epi->act, l.epi->alpha);
        }
        SHP_HIP_CHECK(hipGetLastError());
        return SHP_OK;
    }
    hipLaunchKernelGGL(conv1x1_gap_kernel, dim3((unsigned)(n * cblk)), dim3(256), 0, l.stream,
                       (const float*)l.in0, (const float*)l.in1, (float*)l.out, cin, (int)hw,
                       cout, cblk, l.epi->act, l.epi->alpha);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

}  // namespace

namespace shp {

KernelEntry kBlockKernels[] = {
    {"inverted_residual_nhwc", 16, true, launch_ir},
    {"conv1x1_gap_nhwc", 6, true, launch_conv1x1_gap},
};
const int kBlockKernelCount = sizeof(kBlockKernels) / sizeof(kBlockKernels[0]);

}  // namespace shp
