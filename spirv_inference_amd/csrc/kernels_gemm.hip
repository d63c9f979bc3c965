// Dense contractions on the fp32 matrix cores of gfx950 (v_mfma_f32_32x32x2_f32).
#include "model.h"
//
// One implicit-GEMM kernel template serves every dense kernel of the reference:
//   hlo_conv_nhwc_hwio  kernels/hlo_conv_nhwc_hwio/glsl/hlo_conv_nhwc_hwio.comp:25-49
//                       (host: source/xla_hlo/src/compiler.rs:768-855)
//   conv2d              kernels/conv2d/glsl/conv2d.comp:26-50 (NCHW, OIHW + bias tail,
//                       host: source/tflite_loader/src/scheduler.rs:321-427,1327-1362)
//   fully_connected     kernels/fully_connected/glsl/fully_connected.comp:15-28 ([out,in] +
//                       bias tail, host: scheduler.rs:914-1002,1402-1436)
//   hlo_dot_batched     kernels/hlo_dot_batched/glsl/hlo_dot_batched.comp:19-38
//   hlo_dot_rank2       kernels/hlo_dot_rank2/glsl/hlo_dot_rank2.comp:15-26
// The reference computes one output per invocation with a serial K loop and no tiling.
// Here a 256-thread workgroup (4 wavefronts) owns a BM x BN output tile; K advances in
// tiles of 32 staged through LDS with double buffering; each wavefront accumulates
// FM x FN blocks of 32x32 in the MFMA accumulators.  A and B are read in place in
// whatever layout the caller has (NHWC im2col, NCHW im2col, row-major, transposed,
// strided batch), so no host-side permutes (compiler.rs:1043-1058) are needed.  The
// epilogue fuses bias, residual and activation; K can be split across workgroups with a
// deterministic second pass when the tile grid alone cannot fill 256 CUs.
#include "gemm.h"
#include "coherent.h"

namespace {

using shp::GemmParams;
typedef float floatx16 __attribute__((ext_vector_type(16)));

// Output tile (tm, tn) and K split of this workgroup.  The grid is (tiles, splits, batch);
// a workgroup's linear id within its batch slice, y * tiles + x, runs on XCD id % 8, and each
// XCD has its own L2.  The first (total / 8) * 8 ids are renumbered so XCD x takes the
// contiguous run [x * total / 8, (x + 1) * total / 8) of an order in which the split varies
// slowest (the rest keep their ids): with 2, 4 or 8 splits each XCD then works inside one K
// range and reads only that range of A and B.  Within a split the order walks bands of
// `group` tile rows column by column, so a run covers about group rows x (run / group)
// columns: A and B panels read by one XCD ~ group + run / group instead of 1 + run (row
// major, group 1) when a run spans many columns.  `tile` = tm * tiles_n + tn identifies the
// tile across its splits (the split-K arrival counters).
struct WgCoords {
    int tm, tn, split, tile;
};
__device__ __forceinline__ WgCoords wg_coords(int tiles_m, int tiles_n, int splits, int group) {
    const int ntiles = tiles_m * tiles_n;
    const int total = ntiles * splits;
    int pos = (int)(blockIdx.y * gridDim.x + blockIdx.x);
    const int full = (total / 8) * 8;
    if (pos < full) pos = (pos % 8) * (full / 8) + pos / 8;
    WgCoords c;
    c.split = pos / ntiles;
    const int t = pos - c.split * ntiles;
    const int g = group > 1 ? group : 1;
    const int band = t / (g * tiles_n);
    const int within = t - band * g * tiles_n;
    const int rows = min(g, tiles_m - band * g);
    c.tm = band * g + within % rows;
    c.tn = within / rows;
    c.tile = c.tm * tiles_n + c.tn;
    return c;
}

constexpr int KTAB = 1024;  // im2col offset table entries (scalar conv modes)

struct ConvRow {
    int64_t base;  // element offset of tap (0,0) of this output pixel (may be "negative")
    int iy0, ix0;  // top-left input coordinate of the window
    bool valid;
};

__device__ __forceinline__ ConvRow conv_row(const GemmParams& p, int m, int amode) {
    ConvRow r;
    r.valid = m < p.M;
    int mm = r.valid ? m : 0;
    int ox = mm % p.cow;
    int t = mm / p.cow;
    int oy = t % p.coh;
    int img = t / p.coh;
    r.iy0 = oy * p.csh - p.cpt;
    r.ix0 = ox * p.csw - p.cpl;
    if (amode == shp::A_CONV_NCHW) {
        r.base = (int64_t)img * p.cic * p.cih * p.ciw + (int64_t)r.iy0 * p.ciw + r.ix0;
    } else {
        r.base = (int64_t)img * p.cih * p.ciw * p.cic +
                 ((int64_t)r.iy0 * p.ciw + r.ix0) * p.cic;
    }
    return r;
}

// Decompose a K index of a convolution into (element offset, ky, kx).
__device__ __forceinline__ void conv_k(const GemmParams& p, int k, int amode, int& off, int& ky,
                                       int& kx) {
    if (amode == shp::A_CONV_NCHW) {  // k = (ic, ky, kx)
        kx = k % p.ckw;
        int t = k / p.ckw;
        ky = t % p.ckh;
        int ic = t / p.ckh;
        off = (ic * p.cih + ky) * p.ciw + kx;
    } else {  // k = (ky, kx, ic)
        int ic = k % p.cic;
        int t = k / p.cic;
        kx = t % p.ckw;
        ky = t / p.ckw;
        off = (ky * p.ciw + kx) * p.cic + ic;
    }
}

// ---- epilogue shared by the GEMM kernels.  Accumulator register r of a 32x32 block holds
// row 8*(r/4) + 4*(lane/32) + r%4 and column lane%32.  The tile goes through LDS (Cs, the
// kernel's tile buffer, free again when this is called), RC rows at a time, so global stores
// (and residual loads) are 16-byte and row-contiguous.  With split-K the raw sums go to the
// partial buffer instead.  Then either a separate reduction pass applies the epilogue, or
// (p.fixup) the split that completes a tile last does: every split stores its partials with
// device-coherent stores, waits for them, and counts itself in the tile's arrival counter;
// the one that sees splits - 1 earlier arrivals sums the partials in split order (the
// reduction pass's order), applies the epilogue and resets the counter to zero.
// nsplit: how many K segments share this tile (split is this one's index among them), ctr:
// the tile's arrival counter, nbatch: batches in the partial buffer's layout.
template <int BM, int BN, int WM, int WN, int RC, int CS, int CM>
__device__ __attribute__((always_inline)) inline void gemm_epilogue(
    const GemmParams& p, const floatx16 (&acc)[BM / WM / 32][BN / WN / 32], float* Cs, int m0,
    int n0, int split, int nsplit, int bz, int bo, int bi, int nbatch, int64_t ctr) {
    constexpr int FM = BM / WM / 32;
    constexpr int FN = BN / WN / 32;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lh = lane >> 5;
    const int bcol = wn * (BN / WN) + (lane & 31);
    const int hw = p.coh * p.cow;
    float* __restrict__ C = p.c + bo * p.sc_outer + bi * p.sc_inner;
    const float* __restrict__ R =
        p.residual ? p.residual + bo * p.sc_outer + bi * p.sc_inner : nullptr;
    float* __restrict__ P =
        nsplit > 1 ? p.partial + ((int64_t)split * nbatch + bz) * p.M * p.N : nullptr;
    const bool vec = P ? (p.N & 3) == 0
                       : (CM == shp::C_STRIDED && p.scn == 1 && (p.scm & 3) == 0 &&
                          (p.N & 3) == 0 && (((uintptr_t)C) & 15) == 0 &&
                          (!p.bias || (((uintptr_t)p.bias) & 15) == 0) &&
                          (!R || (((uintptr_t)R) & 15) == 0));
    // fixup partials as 16-byte coherent buffer accesses while every split's slice fits the
    // 32-bit offsets (all of them: < 2 GiB together), else as 8-byte coherent atomics
    const bool coh16 = P && p.fixup && (int64_t)nsplit * nbatch * p.M * p.N < (1ll << 29);
    const __amdgpu_buffer_rsrc_t prs = buffer_rsrc(P ? P : p.c, (int64_t)p.M * p.N);
    constexpr int TPR = BN / 4, RPP = 256 / TPR;
    const int cl4 = (tid % TPR) * 4;
    const int col4 = n0 + cl4;
    float4 bv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (vec && !P && p.bias && col4 < p.N) bv = *reinterpret_cast<const float4*>(p.bias + col4);
#pragma unroll
    for (int c0 = 0; c0 < BM; c0 += RC) {
        if (c0 > 0) __syncthreads();  // the previous chunk has been consumed
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
            const int rb = wm * (BM / WM) + fm * 32;
            if (rb < c0 || rb >= c0 + RC) continue;
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    Cs[(rb - c0 + 8 * (r >> 2) + 4 * lh + (r & 3)) * CS + bcol + fn * 32] =
                        acc[fm][fn][r];
        }
        __syncthreads();
        if (vec) {
#pragma unroll 4
            for (int i = 0; i < RC / RPP; ++i) {
                const int rl = tid / TPR + RPP * i;
                const int row = m0 + c0 + rl;
                if (row >= p.M || col4 >= p.N) continue;
                float4 v = *reinterpret_cast<const float4*>(&Cs[rl * CS + cl4]);
                if (P) {
                    if (coh16) st_coh16(prs, (unsigned)(((int64_t)row * p.N + col4) * 4), v);
                    else if (p.fixup) st_coh4(P + (int64_t)row * p.N + col4, v);
                    else *reinterpret_cast<float4*>(P + (int64_t)row * p.N + col4) = v;
                    continue;
                }
                const int64_t ci = (int64_t)row * p.scm + col4;
                float4 rv = make_float4(0.f, 0.f, 0.f, 0.f);
                if (R) rv = *reinterpret_cast<const float4*>(R + ci);
                v.x = shpd::apply_act(v.x + bv.x + rv.x, p.act, p.alpha);
                v.y = shpd::apply_act(v.y + bv.y + rv.y, p.act, p.alpha);
                v.z = shpd::apply_act(v.z + bv.z + rv.z, p.act, p.alpha);
                v.w = shpd::apply_act(v.w + bv.w + rv.w, p.act, p.alpha);
                *reinterpret_cast<float4*>(C + ci) = v;
            }
        } else {
            // scalar path: consecutive threads walk the contiguous direction of C
            for (int e = tid; e < RC * BN; e += 256) {
                int rl, cl;
                if constexpr (CM == shp::C_NCHW) {
                    rl = e % RC;
                    cl = e / RC;
                } else {
                    rl = e / BN;
                    cl = e % BN;
                }
                const int row = m0 + c0 + rl, col = n0 + cl;
                if (row >= p.M || col >= p.N) continue;
                float v = Cs[rl * CS + cl];
                if (P) {
                    P[(int64_t)row * p.N + col] = v;
                    continue;
                }
                int64_t ci;
                if constexpr (CM == shp::C_NCHW) {
                    const int img = row / hw, pix = row % hw;
                    ci = ((int64_t)img * p.N + col) * hw + pix;
                } else {
                    ci = (int64_t)row * p.scm + (int64_t)col * p.scn;
                }
                if (p.bias) v += p.bias[col];
                if (R) v += R[ci];
                C[ci] = shpd::apply_act(v, p.act, p.alpha);
            }
        }
    }
    if (P && p.fixup) {  // the host sets fixup only where the 16-byte path applies to C
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partials are stored
        __syncthreads();
        int* last = reinterpret_cast<int*>(Cs);
        int* cnt = p.counters + ctr;
        if (tid == 0)
            *last = __hip_atomic_fetch_add((SHP_GLOBAL int*)cnt, 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT) == nsplit - 1;
        __syncthreads();
        if (!*last) return;
        const float* P0 = p.partial + (int64_t)bz * p.M * p.N;
        const int64_t sstride = (int64_t)nbatch * p.M * p.N;
        const __amdgpu_buffer_rsrc_t p0rs = buffer_rsrc(P0, (int64_t)nsplit * sstride);
        if (p.bias && col4 < p.N) bv = *reinterpret_cast<const float4*>(p.bias + col4);
        for (int i = 0; i < BM / RPP; ++i) {
            const int row = m0 + tid / TPR + RPP * i;
            if (row >= p.M || col4 >= p.N) continue;
            const float* pp = P0 + (int64_t)row * p.N + col4;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int s = 0; s < nsplit; ++s) {
                const float4 q = coh16 ? ld_coh16(p0rs, (unsigned)(((int64_t)row * p.N + col4) * 4),
                                                  (unsigned)(s * sstride * 4))
                                       : ld_coh4(pp + s * sstride);
                v.x += q.x;
                v.y += q.y;
                v.z += q.z;
                v.w += q.w;
            }
            const int64_t ci = (int64_t)row * p.scm + col4;
            float4 rv = make_float4(0.f, 0.f, 0.f, 0.f);
            if (R) rv = *reinterpret_cast<const float4*>(R + ci);
            v.x = shpd::apply_act(v.x + bv.x + rv.x, p.act, p.alpha);
            v.y = shpd::apply_act(v.y + bv.y + rv.y, p.act, p.alpha);
            v.z = shpd::apply_act(v.z + bv.z + rv.z, p.act, p.alpha);
            v.w = shpd::apply_act(v.w + bv.w + rv.w, p.act, p.alpha);
            *reinterpret_cast<float4*>(C + ci) = v;
        }
        if (tid == 0)
            __hip_atomic_store((SHP_GLOBAL int*)cnt, 0, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

// PG: global prefetch depth.  1: tile k+1 is loaded into registers while tile k is
// multiplied; 2: tile k+2 (two register sets), so each load has two tiles' worth of MFMA
// time to arrive.
template <int BM, int BN, int WM, int WN, int BK, int AM, int BMD, int CM, int PG = 1>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(GemmParams p) {
    constexpr int FM = BM / WM / 32;
    constexpr int FN = BN / WN / 32;
    static_assert(WM * WN == 4, "four wavefronts per workgroup");
    static_assert(FM >= 1 && FN >= 1, "tile too small for 32x32 blocks");
    constexpr bool A_VEC = (AM == shp::A_KVEC || AM == shp::A_CONV_NHWC4);
    constexpr bool A_CONV = (AM == shp::A_CONV_NHWC4 || AM == shp::A_CONV_NHWC ||
                             AM == shp::A_CONV_NCHW);
    constexpr bool A_TAB = (AM == shp::A_CONV_NHWC || AM == shp::A_CONV_NCHW);
    static_assert(BK == 16 || BK == 32, "K tile of 16 or 32");
    constexpr int KQ = BK / 4;                                        // float4 per A row
    constexpr int NA = A_VEC ? BM * BK / 1024 : BM * BK / 256;        // A loads per thread
    constexpr int NB = (BMD == shp::B_STRIDED) ? BN * BK / 256 : BN * BK / 1024;  // B loads
    constexpr int AP = 4, BP = 4, CP = 4;
    constexpr int AS = BK + AP;        // A tile row stride (floats)
    constexpr int BS = BN + BP;        // B tile row stride
    constexpr int CS = BN + CP;        // C tile row stride (epilogue)
    constexpr int A_FLOATS = 2 * BM * AS;
    constexpr int B_FLOATS = 2 * BK * BS;
    constexpr int SMEM = A_FLOATS + B_FLOATS;
    // epilogue: the output tile goes through LDS in chunks of RC rows (multiple of 32)
    constexpr int RC = BM * CS <= SMEM ? BM : (BM / 2) * CS <= SMEM ? BM / 2 : 32;
    static_assert(RC >= 32 && BM % RC == 0, "epilogue chunk must hold whole 32-row blocks");

    // One LDS allocation: double-buffered A [2][BM][AS] and B [2][BK][BS] tiles during the
    // K loop, reused as the [BM][CS] output tile by the epilogue.
    __shared__ __attribute__((aligned(16))) float smem[SMEM];
    __shared__ int2 ktab[A_TAB ? KTAB : 1];
    float* const As = smem;
    float* const Bs = smem + A_FLOATS;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int li = lane & 31, lh = lane >> 5;

    // ---- tile coordinates: give each XCD (block id mod 8) a contiguous run of tiles so
    // the workgroups sharing A rows / B columns meet in the same L2.
    const int tiles_n = (p.N + BN - 1) / BN;
    const int tiles_m = (p.M + BM - 1) / BM;
    const WgCoords wc = wg_coords(tiles_m, tiles_n, p.splits, p.group_m);
    const int m0 = wc.tm * BM, n0 = wc.tn * BN;

    const int split = wc.split;
    const int bz = blockIdx.z;
    const int bo = bz / p.batch_inner, bi = bz % p.batch_inner;
    const float* __restrict__ A = p.a + bo * p.sa_outer + bi * p.sa_inner;
    const float* __restrict__ B = p.b + bo * p.sb_outer + bi * p.sb_inner;
    const int kbeg = split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int ntk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    // NHWC with IC a multiple of the K tile: a whole K tile sits inside one (ky, kx) tap,
    // so its decomposition is uniform across the workgroup (scalar ALU, no per-lane divide).
    const bool tap_uniform = (AM == shp::A_CONV_NHWC4) && (p.cic % BK == 0) && (kbeg % BK == 0);

    // ---- per-thread load coordinates
    // A: vector modes -> row = tid/KQ + (256/KQ)*j, kq = (tid%KQ)*4; scalar modes ->
    //    m = tid%BM, k = tid/BM + (256/BM)*j.
    ConvRow crow[A_CONV ? (A_VEC ? NA : 1) : 1];
    if constexpr (A_CONV) {
        if constexpr (A_VEC) {
#pragma unroll
            for (int j = 0; j < NA; ++j) crow[j] = conv_row(p, m0 + tid / KQ + (256 / KQ) * j, AM);
        } else {
            crow[0] = conv_row(p, m0 + tid % BM, AM);
        }
    }
    if constexpr (A_TAB) {
        // offsets of every K index this workgroup visits, when they fit the table
        int span = kend - kbeg;
        if (span <= KTAB) {
            for (int k = tid; k < span; k += 256) {
                int off, ky, kx;
                conv_k(p, kbeg + k, AM, off, ky, kx);
                ktab[k] = make_int2(off, (ky << 16) | kx);
            }
        }
        __syncthreads();
    }

    // staging registers of one K tile: A (vector or scalar form) and B
    struct Stage {
        float4 ra[A_VEC ? NA : 1];
        float rs[A_VEC ? 1 : NA];
        float4 rb[BMD == shp::B_STRIDED ? 1 : NB];
        float rbs[BMD == shp::B_STRIDED ? NB : 1];
    };
    Stage st0, st1;

    auto load_a = [&](int kt, Stage& sg) __attribute__((always_inline)) {
        float4 (&ra)[A_VEC ? NA : 1] = sg.ra;
        float (&rs)[A_VEC ? 1 : NA] = sg.rs;
        const int kt0 = kbeg + kt * BK;
        if constexpr (A_VEC) {
            const int kq = (tid % KQ) * 4;
            const int k = kt0 + kq;
            if constexpr (AM == shp::A_KVEC) {
#pragma unroll
                for (int j = 0; j < NA; ++j) {
                    int m = m0 + tid / KQ + (256 / KQ) * j;
                    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (m < p.M && k < kend)
                        v = *reinterpret_cast<const float4*>(A + (int64_t)m * p.sam + k);
                    ra[j] = v;
                }
            } else {  // A_CONV_NHWC4
                int off = 0, ky = 0, kx = 0;
                if (tap_uniform) {
                    int ic0 = kt0 % p.cic;
                    int t = kt0 / p.cic;
                    kx = t % p.ckw;
                    ky = t / p.ckw;
                    off = (ky * p.ciw + kx) * p.cic + ic0 + kq;
                } else if (k < kend) {
                    conv_k(p, k, AM, off, ky, kx);
                }
#pragma unroll
                for (int j = 0; j < NA; ++j) {
                    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                    int iy = crow[j].iy0 + ky, ix = crow[j].ix0 + kx;
                    if (crow[j].valid && k < kend && (unsigned)iy < (unsigned)p.cih &&
                        (unsigned)ix < (unsigned)p.ciw)
                        v = *reinterpret_cast<const float4*>(A + crow[j].base + off);
                    ra[j] = v;
                }
            }
        } else {
            const int ml = tid % BM;
            const int m = m0 + ml;
#pragma unroll
            for (int j = 0; j < NA; ++j) {
                int kl = tid / BM + (256 / BM) * j;
                int k = kt0 + kl;
                float v = 0.f;
                if constexpr (AM == shp::A_STRIDED) {
                    if (m < p.M && k < kend) v = A[(int64_t)m * p.sam + (int64_t)k * p.sak];
                } else {
                    if (crow[0].valid && k < kend) {
                        int off, ky, kx;
                        if (kend - kbeg <= KTAB) {
                            int2 e = ktab[k - kbeg];
                            off = e.x;
                            ky = e.y >> 16;
                            kx = e.y & 0xffff;
                        } else {
                            conv_k(p, k, AM, off, ky, kx);
                        }
                        int iy = crow[0].iy0 + ky, ix = crow[0].ix0 + kx;
                        if ((unsigned)iy < (unsigned)p.cih && (unsigned)ix < (unsigned)p.ciw)
                            v = A[crow[0].base + off];
                    }
                }
                rs[j] = v;
            }
        }
    };

    auto store_a = [&](int buf, const Stage& sg) __attribute__((always_inline)) {
        const float4 (&ra)[A_VEC ? NA : 1] = sg.ra;
        const float (&rs)[A_VEC ? 1 : NA] = sg.rs;
        float* a = As + buf * BM * AS;
        if constexpr (A_VEC) {
            const int kq = (tid % KQ) * 4;
#pragma unroll
            for (int j = 0; j < NA; ++j)
                *reinterpret_cast<float4*>(&a[(tid / KQ + (256 / KQ) * j) * AS + kq]) = ra[j];
        } else {
            const int ml = tid % BM;
#pragma unroll
            for (int j = 0; j < NA; ++j) a[ml * AS + tid / BM + (256 / BM) * j] = rs[j];
        }
    };

    auto load_b = [&](int kt, Stage& sg) __attribute__((always_inline)) {
        float4 (&rb)[BMD == shp::B_STRIDED ? 1 : NB] = sg.rb;
        float (&rbs)[BMD == shp::B_STRIDED ? NB : 1] = sg.rbs;
        const int kt0 = kbeg + kt * BK;
        if constexpr (BMD == shp::B_NVEC) {
            constexpr int TPR = BN / 4;  // threads per k row
            const int n = n0 + (tid % TPR) * 4;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                int k = kt0 + tid / TPR + (256 / TPR) * j;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (k < kend && n < p.N)
                    v = *reinterpret_cast<const float4*>(B + (int64_t)k * p.sbk + n);
                rb[j] = v;
            }
        } else if constexpr (BMD == shp::B_KVEC) {
            const int n = n0 + tid % BN;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                int k = kt0 + (tid / BN) * 4 + (256 / BN) * 4 * j;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (k < kend && n < p.N)
                    v = *reinterpret_cast<const float4*>(B + (int64_t)n * p.sbn + k);
                rb[j] = v;
            }
        } else {
            const int n = n0 + tid % BN;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                int k = kt0 + tid / BN + (256 / BN) * j;
                float v = 0.f;
                if (k < kend && n < p.N) v = B[(int64_t)k * p.sbk + (int64_t)n * p.sbn];
                rbs[j] = v;
            }
        }
    };

    auto store_b = [&](int buf, const Stage& sg) __attribute__((always_inline)) {
        const float4 (&rb)[BMD == shp::B_STRIDED ? 1 : NB] = sg.rb;
        const float (&rbs)[BMD == shp::B_STRIDED ? NB : 1] = sg.rbs;
        float* b = Bs + buf * BK * BS;
        if constexpr (BMD == shp::B_NVEC) {
            constexpr int TPR = BN / 4;
            const int nl = (tid % TPR) * 4;
#pragma unroll
            for (int j = 0; j < NB; ++j)
                *reinterpret_cast<float4*>(&b[(tid / TPR + (256 / TPR) * j) * BS + nl]) = rb[j];
        } else if constexpr (BMD == shp::B_KVEC) {
            const int nl = tid % BN;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                int kl = (tid / BN) * 4 + (256 / BN) * 4 * j;
                b[(kl + 0) * BS + nl] = rb[j].x;
                b[(kl + 1) * BS + nl] = rb[j].y;
                b[(kl + 2) * BS + nl] = rb[j].z;
                b[(kl + 3) * BS + nl] = rb[j].w;
            }
        } else {
            const int nl = tid % BN;
#pragma unroll
            for (int j = 0; j < NB; ++j) b[(tid / BN + (256 / BN) * j) * BS + nl] = rbs[j];
        }
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int arow = wm * (BM / WM) + li;
    const int bcol = wn * (BN / WN) + li;

    // The MFMAs of the K tile in LDS buffer `buf`.  Lanes 0-31 feed k = s, lanes 32-63 feed
    // k = BK/2 + s of the tile: any assignment works as long as A and B agree, and this one
    // lets each lane read BK/2 consecutive k of its A row with 128-bit LDS loads.
    auto compute = [&](int buf) __attribute__((always_inline)) {
        const float* a = As + buf * BM * AS;
        const float* b = Bs + buf * BK * BS;
#pragma unroll
        for (int s4 = 0; s4 < BK / 8; ++s4) {
            float4 af[FM];
            float bf[FN][4];
#pragma unroll
            for (int fm = 0; fm < FM; ++fm)
                af[fm] = *reinterpret_cast<const float4*>(
                    &a[(arow + fm * 32) * AS + lh * (BK / 2) + s4 * 4]);
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    bf[fn][q] = b[(lh * (BK / 2) + s4 * 4 + q) * BS + bcol + fn * 32];
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn) {
                        float av = q == 0 ? af[fm].x : q == 1 ? af[fm].y
                                                     : q == 2 ? af[fm].z : af[fm].w;
                        acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            av, bf[fn][q], acc[fm][fn], 0, 0, 0);
                    }
        }
    };

    if (ntk > 0) {
        if constexpr (PG == 2) {
            // tile t lives in register set t & 1 and LDS buffer t & 1.  Set t & 1 is free
            // again once tile t is in LDS; buffer (t+1) & 1 once the barrier after tile t-1.
            load_a(0, st0);
            load_b(0, st0);
            if (ntk > 1) {
                load_a(1, st1);
                load_b(1, st1);
            }
            store_a(0, st0);
            store_b(0, st0);
            __syncthreads();
            for (int kt = 0; kt < ntk; kt += 2) {
                if (kt + 2 < ntk) {
                    load_a(kt + 2, st0);
                    load_b(kt + 2, st0);
                }
                compute(0);
                if (kt + 1 < ntk) {
                    store_a(1, st1);
                    store_b(1, st1);
                }
                __syncthreads();
                if (kt + 1 >= ntk) break;
                if (kt + 3 < ntk) {
                    load_a(kt + 3, st1);
                    load_b(kt + 3, st1);
                }
                compute(1);
                if (kt + 2 < ntk) {
                    store_a(0, st0);
                    store_b(0, st0);
                }
                __syncthreads();
            }
        } else {
            load_a(0, st0);
            load_b(0, st0);
            store_a(0, st0);
            store_b(0, st0);
            __syncthreads();
            for (int kt = 0; kt < ntk; ++kt) {
                const int buf = kt & 1;
                if (kt + 1 < ntk) {
                    load_a(kt + 1, st0);
                    load_b(kt + 1, st0);
                }
                compute(buf);
                if (kt + 1 < ntk) {
                    store_a(buf ^ 1, st0);
                    store_b(buf ^ 1, st0);
                }
                __syncthreads();
            }
        }
    }

    gemm_epilogue<BM, BN, WM, WN, RC, CS, CM>(p, acc, smem, m0, n0, split, p.splits, bz, bo, bi,
                                              gridDim.z, (int64_t)bz * gridDim.x + wc.tile);
}

// ---- buffer-loaded variant (gemm_bl_kernel) for the row-contiguous operand forms of the
// model paths: A = rows (A_KVEC) or an NHWC im2col whose K tile sits inside one (ky, kx) tap
// (A_CONV_NHWC4 with IC % BK == 0); B = [K][N] (B_NVEC) or [N][K] (B_KVEC); K a multiple of
// BK in every split.
//
// What makes it faster than gemm_mfma_kernel (measured on MI355X): every operand load is one
// buffer_load_dwordx4 whose per-lane byte offset is computed once, outside the K loop, and
// whose K advance is a scalar offset, so the loop issues no address arithmetic and no
// bounds checks.  Rows past M and columns past N are clamped to the last one (their products
// are never stored); a padding tap of a convolution gets an offset past the operand's range,
// for which the buffer load returns zeros.  Each fragment step (four MFMA k-pairs) also
// stores one register-staged chunk of the next K tile into the other LDS buffer and issues
// one load of the tile after it (two tiles in flight), and the next step's fragments are read
// before its MFMAs, so LDS and global latency overlap the MFMA stream instead of sitting
// between dependent MFMAs.
// A byte offset beyond every operand range (the host keeps ranges <= 2 GiB): loads return 0.
constexpr unsigned kOobOffset = 0x80000000u;

__device__ __forceinline__ f4v buffer_load4(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff) {
    return __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Elements an operand spans (per batch), as the buffer range of its loads.
__device__ __host__ inline int64_t bl_a_extent(const GemmParams& p, int amode) {
    if (amode == shp::A_CONV_NHWC4) return (int64_t)p.cn * p.cih * p.ciw * p.cic;
    return (int64_t)(p.M - 1) * p.sam + p.K;
}
__device__ __host__ inline int64_t bl_b_extent(const GemmParams& p, int bmode) {
    if (bmode == shp::B_KVEC) return (int64_t)(p.N - 1) * p.sbn + p.K;
    return (int64_t)(p.K - 1) * p.sbk + p.N;
}

template <int BM, int BN, int BK, int AM, int BMD>
__global__ __launch_bounds__(256) void gemm_bl_kernel(GemmParams p) {
    static_assert(AM == shp::A_KVEC || AM == shp::A_CONV_NHWC4, "row-contiguous A");
    static_assert(BMD == shp::B_NVEC || BMD == shp::B_KVEC, "row-contiguous B");
    constexpr int FM = BM / 64, FN = BN / 64;           // 2x2 waves of FM x FN 32x32 blocks
    constexpr int KQ = BK / 4;                           // float4 chunks per K row of a tile
    constexpr int NA = BM * BK / 1024, NB = BK * BN / 1024, NE = NA + NB;
    constexpr int NS = BK / 8;                           // fragment steps per K tile
    constexpr bool BT = BMD == shp::B_KVEC;              // B tile stored [n][k] (else [k][n])
    constexpr int AS = BK + 4;                           // row stride of K-contiguous tiles
    constexpr int BS = BT ? AS : BN + 4;                 // row stride of the B tile
    constexpr int ABUF = BM * AS;
    constexpr int BBUF = BT ? BN * AS : BK * BS;
    constexpr int SMEM = 2 * (ABUF + BBUF);
    constexpr int CS = BN + 4;
    constexpr int RC = BM * CS <= SMEM ? BM : (BM / 2) * CS <= SMEM ? BM / 2 : 32;
    constexpr int TPR = BN / 4;                          // threads per [k][n] B row
    static_assert(FM >= 1 && FN >= 1 && NA >= 1 && NB >= 1 && NS >= 2, "tile shape");
    static_assert(RC >= 32 && BM % RC == 0, "epilogue chunk must hold whole 32-row blocks");
    __shared__ __attribute__((aligned(16))) float smem[SMEM];
    float* const As = smem;
    float* const Bs = smem + 2 * ABUF;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int li = lane & 31, lh = lane >> 5;

    const int tiles_n = (p.N + BN - 1) / BN;
    const int tiles_m = (p.M + BM - 1) / BM;
    const WgCoords wc = wg_coords(tiles_m, tiles_n, p.splits, p.group_m);
    const int m0 = wc.tm * BM, n0 = wc.tn * BN;

    const int split = wc.split;
    const int bz = blockIdx.z;
    const int bo = bz / p.batch_inner, bi = bz % p.batch_inner;
    const float* A = p.a + bo * p.sa_outer + bi * p.sa_inner;
    const float* B = p.b + bo * p.sb_outer + bi * p.sb_inner;
    const int kbeg = split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int ntk = kend > kbeg ? (kend - kbeg) / BK : 0;
    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(A, bl_a_extent(p, AM));
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(B, bl_b_extent(p, BMD));

    // ---- loop-invariant per-lane load offsets
    const int ka = (tid % KQ) * 4;  // k of this lane's A (and K-contiguous B) chunk
    // A_KVEC: byte offset of the chunk at kbeg.  A_CONV_NHWC4: element offset of the row's
    // tap (0, 0), channel ka (negative where the window starts in the padding), and the
    // window origin for the per-tap range check.
    int aoff[NA], iy0[AM == shp::A_CONV_NHWC4 ? NA : 1], ix0[AM == shp::A_CONV_NHWC4 ? NA : 1];
#pragma unroll
    for (int e = 0; e < NA; ++e) {
        const int m = m0 + tid / KQ + (256 / KQ) * e;
        if constexpr (AM == shp::A_KVEC) {
            aoff[e] = (int)(((int64_t)min(m, p.M - 1) * p.sam + kbeg + ka) * 4);
        } else {
            const ConvRow r = conv_row(p, m, AM);
            aoff[e] = (int)r.base + ka;
            iy0[e] = r.valid ? r.iy0 : -(1 << 28);  // rows past M fail every range check
            ix0[e] = r.ix0;
        }
    }
    // 1x1 convolutions without padding read every row in range: the tap is fixed and the
    // channel advance is a scalar offset, as for A_KVEC.
    const bool tap1 = AM == shp::A_CONV_NHWC4 && p.ckh == 1 && p.ckw == 1 && p.cpt == 0 &&
                      p.cpl == 0;
    unsigned boff[NB];
#pragma unroll
    for (int e = 0; e < NB; ++e) {
        if constexpr (BT) {
            const int n = min(n0 + tid / KQ + (256 / KQ) * e, p.N - 1);
            boff[e] = (unsigned)(((int64_t)n * p.sbn + kbeg + ka) * 4);
        } else {
            const int kr = tid / TPR + (256 / TPR) * e;
            const int n = min(n0 + (tid % TPR) * 4, p.N - 4);
            boff[e] = (unsigned)(((int64_t)(kbeg + kr) * p.sbk + n) * 4);
        }
    }
    const unsigned b_step = BT ? BK * 4u : (unsigned)(BK * p.sbk * 4);

    struct Stage { f4v e[NE]; };
    auto load_e = [&](int kt, Stage& s, int e) __attribute__((always_inline)) {
        if (e < NA) {
            if constexpr (AM == shp::A_KVEC) {
                s.e[e] = buffer_load4(ra, (unsigned)aoff[e], (unsigned)(kt * BK * 4));
            } else if (tap1) {
                const unsigned v = iy0[e] >= 0 ? (unsigned)aoff[e] * 4u : kOobOffset;
                s.e[e] = buffer_load4(ra, v, (unsigned)((kbeg + kt * BK) * 4));
            } else {
                // K tile kt lies inside tap (ky, kx), channels ic0 .. ic0 + BK - 1
                const int k0 = kbeg + kt * BK;
                const int ic0 = k0 % p.cic, t = k0 / p.cic;
                const int kx = t % p.ckw, ky = t / p.ckw;
                const bool ok = (unsigned)(iy0[e] + ky) < (unsigned)p.cih &&
                                (unsigned)(ix0[e] + kx) < (unsigned)p.ciw;
                const int off = aoff[e] + (ky * p.ciw + kx) * p.cic + ic0;
                s.e[e] = buffer_load4(ra, ok ? (unsigned)off * 4u : kOobOffset, 0u);
            }
        } else {
            s.e[e] = buffer_load4(rb, boff[e - NA], (unsigned)kt * b_step);
        }
    };
    auto store_e = [&](int buf, const Stage& s, int e) __attribute__((always_inline)) {
        if (e < NA) {
            *reinterpret_cast<f4v*>(&As[buf * ABUF + (tid / KQ + (256 / KQ) * e) * AS + ka]) = s.e[e];
        } else if constexpr (BT) {
            *reinterpret_cast<f4v*>(&Bs[buf * BBUF + (tid / KQ + (256 / KQ) * (e - NA)) * AS + ka]) =
                s.e[e];
        } else {
            *reinterpret_cast<f4v*>(
                &Bs[buf * BBUF + (tid / TPR + (256 / TPR) * (e - NA)) * BS + (tid % TPR) * 4]) = s.e[e];
        }
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Fragments of one step: lanes 0-31 feed k = s of the tile, lanes 32-63 k = BK/2 + s (A and
    // B agree, so any assignment of the tile's k to MFMA k-pairs works), so each lane reads four
    // consecutive k of its A row (and, from a [n][k] tile, of its B column) at once.
    const int arow = wm * (BM / 2) + li;
    const int bcol = wn * (BN / 2) + li;
    struct Frag { f4v a[FM]; f4v b[FN]; };
    auto read = [&](int buf, int s4, Frag& f) __attribute__((always_inline)) {
        const int kk = lh * (BK / 2) + s4 * 4;
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
            f.a[fm] = *reinterpret_cast<const f4v*>(&As[buf * ABUF + (arow + fm * 32) * AS + kk]);
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
            if constexpr (BT) {
                f.b[fn] = *reinterpret_cast<const f4v*>(&Bs[buf * BBUF + (bcol + fn * 32) * AS + kk]);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) f.b[fn][q] = Bs[buf * BBUF + (kk + q) * BS + bcol + fn * 32];
            }
        }
    };
    auto mma = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                for (int fn = 0; fn < FN; ++fn)
                    acc[fm][fn] =
                        __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[fm][q], f.b[fn][q], acc[fm][fn], 0, 0, 0);
    };
    // One K tile from LDS buffer `buf`; `wr` (the next tile) goes into buffer buf^1 chunk by
    // chunk when `do_store`, and tile `ld_kt` is loaded into `ld` chunk by chunk.  The
    // scheduling fences keep each step's memory instructions ahead of its MFMAs.
    auto tile = [&](int buf, const Stage& wr, bool do_store, Stage& ld, int ld_kt)
                    __attribute__((always_inline)) {
        Frag f0, f1;
        read(buf, 0, f0);
#pragma unroll
        for (int s4 = 0; s4 < NS; ++s4) {
            const int e0 = s4 * NE / NS, e1 = (s4 + 1) * NE / NS;
            if (s4 + 1 < NS) {
                if (s4 & 1) read(buf, s4 + 1, f0);
                else read(buf, s4 + 1, f1);
            }
            if (do_store)
#pragma unroll
                for (int e = e0; e < e1; ++e) store_e(buf ^ 1, wr, e);
#pragma unroll
            for (int e = e0; e < e1; ++e) load_e(ld_kt, ld, e);
            if (s4 & 1) mma(f1);
            else mma(f0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    if (ntk > 0) {
        // Tile t lives in LDS buffer t & 1; register set s0 / s1 holds tile t + 1 and t + 2
        // alternately.  The last two loads re-read the final tile (unused) so every set is
        // redefined each iteration.
        Stage s0, s1;
#pragma unroll
        for (int e = 0; e < NE; ++e) load_e(0, s0, e);
#pragma unroll
        for (int e = 0; e < NE; ++e) load_e(min(1, ntk - 1), s1, e);
#pragma unroll
        for (int e = 0; e < NE; ++e) store_e(0, s0, e);
        __syncthreads();
        int kt = 0;
        for (; kt + 1 < ntk; kt += 2) {
            tile(0, s1, true, s0, min(kt + 2, ntk - 1));
            __syncthreads();
            tile(1, s0, kt + 2 < ntk, s1, min(kt + 3, ntk - 1));
            __syncthreads();
        }
        if (kt < ntk) {
            tile(0, s1, false, s0, kt);
            __syncthreads();
        }
    }

    gemm_epilogue<BM, BN, 2, 2, RC, CS, shp::C_STRIDED>(p, acc, smem, m0, n0, split, p.splits, bz,
                                                        bo, bi, gridDim.z,
                                                        (int64_t)bz * gridDim.x + wc.tile);
}

// ---- persistent small-K variant (gemm_smallk_kernel) for products with K = 64 (KT) whose
// A is plain rows (row-major, or the NHWC input of a 1x1 stride-1 unpadded convolution) and
// whose B is [K][N]: the 1x1 convolutions of bottleneck networks.  A tiled kernel spends
// most of such a tile in its operand prologue and its epilogue (4-8 K steps), so here:
// * one workgroup of 512 threads per CU owns the 32-row tiles [T*r/R, T*(r+1)/R) (T tiles in
//   all) of one TN-column slab of C; the slab of B is transposed into LDS once ([n][k], rows
//   padded by 4 floats);
// * the eight wavefronts form teams of WC; team i takes tiles i, i + 8/WC, ... of the range,
//   each wave 32 rows x 32*FN columns;
// * a wave loads its tile's A rows straight into registers in the MFMA operand layout (lane
//   l: row l % 32, k = 8s + 4*(l / 32) .. +3 of step s, the same k remap as gemm_bl_kernel);
//   the operand of step s is reloaded with the next tile's right after the step's MFMAs;
// * the epilogue stores from the accumulators (each store instruction writes two 128-byte
//   row segments), spread over the next tile's fragment steps (two accumulator sets), so the
//   stores drain under the MFMA stream instead of stalling it; the residual of a tile is
//   loaded into the slots of the elements stored before it.
// M is a multiple of 32 (the host checks it), so no tile needs row checks.  ACT: 0 no
// activation, 1 ReLU (a template parameter, so that the epilogue is straight-line code).
// Workgroup b sits on XCD b % 8; the slabs of one row range go to workgroups of one XCD, so
// A is fetched from HBM once and re-read from that XCD's L2.
template <int KT, int FN, int WC, int ACT, bool RES>
__global__ __launch_bounds__(512, 1) void gemm_smallk_kernel(GemmParams p, int nslab, int nrange) {
    constexpr int KS = KT / 8;               // fragment steps (8 k each) per tile
    constexpr int TN = 32 * FN * WC;          // slab width
    constexpr int BST = KT + 4;               // LDS row stride of the transposed slab
    constexpr int NTEAM = 8 / WC;
    constexpr int NST = 16 * FN;              // output elements per lane and tile
    constexpr int SPS = (NST + KS - 1) / KS;  // of them stored per fragment step
    __shared__ __attribute__((aligned(16))) float Bs[TN * BST];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, lh = lane >> 5;
    const int b = blockIdx.x;
    const int slab = (b >> 3) % nslab;
    const int range = (b & 7) + 8 * (b / (8 * nslab));
    if (range >= nrange) return;
    const int T = p.M / 32;
    const int t_beg = (int)((int64_t)T * range / nrange);
    const int t_end = (int)((int64_t)T * (range + 1) / nrange);
    const int c_slab = slab * TN;

    // B slab -> LDS, transposed to [n][k]; consecutive lanes take consecutive k, so the LDS
    // stores are free of bank conflicts (the reads of the small slab hit L2)
    for (int i = tid; i < KT * TN / 4; i += 512) {
        const int k = i % KT, n4 = (i / KT) * 4;
        const float4 v = *reinterpret_cast<const float4*>(p.b + (int64_t)k * p.sbk + c_slab + n4);
        Bs[(n4 + 0) * BST + k] = v.x;
        Bs[(n4 + 1) * BST + k] = v.y;
        Bs[(n4 + 2) * BST + k] = v.z;
        Bs[(n4 + 3) * BST + k] = v.w;
    }
    __syncthreads();

    const int team = wave / WC, wc = wave % WC;
    const int first = t_beg + team;
    const int n = first < t_end ? (t_end - 1 - first) / NTEAM + 1 : 0;  // tiles of this team
    if (n == 0) return;
    const int col0 = c_slab + wc * 32 * FN + li;  // this lane's column (fn 0)
    float bias[FN];
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) bias[fn] = p.bias ? p.bias[col0 + fn * 32] : 0.0f;
    const char* __restrict__ Ab = reinterpret_cast<const char*>(p.a);
    const char* __restrict__ Rb = reinterpret_cast<const char*>(p.residual);
    char* __restrict__ Cb = reinterpret_cast<char*>(p.c);
    const unsigned sam4 = (unsigned)p.sam * 4u, scm4 = (unsigned)p.scm * 4u;
    const unsigned aoff0 = (unsigned)li * sam4 + 16u * lh;                    // + tile rows
    const unsigned coff0 = (unsigned)(4 * lh) * scm4 + (unsigned)col0 * 4u;  // + tile rows
    const unsigned bsoff = (unsigned)(col0 - c_slab) * BST + 4 * lh;

    auto load_a = [&](f4v& a, int t, int s) __attribute__((always_inline)) {
        a = *reinterpret_cast<const f4v*>(Ab + aoff0 + (unsigned)(t * 32) * sam4 + 32u * s);
    };
    // Output element i of a lane (i = r * FN + fn): row 8*(r/4) + r%4 (+ 4*lh), column fn*32.
    auto eoff = [&](int t, int i) __attribute__((always_inline)) {
        const int r = i / FN, fn = i % FN;
        return coff0 + (unsigned)(t * 32 + 8 * (r >> 2) + (r & 3)) * scm4 + 128u * fn;
    };
    float res[NST];  // the residual of the tile whose results are stored next
    auto load_res = [&](int t, int i0, int i1) __attribute__((always_inline)) {
        if constexpr (RES) {
#pragma unroll
            for (int i = i0; i < i1 && i < NST; ++i)
                res[i] = *reinterpret_cast<const float*>(Rb + eoff(t, i));
        }
    };
    // Stores elements [i0, i1) of tile t from acc; with RES, refills their residual slots with
    // tile tn's, whose results are stored next.
    auto store_some = [&](const floatx16 (&acc)[FN], int t, int tn, int i0, int i1)
                          __attribute__((always_inline)) {
#pragma unroll
        for (int i = i0; i < i1 && i < NST; ++i) {
            float v = acc[i % FN][i / FN] + bias[i % FN];
            if constexpr (RES) v += res[i];
            if constexpr (ACT == 1) v = fmaxf(v, 0.0f);
            *reinterpret_cast<float*>(Cb + eoff(t, i)) = v;
        }
        load_res(tn, i0, i1);
    };
    // The MFMAs of tile t into acc, the A operand of step s replaced by tile ta's right after
    // the step's MFMAs (so it has a tile's MFMA time to arrive); when `store`, tile tp's
    // results (prev) are stored SPS per fragment step in between, so the stores drain under
    // the MFMA stream.
    f4v a[KS];
    auto mma_tile = [&](floatx16 (&acc)[FN], const floatx16 (&prev)[FN], int t, int tp, bool store,
                        int ta) __attribute__((always_inline)) {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fn][r] = 0.0f;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            f4v bf[FN];
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
                bf[fn] = *reinterpret_cast<const f4v*>(&Bs[bsoff + fn * 32 * BST + 8 * s]);
            if (store) store_some(prev, tp, t, s * SPS, (s + 1) * SPS);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int fn = 0; fn < FN; ++fn)
                    acc[fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s][q], bf[fn][q], acc[fn], 0, 0, 0);
            load_a(a[s], ta, s);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Tiles alternate between two accumulator sets (one multiplied while the other is
    // stored); every operand load is unconditional (past the team's last tile it re-reads it).
    const int tlast = first + (n - 1) * NTEAM;
    floatx16 c0[FN], c1[FN];
    load_res(first, 0, NST);
#pragma unroll
    for (int s = 0; s < KS; ++s) load_a(a[s], first, s);
    mma_tile(c0, c1, first, first, false, min(first + NTEAM, tlast));
    int j = 1;
    for (; j + 1 < n; j += 2) {
        const int t = first + j * NTEAM;  // tile j into c1, tile j + 1 into c0
        mma_tile(c1, c0, t, t - NTEAM, true, t + NTEAM);
        mma_tile(c0, c1, t + NTEAM, t, true, min(t + 2 * NTEAM, tlast));
    }
    if (j < n) {
        const int t = first + j * NTEAM;
        mma_tile(c1, c0, t, t - NTEAM, true, t);
        store_some(c1, t, t, 0, NST);
    } else {
        const int t = first + (j - 1) * NTEAM;
        store_some(c0, t, t, 0, NST);
    }
}

// ---- stem variant (conv_stem_kernel): an NHWC convolution with few input channels (the 7x7
// stride-2 3-channel ResNet stem), whose K = KH*KW*CIC is neither a multiple of 4 nor of any
// K tile.  For one output pixel and one kernel row ky, the KW*CIC operands are contiguous in
// the input row, so K is laid out per kernel row, each padded to GW (a multiple of 8, 21 ->
// 24 for the stem): k = ky*GW + e, e = kx*CIC + c.  The weights of the padding slots are zero
// in LDS, and padding taps and slots read zero (an offset past the input's range), so the
// products are exact.
// * One workgroup of 512 threads per CU owns the 32-row tiles [T*r/R, T*(r+1)/R) of a
//   64-column slab; every wavefront works alone on tiles w, w + 8, ... (32 rows x 64 columns).
// * A lane holds row l % 32 of its tile and, per fragment step s, k = 8s + 4*(l / 32) .. +3
//   (the k remap of gemm_bl_kernel), as four dword buffer loads; the validity of each k
//   (kernel row inside the image, column inside the image, slot < KW*CIC) comes from two
//   per-lane bit masks computed once per tile.  The operand of step s is reloaded with the
//   next tile's right after the step's MFMAs, so it has a tile's MFMA time to arrive.
// * The epilogue (bias, optional ReLU) stores tile t's results during tile t+1's steps.
// ACT: 0 none, 1 ReLU.  M is a multiple of 32 (the host checks it).
template <int KH, int KW, int CIC, int ACT>
__global__ __launch_bounds__(512, 1) void conv_stem_kernel(GemmParams p, int nslab, int nrange) {
    constexpr int GW = (KW * CIC + 7) / 8 * 8;  // padded operands per kernel row
    constexpr int GS = GW / 8;                  // fragment steps per kernel row
    constexpr int KS = KH * GS;                 // fragment steps per tile
    constexpr int KT = KH * GW;
    constexpr int BST = KT + 4;
    constexpr int TN = 64, FN = 2;
    constexpr int NST = 16 * FN;
    constexpr int SPS = (NST + KS - 1) / KS;
    static_assert(GW <= 32 && GW - 4 <= 28, "row masks are 32-bit");
    __shared__ __attribute__((aligned(16))) float Bs[TN * BST];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, lh = lane >> 5;
    const int b = blockIdx.x;
    const int slab = (b >> 3) % nslab;
    const int range = (b & 7) + 8 * (b / (8 * nslab));
    if (range >= nrange) return;
    const int T = p.M / 32;
    const int t_beg = (int)((int64_t)T * range / nrange);
    const int t_end = (int)((int64_t)T * (range + 1) / nrange);
    const int c_slab = slab * TN;

    // weight slab -> LDS as [n][ky*GW + e], zero in the padding slots; consecutive lanes take
    // consecutive k, so the LDS stores are free of bank conflicts
    for (int i = tid; i < TN * KT; i += 512) {
        const int kk = i % KT, n = i / KT;
        const int g = kk / GW, e = kk % GW;
        Bs[n * BST + kk] =
            e < KW * CIC ? p.b[(int64_t)(g * KW * CIC + e) * p.sbk + c_slab + n] : 0.0f;
    }
    __syncthreads();

    const int first = t_beg + wave;
    const int n = first < t_end ? (t_end - 1 - first) / 8 + 1 : 0;  // tiles of this wave
    if (n == 0) return;
    const int col0 = c_slab + li;
    float bias[FN];
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) bias[fn] = p.bias ? p.bias[col0 + fn * 32] : 0.0f;
    char* __restrict__ Cb = reinterpret_cast<char*>(p.c);
    const unsigned scm4 = (unsigned)p.scm * 4u;
    const unsigned coff0 = (unsigned)(4 * lh) * scm4 + (unsigned)col0 * 4u;
    const unsigned bsoff = (unsigned)li * BST + 4 * lh;
    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(p.a, (int64_t)p.cn * p.cih * p.ciw * CIC);
    const int row_elems = p.ciw * CIC;

    // Tile geometry of this lane's row: element offset of (ky 0, slot 4*lh), and bit masks of
    // the kernel rows inside the image and of the slots e' (e = e' + 4*lh) that are real
    // operands inside the image.
    struct Geo { int base; unsigned rowm, colm; };
    auto geo = [&](int t) __attribute__((always_inline)) {
        const int m = t * 32 + li;
        const int ox = m % p.cow, q = m / p.cow, oy = q % p.coh, img = q / p.coh;
        const int iy0 = oy * p.csh - p.cpt, ix0 = ox * p.csw - p.cpl;
        Geo g;
        g.base = ((img * p.cih + iy0) * p.ciw + ix0) * CIC + 4 * lh;
        g.rowm = 0;
#pragma unroll
        for (int ky = 0; ky < KH; ++ky) g.rowm |= ((unsigned)(iy0 + ky) < (unsigned)p.cih ? 1u : 0u) << ky;
        unsigned cm = 0;
#pragma unroll
        for (int e = 0; e < KW * CIC; ++e)
            cm |= ((unsigned)(ix0 + e / CIC) < (unsigned)p.ciw ? 1u : 0u) << e;
        g.colm = cm >> (4 * lh);
        return g;
    };
    auto load_step = [&](f4v& a, const Geo& g, int s) __attribute__((always_inline)) {
        const int ky = s / GS;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = 8 * (s % GS) + q;  // slot of lanes 0-31; lanes 32-63 take e + 4
            const bool ok = ((g.rowm >> ky) & (g.colm >> e) & 1u) != 0;
            const int off = g.base + ky * row_elems + e;
            a[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                 ra, ok ? (unsigned)off * 4u : kOobOffset, 0u, 0));
        }
    };
    auto eoff = [&](int t, int i) __attribute__((always_inline)) {
        const int r = i / FN, fn = i % FN;
        return coff0 + (unsigned)(t * 32 + 8 * (r >> 2) + (r & 3)) * scm4 + 128u * fn;
    };
    auto store_some = [&](const floatx16 (&acc)[FN], int t, int i0, int i1) __attribute__((always_inline)) {
#pragma unroll
        for (int i = i0; i < i1 && i < NST; ++i) {
            float v = acc[i % FN][i / FN] + bias[i % FN];
            if constexpr (ACT == 1) v = fmaxf(v, 0.0f);
            *reinterpret_cast<float*>(Cb + eoff(t, i)) = v;
        }
    };
    // Tile t from a (reloaded step by step with tile tn, geometry gn) into acc; when `store`,
    // tile tp's results (prev) are stored SPS per step.
    f4v a[KS];
    auto mma_tile = [&](floatx16 (&acc)[FN], const floatx16 (&prev)[FN], int tp, bool store,
                        const Geo& gn) __attribute__((always_inline)) {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fn][r] = 0.0f;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            f4v bf[FN];
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
                bf[fn] = *reinterpret_cast<const f4v*>(&Bs[bsoff + fn * 32 * BST + 8 * s]);
            if (store) store_some(prev, tp, s * SPS, (s + 1) * SPS);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int fn = 0; fn < FN; ++fn)
                    acc[fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s][q], bf[fn][q], acc[fn], 0, 0, 0);
            load_step(a[s], gn, s);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    const int tlast = first + (n - 1) * 8;
    floatx16 c0[FN], c1[FN];
    {
        const Geo g0 = geo(first);
#pragma unroll
        for (int s = 0; s < KS; ++s) load_step(a[s], g0, s);
    }
    mma_tile(c0, c1, 0, false, geo(min(first + 8, tlast)));
    int j = 1;
    for (; j + 1 < n; j += 2) {
        const int t = first + j * 8;  // tile j into c1, tile j + 1 into c0
        mma_tile(c1, c0, t - 8, true, geo(t + 8));
        mma_tile(c0, c1, t, true, geo(min(t + 16, tlast)));
    }
    if (j < n) {
        const int t = first + j * 8;
        mma_tile(c1, c0, t - 8, true, geo(t));
        store_some(c1, t, 0, NST);
    } else {
        store_some(c0, first + (j - 1) * 8, 0, NST);
    }
}

// ---- pipelined variant: operand tiles go from global memory straight into LDS
// (gfx950 global_load_lds_dwordx4: each lane moves 16 bytes, lane i of a wavefront writes
// bytes 16i..16i+15 of the 1 KiB block that M0 points at), through a ring of DMA_STAGES
// K tiles, so nothing is staged in registers and DMA_STAGES-1 tiles are in flight while one
// is multiplied.  Serves the two row-contiguous operand forms of the model paths: A =
// row-major rows (A_KVEC) or an NHWC im2col whose K tile sits inside one (ky, kx) tap, and
// B = [K][N] rows (B_NVEC).
//
// LDS layout of one stage (byte offsets):
//   A  128 rows x 16 k: block b of 16 rows at b*1024, chunk j (k 4j..4j+3) of row r at
//      (r/16)*1024 + j*256 + (r%16)*16.  A DMA instruction fills one block, lane i taking
//      row 16b + i%16, chunk i/16; a fragment read (16 lanes, consecutive rows, one chunk)
//      covers 256 contiguous bytes, so it is free of bank conflicts.
//   B  16 k rows x BN: each DMA instruction fills 256/BN whole rows (1 KiB) and the blocks
//      are BPAD bytes apart, so lanes 32-63 (k + 8) land 32 banks away from lanes 0-31.
// Chunks outside the operand (padding taps, the K tail, rows/columns past M/N) are read
// from a zero page, so their LDS slots hold zeros.
__device__ __attribute__((aligned(64))) float g_dma_zero[16];

__device__ __forceinline__ void dma16(const float* src, unsigned lds_byte) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds_byte) : "memory");
}

// Wait until at most N of this wavefront's vector-memory operations are outstanding and
// its LDS reads are done, then synchronise the workgroup.
template <int N>
__device__ __forceinline__ void dma_wait_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

constexpr int DMA_STAGES = 4;

template <int BN>
struct DmaTile {
    static constexpr int BM = 128, BK = 16, WM = 2, WN = 2;
    static constexpr int A_BYTES = BM * BK * 4;              // 8 KiB
    static constexpr int B_RPI = 256 / BN;                   // B rows per DMA instruction
    static constexpr int B_INS = BK / B_RPI;                 // DMA instructions per B tile
    static constexpr int BPAD = BN == 128 ? 32 : 64;
    static constexpr int B_STRIDE = 1024 + BPAD;
    static constexpr int STAGE = A_BYTES + B_INS * B_STRIDE;
    static constexpr int A_PW = BM / 16 / 4;                 // A instructions per wavefront
    static constexpr int B_PW = B_INS / 4;                   // B instructions per wavefront
    static constexpr int NDMA = A_PW + B_PW;
    static constexpr int CS = BN + 4;
    static constexpr int SMEM = DMA_STAGES * STAGE;
    static constexpr int RC = BM * CS * 4 <= SMEM ? BM : (BM / 2) * CS * 4 <= SMEM ? BM / 2 : 32;
    static_assert(B_PW >= 1 && B_INS % 4 == 0, "B tile must split over four wavefronts");
};

// One output tile (m0, n0) of batch bz over the K range [kbeg, kend): the whole pipeline from
// the first DMA to the epilogue.  split / nsplit / ctr / nbatch go to the epilogue (the K
// segment's index, how many segments share the tile, its arrival counter, the partial
// buffer's batch count).  Leaves the LDS ring free (every DMA drained, every read done by
// the caller's barrier after it).
template <int BN, int AM>
__device__ __attribute__((always_inline)) inline void dma_segment(
    const GemmParams& p, char* smem, int m0, int n0, int bz, int kbeg, int kend, int split,
    int nsplit, int nbatch, int64_t ctr) {
    using T = DmaTile<BN>;
    constexpr int BM = T::BM, BK = T::BK, WM = T::WM, WN = T::WN;
    constexpr int FM = BM / WM / 32;
    constexpr int FN = BN / WN / 32;
    static_assert(AM == shp::A_KVEC || AM == shp::A_CONV_NHWC4, "row-contiguous A only");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int li = lane & 31, lh = lane >> 5;

    const int bo = bz / p.batch_inner, bi = bz % p.batch_inner;
    const float* __restrict__ A = p.a + bo * p.sa_outer + bi * p.sa_inner;
    const float* __restrict__ B = p.b + bo * p.sb_outer + bi * p.sb_inner;
    const int ntk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const float* const zero = g_dma_zero;

    // ---- DMA source coordinates of this lane
    const int achunk = (lane >> 4) * 4;  // k offset of this lane's A chunk in a K tile
    ConvRow crow[T::A_PW];
    const float* arow[T::A_PW];  // row-major A: this lane's chunk at k = 0 (row 0 past M)
    bool aok[T::A_PW];
#pragma unroll
    for (int u = 0; u < T::A_PW; ++u) {
        const int m = m0 + (wave * T::A_PW + u) * 16 + (lane & 15);
        aok[u] = m < p.M;
        if constexpr (AM == shp::A_CONV_NHWC4) crow[u] = conv_row(p, m, AM);
        else arow[u] = A + (int64_t)(aok[u] ? m : 0) * p.sam + achunk;
    }
    const int bn = n0 + (lane % (BN / 4)) * 4;
    const bool bn_ok = bn < p.N;
    int bkl[T::B_PW];
    const float* brow[T::B_PW];  // B: this lane's chunk of row bkl at k tile 0
#pragma unroll
    for (int u = 0; u < T::B_PW; ++u) {
        bkl[u] = (wave * T::B_PW + u) * T::B_RPI + lane / (BN / 4);
        brow[u] = B + (int64_t)bkl[u] * p.sbk + (bn_ok ? bn : 0);
    }

    // Position of the next K tile to issue (uniform): its first k and, for a convolution,
    // its tap (ky, kx) and first channel, advanced tile by tile instead of divided out.
    int q_tile = 0, q_kt0 = kbeg, q_ic0 = 0, q_kx = 0, q_ky = 0;
    if constexpr (AM == shp::A_CONV_NHWC4) {
        q_ic0 = kbeg % p.cic;
        const int t = kbeg / p.cic;
        q_kx = t % p.ckw;
        q_ky = t / p.ckw;
    }
    const unsigned lds0 = (unsigned)(uintptr_t)smem;

    // One DMA instruction of the tile at q_*: A block u, B block u.  Every tile issues
    // exactly NDMA of them per wavefront, a tile past the end reading only the zero page,
    // so the vmcnt counts below hold on every iteration.
    // (Conditions use '&' and both addresses exist before the select, so this stays
    // straight-line code: no exec-masked branches between the MFMAs.)
    auto dma_a = [&](int u, unsigned sb) __attribute__((always_inline)) {
        const bool kin = (q_tile < ntk) & (q_kt0 + achunk < kend);
        const unsigned dst = __builtin_amdgcn_readfirstlane(sb + (wave * T::A_PW + u) * 1024);
        if constexpr (AM == shp::A_CONV_NHWC4) {
            const int64_t toff = ((int64_t)q_ky * p.ciw + q_kx) * p.cic + q_ic0 + achunk;
            const int iy = crow[u].iy0 + q_ky, ix = crow[u].ix0 + q_kx;
            const bool ok = kin & crow[u].valid & ((unsigned)iy < (unsigned)p.cih) &
                            ((unsigned)ix < (unsigned)p.ciw);
            const float* src = A + crow[u].base + toff;
            dma16(ok ? src : zero, dst);
        } else {
            const float* src = arow[u] + q_kt0;
            dma16((kin && aok[u]) ? src : zero, dst);
        }
    };
    auto dma_b = [&](int u, unsigned sb) __attribute__((always_inline)) {
        const bool ok = (q_tile < ntk) & bn_ok & (q_kt0 + bkl[u] < kend);
        const float* src = brow[u] + (int64_t)q_kt0 * p.sbk;
        dma16(ok ? src : zero,
              __builtin_amdgcn_readfirstlane(sb + T::A_BYTES + (wave * T::B_PW + u) * T::B_STRIDE));
    };
    auto advance = [&]() __attribute__((always_inline)) {
        ++q_tile;
        q_kt0 += BK;
        if constexpr (AM == shp::A_CONV_NHWC4) {
            q_ic0 += BK;
            if (q_ic0 >= p.cic) {
                q_ic0 = 0;
                if (++q_kx == p.ckw) {
                    q_kx = 0;
                    ++q_ky;
                }
            }
        }
    };

    // ---- fragments.  Lanes 0-31 feed k = s and lanes 32-63 k = 8 + s of MFMA step s, so a
    // lane's A values are chunks 2*lh and 2*lh + 1 of its row; B values are scalars.
    int aoff[FM][2];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
        const int r = wm * (BM / WM) + fm * 32 + li;
#pragma unroll
        for (int c = 0; c < 2; ++c) aoff[fm][c] = ((r >> 4) * 4 + 2 * lh + c) * 256 + (r & 15) * 16;
    }
    const int bcol = wn * (BN / WN) + li;
    constexpr int NRA = 2 * FM;  // A fragment reads (float4) per tile
    constexpr int NRB = 4 * FN;  // B fragment reads (pairs of k rows) per tile
    auto read_frag = [&](int j, const char* st, float4 (&af)[FM][2], float (&bf)[FN][8])
        __attribute__((always_inline)) {
        if (j < NRA) {
            af[j / 2][j % 2] = *reinterpret_cast<const float4*>(st + aoff[j / 2][j % 2]);
        } else {
            const int fn = (j - NRA) / 4, pr = (j - NRA) % 4;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int k = lh * 8 + 2 * pr + e;
                bf[fn][2 * pr + e] = *reinterpret_cast<const float*>(
                    st + T::A_BYTES + (k / T::B_RPI) * T::B_STRIDE + (k % T::B_RPI) * BN * 4 +
                    (bcol + fn * 32) * 4);
            }
        }
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // One K tile: its MFMAs, with the other work of the pipeline slotted between them so the
    // matrix pipe keeps running: the barrier that publishes tile kt + 1 a quarter of the way
    // in, then the fragment reads of tile kt + 1 into the other register set, one per MFMA,
    // and the DMA instructions of tile kt + DMA_STAGES - 1 spread out, half before the
    // barrier and half after the reads, so the four wavefronts never queue all of theirs
    // on the CU's address unit at once.
    constexpr int NM = 8 * FM * FN;
    constexpr int BAR = NM / 4;
    constexpr int RD_END = BAR + NRA + NRB;  // last MFMA slot followed by a fragment read
    constexpr int D_PRE = (T::NDMA + 1) / 2;  // DMA instructions before the barrier
    constexpr int D_POST = T::NDMA - D_PRE;
    static_assert(D_PRE <= BAR && RD_END + D_POST < NM, "pipeline slots must fit the MFMAs");
    auto dma_slot = [](int j) constexpr {
        return j < D_PRE ? j * (BAR / D_PRE)
                         : RD_END + 1 + (j - D_PRE) * ((NM - 1 - RD_END) / (D_POST > 0 ? D_POST : 1));
    };
    auto tile = [&](int kt, const float4 (&ac)[FM][2], const float (&bc)[FN][8],
                    float4 (&an)[FM][2], float (&bnx)[FN][8]) __attribute__((always_inline)) {
        const unsigned sb = lds0 + ((kt + DMA_STAGES - 1) % DMA_STAGES) * T::STAGE;
        const char* stn = smem + ((kt + 1) % DMA_STAGES) * T::STAGE;
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            const int st = i / (FM * FN), fm = (i / FN) % FM, fn = i % FN;
            const float4& a4 = ac[fm][st >> 2];
            const int q = st & 3;
            const float av = q == 0 ? a4.x : q == 1 ? a4.y : q == 2 ? a4.z : a4.w;
            acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bc[fn][st], acc[fm][fn], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < T::NDMA; ++j) {
                if (i != dma_slot(j)) continue;
                if (j < T::A_PW) dma_a(j, sb);
                else dma_b(j - T::A_PW, sb);
                if (j == T::NDMA - 1) advance();
            }
            // tile kt + 1 has landed for every wavefront (younger: tile kt + 2 and the first
            // D_PRE instructions of tile kt + 3); every read of tile kt - 1 is done
            if (i == BAR) dma_wait_barrier<(DMA_STAGES - 3) * T::NDMA + D_PRE>();
            if (i > BAR && i <= BAR + NRA + NRB) read_frag(i - BAR - 1, stn, an, bnx);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    float4 fa0[FM][2], fa1[FM][2];
    float fb0[FN][8], fb1[FN][8];
#pragma unroll
    for (int s = 0; s < DMA_STAGES - 1; ++s) {
        const unsigned sb = lds0 + s * T::STAGE;
#pragma unroll
        for (int u = 0; u < T::A_PW; ++u) dma_a(u, sb);
#pragma unroll
        for (int u = 0; u < T::B_PW; ++u) dma_b(u, sb);
        advance();
    }
    dma_wait_barrier<(DMA_STAGES - 2) * T::NDMA>();
#pragma unroll
    for (int j = 0; j < NRA + NRB; ++j) read_frag(j, smem, fa0, fb0);
    for (int kt = 0; kt < ntk; kt += 2) {
        tile(kt, fa0, fb0, fa1, fb1);
        if (kt + 1 < ntk) tile(kt + 1, fa1, fb1, fa0, fb0);
    }
    // the ring is reused by the epilogue: drain the trailing (zero-page) DMAs first
    dma_wait_barrier<0>();
    gemm_epilogue<BM, BN, WM, WN, T::RC, T::CS, shp::C_STRIDED>(
        p, acc, reinterpret_cast<float*>(smem), m0, n0, split, nsplit, bz, bo, bi, nbatch, ctr);
}

// Tiled form: one workgroup per (tile, K split, batch), each XCD (block id mod 8) taking a
// contiguous run of tiles.
template <int BN, int AM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, BN == 128 ? 2 : 3))) void gemm_dma_kernel(GemmParams p) {
    using T = DmaTile<BN>;
    __shared__ __attribute__((aligned(1024))) char smem[T::SMEM];
    const int tiles_n = (p.N + BN - 1) / BN;
    const int tiles_m = (p.M + T::BM - 1) / T::BM;
    const WgCoords wc = wg_coords(tiles_m, tiles_n, p.splits, p.group_m);
    const int kbeg = wc.split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    dma_segment<BN, AM>(p, smem, wc.tm * T::BM, wc.tn * BN, blockIdx.z, kbeg,
                        kend, wc.split, p.splits, gridDim.z,
                        (int64_t)blockIdx.z * gridDim.x + wc.tile);
}

// Split-K second pass: sum the partials in split order, then the epilogue.
template <int CM>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmParams p, int nbatch) {
    const int64_t mn = (int64_t)p.M * p.N;
    const int64_t total = mn * nbatch;
    const int hw = p.coh * p.cow;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        int bz = (int)(i / mn);
        int64_t rem = i % mn;
        int row = (int)(rem / p.N), col = (int)(rem % p.N);
        float v = 0.0f;
        for (int s = 0; s < p.splits; ++s) v += p.partial[((int64_t)s * nbatch + bz) * mn + rem];
        int bo = bz / p.batch_inner, bi = bz % p.batch_inner;
        int64_t ci;
        if constexpr (CM == shp::C_NCHW) {
            int img = row / hw, pix = row % hw;
            ci = ((int64_t)img * p.N + col) * hw + pix;
        } else {
            ci = bo * p.sc_outer + bi * p.sc_inner + (int64_t)row * p.scm + (int64_t)col * p.scn;
        }
        if (p.bias) v += p.bias[col];
        if (p.residual) v += p.residual[ci];
        p.c[ci] = shpd::apply_act(v, p.act, p.alpha);
    }
}

// ---- skinny products: M <= 8 rows against a [N][K] weight (fully_connected at batch
// 1..8).  One wavefront per output column reads that column's K weights once with 16-byte
// loads; the M activation rows come from cache.  HBM-bound like a GEMV.
template <int MR>
__global__ __launch_bounds__(256) void skinny_nt_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ w,
                                                        float* __restrict__ y, int M, int N,
                                                        int K, const float* __restrict__ bias,
                                                        int act, float alpha) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    const float* wr = w + (int64_t)n * K;
    const float bn = bias ? bias[n] : 0.0f;  // loaded with the weights, used by lane 0
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
    const bool vec = (K % 4 == 0) && (((uintptr_t)w & 15) == 0) && (((uintptr_t)x & 15) == 0);
    if (MR == 1 && vec && K <= 2048) {
        // one row: every weight and activation load of the lane (up to eight 256-wide K
        // steps) goes out before the first product, one round trip; the sums run in K order
        // as below
        float4 wv[8], xv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int k = lane * 4 + 256 * j;
            if (k < K) {
                wv[j] = *reinterpret_cast<const float4*>(wr + k);
                xv[j] = *reinterpret_cast<const float4*>(x + k);
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (lane * 4 + 256 * j < K)
                acc[0] += wv[j].x * xv[j].x + wv[j].y * xv[j].y + wv[j].z * xv[j].z +
                          wv[j].w * xv[j].w;
    } else if (vec) {
        // four 256-wide K steps' weight loads go out together (one HBM round trip per four
        // steps, not per step); the sums still run in K order
        for (int k0 = lane * 4; k0 < K; k0 += 1024) {
            float4 wv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (k0 + 256 * j < K) wv[j] = *reinterpret_cast<const float4*>(wr + k0 + 256 * j);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = k0 + 256 * j;
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    if (m < M && k < K) {
                        float4 xv = *reinterpret_cast<const float4*>(x + (int64_t)m * K + k);
                        acc[m] += wv[j].x * xv.x + wv[j].y * xv.y + wv[j].z * xv.z + wv[j].w * xv.w;
                    }
                }
            }
        }
    } else {
        for (int k = lane; k < K; k += 64) {
            float wv = wr[k];
#pragma unroll
            for (int m = 0; m < MR; ++m)
                if (m < M) acc[m] += wv * x[(int64_t)m * K + k];
        }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        float v = acc[m];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
        acc[m] = v;
    }
    if (lane == 0)
        for (int m = 0; m < M; ++m) y[(int64_t)m * N + n] = shpd::apply_act(acc[m] + bn, act, alpha);
}

// The same product for 2..8 rows with the rows staged in LDS once per workgroup: each
// wavefront takes two output columns, so the M activation rows are read from L2 once per
// eight columns (the kernel above reads them once per column, 40 KB per column at M = 8,
// K = 1280).  Per lane and column the sums run in the same order as in the kernel above.
template <int MR>
__global__ __launch_bounds__(256) void skinny_nt_lds_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            float* __restrict__ y, int M, int N,
                                                            int K, const float* __restrict__ bias,
                                                            int act, float alpha) {
    extern __shared__ __attribute__((aligned(16))) float xs[];  // [M][K]
    const int lane = threadIdx.x & 63;
    const int n0 = blockIdx.x * 8 + 2 * (threadIdx.x >> 6);
    const bool col = n0 < N;
    const bool two = n0 + 1 < N;
    const float* w0 = w + (int64_t)(col ? n0 : 0) * K;
    const float* w1 = two ? w0 + K : w0;
    // K <= 2048: all of this lane's weights of both columns are loaded first, so their HBM
    // round trip overlaps the staging of x (longer K loops four K steps at a time below)
    constexpr int KR = 8;
    const bool resident = K <= 256 * KR;
    f4v u[KR], v[KR];
    if (resident && col) {
#pragma unroll
        for (int j = 0; j < KR; ++j) {
            const int k = lane * 4 + 256 * j;
            if (k < K) {
                u[j] = *reinterpret_cast<const f4v*>(w0 + k);
                v[j] = *reinterpret_cast<const f4v*>(w1 + k);
            }
        }
    }
    for (int i0 = threadIdx.x * 4; i0 < M * K; i0 += 8192) {  // 8 loads in flight per thread
        f4v t[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
            if (i0 + 1024 * q < M * K) t[q] = *reinterpret_cast<const f4v*>(x + i0 + 1024 * q);
#pragma unroll
        for (int q = 0; q < 8; ++q)
            if (i0 + 1024 * q < M * K) *reinterpret_cast<f4v*>(xs + i0 + 1024 * q) = t[q];
    }
    __syncthreads();
    if (!col) return;
    float a0[MR], a1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) a0[m] = a1[m] = 0.0f;
    auto step = [&](const f4v& uj, const f4v& vj, int k) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (m < M) {
                const f4v xv = *reinterpret_cast<const f4v*>(xs + m * K + k);
                a0[m] += uj.x * xv.x + uj.y * xv.y + uj.z * xv.z + uj.w * xv.w;
                a1[m] += vj.x * xv.x + vj.y * xv.y + vj.z * xv.z + vj.w * xv.w;
            }
        }
    };
    if (resident) {
#pragma unroll
        for (int j = 0; j < KR; ++j) {
            const int k = lane * 4 + 256 * j;
            if (k < K) step(u[j], v[j], k);
        }
    } else {
        for (int k0 = lane * 4; k0 < K; k0 += 1024) {  // four K steps' weights in flight
            f4v uu[4], vv[4];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                if (k0 + 256 * jj < K) {
                    uu[jj] = *reinterpret_cast<const f4v*>(w0 + k0 + 256 * jj);
                    vv[jj] = *reinterpret_cast<const f4v*>(w1 + k0 + 256 * jj);
                }
            }
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                if (k0 + 256 * jj < K) step(uu[jj], vv[jj], k0 + 256 * jj);
        }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        float p = a0[m], q = a1[m];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            p += __shfl_xor(p, o);
            q += __shfl_xor(q, o);
        }
        a0[m] = p;
        a1[m] = q;
    }
    if (lane == 0) {
        const float b0 = bias ? bias[n0] : 0.0f;
        for (int m = 0; m < M; ++m) y[(int64_t)m * N + n0] = shpd::apply_act(a0[m] + b0, act, alpha);
        if (two) {
            const float b1 = bias ? bias[n0 + 1] : 0.0f;
            for (int m = 0; m < M; ++m)
                y[(int64_t)m * N + n0 + 1] = shpd::apply_act(a1[m] + b1, act, alpha);
        }
    }
}

// ---- small products (small_gemm_kernel): C[M][N] = A[M][K] B[N][K]^T + bias (+ residual),
// activation, for grids the 64x64 tiles would leave half empty (the 1x1 convolutions of
// MobileNetV2 at batch 1: M 49-12,544, N 16-1,280, K 16-960; the expand convolutions of
// EfficientNet-Lite0 at batch 8: M 392-1,568, N 480-1,152, K 80-192).
// A workgroup owns a 32x32 output tile and each wavefront one 16x16 block of it on
// v_mfma_f32_16x16x4_f32.  The tile's 64 operand rows (32 of A, 32 of B) are staged through
// LDS in 16-wide K chunks: thread t owns row t / 4 and K quarter t % 4 of every chunk (16
// contiguous bytes; K past the end reads zeros through the buffer range), and issues the
// loads of all its chunks at once.  Chunk c is stored to an LDS slice and multiplied as soon
// as its load lands, so the MFMAs of early chunks overlap the arrival of later ones; two
// accumulators take alternate chunks.  Measured at 32x32 against register-resident
// fragments (each wavefront loading its own rows), all-loads-then-multiply through LDS, and
// 64-wide tiles: 1.4-1.7x faster on the EfficientNet-Lite0 expand shapes; two 5 KB slices
// instead of one slice per chunk keep the workgroup's LDS small enough for 8 per CU.
typedef float floatx4s __attribute__((ext_vector_type(4)));
__device__ __forceinline__ floatx4s mfma4_16(f4v a, f4v b, floatx4s c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, c, 0, 0, 0);
}
constexpr int kSmallKc = 16;        // 16-wide K chunks of one workgroup at most
constexpr int kSmallMaxSplits = 8;  // K ranges of one tile: K <= 16 * 16 * 8 = 2,048
// LDS: chunk c goes to slice c % 2 of 64 rows x kSmallRs floats (16 + a 4-float pad that
// spreads the 16 rows a fragment read touches over the banks); a slice is rewritten two chunks
// later, after every wavefront has passed the barrier that follows its last read of it
constexpr int kSmallRs = 20;
constexpr int kSmallSlice = 64 * kSmallRs;
// With gridDim.y = S > 1 the workgroups (tile, s) take the s-th of S equal runs of K's
// chunks, store their partial tiles with device-coherent stores into `part` (S x 256 float4
// per tile) and count their arrival on the tile's counter; the last arrival sums the partials
// in split order and applies the epilogue, then clears the counter.
template <int KC>
__global__ __launch_bounds__(256) void small_gemm_kernel(const float* __restrict__ A,
                                                         const float* __restrict__ B,
                                                         float* __restrict__ C, int M, int N,
                                                         int K, int tiles_n,
                                                         const float* __restrict__ bias,
                                                         const float* __restrict__ res, int act,
                                                         float alpha, float* __restrict__ part,
                                                         int* __restrict__ counters) {
    __shared__ float sg_lds[2 * kSmallSlice];
    __shared__ int last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, li = lane & 15;
    const int S = gridDim.y, si = blockIdx.y;
    const int kc_all = (K + 15) >> 4, cps = (kc_all + S - 1) / S;
    const int c0 = si * cps, kc = min(cps, kc_all - c0);
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
    const int mb = tm * 32, nb = tn * 32;
    const __amdgpu_buffer_rsrc_t ar = buffer_rsrc(A, (int64_t)M * K);
    const __amdgpu_buffer_rsrc_t br = buffer_rsrc(B, (int64_t)N * K);
    const int sr = tid >> 2, sq = tid & 3;  // staged row (0-31 of A, 32-63 of B), K quarter
    const bool isa = sr < 32;
    const int grow = isa ? mb + sr : nb + sr - 32;
    const bool rok = grow < (isa ? M : N);
    const unsigned base = rok ? (unsigned)(grow * K + 16 * c0 + 4 * sq) * 4u : 0u;
    f4v st[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c)
        st[c] = buffer_load4(isa ? ar : br,
                             rok && c < kc && 16 * (c0 + c) + 4 * sq < K ? base + 64u * c
                                                                        : kOobOffset,
                             0u);
    const int wm = wave >> 1, wn = wave & 1;
    // the epilogue's bias and residuals load with the operands, not after the products
    const int col = nb + wn * 16 + li;
    const float bv = bias && col < N ? bias[col] : 0.0f;
    float rv[4] = {0.f, 0.f, 0.f, 0.f};
    if (res && col < N) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mb + wm * 16 + 4 * g + r;
            if (m < M) rv[r] = res[(int64_t)m * N + col];
        }
    }
    const int fa = (wm * 16 + li) * kSmallRs + 4 * g;
    const int fb = (32 + wn * 16 + li) * kSmallRs + 4 * g;
    floatx4s e0 = {0.f, 0.f, 0.f, 0.f}, e1 = e0;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        if (c < kc) {  // uniform over the workgroup
            float* sl = sg_lds + (c & 1) * kSmallSlice;
            *(f4v*)(sl + sr * kSmallRs + 4 * sq) = st[c];
            __syncthreads();
            const f4v af = *(const f4v*)(sl + fa), bf = *(const f4v*)(sl + fb);
            if (c & 1) e1 = mfma4_16(af, bf, e1);
            else e0 = mfma4_16(af, bf, e0);
        }
    }
    if (S > 1) {
        const __amdgpu_buffer_rsrc_t prs =
            buffer_rsrc(part + (int64_t)blockIdx.x * S * 1024, (int64_t)S * 1024);
        st_coh16(prs, (unsigned)((si * 256 + tid) * 16),
                 make_float4(e0[0] + e1[0], e0[1] + e1[1], e0[2] + e1[2], e0[3] + e1[3]));
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partial is stored
        __syncthreads();
        if (tid == 0)
            last = __hip_atomic_fetch_add((SHP_GLOBAL int*)(counters + blockIdx.x), 1,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
        __syncthreads();
        if (!last) return;
        if (tid == 0)  // every split has arrived: the counter is free for the next launch
            __hip_atomic_store((SHP_GLOBAL int*)(counters + blockIdx.x), 0, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        float4 q[kSmallMaxSplits];
#pragma unroll
        for (int u = 0; u < kSmallMaxSplits; ++u)
            if (u < S) q[u] = ld_coh16(prs, (unsigned)((u * 256 + tid) * 16), 0);
        f4v t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < kSmallMaxSplits; ++u)
            if (u < S) t += f4v{q[u].x, q[u].y, q[u].z, q[u].w};
        e0 = floatx4s{t.x, t.y, t.z, t.w};
        e1 = floatx4s{0.f, 0.f, 0.f, 0.f};
    }
    if (col >= N) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // accumulator r: row 4g + r of the block, column li
        const int m = mb + wm * 16 + 4 * g + r;
        if (m < M) {
            const int64_t o = (int64_t)m * N + col;
            float v = e0[r] + e1[r] + bv;
            if (res) v += rv[r];
            C[o] = shpd::apply_act(v, act, alpha);
        }
    }
}

// K-splits of the small-product path for an [M][K] x [N][K]^T product (0: not taken).  K <=
// 256 runs unsplit where the 64x64 tiles would give fewer than 512 workgroups; a longer K (up
// to 2,048) is cut into equal runs of at most 16 chunks, more of them (up to 8) while the
// grid has fewer than 1,024 workgroups (swept over 2-8 splits on the MobileNetV2 and
// EfficientNet-Lite0 projections: within 0.5 us of the best count; the same growth for K <= 256
// split the EfficientNet-Lite0 b8 expands and cost that forward 11 us).  `small` is the
// gemm_small tune value: -1 never, 1 wherever the shape fits, k >= 2 with k splits.
int small_gemm_splits(int64_t M, int64_t N, int K, int small) {
    if (small < 0 || M <= 0 || N <= 0 || K <= 0 || K % 4 ||
        K > 16 * kSmallKc * kSmallMaxSplits)
        return 0;
    if (M * K * 4 >= (1ll << 31) || N * K * 4 >= (1ll << 31)) return 0;
    if (small == 0 && ((M + 63) / 64) * ((N + 63) / 64) >= 512) return 0;
    const int kc = (K + 15) / 16;
    const int64_t tiles = ((M + 31) / 32) * ((N + 31) / 32);
    if (tiles >= (1ll << 31)) return 0;
    int sp = small >= 2 ? std::min(small, kSmallMaxSplits) : (kc + kSmallKc - 1) / kSmallKc;
    if (small < 2 && kc > kSmallKc)
        while (sp < kSmallMaxSplits && sp < kc && tiles * sp < 1024) ++sp;
    const int cps = (kc + sp - 1) / sp;
    if (cps > kSmallKc) return 0;
    sp = (kc + cps - 1) / cps;  // every split gets at least one chunk
    if (sp > 1 && tiles * (int64_t)sizeof(int) > (int64_t)shp::kSplitCounterBytes) return 0;
    return sp;
}
size_t small_gemm_workspace(int64_t M, int64_t N, int splits) {
    if (splits <= 1) return 0;
    const int64_t tiles = ((M + 31) / 32) * ((N + 31) / 32);
    return shp::kSplitCounterBytes + (size_t)tiles * splits * 256 * sizeof(float4);
}

// ---- fully_connected with 2-16 rows (fc_mfma_kernel): y[M][N] = x[M][K] W[N][K]^T + bias
// (+ residual), activation.  One workgroup of 16 wavefronts owns 16 output columns, and
// wavefront w takes the w-th sixteenth of K's 16-wide chunks on v_mfma_f32_16x16x4_f32 (rows
// past M, columns past N and K past the end read zeros through the buffer range), with all its
// loads issued before the first MFMA.  The sixteen partial 16x16 tiles are summed in LDS in
// wavefront order.  The weights are the traffic (5 MB at K = 1,280, N = 1,000): ~1,000
// wavefronts stream them once, where the wavefront-per-column kernels gave each wavefront a
// whole 5 KB column plus the M activation rows (EfficientNet-Lite0's classifier at batch 8:
// 12.6 us for one wavefront per column, 6.0 us here, graph-replayed with the weights cold).
constexpr int kFcWaves = 16;
template <int CPW>
__global__ __launch_bounds__(kFcWaves * 64) void fc_mfma_kernel(
    const float* __restrict__ X, const float* __restrict__ W, float* __restrict__ Y, int M, int N,
    int K, const float* __restrict__ bias, const float* __restrict__ res, int act, float alpha) {
    __shared__ float red[kFcWaves * 4 * 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, li = lane & 15;
    const int n0 = blockIdx.x * 16;
    const int kc = (K + 15) >> 4, cpw = (kc + kFcWaves - 1) / kFcWaves, c0 = wave * cpw;
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, (int64_t)M * K);
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(W, (int64_t)N * K);
    const bool xok = li < M, wok = n0 + li < N;
    const unsigned xb = (unsigned)(li * K + 4 * g) * 4u;
    const unsigned wb = (unsigned)((n0 + li) * K + 4 * g) * 4u;
    // the epilogue's bias and residual (thread tid < 256: row tid / 16, column tid % 16) load
    // with the operands
    const int orow = tid >> 4, ocol = n0 + (tid & 15);
    const bool oown = tid < 256 && orow < M && ocol < N;
    const float obias = oown && bias ? bias[ocol] : 0.0f;
    const float ores = oown && res ? res[(int64_t)orow * N + ocol] : 0.0f;
    f4v a[CPW], b[CPW];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
        const bool ok = j < cpw && 16 * (c0 + j) + 4 * g < K;
        b[j] = buffer_load4(wr, ok && wok ? wb + 64u * (c0 + j) : kOobOffset, 0u);
    }
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
        const bool ok = j < cpw && 16 * (c0 + j) + 4 * g < K;
        a[j] = buffer_load4(xr, ok && xok ? xb + 64u * (c0 + j) : kOobOffset, 0u);
    }
    floatx4s e0 = {0.f, 0.f, 0.f, 0.f}, e1 = e0;
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
        if (j & 1) e1 = mfma4_16(a[j], b[j], e1);
        else e0 = mfma4_16(a[j], b[j], e0);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(wave * 4 + r) * 64 + lane] = e0[r] + e1[r];
    __syncthreads();
    if (tid < 256) {  // output row tid / 16, column n0 + tid % 16: lane (row / 4) * 16 + col, r = row % 4
        const int row = tid >> 4, col = tid & 15;
        const int l = (row >> 2) * 16 + col, r = row & 3;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kFcWaves; ++w) v += red[(w * 4 + r) * 64 + l];
        if (oown) {
            v += obias;
            if (res) v += ores;
            Y[(int64_t)row * N + n0 + col] = shpd::apply_act(v, act, alpha);
        }
    }
}

// ---- host-side dispatch --------------------------------------------------------------
struct TileCfg {
    int bm, bn, bk;
    bool dma;         // the pipelined gemm_dma_kernel (BM 128, BK 16) instead of gemm_mfma_kernel
    int pg;           // gemm_mfma_kernel global prefetch depth (0 or 1: one tile, 2: two tiles)
    bool bl = false;  // gemm_bl_kernel (buffer-loaded) instead of gemm_mfma_kernel
};

// The pipelined kernel takes row-contiguous operands whose 16-byte chunks are aligned:
// A rows (or an NHWC input whose channel count is a multiple of its K tile) and [K][N] B.
bool dma_eligible(const GemmParams& p, int am, int bm, int cm) {
    using namespace shp;
    if (cm != C_STRIDED || bm != B_NVEC) return false;
    if (am == A_CONV_NHWC4) {
        if (p.cic % 16 != 0) return false;
    } else if (am == A_KVEC) {
        if (p.sak != 1 || p.K % 4 || p.sam % 4 || p.sa_outer % 4 || p.sa_inner % 4) return false;
    } else {
        return false;
    }
    return p.N % 4 == 0 && p.sbk % 4 == 0 && p.sb_outer % 4 == 0 && p.sb_inner % 4 == 0 &&
           ((uintptr_t)p.a & 15) == 0 && ((uintptr_t)p.b & 15) == 0;
}

// Where the pipelined kernel measured faster than the double-buffered one on MI355X
// (per-layer sweeps of the ResNet-50 b32 convolutions; on the BERT-base row-major products
// it measured slower, so those keep the double-buffered kernel): a 128x64 tile without split-K,
// K from 512 to 1152, and a grid of 192..512 tiles (about one or two per CU).  Shorter
// K loops spend too much of a 128-row tile in its prologue and epilogue; larger grids
// run as well on the 64x64 kernel at four workgroups per CU; smaller grids or longer K
// need split-K, where the 64x64 kernel's finer partials fill the CUs better.
bool dma_preferred(const GemmParams& p, int nbatch) {
    const int64_t tiles = (int64_t)((p.M + 127) / 128) * ((p.N + 63) / 64) * nbatch;
    return p.K >= 512 && p.K <= 1152 && tiles >= 192 && tiles <= 512;
}

int launch_dma(hipStream_t s, const GemmParams& p, int am, int bn, dim3 grid) {
    using namespace shp;
    if (am == A_CONV_NHWC4) {
        if (bn == 128) hipLaunchKernelGGL((gemm_dma_kernel<128, A_CONV_NHWC4>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((gemm_dma_kernel<64, A_CONV_NHWC4>), grid, dim3(256), 0, s, p);
    } else {
        if (bn == 128) hipLaunchKernelGGL((gemm_dma_kernel<128, A_KVEC>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((gemm_dma_kernel<64, A_KVEC>), grid, dim3(256), 0, s, p);
    }
    return SHP_OK;
}

template <int BM, int BN, int BK, int AM, int BMD, int CM, int PG = 1>
void launch_tile(hipStream_t s, const GemmParams& p, dim3 grid) {
    hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, 2, 2, BK, AM, BMD, CM, PG>), grid, dim3(256), 0, s, p);
}

// HOT combos (the model paths) get the BK=16 variants as well.
template <int AM, int BMD, int CM, bool HOT>
void launch_combo(hipStream_t s, const GemmParams& p, TileCfg t, dim3 grid) {
    if constexpr (HOT) {
        if (t.pg == 2) {
            if (t.bk == 16) {
                if (t.bm == 128 && t.bn == 128) return launch_tile<128, 128, 16, AM, BMD, CM, 2>(s, p, grid);
                if (t.bm == 128 && t.bn == 64) return launch_tile<128, 64, 16, AM, BMD, CM, 2>(s, p, grid);
                return launch_tile<64, 64, 16, AM, BMD, CM, 2>(s, p, grid);
            }
            if (t.bm == 128 && t.bn == 128) return launch_tile<128, 128, 32, AM, BMD, CM, 2>(s, p, grid);
            if (t.bm == 128 && t.bn == 64) return launch_tile<128, 64, 32, AM, BMD, CM, 2>(s, p, grid);
            return launch_tile<64, 64, 32, AM, BMD, CM, 2>(s, p, grid);
        }
        if (t.bk == 16) {
            if (t.bm == 128 && t.bn == 128) return launch_tile<128, 128, 16, AM, BMD, CM>(s, p, grid);
            if (t.bm == 128 && t.bn == 64) return launch_tile<128, 64, 16, AM, BMD, CM>(s, p, grid);
            return launch_tile<64, 64, 16, AM, BMD, CM>(s, p, grid);
        }
    }
    if (t.bm == 128 && t.bn == 128) return launch_tile<128, 128, 32, AM, BMD, CM>(s, p, grid);
    if (t.bm == 128 && t.bn == 64) return launch_tile<128, 64, 32, AM, BMD, CM>(s, p, grid);
    return launch_tile<64, 64, 32, AM, BMD, CM>(s, p, grid);
}

bool combo_is_hot(int am, int bm, int cm) {
    using namespace shp;
    return cm == C_STRIDED && ((am == A_CONV_NHWC4 && bm == B_NVEC) ||
                               (am == A_CONV_NHWC4 && bm == B_KVEC) ||
                               (am == A_KVEC && bm == B_NVEC) || (am == A_KVEC && bm == B_KVEC));
}

int dispatch_combo(hipStream_t s, const GemmParams& p, int am, int bm, int cm, TileCfg t,
                   dim3 grid) {
    using namespace shp;
#define SHP_COMBO(A_, B_, C_, HOT_)                      \
    if (am == A_ && bm == B_ && cm == C_) {               \
        launch_combo<A_, B_, C_, HOT_>(s, p, t, grid);   \
        return SHP_OK;                                   \
    }
    SHP_COMBO(A_CONV_NHWC4, B_NVEC, C_STRIDED, true)
    SHP_COMBO(A_CONV_NHWC4, B_KVEC, C_STRIDED, true)
    SHP_COMBO(A_CONV_NHWC4, B_STRIDED, C_STRIDED, false)
    SHP_COMBO(A_CONV_NHWC, B_NVEC, C_STRIDED, false)
    SHP_COMBO(A_CONV_NHWC, B_KVEC, C_STRIDED, false)
    SHP_COMBO(A_CONV_NHWC, B_STRIDED, C_STRIDED, false)
    SHP_COMBO(A_CONV_NCHW, B_KVEC, C_NCHW, false)
    SHP_COMBO(A_CONV_NCHW, B_STRIDED, C_NCHW, false)
    SHP_COMBO(A_KVEC, B_NVEC, C_STRIDED, true)
    SHP_COMBO(A_KVEC, B_KVEC, C_STRIDED, true)
    SHP_COMBO(A_KVEC, B_STRIDED, C_STRIDED, false)
    SHP_COMBO(A_STRIDED, B_NVEC, C_STRIDED, false)
    SHP_COMBO(A_STRIDED, B_KVEC, C_STRIDED, false)
    SHP_COMBO(A_STRIDED, B_STRIDED, C_STRIDED, false)
#undef SHP_COMBO
    return fail(SHP_ERR_UNSUPPORTED, "gemm: unsupported operand mode combination");
}

// gemm_bl_kernel takes 16-byte aligned row-contiguous operands whose ranges fit a buffer
// resource with every offset below kOobOffset, and K in whole K tiles of `bk`.
bool bl_eligible(const GemmParams& p, int am, int bm, int cm, int bk) {
    using namespace shp;
    if (cm != C_STRIDED || p.K < bk || p.K % bk != 0) return false;
    if (am == A_CONV_NHWC4) {
        if (p.cic % bk != 0) return false;
    } else if (am == A_KVEC) {
        if (p.sak != 1 || p.sam % 4) return false;
    } else {
        return false;
    }
    if (bm == B_NVEC) {
        if (p.sbn != 1 || p.sbk % 4 || p.N % 4) return false;
    } else if (bm == B_KVEC) {
        if (p.sbk != 1 || p.sbn % 4) return false;
    } else {
        return false;
    }
    if (p.sa_outer % 4 || p.sa_inner % 4 || p.sb_outer % 4 || p.sb_inner % 4) return false;
    if (((uintptr_t)p.a & 15) || ((uintptr_t)p.b & 15)) return false;
    const int64_t lim = (int64_t)1 << 29;  // floats: byte offsets stay below 2 GiB
    return bl_a_extent(p, am) <= lim && bl_b_extent(p, bm) <= lim;
}

// K tiles (bit 0: 16, bit 1: 32, bit 2: 64) for which the problem fits gemm_bl_kernel.
int bl_mask(const GemmParams& p, int am, int bm, int cm) {
    return (bl_eligible(p, am, bm, cm, 16) ? 1 : 0) | (bl_eligible(p, am, bm, cm, 32) ? 2 : 0) |
           (bl_eligible(p, am, bm, cm, 64) ? 4 : 0);
}

template <int AM, int BMD>
void launch_bl_combo(hipStream_t s, const GemmParams& p, TileCfg t, dim3 grid) {
    if (t.bm == 128 && t.bn == 128)
        hipLaunchKernelGGL((gemm_bl_kernel<128, 128, 32, AM, BMD>), grid, dim3(256), 0, s, p);
    else if (t.bm == 128)
        hipLaunchKernelGGL((gemm_bl_kernel<128, 64, 32, AM, BMD>), grid, dim3(256), 0, s, p);
    else if (t.bk == 64)
        hipLaunchKernelGGL((gemm_bl_kernel<64, 64, 64, AM, BMD>), grid, dim3(256), 0, s, p);
    else if (t.bk == 16)
        hipLaunchKernelGGL((gemm_bl_kernel<64, 64, 16, AM, BMD>), grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((gemm_bl_kernel<64, 64, 32, AM, BMD>), grid, dim3(256), 0, s, p);
}

int dispatch_bl(hipStream_t s, const GemmParams& p, int am, int bm, TileCfg t, dim3 grid) {
    using namespace shp;
    if (am == A_KVEC && bm == B_NVEC) launch_bl_combo<A_KVEC, B_NVEC>(s, p, t, grid);
    else if (am == A_KVEC && bm == B_KVEC) launch_bl_combo<A_KVEC, B_KVEC>(s, p, t, grid);
    else if (am == A_CONV_NHWC4 && bm == B_NVEC) launch_bl_combo<A_CONV_NHWC4, B_NVEC>(s, p, t, grid);
    else if (am == A_CONV_NHWC4 && bm == B_KVEC) launch_bl_combo<A_CONV_NHWC4, B_KVEC>(s, p, t, grid);
    else return fail(SHP_ERR_UNSUPPORTED, "gemm: operand forms outside the buffer-loaded kernel");
    return SHP_OK;
}

// The persistent small-K kernel's variant for a problem, 0 where it does not apply: K 64 with
// N 64 (1) or N a multiple of 256 (2); A plain rows or the input of a 1x1 stride-1 unpadded
// NHWC convolution, B [K][N], one batch, M a multiple of 32 with enough rows that every CU
// gets several 32-row tiles, no activation or ReLU.  (With K 128 the tiled kernel is as fast
// on the ResNet-50 shape: 45.0 against 44.9-47.2 us on 25088x512x128.)
int smallk_variant(const GemmParams& p, int am, int bm, int cm, int nbatch) {
    using namespace shp;
    if (nbatch != 1 || cm != C_STRIDED || p.scn != 1 || bm != B_NVEC || p.sbn != 1) return 0;
    if (p.act != SHP_ACT_NONE && p.act != SHP_ACT_RELU) return 0;
    if (p.sbk % 4 || ((uintptr_t)p.a & 15) || ((uintptr_t)p.b & 15) || p.M < 16384 || p.M % 32)
        return 0;
    // 32-bit byte offsets of A, C and the residual rows
    const int64_t lim = (int64_t)1 << 31;
    const int64_t a_rows = am == A_KVEC ? p.sam : p.cic;
    if ((int64_t)p.M * a_rows * 4 >= lim || (int64_t)p.M * p.scm * 4 >= lim) return 0;
    if (am == A_CONV_NHWC4 || am == A_CONV_NHWC) {
        if (p.ckh != 1 || p.ckw != 1 || p.csh != 1 || p.csw != 1 || p.cpt || p.cpl ||
            p.cih != p.coh || p.ciw != p.cow || p.cic != p.K)
            return 0;
    } else if (am != A_KVEC || p.sak != 1 || p.sam % 4) {
        return 0;
    }
    if (p.K == 64 && p.N == 64) return 1;
    if (p.K == 64 && p.N % 256 == 0) return 2;
    return 0;
}

int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

template <int KT, int FN, int WC, bool RES>
void launch_smallk_act(hipStream_t s, const GemmParams& p, int nslab, int nrange, dim3 grid, int act) {
    if (act == 0)
        hipLaunchKernelGGL((gemm_smallk_kernel<KT, FN, WC, 0, RES>), grid, dim3(512), 0, s, p, nslab, nrange);
    else
        hipLaunchKernelGGL((gemm_smallk_kernel<KT, FN, WC, 1, RES>), grid, dim3(512), 0, s, p, nslab, nrange);
}

// One workgroup per CU: nslab column slabs x nrange row ranges (a multiple of 8, so that the
// slabs of a range share an XCD).
int launch_smallk(hipStream_t s, GemmParams p, int am, int variant) {
    if (am != shp::A_KVEC) p.sam = p.cic;
    const int tn = variant == 1 ? 64 : 256;
    const int nslab = p.N / tn;
    const int nrange = std::max(8, device_cus() / nslab / 8 * 8);
    const dim3 grid((unsigned)(nrange * nslab));
    const int act = p.act == SHP_ACT_RELU ? 1 : 0;
    const bool res = p.residual != nullptr;
    if (variant == 1 && res) launch_smallk_act<64, 2, 1, true>(s, p, nslab, nrange, grid, act);
    else if (variant == 1) launch_smallk_act<64, 2, 1, false>(s, p, nslab, nrange, grid, act);
    else if (res) launch_smallk_act<64, 2, 4, true>(s, p, nslab, nrange, grid, act);
    else launch_smallk_act<64, 2, 4, false>(s, p, nslab, nrange, grid, act);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// The stem kernel takes the 7x7 3-channel NHWC convolution (any stride and padding) with N a
// multiple of 64, M a multiple of 32 and large, no residual, no activation or ReLU.
bool stem_eligible(const GemmParams& p, int am, int bm, int cm, int nbatch) {
    using namespace shp;
    if (am != A_CONV_NHWC || p.cic != 3 || p.ckh != 7 || p.ckw != 7 || p.K != 147) return false;
    if (nbatch != 1 || cm != C_STRIDED || p.scn != 1 || bm != B_NVEC || p.sbn != 1) return false;
    if (p.residual || (p.act != SHP_ACT_NONE && p.act != SHP_ACT_RELU)) return false;
    if (p.N % 64 || p.M % 32 || p.M < 16384) return false;
    const int64_t lim = (int64_t)1 << 31;
    return (int64_t)p.cn * p.cih * p.ciw * p.cic * 4 < lim && (int64_t)p.M * p.scm * 4 < lim;
}

int launch_stem(hipStream_t s, const GemmParams& p) {
    const int nslab = p.N / 64;
    const int nrange = std::max(8, device_cus() / nslab / 8 * 8);
    const dim3 grid((unsigned)(nrange * nslab));
    if (p.act == SHP_ACT_RELU)
        hipLaunchKernelGGL((conv_stem_kernel<7, 7, 3, 1>), grid, dim3(512), 0, s, p, nslab, nrange);
    else
        hipLaunchKernelGGL((conv_stem_kernel<7, 7, 3, 0>), grid, dim3(512), 0, s, p, nslab, nrange);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

struct Plan {
    TileCfg t;
    int splits, kps;
};

// Workgroups resident per CU, as the compiler reports them for each variant (LDS of the
// double-buffered tiles out of 160 KiB per CU, and the VGPR+AGPR budget).
int occupancy(TileCfg t) {
    if (t.bl) {
        if (t.bm == 128) return 2;
        return t.bk == 64 ? 2 : t.bk == 16 ? 7 : 4;
    }
    if (t.dma) return t.bn == 128 ? 2 : 3;
    if (t.bm == 128 && t.bn == 128) return t.bk == 16 ? 4 : 2;
    if (t.bm == 128) return t.bk == 16 ? 4 : 3;
    return t.bk == 16 ? 8 : 4;
}

// Relative MFMA efficiency of a tile shape and K tile (fitted to per-layer sweeps of the
// ResNet-50 convolutions on MI355X).  The 16-deep K tile costs ~15 % on long K loops; with
// at most 256 K per workgroup the work is dominated by operand latency and the epilogue,
// and the twice higher residency of the 16-deep tile wins (K = 64..256 layers measured
// 3-16 % faster with it).
double tile_eff(TileCfg t, int kps) {
    if (t.bl) return t.bk == 16 && kps > 256 ? 0.85 : 1.0;
    if (t.dma) return 1.1;
    double e = (t.bm == 128 && t.bn == 128) ? 1.0 : 0.85;
    return t.bk == 16 && kps > 256 ? e * 0.85 : e;
}

// Estimated time of a plan: the busiest CU's MFMA work at the utilisation its resident
// workgroup count allows (more resident waves hide more load latency), plus the split-K
// reduction pass.
double plan_cost(const GemmParams& p, int nbatch, TileCfg t, int splits, int kps) {
    static const double kUtil[8] = {0.4, 0.6, 0.75, 0.85, 0.9, 0.92, 0.95, 1.0};
    // the buffer-loaded kernel keeps its own MFMA stream fed: one workgroup per CU already
    // runs at ~80 % of the CU's rate (MI355X, 1568x512x4608 on 200 CUs)
    static const double kUtilBl[8] = {0.8, 0.9, 0.94, 0.96, 0.97, 0.98, 0.99, 1.0};
    const double cu_rate = 256.0 * 2.4e9;  // fp32 MFMA FLOP/s per CU
    int64_t tiles = (int64_t)((p.M + t.bm - 1) / t.bm) * ((p.N + t.bn - 1) / t.bn) * nbatch;
    int64_t wgs = tiles * splits;
    int64_t per_cu = (wgs + 255) / 256;
    int resident = (int)std::min<int64_t>(occupancy(t), per_cu);
    double util = (t.bl ? kUtilBl : kUtil)[std::min(resident, 8) - 1];
    double wg_flops = 2.0 * t.bm * t.bn * kps;
    double cost = per_cu * wg_flops / (cu_rate * tile_eff(t, kps) * util);
    if (splits > 1) cost += (splits + 1.0) * p.M * (double)p.N * nbatch * 4.0 / 3.0e12 + 2.0e-6;
    return cost;
}

// Plans measured best on MI355X for the benchmark configs' shapes: sweeps of every tile, K
// tile and split count of both kernels per shape, with split counts down to one K tile per
// split for the 1x1 convolutions of MobileNetV2 b1 and EfficientNet-Lite0 b8.  An entry only
// where the best plan beat the cost model's by more than 2.5 % alone and did not lose inside
// the model's forward pass; the cost model decides every other shape.  Key: operand modes,
// batch count, M, N, K, and for convolutions the input channels, stride and kernel height (0
// for products).
struct TunedPlan {
    int amode, bmode, nbatch, M, N, K, cic, csh, ckh;
    TileCfg t;
    int splits;
};
const TunedPlan kTuned[] = {
{shp::A_CONV_NHWC, shp::B_NVEC, 1, 401408, 64, 147, 3, 2, 7, {64, 64, 32, false, 1, false}, 1},  // resnet50_v1_5 conv1: 146.1 vs 156.1 us
    {shp::A_CONV_NHWC4, shp::B_NVEC, 1, 100352, 64, 576, 64, 1, 3, {64, 64, 16, false, 1, true}, 1},  // resnet50_v1_5 conv2_block1_2: 80.4 vs 87.6 us
    {shp::A_CONV_NHWC4, shp::B_NVEC, 1, 25088, 128, 1152, 128, 2, 3, {64, 64, 16, false, 1, true}, 2},  // resnet50_v1_5 conv3_block1_2: 83.2 vs 89.6 us
    {shp::A_CONV_NHWC4, shp::B_NVEC, 1, 25088, 128, 1152, 128, 1, 3, {64, 64, 16, false, 1, true}, 3},  // resnet50_v1_5 conv3_block2_2: 82.5 vs 93.4 us
    {shp::A_CONV_NHWC4, shp::B_NVEC, 1, 6272, 1024, 512, 512, 2, 1, {64, 64, 16, false, 1, true}, 1},  // resnet50_v1_5 conv4_block1_0: 64.8 vs 68.2 us
    {shp::A_CONV_NHWC4, shp::B_NVEC, 1, 25088, 256, 512, 512, 1, 1, {64, 64, 16, false, 1, true}, 1},  // resnet50_v1_5 conv4_block1_1: 64.5 vs 67.3 us
    {shp::A_CONV_NHWC4, shp::B_NVEC, 1, 6272, 256, 2304, 256, 2, 3, {64, 64, 16, false, 1, true}, 3},  // resnet50_v1_5 conv4_block1_2: 82.4 vs 85.1 us
    {shp::A_CONV_NHWC4, shp::B_NVEC, 1, 6272, 256, 2304, 256, 1, 3, {64, 64, 16, false, 1, true}, 3},  // resnet50_v1_5 conv4_block2_2: 82.1 vs 85.5 us
    {shp::A_CONV_NHWC4, shp::B_NVEC, 1, 1568, 2048, 1024, 1024, 2, 1, {64, 64, 32, false, 1, true}, 1},  // resnet50_v1_5 conv5_block1_0: 69.2 vs 71.2 us
    {shp::A_KVEC, shp::B_KVEC, 96, 128, 128, 64, 0, 0, 0, {64, 64, 16, false, 1, true}, 1},  // bert_base layer0_scores: 9.4 vs 9.9 us
    {shp::A_KVEC, shp::B_NVEC, 96, 128, 64, 128, 0, 0, 0, {64, 64, 16, false, 1, true}, 1},  // bert_base layer0_context: 8.7 vs 9.1 us
    {shp::A_CONV_NHWC, shp::B_STRIDED, 1, 100352, 32, 27, 3, 2, 3, {64, 64, 32, false, 1, false}, 1},  // efficientnet_lite0 stem: 21.4 vs 22.2 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 100352, 96, 16, 16, 1, 1, {64, 64, 16, false, 1, true}, 1},  // efficientnet_lite0 block1_expand: 19.2 vs 19.7 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 6272, 240, 40, 40, 1, 1, {64, 64, 16, false, 1, false}, 1},  // efficientnet_lite0 block4_expand: 10.6 vs 11.5 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 1568, 80, 480, 480, 1, 1, {64, 64, 16, false, 1, true}, 5},  // efficientnet_lite0 block6_project: 12.2 vs 15.3 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 1568, 112, 480, 480, 1, 1, {64, 64, 16, false, 1, true}, 5},  // efficientnet_lite0 block8_project: 12.8 vs 15.0 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 1568, 672, 112, 112, 1, 1, {64, 64, 16, false, 1, true}, 1},  // efficientnet_lite0 block9_expand: 11.2 vs 11.5 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 392, 1152, 192, 192, 1, 1, {64, 64, 32, false, 1, true}, 1},  // efficientnet_lite0 block12_expand: 10.5 vs 11.1 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 392, 192, 1152, 1152, 1, 1, {64, 64, 16, false, 1, true}, 6},  // efficientnet_lite0 block12_project: 13.6 vs 13.9 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 392, 320, 1152, 1152, 1, 1, {64, 64, 16, false, 1, true}, 6},  // efficientnet_lite0 block15_project: 14.2 vs 14.8 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 392, 1280, 320, 320, 1, 1, {64, 64, 32, false, 1, true}, 1},  // efficientnet_lite0 head_conv: 12.9 vs 13.3 us
    {shp::A_CONV_NHWC, shp::B_STRIDED, 1, 12544, 32, 27, 3, 2, 3, {64, 64, 32, false, 1, false}, 1},  // mobilenet_v2 stem: 8.6 vs 8.8 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 12544, 16, 32, 32, 1, 1, {64, 64, 16, false, 1, true}, 1},  // mobilenet_v2 block0_project: 7.3 vs 7.5 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 3136, 24, 96, 96, 1, 1, {64, 64, 16, false, 1, true}, 1},  // mobilenet_v2 block1_project: 8.4 vs 8.7 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 196, 64, 192, 192, 1, 1, {64, 64, 16, false, 1, true}, 1},  // mobilenet_v2 block6_project: 10.0 vs 10.7 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 196, 384, 64, 64, 1, 1, {64, 64, 16, false, 1, true}, 1},  // mobilenet_v2 block7_expand: 7.8 vs 8.4 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 196, 64, 384, 384, 1, 1, {64, 64, 32, false, 1, true}, 6},  // mobilenet_v2 block7_project: 11.0 vs 13.6 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 196, 96, 384, 384, 1, 1, {64, 64, 16, false, 1, true}, 6},  // mobilenet_v2 block10_project: 10.6 vs 13.4 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 196, 576, 96, 96, 1, 1, {64, 64, 16, false, 1, true}, 1},  // mobilenet_v2 block11_expand: 8.5 vs 9.0 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 196, 96, 576, 576, 1, 1, {64, 64, 32, false, 1, true}, 5},  // mobilenet_v2 block11_project: 11.7 vs 12.3 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 49, 160, 576, 576, 1, 1, {64, 64, 16, false, 1, true}, 5},  // mobilenet_v2 block13_project: 11.7 vs 12.2 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 49, 960, 160, 160, 1, 1, {64, 64, 16, false, 1, true}, 1},  // mobilenet_v2 block14_expand: 9.5 vs 9.9 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 49, 160, 960, 960, 1, 1, {64, 64, 16, false, 1, true}, 8},  // mobilenet_v2 block14_project: 12.4 vs 14.1 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 49, 320, 960, 960, 1, 1, {64, 64, 16, false, 1, true}, 6},  // mobilenet_v2 block16_project: 12.4 vs 13.0 us
    {shp::A_CONV_NHWC4, shp::B_KVEC, 1, 49, 1280, 320, 320, 1, 1, {64, 64, 16, false, 1, true}, 5},  // mobilenet_v2 head_conv: 10.8 vs 12.3 us
};

// The table's plan for this problem, if it has one that the problem's operands allow.
bool tuned_plan(const GemmParams& p, int nbatch, int amode, int bmode, bool hot, int blm,
                Plan* out) {
    for (const TunedPlan& e : kTuned) {
        if (e.amode != amode || e.bmode != bmode || e.nbatch != nbatch || e.M != p.M ||
            e.N != p.N || e.K != p.K)
            continue;
        if (e.cic && (e.cic != p.cic || e.csh != p.csh || e.ckh != p.ckh)) continue;
        const TileCfg& t = e.t;
        if (t.bl && !(blm & (t.bk == 16 ? 1 : t.bk == 32 ? 2 : 4))) return false;
        if (!t.bl && !hot && (t.bk != 32 || t.pg > 1)) return false;
        const int kq = t.bl && t.bk == 64 ? 64 : 32;
        int kps = ((p.K + e.splits - 1) / e.splits + kq - 1) / kq * kq;
        if ((p.K + kps - 1) / kps != e.splits) return false;
        *out = Plan{t, e.splits, kps};
        return true;
    }
    return false;
}

const int kSplits[] = {1, 2, 3, 4, 5, 6, 8, 12, 16};

// The buffer-loaded kernel's plan: tile, K tile and split count by the cost model, among the
// K tiles of `blm` (bl_mask) and the tune overrides.  False when no candidate fits.
bool plan_bl(const GemmParams& p, int nbatch, int blm, const shp::GemmTune& tn, Plan* out) {
    static const TileCfg kBl[] = {{128, 128, 32, false, 1, true}, {128, 64, 32, false, 1, true},
                                  {64, 64, 64, false, 1, true},   {64, 64, 32, false, 1, true},
                                  {64, 64, 16, false, 1, true}};
    Plan best{kBl[3], 1, 0};
    double best_cost = 1e30;
    for (const TileCfg& t : kBl) {
        const int bit = t.bk == 16 ? 1 : t.bk == 32 ? 2 : 4;
        if (!(blm & bit)) continue;
        const int ti = t.bm == 128 ? (t.bn == 128 ? 1 : 2) : 3;
        if (tn.tile && tn.tile != ti) continue;
        if (tn.bk && tn.bk != t.bk) continue;
        const int kq = t.bk == 64 ? 64 : 32;
        for (int s : kSplits) {
            if (tn.splits && tn.splits != s) continue;
            int kps = ((p.K + s - 1) / s + kq - 1) / kq * kq;
            int real = (p.K + kps - 1) / kps;
            // the model keeps 128 K per split; a forced split count may go down to one K tile
            if (s > 1 && (real != s || kps < (tn.splits ? kq : 128))) continue;
            double c = plan_cost(p, nbatch, t, s, kps);
            if (c < best_cost * 0.97) {
                best_cost = c;
                best = Plan{t, s, kps};
            }
        }
    }
    if (best.kps <= 0) return false;
    *out = best;
    return true;
}

// `blm`: the K tiles for which the buffer-loaded kernel takes the problem (0: none).  It is
// used wherever it applies unless the tune says otherwise (bl -1, or a dma / pg override).
Plan plan_gemm(const GemmParams& p, int nbatch, bool hot, bool dma_ok, bool conv_a,
               const shp::GemmTune& tn, int amode, int bmode, int blm) {
    static const int kTiles[5][2] = {{128, 128}, {128, 64}, {64, 64}, {128, 128}, {128, 64}};
    Plan tuned;
    if (tn.table >= 0 && !tn.tile && !tn.bk && !tn.splits && !tn.dma && !tn.pg && !tn.bl &&
        tuned_plan(p, nbatch, amode, bmode, hot, blm, &tuned))
        return tuned;
    if (blm && tn.bl >= 0 && (tn.bl > 0 || (tn.dma <= 0 && !tn.pg)) &&
        plan_bl(p, nbatch, blm, tn, &tuned))
        return tuned;
    if (dma_ok && conv_a && tn.dma == 0 && !tn.splits && dma_preferred(p, nbatch))
        return Plan{{128, 64, 16, true}, 1, ((p.K + 31) / 32) * 32};
    Plan best{{128, 128, 32, false}, 1, 0};
    double best_cost = 1e30;
    for (int ti = 0; ti < 5; ++ti) {
        const bool dma = ti >= 3;
        if (dma && (!dma_ok || tn.dma <= 0 || tn.dma != ti - 2)) continue;
        if (!dma && dma_ok && tn.dma > 0) continue;
        if (!dma && tn.tile && tn.tile != ti + 1) continue;
        for (int bk : {32, 16}) {
            if (dma && bk != 16) continue;
            if (!dma && bk == 16 && !hot) continue;
            if (!dma && tn.bk && tn.bk != bk) continue;
            TileCfg t{kTiles[ti][0], kTiles[ti][1], bk, dma};
            for (int s : kSplits) {
                if (tn.splits && tn.splits != s) continue;
                int kps = (p.K + s - 1) / s;
                kps = ((kps + 31) / 32) * 32;  // a multiple of both K tiles
                if (kps <= 0) kps = 32;
                int real = (p.K + kps - 1) / kps;
                if (s > 1 && (real != s || kps < 128)) continue;
                double c = plan_cost(p, nbatch, t, s, kps);
                if (c < best_cost * 0.97) {  // prefer the earlier (simpler) plan on near ties
                    best_cost = c;
                    best = Plan{t, s, kps};
                }
            }
        }
    }
    if (best.kps <= 0) best.kps = ((p.K + 31) / 32) * 32;
    if (best.kps <= 0) best.kps = 32;
    return best;
}

// operand modes of a product with the given strides (defined with the launchers below)
int dot_modes(const GemmParams& p, int& am, int& bm);

}  // namespace

namespace shp {

size_t gemm_workspace_bytes(const GemmParams& p, int amode, int bmode, int cmode,
                            const GemmTune* tune) {
    static const GemmTune kAuto;
    int nbatch = p.batch_outer * p.batch_inner;
    const bool hot = combo_is_hot(amode, bmode, cmode);
    const bool dma_ok = dma_eligible(p, amode, bmode, cmode);
    const int blm = bl_mask(p, amode, bmode, cmode);
    // the larger of the plans with and without the buffer-loaded kernel: its eligibility can
    // depend on pointer alignment the caller of this function may not know yet
    int splits = 1;
    for (int b : {blm, 0}) {
        Plan pl = plan_gemm(p, nbatch, hot, dma_ok, amode == A_CONV_NHWC4, tune ? *tune : kAuto,
                            amode, bmode, b);
        splits = std::max(splits, pl.splits);
    }
    if (splits <= 1) return 0;
    return kSplitCounterBytes + (size_t)splits * nbatch * p.M * p.N * sizeof(float);
}

size_t gemm_workspace_for_kernel(const char* name, const int32_t* q, size_t n,
                                 const GemmTune* tune) {
    GemmParams p;
    memset(&p, 0, sizeof(p));
    p.batch_outer = p.batch_inner = 1;
    std::string k = name ? name : "";
    if (k == "inverted_residual_nhwc") return block_workspace_for_kernel(q, n, tune);
    // operand modes as the launchers pick them for 16-byte aligned bindings (the bindings of
    // a launch are not known here), so the planned split count is the one the launch uses
    int am = A_KVEC, bm = B_NVEC;
    if (k == "hlo_conv_nhwc_hwio" && n >= 14) {
        p.M = q[0] * q[7] * q[8]; p.N = q[6]; p.K = q[4] * q[5] * q[3];
        p.cn = q[0]; p.cih = q[1]; p.ciw = q[2]; p.cic = q[3]; p.ckh = q[4]; p.ckw = q[5];
        p.csh = q[9]; p.csw = q[10];
        p.sbk = p.N; p.sbn = 1;
        am = p.cic % 4 == 0 ? A_CONV_NHWC4 : A_CONV_NHWC;
        bm = p.N % 4 == 0 ? B_NVEC : B_STRIDED;
    } else if ((k == "conv2d" || k == "conv2d_nhwc") && n >= 15) {
        p.M = q[0] * q[5] * q[6]; p.N = q[4]; p.K = q[1] * q[7] * q[8];
        p.cn = q[0]; p.cic = q[1]; p.cih = q[2]; p.ciw = q[3]; p.ckh = q[7]; p.ckw = q[8];
        p.csh = q[9]; p.csw = q[10];
        p.sbk = 1; p.sbn = p.K;
        am = k == "conv2d" ? A_CONV_NCHW : p.cic % 4 == 0 ? A_CONV_NHWC4 : A_CONV_NHWC;
        bm = p.K % 4 == 0 ? B_KVEC : B_STRIDED;
    } else if (k == "fully_connected" && n >= 4) {
        if (q[0] <= 8) return 0;
        p.M = q[0]; p.N = q[2]; p.K = q[1];
        p.sam = p.K; p.sak = 1; p.sbk = 1; p.sbn = p.K;
        am = p.K % 4 == 0 ? A_KVEC : A_STRIDED;
        bm = p.K % 4 == 0 ? B_KVEC : B_STRIDED;
    } else if (k == "hlo_dot_batched" && n >= 5) {
        p.batch_outer = q[0]; p.M = q[1]; p.K = q[2]; p.N = q[3];
        p.sa_outer = (int64_t)p.M * p.K; p.sam = p.K; p.sak = 1;
        p.sb_outer = (int64_t)p.K * p.N; p.sbk = p.N; p.sbn = 1;
        dot_modes(p, am, bm);
    } else if (k == "hlo_dot_rank2" && n >= 4) {
        p.M = q[0]; p.K = q[1]; p.N = q[2];
        p.sam = p.K; p.sak = 1; p.sbk = p.N; p.sbn = 1;
        dot_modes(p, am, bm);
    } else if (k == "dot_general_strided" && n >= 17) {
        p.batch_outer = q[0]; p.batch_inner = q[1]; p.M = q[2]; p.N = q[3]; p.K = q[4];
        p.sa_outer = q[5]; p.sa_inner = q[6]; p.sam = q[7]; p.sak = q[8];
        p.sb_outer = q[9]; p.sb_inner = q[10]; p.sbk = q[11]; p.sbn = q[12];
        dot_modes(p, am, bm);
    } else {
        return 0;
    }
    if (p.M <= 0 || p.N <= 0 || p.K <= 0) return 0;
    size_t small_ws = 0;  // the K-split small-product path of a 1x1 conv2d_nhwc
    if (k == "conv2d_nhwc" && q[7] == 1 && q[8] == 1 && q[9] == 1 && q[10] == 1 &&
        q[12] == 0 && q[13] == 0 && q[5] == q[2] && q[6] == q[3])
        small_ws = small_gemm_workspace(p.M, p.N,
                                        small_gemm_splits(p.M, p.N, p.K, tune ? tune->small : 0));
    const int cm = k == "conv2d" ? C_NCHW : C_STRIDED;
    // and the generic plan too, so a launch whose bindings turn out unaligned finds its partials
    return std::max({gemm_workspace_bytes(p, am, bm, cm, tune),
                     gemm_workspace_bytes(p, A_STRIDED, B_STRIDED, C_STRIDED, tune), small_ws});
}

// Band height of the tile order (GemmParams::group_m, see wg_coords).  For each candidate
// height g it counts, per XCD, the distinct tile rows (A panels, BM x K-range each) and tile
// columns (B panels, K-range x BN) its run of the split-major order touches, and keeps the g
// with the fewest panel bytes summed over the 8 XCDs (row major, g = 1, on ties).  Tile
// results do not depend on the order, only which L2 serves the panels.
int64_t xcd_panel_cost(int tiles_m, int tiles_n, int splits, int g, int bm, int bn) {
    const int64_t ntiles = (int64_t)tiles_m * tiles_n, total = ntiles * splits;
    const int64_t run = total / 8;
    if (run == 0) return 0;
    int64_t cost = 0;
    for (int x = 0; x < 8; ++x) {
        int64_t a = x * run;
        const int64_t end = a + run;
        while (a < end) {  // one split's part of the run: [a, b)
            const int64_t split_end = (a / ntiles + 1) * ntiles;
            const int64_t b = std::min(end, split_end);
            const int64_t t0 = a % ntiles, t1 = t0 + (b - a);  // [t0, t1) within the split
            int64_t rows = 0, col_lo = tiles_n, col_hi = -1;
            for (int64_t t = t0; t < t1;) {  // band by band
                const int64_t band = t / ((int64_t)g * tiles_n);
                const int64_t h = std::min<int64_t>(g, tiles_m - band * g);
                const int64_t bs = band * g * tiles_n, be = bs + h * tiles_n;
                const int64_t u = t - bs, v = std::min(t1, be) - bs;  // [u, v) in the band
                rows += (v - u) >= h ? h : (v - u);
                col_lo = std::min(col_lo, u / h);
                col_hi = std::max(col_hi, (v - 1) / h);
                t = bs + v;
            }
            cost += rows * bm + (col_hi - col_lo + 1) * bn;
            a = b;
        }
    }
    return cost;
}

int tile_group(const GemmParams& p, const TileCfg& t, int64_t ntiles, int forced) {
    const int tiles_m = (p.M + t.bm - 1) / t.bm;
    const int tiles_n = (p.N + t.bn - 1) / t.bn;
    if (forced < 0) return 1;
    if (forced > 0) return std::min(forced, tiles_m);
    if ((ntiles * p.splits) / 8 < 2) return 1;
    int best = 1;
    int64_t best_cost = xcd_panel_cost(tiles_m, tiles_n, p.splits, 1, t.bm, t.bn);
    for (int g = 2; g <= tiles_m && g <= 64; g = g < 8 ? g + 1 : g * 2) {
        const int64_t c = xcd_panel_cost(tiles_m, tiles_n, p.splits, g, t.bm, t.bn);
        if (c < best_cost) {
            best_cost = c;
            best = g;
        }
    }
    return best;
}

int gemm_launch(hipStream_t stream, GemmParams p, int amode, int bmode, int cmode,
                float* workspace, size_t workspace_bytes, const GemmTune* tune) {
    static const GemmTune kAuto;
    const GemmTune& tn = tune ? *tune : kAuto;
    if (p.M <= 0 || p.N <= 0 || p.K < 0)
        return fail(SHP_ERR_SHAPE, "gemm: M, N must be > 0 and K >= 0");
    int nbatch = p.batch_outer * p.batch_inner;
    if (nbatch <= 0 || nbatch > 65535) return fail(SHP_ERR_SHAPE, "gemm: batch out of range");
    if (amode == A_CONV_NHWC4 && p.cic % 4 != 0) amode = A_CONV_NHWC;
    const bool hot = combo_is_hot(amode, bmode, cmode);
    const bool dma_ok = dma_eligible(p, amode, bmode, cmode);
    // in-kernel split-K fixup where the epilogue's 16-byte path holds for every batch of C
    auto a16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
    const bool fix_ok = cmode == C_STRIDED && p.scn == 1 && (p.scm & 3) == 0 && (p.N & 3) == 0 &&
                        (p.sc_outer & 3) == 0 && (p.sc_inner & 3) == 0 && a16(p.c) &&
                        (!p.bias || a16(p.bias)) && (!p.residual || a16(p.residual));
    if (tn.stem >= 0 && stem_eligible(p, amode, bmode, cmode, nbatch)) return launch_stem(stream, p);
    if (tn.sk >= 0) {
        const int v = smallk_variant(p, amode, bmode, cmode, nbatch);
        if (v) return launch_smallk(stream, p, amode, v);
    }
    const int blm = bl_mask(p, amode, bmode, cmode);
    Plan pl = plan_gemm(p, nbatch, hot, dma_ok, amode == A_CONV_NHWC4, tn, amode, bmode, blm);
    size_t need = pl.splits > 1
                      ? kSplitCounterBytes + (size_t)pl.splits * nbatch * p.M * p.N * sizeof(float)
                      : 0;
    if (pl.splits > 1 && (workspace == nullptr || workspace_bytes < need)) {
        pl.splits = 1;
        pl.kps = ((p.K + 31) / 32) * 32;
        if (pl.kps <= 0) pl.kps = 32;
    }
    p.splits = pl.splits;
    p.k_per_split = pl.kps;
    p.partial = pl.splits > 1 ? workspace + kSplitCounterBytes / sizeof(float) : nullptr;
    p.counters = pl.splits > 1 ? reinterpret_cast<int*>(workspace) : nullptr;
    TileCfg t = pl.t;
    // Two-deep prefetch for the split-K 64x64 / K-tile 32 plans of NHWC convolutions: 4-7 %
    // faster on the ResNet-50 K = 1024..2304 layers (MI355X sweeps), ~2 % slower on some
    // short single-split loops, and 3x slower on the M = 32 row-major FC (one tile row).
    if (!t.dma && !t.bl && t.bm == 64 && t.bn == 64 && t.bk == 32 && pl.splits > 1 &&
        amode == A_CONV_NHWC4 && combo_is_hot(amode, bmode, cmode))
        t.pg = 2;
    if (tn.pg && !t.bl) t.pg = tn.pg;
    int64_t ntiles = (int64_t)((p.M + t.bm - 1) / t.bm) * ((p.N + t.bn - 1) / t.bn);
    if (ntiles * p.splits > 0x7fffffff) return fail(SHP_ERR_SHAPE, "gemm: too many tiles");
    // in-kernel split-K fixup where the tile counters fit and few splits share a tile (the last
    // split sums them serially: with 16 splits of the M = 32 ResNet FC it is 2.5x slower than
    // the separate reduction pass); the separate pass otherwise
    p.fixup = pl.splits > 1 && pl.splits <= 4 && fix_ok &&
              ntiles * nbatch <= (int64_t)(kSplitCounterBytes / sizeof(int));
    p.group_m = tile_group(p, t, ntiles, tn.group);
    dim3 grid((unsigned)ntiles, (unsigned)p.splits, (unsigned)nbatch);
    int rc = t.bl    ? dispatch_bl(stream, p, amode, bmode, t, grid)
             : t.dma ? launch_dma(stream, p, amode, t.bn, grid)
                     : dispatch_combo(stream, p, amode, bmode, cmode, t, grid);
    if (rc) return rc;
    SHP_HIP_CHECK(hipGetLastError());
    if (p.splits > 1 && !p.fixup) {
        int64_t total = (int64_t)p.M * p.N * nbatch;
        unsigned g = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
        if (cmode == C_NCHW)
            hipLaunchKernelGGL((splitk_reduce_kernel<C_NCHW>), dim3(g), dim3(256), 0, stream, p,
                               nbatch);
        else
            hipLaunchKernelGGL((splitk_reduce_kernel<C_STRIDED>), dim3(g), dim3(256), 0, stream,
                               p, nbatch);
        SHP_HIP_CHECK(hipGetLastError());
    }
    return SHP_OK;
}

}  // namespace shp

namespace {

using shp::fail;

inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

GemmParams base_params() {
    GemmParams p;
    memset(&p, 0, sizeof(p));
    p.batch_outer = p.batch_inner = 1;
    p.coh = p.cow = 1;
    p.splits = 1;
    return p;
}

// hlo_conv_nhwc_hwio: push {n, ih, iw, ic, kh, kw, oc, oh, ow, sh, sw, pt, pl, total}
int launch_hlo_conv(const shp::Launch& l) {
    if (l.n_push < 14) return fail(SHP_ERR_PUSH, "hlo_conv_nhwc_hwio needs 14 push constants");
    const int32_t* q = l.push;
    for (int i = 0; i < 11; ++i)
        if (q[i] <= 0) return fail(SHP_ERR_SHAPE, "hlo_conv_nhwc_hwio: non-positive dim/stride");
    int rc = shp::check_total(l, (int64_t)q[0] * q[7] * q[8] * q[6], "hlo_conv_nhwc_hwio");
    if (rc) return rc;
    if (q[13] != (int64_t)q[0] * q[7] * q[8] * q[6])
        return fail(SHP_ERR_SHAPE, "hlo_conv_nhwc_hwio: total != n*oh*ow*oc");
    GemmParams p = base_params();
    p.cn = q[0]; p.cih = q[1]; p.ciw = q[2]; p.cic = q[3]; p.ckh = q[4]; p.ckw = q[5];
    p.coh = q[7]; p.cow = q[8]; p.csh = q[9]; p.csw = q[10]; p.cpt = q[11]; p.cpl = q[12];
    p.M = q[0] * q[7] * q[8];
    p.N = q[6];
    p.K = q[4] * q[5] * q[3];
    p.a = (const float*)l.in0;
    p.b = (const float*)l.in1;
    p.sbk = p.N;
    p.sbn = 1;
    p.c = (float*)l.out;
    p.scm = p.N;
    p.scn = 1;
    p.bias = l.epi->bias;
    p.residual = l.epi->residual;
    p.act = l.epi->act;
    p.alpha = l.epi->alpha;
    int am = (p.cic % 4 == 0 && al16(p.a)) ? shp::A_CONV_NHWC4 : shp::A_CONV_NHWC;
    int bm = (p.N % 4 == 0 && al16(p.b)) ? shp::B_NVEC : shp::B_STRIDED;
    return shp::gemm_launch(l.stream, p, am, bm, shp::C_STRIDED, l.workspace, l.workspace_bytes,
                            l.tune);
}

// conv2d (NCHW, weights OIHW followed by the bias tail):
// push {n, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, same, pt, pl, total}
int conv2d_common(const shp::Launch& l, bool nhwc) {
    if (l.n_push < 15) return fail(SHP_ERR_PUSH, "conv2d needs 15 push constants");
    const int32_t* q = l.push;
    for (int i = 0; i < 11; ++i)
        if (q[i] <= 0) return fail(SHP_ERR_SHAPE, "conv2d: non-positive dim/stride");
    int64_t total = (int64_t)q[0] * q[4] * q[5] * q[6];
    int rc = shp::check_total(l, total, "conv2d");
    if (rc) return rc;
    if (q[14] != total) return fail(SHP_ERR_SHAPE, "conv2d: total != n*oc*oh*ow");
    GemmParams p = base_params();
    p.cn = q[0]; p.cic = q[1]; p.cih = q[2]; p.ciw = q[3];
    p.coh = q[5]; p.cow = q[6]; p.ckh = q[7]; p.ckw = q[8];
    p.csh = q[9]; p.csw = q[10]; p.cpt = q[12]; p.cpl = q[13];
    p.M = q[0] * q[5] * q[6];
    p.N = q[4];
    p.K = q[1] * q[7] * q[8];
    p.a = (const float*)l.in0;
    p.b = (const float*)l.in1;
    p.sbk = 1;
    p.sbn = p.K;
    p.c = (float*)l.out;
    p.scm = p.N;
    p.scn = 1;
    p.bias = p.b + (int64_t)p.N * p.K;  // packed bias tail (scheduler.rs:1327-1362)
    p.residual = l.epi->residual;
    p.act = l.epi->act;
    p.alpha = l.epi->alpha;
    if (nhwc && q[1] <= 4 && !(l.tune && l.tune->conv_direct < 0)) {
        rc = shp::conv_nhwc_direct(l);
        if (rc != SHP_ERR_UNSUPPORTED) return rc;
    }
    // 1x1 stride-1 unpadded NHWC convolutions are plain [M][K] x [N][K]^T products: the
    // small-product kernel where the 64x64 tiles would not fill the GPU (K-split past 256)
    const int small = l.tune ? l.tune->small : 0;
    const int ssp = nhwc && q[7] == 1 && q[8] == 1 && q[9] == 1 && q[10] == 1 && q[12] == 0 &&
                            q[13] == 0 && q[5] == q[2] && q[6] == q[3] && al16(p.a) && al16(p.b)
                        ? small_gemm_splits(p.M, p.N, p.K, small)
                        : 0;
    if (ssp == 1 || (ssp > 1 && l.workspace &&
                     l.workspace_bytes >= small_gemm_workspace(p.M, p.N, ssp))) {
        const int tiles_n = (p.N + 31) / 32;
        const int64_t grid = (int64_t)((p.M + 31) / 32) * tiles_n;
        const int cps = ((p.K + 15) / 16 + ssp - 1) / ssp;
        auto kern = cps <= 2 ? small_gemm_kernel<2>
                  : cps <= 4 ? small_gemm_kernel<4>
                  : cps <= 8 ? small_gemm_kernel<8>
                  : cps <= 12 ? small_gemm_kernel<12> : small_gemm_kernel<kSmallKc>;
        float* part = ssp > 1 ? l.workspace + shp::kSplitCounterBytes / sizeof(float) : nullptr;
        int* counters = ssp > 1 ? reinterpret_cast<int*>(l.workspace) : nullptr;
        hipLaunchKernelGGL(kern, dim3((unsigned)grid, (unsigned)ssp), dim3(256), 0, l.stream,
                           p.a, p.b, p.c, p.M, p.N, p.K, tiles_n, p.bias, p.residual, p.act,
                           p.alpha, part, counters);
        SHP_HIP_CHECK(hipGetLastError());
        return SHP_OK;
    }
    int bm = (p.K % 4 == 0 && al16(p.b)) ? shp::B_KVEC : shp::B_STRIDED;
    if (nhwc) {
        int am = (p.cic % 4 == 0 && al16(p.a)) ? shp::A_CONV_NHWC4 : shp::A_CONV_NHWC;
        return shp::gemm_launch(l.stream, p, am, bm, shp::C_STRIDED, l.workspace,
                                l.workspace_bytes, l.tune);
    }
    return shp::gemm_launch(l.stream, p, shp::A_CONV_NCHW, bm, shp::C_NCHW, l.workspace,
                            l.workspace_bytes, l.tune);
}

int launch_conv2d(const shp::Launch& l) { return conv2d_common(l, false); }
// conv2d_nhwc (native): the TFLite Conv2D on NHWC activations with the model's own OHWI
// weights + bias tail — no NCHW relabelling (scheduler.rs:58-62) and no OIHW repack.
int launch_conv2d_nhwc(const shp::Launch& l) { return conv2d_common(l, true); }

// fully_connected: push {batches, input_size, output_size, total}; weights [out][in] + bias
int launch_fully_connected(const shp::Launch& l) {
    if (l.n_push < 4) return fail(SHP_ERR_PUSH, "fully_connected needs 4 push constants");
    const int32_t* q = l.push;
    if (q[0] <= 0 || q[1] <= 0 || q[2] <= 0) return fail(SHP_ERR_SHAPE, "fully_connected: dims");
    int rc = shp::check_total(l, (int64_t)q[0] * q[2], "fully_connected");
    if (rc) return rc;
    if (q[3] != (int64_t)q[0] * q[2]) return fail(SHP_ERR_SHAPE, "fully_connected: total");
    int M = q[0], K = q[1], N = q[2];
    const float* w = (const float*)l.in1;
    const float* bias = w + (int64_t)N * K;
    const int fcm = l.tune ? l.tune->fc : 0;
    if (fcm >= 0 && M >= 2 && M <= 16 && K % 4 == 0 && K <= 16 * kFcWaves * 8 && al16(l.in0) &&
        al16(w) && (int64_t)(N + 16) * K * 4 < (1ll << 31)) {
        const int cpw = ((K + 15) / 16 + kFcWaves - 1) / kFcWaves;
        auto kern = cpw <= 1 ? fc_mfma_kernel<1>
                  : cpw <= 2 ? fc_mfma_kernel<2>
                  : cpw <= 4 ? fc_mfma_kernel<4>
                  : cpw <= 5 ? fc_mfma_kernel<5> : fc_mfma_kernel<8>;
        hipLaunchKernelGGL(kern, dim3((unsigned)((N + 15) / 16)), dim3(kFcWaves * 64), 0,
                           l.stream, (const float*)l.in0, w, (float*)l.out, M, N, K, bias,
                           l.epi->residual, l.epi->act, l.epi->alpha);
        SHP_HIP_CHECK(hipGetLastError());
        return SHP_OK;
    }
    if (M <= 8 && !l.epi->residual) {
        unsigned g = (unsigned)((N + 3) / 4);
        if (M <= 1)
            hipLaunchKernelGGL((skinny_nt_kernel<1>), dim3(g), dim3(256), 0, l.stream,
                               (const float*)l.in0, w, (float*)l.out, M, N, K, bias,
                               l.epi->act, l.epi->alpha);
        else if (K % 4 == 0 && al16(l.in0) && al16(w) && (int64_t)M * K * 4 <= 65536)
            hipLaunchKernelGGL((skinny_nt_lds_kernel<8>), dim3((unsigned)((N + 7) / 8)),
                               dim3(256), (size_t)M * K * 4, l.stream, (const float*)l.in0, w,
                               (float*)l.out, M, N, K, bias, l.epi->act, l.epi->alpha);
        else
            hipLaunchKernelGGL((skinny_nt_kernel<8>), dim3(g), dim3(256), 0, l.stream,
                               (const float*)l.in0, w, (float*)l.out, M, N, K, bias,
                               l.epi->act, l.epi->alpha);
        SHP_HIP_CHECK(hipGetLastError());
        return SHP_OK;
    }
    GemmParams p = base_params();
    p.M = M; p.N = N; p.K = K;
    p.a = (const float*)l.in0; p.sam = K; p.sak = 1;
    p.b = w; p.sbk = 1; p.sbn = K;
    p.c = (float*)l.out; p.scm = N; p.scn = 1;
    p.bias = bias;
    p.residual = l.epi->residual;
    p.act = l.epi->act;
    p.alpha = l.epi->alpha;
    int am = (K % 4 == 0 && al16(p.a)) ? shp::A_KVEC : shp::A_STRIDED;
    int bm = (K % 4 == 0 && al16(p.b)) ? shp::B_KVEC : shp::B_STRIDED;
    return shp::gemm_launch(l.stream, p, am, bm, shp::C_STRIDED, l.workspace, l.workspace_bytes,
                            l.tune);
}

// Pick vector modes for a strided batched product when the layout allows them.
int dot_modes(const GemmParams& p, int& am, int& bm) {
    bool a4 = p.sak == 1 && p.K % 4 == 0 && p.sam % 4 == 0 && p.sa_outer % 4 == 0 &&
              p.sa_inner % 4 == 0 && al16(p.a);
    am = a4 ? shp::A_KVEC : shp::A_STRIDED;
    bool bn4 = p.sbn == 1 && p.N % 4 == 0 && p.sbk % 4 == 0 && p.sb_outer % 4 == 0 &&
               p.sb_inner % 4 == 0 && al16(p.b);
    bool bk4 = p.sbk == 1 && p.K % 4 == 0 && p.sbn % 4 == 0 && p.sb_outer % 4 == 0 &&
               p.sb_inner % 4 == 0 && al16(p.b);
    bm = bn4 ? shp::B_NVEC : bk4 ? shp::B_KVEC : shp::B_STRIDED;
    return SHP_OK;
}

void dot_epilogue(GemmParams& p, const shp::Launch& l) {
    p.bias = l.epi->bias;
    p.residual = l.epi->residual;
    p.act = l.epi->act;
    p.alpha = l.epi->alpha;
}

// hlo_dot_batched: push {batch, m, k, n, total}; lhs [B,M,K], rhs [B,K,N], out [B,M,N]
int launch_dot_batched(const shp::Launch& l) {
    if (l.n_push < 5) return fail(SHP_ERR_PUSH, "hlo_dot_batched needs 5 push constants");
    const int32_t* q = l.push;
    if (q[0] <= 0 || q[1] <= 0 || q[2] < 0 || q[3] <= 0)
        return fail(SHP_ERR_SHAPE, "hlo_dot_batched: dims");
    int64_t total = (int64_t)q[0] * q[1] * q[3];
    int rc = shp::check_total(l, total, "hlo_dot_batched");
    if (rc) return rc;
    if (q[4] != total) return fail(SHP_ERR_SHAPE, "hlo_dot_batched: total");
    GemmParams p = base_params();
    p.batch_outer = q[0];
    p.M = q[1]; p.K = q[2]; p.N = q[3];
    p.a = (const float*)l.in0; p.sa_outer = (int64_t)p.M * p.K; p.sam = p.K; p.sak = 1;
    p.b = (const float*)l.in1; p.sb_outer = (int64_t)p.K * p.N; p.sbk = p.N; p.sbn = 1;
    p.c = (float*)l.out; p.sc_outer = (int64_t)p.M * p.N; p.scm = p.N; p.scn = 1;
    dot_epilogue(p, l);
    int am, bm;
    dot_modes(p, am, bm);
    return shp::gemm_launch(l.stream, p, am, bm, shp::C_STRIDED, l.workspace, l.workspace_bytes,
                            l.tune);
}

// hlo_dot_rank2: push {m, k, n, total}
int launch_dot_rank2(const shp::Launch& l) {
    if (l.n_push < 4) return fail(SHP_ERR_PUSH, "hlo_dot_rank2 needs 4 push constants");
    const int32_t* q = l.push;
    if (q[0] <= 0 || q[1] < 0 || q[2] <= 0) return fail(SHP_ERR_SHAPE, "hlo_dot_rank2: dims");
    int64_t total = (int64_t)q[0] * q[2];
    int rc = shp::check_total(l, total, "hlo_dot_rank2");
    if (rc) return rc;
    if (q[3] != total) return fail(SHP_ERR_SHAPE, "hlo_dot_rank2: total");
    GemmParams p = base_params();
    p.M = q[0]; p.K = q[1]; p.N = q[2];
    p.a = (const float*)l.in0; p.sam = p.K; p.sak = 1;
    p.b = (const float*)l.in1; p.sbk = p.N; p.sbn = 1;
    p.c = (float*)l.out; p.scm = p.N; p.scn = 1;
    dot_epilogue(p, l);
    int am, bm;
    dot_modes(p, am, bm);
    return shp::gemm_launch(l.stream, p, am, bm, shp::C_STRIDED, l.workspace, l.workspace_bytes,
                            l.tune);
}

// dot_general_strided (native): any dot_general with one contracting dim, read in place.
// push {batch_outer, batch_inner, M, N, K, sa_outer, sa_inner, sam, sak, sb_outer,
//       sb_inner, sbk, sbn, sc_outer, sc_inner, scm, scn}  (element strides)
// ---- attention_fused (native): one encoder layer's attention in one launch, ctx[b, s, h, :] =
// softmax_t(Q[b, s, h, :] . K[b, t, h, :] * scale + mask[t]) . V[b, t, h, :], the math of the
// scores dot_general, the row softmax and the context dot_general it replaces
// (bert_base.stablehlo.txt:28-49).  Q, K and V are read in place from the fused QKV activation.
//
// Sequence 128, head dim 64.  A workgroup takes 64 queries of one (batch, head); its four
// wavefronts are 2 query halves x 2 key halves, each 32 queries x 64 keys:
// * K and V of the head are staged in LDS as [key][d] rows padded by 4 floats (coalesced 16-byte
//   copies); Q fragments come straight from memory;
// * scores by fp32 MFMA (k remap of gemm_bl_kernel: lanes 32-63 take d + 4 of each step), then
//   scale + mask, the row maximum over the wave's 64 keys by lane shuffles, the common maximum
//   of the two key halves through LDS, exp, and the row sums;
// * P goes through LDS into the MFMA operand layout and P.V is accumulated per key half; the
//   key-half-1 wave hands its partial output and sum to its partner, which adds, divides and
//   stores (two 128-byte row segments per store).
// The arithmetic differs from the three-op chain only in the order of the sums (the divide
// comes after P.V); the result agrees with it to fp32 rounding.
constexpr int kAttS = 128, kAttHD = 64, kAttQB = 2;  // query blocks of 64 per (batch, head)

__global__ __launch_bounds__(256) void attention_fused_kernel(const float* __restrict__ qkv,
                                                              const float* __restrict__ mask,
                                                              float* __restrict__ out, int H,
                                                              int ld_in, int q_off, int k_off,
                                                              int v_off, int ld_out, float scale) {
    constexpr int S = kAttS, HD = kAttHD, KST = HD + 4, PST = 64 + 4;
    __shared__ __attribute__((aligned(16))) float Ks[S * KST];       // [key][d]
    __shared__ __attribute__((aligned(16))) float Vs[S * KST];       // [key][d]
    __shared__ __attribute__((aligned(16))) float Ps[4][32 * PST];   // per wave: P, then O
    __shared__ float red[4][2][32];                                  // per wave: row max, sum
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, lh = lane >> 5;
    const int wq = wave >> 1, wk = wave & 1;
    const int bh = blockIdx.x / kAttQB, qb = blockIdx.x % kAttQB;
    const int b = bh / H, h = bh % H;
    const float* __restrict__ base = qkv + (int64_t)b * S * ld_in + h * HD;

    for (int i = tid; i < S * HD / 4; i += 256) {
        const int key = i >> 4, d4 = (i & 15) * 4;
        const float* row = base + (int64_t)key * ld_in;
        *reinterpret_cast<float4*>(&Ks[key * KST + d4]) = *reinterpret_cast<const float4*>(row + k_off + d4);
        *reinterpret_cast<float4*>(&Vs[key * KST + d4]) = *reinterpret_cast<const float4*>(row + v_off + d4);
    }
    const int q0 = qb * 64 + wq * 32;  // this wave's first query
    f4v qa[HD / 8];
#pragma unroll
    for (int s = 0; s < HD / 8; ++s)
        qa[s] = *reinterpret_cast<const f4v*>(base + (int64_t)(q0 + li) * ld_in + q_off + 8 * s + 4 * lh);
    const int kb = wk * 64;  // this wave's first key
    const float mk0 = mask ? mask[kb + li] : 0.0f, mk1 = mask ? mask[kb + 32 + li] : 0.0f;
    __syncthreads();

    floatx16 sc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[j][r] = 0.0f;
#pragma unroll
    for (int s = 0; s < HD / 8; ++s) {
        f4v kf[2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
            kf[j] = *reinterpret_cast<const f4v*>(&Ks[(kb + j * 32 + li) * KST + 8 * s + 4 * lh]);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                sc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[s][q], kf[j][q], sc[j], 0, 0, 0);
    }
    // element r of a lane: query row 8*(r/4) + 4*lh + r%4 of the wave, key kb + 32*j + li
    float mx[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        sc[0][r] = sc[0][r] * scale + mk0;
        sc[1][r] = sc[1][r] * scale + mk1;
        float m = fmaxf(sc[0][r], sc[1][r]);
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        mx[r] = m;
    }
    if (li == 0)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wave][0][8 * (r >> 2) + 4 * lh + (r & 3)] = mx[r];
    __syncthreads();
    float sm[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float m = fmaxf(mx[r], red[wave ^ 1][0][8 * (r >> 2) + 4 * lh + (r & 3)]);
        sc[0][r] = expf(sc[0][r] - m);
        sc[1][r] = expf(sc[1][r] - m);
        float t = sc[0][r] + sc[1][r];
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) t += __shfl_xor(t, o);
        sm[r] = t;
    }
    float* P = Ps[wave];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) P[(8 * (r >> 2) + 4 * lh + (r & 3)) * PST + 32 * j + li] = sc[j][r];
    floatx16 o[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[j][r] = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {  // 8 keys per step; lanes 32-63 take keys + 4
        const f4v pa = *reinterpret_cast<const f4v*>(&P[li * PST + 8 * s + 4 * lh]);
        const int k0 = kb + 8 * s + 4 * lh;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(pa[q], Vs[(k0 + q) * KST + 32 * j + li], o[j], 0, 0, 0);
    }
    __syncthreads();  // every wave has read its P
    if (wk == 1) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) P[(8 * (r >> 2) + 4 * lh + (r & 3)) * PST + 32 * j + li] = o[j][r];
        if (li == 0)
#pragma unroll
            for (int r = 0; r < 16; ++r) red[wave][1][8 * (r >> 2) + 4 * lh + (r & 3)] = sm[r];
    }
    __syncthreads();
    if (wk == 0) {
        const float* O1 = Ps[wave ^ 1];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = 8 * (r >> 2) + 4 * lh + (r & 3);
            const float inv = 1.0f / (sm[r] + red[wave ^ 1][1][row]);
            float* orow = out + ((int64_t)b * S + q0 + row) * ld_out + h * HD;
#pragma unroll
            for (int j = 0; j < 2; ++j) orow[32 * j + li] = (o[j][r] + O1[row * PST + 32 * j + li]) * inv;
        }
    }
}

// attention_fused push: {B, H, S, HD, ld_in, q_off, k_off, v_off, ld_out, scale_bits,
// total = B*S*ld_out}.
int launch_attention_fused(const shp::Launch& l) {
    if (l.n_push < 11) return fail(SHP_ERR_PUSH, "attention_fused needs 11 push constants");
    const int32_t* q = l.push;
    const int B = q[0], H = q[1], S = q[2], HD = q[3], ld_in = q[4], q_off = q[5], k_off = q[6],
              v_off = q[7], ld_out = q[8];
    if (B <= 0 || H <= 0 || S <= 0 || HD <= 0) return fail(SHP_ERR_SHAPE, "attention_fused: dims");
    if (S != kAttS || HD != kAttHD)
        return fail(SHP_ERR_UNSUPPORTED, "attention_fused: sequence 128 and head dim 64 only");
    int rc = shp::check_total(l, (int64_t)B * S * ld_out, "attention_fused");
    if (rc) return rc;
    if (q[10] != (int64_t)B * S * ld_out) return fail(SHP_ERR_SHAPE, "attention_fused: total");
    const int64_t span = (int64_t)(H - 1) * HD + HD;
    if (q_off < 0 || k_off < 0 || v_off < 0 || q_off + span > ld_in || k_off + span > ld_in ||
        v_off + span > ld_in || ld_out < H * HD)
        return fail(SHP_ERR_SHAPE, "attention_fused: Q/K/V columns outside the rows");
    if ((ld_in | q_off | k_off | v_off) & 3 || !al16(l.in0))
        return fail(SHP_ERR_SHAPE, "attention_fused: Q/K/V rows must be 16-byte aligned");
    if ((int64_t)B * H * kAttQB > 0x7fffffff) return fail(SHP_ERR_SHAPE, "attention_fused: grid");
    float scale;
    memcpy(&scale, &q[9], 4);
    hipLaunchKernelGGL(attention_fused_kernel, dim3((unsigned)(B * H * kAttQB)), dim3(256), 0, l.stream,
                       (const float*)l.in0, (const float*)l.in1, (float*)l.out, H, ld_in, q_off,
                       k_off, v_off, ld_out, scale);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

int launch_dot_general(const shp::Launch& l) {
    if (l.n_push < 17) return fail(SHP_ERR_PUSH, "dot_general_strided needs 17 push constants");
    const int32_t* q = l.push;
    if (q[0] <= 0 || q[1] <= 0 || q[2] <= 0 || q[3] <= 0 || q[4] < 0)
        return fail(SHP_ERR_SHAPE, "dot_general_strided: dims");
    for (int i = 5; i < 17; ++i)
        if (q[i] < 0) return fail(SHP_ERR_SHAPE, "dot_general_strided: negative stride");
    int64_t total = (int64_t)q[0] * q[1] * q[2] * q[3];
    int rc = shp::check_total(l, total, "dot_general_strided");
    if (rc) return rc;
    GemmParams p = base_params();
    p.batch_outer = q[0]; p.batch_inner = q[1];
    p.M = q[2]; p.N = q[3]; p.K = q[4];
    p.a = (const float*)l.in0; p.sa_outer = q[5]; p.sa_inner = q[6]; p.sam = q[7]; p.sak = q[8];
    p.b = (const float*)l.in1; p.sb_outer = q[9]; p.sb_inner = q[10]; p.sbk = q[11]; p.sbn = q[12];
    p.c = (float*)l.out; p.sc_outer = q[13]; p.sc_inner = q[14]; p.scm = q[15]; p.scn = q[16];
    dot_epilogue(p, l);
    int am, bm;
    dot_modes(p, am, bm);
    return shp::gemm_launch(l.stream, p, am, bm, shp::C_STRIDED, l.workspace, l.workspace_bytes,
                            l.tune);
}

}  // namespace

namespace shp {

KernelEntry kGemmKernels[] = {
    {"hlo_conv_nhwc_hwio", 14, true, launch_hlo_conv},
    {"conv2d", 15, true, launch_conv2d},
    {"fully_connected", 4, true, launch_fully_connected},
    {"hlo_dot_batched", 5, true, launch_dot_batched},
    {"hlo_dot_rank2", 4, true, launch_dot_rank2},
    // native extensions
    {"conv2d_nhwc", 15, true, launch_conv2d_nhwc},
    {"dot_general_strided", 17, true, launch_dot_general},
    {"attention_fused", 11, false, launch_attention_fused},
};
const int kGemmKernelCount = sizeof(kGemmKernels) / sizeof(kGemmKernels[0]);

}  // namespace shp
