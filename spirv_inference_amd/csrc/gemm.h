// Dense-contraction problem description shared by the MFMA implicit-GEMM kernels and
// their host-side launchers.
#pragma once

#include "common.h"

namespace shp {

// How the A operand (M x K) is addressed.
enum AMode {
    A_KVEC = 0,       // A[b][m][k] at a + bofs + m*sam + k, float4 along k
    A_STRIDED = 1,    // A[b][m][k] at a + bofs + m*sam + k*sak, scalar
    A_CONV_NHWC4 = 2, // im2col of an NHWC input, IC % 4 == 0, float4 along k=(ky,kx,ic)
    A_CONV_NHWC = 3,  // im2col of an NHWC input, any IC, scalar
    A_CONV_NCHW = 4,  // im2col of an NCHW input, k = (ic,ky,kx) (conv2d.comp order), scalar
};
// How the B operand (K x N) is addressed.
enum BMode {
    B_NVEC = 0,       // B[b][k][n] at b + bofs + k*sbk + n, float4 along n (HWIO, row-major)
    B_KVEC = 1,       // B[b][k][n] at b + bofs + n*sbn + k, float4 along k ([out,in], OIHW)
    B_STRIDED = 2,    // B[b][k][n] at b + bofs + k*sbk + n*sbn, scalar
};
// How C (M x N) is stored.
enum CMode {
    C_STRIDED = 0,    // C[b][m][n] at c + bofs + m*scm + n*scn
    C_NCHW = 1,       // conv2d.comp output: m = (img, oh, ow), n = oc
};

struct GemmParams {
    int M, N, K;
    int batch_outer, batch_inner;  // batch index = outer * batch_inner + inner
    const float* a;
    int64_t sa_outer, sa_inner, sam, sak;
    const float* b;
    int64_t sb_outer, sb_inner, sbk, sbn;
    float* c;
    int64_t sc_outer, sc_inner, scm, scn;
    // epilogue (applied by the kernel, or by the split-K reduction)
    const float* bias;      // indexed by n
    const float* residual;  // same addressing as c
    int act;
    float alpha;
    // convolution geometry (A_CONV_*), C_NCHW uses oh*ow
    int cn, cih, ciw, cic, ckh, ckw, coh, cow, csh, csw, cpt, cpl;
    // split-K
    int splits;
    int k_per_split;  // multiple of the K tile
    float* partial;   // [splits][batch][M][N] workspace when splits > 1
    int* counters;    // per-tile arrival counters (zero between launches) when fixup
    int fixup;        // 1: the last split of a tile sums the partials and applies the epilogue
    // tile order: bands of group_m tile rows, each band walked column by column (1: row
    // major); each XCD then takes a contiguous run of that order (tile_coords)
    int group_m;
};

// The first kSplitCounterBytes of a split-K workspace hold the per-tile arrival counters of
// the in-kernel fixup; they must be zero when a workspace is first handed out, and every
// launch leaves them zero again.  The partials follow.
constexpr size_t kSplitCounterBytes = 65536;

// Launch C = epilogue(A*B) for the problem; picks tile shape and split-K (`tune` may force
// parts of that choice, or be null).  `workspace`/`workspace_bytes` provide the split-K
// partials (may be null: no split).
int gemm_launch(hipStream_t stream, GemmParams p, int amode, int bmode, int cmode,
                float* workspace, size_t workspace_bytes, const GemmTune* tune);

// Workspace the launcher would like for this problem (0 if it will not split K).
size_t gemm_workspace_bytes(const GemmParams& p, int amode, int bmode, int cmode,
                            const GemmTune* tune);

}  // namespace shp
