// The HLO path's shape ops that the reference runs on the host CPU between its Vulkan
// dispatches, as device kernels so tensors stay resident in HBM:
//   broadcast / broadcast_in_dim  source/xla_hlo/src/compiler.rs:336-347, broadcast_tensor :1361-1393
//   transpose (any rank)          compiler.rs:374-386, transpose_tensor :1395-1418
//   slice                         compiler.rs:570-582, parse_slice_spec :1897-1929, cpu_slice :1931-1952
//   concatenate                   compiler.rs:554-569, cpu_concatenate :1879-1895
//   compare (predicate as f32)    compiler.rs:511-537, binary_tensor :1521-1564, infer_broadcast_dims :1566-1572
//   select                        compiler.rs:538-553, select_tensor :1574-1620
//   reduce over any rank          compiler.rs:939-1007 (rank > 4 -> reduce_tensor :1730-1759), reduce_kind :1722-1728
//   strided copy                  no counterpart: materialises a view of the compiled HLO program
// The reference has no GLSL kernel (so no push layout) for these; the i32 push vectors
// below carry the HLO attributes directly (shapes, `dimensions`, slice starts/limits/strides,
// compare direction), so a host lowering passes what it parsed.  Ranks up to 8.
//
// Broadcast, transpose and slice are one strided gather: output coordinate c reads source
// element base + sum_k c_k * stride_k (stride 0 on broadcast axes, permuted strides for a
// transpose, start/step for a slice).  All are HBM-bound copies: one thread per output
// element, consecutive threads on consecutive outputs.
#include <cstring>

#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kMaxRank = 8;

unsigned hlo_grid(uint64_t n) {
    uint64_t g = (n + kBlock - 1) / kBlock;
    if (g > 256 * 32) g = 256 * 32;
    return g == 0 ? 1u : (unsigned)g;
}

struct Gather {
    int r;
    int dims[kMaxRank];         // output dims
    int64_t stride[kMaxRank];   // source element stride per output axis
    int64_t base;               // source offset of output coordinate 0
    int check;                  // slice: zero where first + c*step >= lim on some axis
    int64_t first[kMaxRank], step[kMaxRank], lim[kMaxRank];
};

__global__ __launch_bounds__(kBlock) void gather_kernel(const float* __restrict__ x,
                                                        float* __restrict__ y, Gather g,
                                                        uint64_t total) {
    const uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += stride) {
        uint64_t rem = i;
        int64_t off = g.base;
        bool ok = true;
        for (int k = g.r - 1; k >= 0; --k) {
            const int64_t c = (int64_t)(rem % (uint64_t)g.dims[k]);
            rem /= (uint64_t)g.dims[k];
            off += c * g.stride[k];
            if (g.check) ok = ok && (g.first[k] + c * g.step[k] < g.lim[k]);
        }
        float v = 0.0f;
        if (ok) v = x[off];
        y[i] = v;
    }
}

// Row-major element strides of a shape.
void strides_of(const int* dims, int r, int64_t* st) {
    int64_t s = 1;
    for (int k = r - 1; k >= 0; --k) {
        st[k] = s;
        s *= dims[k];
    }
}

int64_t elems_of(const int* dims, int r) {
    int64_t n = 1;
    for (int k = 0; k < r; ++k) n *= dims[k];
    return n;
}

int read_dims(const int32_t* q, int r, int* dims, const char* kernel) {
    for (int k = 0; k < r; ++k) {
        if (q[k] <= 0) return shp::fail(SHP_ERR_SHAPE, std::string(kernel) + ": dims must be > 0");
        dims[k] = q[k];
    }
    return SHP_OK;
}

int launch_gather(const shp::Launch& l, const Gather& g) {
    hipLaunchKernelGGL(gather_kernel, dim3(hlo_grid(l.out_elems)), dim3(kBlock), 0, l.stream,
                       (const float*)l.in0, (float*)l.out, g, l.out_elems);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// Operand broadcast as binary_tensor / select_tensor do it: an operand with as many
// elements as the output is taken flat; one element is splatted; otherwise its axes align
// with the trailing output axes (infer_broadcast_dims) and size-1 axes broadcast
// (broadcast_tensor).  Fills per-output-axis strides.
int operand_strides(const int* sd, int rs, const int* od, int ro, int64_t* st,
                    const char* kernel) {
    const int64_t n = elems_of(sd, rs), total = elems_of(od, ro);
    if (n == total) {
        strides_of(od, ro, st);
        return SHP_OK;
    }
    for (int k = 0; k < ro; ++k) st[k] = 0;
    if (n == 1) return SHP_OK;
    if (rs > ro) return shp::fail(SHP_ERR_SHAPE, std::string(kernel) + ": operand rank > output rank");
    int64_t sst[kMaxRank];
    strides_of(sd, rs, sst);
    const int offset = ro - rs;
    for (int a = 0; a < rs; ++a) {
        if (sd[a] == 1) continue;
        if (sd[a] != od[a + offset])
            return shp::fail(SHP_ERR_SHAPE, std::string(kernel) + ": operand does not broadcast");
        st[a + offset] = sst[a];
    }
    return SHP_OK;
}

// ---- hlo_broadcast: push {r_src, r_out, total, src_dims[r_src], out_dims[r_out],
//      dimensions[r_src]} (dimensions[a] = output axis of source axis a, as in HLO).
int launch_broadcast(const shp::Launch& l) {
    const int32_t* q = l.push;
    const int rs = q[0], ro = q[1];
    if (rs < 0 || rs > kMaxRank || ro < 1 || ro > kMaxRank)
        return shp::fail(SHP_ERR_SHAPE, "hlo_broadcast: rank out of range (0..8 / 1..8)");
    if ((int64_t)l.n_push < 3 + 2 * rs + ro)
        return shp::fail(SHP_ERR_PUSH, "hlo_broadcast needs 3 + 2*r_src + r_out push constants");
    int sd[kMaxRank], od[kMaxRank];
    int rc = read_dims(q + 3, rs, sd, "hlo_broadcast");
    if (!rc) rc = read_dims(q + 3 + rs, ro, od, "hlo_broadcast");
    if (rc) return rc;
    const int32_t* map = q + 3 + rs + ro;
    if (elems_of(od, ro) != q[2]) return shp::fail(SHP_ERR_SHAPE, "hlo_broadcast: total != product of out dims");
    rc = shp::check_total(l, q[2], "hlo_broadcast");
    if (rc) return rc;
    Gather g{};
    g.r = ro;
    for (int k = 0; k < ro; ++k) g.dims[k] = od[k];
    const int64_t n = elems_of(sd, rs);
    bool same = (rs == ro);
    for (int k = 0; same && k < rs; ++k) same = sd[k] == od[k];
    if (same) {  // broadcast_tensor: identical shape -> copy
        strides_of(od, ro, g.stride);
    } else if (n == 1) {  // one element -> splat (strides stay 0)
    } else {
        int64_t sst[kMaxRank];
        strides_of(sd, rs, sst);
        for (int a = 0; a < rs; ++a) {
            if (map[a] < 0 || map[a] >= ro)
                return shp::fail(SHP_ERR_SHAPE, "hlo_broadcast: dimensions entry out of range");
            if (sd[a] == 1) continue;
            if (sd[a] != od[map[a]])
                return shp::fail(SHP_ERR_SHAPE, "hlo_broadcast: source dim != mapped output dim");
            g.stride[map[a]] += sst[a];
        }
    }
    return launch_gather(l, g);
}

// ---- hlo_transpose: push {r, total, src_dims[r], perm[r]}; output axis i is source axis
//      perm[i] (HLO `dimensions`), so out dims are src_dims[perm[i]].
int launch_transpose_nd(const shp::Launch& l) {
    const int32_t* q = l.push;
    const int r = q[0];
    if (r < 1 || r > kMaxRank) return shp::fail(SHP_ERR_SHAPE, "hlo_transpose: rank out of range 1..8");
    if ((int64_t)l.n_push < 2 + 2 * r) return shp::fail(SHP_ERR_PUSH, "hlo_transpose needs 2 + 2*r push constants");
    int sd[kMaxRank];
    int rc = read_dims(q + 2, r, sd, "hlo_transpose");
    if (rc) return rc;
    const int32_t* perm = q + 2 + r;
    int seen = 0;
    for (int i = 0; i < r; ++i) {
        if (perm[i] < 0 || perm[i] >= r || (seen >> perm[i]) & 1)
            return shp::fail(SHP_ERR_SHAPE, "hlo_transpose: dimensions is not a permutation");
        seen |= 1 << perm[i];
    }
    if (elems_of(sd, r) != q[1]) return shp::fail(SHP_ERR_SHAPE, "hlo_transpose: total != product of dims");
    rc = shp::check_total(l, q[1], "hlo_transpose");
    if (rc) return rc;
    Gather g{};
    g.r = r;
    int64_t sst[kMaxRank];
    strides_of(sd, r, sst);
    for (int i = 0; i < r; ++i) {
        g.dims[i] = sd[perm[i]];
        g.stride[i] = sst[perm[i]];
    }
    return launch_gather(l, g);
}

// ---- hlo_slice: push {r, total, src_dims[r], starts[r], limits[r], strides[r]}; output dim
//      k is ceil((limit - start) / stride).  As cpu_slice, an output whose source coordinate
//      falls outside the source is 0.
int launch_slice(const shp::Launch& l) {
    const int32_t* q = l.push;
    const int r = q[0];
    if (r < 1 || r > kMaxRank) return shp::fail(SHP_ERR_SHAPE, "hlo_slice: rank out of range 1..8");
    if ((int64_t)l.n_push < 2 + 4 * r) return shp::fail(SHP_ERR_PUSH, "hlo_slice needs 2 + 4*r push constants");
    int sd[kMaxRank];
    int rc = read_dims(q + 2, r, sd, "hlo_slice");
    if (rc) return rc;
    const int32_t *st = q + 2 + r, *lim = q + 2 + 2 * r, *sp = q + 2 + 3 * r;
    Gather g{};
    g.r = r;
    g.check = 1;
    int64_t sst[kMaxRank];
    strides_of(sd, r, sst);
    for (int k = 0; k < r; ++k) {
        if (st[k] < 0 || sp[k] < 1 || lim[k] <= st[k])
            return shp::fail(SHP_ERR_SHAPE, "hlo_slice: need 0 <= start < limit and stride >= 1");
        g.dims[k] = (lim[k] - st[k] + sp[k] - 1) / sp[k];
        g.first[k] = st[k];
        g.step[k] = sp[k];
        g.lim[k] = sd[k];
        g.stride[k] = sst[k] * sp[k];
        if (st[k] < sd[k]) g.base += st[k] * sst[k];
    }
    if (elems_of(g.dims, r) != q[1]) return shp::fail(SHP_ERR_SHAPE, "hlo_slice: total != product of slice dims");
    rc = shp::check_total(l, q[1], "hlo_slice");
    if (rc) return rc;
    // a start past the source end leaves only zeros on that axis: keep the gather in range
    for (int k = 0; k < r; ++k)
        if (st[k] >= sd[k]) g.stride[k] = 0;
    return launch_gather(l, g);
}

// ---- hlo_concatenate_into: writes one operand (in0) into its slab of the output.
//      push {r, dim, offset, out_dims[r], in_dims[r]}; the operand's coordinate along `dim`
//      is shifted by `offset` (the summed extents of the operands before it); coordinates
//      past the output are dropped, as cpu_concatenate does.  N operands = N launches.
struct Slab {
    int r, dim, offset;
    int in_dims[kMaxRank], out_dims[kMaxRank];
    int64_t out_stride[kMaxRank];
};

__global__ __launch_bounds__(kBlock) void concat_into_kernel(const float* __restrict__ x,
                                                             float* __restrict__ y, Slab s,
                                                             uint64_t n_in) {
    const uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n_in; i += stride) {
        uint64_t rem = i;
        int64_t off = 0;
        bool ok = true;
        for (int k = s.r - 1; k >= 0; --k) {
            int64_t c = (int64_t)(rem % (uint64_t)s.in_dims[k]);
            rem /= (uint64_t)s.in_dims[k];
            if (k == s.dim) c += s.offset;
            ok = ok && c < s.out_dims[k];
            off += c * s.out_stride[k];
        }
        if (ok) y[off] = x[i];
    }
}

int launch_concatenate_into(const shp::Launch& l) {
    const int32_t* q = l.push;
    const int r = q[0];
    if (r < 1 || r > kMaxRank) return shp::fail(SHP_ERR_SHAPE, "hlo_concatenate_into: rank out of range 1..8");
    if ((int64_t)l.n_push < 3 + 2 * r)
        return shp::fail(SHP_ERR_PUSH, "hlo_concatenate_into needs 3 + 2*r push constants");
    Slab s{};
    s.r = r;
    s.dim = q[1];
    s.offset = q[2];
    if (s.dim < 0 || s.dim >= r || s.offset < 0)
        return shp::fail(SHP_ERR_SHAPE, "hlo_concatenate_into: bad dim/offset");
    int rc = read_dims(q + 3, r, s.out_dims, "hlo_concatenate_into");
    if (!rc) rc = read_dims(q + 3 + r, r, s.in_dims, "hlo_concatenate_into");
    if (rc) return rc;
    rc = shp::check_total(l, elems_of(s.out_dims, r), "hlo_concatenate_into");
    if (rc) return rc;
    strides_of(s.out_dims, r, s.out_stride);
    const uint64_t n_in = (uint64_t)elems_of(s.in_dims, r);
    hipLaunchKernelGGL(concat_into_kernel, dim3(hlo_grid(n_in)), dim3(kBlock), 0, l.stream,
                       (const float*)l.in0, (float*)l.out, s, n_in);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- hlo_compare: y = (a <dir> b) ? 1 : 0 with binary_tensor's operand broadcast.
//      push {direction, total, r_out, r_a, r_b, out_dims[r_out], a_dims[r_a], b_dims[r_b]};
//      direction 0 LT, 1 LE, 2 EQ, 3 NE, 4 GE, 5 GT (the reference's default).
// ---- hlo_select: y = pred != 0 ? on_true : y, where y holds on_false (already broadcast
//      to the output shape) on entry: the ABI has two inputs, so on_false rides in the
//      output buffer.  push {total, r_out, r_p, r_t, out_dims, pred_dims, true_dims}.
struct Bin {
    int r, dir;
    int dims[kMaxRank];
    int64_t as[kMaxRank], bs[kMaxRank];
};

template <bool SELECT>
__global__ __launch_bounds__(kBlock) void compare_select_kernel(const float* __restrict__ a,
                                                                const float* __restrict__ b,
                                                                float* __restrict__ y, Bin p,
                                                                uint64_t total) {
    const uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += stride) {
        uint64_t rem = i;
        int64_t ai = 0, bi = 0;
        for (int k = p.r - 1; k >= 0; --k) {
            const int64_t c = (int64_t)(rem % (uint64_t)p.dims[k]);
            rem /= (uint64_t)p.dims[k];
            ai += c * p.as[k];
            bi += c * p.bs[k];
        }
        const float u = a[ai], v = b[bi];
        if constexpr (SELECT) {
            if (u != 0.0f) y[i] = v;
        } else {
            bool t;
            switch (p.dir) {
                case 0: t = u < v; break;
                case 1: t = u <= v; break;
                case 2: t = u == v; break;
                case 3: t = u != v; break;
                case 4: t = u >= v; break;
                default: t = u > v; break;
            }
            y[i] = t ? 1.0f : 0.0f;
        }
    }
}

template <bool SELECT>
int launch_compare_select(const shp::Launch& l) {
    const char* kernel = SELECT ? "hlo_select" : "hlo_compare";
    // field k of the compare layout; select's layout lacks the leading direction
    auto q = [&](int k) { return l.push[SELECT ? k - 1 : k]; };
    const int ro = q(2), ra = q(3), rb = q(4);
    if (ro < 1 || ro > kMaxRank || ra < 0 || ra > kMaxRank || rb < 0 || rb > kMaxRank)
        return shp::fail(SHP_ERR_SHAPE, std::string(kernel) + ": rank out of range");
    const int64_t need = (SELECT ? 4 : 5) + ro + ra + rb;
    if ((int64_t)l.n_push < need)
        return shp::fail(SHP_ERR_PUSH, std::string(kernel) + " needs " + std::to_string(need) +
                                           " push constants");
    int od[kMaxRank], ad[kMaxRank], bd[kMaxRank];
    const int32_t* dims = &l.push[SELECT ? 4 : 5];
    int rc = read_dims(dims, ro, od, kernel);
    if (!rc) rc = read_dims(dims + ro, ra, ad, kernel);
    if (!rc) rc = read_dims(dims + ro + ra, rb, bd, kernel);
    if (rc) return rc;
    if (elems_of(od, ro) != q(1)) return shp::fail(SHP_ERR_SHAPE, std::string(kernel) + ": total != product of out dims");
    rc = shp::check_total(l, q(1), kernel);
    if (rc) return rc;
    Bin p{};
    p.r = ro;
    p.dir = SELECT ? 0 : q(0);
    if (!SELECT && (p.dir < 0 || p.dir > 5)) return shp::fail(SHP_ERR_INVALID, "hlo_compare: direction 0..5");
    for (int k = 0; k < ro; ++k) p.dims[k] = od[k];
    rc = operand_strides(ad, ra, od, ro, p.as, kernel);
    if (!rc) rc = operand_strides(bd, rb, od, ro, p.bs, kernel);
    if (rc) return rc;
    hipLaunchKernelGGL((compare_select_kernel<SELECT>), dim3(hlo_grid(l.out_elems)), dim3(kBlock),
                       0, l.stream, (const float*)l.in0, (const float*)l.in1, (float*)l.out, p,
                       l.out_elems);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

// ---- hlo_reduce: push {kind, r, total_out, init (f32 bits), src_dims[r], reduce[r]};
//      kind 0 sum, 1 max (reduce_kind); reduce[k] != 0 marks a reduced axis; the output
//      keeps the other axes in order.  Each output folds its inputs in increasing source
//      index from `init`, as reduce_tensor does (so sums match it bit for bit); max is
//      fmaxf, the NaN-ignoring maximum of Rust's f32::max.
struct Red {
    int kind, rk, rr;
    float init;
    int kdims[kMaxRank], rdims[kMaxRank];
    int64_t kstride[kMaxRank], rstride[kMaxRank];
    int64_t rcount;
};

__global__ __launch_bounds__(kBlock) void reduce_nd_kernel(const float* __restrict__ x,
                                                           float* __restrict__ y, Red p,
                                                           uint64_t total) {
    const uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t o = (uint64_t)blockIdx.x * kBlock + threadIdx.x; o < total; o += stride) {
        uint64_t rem = o;
        int64_t base = 0;
        for (int k = p.rk - 1; k >= 0; --k) {
            base += (int64_t)(rem % (uint64_t)p.kdims[k]) * p.kstride[k];
            rem /= (uint64_t)p.kdims[k];
        }
        float acc = p.init;
        int c[kMaxRank] = {0, 0, 0, 0, 0, 0, 0, 0};
        int64_t off = base;
        for (int64_t j = 0; j < p.rcount; ++j) {
            const float v = x[off];
            acc = p.kind ? fmaxf(acc, v) : acc + v;
            // next reduced coordinate in row-major order (last reduced axis fastest)
            for (int k = p.rr - 1; k >= 0; --k) {
                off += p.rstride[k];
                if (++c[k] < p.rdims[k]) break;
                off -= (int64_t)p.rdims[k] * p.rstride[k];
                c[k] = 0;
            }
        }
        y[o] = acc;
    }
}

// ---- hlo_strided_copy: push {r, total, dims[r], strides[r]}: out (row-major over dims) =
//      in0[sum_k c_k * strides[k]].  Materialises a strided view (a transpose, slice or
//      broadcast the HLO program kept as a view) into a contiguous tensor; in0 points at the
//      view's first element.  Strides >= 0 (0 on broadcast axes).
int launch_strided_copy(const shp::Launch& l) {
    const int32_t* q = l.push;
    const int r = q[0];
    if (r < 1 || r > kMaxRank) return shp::fail(SHP_ERR_SHAPE, "hlo_strided_copy: rank out of range 1..8");
    if ((int64_t)l.n_push < 2 + 2 * r) return shp::fail(SHP_ERR_PUSH, "hlo_strided_copy needs 2 + 2*r push constants");
    int dims[kMaxRank];
    int rc = read_dims(q + 2, r, dims, "hlo_strided_copy");
    if (rc) return rc;
    if (elems_of(dims, r) != q[1]) return shp::fail(SHP_ERR_SHAPE, "hlo_strided_copy: total != product of dims");
    rc = shp::check_total(l, q[1], "hlo_strided_copy");
    if (rc) return rc;
    Gather g{};
    g.r = r;
    for (int k = 0; k < r; ++k) {
        if (q[2 + r + k] < 0) return shp::fail(SHP_ERR_SHAPE, "hlo_strided_copy: negative stride");
        g.dims[k] = dims[k];
        g.stride[k] = q[2 + r + k];
    }
    return launch_gather(l, g);
}

int launch_reduce_nd(const shp::Launch& l) {
    const int32_t* q = l.push;
    const int r = q[1];
    if (r < 1 || r > kMaxRank) return shp::fail(SHP_ERR_SHAPE, "hlo_reduce: rank out of range 1..8");
    if ((int64_t)l.n_push < 4 + 2 * r) return shp::fail(SHP_ERR_PUSH, "hlo_reduce needs 4 + 2*r push constants");
    if (q[0] != 0 && q[0] != 1) return shp::fail(SHP_ERR_INVALID, "hlo_reduce: kind 0 (sum) or 1 (max)");
    int sd[kMaxRank];
    int rc = read_dims(q + 4, r, sd, "hlo_reduce");
    if (rc) return rc;
    Red p{};
    p.kind = q[0];
    std::memcpy(&p.init, &q[3], sizeof(float));
    int64_t sst[kMaxRank];
    strides_of(sd, r, sst);
    p.rcount = 1;
    int64_t kept = 1;
    for (int k = 0; k < r; ++k) {
        if (q[4 + r + k]) {
            p.rdims[p.rr] = sd[k];
            p.rstride[p.rr++] = sst[k];
            p.rcount *= sd[k];
        } else {
            p.kdims[p.rk] = sd[k];
            p.kstride[p.rk++] = sst[k];
            kept *= sd[k];
        }
    }
    if (kept != q[2]) return shp::fail(SHP_ERR_SHAPE, "hlo_reduce: total != product of kept dims");
    rc = shp::check_total(l, q[2], "hlo_reduce");
    if (rc) return rc;
    hipLaunchKernelGGL(reduce_nd_kernel, dim3(hlo_grid(l.out_elems)), dim3(kBlock), 0, l.stream,
                       (const float*)l.in0, (float*)l.out, p, l.out_elems);
    SHP_HIP_CHECK(hipGetLastError());
    return SHP_OK;
}

}  // namespace

namespace shp {

KernelEntry kHloOpKernels[] = {
    {"hlo_broadcast", 3, false, launch_broadcast},
    {"hlo_transpose", 2, false, launch_transpose_nd},
    {"hlo_slice", 2, false, launch_slice},
    {"hlo_concatenate_into", 3, false, launch_concatenate_into},
    {"hlo_compare", 5, false, launch_compare_select<false>},
    {"hlo_select", 4, false, launch_compare_select<true>},
    {"hlo_reduce", 4, false, launch_reduce_nd},
    {"hlo_strided_copy", 2, false, launch_strided_copy},
};
const int kHloOpKernelCount = sizeof(kHloOpKernels) / sizeof(kHloOpKernels[0]);

}  // namespace shp
