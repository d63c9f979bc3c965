// Persistent batch-1 decode: every token of a decode call in ONE cooperative launch.
//
// Same math as the per-op decode kernels (export_llama.py:284-375 with a KV cache): RMSNorm,
// fused QKV, RoPE, GQA attention, Wo + residual, RMSNorm, SwiGLU gate/up, down + residual,
// final RMSNorm, lm_head and a greedy argmax that feeds the next token.
//
// Why one launch: at batch 1 a token is ~115 small HBM-bound GEMVs.  As separate kernels each
// pays a launch gap, a ramp and a drain, and those dominate the 2-90 MB reads.  Here one
// workgroup of 512 threads runs on every CU for the whole call; the phases of a layer are
// separated by grid barriers (per-workgroup epoch flags) or tagged-word waits, and before
// waiting every workgroup already issues the weight loads of its share of the NEXT phase
// (weights do not depend on the wait), so HBM keeps streaming while the grid synchronises.
//
// Phases of one layer (rows of each matrix split evenly over the workgroups):
//   A  qkv = Wqkv . rmsnorm(x) * attn_norm
//   B1 attention, one workgroup per query head (RoPE, online softmax over the cached
//      positions staged in LDS in 64-position tiles); the workgroup of a group's first query
//      head appends its K/V to the cache
//   B2 x[r] += Wo[r] . att
//   C  act = silu(Wg . h) * (Wu . h), h = rmsnorm(x) * ffn_norm (gate/up rows interleaved)
//   D  x[r] += Wdown[r] . act
// After the last layer: E logits = lm_head . rmsnorm(x) * final_norm with a per-workgroup
// argmax, then F the global argmax (every workgroup reduces the candidates itself).
// Layer 0 reads the embedding row directly, so no barrier is needed between tokens.
//
// Grid barriers follow B1, C, D and E.  A and B2 end without one: their outputs are also
// stored as tagged words, (phase epoch << 32) | float bits, in one 64-bit store each, and
// their only consumers (attention for A's q / k / v, the gate/up norm for B2's x) poll
// exactly the words they need until every tag carries the phase's epoch.  That saves the
// producer's wait for its stores, the flag round trip and the separate data load.  The
// write-after-read hazards those barriers also covered stay covered: the next writes of qkv
// and x come after the following grid barrier.
//
// Weight rows are streamed with 16-byte non-temporal loads, up to three chunks (64 KB each per
// CU) ahead of the arithmetic, on a schedule that keeps each CU's load pipe (~30 GB/s, ~64 KB
// in flight) busy through the short latency-bound phases (see the layer loop).  The
// workgroups without an attention head also park two gate/up chunks in LDS during the
// attention phase (five chunks resident when gate/up starts), and the gate/up rows are split
// 1:2 between the workgroups with an attention head and the others.
//
// GEMV layout: a chunk is 8 rows, one per wavefront, and a wavefront reads its row in 1 KB
// contiguous loads against the phase's input vector staged once in LDS.  A row's total is a
// wavefront sum (VALU only: v_permlane32/16_swap, DPP) and lane 0 does its epilogue, so the
// ~300 chunks of a token need no workgroup barrier; only SwiGLU (pairs of rows on two
// wavefronts) and the lm_head argmax combine wavefronts, once at the end of their phase.
// Rows wider than 512 float4 (the down projection) are split into segments of 512 that the
// owning wavefront accumulates.
//
// Cross-workgroup data (qkv, x, act, the KV cache rows, the argmax candidates) is written and
// read with agent-scope relaxed atomics, i.e. stores and loads that go to the device-coherent
// level instead of the per-XCD L2.  A barrier is then only: every wave waits for its stores
// to complete, each workgroup stores the barrier's epoch into its own flag, and four
// wavefronts poll the flags.  No L2 write-back or invalidate is needed, which is what makes a
// barrier ~2.5 us instead of ~10-30 us with release/acquire fences on MI355X.
// Every wait is bounded (spin_limit polls); on expiry the workgroup raises abort_flag and
// every workgroup exits, so the grid always drains.  A wait checks the flag and its limit every
// 128 polls, counting from spin_start (0; 127 makes the first missed poll check already, which
// lets the host force a give-up with a small limit).
#include <cfloat>

#include "decode.h"

namespace {

using shp::ArgmaxCand;
using shp::PersistArgs;
using shp::PersistLayer;

constexpr int NT = 512;  // threads per workgroup
constexpr int NW = NT / 64;
constexpr int NB = 8;    // float4 weight slots per thread per chunk

typedef float nfloat4 __attribute__((ext_vector_type(4)));
// Pointers that arrive through structs are generic; accessing them as global (address space
// 1) keeps the loads off the flat path, whose completion is also counted by the LDS counter
// (a flat load in flight would then stall every LDS wait of the reduction).
#define SHP_GLOBAL __attribute__((address_space(1)))

__device__ __forceinline__ float4 ldw(const float* p) {
    nfloat4 v = __builtin_nontemporal_load((const SHP_GLOBAL nfloat4*)p);
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 ldw_at(const float* base, unsigned byte_off) {
    const SHP_GLOBAL char* p = (const SHP_GLOBAL char*)base + byte_off;
    nfloat4 v = __builtin_nontemporal_load((const SHP_GLOBAL nfloat4*)p);
    return make_float4(v.x, v.y, v.z, v.w);
}
// Global memory only: the cast to address space 1 would misread an LDS pointer.
__device__ __forceinline__ float4 ldg4(const float* p) {
    nfloat4 v = *(const SHP_GLOBAL nfloat4*)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
// Device-coherent (agent scope) accesses for data exchanged between workgroups (global
// memory only, like ldg4).
__device__ __forceinline__ float ld_coh(const float* p) {
    return __hip_atomic_load((SHP_GLOBAL float*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(float* p, float v) {
    __hip_atomic_store((SHP_GLOBAL float*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Device-coherent 16-byte load at a uniform base plus a 32-bit per-lane byte offset: the
// address is formed from scalar registers at the load, so the compiler keeps no 64-bit per-lane
// pointer live (such pointers get spilled, and a spill reload waits for every load in flight).
__device__ __forceinline__ float4 ld_coh4_at(const float* base, unsigned byte_off) {
    SHP_GLOBAL unsigned long long* q =
        (SHP_GLOBAL unsigned long long*)((const SHP_GLOBAL char*)base + byte_off);
    unsigned long long lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned long long hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float4(__uint_as_float((unsigned)lo), __uint_as_float((unsigned)(lo >> 32)),
                       __uint_as_float((unsigned)hi), __uint_as_float((unsigned)(hi >> 32)));
}
__device__ __forceinline__ float dot4(float4 a, float4 b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}
// Cross-lane VALU helpers (gfx950): v_permlane32_swap / v_permlane16_swap exchange halves and
// rows of 16 lanes; DPP row rotations reach lanes within a row.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// Sum / max over the wavefront, in every lane.  Bit for bit the xor butterfly (o = 32 .. 1):
// after the lane-bit-5 and -4 steps every value is symmetric under those bits, and after each
// rotation step under one more, so a row rotation by 8, 4, 2, 1 reads a lane holding the same
// value as lane ^ 8, ^ 4, ^ 2, ^ 1.
__device__ __forceinline__ float wave_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(q[0]) + __uint_as_float(q[1]);
    v += dpp<0x128>(v);  // row_ror:8
    v += dpp<0x124>(v);  // row_ror:4
    v += dpp<0x122>(v);  // row_ror:2
    v += dpp<0x121>(v);  // row_ror:1
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
    v = fmaxf(v, dpp<0x128>(v));
    v = fmaxf(v, dpp<0x124>(v));
    v = fmaxf(v, dpp<0x122>(v));
    v = fmaxf(v, dpp<0x121>(v));
    return v;
}
__device__ __forceinline__ void part(int n, int b, int g, int& r0, int& r1) {
    r0 = (int)((int64_t)n * b / g);
    r1 = (int)((int64_t)n * (b + 1) / g);
}
// As part(), with workgroups b < na weighted wa and the others wb.
__device__ __forceinline__ void part_w(int n, int b, int g, int na, int wa, int wb, int& r0,
                                       int& r1) {
    auto cw = [&](int i) -> int64_t {
        return i <= na ? (int64_t)i * wa : (int64_t)na * wa + (int64_t)(i - na) * wb;
    };
    const int64_t tot = cw(g);
    r0 = (int)((int64_t)n * cw(b) / tot);
    r1 = (int)((int64_t)n * cw(b + 1) / tot);
}

// Sum over the workgroup; `scratch` holds NW floats.  Ends with a barrier so the scratch
// can be reused immediately.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) s += scratch[w];
    __syncthreads();
    return s;
}

// Chunk: 8 rows, row rc + w for wavefront w, of a row-major [rows][K4] float4 matrix, segment
// `seg` of the columns: lane l holds columns seg * 512 + l + 64 i (i < NB), so one load
// instruction of a wavefront reads 1 KB of one row.  Every slot is loaded unconditionally:
// rows >= r1 read the zero row (a few KB that stay in L2), columns >= K4 are clamped to the
// last column (the staged vector is zero there).  The row base is uniform per wavefront.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ void load_chunk(float4 (&b)[NB], const float* __restrict__ W, int K4,
                                           int rc, int seg, int r1, const float* zero_row) {
    // The lane's byte offset passes through an empty asm, so the per-slot offsets derived from
    // it are formed at each load (two VALU operations) instead of being hoisted out of the
    // token loop as 64-bit values, which the compiler then spills.
    unsigned l16 = (threadIdx.x & 63) * 16u;
    asm volatile("" : "+v"(l16));
    const int row = rc + wave_id();
    const float* rowp = row < r1 ? W + (size_t)row * (size_t)K4 * 4 : zero_row;
    const unsigned lim = ((unsigned)K4 - 1u) * 16u;
#pragma unroll
    for (int i = 0; i < NB; ++i)
        b[i] = ldw_at(rowp, min(l16 + (unsigned)(seg * NB * 64 + 64 * i) * 16u, lim));
}

// This lane's part of the chunk row's dot product with the staged vector segment xn (LDS).
__device__ __forceinline__ float chunk_dot(const float4 (&b)[NB], const float4* xn) {
    const int lane = threadIdx.x & 63;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NB; ++i) s += dot4(b[i], xn[lane + 64 * i]);
    return s;
}

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_LOGITS = 3, EPI_QKV = 4 };

struct Epi {
    float* out;
    const float* resid;  // EPI_RESID: LDS copy of the vector added per row
    float* rows;         // EPI_SWIGLU: LDS row results, indexed from row0
    int row0;
    float best;          // EPI_LOGITS: this wavefront's running max / index
    int best_idx;
    unsigned long long* tag;  // EPI_QKV, EPI_RESID: tagged copy of each row,
    unsigned epoch;           // (epoch << 32) | float bits
};

// A row is complete: its total (in every lane), then the epilogue (lane 0 stores).
template <int EPI>
__device__ __forceinline__ void row_done(float part, int row, int r1, Epi& e) {
    const float s = wave_sum(part);
    if (row >= r1) return;  // uniform over the wavefront
    const bool l0 = (threadIdx.x & 63) == 0;
    if constexpr (EPI == EPI_STORE) {
        if (l0) st_coh(e.out + row, s);
    } else if constexpr (EPI == EPI_QKV) {
        if (l0) {
            st_coh(e.out + row, s);
            __hip_atomic_store((SHP_GLOBAL unsigned long long*)(e.tag + row),
                               ((unsigned long long)e.epoch << 32) | __float_as_uint(s),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else if constexpr (EPI == EPI_RESID) {
        if (l0) {
            const float v = s + e.resid[row];
            st_coh(e.out + row, v);
            __hip_atomic_store((SHP_GLOBAL unsigned long long*)(e.tag + row),
                               ((unsigned long long)e.epoch << 32) | __float_as_uint(v),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else if constexpr (EPI == EPI_SWIGLU) {
        if (l0) e.rows[row - e.row0] = s;
    } else {
        if (l0) e.out[row] = s;
        if (s > e.best || (s == e.best && row < e.best_idx)) {
            e.best = s;
            e.best_idx = row;
        }
    }
}

// One chunk of a stream: its dot products, the refill of its registers with chunk q + 3 (so
// the load pipe stays full while this chunk's row is reduced), and, on the row's last
// segment, the row's epilogue.
template <int EPI, int NSEG>
__device__ __forceinline__ void stream_step(float4 (&b)[NB], int q, int nq,
                                            const float* __restrict__ W, int K4, int r0, int r1,
                                            const float4* xn, float& acc, Epi& e,
                                            const float* zero_row) {
    const int rg = q / NSEG, seg = q - rg * NSEG;
    // The vector reads stay in the loop: hoisted (they are loop-invariant per register set),
    // they would hold 32 VGPRs per segment for the whole stream.
    asm volatile("" ::: "memory");
    acc += chunk_dot(b, xn + seg * NB * 64);
    const int q3 = q + 3, rg3 = q3 / NSEG;
    // past the last chunk nothing is loaded: those loads would only delay this workgroup's
    // barrier arrival, which waits for every load issued before its stores
    if (q3 < nq) load_chunk(b, W, K4, r0 + 8 * rg3, q3 - rg3 * NSEG, r1, zero_row);
    if (seg == NSEG - 1) {
        row_done<EPI>(acc, r0 + 8 * rg + wave_id(), r1, e);
        acc = 0.0f;
    }
}

// Rows [r0, r1) of W against the staged vector xn (NSEG segments of 512 float4), in chunks
// q = 0 .. nq-1 (row group q / NSEG, segment q % NSEG) rotating over three register sets.
// On entry b0 holds chunk 0, b1 chunk 1 when PRE >= 2, b2 chunk 2 when PRE == 3.
template <int EPI, int NSEG, int PRE>
__device__ __forceinline__ void stream_rows(const float* __restrict__ W, int K4, int r0, int r1,
                                            const float4* xn, float4 (&b0)[NB],
                                            float4 (&b1)[NB], float4 (&b2)[NB], Epi& e,
                                            const float* zero_row) {
    const int nq = (r1 - r0 + 7) / 8 * NSEG;
    if constexpr (PRE == 1)
        if (nq > 1) load_chunk(b1, W, K4, r0 + 8 * (1 / NSEG), 1 % NSEG, r1, zero_row);
    if constexpr (PRE <= 2)
        if (nq > 2) load_chunk(b2, W, K4, r0 + 8 * (2 / NSEG), 2 % NSEG, r1, zero_row);
    float acc = 0.0f;
    for (int q = 0; q < nq; q += 3) {
        stream_step<EPI, NSEG>(b0, q, nq, W, K4, r0, r1, xn, acc, e, zero_row);
        if (q + 1 >= nq) break;
        stream_step<EPI, NSEG>(b1, q + 1, nq, W, K4, r0, r1, xn, acc, e, zero_row);
        if (q + 2 >= nq) break;
        stream_step<EPI, NSEG>(b2, q + 2, nq, W, K4, r0, r1, xn, acc, e, zero_row);
    }
}

// LDS chunk stage: thread t keeps float4 i of a register chunk at slot[i * NT + t]
// (consecutive threads, consecutive 16 bytes: conflict-free), and reads back only its own.
__device__ __forceinline__ void stage_chunk(float4* slot, const float4 (&b)[NB]) {
#pragma unroll
    for (int i = 0; i < NB; ++i) slot[i * NT + threadIdx.x] = b[i];
}
__device__ __forceinline__ float chunk_dot_lds(const float4* slot, const float4* xn) {
    const int lane = threadIdx.x & 63;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NB; ++i) s += dot4(slot[i * NT + threadIdx.x], xn[lane + 64 * i]);
    return s;
}

// Rows [r0, r1) (one segment) with chunks 0 .. nls-1 staged in LDS (slot k at
// stage + k * NB * NT) and chunks nls .. nls+2 already issued into c0, c1 and c2: the resident
// register chunks first, so that chunk nls + 3 streams from the start, then the LDS chunks.
template <int EPI>
__device__ __forceinline__ void stream_rows_staged(const float* __restrict__ W, int K4, int r0,
                                                   int r1, int nls, const float4* stage,
                                                   const float4* xn, float4 (&c0)[NB],
                                                   float4 (&c1)[NB], float4 (&c2)[NB], Epi& e,
                                                   const float* zero_row) {
    const int nch = (r1 - r0 + 7) / 8;
    const int w = wave_id();
    for (int c = nls; c < nch; c += 3) {
        float acc = 0.0f;
        stream_step<EPI, 1>(c0, c, nch, W, K4, r0, r1, xn, acc, e, zero_row);
        if (c + 1 < nch) {
            stream_step<EPI, 1>(c1, c + 1, nch, W, K4, r0, r1, xn, acc, e, zero_row);
            if (c + 2 < nch) stream_step<EPI, 1>(c2, c + 2, nch, W, K4, r0, r1, xn, acc, e, zero_row);
        }
        if (c == nls) {
            for (int k = 0; k < nls; ++k)
                row_done<EPI>(chunk_dot_lds(stage + k * NB * NT, xn), r0 + 8 * k + w, r1, e);
        }
    }
    for (int k = 0; k < nls && k < nch && nch <= nls; ++k)
        row_done<EPI>(chunk_dot_lds(stage + k * NB * NT, xn), r0 + 8 * k + w, r1, e);
}

// Grid barrier, split so the caller can issue loads between arrival and wait.
// Arrival: every wave waits for its own stores (vmcnt 0: the coherent stores have completed),
// then thread 0 stores the barrier's epoch into the workgroup's flag (64 bytes apart; no
// atomics, so no contention).  Wait: wavefronts 0 .. ceil(grid/64)-1 poll 64 flags each until
// all have reached the epoch.  On MI355X this takes ~2.4 us against ~3.7 us for a two-level
// atomic counter.
__device__ __forceinline__ void bar_arrive(unsigned long long* flags, unsigned long long epoch) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt/lgkmcnt unconstrained
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_store((SHP_GLOBAL unsigned long long*)(flags + 8 * blockIdx.x), epoch,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until every workgroup's flag holds `epoch`; false (uniformly over the workgroup) when
// a wait gave up or another workgroup did.  okw: NW ints of LDS.
__device__ __forceinline__ bool bar_wait(const PersistArgs& a, unsigned long long epoch,
                                         int* okw) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int G = gridDim.x;
    if (wave * 64 < G) {
        const int f = wave * 64 + lane;
        int ok = 1;
        long long n = a.spin_start;
        while (true) {
            const unsigned long long v =
                f < G ? __hip_atomic_load((SHP_GLOBAL unsigned long long*)(a.flags + 8 * f),
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                      : ~0ull;
            if (__all(v >= epoch)) break;
            __builtin_amdgcn_s_sleep(1);
            if ((++n & 127) == 0) {
                if (__hip_atomic_load((SHP_GLOBAL int*)a.abort_flag, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) != 0 ||
                    n > a.spin_limit) {
                    if (lane == 0)
                        __hip_atomic_store((SHP_GLOBAL int*)a.abort_flag, 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                    ok = 0;
                    break;
                }
            }
        }
        asm volatile("" ::: "memory");  // no load of the next phase moves above the wait
        if (lane == 0) okw[wave] = ok;
    }
    __syncthreads();
    int ok = 1;
    for (int w = 0; w * 64 < G; ++w) ok &= okw[w];
    return ok != 0;
}

// RMSNorm of the vector slice, in two steps so weight loads can be issued between them:
// norm_load issues this thread's float4 of x (device-coherent unless it is a read-only row,
// the embedding) and keeps it in xs (LDS) for the residual add of the next phase;
// norm_finish writes xn = (x * rsqrt(mean(x^2) + eps)) * w to LDS (zero beyond K) and
// synchronises the workgroup.  K4 <= NT.
struct NormIn {
    float4 x, w;
};
__device__ __forceinline__ NormIn norm_load(const float* __restrict__ x, bool coherent, int K,
                                            const float* __restrict__ w) {
    const int t = threadIdx.x;
    NormIn r;
    r.x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    r.w = r.x;
    if (t < K / 4) {
        r.x = coherent ? ld_coh4_at(x, (unsigned)t * 16u) : ldg4(x + 4 * t);
        r.w = ldg4(w + 4 * t);
    }
    return r;
}
// norm_load for x written by the phase with epoch `epoch`: this thread's four tagged words
// are polled until all carry it (bounded like the barriers; okw[wave] = 0 when a wait gave
// up).  The caller issues its prefetch loads first, so the first poll returns after them.
__device__ __forceinline__ NormIn norm_load_tagged(const PersistArgs& a, unsigned epoch, int K,
                                                   const float* __restrict__ w, int* okw) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const bool act = t < K / 4;
    NormIn r;
    r.w = act ? ldg4(w + 4 * t) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    SHP_GLOBAL unsigned long long* q = (SHP_GLOBAL unsigned long long*)a.x_tag + 4 * t;
    unsigned long long v[4] = {0, 0, 0, 0};
    int ok = 1;
    long long n = a.spin_start;
    while (true) {
        bool ready = true;
        if (act) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = __hip_atomic_load(q + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ready = ready && (unsigned)(v[i] >> 32) == epoch;
            }
        }
        if (__all(ready)) break;
        __builtin_amdgcn_s_sleep(1);
        if ((++n & 127) == 0) {
            if (__hip_atomic_load((SHP_GLOBAL int*)a.abort_flag, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) != 0 ||
                n > a.spin_limit) {
                if (lane == 0)
                    __hip_atomic_store((SHP_GLOBAL int*)a.abort_flag, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                ok = 0;
                break;
            }
        }
    }
    if (lane == 0) okw[wave] = ok;
    r.x = make_float4(__uint_as_float((unsigned)v[0]), __uint_as_float((unsigned)v[1]),
                      __uint_as_float((unsigned)v[2]), __uint_as_float((unsigned)v[3]));
    return r;
}
__device__ __forceinline__ bool all_ok(const int* okw) {
    int all = 1;
#pragma unroll
    for (int w = 0; w < NW; ++w) all &= okw[w];
    return all != 0;
}

__device__ __forceinline__ void norm_finish(NormIn in, int K, float eps, float* scratch,
                                            float* xs, float4* xn) {
    const int t = threadIdx.x;
    float4 v = in.x;
    if (t < K / 4) *reinterpret_cast<float4*>(xs + 4 * t) = v;
    float ss = block_sum(dot4(v, v), scratch);
    const float inv = 1.0f / sqrtf(ss / (float)K + eps);
    if (t < K / 4) {
        const float4 g = in.w;
        v = make_float4((v.x * inv) * g.x, (v.y * inv) * g.y, (v.z * inv) * g.z,
                        (v.w * inv) * g.w);
    }
    xn[t] = v;  // zero beyond K
    __syncthreads();
}

// Phase timestamp for the optional profile buffer (thread 0 of each workgroup).
__device__ __forceinline__ void stamp(const PersistArgs& a, int it, int k, int which) {
    if (a.prof && threadIdx.x == 0) {
        const int nb = 5 * a.n_layers + 1;
        a.prof[((size_t)(it * nb + k) * 16 + which) * gridDim.x + blockIdx.x] = wall_clock64();
    }
}

constexpr int KSTRIDE = 68;  // LDS row stride of staged K rows: conflict-free 16-byte reads
constexpr int GU_ROWS = 448;   // gate/up rows of one workgroup kept in LDS (persist_plan checks)
constexpr int LDS_MISC = 512;  // floats before the hidden-sized residual copy

__device__ __forceinline__ float lane_bcast(float v, int src) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

// Phase B1: the attention of query heads h = blockIdx.x, + gridDim.x, ... at position `pos`,
// one workgroup per head, written to a.att (device-coherent).
//
// Per tile of 64 cached positions all 512 threads stage the K rows (padded to KSTRIDE) and V
// rows of the head's KV group in LDS with coalesced device-coherent loads (one round trip;
// the first tile also brings q, k and v of the current position).  Wavefront 0 then computes:
// lane = position holds its K row, q[d] comes from lane d by readlane, an online softmax
// (running max m, sum l; output o[lane = dim]) absorbs the tile, and the weights are shared
// through LDS to all 8 wavefronts, which split the PV sum.  The current position comes last,
// from the rotated k / v; the workgroup of the group's first query head appends those to
// the cache.  kv_s: [64][KSTRIDE] K | [64][64] V | q, k, v [3][64] | p [64] | PV [NW][64].
// q, k and v of the current position are read from a.qkv_tag once
// all 192 words carry `epoch` (the qkv phase's); false (uniformly over the workgroup) when that
// wait gave up or another workgroup did.  okw: NW ints of LDS.
__device__ __forceinline__ bool attention_heads(const PersistArgs& a, int l, int pos,
                                                float* kv_s, int it, int kb, unsigned epoch,
                                                int* okw) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int nq = a.n_heads, nkv = a.n_kv, grp = nq / nkv, S = a.max_seq;
    const int64_t per_layer = (int64_t)nkv * S * 64;
    float* kc = a.k_cache + l * per_layer;
    float* vc = a.v_cache + l * per_layer;
    float* ks = kv_s;
    float* vs = ks + 64 * KSTRIDE;
    float* cur = vs + 64 * 64;  // q | k | v of the current position
    float* pe = cur + 3 * 64;   // [64] softmax weights of the tile
    float* po = pe + 64;        // [NW][64] PV partial sums
    pos = __builtin_amdgcn_readfirstlane(pos);
    // RoPE rotate-half, angle pos * theta^(-2j/64), j = lane mod 32
    const int j = lane & 31;
    const float inv_freq = 1.0f / powf(a.theta, (float)(2 * j) / 64.0f);
    const float ang = (float)pos * inv_freq;
    const float cs = cosf(ang), sn = sinf(ang);
    for (int h = blockIdx.x; h < nq; h += gridDim.x) {
        const int g = h / grp;
        const float* kg = kc + (int64_t)g * S * 64;
        const float* vg = vc + (int64_t)g * S * 64;
        float qr = 0.0f, kr = 0.0f, vcur = 0.0f, o = 0.0f, m = -FLT_MAX, lsum = 0.0f;
        for (int t0 = 0;; t0 += 64) {
            const int nrows = min(64, pos - t0);  // cached rows in this tile (<= 0: none)
            float4 k4[2], v4[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int f = t + NT * u, row = f >> 4, c4 = f & 15;
                if (row < nrows) {
                    const unsigned off = (unsigned)((t0 + row) * 64 + c4 * 4) * 4u;
                    k4[u] = ld_coh4_at(kg, off);
                    v4[u] = ld_coh4_at(vg, off);
                }
            }
            if (t0 == 0) {  // q_h, k_g, v_g: wavefronts 0-2 wait for their 64 tagged words
                int ok = 1;
                if (t < 192) {
                    const int which = t >> 6, d = t & 63;
                    const int src = (which == 0 ? h : which == 1 ? nq + g : nq + nkv + g) * 64 + d;
                    unsigned long long w = 0;
                    long long n = a.spin_start;
                    while (true) {
                        w = __hip_atomic_load((SHP_GLOBAL unsigned long long*)(a.qkv_tag + src),
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        if (__all((unsigned)(w >> 32) == epoch)) break;
                        __builtin_amdgcn_s_sleep(1);
                        if ((++n & 127) == 0) {
                            if (__hip_atomic_load((SHP_GLOBAL int*)a.abort_flag, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT) != 0 ||
                                n > a.spin_limit) {
                                if (lane == 0)
                                    __hip_atomic_store((SHP_GLOBAL int*)a.abort_flag, 1,
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                ok = 0;
                                break;
                            }
                        }
                    }
                    cur[which * 64 + d] = __uint_as_float((unsigned)w);
                }
                if (lane == 0) okw[wave] = ok;
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int f = t + NT * u, row = f >> 4, c4 = f & 15;
                if (row < nrows) {
                    *reinterpret_cast<float4*>(ks + row * KSTRIDE + c4 * 4) = k4[u];
                    *reinterpret_cast<float4*>(vs + row * 64 + c4 * 4) = v4[u];
                }
            }
            __syncthreads();
            if (t0 == 0) {
                int all = 1;
                for (int w = 0; w < NW; ++w) all &= okw[w];
                if (!all) return false;
                stamp(a, it, kb, 2);
            }
            float scale = 1.0f;
            if (wave == 0) {
                if (t0 == 0) {
                    const float q = cur[lane], k = cur[64 + lane];
                    vcur = cur[128 + lane];
                    const float qp = __shfl_xor(q, 32), kp = __shfl_xor(k, 32);
                    qr = q * cs + (lane < 32 ? -qp : qp) * sn;
                    kr = k * cs + (lane < 32 ? -kp : kp) * sn;
                    if (h % grp == 0) {
                        st_coh(kc + ((int64_t)g * S + pos) * 64 + lane, kr);
                        st_coh(vc + ((int64_t)g * S + pos) * 64 + lane, vcur);
                    }
                }
                if (nrows > 0) {
                    const bool valid = lane < nrows;
                    const float* krow = ks + lane * KSTRIDE;
                    float sc = 0.0f;
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const float4 kk = *reinterpret_cast<const float4*>(krow + 4 * i);
                        sc += lane_bcast(qr, 4 * i) * kk.x + lane_bcast(qr, 4 * i + 1) * kk.y +
                              lane_bcast(qr, 4 * i + 2) * kk.z + lane_bcast(qr, 4 * i + 3) * kk.w;
                    }
                    sc = valid ? sc * 0.125f : -FLT_MAX;
                    const float m_new = fmaxf(m, wave_max(sc));
                    scale = expf(m - m_new);
                    const float e = valid ? expf(sc - m_new) : 0.0f;
                    lsum = lsum * scale + wave_sum(e);
                    m = m_new;
                    pe[lane] = e;
                }
            }
            if (nrows > 0) {
                __syncthreads();
                // PV partial sums: wavefront w takes positions w*8 .. w*8+7 of the tile
                float acc = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int tt = wave * 8 + i;
                    if (tt < nrows) acc += pe[tt] * vs[tt * 64 + lane];
                }
                po[wave * 64 + lane] = acc;
                __syncthreads();
                if (wave == 0) {
                    float sum = 0.0f;
#pragma unroll
                    for (int w = 0; w < NW; ++w) sum += po[w * 64 + lane];
                    o = o * scale + sum;
                }
            }
            __syncthreads();  // the next tile's staging reuses ks / vs / cur
            if (t0 + 64 >= pos) break;
        }
        if (wave == 0) {  // the current position, last in the sum
            const float sc = wave_sum(qr * kr) * 0.125f;
            const float m_new = fmaxf(m, sc);
            const float scale = expf(m - m_new);
            const float e = expf(sc - m_new);
            st_coh(a.att + h * 64 + lane, (o * scale + e * vcur) / (lsum * scale + e));
        }
    }
    return true;
}

template <int JF>
__global__ __launch_bounds__(NT, 1) void decode_persistent_kernel(PersistArgs a) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int qd = a.n_heads * 64;
    float* scratch = lds;                                  // [NW] block sums
    int* okw = reinterpret_cast<int*>(lds + 16);           // [NW] barrier wait results
    float* best_v = lds + 32;                              // [NW] argmax staging
    int* best_i = reinterpret_cast<int*>(lds + 48);        // [NW]
    float* gu_rows = lds + 64;                             // [GU_ROWS] gate/up row results
    float* xs = lds + LDS_MISC;                            // [hidden] raw x of the last norm
    float4* xn = reinterpret_cast<float4*>(xs + a.hidden);  // [512] the phase's input vector
    float* region = reinterpret_cast<float*>(xn + NB * 64);
    float* kv_s = region;                                  // attention staging (B1)
    float4* stage = reinterpret_cast<float4*>(region);      // gate/up LDS chunks (B1 .. C)
    float4* act_s = reinterpret_cast<float4*>(region);      // the down phase's input (D)

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int b = blockIdx.x, G = gridDim.x;
    const int H = a.hidden, H4 = H / 4, F4 = a.ffn / 4, Q4 = qd / 4;
    const int qkv_rows = (a.n_heads + 2 * a.n_kv) * 64;
    int qa0, qa1, h0, h1, p0, p1, v0, v1;
    part(qkv_rows, b, G, qa0, qa1);
    part(H, b, G, h0, h1);
    // gate/up pairs: a workgroup with an attention head takes half of the others' share
    part_w(a.ffn, b, G, min(a.n_heads, G), 1, 2, p0, p1);
    part(a.vocab, b, G, v0, v1);

    float4 b0[NB], b1[NB], b2[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        b0[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        b1[i] = b0[i];
        b2[i] = b0[i];
    }
    unsigned long long target = a.bar_base;
    // uniform over the workgroup; readfirstlane lets the compiler keep them (and everything
    // derived from them) in scalar registers
    int pos = __builtin_amdgcn_readfirstlane(a.st->pos);
    int step = __builtin_amdgcn_readfirstlane(a.st->step);
    int token = __builtin_amdgcn_readfirstlane(a.forced_token >= 0 ? a.forced_token : a.st->token);

    const bool attn_wg = b < a.n_heads;  // this workgroup computes an attention head
    // The other workgroups stage gate/up chunks 0 and 1 in LDS (over the attention staging,
    // which they do not use) during the attention phase.
    const int nls = attn_wg ? 0 : 2;
    load_chunk(b0, a.layers[0].wqkv, H4, qa0, 0, qa1, a.zero_row);
    load_chunk(b1, a.layers[0].wqkv, H4, qa0 + 8, 0, qa1, a.zero_row);
    for (int it = 0; it < a.n_tokens; ++it) {
        const float* erow = a.embed + (int64_t)token * H;
        int kb = 0;  // barrier index within the token (profile only)
        for (int l = 0; l < a.n_layers; ++l) {
            const PersistLayer L = a.layers[l];
            const float* xin = l == 0 ? erow : a.x;
            Epi e{};
            // Prefetch schedule.  A CU streams ~30 GB/s with ~64 KB in flight; loads return in
            // issue order, so a load issued before a wait delays that wait's poll, and a load
            // issued before a phase's stores delays its barrier arrival.  The pipe is kept busy
            // through the short phases: qkv chunks 0-1 at the previous barrier, Wo at the
            // start of the qkv phase, gate/up 0-1 at the end of the qkv phase (or, for the
            // workgroups that compute attention, after attention), on the others gate/up 0-1
            // moved to LDS and 2-3 issued at the attention barrier, the next gate/up chunk at
            // the end of the Wo phase, down 0-1 at the gate/up barrier.
            // ---- A: qkv (at most two chunks, both resident) -------------------------------
            {
                NormIn xr = norm_load(xin, l != 0, H, L.attn_norm);
                load_chunk(b2, L.wo, Q4, h0, 0, h1, a.zero_row);
                norm_finish(xr, H, a.eps, scratch, xs, xn);
                e.out = a.qkv;
                e.tag = a.qkv_tag;
                e.epoch = (unsigned)(target + 1);
                const int w = wave_id();
                row_done<EPI_QKV>(chunk_dot(b0, xn), qa0 + w, qa1, e);
                row_done<EPI_QKV>(chunk_dot(b1, xn), qa0 + 8 + w, qa1, e);
            }
            // No grid barrier after the qkv phase: only attention consumes qkv, and it waits for
            // the tagged words of its head (the phase's epoch is used for the tags alone).
            stamp(a, it, kb, 0);
            if (!attn_wg) {
                load_chunk(b0, L.w_gu, H4, 2 * p0, 0, 2 * p1, a.zero_row);
                load_chunk(b1, L.w_gu, H4, 2 * p0 + 8, 0, 2 * p1, a.zero_row);
            }
            target += 1;
            stamp(a, it, kb++, 1);
            // ---- B1: attention, one workgroup per query head ------------------------------
            if (attn_wg && !attention_heads(a, l, pos, kv_s, it, kb, (unsigned)target, okw))
                return;
            stamp(a, it, kb, 0);
            bar_arrive(a.flags, target + 1);
            if (attn_wg) {
                load_chunk(b0, L.w_gu, H4, 2 * p0, 0, 2 * p1, a.zero_row);
                load_chunk(b1, L.w_gu, H4, 2 * p0 + 8, 0, 2 * p1, a.zero_row);
            } else {
                stage_chunk(stage, b0);
                load_chunk(b0, L.w_gu, H4, 2 * p0 + 16, 0, 2 * p1, a.zero_row);
                stage_chunk(stage + NB * NT, b1);
                load_chunk(b1, L.w_gu, H4, 2 * p0 + 24, 0, 2 * p1, a.zero_row);
            }
            target += 1;
            if (!bar_wait(a, target, okw)) return;
            stamp(a, it, kb++, 1);
            // ---- B2: Wo + residual (one chunk: h1 - h0 <= 8) ------------------------------
            {
                xn[t] = t < Q4 ? ld_coh4_at(a.att, (unsigned)t * 16u) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                __syncthreads();
                e.out = a.x;
                e.resid = xs;
                e.tag = a.x_tag;
                e.epoch = (unsigned)(target + 1);
                row_done<EPI_RESID>(chunk_dot(b2, xn), h0 + wave_id(), h1, e);
            }
            // No grid barrier: the gate/up phase waits for the tagged x words.
            stamp(a, it, kb, 0);
            load_chunk(b2, L.w_gu, H4, 2 * p0 + 8 * (nls + 2), 0, 2 * p1, a.zero_row);
            target += 1;
            stamp(a, it, kb++, 1);
            // ---- C: gate/up + SwiGLU ------------------------------------------------------
            {
                NormIn xr = norm_load_tagged(a, (unsigned)target, H, L.ffn_norm, okw);
                norm_finish(xr, H, a.eps, scratch, xs, xn);
                if (!all_ok(okw)) return;
                e.rows = gu_rows;
                e.row0 = 2 * p0;
                stream_rows_staged<EPI_SWIGLU>(L.w_gu, H4, 2 * p0, 2 * p1, nls, stage, xn, b0, b1,
                                               b2, e, a.zero_row);
                __syncthreads();  // every row result of the workgroup is in gu_rows
                for (int i = t; i < p1 - p0; i += NT) {
                    const float g = gu_rows[2 * i], u = gu_rows[2 * i + 1];
                    st_coh(a.act + p0 + i, (g * (1.0f / (1.0f + expf(-g)))) * u);
                }
            }
            stamp(a, it, kb, 0);
            bar_arrive(a.flags, target + 1);
            load_chunk(b0, L.w_down, F4, h0, 0, h1, a.zero_row);
            load_chunk(b1, L.w_down, F4, h0 + 8 * (1 / JF), 1 % JF, h1, a.zero_row);
            target += 1;
            if (!bar_wait(a, target, okw)) return;
            stamp(a, it, kb++, 1);
            // ---- D: down + residual -------------------------------------------------------
            {
#pragma unroll
                for (int jj = 0; jj < JF; ++jj) {
                    const int c = t + NT * jj;
                    act_s[c] = c < F4 ? ld_coh4_at(a.act, (unsigned)c * 16u) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
                __syncthreads();
                e.out = a.x;
                e.resid = xs;
                e.tag = a.x_tag;
                e.epoch = (unsigned)(target + 1);
                // one row group (h1 - h0 <= 8): JF segment chunks, summed in segment order
                if constexpr (JF <= 3) {
                    if constexpr (JF == 3) load_chunk(b2, L.w_down, F4, h0, 2, h1, a.zero_row);
                    float acc = chunk_dot(b0, act_s);
                    if constexpr (JF >= 2) acc += chunk_dot(b1, act_s + NB * 64);
                    if constexpr (JF == 3) acc += chunk_dot(b2, act_s + 2 * NB * 64);
                    row_done<EPI_RESID>(acc, h0 + wave_id(), h1, e);
                } else {
                    stream_rows<EPI_RESID, JF, 2>(L.w_down, F4, h0, h1, act_s, b0, b1, b2, e,
                                                  a.zero_row);
                }
            }
            stamp(a, it, kb, 0);
            bar_arrive(a.flags, target + 1);
            {
                // chunks 0-1 of the next layer's qkv, or of the lm_head
                const bool last = l + 1 == a.n_layers;
                const float* Wn = last ? a.lm_head : a.layers[last ? l : l + 1].wqkv;
                const int n0 = last ? v0 : qa0, n1 = last ? v1 : qa1;
                load_chunk(b0, Wn, H4, n0, 0, n1, a.zero_row);
                load_chunk(b1, Wn, H4, n0 + 8, 0, n1, a.zero_row);
            }
            target += 1;
            if (!bar_wait(a, target, okw)) return;
            stamp(a, it, kb++, 1);
        }
        // ---- E: lm_head + per-workgroup argmax ---------------------------------------------
        {
            NormIn xr = norm_load(a.x, true, H, a.final_norm);
            norm_finish(xr, H, a.eps, scratch, xs, xn);
            Epi e{};
            e.out = a.logits;
            e.best = -FLT_MAX;
            e.best_idx = 0x7fffffff;
            stream_rows<EPI_LOGITS, 1, 2>(a.lm_head, H4, v0, v1, xn, b0, b1, b2, e, a.zero_row);
            const int w = wave_id();
            if ((t & 63) == 0) {
                best_v[w] = e.best;
                best_i[w] = e.best_idx;
            }
            __syncthreads();
            if (t == 0) {
                float s = best_v[0];
                int idx = best_i[0];
                for (int q = 1; q < NW; ++q)
                    if (best_v[q] > s || (best_v[q] == s && best_i[q] < idx)) { s = best_v[q]; idx = best_i[q]; }
                const unsigned long long packed =
                    (unsigned long long)__float_as_uint(s) | ((unsigned long long)(unsigned)idx << 32);
                __hip_atomic_store(reinterpret_cast<unsigned long long*>(a.cand + b), packed,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();  // best_v / best_i are reused by the global argmax
        }
        stamp(a, it, kb, 0);
        bar_arrive(a.flags, target + 1);
        // qkv chunks of layer 0 for the next token (after the last token they go unused)
        load_chunk(b0, a.layers[0].wqkv, H4, qa0, 0, qa1, a.zero_row);
        load_chunk(b1, a.layers[0].wqkv, H4, qa0 + 8, 0, qa1, a.zero_row);
        target += 1;
        if (!bar_wait(a, target, okw)) return;
        stamp(a, it, kb++, 1);
        // ---- F: global argmax (lowest index on ties), redundantly in every workgroup ------
        {
            float s = -FLT_MAX;
            int idx = 0x7fffffff;
            for (int i = t; i < G; i += NT) {
                const unsigned long long packed =
                    __hip_atomic_load(reinterpret_cast<unsigned long long*>(a.cand + i),
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const float cv = __uint_as_float((unsigned)packed);
                const int ci = (int)(unsigned)(packed >> 32);
                if (cv > s || (cv == s && ci < idx)) { s = cv; idx = ci; }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                float os = __shfl_xor(s, o);
                int oi = __shfl_xor(idx, o);
                if (os > s || (os == s && oi < idx)) { s = os; idx = oi; }
            }
            if (lane == 0) {
                best_v[wave] = s;
                best_i[wave] = idx;
            }
            __syncthreads();
            s = best_v[0];
            idx = best_i[0];
            for (int w = 1; w < NW; ++w)
                if (best_v[w] > s || (best_v[w] == s && best_i[w] < idx)) { s = best_v[w]; idx = best_i[w]; }
            if (idx == 0x7fffffff) idx = 0;
            __syncthreads();
            if (b == 0 && t == 0) {
                a.st->token = idx;
                if (step < 4096) a.st->out_tokens[step] = idx;
                a.st->step = step + 1;
                a.st->pos = pos + 1;
            }
            token = __builtin_amdgcn_readfirstlane(idx);
            ++step;
            ++pos;
        }
    }
}

template <int JF>
const void* kernel_for() {
    return reinterpret_cast<const void*>(&decode_persistent_kernel<JF>);
}

const void* pick_kernel(int jf) {
    switch (jf) {
        case 1: return kernel_for<1>();
        case 2: return kernel_for<2>();
        case 3: return kernel_for<3>();
        case 4: return kernel_for<4>();
        default: return nullptr;
    }
}


size_t lds_bytes(const PersistArgs& a) {
    const int jf = (a.ffn / 4 + NT - 1) / NT;
    const size_t att = 64 * KSTRIDE + 64 * 64 + 4 * 64 + NW * 64;
    const size_t staged = 2 * NB * NT * 4;  // two gate/up chunks
    const size_t act = (size_t)jf * NB * 64 * 4;
    size_t region = att > staged ? att : staged;
    if (act > region) region = act;
    const size_t floats = LDS_MISC + (size_t)a.hidden + NB * 64 * 4 + region;
    return floats * sizeof(float);
}

}  // namespace

namespace shp {

int persist_plan(int device, PersistArgs* ap, int* grid, size_t* lds, std::string* why) {
    const PersistArgs& a = *ap;
    *grid = 0;
    *lds = 0;
    auto no = [&](const std::string& r) {
        if (why) *why = r;
        return SHP_OK;
    };
    const int qd = a.n_heads * 64;
    if (a.hidden % 4 || a.hidden / 4 > NT) return no("hidden must be a multiple of 4, <= 2048");
    if (qd / 4 > NT) return no("n_heads * 64 must be <= 2048");
    if (a.ffn % 4) return no("ffn must be a multiple of 4");
    const int jf = (a.ffn / 4 + NT - 1) / NT;
    if (!pick_kernel(jf)) return no("ffn must be <= 8192");
    if (a.n_kv <= 0 || a.n_heads % a.n_kv) return no("n_heads must be a multiple of n_kv");
    if (a.max_seq <= 0) return no("max_seq");
    int coop = 0, cus = 0;
    SHP_HIP_CHECK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, device));
    SHP_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
    if (!coop) return no("device has no cooperative launch");
    int max_lds = 0;
    SHP_HIP_CHECK(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device));
    const size_t bytes = lds_bytes(a);
    if (bytes > (size_t)max_lds) return no("LDS for hidden + heads exceeds the device limit");
    const void* k = pick_kernel(jf);
    if (bytes > 64 * 1024)
        SHP_HIP_CHECK(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    int per_cu = 0;
    SHP_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, NT, bytes));
    if (per_cu < 1) return no("persistent kernel does not fit on a CU");
    if (cus > NW * 64) return no("more CUs than barrier-flag pollers");
    if ((a.hidden + cus - 1) / cus > 8)
        return no("more than 8 hidden rows per workgroup (hidden > 8 x CUs)");
    if (((a.n_heads + 2 * a.n_kv) * 64 + cus - 1) / cus > 16)
        return no("more than 16 qkv rows per workgroup");
    {
        // gate/up rows per workgroup (the kernel's 1:2 split) must fit the LDS row buffer
        const int64_t na = std::min(a.n_heads, cus);
        auto cw = [&](int64_t i) { return i <= na ? i : na + 2 * (i - na); };
        const int64_t tot = cw(cus);
        for (int b = 0; b < cus; ++b) {
            const int64_t rows = 2 * ((int64_t)a.ffn * cw(b + 1) / tot - (int64_t)a.ffn * cw(b) / tot);
            if (rows > GU_ROWS) return no("too many gate/up rows per workgroup");
        }
    }
    *grid = cus;  // one workgroup per CU
    *lds = bytes;
    return SHP_OK;
}

int persist_launch(hipStream_t s, const PersistArgs& a, int grid, size_t lds) {
    const int jf = (a.ffn / 4 + NT - 1) / NT;
    const void* k = pick_kernel(jf);
    if (!k || grid <= 0) return fail(SHP_ERR_UNSUPPORTED, "persistent decode: not planned");
    PersistArgs arg = a;
    void* params[] = {&arg};
    SHP_HIP_CHECK(hipLaunchCooperativeKernel(k, dim3(grid), dim3(NT), params, (unsigned)lds, s));
    return SHP_OK;
}

}  // namespace shp
