// Device-coherent global memory access for results that one workgroup writes and a
// workgroup on another XCD reads within the same launch (each XCD's L2 is not coherent with
// the others'): the split-K fixups of the dense kernels and of the fused block kernel.
#pragma once
#include <hip/hip_runtime.h>

#ifndef SHP_GLOBAL
#define SHP_GLOBAL __attribute__((address_space(1)))
#endif

typedef float f4v __attribute__((ext_vector_type(4)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));

// Agent-scope 16-byte store and load as two 8-byte relaxed atomics.
__device__ __forceinline__ void st_coh4(float* p, float4 v) {
    SHP_GLOBAL unsigned long long* q = (SHP_GLOBAL unsigned long long*)p;
    __hip_atomic_store(q, (unsigned long long)__float_as_uint(v.x) |
                              ((unsigned long long)__float_as_uint(v.y) << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, (unsigned long long)__float_as_uint(v.z) |
                                  ((unsigned long long)__float_as_uint(v.w) << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float4 ld_coh4(const float* p) {
    SHP_GLOBAL unsigned long long* q = (SHP_GLOBAL unsigned long long*)p;
    const unsigned long long lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long hi =
        __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float4(__uint_as_float((unsigned)lo), __uint_as_float((unsigned)(lo >> 32)),
                       __uint_as_float((unsigned)hi), __uint_as_float((unsigned)(hi >> 32)));
}

// Raw dword buffer resource word 3 for gfx9-family devices.
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const float* base, int64_t elems) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)(elems * 4), kBufferWord3);
}

// The same device-coherent 16-byte store and load as single buffer instructions with the
// agent-scope coherence bit (sc1), the bit the 8-byte agent-scope atomics above carry: one
// request per 16 bytes instead of two.  Byte offsets are 32-bit (ranges < 2 GiB).
constexpr int kCohSc1 = 16;  // cache-policy operand: sc1
__device__ __forceinline__ void st_coh16(__amdgpu_buffer_rsrc_t r, unsigned byte_off, float4 v) {
    const f4v x = {v.x, v.y, v.z, v.w};
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, x), r, byte_off, 0, kCohSc1);
}
__device__ __forceinline__ float4 ld_coh16(__amdgpu_buffer_rsrc_t r, unsigned byte_off,
                                           unsigned soff) {
    const f4v x = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, soff, kCohSc1));
    return make_float4(x.x, x.y, x.z, x.w);
}
