// Device helpers shared by the kernels: fp16 decode, wavefront reductions, argmax keys.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tfk {

// Global-memory view of a pointer. A pointer read from LDS (or anywhere the compiler
// cannot trace to a kernel argument) is generic, and its accesses compile to FLAT
// instructions, which count in lgkmcnt as well as vmcnt: every later wait for an LDS
// access would also wait for them. Accessing through this view keeps them global.
#define TF_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ TF_GLOBAL T* gptr(T* p) {
    return (TF_GLOBAL T*)p;
}
template <class T>
__device__ __forceinline__ const TF_GLOBAL T* gptr(const T* p) {
    return (const TF_GLOBAL T*)p;
}
// 8- and 16-byte global loads (HIP's vector classes cannot be assigned from an
// address-space-qualified lvalue; clang's native vectors can).
typedef unsigned int tf_u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int tf_u32x4 __attribute__((ext_vector_type(4)));
typedef float tf_f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 gload_u2(const void* p) {
    const tf_u32x2 v = *(const TF_GLOBAL tf_u32x2*)p;
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint4 gload_u4(const void* p) {
    const tf_u32x4 v = *(const TF_GLOBAL tf_u32x4*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 gload_f4(const void* p) {
    const tf_f32x4 v = *(const TF_GLOBAL tf_f32x4*)p;
    return make_float4(v.x, v.y, v.z, v.w);
}

// Direct global -> LDS loads (global_load_lds), issued from inline assembly: lane i of a
// 16-byte load writes LDS at m0 + 16 i (4 i for a dword load), m0 saved and restored around
// it, with the one wait state gfx9 parts need between an SALU write of m0 and an LDS-DMA
// instruction (s_nop 0; the compiler's hazard recognizer does not look inside inline asm).
// Written as assembly so that the compiler does not count these loads: it would wait for
// all of them before every LDS read (it cannot tell the buffer a load targets); the kernel
// waits for them itself (s_waitcnt vmcnt with the count of its later loads).
__device__ __forceinline__ void lds_dma16(const TF_GLOBAL void* g, uint32_t m0) {
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(save)
                 : "s"(m0), "v"(g)
                 : "memory");
}
__device__ __forceinline__ void lds_dma4(const TF_GLOBAL void* g, uint32_t m0) {
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(save)
                 : "s"(m0), "v"(g)
                 : "memory");
}

// IEEE half bits -> float (v_cvt_f32_f16: exact for every half value).
__device__ __forceinline__ float h2f(uint32_t bits16) {
    _Float16 v;
    const uint16_t b = (uint16_t)bits16;
    __builtin_memcpy(&v, &b, 2);
    return (float)v;
}

// Unsigned byte n of a dword as float (v_cvt_f32_ubyte{0..3}).
__device__ __forceinline__ float ub0(uint32_t w) { return (float)(w & 0xFFu); }
__device__ __forceinline__ float ub1(uint32_t w) { return (float)((w >> 8) & 0xFFu); }
__device__ __forceinline__ float ub2(uint32_t w) { return (float)((w >> 16) & 0xFFu); }
__device__ __forceinline__ float ub3(uint32_t w) { return (float)(w >> 24); }
// Signed byte n of a dword as float (one v_cvt_f32_i32 with an SDWA sign-extended byte).
__device__ __forceinline__ float sb0(uint32_t w) { return (float)(int8_t)w; }
__device__ __forceinline__ float sb1(uint32_t w) { return (float)(int8_t)(w >> 8); }
__device__ __forceinline__ float sb2(uint32_t w) { return (float)(int8_t)(w >> 16); }
__device__ __forceinline__ float sb3(uint32_t w) { return (float)((int32_t)w >> 24); }

// DPP lane permutes within a row of 16 lanes (no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15 - i within 16

// Wavefront sum. Each step adds a value and its partner's, and both partners add the
// same two values, so every lane ends with the bit-identical total, independent of
// scheduling: DPP within rows of 16 lanes, then two cross-row exchanges.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppMirror>(v);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o);
    return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Wavefront max (exact in any order): DPP within rows of 16, then row_bcast:15 (row r's
// lane 15 into row r + 1, rows 1 and 3) and row_bcast:31 (lane 31 into rows 2 and 3), so
// lane 63 holds the maximum; it is read back as a uniform value. No LDS round trip.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<kDppXor1>(v));
    v = fmaxf(v, dpp<kDppXor2>(v));
    v = fmaxf(v, dpp<kDppHalfMirror>(v));
    v = fmaxf(v, dpp<kDppMirror>(v));
    const int ninf = __float_as_int(-INFINITY);
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x142, 0xA, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x143, 0xC, 0xF, false)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long w = __shfl_xor(v, o);
        v = w > v ? w : v;
    }
    return v;
}

// Argmax key: unsigned order of the key follows the float order of the value (with
// -0 folded onto +0, as `>` treats them equal) and, for equal values, the lower index
// (sample_greedy keeps the first maximum, sampler.cpp:8-13).
__device__ __forceinline__ unsigned long long argmax_key(float v, int64_t idx) {
    uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)b << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

}  // namespace tfk
