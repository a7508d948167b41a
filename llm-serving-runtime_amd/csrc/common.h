// Shared device types and host-side status helpers for libmxdecode (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "mxdecode.h"

namespace mx {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

// Thread-local message of the last failed ABI call (defined in status.hip).
void set_error(const char* fmt, ...);
void clear_error();

inline int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    set_error("%s", buf);
    return code;
}

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Checks the launch that was just enqueued.
inline int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(MX_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    return MX_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

__host__ __device__ constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Cross-lane butterflies on gfx950 row swaps. v_permlane16_swap_b32 exchanges
// the odd 16-lane rows of its first operand with the even rows of its second;
// v_permlane32_swap_b32 exchanges the upper 32 lanes of the first with the
// lower 32 of the second. Started from two copies of v, a symmetric op of the
// two outputs gives op(v[l], v[l^16]) / op(v[l], v[l^32]) in every lane. They
// are issued as inline asm with two distinct read-write operands: with one
// shared input value the compiler folds the builtin's second result into the
// first. The s_nop covers the VALU-write -> permlane-read hazard.
__device__ __forceinline__ void row_swap16(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void row_swap32(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// Sum / max over lanes l, l^16, l^32, l^48 (all lanes get the result).
__device__ __forceinline__ float xor_sum_16_32(float v) {
    float a = v, b = v;
    row_swap16(a, b);
    float c = a + b, d = a + b;
    row_swap32(c, d);
    return c + d;
}
__device__ __forceinline__ float xor_max_16_32(float v) {
    float a = v, b = v;
    row_swap16(a, b);
    float c = fmaxf(a, b), d = fmaxf(a, b);
    row_swap32(c, d);
    return fmaxf(c, d);
}
// Keeps v in an fp32 register, so a following fp16 conversion rounds the fp32 value
// instead of being folded with the arithmetic that produced v into one mixed-precision
// FMA (a single rounding). Kernels whose outputs must agree bit for bit round the same way.
__device__ __forceinline__ float pin_f32(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// silu(g) = g / (1 + e^-g) with the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32,
// about 1 ulp each): the SwiGLU product is rounded to fp16 right after, and the IEEE
// divide this library otherwise compiles to is several times longer. The result is pinned
// (pin_f32): callers round it to fp16 from fp32, as torch's fp16 SiLU does.
__device__ __forceinline__ float silu_f32(float g) {
    return pin_f32(g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f)));
}

// v + v[l^8] inside each 16-lane row (DPP row_ror:8).
__device__ __forceinline__ float xor8_sum(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
}

}  // namespace mx
