// device_common.hpp -- gfx950 device helpers shared by the packed-matvec kernels.
//
// Exactness rules for everything in this directory:
//  * compiled without -ffast-math; f32 denormals and correctly rounded division
//    stay on (hipcc defaults), contraction is disabled (-ffp-contract=off) and
//    __builtin_fmaf appears only where the reference uses mul_add;
//  * integer block dots are exact int32 (v_dot4_i32_i8), in any order;
//  * the binary32 scale/accumulate chain of each output row runs serially in
//    block order in one lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prism {

// Kinds (src/kernels.rs:75-87; TQ1_0 / TQ2_0 src/kernels/tquants.rs:17-23).
constexpr uint32_t kQ8_0 = 8, kQ2_K = 10, kTQ1_0 = 34, kTQ2_0 = 35, kPQ2 = 142, kPTQ1 = 143;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Q8_K / Q8_0 activation blocks (tools/ternary/src/lib.rs:27-39, src/kernels.rs:528-535).
struct Q8KBlock {
    float scale;
    int8_t values[256];
    int16_t sums[16];
};
struct Q8Block {
    float scale;
    float sum;
    int8_t values[32];
};
static_assert(sizeof(Q8KBlock) == 292, "Q8_K layout");
static_assert(sizeof(Q8Block) == 40, "Q8_0 layout");

__device__ __forceinline__ bool finite(float v) { return (__float_as_uint(v) & 0x7f800000u) != 0x7f800000u; }

// Exact binary16 -> binary32 (v_cvt_f32_f16 is exact, subnormals included).
__device__ __forceinline__ float h2f(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}
// binary32 -> binary16 -> binary32 with ties to even (src/kernels.rs:2824-2830).
// The empty asm materializes the binary32 value first: otherwise the compiler folds a
// preceding binary32 multiply into the conversion (v_fma_mixlo_f16), which rounds the
// exact product once instead of rounding the binary32 product, and differs whenever
// that product lands exactly on a binary16 midpoint.
__device__ __forceinline__ float round_f16(float v) {
    asm volatile("" : "+v"(v));
    return static_cast<float>(static_cast<_Float16>(v));
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
// Bytes [lo.b2, lo.b3, hi.b0, hi.b1]: a dword starting two bytes into `lo`.
__device__ __forceinline__ uint32_t align2(uint32_t hi, uint32_t lo) { return __builtin_amdgcn_alignbyte(hi, lo, 2); }

// Raw buffer resource over [base, base+bytes): loads past the end return zero,
// so partial tiles can never fault.  Word 3 is the gfx9 raw-buffer format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}
__device__ __forceinline__ u32x4 bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0);
}
__device__ __forceinline__ u32x3 bload3(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b96(r, static_cast<int>(off), 0, 0);
}
__device__ __forceinline__ u32x2 bload2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(off), 0, 0);
}
__device__ __forceinline__ uint32_t bload1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, 0);
}

// ggml's vectorised expf polynomial, a published method restated by the reference at
// src/kernels/pinned_activations.rs:26-62, with the same explicit fused multiply-adds.
__device__ __forceinline__ float vector_exp(float value) {
    const float z = __builtin_fmaf(value, __uint_as_float(0x3fb8aa3bu), 12582912.0f);
    const float n = z - 12582912.0f;
    float r = __builtin_fmaf(-n, __uint_as_float(0x3f317200u), value);
    r = __builtin_fmaf(-n, __uint_as_float(0x35bfbe8eu), r);
    const uint32_t e = __float_as_uint(z) << 23;
    const float k = __uint_as_float(e + __float_as_uint(1.0f));
    const float sq = r * r;
    const float inner = __builtin_fmaf(__builtin_fmaf(__uint_as_float(0x3c072010u), r, __uint_as_float(0x3d2b9f17u)), sq,
                                       __builtin_fmaf(__uint_as_float(0x3e2aaf33u), r, __uint_as_float(0x3efffedbu)));
    const float poly = __builtin_fmaf(inner, sq, __uint_as_float(0x3f7ffff6u) * r);
    if (fabsf(n) > 126.0f) {
        const uint32_t shift = n <= 0.0f ? 0x82000000u : 0u;
        const float s1 = __uint_as_float(shift + 0x7f000000u);
        if (fabsf(n) > 192.0f) return s1 * s1;
        const float s2 = __uint_as_float(e - shift);
        return __builtin_fmaf(s2, poly, s2) * s1;
    }
    return __builtin_fmaf(poly, k, k);
}

// binary32 exp / cos / sin evaluated in binary64 and rounded once.  That is the
// correctly rounded result except when the exact value lies within the binary64
// error of a binary32 rounding boundary, so it agrees with the reference's libm
// (Rust's f32::exp / cos / sin, themselves within about half an ulp) far more often
// than the device's single-precision routines, which are within about one ulp.
__device__ __forceinline__ float exp_f32(float x) { return static_cast<float>(exp(static_cast<double>(x))); }
__device__ __forceinline__ float cos_f32(float x) { return static_cast<float>(cos(static_cast<double>(x))); }
__device__ __forceinline__ float sin_f32(float x) { return static_cast<float>(sin(static_cast<double>(x))); }

// One SwiGLU element, h = up * silu(gate).  Source order (src/graph.rs:121-131,
// src/kernels.rs:3365-3368): up * (g / (1 + exp(-g))).  Pinned order
// (src/kernels/pinned_activations.rs:141-178): (g * up) / (1 + vexp(0 - g)) for the
// first n/4*4 elements of the vector and (g * up) / (1 + exp(-g)) for the tail.
__device__ __forceinline__ float swiglu_one(float gate, float up, uint64_t i, uint64_t n, int pinned) {
    if (pinned) {
        const float den = 1.0f + (i < n / 4 * 4 ? vector_exp(0.0f - gate) : exp_f32(-gate));
        return (gate * up) / den;
    }
    const float silu = gate / (1.0f + exp_f32(-gate));
    return up * silu;
}

// A word read with a vector load.  The compiler turns a uniform read from memory that
// the kernel does not write into a scalar load, and scalar loads complete out of
// order: every later wait for a kernel argument would then wait for it as well.
__device__ __forceinline__ uint32_t vector_load(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void raise_error(int *flag, int bits) {
    if (flag) __hip_atomic_fetch_or(flag, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace prism
