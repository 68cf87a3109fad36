// ffn.hip -- FFN epilogue kernels: SwiGLU between gate/up and down, the blockwise Hadamard
// rotation ahead of a rotated down projection, residual add, and the LoRA A dot beside the
// chain.
//
// Source order  (src/graph.rs:121-131, src/kernels.rs:3365-3368):
//     up = up * (g / (1 + exp(-g)))
// Pinned order  (src/kernels/pinned_activations.rs:141-178):
//     up = (g * up) / (1 + vexp(0 - g))   for the first n/4*4 elements,
//     up = (g * up) / (1 + exp(-g))       for the n%4 tail,
// where vexp is ggml's vectorised expf polynomial (a published method restated at
// src/kernels/pinned_activations.rs:26-62); it is evaluated here with the same
// explicit fused multiply-adds, so the pinned epilogue is bit-exact.  exp() is the
// device libm and matches the host's only to within its error bound.
#include <cmath>

#include "device_common.hpp"
#include "kernels.hpp"

namespace prism {

__global__ __launch_bounds__(256) void k_swiglu(const float *__restrict__ g, const float *__restrict__ u,
                                                float *__restrict__ h, uint64_t n, uint64_t total, int pinned,
                                                int *__restrict__ err) {
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) return;
    const uint64_t i = idx % n;
    const float r = swiglu_one(g[idx], u[idx], i, n, pinned);
    h[idx] = r;
    if (!finite(r)) raise_error(err, kErrNonfinite);
}

__global__ __launch_bounds__(256) void k_add_residual(float *__restrict__ out, const float *__restrict__ res,
                                                      uint64_t n, int *__restrict__ err) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = out[i] + res[i];
    out[i] = v;
    if (!finite(v)) raise_error(err, kErrNonfinite);
}

// lora_a_dot (src/kernels.rs:2336-2357): the rank-one LoRA A factor a dotted with the
// SwiGLU vector h (n values), one workgroup of 256 threads; *out receives the result.
//  - pinned with n % 16 == 0, pinned_gdn::dot_scalar (src/kernels/pinned_gdn.rs:205-230):
//    sixteen binary32 FMA chains, chain k = 4r + l over elements k, k+16, ... in order,
//    combined per lane l as (S_l + S_{8+l}) + (S_{4+l} + S_{12+l}), then (L0 + L1) + (L2 + L3).
//  - otherwise float_dot (src/kernels.rs:1256-1273): the binary32 products a_i * h_i summed
//    in binary64 in index order, rounded to binary32.  Every product is an integer multiple
//    of 2^e, e the smallest exponent of a unit in the last place among the nonzero
//    products, so when sum |p_i| <= 2^(52+e) every partial sum of any subset in any order
//    is exact in binary64 and the workgroup's tree sum is the ordered sum bit for bit.
//    Otherwise thread 0 sums the products in index order.
__global__ __launch_bounds__(256) void k_lora_dot(const float *__restrict__ a, const float *__restrict__ h,
                                                  uint32_t n, int pinned, float *__restrict__ out,
                                                  int *__restrict__ err) {
    __shared__ double red_s[4], red_m[4];
    __shared__ int red_e[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    if (pinned && n % 16 == 0) {
        if (wave != 0) return;  // uniform per wavefront; no barrier follows
        float s = 0.0f;
        if (lane < 16)
            for (uint32_t i = lane; i < n; i += 16) s = __builtin_fmaf(a[i], h[i], s);
        const float s4 = __shfl(s, lane + 4), s8 = __shfl(s, lane + 8), s12 = __shfl(s, lane + 12);
        const float l = (s + s8) + (s4 + s12);  // lanes 0..3
        const float l1 = __shfl(l, 1), l2 = __shfl(l, 2), l3 = __shfl(l, 3);
        if (lane == 0) {
            const float r = (l + l1) + (l2 + l3);
            *out = r;
            if (!finite(r)) raise_error(err, kErrNonfinite);
        }
        return;
    }
    double s = 0.0, mag = 0.0;
    int emin = 0x7fffffff;
    for (uint32_t i = tid; i < n; i += 256) {
        const float p = a[i] * h[i];
        s += static_cast<double>(p);
        mag += static_cast<double>(fabsf(p));
        if (p != 0.0f) {
            const int be = static_cast<int>((__float_as_uint(p) >> 23) & 0xffu);
            emin = min(emin, (be ? be : 1) - 150);
        }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        s += __shfl_xor(s, m);
        mag += __shfl_xor(mag, m);
        emin = min(emin, __shfl_xor(emin, m));
    }
    if (lane == 0) {
        red_s[wave] = s;
        red_m[wave] = mag;
        red_e[wave] = emin;
    }
    __syncthreads();
    if (tid != 0) return;
    s = (red_s[0] + red_s[1]) + (red_s[2] + red_s[3]);
    mag = (red_m[0] + red_m[1]) + (red_m[2] + red_m[3]);
    emin = min(min(red_e[0], red_e[1]), min(red_e[2], red_e[3]));
    const bool exact = emin == 0x7fffffff || mag <= ldexp(1.0, 52 + emin);
    if (!exact) {
        s = 0.0;
        for (uint32_t i = 0; i < n; ++i) s += static_cast<double>(a[i] * h[i]);
    }
    const float r = static_cast<float>(s);
    *out = r;
    if (!finite(r)) raise_error(err, kErrNonfinite);
}

// hadamard (src/kernels.rs:3952-3987) of every `block`-sized block of the SwiGLU rows,
// out of place: the butterfly stages half = 1, 2, 4, ... each replace (l, r) by (l + r,
// l - r) in binary32, then every value is multiplied by norm = 1 / sqrt(block) (binary32,
// computed by the caller as the reference does).  Each value of a stage depends only on the
// two values of the previous stage it pairs, so the result is the reference's bit for bit
// whatever thread computes it.  One workgroup per block (grid = blocks of all tokens), the
// block in LDS; non-finite inputs or outputs raise the error flag.
__global__ __launch_bounds__(1024) void k_hadamard(const float *__restrict__ in, float *__restrict__ out,
                                                   uint32_t block, float norm, int *__restrict__ err) {
    extern __shared__ float hv[];
    const size_t base = static_cast<size_t>(blockIdx.x) * block;
    bool bad = false;
    for (uint32_t i = threadIdx.x; i < block; i += blockDim.x) {
        const float v = in[base + i];
        bad |= !finite(v);
        hv[i] = v;
    }
    __syncthreads();
    for (uint32_t half = 1; half < block; half *= 2) {
        for (uint32_t p = threadIdx.x; p < block / 2; p += blockDim.x) {
            const uint32_t i = (p / half) * 2 * half + p % half;
            const float l = hv[i], r = hv[i + half];
            hv[i] = l + r;
            hv[i + half] = l - r;
        }
        __syncthreads();
    }
    for (uint32_t i = threadIdx.x; i < block; i += blockDim.x) {
        const float v = hv[i] * norm;
        bad |= !finite(v);
        out[base + i] = v;
    }
    if (bad) raise_error(err, kErrNonfinite);
}

__global__ void k_fill_i32(int *p, int v, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

int launch_swiglu(const float *gate, const float *up, float *h, uint64_t n, uint32_t tokens, int pinned, int *err,
                  hipStream_t s) {
    const uint64_t total = n * tokens;
    if (total == 0) return 0;
    hipLaunchKernelGGL(k_swiglu, dim3(static_cast<uint32_t>((total + 255) / 256)), dim3(256), 0, s, gate, up, h, n,
                       total, pinned, err);
    return launch_status();
}

int launch_add_residual(float *out, const float *residual, uint64_t n, int *err, hipStream_t s) {
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_add_residual, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, s, out, residual,
                       n, err);
    return launch_status();
}

int launch_lora_dot(const float *a, const float *h, uint32_t n, int pinned, float *out, int *err, hipStream_t s) {
    if (n == 0) return kLaunchUnsupported;
    hipLaunchKernelGGL(k_lora_dot, dim3(1), dim3(256), 0, s, a, h, n, pinned, out, err);
    return launch_status();
}

int launch_hadamard(const float *in, float *out, uint64_t n, uint32_t tokens, uint32_t block, int *err,
                    hipStream_t s) {
    if (block < 2 || (block & (block - 1)) || block > kHadamardMaxBlock || n % block) return kLaunchUnsupported;
    const uint64_t blocks = n / block * tokens;
    if (blocks == 0 || blocks > 0x7fffffffull) return kLaunchUnsupported;
    // The reference's normalization: 1 / sqrt(float(block)), each step rounded to binary32.
    const float norm = 1.0f / std::sqrt(static_cast<float>(block));
    const uint32_t threads = block / 2 < 1024 ? block / 2 : 1024;
    hipLaunchKernelGGL(k_hadamard, dim3(static_cast<uint32_t>(blocks)), dim3(threads), sizeof(float) * block, s, in,
                       out, block, norm, err);
    return launch_status();
}

int launch_fill_i32(int *p, int v, uint32_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_fill_i32, dim3((n + 63) / 64), dim3(64), 0, s, p, v, n);
    return launch_status();
}

}  // namespace prism
