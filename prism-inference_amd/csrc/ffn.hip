// ffn.hip -- FFN epilogue kernels: SwiGLU between gate/up and down, residual add.
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

int launch_fill_i32(int *p, int v, uint32_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_fill_i32, dim3((n + 63) / 64), dim3(64), 0, s, p, v, n);
    return launch_status();
}

}  // namespace prism
