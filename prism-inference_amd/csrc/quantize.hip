// quantize.hip -- bit-exact GPU activation quantizers (f32 -> Q8_K / Q8_0).
//
// Q8_K: src/kernels.rs:463-522 (+ pinned_q8k_integer :420-428).
// Q8_0: src/kernels.rs:552-617 (source / pinned generic / pinned PTQ1 native scale).
//
// One wavefront quantizes four 256-element Q8_K blocks (16 lanes x 16 values per
// block) or 32 Q8_0 blocks (2 lanes x 16 values per block).  Inputs are
// token-major [tokens][cols]; outputs are the reference's in-memory block
// structs, consumed directly by the matvec kernels.
#include "device_common.hpp"
#include "kernels.hpp"
#include "quant_dev.hpp"

namespace prism {

// Four Q8_K blocks per wavefront, four wavefronts per workgroup.
__global__ __launch_bounds__(256) void k_quantize_q8k(const float *__restrict__ x, uint32_t nblocks, int pinned,
                                                      Q8KBlock *__restrict__ out, int *__restrict__ err) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t first = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 4;
    if (first >= nblocks) return;  // uniform per wavefront
    const uint32_t n = nblocks - first < 4 ? nblocks - first : 4;
    const int e = q8k_blocks_wave(x + static_cast<size_t>(first) * 256, n, pinned, out + first, lane);
    if (e && lane == 0) raise_error(err, e);
}

// 32 Q8_0 blocks per wavefront, four wavefronts per workgroup.
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float *__restrict__ x, uint32_t nblocks, int contract,
                                                       Q8Block *__restrict__ out, int *__restrict__ err) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t first = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 32;
    if (first >= nblocks) return;
    const uint32_t n = nblocks - first < 32 ? nblocks - first : 32;
    const int e = q8_0_blocks_wave(x + static_cast<size_t>(first) * 32, n, contract, out + first, lane);
    if (e && lane == 0) raise_error(err, e);
}

int launch_quantize_q8k(const float *x, uint64_t cols, uint32_t tokens, int pinned, void *out, int *err,
                        hipStream_t s) {
    const uint64_t nb = cols / 256 * tokens;
    if (nb == 0) return 0;
    hipLaunchKernelGGL(k_quantize_q8k, dim3(static_cast<uint32_t>((nb + 15) / 16)), dim3(256), 0, s, x,
                       static_cast<uint32_t>(nb), pinned, static_cast<Q8KBlock *>(out), err);
    return launch_status();
}

int launch_quantize_q8_0(const float *x, uint64_t cols, uint32_t tokens, int contract, void *out, int *err,
                         hipStream_t s) {
    const uint64_t nb = cols / 32 * tokens;
    if (nb == 0) return 0;
    hipLaunchKernelGGL(k_quantize_q8_0, dim3(static_cast<uint32_t>((nb + 127) / 128)), dim3(256), 0, s, x,
                       static_cast<uint32_t>(nb), contract, static_cast<Q8Block *>(out), err);
    return launch_status();
}

}  // namespace prism
