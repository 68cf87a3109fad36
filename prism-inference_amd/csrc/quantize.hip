// quantize.hip -- bit-exact GPU activation quantizers (f32 -> Q8_K / Q8_0).
//
// Q8_K: src/kernels.rs:463-522 (+ pinned_q8k_integer :420-428).
// Q8_0: src/kernels.rs:552-617 (source / pinned generic / pinned PTQ1 native scale).
//
// One wavefront quantizes one 256-element Q8_K block (4 values per lane) or
// eight 32-element Q8_0 blocks (8 lanes x 4 values per block).  Inputs are
// token-major [tokens][cols]; outputs are the reference's in-memory block
// structs, consumed directly by the matvec kernels.
#include "device_common.hpp"
#include "kernels.hpp"

namespace prism {

// --- Q8_K ------------------------------------------------------------------------
// Block maximum = the FIRST element with the strictly greatest |x| (sign kept),
// src/kernels.rs:484-492: reduce (|x|, index) with a lowest-index tie-break.
__global__ __launch_bounds__(256) void k_quantize_q8k(const float *__restrict__ x, uint32_t nblocks,
                                                      int pinned, Q8KBlock *__restrict__ out,
                                                      int *__restrict__ err) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t blk = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks) return;  // uniform per wavefront
    const float4 v4 = reinterpret_cast<const float4 *>(x + static_cast<size_t>(blk) * 256)[lane];
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    bool bad = false;
    float best = 0.0f;  // |value| of the running maximum
    int bidx = 0x7fffffff;
    for (int i = 0; i < 4; ++i) {
        bad |= !finite(v[i]);
        const float a = fabsf(v[i]);
        if (a > best) {
            best = a;
            bidx = static_cast<int>(lane * 4 + i);
        }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const float ob = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(bidx, off, 64);
        if (ob > best || (ob == best && oi < bidx)) {
            best = ob;
            bidx = oi;
        }
    }
    const bool anybad = __any(bad);
    Q8KBlock *o = out + blk;
    if (anybad) {
        if (lane == 0) raise_error(err, kErrInput);
        return;
    }
    uint32_t packed = 0;
    float scale = 0.0f;
    if (best != 0.0f) {
        const float maximum = x[static_cast<size_t>(blk) * 256 + bidx];
        const float inv = -127.0f / maximum;
        if (!finite(inv)) {
            if (lane == 0) raise_error(err, kErrQuantRange);
            return;
        }
        scale = 1.0f / inv;
        for (int i = 0; i < 4; ++i) {
            int q;
            if (pinned) {
                const float r = __builtin_fmaf(inv, v[i], 12582912.0f);
                q = static_cast<int>(__float_as_uint(r) & 0x7fffffu) - 0x400000;
                q = q > 127 ? 127 : q;
            } else {
                float r = __builtin_rintf(v[i] * inv);
                r = r > 127.0f ? 127.0f : r;
                q = static_cast<int>(r);
            }
            packed |= (static_cast<uint32_t>(q) & 0xffu) << (8 * i);
        }
    }
    // bsums: elements 16j..16j+15 live in lanes 4j..4j+3.
    int s = __builtin_amdgcn_sdot4(static_cast<int>(packed), 0x01010101, 0, false);
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    const int s_next = __shfl_down(s, 4, 64);
    reinterpret_cast<uint32_t *>(o->values)[lane] = packed;
    if (lane == 0) o->scale = scale;
    if ((lane & 7) == 0) {
        const uint32_t pair = (static_cast<uint32_t>(s) & 0xffffu) | (static_cast<uint32_t>(s_next) << 16);
        reinterpret_cast<uint32_t *>(o->sums)[lane >> 3] = pair;
    }
}

// --- Q8_0 ------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float *__restrict__ x, uint32_t nblocks,
                                                       int contract, Q8Block *__restrict__ out,
                                                       int *__restrict__ err) {
    const uint32_t t = blockIdx.x * 256 + threadIdx.x;
    const uint32_t blk = t >> 3, sub = t & 7;
    const bool active = blk < nblocks;
    float4 v4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (active) v4 = reinterpret_cast<const float4 *>(x + static_cast<size_t>(blk) * 32)[sub];
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    bool bad = false;
    float m = 0.0f;
    for (int i = 0; i < 4; ++i) {
        bad |= !finite(v[i]);
        m = fmaxf(m, fabsf(v[i]));
    }
    for (int off = 4; off >= 1; off >>= 1) {
        m = fmaxf(m, __shfl_xor(m, off, 64));
        bad |= __shfl_xor(static_cast<int>(bad), off, 64) != 0;
    }
    if (!active) return;
    if (bad) {
        if (sub == 0) raise_error(err, kErrInput);
        return;
    }
    const bool pinned = contract != 0, native = contract == 2;
    const float d = native ? m * __uint_as_float(0x3c010204u) : m / 127.0f;
    const float inv = d == 0.0f ? 0.0f : (native ? 127.0f / m : 1.0f / d);
    uint32_t packed = 0;
    int qsum = 0;
    bool range = false;
    for (int i = 0; i < 4; ++i) {
        const float p = v[i] * inv;
        const float r = pinned ? __builtin_rintf(p) : __builtin_roundf(p);
        range |= !(r >= -127.0f && r <= 127.0f);
        const int q = static_cast<int>(r);
        qsum += q;
        packed |= (static_cast<uint32_t>(q) & 0xffu) << (8 * i);
    }
    for (int off = 4; off >= 1; off >>= 1) {
        qsum += __shfl_xor(qsum, off, 64);
        range |= __shfl_xor(static_cast<int>(range), off, 64) != 0;
    }
    const float scale = round_f16(d);
    if (range || !finite(scale)) {
        if (sub == 0) raise_error(err, kErrQuantRange);
        return;
    }
    Q8Block *o = out + blk;
    reinterpret_cast<uint32_t *>(o->values)[sub] = packed;
    if (sub == 0) {
        o->scale = scale;
        o->sum = round_f16(static_cast<float>(qsum) * d);
    }
}

int launch_quantize_q8k(const float *x, uint64_t cols, uint32_t tokens, int pinned, void *out, int *err,
                        hipStream_t s) {
    const uint64_t nb = cols / 256 * tokens;
    if (nb == 0) return 0;
    hipLaunchKernelGGL(k_quantize_q8k, dim3(static_cast<uint32_t>((nb + 3) / 4)), dim3(256), 0, s, x,
                       static_cast<uint32_t>(nb), pinned, static_cast<Q8KBlock *>(out), err);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_quantize_q8_0(const float *x, uint64_t cols, uint32_t tokens, int contract, void *out, int *err,
                         hipStream_t s) {
    const uint64_t nb = cols / 32 * tokens;
    if (nb == 0) return 0;
    hipLaunchKernelGGL(k_quantize_q8_0, dim3(static_cast<uint32_t>((nb * 8 + 255) / 256)), dim3(256), 0, s, x,
                       static_cast<uint32_t>(nb), contract, static_cast<Q8Block *>(out), err);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace prism
