// quant_dev.hpp -- wavefront-level activation quantizers (f32 -> Q8_K / Q8_0), bit-exact.
//
// Q8_K: src/kernels.rs:463-522 (+ pinned_q8k_integer :420-428).
// Q8_0: src/kernels.rs:552-617 (source / pinned generic / pinned PTQ1 native scale).
//
// Shared by the standalone quantize kernels and by the matvec prologues that
// quantize straight into LDS.  Each function is called by a whole wavefront with
// wave-uniform arguments and returns the error bits it found (wave-uniform).
// Blocks are spread wide over the lanes (16 lanes per Q8_K block, 2 per Q8_0
// block) so that most of the work is in-lane and the cross-lane reductions are
// only 4 (Q8_K) or 1 (Q8_0) shuffle steps deep.
#pragma once

#include "device_common.hpp"
#include "kernels.hpp"

namespace prism {

// Up to four Q8_K blocks (256 values each): block lane/16; lane s of a block owns
// elements 16s..16s+15, which is exactly bsums group s.  The block maximum is the
// FIRST element with the strictly greatest |x|, sign kept (src/kernels.rs:484-492),
// found by an (|x|, index) reduction with a lowest-index tie-break.
template <typename XPtr, typename OutPtr>
__device__ __forceinline__ int q8k_blocks_wave(XPtr x, uint32_t nblocks, int pinned, OutPtr o, uint32_t lane) {
    const uint32_t b = lane >> 4, s = lane & 15;
    const bool active = b < nblocks;
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
        if (active) q = reinterpret_cast<const float4 *>(x + 256 * b + 16 * s)[i];
        v[4 * i] = q.x;
        v[4 * i + 1] = q.y;
        v[4 * i + 2] = q.z;
        v[4 * i + 3] = q.w;
    }
    bool bad = false;
    float best = 0.0f, bval = 0.0f;
    int bidx = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        bad |= !finite(v[i]);
        const float a = fabsf(v[i]);
        if (a > best) {
            best = a;
            bidx = static_cast<int>(16 * s + i);
            bval = v[i];
        }
    }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) {
        const float ob = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(bidx, off, 64);
        const float ov = __shfl_xor(bval, off, 64);
        if (ob > best || (ob == best && oi < bidx)) {
            best = ob;
            bidx = oi;
            bval = ov;
        }
    }
    if (__any(bad)) return kErrInput;
    const float inv = best != 0.0f ? -127.0f / bval : 0.0f;
    if (__any(active && !finite(inv))) return kErrQuantRange;
    const float scale = best != 0.0f ? 1.0f / inv : 0.0f;
    uint32_t packed[4] = {0, 0, 0, 0};
    if (best != 0.0f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
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
            packed[i >> 2] |= (static_cast<uint32_t>(q) & 0xffu) << (8 * (i & 3));
        }
    }
    if (active) {
        int bs = 0;
        uint32_t *vals = reinterpret_cast<uint32_t *>(o[b].values) + 4 * s;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            bs = sdot4(packed[i], 0x01010101u, bs);
            vals[i] = packed[i];
        }
        o[b].sums[s] = static_cast<int16_t>(bs);
        if (s == 0) o[b].scale = scale;
    }
    return 0;
}

// Up to 32 Q8_0 blocks (32 values each): block lane/2, 16 values per lane.
template <typename XPtr, typename OutPtr>
__device__ __forceinline__ int q8_0_blocks_wave(XPtr x, uint32_t nblocks, int contract, OutPtr o, uint32_t lane) {
    const uint32_t b = lane >> 1, h = lane & 1;
    const bool active = b < nblocks;
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
        if (active) q = reinterpret_cast<const float4 *>(x + 32 * b + 16 * h)[i];
        v[4 * i] = q.x;
        v[4 * i + 1] = q.y;
        v[4 * i + 2] = q.z;
        v[4 * i + 3] = q.w;
    }
    bool bad = false;
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        bad |= !finite(v[i]);
        m = fmaxf(m, fabsf(v[i]));
    }
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    if (__any(bad)) return kErrInput;
    const bool pinned = contract != 0, native = contract == 2;
    const float d = native ? m * __uint_as_float(0x3c010204u) : m / 127.0f;
    const float inv = d == 0.0f ? 0.0f : (native ? 127.0f / m : 1.0f / d);
    uint32_t packed[4] = {0, 0, 0, 0};
    int qsum = 0;
    bool range = false;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float p = v[i] * inv;
        const float r = pinned ? __builtin_rintf(p) : __builtin_roundf(p);
        range |= !(r >= -127.0f && r <= 127.0f);
        const int q = static_cast<int>(r);
        qsum += q;
        packed[i >> 2] |= (static_cast<uint32_t>(q) & 0xffu) << (8 * (i & 3));
    }
    qsum += __shfl_xor(qsum, 1, 64);
    const float scale = round_f16(d);
    if (__any(active && (range || !finite(scale)))) return kErrQuantRange;
    if (active) {
        uint32_t *vals = reinterpret_cast<uint32_t *>(o[b].values) + 4 * h;
#pragma unroll
        for (int i = 0; i < 4; ++i) vals[i] = packed[i];
        if (h == 0) {
            o[b].scale = scale;
            o[b].sum = round_f16(static_cast<float>(qsum) * d);
        }
    }
    return 0;
}

}  // namespace prism
