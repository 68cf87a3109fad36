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
// only 4 (Q8_K) or 1 (Q8_0) DPP steps deep.
#pragma once

#include "device_common.hpp"
#include "kernels.hpp"

namespace prism {

// DPP lane exchanges within rows of 16 lanes (register speed, no LDS round trip).
// XOR masks 15, 7, 3 and 1 (row mirror, half-row mirror, two quad permutes) span
// the four lane-index bits, so a butterfly over them combines all 16 lanes.
constexpr int kDppRowMirror = 0x140, kDppHalfMirror = 0x141, kDppQuadRev = 0x1B, kDppQuadSwap = 0xB1;
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}

// One butterfly step of the (|x|, index, x) maximum: the lower index wins ties.
template <int CTRL>
__device__ __forceinline__ void max_step(float &best, int &bidx, float &bval) {
    const float ob = dpp_f<CTRL>(best), ov = dpp_f<CTRL>(bval);
    const int oi = dpp_i<CTRL>(bidx);
    const bool take = ob > best || (ob == best && oi < bidx);
    best = take ? ob : best;
    bidx = take ? oi : bidx;
    bval = take ? ov : bval;
}

// Up to four Q8_K blocks (256 values each): block lane/16; lane s of a block owns
// elements 16s..16s+15, which is exactly bsums group s.  The block maximum is the
// FIRST element with the strictly greatest |x|, sign kept (src/kernels.rs:484-492),
// found by an (|x|, index) reduction with a lowest-index tie-break.
// This lane's 16 inputs of a four-block Q8_K set (zeros past nblocks).
template <typename XPtr>
__device__ __forceinline__ void q8k_load(XPtr x, uint32_t nblocks, uint32_t lane, float (&v)[16]) {
    const uint32_t b = lane >> 4, s = lane & 15;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
        if (b < nblocks) q = reinterpret_cast<const float4 *>(x + 256 * b + 16 * s)[i];
        v[4 * i] = q.x;
        v[4 * i + 1] = q.y;
        v[4 * i + 2] = q.z;
        v[4 * i + 3] = q.w;
    }
}

template <typename OutPtr>
__device__ __forceinline__ int q8k_process(const float (&v)[16], uint32_t nblocks, int pinned, OutPtr o,
                                           uint32_t lane) {
    const uint32_t b = lane >> 4, s = lane & 15;
    const bool active = b < nblocks;
    bool bad = false;
    float best = 0.0f, bval = 0.0f;
    int bidx = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        bad |= !finite(v[i]);
        const float a = fabsf(v[i]);
        const bool take = a > best;
        best = take ? a : best;
        bidx = take ? static_cast<int>(16 * s + i) : bidx;
        bval = take ? v[i] : bval;
    }
    max_step<kDppRowMirror>(best, bidx, bval);
    max_step<kDppHalfMirror>(best, bidx, bval);
    max_step<kDppQuadRev>(best, bidx, bval);
    max_step<kDppQuadSwap>(best, bidx, bval);
    if (__any(bad)) return kErrInput;
    const float inv = best != 0.0f ? -127.0f / bval : 0.0f;
    if (__any(active && !finite(inv))) return kErrQuantRange;
    const float scale = best != 0.0f ? 1.0f / inv : 0.0f;
    uint32_t packed[4] = {0, 0, 0, 0};
    // inv == 0 (an all-zero block) yields all-zero codes in both contracts.
    if (pinned) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float r = __builtin_fmaf(inv, v[i], 12582912.0f);
            int q = static_cast<int>(__float_as_uint(r) & 0x7fffffu) - 0x400000;
            q = q > 127 ? 127 : q;
            packed[i >> 2] |= (static_cast<uint32_t>(q) & 0xffu) << (8 * (i & 3));
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float r = __builtin_rintf(v[i] * inv);
            r = r > 127.0f ? 127.0f : r;
            packed[i >> 2] |= (static_cast<uint32_t>(static_cast<int>(r)) & 0xffu) << (8 * (i & 3));
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

template <typename XPtr, typename OutPtr>
__device__ __forceinline__ int q8k_blocks_wave(XPtr x, uint32_t nblocks, int pinned, OutPtr o, uint32_t lane) {
    float v[16];
    q8k_load(x, nblocks, lane, v);
    return q8k_process(v, nblocks, pinned, o, lane);
}

// Up to 32 Q8_0 blocks (32 values each): block lane/2, 16 values per lane.
template <typename XPtr>
__device__ __forceinline__ void q8_0_load(XPtr x, uint32_t nblocks, uint32_t lane, float (&v)[16]) {
    const uint32_t b = lane >> 1, h = lane & 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
        if (b < nblocks) q = reinterpret_cast<const float4 *>(x + 32 * b + 16 * h)[i];
        v[4 * i] = q.x;
        v[4 * i + 1] = q.y;
        v[4 * i + 2] = q.z;
        v[4 * i + 3] = q.w;
    }
}

template <typename OutPtr>
__device__ __forceinline__ int q8_0_process(const float (&v)[16], uint32_t nblocks, int contract, OutPtr o,
                                            uint32_t lane) {
    const uint32_t b = lane >> 1, h = lane & 1;
    const bool active = b < nblocks;
    bool bad = false;
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        bad |= !finite(v[i]);
        m = fmaxf(m, fabsf(v[i]));
    }
    m = fmaxf(m, dpp_f<kDppQuadSwap>(m));
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
    qsum += dpp_i<kDppQuadSwap>(qsum);
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

template <typename XPtr, typename OutPtr>
__device__ __forceinline__ int q8_0_blocks_wave(XPtr x, uint32_t nblocks, int contract, OutPtr o, uint32_t lane) {
    float v[16];
    q8_0_load(x, nblocks, lane, v);
    return q8_0_process(v, nblocks, contract, o, lane);
}

// Element transforms applied to a lane's 16 consecutive inputs (first element index
// `first`) before they are quantized; `active` is false for lanes past the last block,
// which hold zeros and must not read the transform's own data.
struct NoPre {
    __device__ __forceinline__ void operator()(float (&)[16], uint32_t, bool) const {}
};
// RMSNorm in the reference's source order, (x * scale) * w (src/kernels.rs:3389-3418).
struct NormPre {
    const float *w;
    float scale;
    __device__ __forceinline__ void operator()(float (&v)[16], uint32_t first, bool active) const {
        if (!active) return;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 q = reinterpret_cast<const float4 *>(w + first)[i];
            v[4 * i] = (v[4 * i] * scale) * q.x;
            v[4 * i + 1] = (v[4 * i + 1] * scale) * q.y;
            v[4 * i + 2] = (v[4 * i + 2] * scale) * q.z;
            v[4 * i + 3] = (v[4 * i + 3] * scale) * q.w;
        }
    }
};

// A workgroup's prologue: quantizes the f32 vector x (cols values, global memory)
// into blocks `o` (LDS).  Wavefront w takes block sets w, w + nwaves, ...; the next
// set's loads are issued before the current one is processed, so the global reads
// cost one round trip, not one per set.  `pre` transforms the inputs first.
// Returns the error bits seen.
template <bool Q8K, typename OutPtr, typename Pre = NoPre>
__device__ __forceinline__ int quantize_prologue(const float *__restrict__ x, uint32_t cols, int contract, OutPtr o,
                                                 uint32_t wave, uint32_t nwaves, uint32_t lane, const Pre &pre = Pre{}) {
    constexpr uint32_t per_set = Q8K ? 4 : 32, blk = Q8K ? 256 : 32;
    const uint32_t nb = cols / blk;
    uint32_t b = per_set * wave;
    if (b >= nb) return 0;
    int e = 0;
    float v[16];
    auto load = [&](uint32_t at, float (&dst)[16]) {
        const uint32_t n = nb - at < per_set ? nb - at : per_set;
        if constexpr (Q8K)
            q8k_load(x + static_cast<size_t>(blk) * at, n, lane, dst);
        else
            q8_0_load(x + static_cast<size_t>(blk) * at, n, lane, dst);
    };
    // This lane's block within a set and the index of its first input.
    const uint32_t lb = Q8K ? lane >> 4 : lane >> 1;
    const uint32_t lo = Q8K ? 16u * (lane & 15u) : 16u * (lane & 1u);
    load(b, v);
    while (true) {
        const uint32_t nxt = b + per_set * nwaves;
        float vn[16];
        if (nxt < nb) load(nxt, vn);
        const uint32_t n = nb - b < per_set ? nb - b : per_set;
        pre(v, blk * (b + lb) + lo, lb < n);
        if constexpr (Q8K)
            e |= q8k_process(v, n, contract, o + b, lane);
        else
            e |= q8_0_process(v, n, contract, o + b, lane);
        if (nxt >= nb) break;
        b = nxt;
        for (int i = 0; i < 16; ++i) v[i] = vn[i];
    }
    return e;
}

// A workgroup's input held in registers for the quantizing prologue: wavefront w
// holds the block sets w, w + nwaves, ... (at most S of them) of the f32 vector x and,
// for an RMSNorm ahead of the quantizer, the matching norm weights.  load() issues
// every read at once (at the top of a kernel, before anything else waits on memory);
// sumsq() and quantize() then work from registers, so the prologue costs one memory
// round trip instead of one for the norm's sum and another for the quantizer.  The
// quantized result is bit-identical to quantize_prologue's for the same scale.
template <bool Q8K, uint32_t S>
struct HeldInput {
    static constexpr uint32_t per_set = Q8K ? 4 : 32, blk = Q8K ? 256 : 32;
    float v[S][16];
    float w[S][16];

    // Block sets of `cols` inputs and whether nwaves wavefronts can hold them all.
    __host__ __device__ static uint32_t sets(uint32_t cols) { return (cols / blk + per_set - 1) / per_set; }
    __host__ __device__ static bool fits(uint32_t cols, uint32_t nwaves) {
        return (sets(cols) + nwaves - 1) / nwaves <= S;
    }

    // nw: the norm weights, or x itself when there is no norm (read, never used).
    // Lanes past the last block read the last block (zeroed afterwards), so the loads
    // carry no branches for the compiler to wait on.
    __device__ __forceinline__ void load(const float *__restrict__ x, const float *__restrict__ nw, uint32_t cols,
                                         uint32_t wave, uint32_t nwaves, uint32_t lane) {
        const uint32_t nb = cols / blk;
        const uint32_t lb = Q8K ? lane >> 4 : lane >> 1, lo = Q8K ? 16u * (lane & 15u) : 16u * (lane & 1u);
#pragma unroll
        for (uint32_t j = 0; j < S; ++j) {
            const uint32_t b = per_set * (wave + j * nwaves) + lb, bc = b < nb ? b : nb - 1;
            const float4 *xs = reinterpret_cast<const float4 *>(x + static_cast<size_t>(blk) * bc + lo);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 q = xs[i];
                v[j][4 * i] = q.x;
                v[j][4 * i + 1] = q.y;
                v[j][4 * i + 2] = q.z;
                v[j][4 * i + 3] = q.w;
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < S; ++j) {
            const uint32_t b = per_set * (wave + j * nwaves) + lb, bc = b < nb ? b : nb - 1;
            const float4 *ws = reinterpret_cast<const float4 *>(nw + static_cast<size_t>(blk) * bc + lo);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 q = ws[i];
                w[j][4 * i] = q.x;
                w[j][4 * i + 1] = q.y;
                w[j][4 * i + 2] = q.z;
                w[j][4 * i + 3] = q.w;
            }
        }
    }

    // Zeroes the lanes past the last block.  Called when the values are first used, not
    // in load(): a use right after the reads would wait for them there.
    __device__ __forceinline__ void mask(uint32_t cols, uint32_t wave, uint32_t nwaves, uint32_t lane) {
        const uint32_t nb = cols / blk, lb = Q8K ? lane >> 4 : lane >> 1;
#pragma unroll
        for (uint32_t j = 0; j < S; ++j)
            if (per_set * (wave + j * nwaves) + lb >= nb)
#pragma unroll
                for (int i = 0; i < 16; ++i) v[j][i] = 0.0f;
    }

    // This lane's binary64 sum of the binary32 squares of its inputs (after mask()).
    __device__ __forceinline__ double sumsq() const {
        double s = 0.0;
#pragma unroll
        for (uint32_t j = 0; j < S; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i) s += static_cast<double>(v[j][i] * v[j][i]);
        return s;
    }

    // Quantizes the held sets (after mask()) into `o` (LDS); `norm` applies the RMSNorm
    // (x * scale) * w first.  Returns the error bits seen.
    template <typename OutPtr>
    __device__ __forceinline__ int quantize(uint32_t cols, int contract, OutPtr o, uint32_t wave, uint32_t nwaves,
                                            uint32_t lane, bool norm, float scale) {
        const uint32_t nb = cols / blk;
        const uint32_t lb = Q8K ? lane >> 4 : lane >> 1;
        int e = 0;
#pragma unroll
        for (uint32_t j = 0; j < S; ++j) {
            const uint32_t b0 = per_set * (wave + j * nwaves);
            if (b0 >= nb) break;
            const uint32_t n = nb - b0 < per_set ? nb - b0 : per_set;
            if (norm && lb < n)
#pragma unroll
                for (int i = 0; i < 16; ++i) v[j][i] = (v[j][i] * scale) * w[j][i];
            if constexpr (Q8K)
                e |= q8k_process(v[j], n, contract, o + b0, lane);
            else
                e |= q8_0_process(v[j], n, contract, o + b0, lane);
        }
        return e;
    }
};

// RMSNorm scale of x[0..n) over a whole workgroup (rms_norm_scale_inner,
// src/kernels.rs:3823-3878): binary64 sum of the binary32 squares, mean rounded to
// binary32, 1 / sqrt(mean + eps).  Threads sum strided elements, wavefronts reduce
// with cross-lane shuffles and wavefront 0 folds the wavefront sums in order, so
// only the order of the binary64 additions differs from the reference's sequential
// sum.  `red` is LDS scratch for 16 doubles.  Returns a non-positive or non-finite
// scale as 0 (the caller raises the error); every thread gets the same value.
__device__ __forceinline__ float rms_scale_wg(const float *__restrict__ x, uint32_t n, float eps, double *red) {
    // Eight strided loads in flight before the first is summed: the reduction costs
    // one memory round trip per eight elements of a thread, not one per element.
    double s = 0.0;
    for (uint32_t i0 = threadIdx.x; i0 < n; i0 += 8 * blockDim.x) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t i = i0 + k * blockDim.x;
            v[k] = i < n ? x[i] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (i0 + k * blockDim.x < n) s += static_cast<double>(v[k] * v[k]);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
    const uint32_t wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63u) == 0) red[wave] = s;
    __syncthreads();
    double t = 0.0;
    for (uint32_t w = 0; w < nw; ++w) t += red[w];
    __syncthreads();
    const float mean = static_cast<float>(t / static_cast<double>(n));
    const float scale = 1.0f / __builtin_sqrtf(mean + eps);
    return (finite(scale) && scale > 0.0f) ? scale : 0.0f;
}

}  // namespace prism
