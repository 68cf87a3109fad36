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

#include <type_traits>

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
    auto code = [&](int i, float r) {
        range |= !(r >= -127.0f && r <= 127.0f);
        const int q = static_cast<int>(r);
        qsum += q;
        packed[i >> 2] |= (static_cast<uint32_t>(q) & 0xffu) << (8 * (i & 3));
    };
    if (pinned) {
#pragma unroll
        for (int i = 0; i < 16; ++i) code(i, __builtin_rintf(v[i] * inv));
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) code(i, __builtin_roundf(v[i] * inv));
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

// Cross-lane steps of the register-held quantizer.  xor 1 and xor 2 are quad
// permutes, the two mirrors pair lanes within 8 and 16, and lanes 16 and 32 apart
// are reached with LDS-routed shuffles.  Each step combines a lane with one partner;
// a sequence of steps whose partner patterns span the lane-index bits 0..k-1 leaves
// every lane of an aligned group of 2^k lanes with the group's combined value.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E;

// Maximum and sum over the 64 lanes of a wavefront, every lane getting the result:
// four DPP steps within each row of 16 lanes (register speed), then two shuffles
// across rows.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u), CTRL, 0xF, 0xF, false));
    const uint32_t hi =
        static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u >> 32), CTRL, 0xF, 0xF, false));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ float wave_max(float m) {
    m = fmaxf(m, dpp_f<kDppXor1>(m));
    m = fmaxf(m, dpp_f<kDppXor2>(m));
    m = fmaxf(m, dpp_f<kDppHalfMirror>(m));
    m = fmaxf(m, dpp_f<kDppRowMirror>(m));
    m = fmaxf(m, __shfl_xor(m, 16));
    return fmaxf(m, __shfl_xor(m, 32));
}
__device__ __forceinline__ double wave_sum(double s) {
    s += dpp_d<kDppXor1>(s);
    s += dpp_d<kDppXor2>(s);
    s += dpp_d<kDppHalfMirror>(s);
    s += dpp_d<kDppRowMirror>(s);
    s += __shfl_xor(s, 16);
    s += __shfl_xor(s, 32);
    return s;
}

// A workgroup's input held in registers for the quantizing prologue.  The input is
// cut into chunks of 64*E values; wavefront w holds chunks w, w + nwaves, ... (at
// most S), lane l the E consecutive values l*E.. of each chunk, and, for an RMSNorm
// ahead of the quantizer, the matching norm weights.  load() issues every read at
// once (at the top of a kernel, before anything else waits on memory); sumsq() and
// quantize() then work from registers.  A Q8_0 block spans 32/E lanes and a Q8_K
// block 256/E lanes; their maxima, code sums and bsums are combined across those
// lanes, so the blocks written are bit-identical to q8_0_process / q8k_process's
// (src/kernels.rs:463-522, 552-617) for the same input.
template <bool Q8K, uint32_t E, uint32_t S>
struct HeldInput {
    static_assert(E == 4 || E == 8 || E == 16, "values per lane");
    static constexpr uint32_t blk = Q8K ? 256 : 32, lpb = blk / E, chunk = 64 * E;
    float v[S][E];
    float w[S][E];

    __host__ __device__ static bool fits(uint32_t cols, uint32_t nwaves) {
        return cols % blk == 0 && (cols + chunk - 1) / chunk <= S * nwaves;
    }

    // nw: the norm weights, or x itself when there is no norm (read, never used).
    // Lanes past the end read the last E values (masked later), so the loads carry no
    // branches for the compiler to wait on.
    __device__ __forceinline__ void load(const float *__restrict__ x, const float *__restrict__ nw, uint32_t cols,
                                         uint32_t wave, uint32_t nwaves, uint32_t lane) {
#pragma unroll
        for (uint32_t j = 0; j < S; ++j) {
            const uint32_t e = (wave + j * nwaves) * chunk + lane * E, ec = e < cols ? e : cols - E;
            const float4 *xs = reinterpret_cast<const float4 *>(x + ec);
#pragma unroll
            for (uint32_t i = 0; i < E / 4; ++i) {
                const float4 q = xs[i];
                v[j][4 * i] = q.x;
                v[j][4 * i + 1] = q.y;
                v[j][4 * i + 2] = q.z;
                v[j][4 * i + 3] = q.w;
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < S; ++j) {
            const uint32_t e = (wave + j * nwaves) * chunk + lane * E, ec = e < cols ? e : cols - E;
            const float4 *ws = reinterpret_cast<const float4 *>(nw + ec);
#pragma unroll
            for (uint32_t i = 0; i < E / 4; ++i) {
                const float4 q = ws[i];
                w[j][4 * i] = q.x;
                w[j][4 * i + 1] = q.y;
                w[j][4 * i + 2] = q.z;
                w[j][4 * i + 3] = q.w;
            }
        }
    }

    // Zeroes the values past the end.  Called when the values are first used, not in
    // load(): a use right after the reads would wait for them there.
    __device__ __forceinline__ void mask(uint32_t cols, uint32_t wave, uint32_t nwaves, uint32_t lane) {
#pragma unroll
        for (uint32_t j = 0; j < S; ++j)
            if ((wave + j * nwaves) * chunk + lane * E >= cols)
#pragma unroll
                for (uint32_t i = 0; i < E; ++i) v[j][i] = 0.0f;
    }

    // This lane's binary64 sum of the binary32 squares of its inputs (after mask()).
    __device__ __forceinline__ double sumsq() const {
        double s = 0.0;
#pragma unroll
        for (uint32_t j = 0; j < S; ++j)
#pragma unroll
            for (uint32_t i = 0; i < E; ++i) s += static_cast<double>(v[j][i] * v[j][i]);
        return s;
    }

    template <typename T, typename F>
    __device__ __forceinline__ static T across(T x, F op) {  // combine over the lpb lanes of a block
        if constexpr (sizeof(T) == 4) {
            auto step = [&](auto dpp) {
                const int o = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(dpp)::value, 0xF,
                                                          0xF, false);
                x = op(x, __builtin_bit_cast(T, o));
            };
            if constexpr (lpb >= 2) step(std::integral_constant<int, kDppXor1>{});
            if constexpr (lpb >= 4) step(std::integral_constant<int, kDppXor2>{});
            if constexpr (lpb >= 8) step(std::integral_constant<int, kDppHalfMirror>{});
            if constexpr (lpb >= 16) step(std::integral_constant<int, kDppRowMirror>{});
            if constexpr (lpb >= 32) x = op(x, __shfl_xor(x, 16));
            if constexpr (lpb >= 64) x = op(x, __shfl_xor(x, 32));
        }
        return x;
    }

    // (|x|, index, x) maximum over a block's lanes, lowest index first among equals.
    template <int CTRL>
    __device__ __forceinline__ static void max_dpp(float &best, int &bidx, float &bval) {
        max_step<CTRL>(best, bidx, bval);
    }
    __device__ __forceinline__ static void max_shfl(float &best, int &bidx, float &bval, int m) {
        const float ob = __shfl_xor(best, m), ov = __shfl_xor(bval, m);
        const int oi = __shfl_xor(bidx, m);
        const bool take = ob > best || (ob == best && oi < bidx);
        best = take ? ob : best;
        bidx = take ? oi : bidx;
        bval = take ? ov : bval;
    }

    // Quantizes the held chunks (after mask()) into `o` (LDS); `norm` applies the
    // RMSNorm (x * scale) * w first.  Returns the error bits seen.
    template <typename OutPtr>
    __device__ __forceinline__ int quantize(uint32_t cols, int contract, OutPtr o, uint32_t wave, uint32_t nwaves,
                                            uint32_t lane, bool norm, float scale) {
        int e = 0;
        const uint32_t sub = lane % lpb;  // this lane's place within its block
#pragma unroll
        for (uint32_t j = 0; j < S; ++j) {
            const uint32_t c0 = (wave + j * nwaves) * chunk;
            if (c0 >= cols) break;  // wave-uniform
            const uint32_t first = c0 + lane * E;
            const bool active = first < cols;
            const uint32_t b = first / blk;
            float *vj = v[j];
            if (norm && active)
#pragma unroll
                for (uint32_t i = 0; i < E; ++i) vj[i] = (vj[i] * scale) * w[j][i];
            bool bad = false;
#pragma unroll
            for (uint32_t i = 0; i < E; ++i) bad |= !finite(vj[i]);
            if (__any(bad)) return e | kErrInput;
            uint32_t packed[E / 4];
#pragma unroll
            for (uint32_t i = 0; i < E / 4; ++i) packed[i] = 0;
            if constexpr (Q8K) {
                // q8k_with_input (src/kernels.rs:463-522): the first element with the
                // strictly largest |x| sets inv = -127 / x.
                float best = 0.0f, bval = 0.0f;
                int bidx = 0x7fffffff;
#pragma unroll
                for (uint32_t i = 0; i < E; ++i) {
                    const float a = fabsf(vj[i]);
                    const bool take = a > best;
                    best = take ? a : best;
                    bidx = take ? static_cast<int>(sub * E + i) : bidx;
                    bval = take ? vj[i] : bval;
                }
                if constexpr (lpb >= 2) max_dpp<kDppXor1>(best, bidx, bval);
                if constexpr (lpb >= 4) max_dpp<kDppXor2>(best, bidx, bval);
                if constexpr (lpb >= 8) max_dpp<kDppHalfMirror>(best, bidx, bval);
                if constexpr (lpb >= 16) max_dpp<kDppRowMirror>(best, bidx, bval);
                if constexpr (lpb >= 32) max_shfl(best, bidx, bval, 16);
                if constexpr (lpb >= 64) max_shfl(best, bidx, bval, 32);
                const float inv = best != 0.0f ? -127.0f / bval : 0.0f;
                if (__any(active && !finite(inv))) return e | kErrQuantRange;
                const float qscale = best != 0.0f ? 1.0f / inv : 0.0f;
                if (contract) {
#pragma unroll
                    for (uint32_t i = 0; i < E; ++i) {
                        const float r = __builtin_fmaf(inv, vj[i], 12582912.0f);
                        int q = static_cast<int>(__float_as_uint(r) & 0x7fffffu) - 0x400000;
                        q = q > 127 ? 127 : q;
                        packed[i >> 2] |= (static_cast<uint32_t>(q) & 0xffu) << (8 * (i & 3));
                    }
                } else {
#pragma unroll
                    for (uint32_t i = 0; i < E; ++i) {
                        float r = __builtin_rintf(vj[i] * inv);
                        r = r > 127.0f ? 127.0f : r;
                        packed[i >> 2] |= (static_cast<uint32_t>(static_cast<int>(r)) & 0xffu) << (8 * (i & 3));
                    }
                }
                // bsums group g = 16 values = 16/E lanes (or a part of one lane's E).
                int bs = 0;
#pragma unroll
                for (uint32_t i = 0; i < E / 4; ++i) bs = sdot4(packed[i], 0x01010101u, bs);
                if constexpr (E == 4) {
                    bs += __builtin_bit_cast(int, __builtin_amdgcn_update_dpp(0, bs, kDppXor1, 0xF, 0xF, false));
                    bs += __builtin_bit_cast(int, __builtin_amdgcn_update_dpp(0, bs, kDppXor2, 0xF, 0xF, false));
                } else if constexpr (E == 8) {
                    bs += __builtin_bit_cast(int, __builtin_amdgcn_update_dpp(0, bs, kDppXor1, 0xF, 0xF, false));
                }
                if (active) {
                    uint32_t *vals = reinterpret_cast<uint32_t *>(o[b].values) + sub * (E / 4);
#pragma unroll
                    for (uint32_t i = 0; i < E / 4; ++i) vals[i] = packed[i];
                    if constexpr (E == 16) {
                        o[b].sums[sub] = static_cast<int16_t>(bs);
                    } else {
                        if (sub % (16 / E) == 0) o[b].sums[sub / (16 / E)] = static_cast<int16_t>(bs);
                    }
                    if (sub == 0) o[b].scale = qscale;
                }
            } else {
                // q8_with_input (src/kernels.rs:552-617), contracts as in q8_0_process.
                float m = 0.0f;
#pragma unroll
                for (uint32_t i = 0; i < E; ++i) m = fmaxf(m, fabsf(vj[i]));
                m = across(m, [](float a, float c) { return fmaxf(a, c); });
                const bool pinned = contract != 0, native = contract == 2;
                const float d = native ? m * __uint_as_float(0x3c010204u) : m / 127.0f;
                const float inv = d == 0.0f ? 0.0f : (native ? 127.0f / m : 1.0f / d);
                int qsum = 0;
                bool range = false;
                auto code = [&](uint32_t i, float r) {
                    range |= !(r >= -127.0f && r <= 127.0f);
                    const int q = static_cast<int>(r);
                    qsum += q;
                    packed[i >> 2] |= (static_cast<uint32_t>(q) & 0xffu) << (8 * (i & 3));
                };
                // One loop per rounding (half-even pinned, half-away source): a select
                // inside one loop would evaluate both roundings of every value.
                if (pinned) {
#pragma unroll
                    for (uint32_t i = 0; i < E; ++i) code(i, __builtin_rintf(vj[i] * inv));
                } else {
#pragma unroll
                    for (uint32_t i = 0; i < E; ++i) code(i, __builtin_roundf(vj[i] * inv));
                }
                qsum = across(qsum, [](int a, int c) { return a + c; });
                const float qscale = round_f16(d);
                if (__any(active && (range || !finite(qscale)))) return e | kErrQuantRange;
                if (active) {
                    uint32_t *vals = reinterpret_cast<uint32_t *>(o[b].values) + sub * (E / 4);
#pragma unroll
                    for (uint32_t i = 0; i < E / 4; ++i) vals[i] = packed[i];
                    if (sub == 0) {
                        o[b].scale = qscale;
                        o[b].sum = round_f16(static_cast<float>(qsum) * d);
                    }
                }
            }
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

// One Q8_0 block per 32 lanes with one value per lane (lane j of a 32-lane half holds
// element j): q8_with_input's arithmetic (src/kernels.rs:552-617, as q8_0_process), the
// block maximum and code sum combined across the 32 lanes.  Every lane of the wavefront
// calls it; lanes with own == false hold 0 and write nothing.  Returns this lane's
// error bits.
__device__ __forceinline__ int q8_0_lanes32(float v, bool own, int contract, Q8Block *blk, uint32_t j) {
    const bool bad = own && !finite(v);
    float m = fabsf(v);
    m = fmaxf(m, dpp_f<kDppXor1>(m));
    m = fmaxf(m, dpp_f<kDppXor2>(m));
    m = fmaxf(m, dpp_f<kDppHalfMirror>(m));
    m = fmaxf(m, dpp_f<kDppRowMirror>(m));
    m = fmaxf(m, __shfl_xor(m, 16));
    const bool pinned = contract != 0, native = contract == 2;
    const float d = native ? m * __uint_as_float(0x3c010204u) : m / 127.0f;
    const float inv = d == 0.0f ? 0.0f : (native ? 127.0f / m : 1.0f / d);
    const float r = pinned ? __builtin_rintf(v * inv) : __builtin_roundf(v * inv);
    const bool range = !(r >= -127.0f && r <= 127.0f);
    const int q = range ? 0 : static_cast<int>(r);
    int qs = q;
    qs += dpp_i<kDppXor1>(qs);
    qs += dpp_i<kDppXor2>(qs);
    qs += dpp_i<kDppHalfMirror>(qs);
    qs += dpp_i<kDppRowMirror>(qs);
    qs += __shfl_xor(qs, 16);
    const float scale = round_f16(d);
    if (own) {
        blk->values[j] = static_cast<int8_t>(q);
        if (j == 0) {
            blk->scale = scale;
            blk->sum = round_f16(static_cast<float>(qs) * d);
        }
    }
    if (bad) return kErrInput;
    return own && (range || !finite(scale)) ? kErrQuantRange : 0;
}

}  // namespace prism
