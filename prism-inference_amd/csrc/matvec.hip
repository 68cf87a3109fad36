// matvec.hip -- batch-1 packed matvec kernels for gfx950 (PTQ1, PQ2, Q2_K, Q8_0).
//
// Work decomposition (all formats): a row of K weights is cut into K/128 "units"
// of 128 weights (PTQ1/PQ2: one block; Q2_K: half a 256-block; Q8_0: four
// 32-blocks).  LPR lanes share a row; lane l owns units l, l+LPR, ... and keeps
// those units' prepared activation codes resident in VGPRs for the whole launch,
// while the wavefront walks down RPI = 64/LPR rows per iteration.  Consecutive
// lanes therefore read consecutive bytes of consecutive rows: every weight load
// is a coalesced dword-aligned buffer load, and loads past the end of the tile
// return zero, so partial tiles never fault.
//
// Bit-exactness: each unit's integer dots are exact (v_dot4_i32_i8); the unit's
// binary32 contribution(s) ("terms") are computed in the unit's lane exactly as
// the reference orders them, written to LDS, and one lane per row then folds the
// terms in block order starting from +0.0 -- the reference's serial chain.
#include "device_common.hpp"
#include "kernels.hpp"

namespace prism {

enum class Op : int { PTQ1_SRC, PTQ1_PINNED, PTQ1_Q8K, PQ2_UNFUSED, PQ2_FUSED, Q2K, Q8_0 };

template <Op O>
constexpr bool uses_q8k() {
    return O == Op::PTQ1_Q8K || O == Op::PQ2_UNFUSED || O == Op::PQ2_FUSED || O == Op::Q2K;
}
// Terms per unit written to LDS.
template <Op O>
constexpr int terms_per_unit() {
    return O == Op::PTQ1_PINNED ? 9 : O == Op::PQ2_FUSED ? 2 : O == Op::Q8_0 ? 4 : 1;
}
template <Op O>
__host__ __device__ constexpr uint32_t term_count(uint32_t nu) {
    return O == Op::Q2K ? nu / 2 : nu * terms_per_unit<O>();
}

constexpr uint32_t sel(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
    return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

struct alignas(4) U2 {
    uint32_t x, y;
};
struct alignas(4) U4 {
    uint32_t x, y, z, w;
};

// Per-lane resident activation for one unit (128 activation codes + side data).
struct Slot {
    uint32_t a[32];  // codes (PQ2: 4x4 byte-transposed per 16-byte group)
    float sc[4];     // Q8: scales of the unit's four 32-blocks; Q8K: sc[0] = block scale
    int sa[16];      // code sums used by the t-1 / c-1 corrections; Q2_K: sub-block bsums
};

// ---- activation prologue ------------------------------------------------------------
template <Op O>
__device__ __forceinline__ void load_slot(Slot &s, const void *act, uint32_t u) {
    if constexpr (uses_q8k<O>()) {
        const Q8KBlock *b = static_cast<const Q8KBlock *>(act) + (u >> 1);
        const uint32_t half = u & 1u;
        const U4 *v = reinterpret_cast<const U4 *>(b->values + 128 * half);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const U4 q = v[i];
            s.a[4 * i] = q.x;
            s.a[4 * i + 1] = q.y;
            s.a[4 * i + 2] = q.z;
            s.a[4 * i + 3] = q.w;
        }
        s.sc[0] = b->scale;
        if constexpr (O == Op::Q2K) {
#pragma unroll
            for (int g = 0; g < 8; ++g) s.sa[g] = b->sums[8 * half + g];
        } else {
            int t = 0;
#pragma unroll
            for (int i = 0; i < 32; ++i) t = sdot4(s.a[i], 0x01010101u, t);
            s.sa[0] = t;
        }
        if constexpr (O == Op::PQ2_UNFUSED || O == Op::PQ2_FUSED) {
            // a'[4i+j] = bytes (a[16i+j], a[16i+4+j], a[16i+8+j], a[16i+12+j]): pairs with the
            // 2-bit field j of code dword i.
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t a0 = s.a[4 * i], a1 = s.a[4 * i + 1], a2 = s.a[4 * i + 2], a3 = s.a[4 * i + 3];
                const uint32_t t0 = perm(a1, a0, sel(0, 4, 1, 5)), t1 = perm(a3, a2, sel(0, 4, 1, 5));
                const uint32_t t2 = perm(a1, a0, sel(2, 6, 3, 7)), t3 = perm(a3, a2, sel(2, 6, 3, 7));
                s.a[4 * i] = perm(t1, t0, sel(0, 1, 4, 5));
                s.a[4 * i + 1] = perm(t1, t0, sel(2, 3, 6, 7));
                s.a[4 * i + 2] = perm(t3, t2, sel(0, 1, 4, 5));
                s.a[4 * i + 3] = perm(t3, t2, sel(2, 3, 6, 7));
            }
        }
    } else {
        const Q8Block *b = static_cast<const Q8Block *>(act) + 4 * u;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const U2 *v = reinterpret_cast<const U2 *>(b[g].values);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const U2 q = v[i];
                s.a[8 * g + 2 * i] = q.x;
                s.a[8 * g + 2 * i + 1] = q.y;
            }
            s.sc[g] = b[g].scale;
        }
        if constexpr (O == Op::PTQ1_SRC) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                int t = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) t = sdot4(s.a[8 * g + i], 0x01010101u, t);
                s.sa[g] = t;
            }
        } else if constexpr (O == Op::PTQ1_PINNED) {
            // Lane l of group g owns positions 4l..4l+3 and 16+4l..16+4l+3
            // (q8_native_lanes, src/kernels.rs:1066-1076).
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int l = 0; l < 4; ++l)
                    s.sa[4 * g + l] = sdot4(s.a[8 * g + 4 + l], 0x01010101u, sdot4(s.a[8 * g + l], 0x01010101u, 0));
        }
    }
}

// ---- PTQ1 trit decode + dot ----------------------------------------------------------
// Byte x carries five trits t_k = ((x*3^k mod 256)*3) >> 8 (tools/ternary/src/lib.rs:202-250).
// Two bytes sit in the 16-bit lanes of a dword; x*3 never carries across lanes, the
// digit lands in each lane's high byte and the low byte is the next remainder.  One
// v_perm gathers four digits (0..2) into a dword for v_dot4 against the activation
// codes the digits multiply; the t-1 offset is removed with the code sums.
// acc(q) returns the accumulator (int&) for quad q (elements 4q..4q+3 of the block).
template <typename Acc>
__device__ __forceinline__ void ptq1_dots(const uint32_t x[7], const uint32_t a[32], Acc &&acc) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {  // bytes 0..15: element 16k + byte
        uint32_t L = x[w] & 0x00ff00ffu, H = (x[w] >> 8) & 0x00ff00ffu;
#pragma unroll
        for (int k = 0; k < 5; ++k) {
            const uint32_t mL = L * 3u, mH = H * 3u;
            {
                int &r = acc(4 * k + w);
                r = sdot4(perm(mH, mL, sel(1, 5, 3, 7)), a[4 * k + w], r);
            }
            L = mL & 0x00ff00ffu;
            H = mH & 0x00ff00ffu;
        }
    }
#pragma unroll
    for (int w = 0; w < 2; ++w) {  // bytes 16..23: element 80 + 8k + (byte-16)
        uint32_t L = x[4 + w] & 0x00ff00ffu, H = (x[4 + w] >> 8) & 0x00ff00ffu;
#pragma unroll
        for (int k = 0; k < 5; ++k) {
            const uint32_t mL = L * 3u, mH = H * 3u;
            {
                int &r = acc(20 + 2 * k + w);
                r = sdot4(perm(mH, mL, sel(1, 5, 3, 7)), a[20 + 2 * k + w], r);
            }
            L = mL & 0x00ff00ffu;
            H = mH & 0x00ff00ffu;
        }
    }
    // bytes 24, 25: element 120 + 2k + (byte-24), k = 0..3
    uint32_t T = (x[6] & 0xffu) | ((x[6] & 0xff00u) << 8);
    const uint32_t m0 = T * 3u;
    T = m0 & 0x00ff00ffu;
    const uint32_t m1 = T * 3u;
    T = m1 & 0x00ff00ffu;
    const uint32_t m2 = T * 3u;
    T = m2 & 0x00ff00ffu;
    const uint32_t m3 = T * 3u;
    int &r30 = acc(30);
    r30 = sdot4(perm(m1, m0, sel(1, 3, 5, 7)), a[30], r30);
    int &r31 = acc(31);
    r31 = sdot4(perm(m3, m2, sel(1, 3, 5, 7)), a[31], r31);
}

// ---- unit evaluation -------------------------------------------------------------------
// Loads one unit of row `rowoff` (byte offset in the tile) and writes its terms to t[].
template <Op O>
__device__ __forceinline__ void unit_terms(__amdgpu_buffer_rsrc_t rs, uint32_t rowoff, uint32_t u, const Slot &s,
                                           float *t) {
    if constexpr (O == Op::PTQ1_SRC || O == Op::PTQ1_PINNED || O == Op::PTQ1_Q8K) {
        const uint32_t off = rowoff + 28u * u;
        const u32x4 v0 = bload4(rs, off);
        const u32x3 v1 = bload3(rs, off + 16);
        const uint32_t x[7] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z};
        const float d = h2f(x[6] >> 16);
        if constexpr (O == Op::PTQ1_SRC) {
            int acc[4] = {0, 0, 0, 0};
            ptq1_dots(x, s.a, [&](int q) -> int & { return acc[q >> 3]; });
            // dot_q8_groups, src/kernels.rs:1043-1064: fl(tt + fl(scale * I)) is one FMA, since
            // the binary16 scale (11 significant bits) times |I| < 2^13 is exact in binary32.
            float tt = 0.0f;
#pragma unroll
            for (int g = 0; g < 4; ++g) tt = __builtin_fmaf(s.sc[g], static_cast<float>(acc[g] - s.sa[g]), tt);
            t[0] = d * tt;
        } else if constexpr (O == Op::PTQ1_Q8K) {
            int acc = 0;
            ptq1_dots(x, s.a, [&](int) -> int & { return acc; });
            // dot_ptq1_q8k, src/kernels.rs:1026-1034
            t[0] = (d * s.sc[0]) * static_cast<float>(acc - s.sa[0]);
        } else {
            int acc[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = 0;
            // quad q -> group q/8, native lane (q%8)%4
            ptq1_dots(x, s.a, [&](int q) -> int & { return acc[4 * (q >> 3) + (q & 3)]; });
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int lo = acc[2 * i] - s.sa[2 * i], hi = acc[2 * i + 1] - s.sa[2 * i + 1];
                t[i] = __uint_as_float((static_cast<uint32_t>(lo) & 0xffffu) | (static_cast<uint32_t>(hi) << 16));
            }
            t[8] = d;
        }
    } else if constexpr (O == Op::PQ2_UNFUSED || O == Op::PQ2_FUSED) {
        // Block u starts at 34u; the 9 dwords from 34u-2(u&1) are dword aligned.
        const uint32_t odd = u & 1u;
        const uint32_t off = rowoff + 34u * u - 2u * odd;
        const u32x4 v0 = bload4(rs, off);
        const u32x4 v1 = bload4(rs, off + 16);
        const uint32_t v2 = bload1(rs, off + 32);
        const uint32_t x[9] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, v2};
        const float d = h2f(odd ? (x[0] >> 16) : (x[0] & 0xffffu));
        int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = odd ? x[i + 1] : align2(x[i + 1], x[i]);
            a0 = sdot4(c & 0x03030303u, s.a[4 * i], a0);
            a1 = sdot4(c & 0x0c0c0c0cu, s.a[4 * i + 1], a1);
            a2 = sdot4(c & 0x30303030u, s.a[4 * i + 2], a2);
            a2 = sdot4((c >> 2) & 0x30303030u, s.a[4 * i + 3], a2);
        }
        const int I = a0 + (a1 >> 2) + (a2 >> 4) - s.sa[0];  // sum (c-1)*a, exact
        // dot_pq2::<FUSED>, src/kernels.rs:941-955
        const float dd = d * s.sc[0];
        const float sf = static_cast<float>(I);
        if constexpr (O == Op::PQ2_UNFUSED) {
            t[0] = dd * sf;
        } else {
            t[0] = dd;
            t[1] = sf;
        }
    } else if constexpr (O == Op::Q2K) {
        // Half h of block j: scales bytes 8h..8h+7, codes bytes 16+32h..+31, d/dmin at 80.
        const uint32_t j = u >> 1, h = u & 1u;
        const uint32_t base = rowoff + 84u * j;
        const u32x2 scb = bload2(rs, base + 8u * h);
        const u32x4 q0 = bload4(rs, base + 16u + 32u * h);
        const u32x4 q1 = bload4(rs, base + 32u + 32u * h);
        const uint32_t dm = bload1(rs, base + 80u);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        int sb[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) sb[i] = 0;
        // element 128h + 32p + 4w + b lives in code byte 4w+b at bits 2p..2p+1
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const int hi = w >> 2;
            sb[0 + hi] = sdot4(q[w] & 0x03030303u, s.a[w], sb[0 + hi]);
            sb[2 + hi] = sdot4(q[w] & 0x0c0c0c0cu, s.a[8 + w], sb[2 + hi]);
            sb[4 + hi] = sdot4(q[w] & 0x30303030u, s.a[16 + w], sb[4 + hi]);
            sb[6 + hi] = sdot4((q[w] >> 2) & 0x30303030u, s.a[24 + w], sb[6 + hi]);
        }
        int isum = 0, msum = 0;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint32_t byte = ((g < 4 ? scb.x : scb.y) >> (8 * (g & 3))) & 0xffu;
            const int shift = g < 2 ? 0 : (g < 4 ? 2 : 4);
            isum += static_cast<int>(byte & 15u) * (sb[g] >> shift);
            msum += s.sa[g] * static_cast<int>(byte >> 4);
        }
        // The two halves of a block sit in lanes l and l^1.
        isum += __shfl_xor(isum, 1, 64);
        msum += __shfl_xor(msum, 1, 64);
        // dot_q2_k_block, src/kernels/kquants.rs:193-196
        const float as = s.sc[0];
        t[0] = (as * h2f(dm & 0xffffu)) * static_cast<float>(isum) - (as * h2f(dm >> 16)) * static_cast<float>(msum);
    } else {  // Q8_0: four 34-byte blocks at 136u
        const uint32_t off = rowoff + 136u * u;
        uint32_t x[34];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const u32x4 v = bload4(rs, off + 16u * i);
            x[4 * i] = v.x;
            x[4 * i + 1] = v.y;
            x[4 * i + 2] = v.z;
            x[4 * i + 3] = v.w;
        }
        const u32x2 tail = bload2(rs, off + 128u);
        x[32] = tail.x;
        x[33] = tail.y;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // blocks 0,2: scale in the low half of dword 0/17, codes two bytes in;
            // blocks 1,3: scale in the high half of dword 8/25, codes dword aligned.
            const int base = j == 0 ? 0 : j == 1 ? 8 : j == 2 ? 17 : 25;
            const uint32_t sbits = (j & 1) ? (x[base] >> 16) : (x[base] & 0xffffu);
            int I = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t c = (j & 1) ? x[base + 1 + i] : align2(x[base + 1 + i], x[base + i]);
                I = sdot4(c, s.a[8 * j + i], I);
            }
            // dot_legacy, src/kernels.rs:1241-1244
            t[j] = (h2f(sbits) * s.sc[j]) * static_cast<float>(I);
        }
    }
}

// ---- the kernel -------------------------------------------------------------------------
template <Op O, int S, int LPR, int R, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_matvec(const uint8_t *__restrict__ W, uint32_t row_bytes,
                                                       uint32_t rows, uint32_t nu, const void *__restrict__ act,
                                                       float *__restrict__ out, int *__restrict__ err) {
    extern __shared__ float lds[];
    constexpr int RPI = 64 / LPR;
    static_assert(R % RPI == 0, "tile rows");
    const uint32_t T = term_count<O>(nu);
    const uint32_t stride = T + 1;  // odd-ish padding keeps phase-2 reads conflict-free
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    float *terms = lds + static_cast<size_t>(wave) * R * stride;
    const uint32_t row0 = (blockIdx.x * WAVES + wave) * R;
    const uint32_t lr = lane % LPR, rq = lane / LPR;
    const uint32_t tile_rows = row0 < rows ? min(static_cast<uint32_t>(R), rows - row0) : 0u;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(W + static_cast<size_t>(row0) * row_bytes, tile_rows * row_bytes);

    Slot slot[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const uint32_t u = lr + LPR * s;
        if (u < nu) load_slot<O>(slot[s], act, u);
    }

    for (int it = 0; it < R / RPI; ++it) {
        const uint32_t rt = it * RPI + rq;  // row within the tile
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const uint32_t u = lr + LPR * s;
            if (u < nu) {
                float t[terms_per_unit<O>()];
                unit_terms<O>(rs, rt * row_bytes, u, slot[s], t);
                if constexpr (O == Op::Q2K) {
                    if ((u & 1u) == 0) terms[rt * stride + (u >> 1)] = t[0];
                } else {
#pragma unroll
                    for (int j = 0; j < terms_per_unit<O>(); ++j) terms[rt * stride + u * terms_per_unit<O>() + j] = t[j];
                }
            }
        }
    }
    __syncthreads();
    if (lane < static_cast<uint32_t>(R) && lane < tile_rows) {
        const float *tr = terms + lane * stride;
        float o = 0.0f;
        if constexpr (O == Op::PQ2_FUSED) {
            for (uint32_t i = 0; i < nu; ++i) o = __builtin_fmaf(tr[2 * i], tr[2 * i + 1], o);
        } else if constexpr (O == Op::PTQ1_PINNED) {
            // dot_q8_groups_pinned, src/kernels.rs:1134-1146: four FMA lanes over the row.
            const Q8Block *ab = static_cast<const Q8Block *>(act);
            float L0 = 0.0f, L1 = 0.0f, L2 = 0.0f, L3 = 0.0f;
            for (uint32_t i = 0; i < nu; ++i) {
                const float dw = tr[9 * i + 8];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float dd = dw * ab[4 * i + g].scale;
                    const uint32_t p0 = __float_as_uint(tr[9 * i + 2 * g]), p1 = __float_as_uint(tr[9 * i + 2 * g + 1]);
                    L0 = __builtin_fmaf(static_cast<float>(static_cast<int16_t>(p0 & 0xffffu)), dd, L0);
                    L1 = __builtin_fmaf(static_cast<float>(static_cast<int16_t>(p0 >> 16)), dd, L1);
                    L2 = __builtin_fmaf(static_cast<float>(static_cast<int16_t>(p1 & 0xffffu)), dd, L2);
                    L3 = __builtin_fmaf(static_cast<float>(static_cast<int16_t>(p1 >> 16)), dd, L3);
                }
            }
            o = (L0 + L1) + (L2 + L3);
        } else {
            for (uint32_t i = 0; i < T; ++i) o = o + tr[i];
        }
        out[row0 + lane] = o;
        if (!finite(o)) raise_error(err, kErrNonfinite);
    }
}

// ---- generic fallback: one thread per row, reference order (odd shapes only) -------
__device__ __forceinline__ uint32_t ld16(const uint8_t *p) { return p[0] | (static_cast<uint32_t>(p[1]) << 8); }

__device__ int trit_of(uint32_t x, int k) {
    for (int i = 0; i < k; ++i) x = (x * 3u) & 255u;
    return static_cast<int>((x * 3u) >> 8);
}

__device__ int ptq1_weight(const uint8_t *b, int i) {
    int lane, digit;
    if (i < 80) {
        lane = i % 16;
        digit = i / 16;
    } else if (i < 120) {
        lane = 16 + (i - 80) % 8;
        digit = (i - 80) / 8;
    } else {
        lane = 24 + (i - 120) % 2;
        digit = (i - 120) / 2;
    }
    return trit_of(b[lane], digit) - 1;
}

__global__ void k_matvec_generic(uint32_t kind, int q8k, int pinned, const uint8_t *__restrict__ W,
                                 uint64_t row_bytes, uint32_t rows, uint32_t cols, const void *__restrict__ act,
                                 float *__restrict__ out, int *__restrict__ err) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const uint8_t *row = W + r * row_bytes;
    float o = 0.0f;
    if (kind == kQ8_0) {
        const Q8Block *a = static_cast<const Q8Block *>(act);
        for (uint32_t b = 0; b < cols / 32; ++b) {
            const uint8_t *p = row + 34 * b;
            int I = 0;
            for (int i = 0; i < 32; ++i) I += static_cast<int8_t>(p[2 + i]) * a[b].values[i];
            o = o + (h2f(ld16(p)) * a[b].scale) * static_cast<float>(I);
        }
    } else if (kind == kQ2_K) {
        const Q8KBlock *a = static_cast<const Q8KBlock *>(act);
        for (uint32_t b = 0; b < cols / 256; ++b) {
            const uint8_t *p = row + 84 * b;
            int isum = 0, msum = 0;
            for (int g = 0; g < 16; ++g) {
                int sd = 0;
                for (int j = 0; j < 16; ++j) {
                    const int i = 16 * g + j;
                    sd += ((p[16 + i / 128 * 32 + i % 32] >> (2 * (i % 128 / 32))) & 3) * a[b].values[i];
                }
                isum += (p[g] & 15) * sd;
                msum += a[b].sums[g] * (p[g] >> 4);
            }
            const float as = a[b].scale;
            o = o + ((as * h2f(ld16(p + 80))) * static_cast<float>(isum) -
                     (as * h2f(ld16(p + 82))) * static_cast<float>(msum));
        }
    } else if (kind == kTQ1_0 || kind == kTQ2_0) {
        // src/kernels/tquants.rs:255-273 (element maps :145-190)
        const Q8KBlock *a = static_cast<const Q8KBlock *>(act);
        const uint32_t bb = kind == kTQ1_0 ? 54 : 66;
        for (uint32_t b = 0; b < cols / 256; ++b) {
            const uint8_t *p = row + bb * b;
            int I = 0;
            for (int i = 0; i < 256; ++i) {
                int wv;
                if (kind == kTQ2_0) {
                    wv = static_cast<int>((p[i / 128 * 32 + i % 32] >> (2 * (i % 128 / 32))) & 3) - 1;
                } else if (i < 160) {
                    wv = trit_of(p[i % 32], i / 32) - 1;
                } else if (i < 240) {
                    wv = trit_of(p[32 + (i - 160) % 16], (i - 160) / 16) - 1;
                } else {
                    wv = trit_of(p[48 + (i - 240) % 4], (i - 240) / 4) - 1;
                }
                I += wv * a[b].values[i];
            }
            o = o + static_cast<float>(I) * (h2f(ld16(p + bb - 2)) * a[b].scale);
        }
    } else {
        const bool pq2 = kind == kPQ2;
        const uint32_t bb = pq2 ? 34 : 28;
        float L[4] = {0.f, 0.f, 0.f, 0.f};
        for (uint32_t b = 0; b < cols / 128; ++b) {
            const uint8_t *p = row + bb * b;
            const float d = h2f(ld16(pq2 ? p : p + 26));
            if (q8k) {
                const Q8KBlock *a = static_cast<const Q8KBlock *>(act) + b / 2;
                int I = 0;
                for (int i = 0; i < 128; ++i) {
                    const int wv = pq2 ? static_cast<int>((p[2 + i / 4] >> (2 * (i % 4))) & 3) - 1 : ptq1_weight(p, i);
                    I += wv * a->values[128 * (b & 1) + i];
                }
                const float dd = d * a->scale;
                o = (pq2 && pinned) ? __builtin_fmaf(dd, static_cast<float>(I), o) : o + dd * static_cast<float>(I);
            } else {
                const Q8Block *a = static_cast<const Q8Block *>(act) + 4 * b;
                if (!pq2 && pinned) {
                    for (int g = 0; g < 4; ++g) {
                        const float dd = d * a[g].scale;
                        for (int l = 0; l < 4; ++l) {
                            int I = 0;
                            for (int j = 0; j < 4; ++j) {
                                I += ptq1_weight(p, 32 * g + 4 * l + j) * a[g].values[4 * l + j];
                                I += ptq1_weight(p, 32 * g + 16 + 4 * l + j) * a[g].values[16 + 4 * l + j];
                            }
                            L[l] = __builtin_fmaf(static_cast<float>(I), dd, L[l]);
                        }
                    }
                } else {
                    float t = 0.0f;
                    for (int g = 0; g < 4; ++g) {
                        int I = 0;
                        for (int i = 0; i < 32; ++i) {
                            const int e = 32 * g + i;
                            const int wv = pq2 ? static_cast<int>((p[2 + e / 4] >> (2 * (e % 4))) & 3) - 1 : ptq1_weight(p, e);
                            I += wv * a[g].values[i];
                        }
                        t = t + a[g].scale * static_cast<float>(I);
                    }
                    o = o + d * t;
                }
            }
        }
        if (!pq2 && pinned && !q8k) o = (L[0] + L[1]) + (L[2] + L[3]);
    }
    out[r] = o;
    if (!finite(o)) raise_error(err, kErrNonfinite);
}

// ---- dispatch ---------------------------------------------------------------------------
constexpr int kTileRows = 16;
constexpr size_t kLdsLimit = 64 * 1024;

template <Op O>
static size_t tile_lds_bytes(uint64_t cols) {
    return sizeof(float) * kTileRows * (term_count<O>(static_cast<uint32_t>(cols / 128)) + 1);
}

template <Op O, int S, int LPR, int WAVES>
static int launch_waves(const MatvecArgs &a, const void *act, float *out) {
    const uint32_t nu = static_cast<uint32_t>(a.cols / 128);
    const size_t lds = WAVES * tile_lds_bytes<O>(a.cols);
    const uint32_t tiles = static_cast<uint32_t>((a.rows + kTileRows - 1) / kTileRows);
    const uint32_t grid = (tiles + WAVES - 1) / WAVES;
    hipLaunchKernelGGL((k_matvec<O, S, LPR, kTileRows, WAVES>), dim3(grid), dim3(64 * WAVES), lds, a.stream, a.w,
                       static_cast<uint32_t>(a.row_bytes), static_cast<uint32_t>(a.rows), nu, act, out, a.err);
    return launch_status();
}

// Four independent wavefronts per workgroup when their LDS tiles fit, else one.
template <Op O, int S, int LPR>
static int launch_op(const MatvecArgs &a, const void *act, float *out) {
    if (4 * tile_lds_bytes<O>(a.cols) <= kLdsLimit) return launch_waves<O, S, LPR, 4>(a, act, out);
    return launch_waves<O, S, LPR, 1>(a, act, out);
}

template <Op O>
static int launch_sized(const MatvecArgs &a, const void *act, float *out) {
    const uint64_t nu = a.cols / 128;
    if (nu <= 16) return launch_op<O, 1, 16>(a, act, out);
    if (nu <= 32) return launch_op<O, 2, 16>(a, act, out);
    if (nu <= 48) return launch_op<O, 3, 16>(a, act, out);
    if (nu <= 64) return launch_op<O, 4, 16>(a, act, out);
    if (nu <= 128) return launch_op<O, 2, 64>(a, act, out);
    if (nu <= 256) return launch_op<O, 4, 64>(a, act, out);
    return -2;
}

template <Op O>
static bool fits(const MatvecArgs &a) {
    return tile_lds_bytes<O>(a.cols) <= kLdsLimit;
}

static bool fast_path(const MatvecArgs &a) {
    if (a.kind == kTQ1_0 || a.kind == kTQ2_0) return false;  // native TQ rows: generic kernel only
    if (a.cols % 128 != 0 || a.cols / 128 > 256) return false;
    if (a.kind == kPTQ1 && a.act_format == kActQ8 && a.pinned && !fits<Op::PTQ1_PINNED>(a)) return false;
    if (a.kind == kQ8_0 && !fits<Op::Q8_0>(a)) return false;
    if (a.kind == kPQ2 && a.pinned && !fits<Op::PQ2_FUSED>(a)) return false;
    if (a.rows * a.row_bytes >= (1ull << 32)) return false;  // 32-bit buffer offsets per tile
    if (a.kind == kPQ2) return a.act_format == kActQ8K;      // odd-group PQ2 uses the fallback
    if (a.kind == kQ2_K) return a.cols % 256 == 0;
    return true;
}

int launch_matvec(const MatvecArgs &a) {
    const size_t act_stride = a.act_format == kActQ8K ? sizeof(Q8KBlock) * ((a.cols + 255) / 256)
                                                      : sizeof(Q8Block) * (a.cols / 32);
    for (uint32_t tok = 0; tok < a.tokens; ++tok) {
        const void *act = static_cast<const uint8_t *>(a.act) + act_stride * tok;
        float *out = a.out + a.rows * tok;
        int rc;
        if (!fast_path(a)) {
            hipLaunchKernelGGL(k_matvec_generic, dim3(static_cast<uint32_t>((a.rows + 127) / 128)), dim3(128), 0,
                               a.stream, a.kind, a.act_format == kActQ8K ? 1 : 0, a.pinned, a.w, a.row_bytes,
                               static_cast<uint32_t>(a.rows), static_cast<uint32_t>(a.cols), act, out, a.err);
            rc = launch_status();
        } else if (a.kind == kPTQ1) {
            if (a.act_format == kActQ8K)
                rc = launch_sized<Op::PTQ1_Q8K>(a, act, out);
            else
                rc = a.pinned ? launch_sized<Op::PTQ1_PINNED>(a, act, out) : launch_sized<Op::PTQ1_SRC>(a, act, out);
        } else if (a.kind == kPQ2) {
            rc = a.pinned ? launch_sized<Op::PQ2_FUSED>(a, act, out) : launch_sized<Op::PQ2_UNFUSED>(a, act, out);
        } else if (a.kind == kQ2_K) {
            rc = launch_sized<Op::Q2K>(a, act, out);
        } else {
            rc = launch_sized<Op::Q8_0>(a, act, out);
        }
        if (rc) return rc;
    }
    return 0;
}

}  // namespace prism
