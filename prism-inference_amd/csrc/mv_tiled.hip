// mv_tiled.hip -- batch-1 packed matvec over the 64-row tiled weight layout (gfx950).
//
// Lane r of a wavefront owns row r of a 64-row tile and walks the row's units
// (128 weights; a 256-weight super-block for Q2_K) in order, so the reference's
// binary32 chain out = ((0 + t0) + t1) + ... is evaluated serially in the lane
// that owns the row, with no cross-lane float reduction at all.  Every weight load
// is one contiguous 16/8/4/2-byte-per-lane buffer load (the tiled layout puts the
// same piece of 64 rows side by side), and out-of-range lanes read the buffer's
// zero padding.  All lanes of a wavefront process the same unit at the same time,
// so the prepared activation is wave-uniform: it is fetched with scalar loads and
// fed to v_dot4 as a scalar operand, costing no LDS or vector bandwidth.
//
// Small matrices split K across the KS wavefronts of a workgroup: each wavefront
// computes the per-unit terms of its K range, the terms meet in LDS, and wavefront
// 0 folds them in unit order -- the same serial chain, only computed later.
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"
#include "quant_dev.hpp"
#include "tiled.hpp"

namespace prism {

namespace {

enum class Op : int { PTQ1_SRC, PTQ1_PINNED, PTQ1_Q8K, PQ2_UNFUSED, PQ2_FUSED, PQ2_Q8, Q2K, Q8_0, TQ1, TQ2 };

template <Op O>
constexpr uint32_t kind_of() {
    return O == Op::Q2K    ? kQ2_K
           : O == Op::Q8_0 ? kQ8_0
           : O == Op::TQ1  ? kTQ1_0
           : O == Op::TQ2  ? kTQ2_0
           : (O == Op::PQ2_UNFUSED || O == Op::PQ2_FUSED || O == Op::PQ2_Q8) ? kPQ2
                                                                              : kPTQ1;
}
// Native bytes per unit.
template <Op O>
constexpr uint32_t unit_bytes() {
    return kind_of<O>() == kPTQ1   ? 28
           : kind_of<O>() == kPQ2  ? 34
           : kind_of<O>() == kQ2_K ? 84
           : O == Op::TQ1          ? 54
           : O == Op::TQ2          ? 66
                                   : 136;
}
// Weights per unit: a 256-element super-block (Q2_K, TQ1_0, TQ2_0) or 128.
template <Op O>
constexpr uint32_t unit_weights() {
    return (O == Op::Q2K || O == Op::TQ1 || O == Op::TQ2) ? 256 : 128;
}
// binary32 terms per unit handed to the fold when K is split across wavefronts.
template <Op O>
constexpr int terms_per_unit() {
    return O == Op::PTQ1_PINNED ? 9 : O == Op::PQ2_FUSED ? 2 : O == Op::Q8_0 ? 4 : 1;
}

constexpr uint32_t sel(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
    return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

// Sum of the four signed bytes of a dword.
__device__ __forceinline__ int bsum4(uint32_t a, int c) { return sdot4(a, 0x01010101u, c); }

// ---- PTQ1 trit decode ---------------------------------------------------------------
// Byte x carries trits t_k = ((x*3^k mod 256)*3) >> 8 (tools/ternary/src/lib.rs:202-250).
// Two bytes travel in the 16-bit lanes of a dword: x*3 never carries across lanes,
// the digit lands in each lane's high byte and the low byte is the next remainder.
// One v_perm gathers the four digits (0..2) of bytes 4w..4w+3 into a dword for v_dot4
// against the activation codes they multiply; sum (t-1)a = sum t*a - sum a.
// Element map: byte b<16 digit k -> 16k+b; byte 16+b (b<8) digit k -> 80+8k+b;
// byte 24+b (b<2) digit k<4 -> 120+2k+b.  acc(q) receives quad q (elements 4q..4q+3).
// A PTQ1 unit with its trits extracted: q[i] holds the digits (0..2) of elements
// 4i..4i+3 as bytes, d the binary16 scale bits.  The extraction needs no activation,
// so a kernel can run it while its activation is still being staged.
struct Ptq1Dec {
    uint32_t q[32];
    uint32_t d;
};

__device__ __forceinline__ void ptq1_decode(const uint32_t x[7], Ptq1Dec &o) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t L = x[w] & 0x00ff00ffu, H = (x[w] >> 8) & 0x00ff00ffu;
#pragma unroll
        for (int k = 0; k < 5; ++k) {
            const uint32_t mL = L * 3u, mH = H * 3u;
            o.q[4 * k + w] = perm(mH, mL, sel(1, 5, 3, 7));
            L = mL & 0x00ff00ffu;
            H = mH & 0x00ff00ffu;
        }
    }
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        uint32_t L = x[4 + w] & 0x00ff00ffu, H = (x[4 + w] >> 8) & 0x00ff00ffu;
#pragma unroll
        for (int k = 0; k < 5; ++k) {
            const uint32_t mL = L * 3u, mH = H * 3u;
            o.q[20 + 2 * k + w] = perm(mH, mL, sel(1, 5, 3, 7));
            L = mL & 0x00ff00ffu;
            H = mH & 0x00ff00ffu;
        }
    }
    uint32_t T = (x[6] & 0xffu) | ((x[6] & 0xff00u) << 8);
    const uint32_t m0 = T * 3u;
    T = m0 & 0x00ff00ffu;
    const uint32_t m1 = T * 3u;
    T = m1 & 0x00ff00ffu;
    const uint32_t m2 = T * 3u;
    T = m2 & 0x00ff00ffu;
    const uint32_t m3 = T * 3u;
    o.q[30] = perm(m1, m0, sel(1, 3, 5, 7));
    o.q[31] = perm(m3, m2, sel(1, 3, 5, 7));
    o.d = x[6] >> 16;
}

template <typename Act, typename Acc>
__device__ __forceinline__ void ptq1_dot(const Ptq1Dec &D, const Act &a, Acc &&acc) {
#pragma unroll
    for (int q = 0; q < 32; ++q) {
        int &r = acc(q);
        r = sdot4(D.q[q], a(q), r);
    }
}

template <typename Act, typename Acc>
__device__ __forceinline__ void ptq1_dots(const uint32_t x[7], const Act &a, Acc &&acc) {
    Ptq1Dec D;
    ptq1_decode(x, D);
    ptq1_dot(D, a, acc);
}

// ---- PTQ1 decode table (LDS) ----------------------------------------------------------
// Entry e (a code byte) holds its trits minus one as signed bytes: lo = (t0-1, t1-1,
// t2-1, t3-1), hi = (t4-1, 0, 0, 0).  Looking a byte up costs one v_perm (address) and
// one ds_read_b64 instead of the ~7.5 VALU instructions per byte of the SWAR form, and
// the signed trits need no activation-sum correction.  The table is replicated 32
// times, entry-major (copy c of entry e at byte 256e + 8c), and lane l reads copy l%32:
// the 32 lanes of each half-wavefront then hit 32 distinct bank pairs whatever the
// codes, and a lane's address is the code byte in bits 8..15 over its copy offset.
constexpr uint32_t kLutCopies = 32;
__shared__ __attribute__((aligned(16))) uint2 g_ptq1_lut[256 * kLutCopies];

__device__ __forceinline__ void ptq1_lut_fill(uint32_t tid, uint32_t nthreads) {
    for (uint32_t i = tid; i < 256 * kLutCopies; i += nthreads) {
        uint32_t r = i / kLutCopies, lo = 0, hi = 0;
#pragma unroll
        for (int k = 0; k < 5; ++k) {
            const uint32_t m = r * 3u;
            const uint32_t t = ((m >> 8) - 1u) & 0xffu;  // trit_k - 1 as a byte
            r = m & 0xffu;
            if (k < 4)
                lo |= t << (8 * k);
            else
                hi = t;
        }
        g_ptq1_lut[i] = make_uint2(lo, hi);
    }
}

// Table entry of byte b of code dword x; `lbase` = 8 * (lane % 32).
__device__ __forceinline__ uint2 lut_at(uint32_t x, uint32_t lbase, uint32_t b) {
    const uint32_t addr = perm(x, lbase, sel(0, 4 + b, 12, 12));
    return *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint8_t *>(g_ptq1_lut) + addr);
}

// The unit's 32 quads from the table in slot order, for kernels that stage the
// activation in the same order (an integer dot is exact in any element order):
// f(s, t) receives slot s.  Slots 5w..5w+4 come from code dword w < 6 (entries
// E0..E3 of its bytes): (E0.d0, E0.d1, E1.d0, E1.d1), (E2.d0, E2.d1, E3.d0, E3.d1),
// the same two with digits 2 and 3, and the four digit-4s -- one v_perm per slot
// where the natural order takes two.  Every slot lies in one 32-element group.  With
// NATIVE, dwords 4 and 5 keep the natural quads (digit k of four bytes in slot 5w+k),
// and every slot also lies in one native lane subset (positions 4l..4l+3 and
// 16+4l..16+4l+3 of its group).  Slots 30 and 31 are dword 6's two natural quads.
// ptq1_slot_byte gives each element's slot and byte.
template <bool NATIVE, typename F>
__device__ __forceinline__ void ptq1_slots_lut(const uint32_t x[7], uint32_t lbase, F &&f) {
#pragma unroll
    for (int w = 0; w < 6; ++w) {
        const uint2 e0 = lut_at(x[w], lbase, 0), e1 = lut_at(x[w], lbase, 1);
        const uint2 e2 = lut_at(x[w], lbase, 2), e3 = lut_at(x[w], lbase, 3);
        const uint32_t d4 = perm(e1.y, e0.y, sel(0, 4, 12, 12)) | perm(e3.y, e2.y, sel(12, 12, 0, 4));
        if (NATIVE && w >= 4) {
            const uint32_t l01 = perm(e1.x, e0.x, sel(0, 4, 1, 5)), h01 = perm(e1.x, e0.x, sel(2, 6, 3, 7));
            const uint32_t l23 = perm(e3.x, e2.x, sel(0, 4, 1, 5)), h23 = perm(e3.x, e2.x, sel(2, 6, 3, 7));
            f(5 * w + 0, perm(l23, l01, sel(0, 1, 4, 5)));
            f(5 * w + 1, perm(l23, l01, sel(2, 3, 6, 7)));
            f(5 * w + 2, perm(h23, h01, sel(0, 1, 4, 5)));
            f(5 * w + 3, perm(h23, h01, sel(2, 3, 6, 7)));
        } else {
            f(5 * w + 0, perm(e1.x, e0.x, sel(0, 1, 4, 5)));
            f(5 * w + 1, perm(e3.x, e2.x, sel(0, 1, 4, 5)));
            f(5 * w + 2, perm(e1.x, e0.x, sel(2, 3, 6, 7)));
            f(5 * w + 3, perm(e3.x, e2.x, sel(2, 3, 6, 7)));
        }
        f(5 * w + 4, d4);
    }
    const uint2 e0 = lut_at(x[6], lbase, 0), e1 = lut_at(x[6], lbase, 1);
    f(30, perm(e1.x, e0.x, sel(0, 4, 1, 5)));
    f(31, perm(e1.x, e0.x, sel(2, 6, 3, 7)));
}

// 4 * slot + byte of element e (0..127) of a unit in ptq1_slots_lut's order.  Digit k
// of code byte b < 16 is element 16k + b, of byte 16 + b (b < 8) element 80 + 8k + b,
// of byte 24 + b (b < 2) element 120 + 2k + b.
__host__ __device__ constexpr uint32_t ptq1_slot_byte(uint32_t e, bool native) {
    uint32_t B = 0, k = 0;
    if (e < 64) {
        k = e >> 4;
        B = e & 15u;
    } else if (e < 80) {
        B = e - 64;
        k = 4;
    } else if (e < 120) {
        k = (e - 80) >> 3;
        B = 16 + ((e - 80) & 7u);
    } else {
        k = (e - 120) >> 1;
        B = 24 + ((e - 120) & 1u);
    }
    if (B >= 24) return 4 * (30 + (k >> 1)) + 2 * (k & 1u) + (B - 24);
    const uint32_t w = B >> 2, i = B & 3u;
    if (k == 4) return 4 * (5 * w + 4) + i;
    if (native && w >= 4) return 4 * (5 * w + k) + i;
    return 4 * (5 * w + (i >> 1) + 2 * (k >> 1)) + 2 * (i & 1u) + (k & 1u);
}

// Slots of 32-element group g in ptq1_slots_lut's order, and (NATIVE) the two slots of
// native lane l of group g.
constexpr int kPtq1GroupSlots[4][8] = {{0, 1, 5, 6, 10, 11, 15, 16},
                                       {2, 3, 7, 8, 12, 13, 17, 18},
                                       {4, 9, 14, 19, 20, 21, 25, 26},
                                       {22, 23, 24, 27, 28, 29, 30, 31}};
constexpr int kPtq1LaneSlots[4][4][2] = {{{0, 1}, {5, 6}, {10, 11}, {15, 16}},
                                         {{2, 3}, {7, 8}, {12, 13}, {17, 18}},
                                         {{4, 20}, {9, 25}, {14, 21}, {19, 26}},
                                         {{22, 24}, {27, 29}, {23, 30}, {28, 31}}};

// Same contract as ptq1_dots, but acc(q) receives sum (t-1)*a directly, from the table
// in a "pair" order that costs one v_perm per dword on the weight side: for code dword w
// (bytes b0..b3) and digits (k, k+1), (E0.dk, E1.dk, E0.dk+1, E1.dk+1) and the same of E2,
// E3 pair with the activation halves pk_ll / pk_hh of the natural dwords of digits k and
// k+1 -- wave-uniform values, so the repacking runs on the scalar unit (s_pack_*_b32_b16)
// beside the vector decode.  Digit 4 of each dword and code dword 6 keep their natural
// quads.  acc(q) is called with the natural index q of the slot's first quad; the slot's
// elements lie in q's 32-element group and, for NATIVE below, in q's native lane subset
// (positions 4l..4l+3 and 16+4l..16+4l+3 of the group): code dwords 4 and 5 pair positions
// of two native lanes, so NATIVE keeps their natural quads.
template <bool NATIVE = false, typename Act, typename Acc>
__device__ __forceinline__ void ptq1_dots_lut(const uint32_t x[7], uint32_t lbase, const Act &a, Acc &&acc) {
    auto dot = [&](int q, uint32_t t, uint32_t av) {
        int &r = acc(q);
        r = sdot4(t, av, r);
    };
#pragma unroll
    for (int w = 0; w < 6; ++w) {
        const uint2 e0 = lut_at(x[w], lbase, 0), e1 = lut_at(x[w], lbase, 1);
        const uint2 e2 = lut_at(x[w], lbase, 2), e3 = lut_at(x[w], lbase, 3);
        auto nat = [&](int k) { return w < 4 ? 4 * k + w : 20 + 2 * k + (w - 4); };  // natural quad of digit k
        if (NATIVE && w >= 4) {
            const uint32_t l01 = perm(e1.x, e0.x, sel(0, 4, 1, 5)), h01 = perm(e1.x, e0.x, sel(2, 6, 3, 7));
            const uint32_t l23 = perm(e3.x, e2.x, sel(0, 4, 1, 5)), h23 = perm(e3.x, e2.x, sel(2, 6, 3, 7));
            dot(nat(0), perm(l23, l01, sel(0, 1, 4, 5)), a(nat(0)));
            dot(nat(1), perm(l23, l01, sel(2, 3, 6, 7)), a(nat(1)));
            dot(nat(2), perm(h23, h01, sel(0, 1, 4, 5)), a(nat(2)));
            dot(nat(3), perm(h23, h01, sel(2, 3, 6, 7)), a(nat(3)));
        } else {
#pragma unroll
            for (int k = 0; k < 4; k += 2) {
                const uint32_t x0 = a(nat(k)), x1 = a(nat(k + 1));
                typedef uint16_t h2 __attribute__((ext_vector_type(2)));  // s_pack_ll / s_pack_hh
                const uint32_t lo = __builtin_bit_cast(uint32_t, h2{static_cast<uint16_t>(x0), static_cast<uint16_t>(x1)});
                const uint32_t hi =
                    __builtin_bit_cast(uint32_t, h2{static_cast<uint16_t>(x0 >> 16), static_cast<uint16_t>(x1 >> 16)});
                const uint32_t s01 = k ? sel(2, 6, 3, 7) : sel(0, 4, 1, 5);
                dot(nat(k), perm(e1.x, e0.x, s01), lo);
                dot(nat(k), perm(e3.x, e2.x, s01), hi);
            }
        }
        dot(nat(4), perm(e1.y, e0.y, sel(0, 4, 12, 12)) | perm(e3.y, e2.y, sel(12, 12, 0, 4)), a(nat(4)));
    }
    const uint2 e0 = lut_at(x[6], lbase, 0), e1 = lut_at(x[6], lbase, 1);
    dot(30, perm(e1.x, e0.x, sel(0, 4, 1, 5)), a(30));
    dot(31, perm(e1.x, e0.x, sel(2, 6, 3, 7)), a(31));
}

// PQ2 code dword i holds elements 16i..16i+15, element 16i+4q+p in byte q, bits 2p.
// Given the 16 activation codes of those elements (natural order, dwords q0..q3),
// accumulates sum c*a into a0 + a1/4 + a2/16 (the masks leave field p scaled by 4^p)
// and the code sum into s.  The activation quad paired with field p is
// (a[p], a[4+p], a[8+p], a[12+p]): a 4x4 byte transpose.
__device__ __forceinline__ void pq2_dword(uint32_t c, uint32_t q0, uint32_t q1, uint32_t q2, uint32_t q3, int &a0,
                                          int &a1, int &a2, int &s) {
    s = bsum4(q3, bsum4(q2, bsum4(q1, bsum4(q0, s))));
    const uint32_t t0 = perm(q1, q0, sel(0, 4, 1, 5)), t1 = perm(q3, q2, sel(0, 4, 1, 5));
    const uint32_t t2 = perm(q1, q0, sel(2, 6, 3, 7)), t3 = perm(q3, q2, sel(2, 6, 3, 7));
    a0 = sdot4(c & 0x03030303u, perm(t1, t0, sel(0, 1, 4, 5)), a0);
    a1 = sdot4(c & 0x0c0c0c0cu, perm(t1, t0, sel(2, 3, 6, 7)), a1);
    a2 = sdot4(c & 0x30303030u, perm(t3, t2, sel(0, 1, 4, 5)), a2);
    a2 = sdot4((c >> 2) & 0x30303030u, perm(t3, t2, sel(2, 3, 6, 7)), a2);
}

// ---- per-unit raw weight data ---------------------------------------------------------
template <Op O>
struct Raw;
template <>
struct Raw<Op::PTQ1_SRC> {
    uint32_t x[7];
};
template <>
struct Raw<Op::PTQ1_PINNED> : Raw<Op::PTQ1_SRC> {};
template <>
struct Raw<Op::PTQ1_Q8K> : Raw<Op::PTQ1_SRC> {};
template <>
struct Raw<Op::PQ2_UNFUSED> {
    uint32_t c[8];
    uint32_t d;
};
template <>
struct Raw<Op::PQ2_FUSED> : Raw<Op::PQ2_UNFUSED> {};
template <>
struct Raw<Op::PQ2_Q8> : Raw<Op::PQ2_UNFUSED> {};
template <>
struct Raw<Op::Q2K> {
    uint32_t q[16];
    uint32_t sc[4];
    uint32_t dm;
};
template <>
struct Raw<Op::Q8_0> {
    uint32_t c[32];
    uint32_t s[2];
};
template <>
struct Raw<Op::TQ1> {
    uint32_t q[13];  // code bytes 0..51
    uint32_t d;      // binary16 scale
};
template <>
struct Raw<Op::TQ2> {
    uint32_t q[16];  // code bytes 0..63
    uint32_t d;
};

// Loads unit `seg` (byte offset of the unit's segment in the tile) for tile-row `r`.
template <Op O>
__device__ __forceinline__ void load_unit(Raw<O> &w, __amdgpu_buffer_rsrc_t rs, uint32_t seg, uint32_t trp,
                                          uint32_t r) {
    if constexpr (kind_of<O>() == kPTQ1) {
        const u32x4 a = bload4(rs, seg + 16u * r);
        const u32x2 b = bload2(rs, seg + 16u * trp + 8u * r);
        const uint32_t c = bload1(rs, seg + 24u * trp + 4u * r);
        w.x[0] = a.x; w.x[1] = a.y; w.x[2] = a.z; w.x[3] = a.w;
        w.x[4] = b.x; w.x[5] = b.y; w.x[6] = c;
    } else if constexpr (kind_of<O>() == kPQ2) {
        const u32x4 a = bload4(rs, seg + 16u * r);
        const u32x4 b = bload4(rs, seg + 16u * trp + 16u * r);
        w.c[0] = a.x; w.c[1] = a.y; w.c[2] = a.z; w.c[3] = a.w;
        w.c[4] = b.x; w.c[5] = b.y; w.c[6] = b.z; w.c[7] = b.w;
        w.d = __builtin_amdgcn_raw_buffer_load_b16(rs, static_cast<int>(seg + 32u * trp + 2u * r), 0, 0);
    } else if constexpr (O == Op::TQ1 || O == Op::TQ2) {
        constexpr int P = O == Op::TQ1 ? 3 : 4;  // 16-byte code pieces
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const u32x4 a = bload4(rs, seg + 16u * p * trp + 16u * r);
            w.q[4 * p] = a.x; w.q[4 * p + 1] = a.y; w.q[4 * p + 2] = a.z; w.q[4 * p + 3] = a.w;
        }
        if constexpr (O == Op::TQ1) w.q[12] = bload1(rs, seg + 48u * trp + 4u * r);
        constexpr uint32_t kScale = O == Op::TQ1 ? 52 : 64;  // scale piece offset (in TRP bytes)
        w.d = __builtin_amdgcn_raw_buffer_load_b16(rs, static_cast<int>(seg + kScale * trp + 2u * r), 0, 0);
    } else if constexpr (kind_of<O>() == kQ2_K) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const u32x4 a = bload4(rs, seg + 16u * p * trp + 16u * r);
            w.q[4 * p] = a.x; w.q[4 * p + 1] = a.y; w.q[4 * p + 2] = a.z; w.q[4 * p + 3] = a.w;
        }
        const u32x4 s = bload4(rs, seg + 64u * trp + 16u * r);
        w.sc[0] = s.x; w.sc[1] = s.y; w.sc[2] = s.z; w.sc[3] = s.w;
        w.dm = bload1(rs, seg + 80u * trp + 4u * r);
    } else {
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const u32x4 a = bload4(rs, seg + 16u * p * trp + 16u * r);
            w.c[4 * p] = a.x; w.c[4 * p + 1] = a.y; w.c[4 * p + 2] = a.z; w.c[4 * p + 3] = a.w;
        }
        const u32x2 s = bload2(rs, seg + 128u * trp + 8u * r);
        w.s[0] = s.x;
        w.s[1] = s.y;
    }
}

// ---- per-unit arithmetic ------------------------------------------------------------
// `act` is the token's prepared activation; every index into it is wave-uniform.
// Terms go to t[] in the order the reference's chain consumes them.
// LUT selects the PTQ1 decoder: the SWAR digit extraction (trits 0..2, corrected by
// the activation sums) or the LDS table (trits already minus one); `lbase` is the
// lane's table-copy offset.
// W is the unit's Raw<O>, or for the PTQ1 ops (without LUT) its Ptq1Dec.
__device__ __forceinline__ uint32_t ptq1_scale_bits(const Raw<Op::PTQ1_SRC> &w) { return w.x[6] >> 16; }
__device__ __forceinline__ uint32_t ptq1_scale_bits(const Ptq1Dec &w) { return w.d; }

template <Op O, bool LUT = false, typename W = Raw<O>>
__device__ __forceinline__ void unit_terms(const W &w, const void *__restrict__ act, uint32_t u, float *t,
                                           uint32_t lbase = 0) {
    auto trits = [&](const auto &raw, const auto &a, auto &&acc) {
        if constexpr (std::is_same_v<W, Ptq1Dec>)
            ptq1_dot(raw, a, acc);
        else if constexpr (LUT)
            ptq1_dots_lut<O == Op::PTQ1_PINNED>(raw.x, lbase, a, acc);
        else
            ptq1_dots(raw.x, a, acc);
    };
    if constexpr (O == Op::PTQ1_SRC || O == Op::PTQ1_PINNED) {
        const Q8Block *b = static_cast<const Q8Block *>(act) + 4 * u;
        const uint32_t *av[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) av[g] = reinterpret_cast<const uint32_t *>(b[g].values);
        auto a = [&](int q) -> uint32_t { return av[q >> 3][q & 7]; };
        const float d = h2f(ptq1_scale_bits(w));
        if constexpr (O == Op::PTQ1_SRC) {
            int acc[4] = {0, 0, 0, 0};
            trits(w, a, [&](int q) -> int & { return acc[q >> 3]; });
            // dot_q8_groups, src/kernels.rs:1043-1064: fl(tt + fl(scale * I)) is one FMA, since
            // the binary16 scale (11 significant bits) times |I| < 2^13 is exact in binary32.
            float tt = 0.0f;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                int s = 0;
                if constexpr (!LUT) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) s = bsum4(av[g][i], s);
                }
                tt = __builtin_fmaf(b[g].scale, static_cast<float>(acc[g] - s), tt);
            }
            t[0] = d * tt;
        } else {
            // q8_native_lanes (src/kernels.rs:1066-1076): lane l of group g owns positions
            // 4l..4l+3 and 16+4l..16+4l+3, i.e. quads l and l+4 of the group.
            int acc[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = 0;
            trits(w, a, [&](int q) -> int & { return acc[4 * (q >> 3) + (q & 3)]; });
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int g0 = i >> 1, l0 = 2 * (i & 1);
                int s0 = 0, s1 = 0;
                if constexpr (!LUT) {
                    s0 = bsum4(av[g0][l0 + 4], bsum4(av[g0][l0], 0));
                    s1 = bsum4(av[g0][l0 + 5], bsum4(av[g0][l0 + 1], 0));
                }
                const int lo = acc[2 * i] - s0, hi = acc[2 * i + 1] - s1;
                t[i] = __uint_as_float((static_cast<uint32_t>(lo) & 0xffffu) | (static_cast<uint32_t>(hi) << 16));
            }
            t[8] = d;
        }
    } else if constexpr (O == Op::PTQ1_Q8K) {
        const Q8KBlock *b = static_cast<const Q8KBlock *>(act) + (u >> 1);
        const uint32_t *av = reinterpret_cast<const uint32_t *>(b->values) + 32 * (u & 1);
        auto a = [&](int q) -> uint32_t { return av[q]; };
        int acc = 0;
        trits(w, a, [&](int) -> int & { return acc; });
        int s = 0;
        if constexpr (!LUT) {
#pragma unroll
            for (int i = 0; i < 32; ++i) s = bsum4(av[i], s);
        }
        // dot_ptq1_q8k, src/kernels.rs:1026-1034
        t[0] = (h2f(ptq1_scale_bits(w)) * b->scale) * static_cast<float>(acc - s);
    } else if constexpr (O == Op::PQ2_UNFUSED || O == Op::PQ2_FUSED) {
        const Q8KBlock *b = static_cast<const Q8KBlock *>(act) + (u >> 1);
        const uint32_t *av = reinterpret_cast<const uint32_t *>(b->values) + 32 * (u & 1);
        int a0 = 0, a1 = 0, a2 = 0, s = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            pq2_dword(w.c[i], av[4 * i], av[4 * i + 1], av[4 * i + 2], av[4 * i + 3], a0, a1, a2, s);
        const int I = a0 + (a1 >> 2) + (a2 >> 4) - s;  // sum (c-1)*a, exact
        // dot_pq2::<FUSED>, src/kernels.rs:941-955
        const float dd = h2f(w.d) * b->scale;
        const float sf = static_cast<float>(I);
        if constexpr (O == Op::PQ2_UNFUSED) {
            t[0] = dd * sf;
        } else {
            t[0] = dd;
            t[1] = sf;
        }
    } else if constexpr (O == Op::PQ2_Q8) {
        // dot_q8_groups for an odd-group PQ2 row (src/kernels.rs:1043-1064); the pinned
        // contract keeps this order for PQ2 (:1109-1121).  One FMA per group: the binary16
        // scale times |I| <= 32 * 2 * 127 < 2^13 is exact in binary32.
        const Q8Block *b = static_cast<const Q8Block *>(act) + 4 * u;
        float tt = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t *av = reinterpret_cast<const uint32_t *>(b[g].values);
            int a0 = 0, a1 = 0, a2 = 0, s = 0;
#pragma unroll
            for (int h = 0; h < 2; ++h)
                pq2_dword(w.c[2 * g + h], av[4 * h], av[4 * h + 1], av[4 * h + 2], av[4 * h + 3], a0, a1, a2, s);
            tt = __builtin_fmaf(b[g].scale, static_cast<float>(a0 + (a1 >> 2) + (a2 >> 4) - s), tt);
        }
        t[0] = h2f(w.d) * tt;
    } else if constexpr (O == Op::Q2K) {
        const Q8KBlock *b = static_cast<const Q8KBlock *>(act) + u;
        const uint32_t *av = reinterpret_cast<const uint32_t *>(b->values);
        // Code dword w: half h = w/8, bytes 4(w%8).. ; field p -> elements 128h+32p+4(w%8)..+3,
        // sub-block g = 8h + 2p + (w%8 >= 4).  Masking in place scales field p by 4^p; the
        // top field is shifted down first so every code byte stays below 128 (v_dot4 reads
        // signed bytes), leaving fields 2 and 3 both scaled by 16.
        int sb[16];
#pragma unroll
        for (int g = 0; g < 16; ++g) sb[g] = 0;
#pragma unroll
        for (int wd = 0; wd < 16; ++wd) {
            const int h = wd >> 3, wh = wd & 7;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int g = 8 * h + 2 * p + (wh >> 2);
                const uint32_t m = p < 3 ? w.q[wd] & (0x03030303u << (2 * p)) : (w.q[wd] >> 2) & 0x30303030u;
                sb[g] = sdot4(m, av[32 * h + 8 * p + wh], sb[g]);
            }
        }
        int isum = 0, msum = 0;
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            const uint32_t byte = (w.sc[g >> 2] >> (8 * (g & 3))) & 0xffu;
            const int p = (g & 7) >> 1;
            const int shift = p < 3 ? 2 * p : 4;
            isum += static_cast<int>(byte & 15u) * (sb[g] >> shift);
            msum += static_cast<int>(b->sums[g]) * static_cast<int>(byte >> 4);
        }
        // dot_q2_k_block, src/kernels/kquants.rs:193-196
        const float as = b->scale;
        t[0] = (as * h2f(w.dm & 0xffffu)) * static_cast<float>(isum) -
               (as * h2f(w.dm >> 16)) * static_cast<float>(msum);
    } else if constexpr (O == Op::TQ1) {
        // TQ1_0 (src/kernels/tquants.rs:192-215): byte b < 32 digit k -> element b + 32k,
        // byte 32 + b digit k -> 160 + b + 16k, byte 48 + b digit k < 4 -> 240 + b + 4k, so
        // the digit-k quad of a code dword pairs with one natural activation dword.  The
        // digits (trit_k = ((x * 3^k mod 256) * 3) >> 8, as PTQ1) become signed bytes t - 1.
        const Q8KBlock *b = static_cast<const Q8KBlock *>(act) + u;
        const uint32_t *av = reinterpret_cast<const uint32_t *>(b->values);
        int I = 0;
        auto digits = [&](uint32_t x, int nd, int a0, int astep) {
            uint32_t L = x & 0x00ff00ffu, H = (x >> 8) & 0x00ff00ffu;
            for (int k = 0; k < nd; ++k) {
                const uint32_t mL = L * 3u, mH = H * 3u;
                I = sdot4(perm(0u, 0x000100ffu, perm(mH, mL, sel(1, 5, 3, 7))), av[a0 + astep * k], I);
                L = mL & 0x00ff00ffu;
                H = mH & 0x00ff00ffu;
            }
        };
#pragma unroll
        for (int wd = 0; wd < 8; ++wd) digits(w.q[wd], 5, wd, 8);
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) digits(w.q[8 + wd], 5, 40 + wd, 4);
        digits(w.q[12], 4, 60, 1);
        // dot(), src/kernels/tquants.rs:264-270
        t[0] = static_cast<float>(I) * (h2f(w.d) * b->scale);
    } else if constexpr (O == Op::TQ2) {
        // TQ2_0 (src/kernels/tquants.rs:217-238): byte 32h + b field k -> element
        // 128h + 32k + b; fields become signed bytes c - 1.
        const Q8KBlock *b = static_cast<const Q8KBlock *>(act) + u;
        const uint32_t *av = reinterpret_cast<const uint32_t *>(b->values);
        int I = 0;
#pragma unroll
        for (int wd = 0; wd < 16; ++wd) {
            const int h = wd >> 3, wh = wd & 7;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                I = sdot4(perm(0u, 0x020100ffu, (w.q[wd] >> (2 * k)) & 0x03030303u), av[32 * h + 8 * k + wh], I);
        }
        // dot(), src/kernels/tquants.rs:264-270
        t[0] = static_cast<float>(I) * (h2f(w.d) * b->scale);
    } else {
        const Q8Block *b = static_cast<const Q8Block *>(act) + 4 * u;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t *av = reinterpret_cast<const uint32_t *>(b[j].values);
            int I = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) I = sdot4(w.c[8 * j + i], av[i], I);
            const uint32_t sbits = (w.s[j >> 1] >> (16 * (j & 1))) & 0xffffu;
            // dot_legacy, src/kernels.rs:1241-1244
            t[j] = (h2f(sbits) * b[j].scale) * static_cast<float>(I);
        }
    }
}

// Running state of one row's chain.
template <Op O>
struct Chain {
    float o = 0.0f;
    float L[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // pinned PTQ1 lanes

    __device__ __forceinline__ void fold(const float *t, const void *__restrict__ act, uint32_t u) {
        if constexpr (O == Op::PQ2_FUSED) {
            o = __builtin_fmaf(t[0], t[1], o);
        } else if constexpr (O == Op::PTQ1_PINNED) {
            // dot_q8_groups_pinned, src/kernels.rs:1134-1146
            const Q8Block *b = static_cast<const Q8Block *>(act) + 4 * u;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float dd = t[8] * b[g].scale;
                const uint32_t p0 = __float_as_uint(t[2 * g]), p1 = __float_as_uint(t[2 * g + 1]);
                L[0] = __builtin_fmaf(static_cast<float>(static_cast<int16_t>(p0 & 0xffffu)), dd, L[0]);
                L[1] = __builtin_fmaf(static_cast<float>(static_cast<int16_t>(p0 >> 16)), dd, L[1]);
                L[2] = __builtin_fmaf(static_cast<float>(static_cast<int16_t>(p1 & 0xffffu)), dd, L[2]);
                L[3] = __builtin_fmaf(static_cast<float>(static_cast<int16_t>(p1 >> 16)), dd, L[3]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < terms_per_unit<O>(); ++j) o = o + t[j];
        }
    }
    __device__ __forceinline__ float result() const {
        if constexpr (O == Op::PTQ1_PINNED) return (L[0] + L[1]) + (L[2] + L[3]);
        return o;
    }
};

// Kernel parameters (passed by value).
struct MvParams {
    const uint8_t *w[2];  // tiled weights; w[1] is the FFN up matrix when NMAT == 2
    uint32_t rows, nu, cols;
    const void *act;      // prepared blocks, or f32 input when the prologue quantizes
    int qcontract;        // prologue quantizer: Q8_K pinned flag / Q8_0 contract
    int pinned;           // SwiGLU order (NMAT == 2)
    uint32_t ks, lpr;     // split mode: wavefronts per matrix, lanes per row (powers of two)
    uint32_t lg_ks, lg_lpr;  // their base-2 logarithms
    uint32_t xcd_tiles;      // split mode: a tile's lpr workgroups share one XCD (tiles % 8 == 0)
    float *out;
    const float *residual;
    int *err;
    const float *norm_w;  // QUANT prologue: RMSNorm weights applied before quantizing (or null)
    float eps;            // RMSNorm epsilon
    Q8Block *q8_out;      // NMAT == 2: the SwiGLU vector quantized to Q8_0 blocks (or null)
    int q8_contract;      // their contract (PRISM_Q8_*)
    TileBest *tile_best;  // k_mv_rows: per tile, its largest output and first row (or null)
};

template <Op O>
constexpr bool act_is_q8k() {
    return O == Op::PTQ1_Q8K || O == Op::PQ2_UNFUSED || O == Op::PQ2_FUSED || O == Op::Q2K || O == Op::TQ1 ||
           O == Op::TQ2;
}

// Prepared-activation bytes for `cols` inputs (one token).
template <Op O>
__host__ __device__ constexpr uint32_t act_bytes_for(uint32_t cols) {
    return act_is_q8k<O>() ? cols / 256 * static_cast<uint32_t>(sizeof(Q8KBlock))
                           : cols / 32 * static_cast<uint32_t>(sizeof(Q8Block));
}

__host__ __device__ constexpr uint32_t align16(uint32_t v) { return (v + 15u) & ~15u; }

template <Op O>
struct ActBlock {
    using type = typename std::conditional<act_is_q8k<O>(), Q8KBlock, Q8Block>::type;
};

// Big matrices: one wavefront per 64-row tile walks the whole row; the prepared
// activation (global, wave-uniform) arrives through scalar loads and the chain
// stays in registers.
template <Op O, bool LUT>
__device__ __forceinline__ void rows_tile(const MvParams &p, const void *__restrict__ act, uint32_t tile, uint32_t lane,
                                          uint32_t lbase) {
    constexpr uint32_t UB = unit_bytes<O>();
    const uint32_t nu = p.nu, row_bytes = nu * UB;
    const uint32_t left = p.rows - tile * kTile;
    const uint32_t trows = left < kTile ? left : kTile;
    const uint32_t trp = (trows + 7u) & ~7u;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.w[0] + static_cast<size_t>(tile) * kTile * row_bytes, trp * row_bytes);
    Chain<O> ch;
    auto step = [&](const Raw<O> &w, uint32_t u) {
        float t[terms_per_unit<O>()];
        unit_terms<O, LUT>(w, act, u, t, lbase);
        ch.fold(t, act, u);
    };
    // Two register buffers in ping-pong: the next unit's loads are in flight while the
    // current one is decoded, and no buffer is copied (a copy would wait for the loads).
    // Deeper rings spill at the table kernel's 128 registers (measured: three buffers
    // 2.5x slower at 151936 rows).
    Raw<O> A, B;
    uint32_t u = 0;
    load_unit<O>(A, rs, 0, trp, lane);
    while (u + 1 < nu) {
        load_unit<O>(B, rs, (u + 1) * trp * UB, trp, lane);
        step(A, u);
        if (u + 2 < nu) load_unit<O>(A, rs, (u + 2) * trp * UB, trp, lane);
        step(B, u + 1);
        u += 2;
    }
    if (u < nu) step(A, u);
    const size_t row = static_cast<size_t>(tile) * kTile + lane;
    float o = 0.0f;
    if (lane < trows) {
        o = ch.result();
        if (p.residual) o = o + p.residual[row];
        p.out[row] = o;
        if (!finite(o)) raise_error(p.err, kErrNonfinite);
    }
    if (p.tile_best) {
        // The tile's largest output and its first row: lanes past the tile's rows hold no
        // row, and of equal values the lower row wins (the order of a first-index argmax).
        uint32_t r = lane < trows ? static_cast<uint32_t>(row) : 0xffffffffu;
#pragma unroll
        for (int k = 32; k >= 1; k >>= 1) {
            const float ov = __shfl_xor(o, k);
            const uint32_t orow = __shfl_xor(r, k);
            if (r == 0xffffffffu || (orow != 0xffffffffu && (ov > o || (ov == o && orow < r)))) {
                o = ov;
                r = orow;
            }
        }
        if (lane == 0) p.tile_best[tile] = TileBest{o, r};
    }
}

template <Op O>
__global__ __launch_bounds__(64) void k_mv_rows(MvParams p) {
    rows_tile<O, false>(p, p.act, blockIdx.x, threadIdx.x, 0);
}

// Units [u0, u1) of one 64-row tile: folded into `ch`, or, with `tout`, their terms
// stored to tout[(u - u0) * TPU + j] for another wavefront to fold.
template <Op O, bool LUT>
__device__ __forceinline__ void rows_part(const MvParams &p, const void *__restrict__ act, uint32_t tile, uint32_t lane,
                                          uint32_t lbase, uint32_t u0, uint32_t u1, Chain<O> &ch, float *tout) {
    constexpr uint32_t UB = unit_bytes<O>();
    const uint32_t row_bytes = p.nu * UB;
    const uint32_t left = p.rows - tile * kTile;
    const uint32_t trows = left < kTile ? left : kTile;
    const uint32_t trp = (trows + 7u) & ~7u;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.w[0] + static_cast<size_t>(tile) * kTile * row_bytes, trp * row_bytes);
    auto step = [&](const Raw<O> &w, uint32_t u) {
        float t[terms_per_unit<O>()];
        unit_terms<O, LUT>(w, act, u, t, lbase);
        if (tout) {
#pragma unroll
            for (int j = 0; j < terms_per_unit<O>(); ++j) tout[(u - u0) * terms_per_unit<O>() + j] = t[j];
        } else {
            ch.fold(t, act, u);
        }
    };
    Raw<O> A, B;
    uint32_t u = u0;
    load_unit<O>(A, rs, u * trp * UB, trp, lane);
    while (u + 1 < u1) {
        load_unit<O>(B, rs, (u + 1) * trp * UB, trp, lane);
        step(A, u);
        if (u + 2 < u1) load_unit<O>(A, rs, (u + 2) * trp * UB, trp, lane);
        step(B, u + 1);
        u += 2;
    }
    if (u < u1) step(A, u);
}

// Two wavefronts per 64-row tile: wavefront 1 computes the terms of the second half of
// the units into LDS (dynamic, 64 rows x `stride` floats), wavefront 0 folds the first
// half and then, after one barrier, those terms in unit order: the unsplit row's
// arithmetic, with twice the wavefronts and half the serial chain each.
template <Op O>
__global__ __launch_bounds__(128) void k_mv_rows2(MvParams p, uint32_t stride) {
    static_assert(O != Op::PTQ1_PINNED, "four-lane chains fold nine terms per unit");
    extern __shared__ float second[];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t half = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tile = blockIdx.x, nh = (p.nu + 1) / 2;
    float *mine = second + lane * stride;
    Chain<O> ch;
    if (half == 0)
        rows_part<O, false>(p, p.act, tile, lane, 0, 0, nh, ch, nullptr);
    else
        rows_part<O, false>(p, p.act, tile, lane, 0, nh, p.nu, ch, mine);
    __syncthreads();
    if (half == 0) {
        for (uint32_t u = nh; u < p.nu; ++u) ch.fold(mine + (u - nh) * terms_per_unit<O>(), p.act, u);
        const uint32_t left = p.rows - tile * kTile;
        if (lane < (left < kTile ? left : kTile)) {
            const size_t row = static_cast<size_t>(tile) * kTile + lane;
            float o = ch.result();
            if (p.residual) o = o + p.residual[row];
            p.out[row] = o;
            if (!finite(o)) raise_error(p.err, kErrNonfinite);
        }
    }
}

// NW wavefronts per 64-row tile (half a tile to four tiles per CU, prepared activations): wavefront
// k walks the contiguous units [k * nu / NW, (k + 1) * nu / NW); wavefront 0 folds its own
// units straight into the chain and the others leave their units' terms in LDS (row-major,
// odd `stride`), which wavefront 0 folds after one barrier in unit order: the unsplit
// row's arithmetic with NW wavefronts loading and decoding.
template <Op O, uint32_t NW>
__global__ __launch_bounds__(64 * NW) void k_mv_rowsn(MvParams p, uint32_t stride) {
    static_assert(O != Op::PTQ1_PINNED, "four-lane chains fold nine terms per unit");
    extern __shared__ float later[];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t k = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tile = blockIdx.x, nu = p.nu, c1 = nu / NW;
    const uint32_t u0 = k * nu / NW, u1 = (k + 1) * nu / NW;
    float *mine = later + lane * stride;
    Chain<O> ch;
    if (k == 0)
        rows_part<O, false>(p, p.act, tile, lane, 0, 0, c1, ch, nullptr);
    else if (u0 < u1)
        rows_part<O, false>(p, p.act, tile, lane, 0, u0, u1, ch, mine + (u0 - c1) * terms_per_unit<O>());
    __syncthreads();
    if (k == 0) {
        for (uint32_t u = c1; u < nu; ++u) ch.fold(mine + (u - c1) * terms_per_unit<O>(), p.act, u);
        const uint32_t left = p.rows - tile * kTile;
        if (lane < (left < kTile ? left : kTile)) {
            const size_t row = static_cast<size_t>(tile) * kTile + lane;
            float o = ch.result();
            if (p.residual) o = o + p.residual[row];
            p.out[row] = o;
            if (!finite(o)) raise_error(p.err, kErrNonfinite);
        }
    }
}

// PTQ1 with the LDS decode table: one workgroup per CU builds the 64 KiB table once and
// works through its tiles (tile = block + j * grid, j = 0, 1, ...), which spreads the
// tiles evenly over the CUs.  The activation comes as its own __restrict__ argument: the
// row stores of one tile then provably leave it intact for the next, and its loads stay
// scalar.
//
// When a workgroup has at most eight tiles (up to 131072 rows on 256 CUs), single-term
// formats split every tile's units in two halves run by two wavefronts (wavefront w
// takes half w % 2 of tile w / 2): the second half stores its terms in LDS, and after a
// barrier the first half's wavefront continues its chain with them in unit order, so the
// arithmetic is the unsplit row's.  Two to eight tiles then keep twice as many
// wavefronts (and SIMDs) busy.  With more tiles the wavefronts already fill the SIMDs
// and take whole tiles (measured: splitting nine tiles per CU in two rounds was slower).
constexpr uint32_t kLutThreads = 1024;
constexpr uint32_t kLutWaves = kLutThreads / 64;
// Modes: kLutWhole: every wavefront takes whole tiles round-robin.  kLutSplit (single-term
// formats, at most kLutSlots tiles per workgroup and 64 units per row, lut_split()): the
// two-wavefront halves above.  kLutTail (8 to 12 tiles per CU, lut_tail_lds()): wavefronts
// 0..7 take one whole tile each, and wavefronts 8..15 take the remaining tiles as split
// pairs, so the last round of tiles costs half a tile on the busiest SIMD instead of a
// whole one.  Their second halves' terms go to dynamic LDS, 64 rows x lut_tail_stride()
// floats per pair, beside the 64 KiB table: pinned PTQ1 (nine terms per unit) fits two
// pairs at 4096 columns, so it takes this form up to ten tiles per CU.
// kLutSpread (prepared activations, half a tile to eight tiles per CU): a workgroup takes
// `per` = 1, 2, 4 or 8 tiles (lut_spread_slots) and gives each 16 / per wavefronts, which
// take its units round-robin and leave each unit's terms for the tile's 64 rows in dynamic
// LDS ([tile slot][unit][term][row], lut_spread_lds()); after one barrier the first
// wavefront of each tile folds them in unit order: the unsplit row's arithmetic.
constexpr uint32_t kLutSlots = kLutWaves / 2;
constexpr int kLutWhole = 0, kLutSplit = 1, kLutTail = 2, kLutSpread = 3;
__host__ __device__ inline uint32_t lut_spread_slots(uint32_t tiles, uint32_t grid) {
    const uint32_t need = (tiles + grid - 1) / grid;
    return need <= 1 ? 1u : need <= 2 ? 2u : need <= 4 ? 4u : 8u;
}
// Dynamic LDS bytes of the spread form for this launch (grid = min(tiles, CUs)), 0 where
// it does not apply.
template <Op O>
inline uint32_t lut_spread_lds(uint32_t tiles, uint32_t grid, uint32_t nu) {
    if (tiles > 8 * grid) return 0u;
    const uint32_t bytes =
        lut_spread_slots(tiles, grid) * nu * terms_per_unit<O>() * kTile * static_cast<uint32_t>(sizeof(float));
    return bytes + sizeof(g_ptq1_lut) <= 160u * 1024u ? bytes : 0u;
}
template <Op O>
__host__ __device__ constexpr bool lut_can_split() {
    return terms_per_unit<O>() == 1;
}
__host__ __device__ inline bool lut_split(uint32_t tiles, uint32_t grid, uint32_t nu) {
    return tiles <= kLutSlots * grid && nu - (nu + 1) / 2 <= 32;
}
// Second-half terms per row, odd (no bank conflicts between the rows' lanes).
template <Op O>
__host__ __device__ constexpr uint32_t lut_tail_stride(uint32_t nu) {
    return ((nu - (nu + 1) / 2) * terms_per_unit<O>()) | 1u;
}
// Dynamic LDS bytes of the tail form for this launch, 0 where it does not apply.
template <Op O>
inline uint32_t lut_tail_lds(uint32_t tiles, uint32_t grid, uint32_t nu) {
    if (tiles <= 8 * grid || tiles > 12 * grid) return 0;
    const uint32_t pairs = (tiles - 8 * grid + grid - 1) / grid;
    const uint32_t bytes = pairs * kTile * lut_tail_stride<O>(nu) * static_cast<uint32_t>(sizeof(float));
    return bytes + sizeof(g_ptq1_lut) <= 160u * 1024u ? bytes : 0u;
}
template <Op O, int MODE>
__global__ __launch_bounds__(kLutThreads) void k_mv_rows_lut(MvParams p, const void *__restrict__ act) {
    ptq1_lut_fill(threadIdx.x, blockDim.x);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tiles = (p.rows + kTile - 1) / kTile;
    const uint32_t lbase = 8u * (lane & 31u);
    if constexpr (MODE == kLutWhole) {
        const uint32_t step = gridDim.x * kLutWaves;
        for (uint32_t tile = wave * gridDim.x + blockIdx.x; tile < tiles; tile += step)
            rows_tile<O, true>(p, act, tile, lane, lbase);
    } else if constexpr (MODE == kLutSpread) {
        extern __shared__ float spread_terms[];
        constexpr uint32_t UB = unit_bytes<O>(), TPU = terms_per_unit<O>();
        const uint32_t nu = p.nu, grid = __builtin_amdgcn_readfirstlane(gridDim.x);
        const uint32_t per = lut_spread_slots(tiles, grid), W = kLutWaves / per;
        const uint32_t slot = wave / W, sub = wave % W;
        const uint32_t tile = blockIdx.x + slot * grid;
        const bool active = tile < tiles;  // uniform per wavefront
        float *mine = spread_terms + static_cast<size_t>(slot) * nu * TPU * kTile;
        const uint32_t left = active ? p.rows - tile * kTile : 0u;
        const uint32_t trows = left < kTile ? left : kTile;
        const uint32_t trp = (trows + 7u) & ~7u;
        if (active) {
            const __amdgpu_buffer_rsrc_t rs =
                make_rsrc(p.w[0] + static_cast<size_t>(tile) * kTile * nu * UB, trp * nu * UB);
            auto terms = [&](const Raw<O> &w, uint32_t u) {
                float t[TPU];
                unit_terms<O, true>(w, act, u, t, lbase);
#pragma unroll
                for (uint32_t j = 0; j < TPU; ++j) mine[(u * TPU + j) * kTile + lane] = t[j];
            };
            // Units sub, sub + W, ...: two register buffers in ping-pong.
            Raw<O> A, B;
            uint32_t u = sub;
            if (u < nu) load_unit<O>(A, rs, u * trp * UB, trp, lane);
            while (u + W < nu) {
                load_unit<O>(B, rs, (u + W) * trp * UB, trp, lane);
                terms(A, u);
                if (u + 2 * W < nu) load_unit<O>(A, rs, (u + 2 * W) * trp * UB, trp, lane);
                terms(B, u + W);
                u += 2 * W;
            }
            if (u < nu) terms(A, u);
        }
        __syncthreads();  // every wavefront reaches this one barrier
        if (active && sub == 0) {
            Chain<O> ch;
            for (uint32_t v = 0; v < nu; ++v) {
                float t[TPU];
#pragma unroll
                for (uint32_t j = 0; j < TPU; ++j) t[j] = mine[(v * TPU + j) * kTile + lane];
                ch.fold(t, act, v);
            }
            if (lane < trows) {
                const size_t row = static_cast<size_t>(tile) * kTile + lane;
                float o = ch.result();
                if (p.residual) o = o + p.residual[row];
                p.out[row] = o;
                if (!finite(o)) raise_error(p.err, kErrNonfinite);
            }
        }
    } else if constexpr (MODE == kLutTail) {
        // Terms of the tail tiles' second halves: pair `slot` at slot * kTile * stride,
        // row `lane` at lane * stride.  A pair is active only if its tile exists, and the
        // host sized the buffer for every pair a workgroup can have.
        extern __shared__ float tail_terms[];
        constexpr uint32_t TPU = terms_per_unit<O>();
        const uint32_t nh = (p.nu + 1) / 2, stride = lut_tail_stride<O>(p.nu);
        const uint32_t slot = (wave - 8) >> 1, half = wave & 1u;
        const uint32_t tile = wave < 8 ? wave * gridDim.x + blockIdx.x : 8 * gridDim.x + slot * gridDim.x + blockIdx.x;
        const bool active = tile < tiles;
        float *mine = tail_terms + (static_cast<size_t>(slot) * kTile + lane) * stride;
        Chain<O> ch;
        if (wave < 8) {
            rows_tile<O, true>(p, act, tile, lane, lbase);  // tile < 8 * gridDim.x < tiles
        } else if (active) {
            if (half == 0)
                rows_part<O, true>(p, act, tile, lane, lbase, 0, nh, ch, nullptr);
            else
                rows_part<O, true>(p, act, tile, lane, lbase, nh, p.nu, ch, mine);
        }
        __syncthreads();  // every wavefront reaches this one barrier
        if (wave >= 8 && active && half == 0) {
            for (uint32_t u = nh; u < p.nu; ++u) ch.fold(mine + (u - nh) * TPU, act, u);
            const uint32_t left = p.rows - tile * kTile;
            if (lane < (left < kTile ? left : kTile)) {
                const size_t row = static_cast<size_t>(tile) * kTile + lane;
                float o = ch.result();
                if (p.residual) o = o + p.residual[row];
                p.out[row] = o;
                if (!finite(o)) raise_error(p.err, kErrNonfinite);
            }
        }
    } else {
        static_assert(lut_can_split<O>(), "single-term formats only");
        __shared__ float second[kLutSlots][kTile][33];  // terms of a tile's second half (<= 32 units)
        const uint32_t mine = blockIdx.x < tiles ? (tiles - blockIdx.x + gridDim.x - 1) / gridDim.x : 0;
        const uint32_t nh = (p.nu + 1) / 2;  // units of the first half
        {
            const uint32_t slot = wave >> 1, half = wave & 1u, j = slot;
            const bool active = j < mine;
            const uint32_t tile = blockIdx.x + j * gridDim.x;
            Chain<O> ch;
            if (active) {
                if (half == 0)
                    rows_part<O, true>(p, act, tile, lane, lbase, 0, nh, ch, nullptr);
                else
                    rows_part<O, true>(p, act, tile, lane, lbase, nh, p.nu, ch, second[slot][lane]);
            }
            __syncthreads();
            if (active && half == 0) {
                const float *t = second[slot][lane];
                for (uint32_t u = nh; u < p.nu; ++u) ch.fold(t + (u - nh), act, u);
                const uint32_t left = p.rows - tile * kTile;
                if (lane < (left < kTile ? left : kTile)) {
                    const size_t row = static_cast<size_t>(tile) * kTile + lane;
                    float o = ch.result();
                    if (p.residual) o = o + p.residual[row];
                    p.out[row] = o;
                    if (!finite(o)) raise_error(p.err, kErrNonfinite);
                }
            }
        }
    }
}

// PTQ1 batches of NB = 2 or 3 tokens on the table kernel: each unit of weights is loaded
// and decoded once and folded into one chain per token (every chain in its own token's
// unit order, the batch-1 arithmetic).  Token t's prepared activation sits at
// act + t * act_stride bytes and its output rows at out + t * rows (residual likewise).
// With the tokens' decode shared, a few tokens cost little more than one, where the
// matrix-core skinny kernel pays its own decode.
template <Op O, int NB>
__global__ __launch_bounds__(kLutThreads) void k_mv_rows_lut_batch(MvParams p, const void *__restrict__ act,
                                                                   uint32_t act_stride) {
    constexpr uint32_t UB = unit_bytes<O>();
    ptq1_lut_fill(threadIdx.x, blockDim.x);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tiles = (p.rows + kTile - 1) / kTile;
    const uint32_t lbase = 8u * (lane & 31u);
    const uint32_t nu = p.nu, row_bytes = nu * UB;
    for (uint32_t tile = wave * gridDim.x + blockIdx.x; tile < tiles; tile += gridDim.x * kLutWaves) {
        const uint32_t left = p.rows - tile * kTile;
        const uint32_t trows = left < kTile ? left : kTile;
        const uint32_t trp = (trows + 7u) & ~7u;
        const __amdgpu_buffer_rsrc_t rs =
            make_rsrc(p.w[0] + static_cast<size_t>(tile) * kTile * row_bytes, trp * row_bytes);
        Chain<O> ch[NB];
        auto step = [&](const Raw<O> &w, uint32_t u) {
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                const void *a = static_cast<const uint8_t *>(act) + static_cast<size_t>(t) * act_stride;
                float tt[terms_per_unit<O>()];
                unit_terms<O, true>(w, a, u, tt, lbase);
                ch[t].fold(tt, a, u);
            }
        };
        Raw<O> A, B;
        uint32_t u = 0;
        load_unit<O>(A, rs, 0, trp, lane);
        while (u + 1 < nu) {
            load_unit<O>(B, rs, (u + 1) * trp * UB, trp, lane);
            step(A, u);
            if (u + 2 < nu) load_unit<O>(A, rs, (u + 2) * trp * UB, trp, lane);
            step(B, u + 1);
            u += 2;
        }
        if (u < nu) step(A, u);
        if (lane < trows) {
            const size_t row = static_cast<size_t>(tile) * kTile + lane;
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                const size_t at = static_cast<size_t>(t) * p.rows + row;
                float o = ch[t].result();
                if (p.residual) o = o + p.residual[at];
                p.out[at] = o;
                if (!finite(o)) raise_error(p.err, kErrNonfinite);
            }
        }
    }
}

// Skinny batches (2..NB tokens, the matvec-to-matmul transition): one wavefront per
// 64-row tile loads each unit of weights once and folds it into one chain per token,
// every chain in its own token's unit order.  Token t's prepared activation sits at
// act + t * act_stride bytes and its output row block at out + t * rows (residual
// likewise).  The per-token chain and arithmetic are exactly the batch-1 ones.
template <Op O, int NB>
__global__ __launch_bounds__(64) void k_mv_rows_batch(MvParams p, const void *__restrict__ act, uint32_t ntok,
                                                      uint32_t act_stride) {
    constexpr uint32_t UB = unit_bytes<O>();
    const uint32_t lane = threadIdx.x, tile = blockIdx.x;
    const uint32_t nu = p.nu, row_bytes = nu * UB;
    const uint32_t left = p.rows - tile * kTile;
    const uint32_t trows = left < kTile ? left : kTile;
    const uint32_t trp = (trows + 7u) & ~7u;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.w[0] + static_cast<size_t>(tile) * kTile * row_bytes, trp * row_bytes);
    Chain<O> ch[NB];
    auto step = [&](const Raw<O> &w, uint32_t u) {
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            if (t < static_cast<int>(ntok)) {
                const void *a = static_cast<const uint8_t *>(act) + static_cast<size_t>(t) * act_stride;
                float tt[terms_per_unit<O>()];
                unit_terms<O>(w, a, u, tt);
                ch[t].fold(tt, a, u);
            }
        }
    };
    Raw<O> A, B;
    uint32_t u = 0;
    load_unit<O>(A, rs, 0, trp, lane);
    while (u + 1 < nu) {
        load_unit<O>(B, rs, (u + 1) * trp * UB, trp, lane);
        step(A, u);
        if (u + 2 < nu) load_unit<O>(A, rs, (u + 2) * trp * UB, trp, lane);
        step(B, u + 1);
        u += 2;
    }
    if (u < nu) step(A, u);
    if (lane < trows) {
        const size_t row = static_cast<size_t>(tile) * kTile + lane;
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            if (t < static_cast<int>(ntok)) {
                const size_t at = static_cast<size_t>(t) * p.rows + row;
                float o = ch[t].result();
                if (p.residual) o = o + p.residual[at];
                p.out[at] = o;
                if (!finite(o)) raise_error(p.err, kErrNonfinite);
            }
        }
    }
}

// ---- long rows on few tiles: split-K through global memory -----------------------------
// With fewer tiles than CUs and long rows, one workgroup per tile walks a long serial chain of
// units.  Here the units are split over workgroups instead: k_mv_terms (one wavefront per
// tile and range of upw units) computes every unit's terms of the tile's rows for every token
// and stores them at terms[((t * nu + u) * TPU + j) * rp + row] (rp: rows rounded up to whole
// tiles); k_mv_fold then folds each (token, row) element's terms in unit order -- the unsplit
// chain, so every output equals its matvec bit for bit.
template <Op O>
__global__ __launch_bounds__(64) void k_mv_terms(MvParams p, const void *__restrict__ act, uint32_t act_stride,
                                                 uint32_t ntok, uint32_t upw, float *__restrict__ terms, uint32_t rp) {
    constexpr uint32_t UB = unit_bytes<O>();
    constexpr int TPU = terms_per_unit<O>();
    const uint32_t lane = threadIdx.x, tile = blockIdx.x;
    const uint32_t nu = p.nu, row_bytes = nu * UB;
    const uint32_t u0 = blockIdx.y * upw, u1 = u0 + upw < nu ? u0 + upw : nu;
    const uint32_t left = p.rows - tile * kTile;
    const uint32_t trows = left < kTile ? left : kTile;
    const uint32_t trp = (trows + 7u) & ~7u;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.w[0] + static_cast<size_t>(tile) * kTile * row_bytes, trp * row_bytes);
    float *tr = terms + static_cast<size_t>(tile) * kTile + lane;  // rows past the matrix: zero weights, never folded
    auto step = [&](const Raw<O> &w, uint32_t u) {
        // A PTQ1 unit's trits are extracted once for all tokens.
        auto unit = [&](const auto &dec) {
            for (uint32_t t = 0; t < ntok; ++t) {
                const void *a = static_cast<const uint8_t *>(act) + static_cast<size_t>(t) * act_stride;
                float tt[TPU];
                unit_terms<O, false, std::remove_cvref_t<decltype(dec)>>(dec, a, u, tt);
#pragma unroll
                for (int j = 0; j < TPU; ++j) tr[((static_cast<size_t>(t) * nu + u) * TPU + j) * rp] = tt[j];
            }
        };
        if constexpr (kind_of<O>() == kPTQ1) {
            Ptq1Dec D;
            ptq1_decode(w.x, D);
            unit(D);
        } else {
            unit(w);
        }
    };
    Raw<O> A, B;
    uint32_t u = u0;
    load_unit<O>(A, rs, u * trp * UB, trp, lane);
    while (u + 1 < u1) {
        load_unit<O>(B, rs, (u + 1) * trp * UB, trp, lane);
        step(A, u);
        if (u + 2 < u1) load_unit<O>(A, rs, (u + 2) * trp * UB, trp, lane);
        step(B, u + 1);
        u += 2;
    }
    if (u < u1) step(A, u);
}

// Rows per k_mv_fold workgroup whose terms fit kFoldLds (0: none do).
constexpr uint32_t kFoldLds = 64 * 1024;
template <Op O>
uint32_t fold_rows(uint32_t nu) {
    for (uint32_t rf = 64; rf >= 8; rf >>= 1)
        if (static_cast<uint64_t>(rf) * nu * terms_per_unit<O>() * sizeof(float) <= kFoldLds) return rf;
    return 0;
}

// Workgroup (block of rf rows, token t): every unit's terms of its rows staged in LDS with
// all loads issued at once (consecutive threads take consecutive rows of one term), then rf
// threads fold their row's terms in unit order.
template <Op O>
__global__ __launch_bounds__(256) void k_mv_fold(MvParams p, const void *__restrict__ act, uint32_t act_stride,
                                                 const float *__restrict__ terms, uint32_t rp, uint32_t lg_rf) {
    constexpr int TPU = terms_per_unit<O>();
    constexpr uint32_t kBatch = 8;  // loads in flight per thread, and LDS reads ahead of the chain
    extern __shared__ float staged[];  // [nu * TPU][rf]
    const uint32_t rf = 1u << lg_rf, t = blockIdx.y, row0 = blockIdx.x * rf, n = p.nu * TPU;
    const float *src = terms + static_cast<size_t>(t) * n * rp + row0;
    const uint32_t total = n * rf;
    for (uint32_t i0 = threadIdx.x; i0 < total; i0 += 256 * kBatch) {
        float v[kBatch];
#pragma unroll
        for (uint32_t b = 0; b < kBatch; ++b) {
            const uint32_t i = i0 + 256 * b;
            v[b] = i < total ? src[static_cast<size_t>(i >> lg_rf) * rp + (i & (rf - 1))] : 0.0f;
        }
#pragma unroll
        for (uint32_t b = 0; b < kBatch; ++b)
            if (i0 + 256 * b < total) staged[i0 + 256 * b] = v[b];
    }
    __syncthreads();
    const uint32_t r = threadIdx.x;
    if (r >= rf || row0 + r >= p.rows) return;
    const void *a = static_cast<const uint8_t *>(act) + static_cast<size_t>(t) * act_stride;
    Chain<O> ch;
    uint32_t u = 0;
    for (; u + kBatch <= p.nu; u += kBatch) {
        float tt[kBatch][TPU];
#pragma unroll
        for (uint32_t b = 0; b < kBatch; ++b)
#pragma unroll
            for (int j = 0; j < TPU; ++j) tt[b][j] = staged[(((u + b) * TPU + j) << lg_rf) + r];
#pragma unroll
        for (uint32_t b = 0; b < kBatch; ++b) ch.fold(tt[b], a, u + b);
    }
    for (; u < p.nu; ++u) {
        float tt[TPU];
#pragma unroll
        for (int j = 0; j < TPU; ++j) tt[j] = staged[((u * TPU + j) << lg_rf) + r];
        ch.fold(tt, a, u);
    }
    const size_t at = static_cast<size_t>(t) * p.rows + row0 + r;
    float o = ch.result();
    if (p.residual) o = o + p.residual[at];
    p.out[at] = o;
    if (!finite(o)) raise_error(p.err, kErrNonfinite);
}

// Row count from which a skinny batch runs weights-once: one wavefront per tile needs
// several tiles per SIMD before the per-token chains stop dominating (measured: at
// 12288 rows token-by-token launches are faster, at 151936 weights-once is 1.5-4x).
constexpr uint64_t kBatchMinRows = 65536;
constexpr uint32_t kBatchMax = 16;

// ---- skinny batches on the int8 matrix cores ------------------------------------------
// 2..16 tokens.  A wavefront owns 16 rows (a quarter of a 64-row tile) and every token,
// and computes the exact integer dot of each (row, token, group) with one
// v_mfma_i32_16x16x32_i8 (a 32-element group) or v_mfma_i32_16x16x64_i8: rows on the M
// side (lane l supplies row l%16), tokens on the N side (lane l supplies token l%16),
// and the group's elements spread over the four lane groups s = l/16 in any order, as
// long as a lane's weight and activation bytes pair the same elements -- the integer
// dot is exact in every order.  Lane l receives rows 4s..4s+3 of token l%16 and runs
// those four rows' binary32 chains for that token in unit order, with the batch-1
// arithmetic, so every output equals its own matvec bit for bit.  The weights of the
// 16 rows are decoded once for all tokens, straight into the operand layout (no LDS).
typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

struct SkParams {
    const uint8_t *w;   // tiled weights
    const uint8_t *sw;  // lane-ordered activations (k_sk_prep), or the prepared blocks
    float *out;         // [ntok][rows]
    const float *residual;
    int *err;
    uint32_t rows, nu, ntok;  // ntok: every chunk's tokens (16 per chunk, the last one fewer)
    uint32_t act_stride;      // prepared blocks: bytes per token
    uint32_t sw_chunk;        // bytes from one chunk's activations in `sw` to the next's
};

// binary32 terms per unit and (row, token) element of the skinny kernel: those of the
// row kernels, except pinned PTQ1, whose four group scales are already multiplied by
// the token's block scales: 8 dwords of packed 16-bit lane sums, then the four dd_g.
template <Op O>
constexpr int sk_terms_per_unit() {
    return O == Op::PTQ1_PINNED ? 12 : terms_per_unit<O>();
}

// Chain of one (row, token) element of the skinny kernel.
template <Op O>
struct SkChain : Chain<O> {
    __device__ __forceinline__ void fold(const float *t) { Chain<O>::fold(t, nullptr, 0); }
};
template <>
struct SkChain<Op::PTQ1_PINNED> : Chain<Op::PTQ1_PINNED> {
    // dot_q8_groups_pinned, src/kernels.rs:1134-1146: per group, L[l] = fma(I_l, dd_g, L[l]).
    __device__ __forceinline__ void fold(const float *t) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float dd = t[8 + g];
            const uint32_t p0 = __float_as_uint(t[2 * g]), p1 = __float_as_uint(t[2 * g + 1]);
            L[0] = __builtin_fmaf(static_cast<float>(static_cast<int16_t>(p0 & 0xffffu)), dd, L[0]);
            L[1] = __builtin_fmaf(static_cast<float>(static_cast<int16_t>(p0 >> 16)), dd, L[1]);
            L[2] = __builtin_fmaf(static_cast<float>(static_cast<int16_t>(p1 & 0xffffu)), dd, L[2]);
            L[3] = __builtin_fmaf(static_cast<float>(static_cast<int16_t>(p1 >> 16)), dd, L[3]);
        }
    }
};

// Per-lane geometry: the tile's buffer, the lane's A row and first output row.
struct SkLane {
    __amdgpu_buffer_rsrc_t rs;
    uint32_t trp, ra, rc, s, lane, tok;
    const uint8_t *sw, *scales;  // lane-ordered activation operands and token scales
};

__device__ __forceinline__ v4i mfma32(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, v4i c) {
    const long a = static_cast<long>((static_cast<uint64_t>(a1) << 32) | a0);
    const long b = static_cast<long>((static_cast<uint64_t>(b1) << 32) | b0);
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4i mfma64(const u32x4 &a, const u32x4 &b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, a), __builtin_bit_cast(v4i, b), c, 0, 0, 0);
}
// Four signed bytes from four small codes: byte value c becomes map's byte c.
__device__ __forceinline__ uint32_t code_map(uint32_t codes, uint32_t map) { return perm(0u, map, codes); }
// Bytes x*m (two 16-bit lanes, each byte times m, products below 256).
__device__ __forceinline__ uint32_t bytes_times(uint32_t x, uint32_t m) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, x) * u16x2{static_cast<uint16_t>(m),
                                                                               static_cast<uint16_t>(m)});
}
// PTQ1 digits of the four bytes of x: byte j gets digit k_j, selected by the per-16-bit
// lane multipliers pl (bytes 0, 2) and ph (bytes 1, 3), each 3^k (mod-256 remainder
// then times 3, the digit in the high byte), as signed trits t-1.
__device__ __forceinline__ uint32_t trit_quad(uint32_t x, uint32_t pl, uint32_t ph) {
    const uint32_t L = x & 0x00ff00ffu, H = (x >> 8) & 0x00ff00ffu;
    const uint32_t mL = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, L) * __builtin_bit_cast(u16x2, pl)) &
                        0x00ff00ffu;
    const uint32_t mH = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, H) * __builtin_bit_cast(u16x2, ph)) &
                        0x00ff00ffu;
    return code_map(perm(mH * 3u, mL * 3u, sel(1, 5, 3, 7)), 0x000100ffu);
}

// Activation operand bytes per lane and unit in the lane-ordered copy (k_sk_prep).
template <Op O>
constexpr uint32_t sk_lane_bytes() {
    return O == Op::Q2K || O == Op::TQ1 || O == Op::TQ2 ? 64 : 32;
}
// 256-element units with one Q8_K block each.
template <Op O>
constexpr bool sk_super_block() {
    return O == Op::Q2K || O == Op::TQ1 || O == Op::TQ2;
}

template <Op O>
struct SkFrag;
template <>
struct SkFrag<Op::Q8_0> {
    u32x2 a[4];
    u32x4 sc0, sc1;  // binary16 block scales of the lane's four output rows
    u32x4 b[2];      // block j's eight activation bytes in dwords 2j, 2j+1
    u32x4 as;        // the token's block scales
};
template <>
struct SkFrag<Op::Q2K> {
    u32x4 q;   // code bytes 16s..16s+15 of the A row
    u32x2 sc;  // its scale bytes 8(s/2)..+7
    u32x4 dm;  // d | dmin << 16 of the four output rows
    u32x4 b[4];
    u32x4 as;
};
template <>
struct SkFrag<Op::TQ2> {
    u32x4 q;   // code bytes 16s..16s+15 of the A row
    u32x2 dd;  // binary16 scales of the four output rows
    u32x4 b[4];
    u32x4 as;
};
template <>
struct SkFrag<Op::TQ1> {
    u32x2 c01;    // code bytes 8s..8s+7 of the A row
    uint32_t c2;  // its code bytes 32+4s..35+4s
    uint32_t tl;  // its code bytes 48..51 (the lane group's byte: 48+s)
    u32x2 dd;     // binary16 scales of the four output rows
    u32x4 b[4];
    u32x4 as;
};
template <>
struct SkFrag<Op::PTQ1_SRC> {
    uint32_t a, b0, b1, tl;  // A-piece dword s, B piece, tail dword of the A row
    u32x4 dd;                // tail dwords (scale in the high half) of the four output rows
    u32x4 b[2];              // activation quads paired with the eight digit quads
    u32x4 as;
};
template <>
struct SkFrag<Op::PTQ1_Q8K> : SkFrag<Op::PTQ1_SRC> {};
template <>
struct SkFrag<Op::PTQ1_PINNED> : SkFrag<Op::PTQ1_SRC> {};
template <>
struct SkFrag<Op::PQ2_UNFUSED> {
    u32x4 ca, cb;  // code dwords 0..3 and 4..7 of the A row
    u32x2 dd;      // binary16 scales of the four output rows
    u32x4 b[2];    // group g's activation bytes (gathered at stride 4) in dwords 2g, 2g+1
    u32x4 as;
};
template <>
struct SkFrag<Op::PQ2_FUSED> : SkFrag<Op::PQ2_UNFUSED> {};
template <>
struct SkFrag<Op::PQ2_Q8> : SkFrag<Op::PQ2_UNFUSED> {};

// PTQ1 lane plan.  Unit element map (tools/ternary/src/lib.rs:202-250): A-piece byte b
// digit k -> 16k+b, B-piece byte b digit k -> 80+8k+b, tail byte b digit k<4 -> 120+2k+b.
// Lane group s takes, as (dword, digit) quads of natural consecutive elements:
//   group 0: (A_s, 0) (A_s, 1)        -> 4s, 16+4s
//   group 1: (A_s, 2) (A_s, 3)        -> 32+4s, 48+4s
//   group 2: (A_s, 4) (B_{s/2}, s%2)  -> 64+4s, 80+8(s%2)+4(s/2)
//   group 3: s<3: (B_0, 2+s) (B_1, 2+s) -> 96+8s, 100+8s;  s=3: the tail bytes
//            repeated (b24 b25 b24 b25) with digits (0,0,1,1) and (2,2,3,3) -> 120, 124
struct Ptq1Plan {
    uint32_t off[8];  // element offsets of the eight quads within the unit
    uint32_t p2h, p3l_l, p3l_h, p3h_l, p3h_h;
};
__device__ __forceinline__ Ptq1Plan ptq1_plan(uint32_t s) {
    Ptq1Plan q;
    q.off[0] = 4 * s;
    q.off[1] = 16 + 4 * s;
    q.off[2] = 32 + 4 * s;
    q.off[3] = 48 + 4 * s;
    q.off[4] = 64 + 4 * s;
    q.off[5] = 80 + 8 * (s & 1) + 4 * (s >> 1);
    q.off[6] = s < 3 ? 96 + 8 * s : 120;
    q.off[7] = s < 3 ? 100 + 8 * s : 124;
    q.p2h = (s & 1) ? 0x00030003u : 0x00010001u;
    const uint32_t p3 = s == 0 ? 9u : s == 1 ? 27u : 81u;
    q.p3l_l = q.p3l_h = s < 3 ? p3 * 0x00010001u : (1u | (3u << 16));
    q.p3h_l = q.p3h_h = s < 3 ? p3 * 0x00010001u : (9u | (27u << 16));
    return q;
}

// First activation element (within the unit) of dword k of lane group s's operand
// bytes, and the element stride of its four bytes.
template <Op O>
__device__ __forceinline__ uint32_t sk_elem(uint32_t s, uint32_t k, uint32_t &stride) {
    stride = 1;
    if constexpr (O == Op::Q8_0) {
        return 32u * (k >> 1) + 8u * s + 4u * (k & 1u);
    } else if constexpr (O == Op::Q2K || O == Op::TQ2) {
        return 128u * (s >> 1) + 32u * (k >> 2) + 16u * (s & 1u) + 4u * (k & 3u);
    } else if constexpr (O == Op::TQ1) {
        // Digits 0..4 of code bytes 8s..8s+3 and 8s+4..8s+7 (elements b + 32k), of code
        // bytes 32+4s..35+4s (elements 160 + 4s + 16k), then the four digits of code byte
        // 48+s (elements 240 + s + 4k: stride 4).
        if (k < 10) return 8u * s + 4u * (k >= 5) + 32u * (k % 5);
        if (k < 15) return 160u + 4u * s + 16u * (k - 10);
        stride = 4;
        return 240u + s;
    } else if constexpr (kind_of<O>() == kPTQ1) {
        return ptq1_plan(s).off[k];
    } else {
        stride = 4;
        return 16u * (2u * (k >> 1) + (s >> 1)) + 2u * (s & 1u) + (k & 1u);
    }
}
template <Op O>
constexpr bool sk_q8_groups() {
    return O == Op::Q8_0 || O == Op::PTQ1_SRC || O == Op::PTQ1_PINNED || O == Op::PQ2_Q8;
}
// Byte of activation element e of unit u in a token's prepared blocks.
template <Op O>
__device__ __forceinline__ const int8_t *sk_value(const uint8_t *a, uint32_t u, uint32_t e) {
    if constexpr (sk_q8_groups<O>())
        return reinterpret_cast<const Q8Block *>(a)[4u * u + (e >> 5)].values + (e & 31u);
    else if constexpr (sk_super_block<O>())
        return reinterpret_cast<const Q8KBlock *>(a)[u].values + e;
    else
        return reinterpret_cast<const Q8KBlock *>(a)[u >> 1].values + 128u * (u & 1u) + e;
}

// Lane-ordered copy of a skinny batch's activations: for unit u and lane l (token l%16,
// clamped to the batch; lane group s = l/16) the sk_lane_bytes the lane feeds the
// matrix cores, at sw + (u*64 + l) * sk_lane_bytes, then the scales [u][16 tokens][4]
// (group scales, or the block scale repeated).  Every skinny wavefront then reads its
// activation operands with contiguous loads.
template <Op O>
__global__ __launch_bounds__(256) void k_sk_prep(const uint8_t *__restrict__ act, uint32_t act_stride, uint32_t ntok,
                                                 uint32_t nu, uint32_t *__restrict__ sw) {
    constexpr uint32_t LD = sk_lane_bytes<O>() / 4;
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    // Chunk blockIdx.y: tokens 16y .. 16y + 15 of the batch, its copy nu * 64 * (LD + 1)
    // dwords after the previous chunk's.
    act += static_cast<size_t>(16u * blockIdx.y) * act_stride;
    ntok = ntok - 16u * blockIdx.y < 16u ? ntok - 16u * blockIdx.y : 16u;
    sw += static_cast<size_t>(blockIdx.y) * nu * 64u * (LD + 1u);
    if (idx < nu * 64u * LD) {
        const uint32_t k = idx % LD, lane = (idx / LD) & 63u, u = idx / (LD * 64u);
        const uint32_t i = lane & 15u, tok = i < ntok ? i : ntok - 1u;
        uint32_t stride;
        const uint32_t e = sk_elem<O>(lane >> 4, k, stride);
        const int8_t *src = sk_value<O>(act + static_cast<size_t>(tok) * act_stride, u, e);
        uint32_t v;
        if (stride == 1)
            v = *reinterpret_cast<const uint32_t *>(src);
        else
            v = static_cast<uint8_t>(src[0]) | (static_cast<uint32_t>(static_cast<uint8_t>(src[4])) << 8) |
                (static_cast<uint32_t>(static_cast<uint8_t>(src[8])) << 16) |
                (static_cast<uint32_t>(static_cast<uint8_t>(src[12])) << 24);
        sw[idx] = v;
    }
    if (idx < nu * 64u) {
        const uint32_t g = idx & 3u, i = (idx >> 2) & 15u, u = idx >> 6;
        const uint8_t *a = act + static_cast<size_t>(i < ntok ? i : ntok - 1u) * act_stride;
        float sc;
        if constexpr (sk_q8_groups<O>())
            sc = reinterpret_cast<const Q8Block *>(a)[4u * u + g].scale;
        else if constexpr (sk_super_block<O>())
            sc = reinterpret_cast<const Q8KBlock *>(a)[u].scale;
        else
            sc = reinterpret_cast<const Q8KBlock *>(a)[u >> 1].scale;
        reinterpret_cast<float *>(sw + nu * 64u * LD)[idx] = sc;
    }
}

// The same operand dwords and scales straight from the token's prepared blocks (no
// lane-ordered copy): scattered loads, cheaper than a second launch on small matrices.
template <Op O>
__device__ __forceinline__ void sk_load_act_raw(SkFrag<O> &f, const uint8_t *a, uint32_t u, uint32_t s,
                                                const Ptq1Plan &pp) {
    if constexpr (O == Op::Q8_0) {
        const Q8Block *blk = reinterpret_cast<const Q8Block *>(a) + 4u * u;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const u32x2 lo = *reinterpret_cast<const u32x2 *>(blk[2 * h].values + 8u * s);
            const u32x2 hi = *reinterpret_cast<const u32x2 *>(blk[2 * h + 1].values + 8u * s);
            f.b[h] = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
        f.as = u32x4{__float_as_uint(blk[0].scale), __float_as_uint(blk[1].scale), __float_as_uint(blk[2].scale),
                     __float_as_uint(blk[3].scale)};
    } else if constexpr (O == Op::Q2K || O == Op::TQ2) {
        const Q8KBlock *blk = reinterpret_cast<const Q8KBlock *>(a) + u;
#pragma unroll
        for (int p = 0; p < 4; ++p)
            f.b[p] = *reinterpret_cast<const u32x4a *>(blk->values + 128u * (s >> 1) + 32u * p + 16u * (s & 1u));
        f.as.x = __float_as_uint(blk->scale);
    } else if constexpr (O == Op::TQ1) {
        const Q8KBlock *blk = reinterpret_cast<const Q8KBlock *>(a) + u;
        const int8_t *v = blk->values;
        uint32_t x[16];
#pragma unroll
        for (uint32_t k = 0; k < 15; ++k) {
            uint32_t stride;
            x[k] = *reinterpret_cast<const uint32_t *>(v + sk_elem<O>(s, k, stride));
        }
        x[15] = static_cast<uint8_t>(v[240u + s]) | static_cast<uint32_t>(static_cast<uint8_t>(v[244u + s])) << 8 |
                static_cast<uint32_t>(static_cast<uint8_t>(v[248u + s])) << 16 |
                static_cast<uint32_t>(static_cast<uint8_t>(v[252u + s])) << 24;
#pragma unroll
        for (int p = 0; p < 4; ++p) f.b[p] = u32x4{x[4 * p], x[4 * p + 1], x[4 * p + 2], x[4 * p + 3]};
        f.as.x = __float_as_uint(blk->scale);
    } else if constexpr (kind_of<O>() == kPTQ1) {
        uint32_t x[8];
        if constexpr (O == Op::PTQ1_SRC || O == Op::PTQ1_PINNED) {
            const Q8Block *blk = reinterpret_cast<const Q8Block *>(a) + 4u * u;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                x[k] = *reinterpret_cast<const uint32_t *>(blk[k >> 1].values + (pp.off[k] - 32u * (k >> 1)));
            f.as = u32x4{__float_as_uint(blk[0].scale), __float_as_uint(blk[1].scale), __float_as_uint(blk[2].scale),
                         __float_as_uint(blk[3].scale)};
        } else {
            const Q8KBlock *blk = reinterpret_cast<const Q8KBlock *>(a) + (u >> 1);
            const int8_t *v = blk->values + 128u * (u & 1u);
#pragma unroll
            for (int k = 0; k < 8; ++k) x[k] = *reinterpret_cast<const uint32_t *>(v + pp.off[k]);
            f.as.x = __float_as_uint(blk->scale);
        }
        f.b[0] = u32x4{x[0], x[1], x[2], x[3]};
        f.b[1] = u32x4{x[4], x[5], x[6], x[7]};
    } else {
        // Natural bytes 16m..16m+15 (m = 2g + s/2), transposed to stride-4 gathers.
        const uint32_t p0 = 2u * (s & 1u);
        const uint32_t gsel = p0 | ((4u + p0) << 8) | ((p0 + 1u) << 16) | ((5u + p0) << 24);
        uint32_t x[8];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            u32x4 q;
            if constexpr (O == Op::PQ2_Q8)
                q = *reinterpret_cast<const u32x4a *>(reinterpret_cast<const Q8Block *>(a)[4u * u + g].values +
                                                      16u * (s >> 1));
            else
                q = *reinterpret_cast<const u32x4a *>(reinterpret_cast<const Q8KBlock *>(a)[u >> 1].values +
                                                      128u * (u & 1u) + 16u * (2u * g + (s >> 1)));
            const uint32_t t01 = perm(q.y, q.x, gsel), t23 = perm(q.w, q.z, gsel);
            x[2 * g] = perm(t23, t01, sel(0, 1, 4, 5));
            x[2 * g + 1] = perm(t23, t01, sel(2, 3, 6, 7));
        }
        f.b[0] = u32x4{x[0], x[1], x[2], x[3]};
        f.b[1] = u32x4{x[4], x[5], x[6], x[7]};
        if constexpr (O == Op::PQ2_Q8) {
            const Q8Block *blk = reinterpret_cast<const Q8Block *>(a) + 4u * u;
            f.as = u32x4{__float_as_uint(blk[0].scale), __float_as_uint(blk[1].scale), __float_as_uint(blk[2].scale),
                         __float_as_uint(blk[3].scale)};
        } else {
            f.as.x = __float_as_uint(reinterpret_cast<const Q8KBlock *>(a)[u >> 1].scale);
        }
    }
}

template <Op O, bool SW>
__device__ __forceinline__ void sk_load(SkFrag<O> &f, const SkLane &L, uint32_t u, const Ptq1Plan &pp) {
    constexpr uint32_t UB = unit_bytes<O>(), LB = sk_lane_bytes<O>();
    const uint32_t seg = u * L.trp * UB, s = L.s;
    if constexpr (SW) {
        const u32x4 *b = reinterpret_cast<const u32x4 *>(L.sw + (static_cast<size_t>(u) * 64u + L.lane) * LB);
#pragma unroll
        for (uint32_t k = 0; k < LB / 16; ++k) f.b[k] = b[k];
        f.as = *reinterpret_cast<const u32x4 *>(L.scales + (u * 16u + L.tok) * 16u);
    } else {
        sk_load_act_raw<O>(f, L.sw, u, s, pp);
    }
    if constexpr (O == Op::Q8_0) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            f.a[j] = bload2(L.rs, seg + (2u * j + (s >> 1)) * 16u * L.trp + 16u * L.ra + 8u * (s & 1u));
        f.sc0 = bload4(L.rs, seg + 128u * L.trp + 8u * L.rc);
        f.sc1 = bload4(L.rs, seg + 128u * L.trp + 8u * L.rc + 16u);
    } else if constexpr (O == Op::Q2K) {
        f.q = bload4(L.rs, seg + 16u * s * L.trp + 16u * L.ra);
        f.sc = bload2(L.rs, seg + 64u * L.trp + 16u * L.ra + 8u * (s >> 1));
        f.dm = bload4(L.rs, seg + 80u * L.trp + 4u * L.rc);
    } else if constexpr (O == Op::TQ2) {
        f.q = bload4(L.rs, seg + 16u * s * L.trp + 16u * L.ra);
        f.dd = bload2(L.rs, seg + 64u * L.trp + 2u * L.rc);
    } else if constexpr (O == Op::TQ1) {
        f.c01 = bload2(L.rs, seg + 16u * (s >> 1) * L.trp + 16u * L.ra + 8u * (s & 1u));
        f.c2 = bload1(L.rs, seg + 32u * L.trp + 16u * L.ra + 4u * s);
        f.tl = bload1(L.rs, seg + 48u * L.trp + 4u * L.ra);
        f.dd = bload2(L.rs, seg + 52u * L.trp + 2u * L.rc);
    } else if constexpr (kind_of<O>() == kPTQ1) {
        f.a = bload1(L.rs, seg + 16u * L.ra + 4u * s);
        const u32x2 bb = bload2(L.rs, seg + 16u * L.trp + 8u * L.ra);
        f.b0 = bb.x;
        f.b1 = bb.y;
        f.tl = bload1(L.rs, seg + 24u * L.trp + 4u * L.ra);
        f.dd = bload4(L.rs, seg + 24u * L.trp + 4u * L.rc);
    } else {
        f.ca = bload4(L.rs, seg + 16u * L.ra);
        f.cb = bload4(L.rs, seg + 16u * L.trp + 16u * L.ra);
        f.dd = bload2(L.rs, seg + 32u * L.trp + 2u * L.rc);
    }
}

// One unit's binary32 terms tv[v][...] of the lane's four chains (rows rc+v, this lane's
// token), in the order Chain<O>::fold consumes them.
template <Op O>
__device__ __forceinline__ void sk_terms(const SkFrag<O> &f, const SkLane &L, const Ptq1Plan &pp,
                                         float tv[4][sk_terms_per_unit<O>()]) {
    const uint32_t s = L.s;
    const v4i zero = {0, 0, 0, 0};
    if constexpr (O == Op::Q8_0) {
        v4i acc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[j] = mfma32(f.a[j].x, f.a[j].y, f.b[j >> 1][2 * (j & 1)], f.b[j >> 1][2 * (j & 1) + 1], zero);
        const float as[4] = {__uint_as_float(f.as.x), __uint_as_float(f.as.y), __uint_as_float(f.as.z),
                             __uint_as_float(f.as.w)};
        const uint32_t sw[8] = {f.sc0.x, f.sc0.y, f.sc0.z, f.sc0.w, f.sc1.x, f.sc1.y, f.sc1.z, f.sc1.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t bits = (sw[2 * v + (j >> 1)] >> (16 * (j & 1))) & 0xffffu;
                // dot_legacy, src/kernels.rs:1241-1244
                tv[v][j] = (h2f(bits) * as[j]) * static_cast<float>(acc[j][v]);
            }
        }
    } else if constexpr (O == Op::Q2K) {
        // Lane group s holds code bytes 16s..16s+15: half h = s/2, elements
        // 128h + 32p + 16(s%2) + e of sub-block g = 8h + 2p + s%2 in field p.  The
        // weight operand carries scale_g * q (at most 45, still a byte), so one dot
        // gives sum_g scale_g * dot_g; a second one with min_g repeated gives
        // sum_g min_g * bsum_g: both exact integers of kquants::dot.
        v4i isum = zero, msum = zero;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t byte = (f.sc[p >> 1] >> (16u * (p & 1) + 8u * (s & 1u))) & 0xffu;
            const uint32_t scale = byte & 15u, mn = byte >> 4;
            u32x4 a1;
            a1.x = bytes_times((f.q.x >> (2 * p)) & 0x03030303u, scale);
            a1.y = bytes_times((f.q.y >> (2 * p)) & 0x03030303u, scale);
            a1.z = bytes_times((f.q.z >> (2 * p)) & 0x03030303u, scale);
            a1.w = bytes_times((f.q.w >> (2 * p)) & 0x03030303u, scale);
            const uint32_t m4 = mn * 0x01010101u;
            const u32x4 a2 = {m4, m4, m4, m4};
            isum = mfma64(a1, f.b[p], isum);
            msum = mfma64(a2, f.b[p], msum);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            // dot_q2_k_block, src/kernels/kquants.rs:193-196
            const float as = __uint_as_float(f.as.x);
            tv[v][0] = (as * h2f(f.dm[v] & 0xffffu)) * static_cast<float>(isum[v]) -
                       (as * h2f(f.dm[v] >> 16)) * static_cast<float>(msum[v]);
        }
    } else if constexpr (O == Op::TQ1 || O == Op::TQ2) {
        // The unit's integer dot over the lane groups' 64 elements each: signed fields
        // c - 1 (TQ2_0, Q2_K's element order) or signed digits t - 1 (TQ1_0, sk_elem's).
        u32x4 a[4];
        if constexpr (O == Op::TQ2) {
#pragma unroll
            for (int p = 0; p < 4; ++p)
#pragma unroll
                for (int d = 0; d < 4; ++d) a[p][d] = code_map((f.q[d] >> (2 * p)) & 0x03030303u, 0x020100ffu);
        } else {
            uint32_t q[16];
            auto digits = [&](uint32_t x, int n0) {  // digits 0..4 of four code bytes
                uint32_t Lw = x & 0x00ff00ffu, Hw = (x >> 8) & 0x00ff00ffu;
#pragma unroll
                for (int k = 0; k < 5; ++k) {
                    const uint32_t mL = Lw * 3u, mH = Hw * 3u;
                    q[n0 + k] = code_map(perm(mH, mL, sel(1, 5, 3, 7)), 0x000100ffu);
                    Lw = mL & 0x00ff00ffu;
                    Hw = mH & 0x00ff00ffu;
                }
            };
            digits(f.c01.x, 0);
            digits(f.c01.y, 5);
            digits(f.c2, 10);
            // Code byte 48+s in all four bytes, byte k taking digit k.
            q[15] = trit_quad(((f.tl >> (8u * s)) & 0xffu) * 0x01010101u, 1u | (9u << 16), 3u | (27u << 16));
#pragma unroll
            for (int p = 0; p < 4; ++p) a[p] = u32x4{q[4 * p], q[4 * p + 1], q[4 * p + 2], q[4 * p + 3]};
        }
        v4i acc = mfma64(a[0], f.b[0], zero);
        acc = mfma64(a[1], f.b[1], acc);
        acc = mfma64(a[2], f.b[2], acc);
        acc = mfma64(a[3], f.b[3], acc);
        const float as = __uint_as_float(f.as.x);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            // dot(), src/kernels/tquants.rs:283
            tv[v][0] = static_cast<float>(acc[v]) * (h2f((f.dd[v >> 1] >> (16 * (v & 1))) & 0xffffu) * as);
        }
    } else if constexpr (kind_of<O>() == kPTQ1) {
        // A_s digits 0..4, sequentially (remainder times 3 per digit).
        uint32_t q[8];
        {
            uint32_t Lw = f.a & 0x00ff00ffu, Hw = (f.a >> 8) & 0x00ff00ffu;
#pragma unroll
            for (int k = 0; k < 5; ++k) {
                const uint32_t mL = Lw * 3u, mH = Hw * 3u;
                q[k] = code_map(perm(mH, mL, sel(1, 5, 3, 7)), 0x000100ffu);
                Lw = mL & 0x00ff00ffu;
                Hw = mH & 0x00ff00ffu;
            }
        }
        const uint32_t trep = perm(f.tl, f.tl, sel(0, 1, 0, 1));
        q[5] = trit_quad((s >> 1) ? f.b1 : f.b0, pp.p2h, pp.p2h);
        q[6] = trit_quad(s < 3 ? f.b0 : trep, pp.p3l_l, pp.p3l_h);
        q[7] = trit_quad(s < 3 ? f.b1 : trep, pp.p3h_l, pp.p3h_h);
        // Quad order: group 0 = (q0, q1), group 1 = (q2, q3), group 2 = (q4, q5), group 3 = (q6, q7).
        const float as[4] = {__uint_as_float(f.as.x), __uint_as_float(f.as.y), __uint_as_float(f.as.z),
                             __uint_as_float(f.as.w)};
        if constexpr (O == Op::PTQ1_PINNED) {
            // dot_q8_groups_pinned needs, per group g and native lane l, the integer sum
            // over the group's elements 4l..4l+3 and 16+4l..16+4l+3
            // (q8_native_lanes, src/kernels.rs:1066-1076).  Every quad of consecutive
            // elements a lane feeds lies in one such lane subset (its offset within the
            // group, /4, mod 4), so one MFMA per (g, l) with the other lanes' quads
            // zeroed gives I_{g,l} exactly.  Quad lanes of lane group s:
            //   groups 0, 1: (s, s); group 2: (s, lane of 80+8(s%2)+4(s/2));
            //   group 3: s < 3: (2s%4, (2s+1)%4), s = 3: (2, 3).
            const uint32_t l5 = (4u + 2u * (s & 1u) + (s >> 1)) & 3u;
            const uint32_t l6 = s < 3 ? (2u * s) & 3u : 2u, l7 = s < 3 ? (2u * s + 1u) & 3u : 3u;
            const uint32_t qa[4] = {s, s, s, l6}, qb[4] = {s, s, l5, l7};
            const uint32_t b0[4] = {f.b[0].x, f.b[0].z, f.b[1].x, f.b[1].z};
            const uint32_t b1[4] = {f.b[0].y, f.b[0].w, f.b[1].y, f.b[1].w};
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                v4i il[4];
#pragma unroll
                for (uint32_t l = 0; l < 4; ++l)
                    il[l] = mfma32(qa[g] == l ? q[2 * g] : 0u, qb[g] == l ? q[2 * g + 1] : 0u, b0[g], b1[g], zero);
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    // |I| <= 8 * 127: 16 bits hold it.
                    tv[v][2 * g] = __uint_as_float((static_cast<uint32_t>(il[0][v]) & 0xffffu) |
                                                   (static_cast<uint32_t>(il[1][v]) << 16));
                    tv[v][2 * g + 1] = __uint_as_float((static_cast<uint32_t>(il[2][v]) & 0xffffu) |
                                                       (static_cast<uint32_t>(il[3][v]) << 16));
                }
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float dw = h2f(f.dd[v] >> 16);
#pragma unroll
                for (int g = 0; g < 4; ++g) tv[v][8 + g] = dw * as[g];  // fl(d_w * A_g.scale)
            }
        } else if constexpr (O == Op::PTQ1_SRC) {
            v4i acc[4];
            acc[0] = mfma32(q[0], q[1], f.b[0].x, f.b[0].y, zero);
            acc[1] = mfma32(q[2], q[3], f.b[0].z, f.b[0].w, zero);
            acc[2] = mfma32(q[4], q[5], f.b[1].x, f.b[1].y, zero);
            acc[3] = mfma32(q[6], q[7], f.b[1].z, f.b[1].w, zero);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                // dot_q8_groups, src/kernels.rs:1043-1064: fl(tt + fl(scale * I)) is one FMA, since
                // the binary16 scale (11 significant bits) times |I| < 2^13 is exact in binary32.
                float tt = 0.0f;
#pragma unroll
                for (int g = 0; g < 4; ++g) tt = __builtin_fmaf(as[g], static_cast<float>(acc[g][v]), tt);
                tv[v][0] = h2f(f.dd[v] >> 16) * tt;
            }
        } else {
            v4i acc = mfma32(q[0], q[1], f.b[0].x, f.b[0].y, zero);
            acc = mfma32(q[2], q[3], f.b[0].z, f.b[0].w, acc);
            acc = mfma32(q[4], q[5], f.b[1].x, f.b[1].y, acc);
            acc = mfma32(q[6], q[7], f.b[1].z, f.b[1].w, acc);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                // dot_ptq1_q8k, src/kernels.rs:1026-1034
                tv[v][0] = (h2f(f.dd[v] >> 16) * as[0]) * static_cast<float>(acc[v]);
            }
        }
    } else {
        // PQ2: group g = code dwords 2g, 2g+1 (element 16i+4q+p in byte q, bits 2p).  Lane
        // group s takes dword m = 2g + s/2, fields p0 = 2(s%2) and p0+1: elements
        // 16m + 4q + p, paired with the activation bytes gathered at stride 4.
        const uint32_t p0 = 2u * (s & 1u);
        const uint32_t c[8] = {f.ca.x, f.ca.y, f.ca.z, f.ca.w, f.cb.x, f.cb.y, f.cb.z, f.cb.w};
        const uint32_t ab[8] = {f.b[0].x, f.b[0].y, f.b[0].z, f.b[0].w, f.b[1].x, f.b[1].y, f.b[1].z, f.b[1].w};
        const float as[4] = {__uint_as_float(f.as.x), __uint_as_float(f.as.y), __uint_as_float(f.as.z),
                             __uint_as_float(f.as.w)};
        v4i acc[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t x = (s >> 1) ? c[2 * g + 1] : c[2 * g];
            const uint32_t wlo = code_map((x >> (2u * p0)) & 0x03030303u, 0x020100ffu);
            const uint32_t whi = code_map((x >> (2u * p0 + 2u)) & 0x03030303u, 0x020100ffu);
            const uint32_t alo = ab[2 * g], ahi = ab[2 * g + 1];
            if constexpr (O == Op::PQ2_Q8)
                acc[g] = mfma32(wlo, whi, alo, ahi, zero);
            else
                acc[0] = mfma32(wlo, whi, alo, ahi, g == 0 ? zero : acc[0]);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float d = h2f((f.dd[v >> 1] >> (16 * (v & 1))) & 0xffffu);
            if constexpr (O == Op::PQ2_Q8) {
                // dot_q8_groups for an odd-group PQ2 row, src/kernels.rs:1043-1064 (one FMA per
                // group: the scale times |I| < 2^13 is exact in binary32)
                float tt = 0.0f;
#pragma unroll
                for (int g = 0; g < 4; ++g) tt = __builtin_fmaf(as[g], static_cast<float>(acc[g][v]), tt);
                tv[v][0] = d * tt;
            } else {
                // dot_pq2::<FUSED>, src/kernels.rs:941-955
                const float dd = d * as[0];
                const float sf = static_cast<float>(acc[0][v]);
                if constexpr (O == Op::PQ2_UNFUSED) {
                    tv[v][0] = dd * sf;
                } else {
                    tv[v][0] = dd;
                    tv[v][1] = sf;
                }
            }
        }
    }
}

// KS == 1: one wavefront per 16-row block runs every unit and keeps the four chains in
// registers.  KS > 1 (fewer blocks than the chip has SIMDs): the KS wavefronts of a
// workgroup share one block and take its units in chunks of KS (wavefront w: unit
// c*KS + w); each writes its unit's terms to LDS, and after a barrier every thread folds
// one (row, token) element through the chunk's units in unit order -- the same serial
// chain, computed by a different lane.  Chunk parity double-buffers the terms, so one
// barrier per chunk suffices.
template <Op O, bool SW, int KS>
__global__ __launch_bounds__(64 * KS) void k_mv_skinny(SkParams p) {
    constexpr uint32_t UB = unit_bytes<O>();
    constexpr int TPU = sk_terms_per_unit<O>();
    const uint32_t lane = threadIdx.x & 63u, i = lane & 15u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tile = blockIdx.x >> 2, quarter = blockIdx.x & 3u;
    const uint32_t left = p.rows - tile * kTile;
    const uint32_t trows = left < kTile ? left : kTile;
    if (16u * quarter >= trows) return;
    // Chunk blockIdx.y: tokens 16y .. 16y + ntok - 1.
    const uint32_t t0 = 16u * blockIdx.y, ntok = p.ntok - t0 < 16u ? p.ntok - t0 : 16u;
    const uint8_t *sw = p.sw + static_cast<size_t>(blockIdx.y) * p.sw_chunk;
    SkLane L;
    L.s = lane >> 4;
    L.lane = lane;
    L.tok = i;
    L.trp = (trows + 7u) & ~7u;
    L.rs = make_rsrc(p.w + static_cast<size_t>(tile) * kTile * p.nu * UB, L.trp * p.nu * UB);
    L.ra = 16u * quarter + i;
    L.rc = 16u * quarter + 4u * L.s;
    if constexpr (SW) {
        L.sw = sw;
        L.scales = sw + static_cast<size_t>(p.nu) * 64u * sk_lane_bytes<O>();
    } else {
        L.sw = sw + static_cast<size_t>(i < ntok ? i : ntok - 1u) * p.act_stride;
        L.scales = nullptr;
    }
    const Ptq1Plan pp = ptq1_plan(L.s);
    const size_t obase = static_cast<size_t>(t0) * p.rows + static_cast<size_t>(tile) * kTile + 16u * quarter;
    auto store = [&](uint32_t tok, uint32_t r, float v) {  // r: row within the 16-row block
        if (tok < ntok && 16u * quarter + r < trows) {
            const size_t at = static_cast<size_t>(tok) * p.rows + obase + r;
            if (p.residual) v = v + p.residual[at];
            p.out[at] = v;
            if (!finite(v)) raise_error(p.err, kErrNonfinite);
        }
    };
    if constexpr (KS == 1) {
        SkChain<O> ch[4];
        auto fold = [&](const SkFrag<O> &f) {
            float tv[4][TPU];
            sk_terms<O>(f, L, pp, tv);
#pragma unroll
            for (int v = 0; v < 4; ++v) ch[v].fold(tv[v]);
        };
        // Two fragments in ping-pong: the next unit's loads are in flight during a fold.
        SkFrag<O> A, B;
        uint32_t u = 0;
        sk_load<O, SW>(A, L, 0, pp);
        while (u + 1 < p.nu) {
            sk_load<O, SW>(B, L, u + 1, pp);
            fold(A);
            if (u + 2 < p.nu) sk_load<O, SW>(A, L, u + 2, pp);
            fold(B);
            u += 2;
        }
        if (u < p.nu) fold(A);
#pragma unroll
        for (int v = 0; v < 4; ++v) store(i, 4u * L.s + v, ch[v].result());
    } else {
        // terms[parity][wave][term][element], element e = 4 * lane + v
        __shared__ float terms[2][KS][TPU][256];
        constexpr int EPT = KS <= 4 ? 4 / KS : 1;  // elements folded per thread: e = tid + 64 * KS * k
        SkChain<O> ch[EPT];
        const uint32_t chunks = (p.nu + KS - 1) / KS;
        auto produce = [&](const SkFrag<O> &f, uint32_t c) {
            float tv[4][TPU];
            sk_terms<O>(f, L, pp, tv);
#pragma unroll
            for (int j = 0; j < TPU; ++j)
                *reinterpret_cast<float4 *>(&terms[c & 1u][wave][j][4u * lane]) =
                    make_float4(tv[0][j], tv[1][j], tv[2][j], tv[3][j]);
        };
        auto consume = [&](uint32_t c) {
            __syncthreads();
#pragma unroll
            for (int k = 0; k < EPT; ++k) {
                const uint32_t e = threadIdx.x + 64u * KS * k;
                if (e >= 256u) break;
#pragma unroll
                for (int w = 0; w < KS; ++w) {
                    if (c * KS + w < p.nu) {
                        float t[TPU];
#pragma unroll
                        for (int j = 0; j < TPU; ++j) t[j] = terms[c & 1u][w][j][e];
                        ch[k].fold(t);
                    }
                }
            }
        };
        SkFrag<O> A, B;
        uint32_t c = 0;
        if (wave < p.nu) sk_load<O, SW>(A, L, wave, pp);
        while (c + 1 < chunks) {
            const uint32_t u1 = (c + 1) * KS + wave;
            if (u1 < p.nu) sk_load<O, SW>(B, L, u1, pp);
            if (c * KS + wave < p.nu) produce(A, c);
            consume(c);
            const uint32_t u2 = (c + 2) * KS + wave;
            if (c + 2 < chunks && u2 < p.nu) sk_load<O, SW>(A, L, u2, pp);
            if (u1 < p.nu) produce(B, c + 1);
            consume(c + 1);
            c += 2;
        }
        if (c < chunks) {
            if (c * KS + wave < p.nu) produce(A, c);
            consume(c);
        }
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const uint32_t e = threadIdx.x + 64u * KS * k, src = e >> 2;
            if (e < 256u) store(src & 15u, 4u * (src >> 4) + (e & 3u), ch[k].result());
        }
    }
}

// Split-mode workgroups hold at most eight wavefronts: the bound leaves each thread up
// to 256 registers, room for a quantizing prologue's input held in registers next to
// the weights in flight.
constexpr uint32_t kSplitMaxWaves = 8, kSplitMaxThreads = 64 * kSplitMaxWaves;

// Small matrices: a workgroup owns rw = 64/lpr rows of a tile; its ks wavefronts
// (per matrix) and the lpr lane groups of each wavefront split the row's units
// (lane group c of wavefront w takes units w*lpr+c, +ks*lpr, ...).  Each unit's
// terms land in LDS and wavefront 0 folds them in unit order.  The activation is
// staged in LDS by the prologue: either the prepared blocks are copied (COPY), or
// the f32 input is quantized with the contract matvec_into uses (QUANT), which
// makes the whole projection one launch.  NMAT == 2: gate (wavefronts 0..ks-1) and
// up (ks..2ks-1) share the activation and the epilogue writes SwiGLU(gate, up), and
// optionally (q8_out) the SwiGLU vector's Q8_0 blocks, so that the projection after
// it takes prepared blocks.
// The kernel is latency-bound at decode sizes, so its critical path is kept short:
// indices are shifts (lpr and ks are powers of two); the activation's reads are
// issued first, then every weight unit's; a PTQ1 unit's trits are extracted while
// the activation is staged, so after the staging barrier only the dot products remain.
// HELD (QUANT only): 8 or 16 input values held per lane (HeldInput), 0 to stream the
// input through the quantizer instead.
template <Op O, bool QUANT, int NMAT, int HELD>
__global__ __launch_bounds__(kSplitMaxThreads) void k_mv_split(MvParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr uint32_t UB = unit_bytes<O>();
    constexpr int TPU = terms_per_unit<O>();
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nwaves = blockDim.x >> 6;
    const uint32_t ks = p.ks, lg_lpr = p.lg_lpr, lg_rw = 6u - lg_lpr, rw = 1u << lg_rw;
    const uint32_t mat = (NMAT == 2 && wave >= ks) ? 1u : 0u;
    const uint32_t mw = wave - mat * ks;
    // Workgroups go to the eight XCDs round-robin in dispatch order, each XCD with its own
    // L2.  A workgroup of lpr > 1 reads 64/lpr rows of its tile's pieces, less than a
    // cache line of the 8- and 4-byte pieces, so with xcd_tiles the tile's lpr workgroups
    // are all placed on one XCD (workgroup b runs on XCD b % 8) and each line is fetched
    // into one L2 only.
    uint32_t tile, sub;
    if (p.xcd_tiles) {
        const uint32_t k = blockIdx.x >> 3;
        tile = ((k >> lg_lpr) << 3) + (blockIdx.x & 7u);
        sub = k & ((1u << lg_lpr) - 1u);
    } else {
        tile = blockIdx.x >> lg_lpr;
        sub = blockIdx.x & ((1u << lg_lpr) - 1u);
    }
    const uint32_t c = lane >> lg_rw, r = lane & (rw - 1u);
    const uint32_t lg_kt = p.lg_ks + lg_lpr, kt = 1u << lg_kt, kk = (mw << lg_lpr) + c;
    const uint32_t nu = p.nu, row_bytes = nu * UB;
    const uint32_t left = p.rows - tile * kTile;
    const uint32_t trows = left < kTile ? left : kTile;
    const uint32_t trp = (trows + 7u) & ~7u;
    const uint32_t tr = (sub << lg_rw) + r;  // row within the tile

    const uint32_t abytes = align16(act_bytes_for<O>(p.cols));
    const uint32_t stride = nu * TPU + 1;
    float *terms = reinterpret_cast<float *>(smem + abytes) + mat * rw * stride;
    float *res = reinterpret_cast<float *>(smem + abytes) + NMAT * rw * stride;
    double *red = reinterpret_cast<double *>(smem + abytes + align16(4u * (NMAT * rw * stride + 2 * rw)));

    // The activation's reads come first: memory counters complete in issue order, so
    // staging it waits for these reads only, not for the weights behind them.
    // QUANT: a prologue whose input fits in the wavefronts' registers reads it (and the
    // norm weights) here, in one round trip.  The holder is chosen at compile time: a
    // branch around these loads would make the prologue wait for the weights too.
    using Held = HeldInput<act_is_q8k<O>(), HELD == 8 ? 8 : 16, HELD == 8 ? 1 : 2>;
    Held hin;
    if constexpr (QUANT && HELD != 0) {
        const float *x = static_cast<const float *>(p.act);
        hin.load(x, p.norm_w ? p.norm_w : x, p.cols, wave, nwaves, lane);
    }
    // COPY: the first 16 words per thread of the prepared blocks.
    constexpr uint32_t kCopy = 16;
    const uint32_t *asrc = static_cast<const uint32_t *>(p.act);
    const uint32_t an = act_bytes_for<O>(p.cols) / 4;
    uint32_t atmp[kCopy];
    if constexpr (!QUANT) {
#pragma unroll
        for (uint32_t j = 0; j < kCopy; ++j) {
            const uint32_t i = j * blockDim.x + threadIdx.x;
            atmp[j] = i < an ? asrc[i] : 0u;
        }
    }

    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(p.w[mat] + static_cast<size_t>(tile) * kTile * row_bytes, trp * row_bytes);
    // When every lane takes at most kPre units (the decode-sized projections), all of
    // them are loaded here, ahead of the prologue, and the main loop issues no load.
    // Units past the row fall outside the buffer resource and read as zeros.
    // W[0] and W[1] double as the ping-pong pair of the streaming loop otherwise.
    // Larger units keep the streaming loop only (their registers are spoken for).
    constexpr uint32_t kPre = UB <= 36 ? 3 : 2;
    const uint32_t cmax = (nu + kt - 1) >> lg_kt;  // most units any lane takes
    const bool pre = UB <= 36 && cmax <= kPre;
    Raw<O> W[kPre];
    uint32_t u = kk;
    if (pre) {
#pragma unroll
        for (uint32_t j = 0; j < kPre; ++j) load_unit<O>(W[j], rs, (kk + (j << lg_kt)) * trp * UB, trp, tr);
    } else if (u < nu) {
        load_unit<O>(W[0], rs, u * trp * UB, trp, tr);
    }
    // The folding lanes' residual is read now, so that its latency hides behind the
    // prologue and the main loop instead of following the fold.
    const bool folder = mw == 0 && lane < rw;
    const bool valid = tr < trows;
    const size_t row = static_cast<size_t>(tile) * kTile + tr;
    const float resid = (NMAT == 1 && p.residual && folder && valid) ? p.residual[row] : 0.0f;

    // ---- prologue: stage the activation in LDS -------------------------------------
    if constexpr (QUANT) {
        const float *x = static_cast<const float *>(p.act);
        auto *blocks = reinterpret_cast<typename ActBlock<O>::type *>(smem);
        int e;
        // RMSNorm fused ahead of the quantizer (as below), from the held registers:
        // lane sums in element order, the wavefront's butterfly, then the wavefronts in
        // order, in binary64 (rms_norm_scale_inner's order up to the binary64 additions).
        auto held_prologue = [&](auto &hin) -> int {
            float scale = 1.0f;
            hin.mask(p.cols, wave, nwaves, lane);
            if (p.norm_w) {
                const double s = wave_sum(hin.sumsq());
                if (lane == 0) red[wave] = s;
                __syncthreads();
                double t = 0.0;
#pragma unroll
                for (uint32_t v = 0; v < kSplitMaxWaves; ++v)
                    if (v < nwaves) t += red[v];
                const float mean = static_cast<float>(t / static_cast<double>(p.cols));
                scale = 1.0f / __builtin_sqrtf(mean + p.eps);
                if (!(finite(scale) && scale > 0.0f)) return kErrNonfinite;
            }
            return hin.quantize(p.cols, p.qcontract, blocks, wave, nwaves, lane, p.norm_w != nullptr, scale);
        };
        if constexpr (HELD != 0) {
            e = held_prologue(hin);
        } else if (p.norm_w) {
            // RMSNorm fused ahead of the quantizer: every workgroup normalizes the whole
            // input itself, so the projection stays one launch.
            const float scale = rms_scale_wg(x, p.cols, p.eps, red);
            e = scale == 0.0f ? kErrNonfinite
                              : quantize_prologue<act_is_q8k<O>()>(x, p.cols, p.qcontract, blocks, wave, nwaves, lane,
                                                                   NormPre{p.norm_w, scale});
        } else {
            e = quantize_prologue<act_is_q8k<O>()>(x, p.cols, p.qcontract, blocks, wave, nwaves, lane);
        }
        // Every workgroup sees the same input; the first one reports its errors.
        if (e && lane == 0 && blockIdx.x == 0) raise_error(p.err, e);
    } else {
        uint32_t *dst = reinterpret_cast<uint32_t *>(smem);
#pragma unroll
        for (uint32_t j = 0; j < kCopy; ++j) {
            const uint32_t i = j * blockDim.x + threadIdx.x;
            if (i < an) dst[i] = atmp[j];
        }
        // Longer activations: the rest, 16 loads per thread in flight before any store.
        for (uint32_t base = kCopy * blockDim.x; base < an; base += kCopy * blockDim.x) {
            uint32_t tmp[kCopy];
#pragma unroll
            for (uint32_t j = 0; j < kCopy; ++j) {
                const uint32_t i = base + j * blockDim.x + threadIdx.x;
                tmp[j] = i < an ? asrc[i] : 0u;
            }
#pragma unroll
            for (uint32_t j = 0; j < kCopy; ++j) {
                const uint32_t i = base + j * blockDim.x + threadIdx.x;
                if (i < an) dst[i] = tmp[j];
            }
        }
    }
    // PTQ1 units held in registers: their trits are extracted now, ahead of the barrier,
    // while the other wavefronts finish staging the activation.
    constexpr bool kDec = kind_of<O>() == kPTQ1;
    using DecT = typename std::conditional<kDec, Ptq1Dec, Raw<O>>::type;
    DecT D[kDec ? kPre : 1];
    if constexpr (kDec) {
        if (pre) {
#pragma unroll
            for (uint32_t j = 0; j < kPre; ++j)
                if (kk + (j << lg_kt) < nu) ptq1_decode(W[j].x, D[j]);
        }
    }
    __syncthreads();
    const void *act = smem;

    // ---- main loop: ping-pong over this lane's units --------------------------------
    auto step = [&](const auto &w, uint32_t v) {
        float t[TPU];
        unit_terms<O>(w, act, v, t);
#pragma unroll
        for (int j = 0; j < TPU; ++j) terms[r * stride + v * TPU + j] = t[j];
    };
    if (pre) {
#pragma unroll
        for (uint32_t j = 0; j < kPre; ++j) {
            const uint32_t v = kk + (j << lg_kt);
            if (v < nu) {
                if constexpr (kDec)
                    step(D[j], v);
                else
                    step(W[j], v);
            }
        }
    } else {
        while (u + kt < nu) {
            load_unit<O>(W[1], rs, (u + kt) * trp * UB, trp, tr);
            step(W[0], u);
            if (u + 2 * kt < nu) load_unit<O>(W[0], rs, (u + 2 * kt) * trp * UB, trp, tr);
            step(W[1], u + kt);
            u += 2 * kt;
        }
        if (u < nu) step(W[0], u);
    }
    __syncthreads();

    // ---- fold in unit order and epilogue ---------------------------------------------
    float o = 0.0f;
    if (folder) {
        Chain<O> ch;
        const float *t = terms + lane * stride;
        for (uint32_t v = 0; v < nu; ++v) ch.fold(t + v * TPU, act, v);
        o = ch.result();
    }
    if constexpr (NMAT == 1) {
        if (folder && valid) {
            if (p.residual) o = o + resid;
            p.out[row] = o;
            if (!finite(o)) raise_error(p.err, kErrNonfinite);
        }
    } else {
        if (folder) res[mat * rw + lane] = o;
        __syncthreads();
        if (wave == 0) {
            const bool own = lane < rw && valid;
            float h = 0.0f;
            if (own) {
                h = swiglu_one(res[lane], res[rw + lane], row, p.rows, p.pinned);
                if (p.out) p.out[row] = h;
                if (!finite(h)) raise_error(p.err, kErrNonfinite);
            }
            // Rows 32j..32j+31 of the vector are Q8_0 block j (q8_with_input,
            // src/kernels.rs:552-617): every 32 lanes hold one block (rw >= 32 and the
            // row count a multiple of 32, checked at launch).
            if (p.q8_out) {
                const int e = q8_0_lanes32(h, own, p.q8_contract, p.q8_out + (row >> 5), lane & 31u);
                if (e && own) raise_error(p.err, e);
            }
        }
    }
}

// ---- batches of up to four tokens on the 4x4x4 matrix cores --------------------------
// v_mfma_i32_4x4x4_16b_i8 runs sixteen independent 4x4x4 integer products per
// wavefront: block b = lane/4 takes row i of A from lane 4b+i and column j of B from
// lane 4b+j, and leaves D[i][j] in register i of lane 4b+j.  With the tokens on A (lane
// l supplies token l%4's activation quad, from LDS) and the weights on B (lane l
// supplies a quad of its own row), lane l receives its row's exact integer dots with
// all four tokens and every product of the instruction is a real one.  The kernel so
// keeps the batch-1 layout -- one row per lane, each unit decoded once -- and runs four
// binary32 chains per lane, one per token, with the batch-1 arithmetic: every output
// equals its own matvec bit for bit.  With fewer than four tokens the missing ones
// repeat the last token and are not stored.
constexpr uint32_t kQuadTok = 4;
constexpr uint32_t kQuadRowDw = 36;  // LDS dwords per (unit, token): 32 codes + 4 of padding
constexpr uint32_t kQuadMaxCols = 16384;

template <Op O>
constexpr bool quad_supported() {
    return O == Op::PTQ1_SRC || O == Op::PTQ1_PINNED || O == Op::Q8_0 || O == Op::Q2K;
}

// Staged activation per unit: LDS dwords per (unit, token) row -- Q8_0 units (128
// elements) 32 codes, Q2_K units (one Q8_K block of 256) 64, plus 4 of padding -- and
// scales per unit (Q8_0: [group][token], Q8_K: [token]).
template <Op O>
constexpr uint32_t quad_row_dw() {
    return O == Op::Q2K ? 68u : kQuadRowDw;
}
template <Op O>
constexpr uint32_t quad_unit_scales() {
    return O == Op::Q2K ? kQuadTok : 4u * kQuadTok;
}
template <Op O>
constexpr uint32_t quad_unit_lds() {
    return (kQuadTok * quad_row_dw<O>() + quad_unit_scales<O>()) * static_cast<uint32_t>(sizeof(uint32_t));
}

// Threads per workgroup: the PTQ1 table (64 KiB of LDS) is filled once per CU for 16
// wavefronts; Q8_0 and Q2_K need no table and run four.
template <Op O>
constexpr uint32_t quad_threads() {
    return kind_of<O>() == kPTQ1 ? 1024u : 256u;
}

__device__ __forceinline__ v4i mfma4(uint32_t a, uint32_t b, v4i c) {
    return __builtin_amdgcn_mfma_i32_4x4x4i8(static_cast<int>(a), static_cast<int>(b), c, 0, 0, 0);
}

// Chains of one row and four tokens.
template <Op O>
struct QuadChain {
    float o[kQuadTok] = {0.0f, 0.0f, 0.0f, 0.0f};
    float L[4][kQuadTok] = {};  // pinned PTQ1: [native lane][token]

    __device__ __forceinline__ float result(int t) const {
        if constexpr (O == Op::PTQ1_PINNED) return (L[0][t] + L[1][t]) + (L[2][t] + L[3][t]);
        return o[t];
    }
};

// One unit of one row into the four chains.  `qa` holds the unit's 32 activation dwords
// of the lane's token (l%4), `qs` the unit's token scales as [group][token].  TERMS
// (source PTQ1 only): ch.o[t] receives the unit's term of token t instead, for a chain
// folded elsewhere.
template <Op O, bool TERMS = false>
__device__ __forceinline__ void quad_unit(const Raw<O> &w, const uint32_t *qa, const float *qs, uint32_t lbase,
                                          QuadChain<O> &ch) {
    static_assert(!TERMS || O == Op::PTQ1_SRC, "one term per unit and token");
    if constexpr (O == Op::Q2K) {
        // kquants::dot per token (dot_q2_k_block, src/kernels/kquants.rs:193-196): isum =
        // sum_g scale_g * dot_g and msum = sum_g min_g * bsum_g, exact integers.  The weight
        // operand carries scale_g * q (at most 45, still a byte); a second product with
        // min_g repeated gives min_g times the sub-block's activation sum.  Code dword 8h +
        // wh, field p holds elements 128h + 32p + 4wh..+3 of sub-block g = 8h + 2p + wh/4,
        // which meet the natural activation dword 32h + 8p + wh; four interleaved
        // accumulator chains of each sum, added at the end.
        v4i is[4] = {}, ms[4] = {};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const u32x4 a0 = *reinterpret_cast<const u32x4 *>(qa + 32 * h + 8 * p);
                const u32x4 a1 = *reinterpret_cast<const u32x4 *>(qa + 32 * h + 8 * p + 4);
                const uint32_t A[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int g = 8 * h + 2 * p + half;
                    const uint32_t byte = (w.sc[g >> 2] >> (8 * (g & 3))) & 0xffu;
                    const uint32_t scale = byte & 15u, mn = (byte >> 4) * 0x01010101u;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int wh = 4 * half + i;
                        const uint32_t q = (w.q[8 * h + wh] >> (2 * p)) & 0x03030303u;
                        is[i] = mfma4(A[wh], bytes_times(q, scale), is[i]);
                        ms[i] = mfma4(A[wh], mn, ms[i]);
                    }
                }
            }
        }
        const float d = h2f(w.dm & 0xffffu), dmin = h2f(w.dm >> 16);
#pragma unroll
        for (int t = 0; t < static_cast<int>(kQuadTok); ++t) {
            const int isum = (is[0][t] + is[1][t]) + (is[2][t] + is[3][t]);
            const int msum = (ms[0][t] + ms[1][t]) + (ms[2][t] + ms[3][t]);
            const float as = qs[t];
            ch.o[t] = ch.o[t] + ((as * d) * static_cast<float>(isum) - (as * dmin) * static_cast<float>(msum));
        }
    } else {
        uint32_t A[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(qa + 4 * i);
            A[4 * i] = v.x; A[4 * i + 1] = v.y; A[4 * i + 2] = v.z; A[4 * i + 3] = v.w;
        }
        float S[4][kQuadTok];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4 v = *reinterpret_cast<const float4 *>(qs + 4 * g);
            S[g][0] = v.x; S[g][1] = v.y; S[g][2] = v.z; S[g][3] = v.w;
        }
        // PTQ1 weights and activations are both in ptq1_slots_lut's slot order; Q8_0's in the
        // natural order (slot 8g + i is quad i of group g).
        uint32_t W[32];
        if constexpr (kind_of<O>() == kPTQ1) {
            ptq1_slots_lut<O == Op::PTQ1_PINNED>(w.x, lbase, [&](int s, uint32_t t) { W[s] = t; });
        } else {
#pragma unroll
            for (int q = 0; q < 32; ++q) W[q] = w.c[q];
        }
        auto slot = [](int g, int i) { return kind_of<O>() == kPTQ1 ? kPtq1GroupSlots[g][i] : 8 * g + i; };
        if constexpr (O == Op::PTQ1_PINNED) {
            // dot_q8_groups_pinned, src/kernels.rs:1134-1146: native lane l sums positions
            // 4l..4l+3 and 16+4l..16+4l+3 of the group (two slots), then
            // L[l] = fma(I_l, d * scale_g, L[l]).
            const float d = h2f(ptq1_scale_bits(w));
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                v4i acc[4];
#pragma unroll
                for (int l = 0; l < 4; ++l) {
                    const int s = kPtq1LaneSlots[g][l][0];
                    acc[l] = mfma4(A[s], W[s], v4i{0, 0, 0, 0});
                }
#pragma unroll
                for (int l = 0; l < 4; ++l) {
                    const int s = kPtq1LaneSlots[g][l][1];
                    acc[l] = mfma4(A[s], W[s], acc[l]);
                }
#pragma unroll
                for (int t = 0; t < static_cast<int>(kQuadTok); ++t) {
                    const float dd = d * S[g][t];
#pragma unroll
                    for (int l = 0; l < 4; ++l)
                        ch.L[l][t] = __builtin_fmaf(static_cast<float>(acc[l][t]), dd, ch.L[l][t]);
                }
            }
        } else {
            // The four groups' integer dots as four interleaved accumulator chains.
            v4i acc[4] = {};
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int g = 0; g < 4; ++g) acc[g] = mfma4(A[slot(g, i)], W[slot(g, i)], acc[g]);
            if constexpr (O == Op::PTQ1_SRC) {
                // dot_q8_groups, src/kernels.rs:1043-1064: fl(tt + fl(scale * I)) is one FMA, since
                // the binary16 scale (11 significant bits) times |I| < 2^13 is exact in binary32.
                const float d = h2f(ptq1_scale_bits(w));
#pragma unroll
                for (int t = 0; t < static_cast<int>(kQuadTok); ++t) {
                    float tt = 0.0f;
#pragma unroll
                    for (int g = 0; g < 4; ++g) tt = __builtin_fmaf(S[g][t], static_cast<float>(acc[g][t]), tt);
                    if constexpr (TERMS)
                        ch.o[t] = d * tt;
                    else
                        ch.o[t] = ch.o[t] + d * tt;
                }
            } else {
                // dot_legacy, src/kernels.rs:1241-1244; the row's chain adds the four group
                // terms in order.
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float sw = h2f((w.s[g >> 1] >> (16 * (g & 1))) & 0xffffu);
#pragma unroll
                    for (int t = 0; t < static_cast<int>(kQuadTok); ++t)
                        ch.o[t] = ch.o[t] + (sw * S[g][t]) * static_cast<float>(acc[g][t]);
                }
            }
        }
    }
}

// LDS bytes per unit: the four tokens' codes, then their 16 scales.
constexpr uint32_t kQuadUnitLds = (kQuadTok * kQuadRowDw + 4 * kQuadTok) * sizeof(uint32_t);

// The workgroup's staging of 2..4 tokens' prepared Q8_0 blocks (token t at act + t *
// act_stride bytes; missing tokens repeat the last): codes as [unit][token][36 dwords]
// (PTQ1 in ptq1_slots_lut's slot order), scales as [unit][group][token] floats.
template <Op O>
__device__ __forceinline__ void quad_stage(const void *__restrict__ act, uint32_t act_stride, uint32_t ntok,
                                           uint32_t nu, uint32_t *codes, float *scales) {
    if constexpr (O == Op::Q2K) {
        // Q8_K blocks, one per unit: codes as [unit][token][68 dwords], scales as [unit][token].
        for (uint32_t i = threadIdx.x; i < nu * kQuadTok * 64u; i += blockDim.x) {
            const uint32_t dw = i & 63u, t = (i >> 6) & 3u, u = i >> 8;
            const Q8KBlock *blk = reinterpret_cast<const Q8KBlock *>(static_cast<const uint8_t *>(act) +
                                                                     static_cast<size_t>(t < ntok ? t : ntok - 1) *
                                                                         act_stride) + u;
            codes[(u * kQuadTok + t) * quad_row_dw<O>() + dw] = reinterpret_cast<const uint32_t *>(blk->values)[dw];
            if (dw == 0) scales[u * kQuadTok + t] = blk->scale;
        }
        return;
    }
    for (uint32_t i = threadIdx.x; i < nu * 128u; i += blockDim.x) {
        const uint32_t dw = i & 7u, t = (i >> 3) & 3u, g = (i >> 5) & 3u, u = i >> 7;
        const Q8Block *blk = reinterpret_cast<const Q8Block *>(static_cast<const uint8_t *>(act) +
                                                               static_cast<size_t>(t < ntok ? t : ntok - 1) *
                                                                   act_stride) + 4 * u + g;
        const uint32_t v = reinterpret_cast<const uint32_t *>(blk->values)[dw];
        uint32_t *row = codes + (u * kQuadTok + t) * kQuadRowDw;
        if constexpr (kind_of<O>() == kPTQ1) {
            uint8_t *rb = reinterpret_cast<uint8_t *>(row);
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j)
                rb[ptq1_slot_byte(32 * g + 4 * dw + j, O == Op::PTQ1_PINNED)] = static_cast<uint8_t>(v >> (8 * j));
        } else {
            row[8 * g + dw] = v;
        }
        if (dw == 0) scales[(u * 4 + g) * kQuadTok + t] = blk->scale;
    }
}

// 2..4 tokens of prepared Q8_0 blocks (token t at act + t * act_stride bytes, outputs
// and residual at t * rows).  The workgroup stages every token's activation codes in
// LDS ([unit][token][36] dwords; PTQ1 codes in the decode's slot order) and their
// scales ([unit][group][token] floats) once; its wavefronts then walk 64-row tiles as
// the batch-1 row kernel does.
template <Op O, bool TAIL = false>
__global__ __launch_bounds__(quad_threads<O>()) void k_mv_quad(MvParams p, const void *__restrict__ act,
                                                              uint32_t act_stride, uint32_t ntok) {
    extern __shared__ __attribute__((aligned(16))) uint32_t quad_lds[];
    constexpr uint32_t UB = unit_bytes<O>();
    constexpr uint32_t kWaves = quad_threads<O>() / 64;
    constexpr uint32_t RDW = quad_row_dw<O>(), USC = quad_unit_scales<O>();
    const uint32_t nu = p.nu;
    uint32_t *codes = quad_lds;
    float *scales = reinterpret_cast<float *>(quad_lds + nu * kQuadTok * RDW);
    if constexpr (kind_of<O>() == kPTQ1) ptq1_lut_fill(threadIdx.x, blockDim.x);
    quad_stage<O>(act, act_stride, ntok, nu, codes, scales);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tiles = (p.rows + kTile - 1) / kTile;
    const uint32_t lbase = 8u * (lane & 31u);
    const uint32_t *qa = codes + (lane & 3u) * RDW;
    const uint32_t row_bytes = nu * UB;
    // Wave-uniform by construction (the buffer descriptors below must live in SGPRs).
    const uint32_t grid = __builtin_amdgcn_readfirstlane(gridDim.x);
    // Units [u0, u1) of a tile through step(raw unit, u), two buffers in ping-pong.
    auto walk = [&](uint32_t tile, uint32_t u0, uint32_t u1, auto &&step) {
        const uint32_t left = p.rows - tile * kTile;
        const uint32_t trp = ((left < kTile ? left : kTile) + 7u) & ~7u;
        const __amdgpu_buffer_rsrc_t rs =
            make_rsrc(p.w[0] + static_cast<size_t>(tile) * kTile * row_bytes, trp * row_bytes);
        Raw<O> A, B;
        uint32_t u = u0;
        if (u < u1) load_unit<O>(A, rs, u * trp * UB, trp, lane);
        while (u + 1 < u1) {
            load_unit<O>(B, rs, (u + 1) * trp * UB, trp, lane);
            step(A, u);
            if (u + 2 < u1) load_unit<O>(A, rs, (u + 2) * trp * UB, trp, lane);
            step(B, u + 1);
            u += 2;
        }
        if (u < u1) step(A, u);
    };
    auto chain = [&](QuadChain<O> &ch) {
        return [&](const Raw<O> &w, uint32_t u) { quad_unit<O>(w, qa + u * kQuadTok * RDW, scales + u * USC, lbase, ch); };
    };
    auto store = [&](uint32_t tile, const QuadChain<O> &ch) {
        const uint32_t left = p.rows - tile * kTile;
        if (lane < (left < kTile ? left : kTile)) {
            const size_t row = static_cast<size_t>(tile) * kTile + lane;
#pragma unroll
            for (uint32_t t = 0; t < kQuadTok; ++t) {
                if (t < ntok) {
                    const size_t at = static_cast<size_t>(t) * p.rows + row;
                    float o = ch.result(static_cast<int>(t));
                    if (p.residual) o = o + p.residual[at];
                    p.out[at] = o;
                    if (!finite(o)) raise_error(p.err, kErrNonfinite);
                }
            }
        }
    };
    if constexpr (!TAIL) {
        for (uint32_t tile = wave * grid + blockIdx.x; tile < tiles; tile += grid * kWaves) {
            QuadChain<O> ch;
            walk(tile, 0, nu, chain(ch));
            store(tile, ch);
        }
    } else {
        // Eight to twelve tiles per workgroup (source PTQ1): wavefronts 0..7 take one whole
        // tile each; wavefronts 8..15 take the remaining tiles in pairs, the second of a
        // pair leaving its units' terms in LDS ([slot][unit - nh][token][row]) for the
        // first, which continues its chains with them in unit order after the barrier.
        static_assert(O == Op::PTQ1_SRC && kWaves == 16, "single-term order, 16 wavefronts");
        float *second = scales + nu * USC;
        const uint32_t nh = (nu + 1) / 2, n2 = nu - nh;
        const uint32_t slot = (wave - 8) >> 1, half = wave & 1u;
        const uint32_t tile = wave < 8 ? wave * grid + blockIdx.x : 8 * grid + slot * grid + blockIdx.x;
        const bool active = tile < tiles;
        QuadChain<O> ch;
        if (wave < 8) {
            walk(tile, 0, nu, chain(ch));  // tile < 8 * grid < tiles
            store(tile, ch);
        } else if (active) {
            if (half == 0) {
                walk(tile, 0, nh, chain(ch));
            } else {
                float *mine = second + static_cast<size_t>(slot) * n2 * kQuadTok * kTile;
                walk(tile, nh, nu, [&](const Raw<O> &w, uint32_t u) {
                    QuadChain<O> tc;
                    quad_unit<O, true>(w, qa + u * kQuadTok * RDW, scales + u * USC, lbase, tc);
#pragma unroll
                    for (uint32_t t = 0; t < kQuadTok; ++t) mine[((u - nh) * kQuadTok + t) * kTile + lane] = tc.o[t];
                });
            }
        }
        __syncthreads();  // every wavefront reaches this one barrier
        if (wave >= 8 && active && half == 0) {
            const float *theirs = second + static_cast<size_t>(slot) * n2 * kQuadTok * kTile;
            for (uint32_t u = 0; u < n2; ++u)
#pragma unroll
                for (uint32_t t = 0; t < kQuadTok; ++t) ch.o[t] = ch.o[t] + theirs[(u * kQuadTok + t) * kTile + lane];
            store(tile, ch);
        }
    }
}

// Matrices of fewer tiles than CUs (source PTQ1, 2..4 tokens): one 1024-thread workgroup
// per 64-row tile.  Its wavefronts take the tile's units round-robin, each unit decoded
// once for all tokens as in k_mv_quad, and leave every (unit, token, row) term in LDS;
// after one barrier, 256 threads fold the 64 rows x 4 tokens chains in unit order, so each
// output is its batch-1 chain, only computed later.  LDS: the table, the staged codes
// and scales, and the terms ([unit][token][row] floats).
constexpr uint32_t kQuadSplitThreads = 1024;
constexpr uint32_t kQuadSplitUnitLds = kQuadUnitLds + kQuadTok * kTile * sizeof(float);
constexpr uint32_t kQuadSplitMaxUnits = 56;  // with the 64 KiB table, at most 155 KiB of LDS

__global__ __launch_bounds__(kQuadSplitThreads) void k_mv_quad_split(MvParams p, const void *__restrict__ act,
                                                                    uint32_t act_stride, uint32_t ntok) {
    constexpr Op O = Op::PTQ1_SRC;
    constexpr uint32_t UB = unit_bytes<O>();
    extern __shared__ __attribute__((aligned(16))) uint32_t quad_lds[];
    const uint32_t nu = p.nu;
    uint32_t *codes = quad_lds;
    float *scales = reinterpret_cast<float *>(quad_lds + nu * kQuadTok * kQuadRowDw);
    float *terms = scales + nu * 4 * kQuadTok;
    ptq1_lut_fill(threadIdx.x, blockDim.x);
    quad_stage<O>(act, act_stride, ntok, nu, codes, scales);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nwaves = kQuadSplitThreads / 64;
    const uint32_t tile = blockIdx.x;
    const uint32_t left = p.rows - tile * kTile;
    const uint32_t trows = left < kTile ? left : kTile;
    const uint32_t trp = (trows + 7u) & ~7u;
    const uint32_t row_bytes = nu * UB;
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(p.w[0] + static_cast<size_t>(tile) * kTile * row_bytes, trp * row_bytes);
    const uint32_t lbase = 8u * (lane & 31u);
    const uint32_t *qa = codes + (lane & 3u) * kQuadRowDw;
    auto step = [&](const Raw<O> &w, uint32_t u) {
        QuadChain<O> ch;
        quad_unit<O, true>(w, qa + u * kQuadTok * kQuadRowDw, scales + u * 4 * kQuadTok, lbase, ch);
#pragma unroll
        for (uint32_t t = 0; t < kQuadTok; ++t) terms[(u * kQuadTok + t) * kTile + lane] = ch.o[t];
    };
    Raw<O> A, B;
    uint32_t u = wave;
    if (u < nu) load_unit<O>(A, rs, u * trp * UB, trp, lane);
    while (u + nwaves < nu) {
        load_unit<O>(B, rs, (u + nwaves) * trp * UB, trp, lane);
        step(A, u);
        if (u + 2 * nwaves < nu) load_unit<O>(A, rs, (u + 2 * nwaves) * trp * UB, trp, lane);
        step(B, u + nwaves);
        u += 2 * nwaves;
    }
    if (u < nu) step(A, u);
    __syncthreads();
    if (threadIdx.x < kQuadTok * kTile) {
        const uint32_t t = threadIdx.x >> 6, r = threadIdx.x & 63u;
        if (t < ntok && r < trows) {
            // dot_q8_groups' row chain, src/kernels.rs:1043-1064: ((0 + t_0) + t_1) + ...
            float o = 0.0f;
            for (uint32_t v = 0; v < nu; ++v) o = o + terms[(v * kQuadTok + t) * kTile + r];
            const size_t at = static_cast<size_t>(t) * p.rows + static_cast<size_t>(tile) * kTile + r;
            if (p.residual) o = o + p.residual[at];
            p.out[at] = o;
            if (!finite(o)) raise_error(p.err, kErrNonfinite);
        }
    }
}

// ---- native -> tiled repack ------------------------------------------------------------
// One thread per (row, unit).  Byte copies: this runs once per uploaded tensor.
__global__ void k_repack(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, uint32_t kind, uint64_t rows,
                         uint32_t nu) {
    TiledFormat f;
    tiled_format(kind, &f);
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= rows * nu) return;
    const uint64_t r = idx / nu;
    const uint32_t u = static_cast<uint32_t>(idx % nu);
    const uint64_t row_bytes = static_cast<uint64_t>(nu) * f.unit_bytes;
    const uint64_t tile = r / kTile;
    const uint32_t lr = static_cast<uint32_t>(r % kTile);
    const uint32_t trp = tile_rows_padded(rows, tile);
    const uint8_t *s = src + r * row_bytes + static_cast<uint64_t>(u) * f.unit_bytes;
    uint8_t *seg = dst + tile * kTile * row_bytes + static_cast<uint64_t>(u) * trp * f.unit_bytes;
    for (uint32_t p = 0; p < f.npieces; ++p) {
        uint8_t *d = seg + static_cast<uint64_t>(f.poff[p]) * trp + static_cast<uint64_t>(lr) * f.psize[p];
        if (kind == kQ8_0 && p == 8) {
            for (int j = 0; j < 4; ++j) {
                d[2 * j] = s[34 * j];
                d[2 * j + 1] = s[34 * j + 1];
            }
        } else {
            for (uint32_t i = 0; i < f.psize[p]; ++i) d[i] = s[f.nsrc[p] + i];
        }
    }
}

constexpr size_t kSplitLds = 64 * 1024;

struct SplitPlan {
    uint32_t ks, lpr, lg_ks, lg_lpr;
    size_t lds;
};

// Split-mode geometry: enough lane groups per row that the tiles cover every CU,
// then enough wavefronts per workgroup for ~8 resident wavefronts per CU, never
// more K-split ways than the row has units.
// max_lpr caps the lane groups per row (a workgroup then owns at least 64/max_lpr rows).
template <Op O>
bool plan_split(uint64_t rows, uint32_t nu, uint32_t cols, bool quant, uint32_t nmat, uint32_t cus, SplitPlan *pl,
                uint32_t max_lpr = 8) {
    const uint64_t tiles = (rows + kTile - 1) / kTile;
    uint32_t lpr = 1;
    while (lpr < max_lpr && tiles * lpr < cus && lpr * 2 <= nu) lpr *= 2;
    uint32_t ks = 1;
    while (ks * 2 * nmat <= kSplitMaxWaves && ks * 2 * lpr <= nu && tiles * lpr * ks * 2 * nmat <= 8ull * cus) ks *= 2;
    // A quantizing prologue wants several wavefronts per workgroup: trade lane groups
    // for wavefronts while the workgroup has fewer than four.
    while (quant && ks * nmat < 4 && lpr > 1 && ks * 2 * nmat <= kSplitMaxWaves) {
        lpr /= 2;
        ks *= 2;
    }
    // activation blocks | terms (| SwiGLU inputs) | 16 doubles for the RMSNorm reduction
    auto lds = [&](uint32_t groups) -> size_t {
        const uint32_t rw = kTile / groups;
        return align16(act_bytes_for<O>(cols)) +
               align16(static_cast<uint32_t>(sizeof(float) * (nmat * rw * (nu * terms_per_unit<O>() + 1) + 2 * rw))) +
               16 * sizeof(double);
    };
    // Long rows whose terms overflow LDS at this split: more lane groups per row, so a
    // workgroup holds fewer rows' terms (pinned PTQ1 at 17408 inputs: 16 rows' terms take
    // 78 KiB, 8 rows' 39 KiB).
    while (lds(lpr) > kSplitLds && lpr < max_lpr && ks * lpr * 2 <= nu) lpr *= 2;
    pl->ks = ks;
    pl->lpr = lpr;
    pl->lg_ks = static_cast<uint32_t>(__builtin_ctz(ks));
    pl->lg_lpr = static_cast<uint32_t>(__builtin_ctz(lpr));
    pl->lds = lds(lpr);
    return pl->lds <= kSplitLds;
}

template <Op O>
int launch_op(const MatvecArgs &a, const void *act, float *out) {
    const uint32_t nu = static_cast<uint32_t>(a.cols / unit_weights<O>());
    const uint64_t tiles = (a.rows + kTile - 1) / kTile;
    const bool quant = a.act_format == kActF32;
    const uint32_t nmat = a.w2 ? 2u : 1u;
    MvParams p{};
    p.w[0] = a.w;
    p.w[1] = a.w2 ? a.w2 : a.w;
    p.rows = static_cast<uint32_t>(a.rows);
    p.nu = nu;
    p.cols = static_cast<uint32_t>(a.cols);
    p.act = act;
    p.qcontract = a.qcontract;
    p.pinned = a.pinned;
    p.out = out;
    p.residual = a.residual;
    p.err = a.err;
    p.norm_w = a.norm_w;
    p.eps = a.eps;
    // SwiGLU blocks (q8_out): every 32 rows of a workgroup form one Q8_0 block.
    if (a.q8_out && (nmat != 2 || a.rows % 32 != 0)) return -2;
    p.q8_out = static_cast<Q8Block *>(a.q8_out);
    p.q8_contract = a.q8_contract;
    p.tile_best = static_cast<TileBest *>(a.tile_best);
    if constexpr (kind_of<O>() != kPTQ1) {
        if (p.tile_best) {
            if (quant || nmat != 1) return -2;
            hipLaunchKernelGGL(k_mv_rows<O>, dim3(static_cast<uint32_t>(tiles)), dim3(64), 0, a.stream, p);
            return launch_status();
        }
    } else {
        if (p.tile_best) return -2;
    }
    if constexpr (kind_of<O>() == kPTQ1) {
        // Measured, prepared activations (us, split kernel -> spread): 12288x4096 8.6 -> 6.9
        // (pinned 14.0 -> 10.8), 8192x4096 6.7 -> 6.6; fewer tiles or longer rows lose to
        // the split kernel (2048x2048 4.2 -> 4.8, 6144x2048 5.0 -> 5.1, 2048x6144 5.4 -> 7.6).
        // Rows of up to 64 units from half a tile per CU (against the split kernel below one
        // tile per CU, the split-pair table kernel above): 10240x5120 10.0 -> 7.3, 12288x5120
        // 10.1 -> 7.6, 17408x5120 21.3 -> 10.6.
        const uint32_t sgrid = static_cast<uint32_t>(tiles < a.cus ? tiles : a.cus);
        if (!quant && nmat == 1 && 2 * tiles > a.cus && nu <= 64) {
            if (const uint32_t lds = lut_spread_lds<O>(static_cast<uint32_t>(tiles), sgrid, nu)) {
                hipLaunchKernelGGL((k_mv_rows_lut<O, kLutSpread>), dim3(sgrid), dim3(kLutThreads), lds, a.stream, p,
                                   act);
                return launch_status();
            }
        }
    }
    if constexpr (kind_of<O>() != kPTQ1) {
        // Half a tile to one tile per CU, prepared activations: 16 wavefronts per tile from
        // 16 units per row, 8 from 8.  Measured (us, split kernel -> N wavefronts), 12288
        // rows x 4096: Q8_0 12.6 -> 12.0, Q2_K 7.4 -> 6.0, PQ2 7.9 -> 6.9, TQ1_0 8.2 -> 6.7,
        // TQ2_0 6.9 -> 5.5; 10240 x 4096 Q8_0 12.2 -> 10.9; 12288 x 2048 Q2_K 5.6 -> 4.2 (8
        // wavefronts; 4 gave 4.4).  One to four tiles per CU: 8 wavefronts per tile, against
        // the one- or two-wavefront row kernels (us): 17408 x 5120 Q8_0 26.1 -> 24.1, Q2_K 13.0
        // -> 10.2, PQ2 18.1 -> 11.9; 32768 x 4096 Q2_K 12.4 -> 10.8, PQ2 16.5 -> 11.2 (16
        // wavefronts per tile lost there: Q2_K 17408 x 5120 13.1).
        auto rowsn = [&]<uint32_t NW>() -> int {
            const uint32_t c1 = nu / NW;
            const uint32_t stride = ((nu - c1) * terms_per_unit<O>()) | 1u;
            if (kTile * stride * sizeof(float) > 64u * 1024u) return -1;
            hipLaunchKernelGGL((k_mv_rowsn<O, NW>), dim3(static_cast<uint32_t>(tiles)), dim3(64 * NW),
                               kTile * stride * sizeof(float), a.stream, p, stride);
            return launch_status();
        };
        if (!quant && nmat == 1 && tiles < 4ull * a.cus && 2 * tiles > a.cus && nu >= 8) {
            const int rc = nu >= 16 && tiles < a.cus ? rowsn.template operator()<16>() : rowsn.template operator()<8>();
            if (rc >= 0) return rc;
        }
    }
    if (!quant && nmat == 1 && tiles >= a.cus) {
        if constexpr (kind_of<O>() == kPTQ1) {
            constexpr int kSplitMode = lut_can_split<O>() ? kLutSplit : kLutWhole;
            const uint32_t tail_lds = lut_tail_lds<O>(static_cast<uint32_t>(tiles), a.cus, nu);
            if (lut_can_split<O>() && lut_split(static_cast<uint32_t>(tiles), a.cus, nu))
                hipLaunchKernelGGL((k_mv_rows_lut<O, kSplitMode>), dim3(a.cus), dim3(kLutThreads), 0, a.stream, p,
                                   act);
            else if (tail_lds)
                hipLaunchKernelGGL((k_mv_rows_lut<O, kLutTail>), dim3(a.cus), dim3(kLutThreads), tail_lds, a.stream,
                                   p, act);
            else
                hipLaunchKernelGGL((k_mv_rows_lut<O, kLutWhole>), dim3(a.cus), dim3(kLutThreads), 0, a.stream, p,
                                   act);
            return launch_status();
        }
        if constexpr (O != Op::PTQ1_PINNED) {
            // Two wavefronts per tile up to eight tiles per CU (Q8_0: two), and for Q2_K at
            // any size.  Measured at 4096 columns: Q2_K 16.8 -> 12.1 us (32768 rows), 20.5 ->
            // 18.2 (65536), 41.8 -> 40.7 (151936); TQ2_0 22.5 -> 17.0 (65536); PQ2 25.4 ->
            // 16.4 and TQ1_0 20.6 -> 16.4 (32768); Q8_0 28.0 -> 27.2 at 32768 rows but 2 %
            // slower at 65536, and Q8_0 / TQ2_0 1-5 % slower split at 151936 rows.
            // Second-half terms per row, odd stride (no bank conflicts).
            const uint32_t stride = ((nu - (nu + 1) / 2) * terms_per_unit<O>()) | 1u;
            const uint64_t most = O == Op::Q8_0 ? 2ull * a.cus : 8ull * a.cus;
            if (nu >= 4 && stride <= 129 && (O == Op::Q2K || tiles <= most)) {
                hipLaunchKernelGGL(k_mv_rows2<O>, dim3(static_cast<uint32_t>(tiles)), dim3(128),
                                   kTile * stride * sizeof(float), a.stream, p, stride);
                return launch_status();
            }
        }
        hipLaunchKernelGGL(k_mv_rows<O>, dim3(static_cast<uint32_t>(tiles)), dim3(64), 0, a.stream, p);
        return launch_status();
    }
    SplitPlan pl;
    if (!plan_split<O>(a.rows, nu, p.cols, quant, nmat, a.cus, &pl, a.q8_out ? 2u : 8u)) {
        // Rows too wide for the split kernel's LDS (the activation and every unit's terms of a
        // workgroup's rows): prepared activations take a row-tile kernel, which has no width
        // limit (f32 input is quantized by the caller first, op_needs_prepared).
        if (quant || nmat != 1) return -2;
        const uint32_t grid = static_cast<uint32_t>(tiles < a.cus ? tiles : a.cus);
        if constexpr (kind_of<O>() == kPTQ1) {
            // The tile's units over 16 wavefronts with their terms in LDS when they fit beside
            // the table, else one wavefront per tile.
            if (const uint32_t lds = lut_spread_lds<O>(static_cast<uint32_t>(tiles), grid, nu))
                hipLaunchKernelGGL((k_mv_rows_lut<O, kLutSpread>), dim3(grid), dim3(kLutThreads), lds, a.stream, p, act);
            else
                hipLaunchKernelGGL((k_mv_rows_lut<O, kLutWhole>), dim3(grid), dim3(kLutThreads), 0, a.stream, p, act);
            return launch_status();
        } else {
            const uint32_t stride = ((nu - (nu + 1) / 2) * terms_per_unit<O>()) | 1u;
            if (O != Op::PTQ1_PINNED && nu >= 4 && stride <= 129)
                hipLaunchKernelGGL(k_mv_rows2<O>, dim3(static_cast<uint32_t>(tiles)), dim3(128),
                                   kTile * stride * sizeof(float), a.stream, p, stride);
            else
                hipLaunchKernelGGL(k_mv_rows<O>, dim3(static_cast<uint32_t>(tiles)), dim3(64), 0, a.stream, p);
            return launch_status();
        }
    }
    p.ks = pl.ks;
    p.lpr = pl.lpr;
    p.lg_ks = pl.lg_ks;
    p.lg_lpr = pl.lg_lpr;
    p.xcd_tiles = pl.lpr > 1 && tiles % 8 == 0;
    const dim3 grid(static_cast<uint32_t>(tiles * pl.lpr)), block(64 * pl.ks * nmat);
    // Held prologue input: eight values per lane when one chunk per wavefront covers the
    // input, else sixteen in up to two chunks (each chunk's block reductions are a fixed
    // cost, so fewer chunks win over fewer values), else streamed.
    const uint32_t nwaves = pl.ks * nmat;
    constexpr bool q8k = act_is_q8k<O>();
    const int held = HeldInput<q8k, 8, 1>::fits(p.cols, nwaves) ? 8 : HeldInput<q8k, 16, 2>::fits(p.cols, nwaves) ? 16 : 0;
    auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, block, pl.lds, a.stream, p); };
    if (nmat == 2) {
        if (!quant) return -2;
        if (held == 8)
            go(k_mv_split<O, true, 2, 8>);
        else if (held == 16)
            go(k_mv_split<O, true, 2, 16>);
        else
            go(k_mv_split<O, true, 2, 0>);
    } else if (quant) {
        if (held == 8)
            go(k_mv_split<O, true, 1, 8>);
        else if (held == 16)
            go(k_mv_split<O, true, 1, 16>);
        else
            go(k_mv_split<O, true, 1, 0>);
    } else {
        go(k_mv_split<O, false, 1, 0>);
    }
    return launch_status();
}

// Whether an f32-input call must quantize in a separate launch: the row-tile kernels take
// prepared blocks, and the split kernel's quantizing prologue needs its plan to fit LDS.
// A gate+up pair (w2) has no prepared-block kernel: true there sends the caller to
// separate gate and up projections.
template <Op O>
bool op_needs_prepared(const MatvecArgs &a) {
    const uint64_t tiles = (a.rows + kTile - 1) / kTile;
    if (!a.w2 && tiles >= a.cus) return true;
    SplitPlan pl;
    const uint32_t nu = static_cast<uint32_t>(a.cols / unit_weights<O>());
    return !plan_split<O>(a.rows, nu, static_cast<uint32_t>(a.cols), true, a.w2 ? 2u : 1u, a.cus, &pl,
                          a.q8_out ? 2u : 8u);
}

// Selects the arithmetic order from (kind, activation format, pinned): the orders of
// dot_q8_groups / dot_q8_groups_pinned / dot_ptq1_q8k / dot_pq2::<FUSED> /
// kquants::dot / dot_legacy (src/kernels.rs:941-1248, src/kernels/kquants.rs:346-430).
template <typename F>
int dispatch(const MatvecArgs &a, F &&f) {
    const bool q8k = a.act_format == kActQ8K || (a.act_format == kActF32 && a.qcontract_is_q8k);
    if (a.kind == kPTQ1) {
        if (q8k) return f.template operator()<Op::PTQ1_Q8K>();
        return a.pinned ? f.template operator()<Op::PTQ1_PINNED>() : f.template operator()<Op::PTQ1_SRC>();
    }
    if (a.kind == kPQ2) {
        if (!q8k) return f.template operator()<Op::PQ2_Q8>();
        return a.pinned ? f.template operator()<Op::PQ2_FUSED>() : f.template operator()<Op::PQ2_UNFUSED>();
    }
    if (a.kind == kQ2_K) return f.template operator()<Op::Q2K>();
    if (a.kind == kQ8_0) return f.template operator()<Op::Q8_0>();
    // TQ1_0 / TQ2_0 take Q8_K activations only (ActivationContract::for_tensor,
    // src/kernels.rs:1663-1673).
    if (a.kind == kTQ1_0 && q8k) return f.template operator()<Op::TQ1>();
    if (a.kind == kTQ2_0 && q8k) return f.template operator()<Op::TQ2>();
    return -2;
}

}  // namespace

bool tiled_supported(uint32_t kind, uint64_t cols, uint64_t rows, uint32_t cus) {
    if (rows == 0 || rows > 0xffffffffull) return false;
    TiledFormat f;
    if (!tiled_format(kind, &f) || cols % f.unit_weights) return false;
    const uint64_t row_bytes = cols / f.unit_weights * f.unit_bytes;
    if (row_bytes * kTile >= (1ull << 31)) return false;  // 32-bit in-tile offsets
    (void)cus;
    // Every width has a tiled kernel: fewer tiles than CUs run the split kernel where its LDS
    // holds the activation and every unit's terms of its rows, else a row-tile kernel.
    return true;
}

int launch_repack(const void *native, void *tiled, uint32_t kind, uint64_t cols, uint64_t rows, hipStream_t s) {
    TiledFormat f;
    if (!tiled_format(kind, &f)) return -2;
    const uint32_t nu = static_cast<uint32_t>(cols / f.unit_weights);
    const uint64_t n = rows * nu;
    hipLaunchKernelGGL(k_repack, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, s,
                       static_cast<const uint8_t *>(native), static_cast<uint8_t *>(tiled), kind, rows, nu);
    return launch_status();
}

template <Op O>
int launch_batch(const MatvecArgs &a, const void *act, uint32_t ntok, uint32_t act_stride, float *out,
                 const float *residual) {
    const uint64_t tiles = (a.rows + kTile - 1) / kTile;
    MvParams p{};
    p.w[0] = p.w[1] = a.w;
    p.rows = static_cast<uint32_t>(a.rows);
    p.nu = static_cast<uint32_t>(a.cols / unit_weights<O>());
    p.cols = static_cast<uint32_t>(a.cols);
    p.pinned = a.pinned;
    p.out = out;
    p.residual = residual;
    p.err = a.err;
    const dim3 grid(static_cast<uint32_t>(tiles)), block(64);
    if (ntok <= 4)
        hipLaunchKernelGGL((k_mv_rows_batch<O, 4>), grid, block, 0, a.stream, p, act, ntok, act_stride);
    else if (ntok <= 8)
        hipLaunchKernelGGL((k_mv_rows_batch<O, 8>), grid, block, 0, a.stream, p, act, ntok, act_stride);
    else
        hipLaunchKernelGGL((k_mv_rows_batch<O, 16>), grid, block, 0, a.stream, p, act, ntok, act_stride);
    return launch_status();
}

// Row count from which 2..16 tokens run on the matrix cores (16 rows per wavefront).
constexpr uint64_t kSkinnyMinRows = 1024;

// The row-tile batch kernel (one wavefront per 64-row tile runs every token's chain, each
// unit decoded once per batch): large matrices the skinny kernel leaves (pinned PTQ1 up
// to four tokens).
bool batch_eligible(const MatvecArgs &a) {
    return a.tokens >= 2 && !a.w2 && a.rows >= kBatchMinRows;
}

// Whether a skinny batch first copies its activations into lane order (one more launch,
// then contiguous loads) instead of gathering them from the prepared blocks in every
// wavefront.  Measured on 2048..151936 rows: the copy pays from 8192 rows or from 5
// tokens; Q2_K's 256-element units halve its gathers (as TQ2_0's, in the same order), and
// the copy pays only from 32768 rows.  PQ2 and Q8_0 rows of 12288 inputs or more take it
// from two tokens (us, gathered / copied: PQ2 5120 x 17408 3 tokens 37.6 / 30.1, 4096 x
// 14336 4 tokens 26.5 / 24.6; Q8_0 4096 x 14336 2 tokens 31.6 / 28.6); PTQ1 there is mixed
// (4096 x 14336 4 tokens 31.3 / 38.4, 5120 x 17408 55.4 / 45.9) and keeps the rule above.
template <Op O>
bool skinny_lane_ordered(uint64_t rows, uint64_t cols, uint32_t ntok) {
    if constexpr (O == Op::Q2K || O == Op::TQ2) return rows >= 32768;
    if constexpr (O == Op::Q8_0 || kind_of<O>() == kPQ2)
        if (cols >= 12288) return true;
    return rows >= 8192 || ntok > 4;
}

// 16-token chunks per skinny launch: the chunks run side by side (grid y), each a batch
// of its own, so a launch of up to kSkChunks * 16 tokens fills the chip where one chunk
// leaves it latency-bound.  Four chunks keep the lane-ordered copies under 10 MB at
// 65536 inputs.
constexpr uint32_t kSkChunks = 4;

template <Op O>
size_t skinny_scratch(const MatvecArgs &a) {
    if (!skinny_lane_ordered<O>(a.rows, a.cols, a.tokens < kBatchMax ? a.tokens : kBatchMax)) return 0;
    const uint64_t nu = a.cols / unit_weights<O>();
    const uint64_t chunks = (a.tokens + kBatchMax - 1) / kBatchMax;
    return nu * 64u * (sk_lane_bytes<O>() + 4u) * (chunks < kSkChunks ? chunks : kSkChunks);
}

// ntok: up to kSkChunks * 16 tokens, one chunk of 16 per grid row.
template <Op O>
int launch_skinny(const MatvecArgs &a, const void *act, uint32_t ntok, uint32_t act_stride, float *out,
                  const float *residual) {
    const uint32_t chunks = (ntok + kBatchMax - 1) / kBatchMax;
    if (chunks > kSkChunks) return -2;
    const bool sw = skinny_lane_ordered<O>(a.rows, a.cols, ntok < kBatchMax ? ntok : kBatchMax);
    if (sw && (!a.scratch || a.scratch_bytes < skinny_scratch<O>(a))) return -2;
    const uint32_t nu = static_cast<uint32_t>(a.cols / unit_weights<O>());
    const uint32_t sw_chunk = nu * 64u * (sk_lane_bytes<O>() + 4u);
    if (sw) {
        const uint32_t nprep = nu * 64u * (sk_lane_bytes<O>() / 4u);
        hipLaunchKernelGGL(k_sk_prep<O>, dim3((nprep + 255u) / 256u, chunks), dim3(256), 0, a.stream,
                           static_cast<const uint8_t *>(act), act_stride, ntok, nu, static_cast<uint32_t *>(a.scratch));
    }
    SkParams p{};
    p.w = a.w;
    p.sw = static_cast<const uint8_t *>(sw ? a.scratch : act);
    p.sw_chunk = sw ? sw_chunk : kBatchMax * act_stride;
    p.act_stride = act_stride;
    p.out = out;
    p.residual = residual;
    p.err = a.err;
    p.rows = static_cast<uint32_t>(a.rows);
    p.nu = nu;
    p.ntok = ntok;
    const uint64_t tiles = (a.rows + kTile - 1) / kTile;
    // Wavefronts per 16-row block: enough to give the chip about eight per SIMD.
    const uint64_t blocks = tiles * 4;
    const uint64_t want = 32ull * a.cus;
    int ks = blocks >= want ? 1 : blocks * 2 >= want ? 2 : blocks * 4 >= want ? 4 : 8;
    // The LDS terms buffer is 2 * KS * terms * 1 KiB: pinned PTQ1's twelve terms per
    // element cap it at two wavefronts per block (48 KiB).
    constexpr int kMaxKs = sk_terms_per_unit<O>() > 8 ? 2 : 8;
    if (ks > kMaxKs) ks = kMaxKs;
    const dim3 grid(static_cast<uint32_t>(blocks), chunks), block(64 * ks);
    auto go = [&]<bool SWv>() {
        if (ks == 1) hipLaunchKernelGGL((k_mv_skinny<O, SWv, 1>), grid, block, 0, a.stream, p);
        else if (ks == 2) hipLaunchKernelGGL((k_mv_skinny<O, SWv, 2>), grid, block, 0, a.stream, p);
        else if constexpr (kMaxKs >= 8) {
            if (ks == 4) hipLaunchKernelGGL((k_mv_skinny<O, SWv, 4>), grid, block, 0, a.stream, p);
            else hipLaunchKernelGGL((k_mv_skinny<O, SWv, 8>), grid, block, 0, a.stream, p);
        }
    };
    if (sw)
        go.template operator()<true>();
    else
        go.template operator()<false>();
    return launch_status();
}

// PTQ1 batches of two tokens on matrices of at least four tiles per CU, and of three
// tokens from eight tiles per CU, take the table kernel (decode once, one chain per
// token).  Measured (4096 inputs): two tokens 40 / 43 / 50 us at 65536 / 131072 /
// 151936 rows against 52 / 80 / 94 us on the matrix cores; three tokens 71 against
// 80 and 94 us from 131072 rows, but slower at 65536; four tokens slower everywhere.
bool lut_batch_eligible(const MatvecArgs &a) {
    if (a.w2 || a.kind != kPTQ1) return false;
    const uint64_t tiles = (a.rows + kTile - 1) / kTile;
    return (a.tokens == 2 && tiles >= 4ull * a.cus) || (a.tokens == 3 && tiles >= 8ull * a.cus);
}

template <Op O>
int launch_lut_batch(const MatvecArgs &a, uint32_t act_stride) {
    if constexpr (kind_of<O>() != kPTQ1) {
        return -2;
    } else {
        MvParams p{};
        p.w[0] = p.w[1] = a.w;
        p.rows = static_cast<uint32_t>(a.rows);
        p.nu = static_cast<uint32_t>(a.cols / unit_weights<O>());
        p.cols = static_cast<uint32_t>(a.cols);
        p.pinned = a.pinned;
        p.out = a.out;
        p.residual = a.residual;
        p.err = a.err;
        const dim3 grid(a.cus), block(kLutThreads);
        if (a.tokens == 2)
            hipLaunchKernelGGL((k_mv_rows_lut_batch<O, 2>), grid, block, 0, a.stream, p, a.act, act_stride);
        else
            hipLaunchKernelGGL((k_mv_rows_lut_batch<O, 3>), grid, block, 0, a.stream, p, a.act, act_stride);
        return launch_status();
    }
}

// Two to four tokens of a large PTQ1 (Q8_0 activations) or Q8_0 matrix run on the 4x4x4
// matrix cores: one row per lane and each unit decoded once, as at batch 1.  Source PTQ1
// from two tiles per CU (measured at 4096 columns and 4 tokens: 40960 rows 31.8 us against
// 33.1 split per tile and 38.0 on the skinny kernel); the other orders from 65536 rows.
bool quad_eligible(const MatvecArgs &a) {
    if (a.w2 || a.tokens < 2 || a.tokens > kQuadTok || a.act_format == kActF32 || a.cols > kQuadMaxCols)
        return false;
    const uint64_t tiles = (a.rows + kTile - 1) / kTile;
    return dispatch(a, [&]<Op O>() {
               if constexpr (!quad_supported<O>())
                   return 0;
               else
                   return a.rows >= kBatchMinRows || (O == Op::PTQ1_SRC && tiles > 2ull * a.cus) ? 1 : 0;
           }) == 1;
}

template <Op O>
int launch_quad(const MatvecArgs &a, uint32_t act_stride) {
    if constexpr (!quad_supported<O>()) {
        return -2;
    } else {
        MvParams p{};
        p.w[0] = p.w[1] = a.w;
        p.rows = static_cast<uint32_t>(a.rows);
        p.nu = static_cast<uint32_t>(a.cols / unit_weights<O>());
        p.cols = static_cast<uint32_t>(a.cols);
        p.pinned = a.pinned;
        p.out = a.out;
        p.residual = a.residual;
        p.err = a.err;
        const size_t lds = static_cast<size_t>(p.nu) * quad_unit_lds<O>();
        constexpr uint32_t kWaves = quad_threads<O>() / 64;
        const uint64_t tiles = (a.rows + kTile - 1) / kTile;
        // PTQ1: one workgroup per CU walks tiles (its table is filled once); Q8_0: one
        // tile per wavefront.
        uint64_t grid = kind_of<O>() == kPTQ1 ? a.cus : (tiles + kWaves - 1) / kWaves;
        if (grid > tiles) grid = tiles;
        if constexpr (O == Op::PTQ1_SRC) {
            // Eight to twelve tiles per CU: the last round as split pairs, when their terms
            // fit LDS beside the table (measured, 151936x4096: 4 tokens 50.3 -> 46.1 us, 2
            // tokens 50.1 -> 45.4 us).
            const size_t tail_lds =
                lds + 4 * static_cast<size_t>(p.nu - (p.nu + 1) / 2) * kQuadTok * kTile * sizeof(float);
            if (tiles > 8ull * a.cus && tiles <= 12ull * a.cus && tail_lds + 64 * 1024 <= 160 * 1024) {
                hipLaunchKernelGGL((k_mv_quad<O, true>), dim3(a.cus), dim3(quad_threads<O>()), tail_lds, a.stream, p,
                                   a.act, act_stride, a.tokens);
                return launch_status();
            }
        }
        hipLaunchKernelGGL(k_mv_quad<O>, dim3(static_cast<uint32_t>(grid)), dim3(quad_threads<O>()), lds, a.stream,
                           p, a.act, act_stride, a.tokens);
        return launch_status();
    }
}

// Source PTQ1, two to four tokens, from 3/8 of a tile per CU up to two tiles per CU: one
// workgroup per tile, its units split over 16 wavefronts.  Measured at 4 tokens against
// the skinny kernel (us): 6144x2048 8.0 / 8.9, 12288x4096 12.1 / 19.4, 16384x4096 12.7 /
// 22.4, 24576x4096 22.9 / 27.3; smaller matrices keep the skinny kernel (2048x2048 6.1
// against 7.7: the table and the staging are a fixed cost per tile).
bool quad_split_eligible(const MatvecArgs &a) {
    if (a.w2 || a.tokens < 2 || a.tokens > kQuadTok || a.act_format == kActF32) return false;
    const uint64_t tiles = (a.rows + kTile - 1) / kTile;
    if (tiles * 8 < 3ull * a.cus || tiles > 2ull * a.cus) return false;
    if (a.cols / unit_weights<Op::PTQ1_SRC>() > kQuadSplitMaxUnits) return false;
    return dispatch(a, [&]<Op O>() { return O == Op::PTQ1_SRC ? 1 : 0; }) == 1;
}

int launch_quad_split(const MatvecArgs &a, uint32_t act_stride) {
    MvParams p{};
    p.w[0] = p.w[1] = a.w;
    p.rows = static_cast<uint32_t>(a.rows);
    p.nu = static_cast<uint32_t>(a.cols / unit_weights<Op::PTQ1_SRC>());
    p.cols = static_cast<uint32_t>(a.cols);
    p.out = a.out;
    p.residual = a.residual;
    p.err = a.err;
    const uint64_t tiles = (a.rows + kTile - 1) / kTile;
    hipLaunchKernelGGL(k_mv_quad_split, dim3(static_cast<uint32_t>(tiles)), dim3(kQuadSplitThreads),
                       static_cast<size_t>(p.nu) * kQuadSplitUnitLds, a.stream, p, a.act, act_stride, a.tokens);
    return launch_status();
}

// Long rows on few tiles take the two-pass split-K (k_mv_terms + k_mv_fold) for source-order
// PTQ1 (prepared Q8_0 blocks, one term per unit; PQ2 below) at two to eight tokens, where the other paths
// run token by token or leave the skinny kernel's 16-token width mostly empty.  Measured
// (prepared activations, us, before -> split-K): 5120 x 17408 2 / 4 / 8 tokens 31.2 -> 21.0,
// 53.0 -> 28.1, 43.1 -> 35.3; 6144 x 16384 8 tokens 40.4 -> 35.4; 4096 x 14336 4 tokens 27.8 ->
// 20.5; 2048 x 16384 4 tokens 32.3 -> 18.2; 5120 x 6144 2 / 8 tokens 14.2 -> 11.7, 20.1 ->
// 17.7; 17408 x 5120 2 / 4 tokens 25.0 -> 16.0, 25.5 -> 20.3, where the quad-split kernel's
// one workgroup per tile runs in two rounds.  Rows under 64 units take it up to three tokens
// (four from 48 units): with f32 input the separate quantizing launch outweighs the gain from
// eight tokens (6144 x 5120 21.2 -> 23.4).  It loses at one token (two launches: 4096 x
// 14336 8.8 -> 12.8), at two tokens on small matrices (2048 x 8192 10.4 -> 12.1), from five
// tokens above half a tile per CU (12288 x 8192 8 tokens 29.1 -> 32.8), at sixteen (5120 x
// 17408 43.5 -> 67.8), and between half a tile and one tile per CU on rows under 64 units,
// where the quad-split kernel fits one round (10240 x 5120 4 tokens 13.4 against 16.3).  The
// terms it stores grow with tokens x units x terms per unit, so the other formats (Q8_0 4
// terms per unit: 5120 x 17408 16 tokens 37.5 -> 165.2) and the pinned orders (PTQ1 9 terms,
// fused PQ2 2) keep their kernels.
constexpr uint32_t kSplitKUnits = 4, kSplitKMinUnits = 40;

// Both users (source PTQ1, unfused PQ2) have 128-weight units and one term per unit.
static_assert(unit_weights<Op::PTQ1_SRC>() == unit_weights<Op::PQ2_UNFUSED>() &&
              terms_per_unit<Op::PTQ1_SRC>() == 1 && terms_per_unit<Op::PQ2_UNFUSED>() == 1, "split-K terms layout");
size_t splitk_scratch(const MatvecArgs &a) {
    const uint64_t rp = (a.rows + kTile - 1) / kTile * kTile, nu = a.cols / unit_weights<Op::PTQ1_SRC>();
    return a.tokens * nu * terms_per_unit<Op::PTQ1_SRC>() * rp * sizeof(float);
}

// PQ2 in the unfused order (Q8_K activations, one term per unit) takes it at two tokens from
// 5120 rows, where it otherwise runs token by token (prepared, us: 5120 x 17408 27.5 -> 19.4,
// 6144 x 16384 25.5 -> 20.1; the reference's case with f32 input 31.0 -> 23.1).  From three
// tokens its skinny kernel stays ahead with f32 input, whose quantizing launch split-K adds to
// (4096 x 14336, 4 tokens: 25.0 against 26.6; prepared 22.2 against 21.1).
static bool splitk_pq2(const MatvecArgs &a, uint64_t tiles, uint64_t nu) {
    return a.act_format == kActQ8K && !a.pinned && tiles < a.cus && nu >= 64 && a.tokens == 2 && a.rows >= 5120;
}

bool splitk_eligible(const MatvecArgs &a) {
    if ((a.kind != kPTQ1 && a.kind != kPQ2) || a.w2 || a.tile_best) return false;
    const uint64_t tiles = (a.rows + kTile - 1) / kTile, nu = a.cols / unit_weights<Op::PTQ1_SRC>();
    if (nu < kSplitKMinUnits || !fold_rows<Op::PTQ1_SRC>(static_cast<uint32_t>(nu))) return false;
    if (a.kind == kPQ2) return splitk_pq2(a, tiles, nu) && splitk_scratch(a) <= a.scratch_cap;
    if (a.act_format != kActQ8 || a.pinned) return false;
    const uint32_t n = a.tokens;
    const bool half = 2 * tiles <= a.cus;  // at most half a tile per CU
    bool take;
    if (n < 2 || n > 8 || tiles >= 2ull * a.cus)
        take = false;
    else if (tiles > a.cus)
        take = n <= 4;
    else if (n == 2 && nu >= 64)
        take = a.rows >= 5120;
    else if (nu >= 64)
        take = n <= 4 || half;
    else  // shorter rows: f32 input pays a separate quantizing launch here (6144 x 5120, 8 tokens, 21.2 -> 23.4)
        take = half && (n <= 3 || (n == 4 && nu >= 48));
    return take && splitk_scratch(a) <= a.scratch_cap;
}

template <Op O>
int launch_splitk(const MatvecArgs &a, uint32_t act_stride) {
    const uint32_t nu = static_cast<uint32_t>(a.cols / unit_weights<O>());
    const uint32_t rf = fold_rows<O>(nu);
    if (!rf || !a.scratch || a.scratch_bytes < splitk_scratch(a)) return -2;
    const uint32_t tiles = static_cast<uint32_t>((a.rows + kTile - 1) / kTile), rp = tiles * kTile;
    MvParams p{};
    p.w[0] = p.w[1] = a.w;
    p.rows = static_cast<uint32_t>(a.rows);
    p.nu = nu;
    p.cols = static_cast<uint32_t>(a.cols);
    p.out = a.out;
    p.residual = a.residual;
    p.err = a.err;
    float *terms = static_cast<float *>(a.scratch);
    const uint32_t chunks = (nu + kSplitKUnits - 1) / kSplitKUnits;
    hipLaunchKernelGGL(k_mv_terms<O>, dim3(tiles, chunks), dim3(64), 0, a.stream, p, a.act, act_stride, a.tokens,
                       kSplitKUnits, terms, rp);
    if (const int e = launch_status()) return e;
    const uint32_t lds = rf * nu * terms_per_unit<O>() * static_cast<uint32_t>(sizeof(float));
    hipLaunchKernelGGL(k_mv_fold<O>, dim3((p.rows + rf - 1) / rf, a.tokens), dim3(256), lds, a.stream, p, a.act,
                       act_stride, terms, rp, static_cast<uint32_t>(__builtin_ctz(rf)));
    return launch_status();
}

// Prepared activations of many tokens on the prefill GEMMs, from the token counts at which
// they beat the skinny kernel for f32 input: Q8_K blocks for Q2_K, PQ2, TQ1_0 and TQ2_0, Q8_0
// blocks for Q8_0 (int8 GEMM, prefill_k.hip) and PTQ1 in either order (f16 GEMM,
// prefill.hip).  Measured, 151936 x 4096, 16 tokens, us, skinny -> GEMM: Q2_K 79.6 -> 71.4,
// Q8_0 167.8 -> 136.4.  Not with a residual, and not when the caller's scratch cannot hold the
// token codes.
bool gemm_eligible(const MatvecArgs &a) {
    if (a.act_format == kActF32 || a.w2 || a.residual || a.tile_best || a.tokens < 2) return false;
    const bool fits = a.act_format == kActQ8K
                          ? a.kind == kQ2_K || a.kind == kPQ2 || a.kind == kTQ1_0 || a.kind == kTQ2_0
                          : a.kind == kQ8_0 || a.kind == kPTQ1;
    return fits && prefill_supported(a.kind, a.cols, a.rows, a.pinned, a.tokens) &&
           prefill_scratch_bytes(a.kind, a.cols, a.tokens) <= a.scratch_cap;
}

bool skinny_eligible(const MatvecArgs &a) {
    if (a.tokens < 2 || a.w2 || a.rows < kSkinnyMinRows || lut_batch_eligible(a) || quad_eligible(a) ||
        quad_split_eligible(a))
        return false;
    // Pinned PTQ1 (four masked MFMAs per group) and TQ1_0 / TQ2_0 (digits decoded for 16
    // rows per wavefront) on large matrices: up to four tokens the row-tile batch kernel is
    // faster (151936x4096 x 4: pinned PTQ1 148 against 165 us, TQ2_0 56.8 against 61.3, TQ1_0
    // 72.3 against 72.7; x 2: TQ2_0 40.6 against 60.9), from eight the skinny kernel (TQ1_0
    // 73.7 against 116; pinned PTQ1 x 16: 171 against 558).
    const bool pinned_q8 = a.kind == kPTQ1 && a.pinned && a.act_format != kActQ8K &&
                           !(a.act_format == kActF32 && a.qcontract_is_q8k);
    const bool tq = a.kind == kTQ1_0 || a.kind == kTQ2_0;
    if ((pinned_q8 || tq) && a.rows >= kBatchMinRows && a.tokens <= 4) return false;
    return dispatch(a, [&]<Op>() { return 1; }) == 1;  // a kind and contract of the tiled kernels
}

// Two PTQ1 / PQ2 tokens (three PTQ1 tokens from 12288 inputs) of rows of at least 6144 inputs on
// fewer than two tiles per CU run token by token on the single-token kernels, whose split
// spreads a long row over lane groups and wavefronts; the batch kernels leave most of their
// matrix-core width or table workgroup idle there.  Measured (us, f32 input with its
// quantization; batch kernel -> token by token): PTQ1 5120x17408 49.7 -> 34.5, 4096x14336
// 29.6 -> 19.1 (three tokens 30.4 -> 26.7), 5120x6144 21.5 -> 17.1; PQ2 4096x14336 25.9 ->
// 18.1, 5120x17408 37.0 -> 30.6.  Shorter rows lose (PTQ1 6144x5120 16.0 -> 16.4), and so do
// Q8_0 and Q2_K (4096x14336: 31.4 -> 32.9, 14.2 -> 17.1).
bool token_by_token(const MatvecArgs &a) {
    const uint64_t tiles = (a.rows + kTile - 1) / kTile;
    if (a.w2 || tiles >= 2ull * a.cus || a.cols < 6144 || (a.kind != kPTQ1 && a.kind != kPQ2)) return false;
    return a.tokens == 2 || (a.tokens == 3 && a.kind == kPTQ1 && a.cols >= 12288);
}

int launch_matvec_tiled(const MatvecArgs &a) {
    if (a.tile_best) {
        // Only the one-token row-tile path writes the tile maxima (launch_op).
        if (a.tokens != 1 || a.act_format == kActF32 || a.w2 || a.kind == kPTQ1) return -2;
        return dispatch(a, [&]<Op O>() { return launch_op<O>(a, a.act, a.out); });
    }
    const size_t in_stride = a.act_format == kActF32 ? sizeof(float) * a.cols
                             : a.act_format == kActQ8K ? sizeof(Q8KBlock) * ((a.cols + 255) / 256)
                                                       : sizeof(Q8Block) * (a.cols / 32);
    if (splitk_eligible(a))
        return a.kind == kPQ2 ? launch_splitk<Op::PQ2_UNFUSED>(a, static_cast<uint32_t>(in_stride))
                              : launch_splitk<Op::PTQ1_SRC>(a, static_cast<uint32_t>(in_stride));
    const bool batched = a.act_format != kActF32 && !token_by_token(a);
    if (batched && gemm_eligible(a)) {
        if (!a.scratch || a.scratch_bytes < prefill_scratch_bytes(a.kind, a.cols, a.tokens)) return -2;
        return launch_prefill_blocks(a.kind, a.w, a.cols, a.rows, a.act, static_cast<uint32_t>(in_stride), a.tokens,
                                     a.pinned, a.out, a.scratch, a.err, a.stream, a.cus);
    }
    if (batched && quad_eligible(a))
        return dispatch(a, [&]<Op O>() { return launch_quad<O>(a, static_cast<uint32_t>(in_stride)); });
    if (batched && quad_split_eligible(a)) return launch_quad_split(a, static_cast<uint32_t>(in_stride));
    if (batched && lut_batch_eligible(a))
        return dispatch(a, [&]<Op O>() { return launch_lut_batch<O>(a, static_cast<uint32_t>(in_stride)); });
    if (batched && skinny_eligible(a)) {
        for (uint32_t tok = 0; tok < a.tokens; tok += kSkChunks * kBatchMax) {
            const uint32_t n = a.tokens - tok < kSkChunks * kBatchMax ? a.tokens - tok : kSkChunks * kBatchMax;
            const void *act = static_cast<const uint8_t *>(a.act) + in_stride * tok;
            float *out = a.out + a.rows * tok;
            const float *res = a.residual ? a.residual + a.rows * tok : nullptr;
            const int rc = dispatch(a, [&]<Op O>() {
                return launch_skinny<O>(a, act, n, static_cast<uint32_t>(in_stride), out, res);
            });
            if (rc) return rc;
        }
        return 0;
    }
    if (batched && batch_eligible(a)) {
        for (uint32_t tok = 0; tok < a.tokens; tok += kBatchMax) {
            const uint32_t n = a.tokens - tok < kBatchMax ? a.tokens - tok : kBatchMax;
            const void *act = static_cast<const uint8_t *>(a.act) + in_stride * tok;
            float *out = a.out + a.rows * tok;
            const float *res = a.residual ? a.residual + a.rows * tok : nullptr;
            const int rc = dispatch(a, [&]<Op O>() {
                return launch_batch<O>(a, act, n, static_cast<uint32_t>(in_stride), out, res);
            });
            if (rc) return rc;
        }
        return 0;
    }
    for (uint32_t tok = 0; tok < a.tokens; ++tok) {
        const void *act = static_cast<const uint8_t *>(a.act) + in_stride * tok;
        float *out = a.out + a.rows * tok;
        MatvecArgs at = a;
        if (at.residual) at.residual += a.rows * tok;
        const int rc = dispatch(a, [&]<Op O>() { return launch_op<O>(at, act, out); });
        if (rc) return rc;
    }
    return 0;
}

size_t tiled_scratch_bytes(const MatvecArgs &a) {
    if (splitk_eligible(a)) return splitk_scratch(a);
    if (a.act_format != kActF32 && !token_by_token(a) && gemm_eligible(a))
        return prefill_scratch_bytes(a.kind, a.cols, a.tokens);
    if (!skinny_eligible(a)) return 0;
    return static_cast<size_t>(dispatch(a, [&]<Op O>() { return static_cast<int>(skinny_scratch<O>(a)); }));
}

bool tiled_prologue_fits(const MatvecArgs &a) {
    const bool f32 = a.act_format == kActF32;
    return f32 && dispatch(a, [&]<Op O>() {
               SplitPlan pl;
               return plan_split<O>(a.rows, static_cast<uint32_t>(a.cols / unit_weights<O>()),
                                    static_cast<uint32_t>(a.cols), true, a.w2 ? 2u : 1u, a.cus, &pl,
                                    a.q8_out ? 2u : 8u)
                          ? 1
                          : 0;
           }) == 1;
}

bool tiled_needs_prepared(const MatvecArgs &a) {
    if (quad_eligible(a) || quad_split_eligible(a) || lut_batch_eligible(a) || skinny_eligible(a) ||
        batch_eligible(a))
        return true;
    return dispatch(a, [&]<Op O>() { return op_needs_prepared<O>(a) ? 1 : 0; }) == 1;
}

}  // namespace prism
