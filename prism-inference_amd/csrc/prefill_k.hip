// prefill_k.hip -- tiled prefill GEMM for Q2_K, PQ2, TQ1_0 and TQ2_0 weights (Q8_K
// activations) and Q8_0 weights (Q8_0 activations) on the int8 matrix cores (gfx950).
//
// dot_q2_k_block (src/kernels/kquants.rs:162-197, row order :346-430), per 256-element
// unit u of a row and a token's Q8_K block:
//     isum = sum_g sc_g * dot_g        msum = sum_g mn_g * bsum_g       (exact integers)
//     Y    = Y + ((as * d) * isum - (as * dmin) * msum)                  (binary32, this order)
// with sc_g / mn_g the 4-bit scale and min of sub-block g, d / dmin the unit's binary16
// factors and as, bsum_g the token's scale and 16-element code sums.  Every term is the
// batch-1 expression (mv_tiled.hip), so each token row equals its own matvec bit for bit.
//
// The integers come from the matrix cores, exactly:
// - isum from eight v_mfma_i32_32x32x32_i8 per unit: the weight operand carries sc_g * q
//   (q in 0..3, so at most 45: still a signed byte) and the token operand the codes, so the
//   i32 sum over the unit's 256 elements is sum_g sc_g * dot_g.  Which 32 elements a K-step
//   holds is free (an integer dot is exact in any order), as long as a lane's weight and
//   token bytes pair the same elements; the order below is the one the 2-bit codes decode
//   into most cheaply.
// - msum from one v_mfma_f32_32x32x16_f16 with K = the 16 sub-blocks: mn_g <= 15 and
//   |bsum_g| <= 16 * 127 = 2032 are exact in binary16, and every partial sum (at most
//   16 * 15 * 2032 < 2^24) is exact in the f32 accumulator.
// - as * d and as * dmin from v_mfma_f32_32x32x2_f32 outer products (K = 2, the second term
//   zero): one rounding each, the product itself, straight into the output layout.
// Per (token, row, unit) the VALU then runs the conversion of isum and the four binary32
// operations of the expression.
//
// dot_pq2<FUSED> (src/kernels.rs:941-955), per 128-element block b of a row (the token's
// Q8_K block b / 2 holds its codes): d = fl(ws_b * as), s = float(sum (c - 1) * a) and
// Y = fma(d, s, Y) (fused, the pinned contract) or Y + fl(d * s).  The block's integer
// dot is four v_mfma_i32_32x32x32_i8 on the signed codes c - 1, d one outer product.
//
// dot_legacy (src/kernels.rs:1204-1248), per 32-element block b of a Q8_0 row and the
// token's Q8_0 block b: Y = Y + fl(fl(ws_b * as_b) * float(I_b)), I_b one K-step on the codes
// as they are (no decode), the scale product one outer product.
//
// TQ1_0 / TQ2_0 dot (src/kernels/tquants.rs:255-285), per 256-element unit and the token's
// Q8_K block: Y = Y + float(I) * fl(d * as), I = sum (t - 1) * a over the unit (eight K-steps
// on the signed codes), fl(d * as) one outer product.
//
// Work split: a workgroup of four wavefronts owns 128 weight rows (two 64-row tiles) and
// NT = 32 * CT tokens, and walks the rows' 256-element units (one Q8_K block each; two
// PQ2 blocks).  Wavefront w owns 32 rows and decodes them itself into the int8 operand
// registers: lane l supplies row l % 32 and, in half h = l / 32, bytes 8h..8h+7 of each of
// the unit's 16-byte code pieces.  The tokens' codes, prepared once per call
// in exactly that order, stream unit by unit into a double-buffered LDS ring with
// direct-to-LDS buffer loads, with the tokens' scales and sub-block sums beside them; one
// barrier per unit hands a buffer from the loads to the readers and back.
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"
#include "quant_dev.hpp"
#include "tiled.hpp"

namespace prism {

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr uint32_t kRowsPerWg = 128, kTokAlign = 128, kUnit = 256;

// Operand orders.  K-step s (0..7) of a 256-element unit, half h of the wavefront (lanes
// 32h..32h+31), operand dword i (0..3) -- four bytes, four elements:
// Q2_K: code piece p (bytes 16 + 16p .. 31 + 16p of the native block, tiled piece p) byte j
// holds, in bits 2*part, the code of element 16g + j with g = 8 * (p / 2) + 2 * part + p % 2
// (dot_q2_k_block's half / part / sub loops).  K-step s takes piece p = s / 2 and parts
// 2 * (s % 2) + {0, 1}; dword i is bytes 8h + 4 * (i % 2) .. +3 of the piece at part
// 2 * (s % 2) + i / 2: the four consecutive elements starting at
__host__ __device__ constexpr uint32_t q2k_elem(uint32_t s, uint32_t h, uint32_t i) {
    const uint32_t p = s >> 1, part = 2 * (s & 1) + (i >> 1);
    return 16 * (8 * (p >> 1) + 2 * part + (p & 1)) + 8 * h + 4 * (i & 1);
}
// PQ2 (block b = s / 4 of the unit's two 128-element blocks): code dword c of a block holds
// element 16c + 4q + f in byte q, bits 2f (pq2_code).  K-step s takes code dword
// c = 4 * ((s / 2) % 2) + 2h + s % 2 (piece (s / 2) % 2, bytes 8h + 4 * (s % 2)), and
// operand dword i its field f = i: elements e, e + 4, e + 8, e + 12 with e =
__host__ __device__ constexpr uint32_t pq2_elem(uint32_t s, uint32_t h, uint32_t i) {
    return 128 * (s >> 2) + 16 * (4 * ((s >> 1) & 1) + 2 * h + (s & 1)) + i;
}
// Q8_0: K-step s is the 32-element block s of the unit, half h its codes 16h .. 16h+15 (tiled
// code piece 2 * (s % 4) + h of tiled unit 2u + s / 4), in their own order: no decode.
// TQ2_0: bits 2k of code byte 32q + b hold element 128q + 32k + b (dot_tq2_block).  K-step s
// takes piece p = s / 2 (bytes 16p .. 16p+15) and fields k = 2 * (s % 2) + {0, 1}; dword i is
// bytes 8h + 4 * (i % 2) .. +3 of the piece at field 2 * (s % 2) + i / 2: the four
// consecutive elements starting at
__host__ __device__ constexpr uint32_t tq2_elem(uint32_t s, uint32_t h, uint32_t i) {
    const uint32_t p = s >> 1, k = 2 * (s & 1) + (i >> 1);
    return 128 * (p >> 1) + 32 * k + 16 * (p & 1) + 8 * h + 4 * (i & 1);
}
// TQ1_0: base-3 digit k of code byte b holds element b + 32k (b < 32, k < 5), 160 + (b - 32)
// + 16k (32 <= b < 48) or 240 + (b - 48) + 4k (48 <= b < 52, k < 4) (dot_tq1_block).  Half h
// takes bytes 8h .. 8h+7 of the three 16-byte pieces (six code dwords of five digits) and bytes
// 2h, 2h+1 of the 4-byte piece (four digits each).  Operand dword n = 4s + i (0..31) is digit
// n % 5 of code dword c = n / 5 (piece c / 2, bytes 8h + 4 * (c % 2) .. +3) for n < 30, and
// for n = 30 + m digits 2m, 2m + 1 of the two short-piece bytes.  Byte j of it holds element
__host__ __device__ constexpr uint32_t tq1_elem(uint32_t s, uint32_t h, uint32_t i, uint32_t j) {
    const uint32_t n = 4 * s + i;
    if (n >= 30) return 240 + 2 * h + (j & 1) + 4 * (2 * (n - 30) + (j >> 1));
    const uint32_t c = n / 5, k = n % 5, p = c >> 1, b = 8 * h + 4 * (c & 1) + j;
    return p < 2 ? 16 * p + b + 32 * k : 160 + b + 16 * k;
}

// Each order names every element of the unit exactly once over its 256 byte slots (eight
// K-steps, two halves, four dwords of four bytes), byte j of an operand dword at elem(s, h, i, j).
template <typename F>
constexpr bool names_every_element_once(F elem) {
    bool seen[256] = {};
    for (uint32_t s = 0; s < 8; ++s)
        for (uint32_t h = 0; h < 2; ++h)
            for (uint32_t i = 0; i < 4; ++i)
                for (uint32_t j = 0; j < 4; ++j) {
                    const uint32_t e = elem(s, h, i, j);
                    if (e >= 256 || seen[e]) return false;
                    seen[e] = true;
                }
    return true;
}
static_assert(names_every_element_once([](uint32_t s, uint32_t h, uint32_t i, uint32_t j) {
    return q2k_elem(s, h, i) + j;
}));
static_assert(names_every_element_once([](uint32_t s, uint32_t h, uint32_t i, uint32_t j) {
    return pq2_elem(s, h, i) + 4 * j;
}));
static_assert(names_every_element_once([](uint32_t s, uint32_t h, uint32_t i, uint32_t j) {
    return tq2_elem(s, h, i) + j;
}));
static_assert(names_every_element_once(tq1_elem));

// ---- activation prep ------------------------------------------------------------------
// A workgroup of TOK wavefronts quantizes TOK consecutive tokens (one each, 1024 inputs =
// four Q8_K blocks, pinned selecting pinned_q8k_integer's rounding; for Q8_0 weights 32 Q8_0
// blocks in the source or pinned generic contract), or with BLOCKS copies the tokens' prepared
// blocks of those inputs (src_stride bytes per token), then writes, per 256-element unit u and
// token t (tokens padded to Mp with zeros):
//   xq[u][s][h][t][16 bytes]   codes in the kind's operand order (16 slots of 16 bytes),
//   as[u][t]                   the Q8_K block scale (Q8_0: as[u][s][t], the 8 block scales),
//   bs[u][h][t][8 x f16]       Q2_K only: the sums of sub-blocks 8h .. 8h+7,
// consecutive threads taking consecutive tokens of one slot, so each slot's TOK tokens
// leave as one contiguous run.  A quantizer error is raised and the wavefront carries on.
template <uint32_t KIND, uint32_t TOK, bool BLOCKS>
__global__ __launch_bounds__(64 * TOK) void k_prefill_k_prep(const void *__restrict__ src, uint32_t src_stride,
                                                             uint32_t M, uint32_t Mp, uint32_t K, int pinned,
                                                             uint8_t *__restrict__ xq, float *__restrict__ as,
                                                             _Float16 *__restrict__ bs, int *__restrict__ err) {
    constexpr bool kQ8 = KIND == kQ8_0;
    using Blk = typename std::conditional<kQ8, Q8Block[TOK][32], Q8KBlock[TOK][4]>::type;
    __shared__ Blk blk;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t chunks = (K + 1023) / 1024;
    const uint32_t c = blockIdx.x % chunks, tb = blockIdx.x / chunks * TOK;
    const uint32_t k0 = c * 1024, nb = (K - k0 < 1024 ? K - k0 : 1024) / kUnit;  // 1..4 units
    const uint32_t t = tb + wave;
    if (t < M) {
        if constexpr (BLOCKS) {
            constexpr uint32_t kUnitBytes = kQ8 ? 8 * sizeof(Q8Block) : sizeof(Q8KBlock);  // per 256 inputs
            const uint32_t *from = reinterpret_cast<const uint32_t *>(
                static_cast<const uint8_t *>(src) + static_cast<size_t>(t) * src_stride + (k0 / kUnit) * kUnitBytes);
            uint32_t *to = reinterpret_cast<uint32_t *>(&blk[wave]);
            for (uint32_t i = lane; i < nb * kUnitBytes / 4; i += 64) to[i] = from[i];
        } else {
            const float *x = static_cast<const float *>(src) + static_cast<size_t>(t) * K + k0;
            int e;
            if constexpr (kQ8)  // the source (0) or pinned generic (1) contract, 32-element blocks
                e = q8_0_blocks_wave(x, nb * 8, pinned ? 1 : 0, blk[wave], lane);
            else
                e = q8k_blocks_wave(x, nb, pinned, blk[wave], lane);
            if (e && lane == 0) raise_error(err, e);
        }
    }
    __syncthreads();
    const uint32_t u0 = k0 / kUnit;
    for (uint32_t i = tid; i < nb * 16 * TOK; i += 64 * TOK) {
        const uint32_t w = i % TOK, q = (i / TOK) % 16, ub = i / (16 * TOK);
        const uint32_t s = q >> 1, h = q & 1u;
        uint32_t v[4] = {0, 0, 0, 0};
        if (tb + w < M) {
            const uint8_t *vals = kQ8 ? reinterpret_cast<const uint8_t *>(blk[w][8 * ub + s].values) + 16 * h
                                      : reinterpret_cast<const uint8_t *>(blk[w][ub].values);
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                if constexpr (kQ8) {
                    v[j] = *reinterpret_cast<const uint32_t *>(vals + 4 * j);
                } else if constexpr (KIND == kQ2_K) {
                    v[j] = *reinterpret_cast<const uint32_t *>(vals + q2k_elem(s, h, j));
                } else if constexpr (KIND == kTQ2_0) {
                    v[j] = *reinterpret_cast<const uint32_t *>(vals + tq2_elem(s, h, j));
                } else if constexpr (KIND == kTQ1_0) {
#pragma unroll
                    for (uint32_t b = 0; b < 4; ++b) v[j] |= static_cast<uint32_t>(vals[tq1_elem(s, h, j, b)]) << (8 * b);
                } else {
                    const uint8_t *e = vals + pq2_elem(s, h, j);  // elements e, e+4, e+8, e+12
                    v[j] = static_cast<uint32_t>(e[0]) | static_cast<uint32_t>(e[4]) << 8 |
                           static_cast<uint32_t>(e[8]) << 16 | static_cast<uint32_t>(e[12]) << 24;
                }
            }
        }
        *reinterpret_cast<uint4 *>(xq + ((static_cast<size_t>(u0 + ub) * 16 + q) * Mp + tb + w) * 16) =
            make_uint4(v[0], v[1], v[2], v[3]);
    }
    if constexpr (KIND == kQ2_K) {
        for (uint32_t i = tid; i < nb * 2 * TOK; i += 64 * TOK) {
            const uint32_t w = i % TOK, h = (i / TOK) % 2, ub = i / (2 * TOK);
            const bool real = tb + w < M;
            uint32_t p[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int16_t s0 = real ? blk[w][ub].sums[8 * h + 2 * k] : 0;
                const int16_t s1 = real ? blk[w][ub].sums[8 * h + 2 * k + 1] : 0;
                p[k] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(s0))) |
                       static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(s1))) << 16;
            }
            *reinterpret_cast<uint4 *>(bs + ((static_cast<size_t>(u0 + ub) * 2 + h) * Mp + tb + w) * 8) =
                make_uint4(p[0], p[1], p[2], p[3]);
        }
    }
    if constexpr (kQ8) {
        for (uint32_t i = tid; i < nb * 8 * TOK; i += 64 * TOK) {  // as[u][s][t]: the 8 block scales
            const uint32_t w = i % TOK, b = i / TOK;
            as[(static_cast<size_t>(u0) * 8 + b) * Mp + tb + w] = tb + w < M ? blk[w][b].scale : 0.0f;
        }
    } else if (tid < nb * TOK) {
        const uint32_t w = tid % TOK, ub = tid / TOK;
        as[static_cast<size_t>(u0 + ub) * Mp + tb + w] = tb + w < M ? blk[w][ub].scale : 0.0f;
    }
}

// ---- the GEMM --------------------------------------------------------------------------
// One lane's raw weights of a 256-element unit.  Q2_K: bytes 8h..8h+7 of the four code
// pieces of its row, the sub-block scale piece and (d, dmin).  PQ2: bytes 8h..8h+7 of both
// code pieces of each of the unit's two 128-element blocks, and their binary16 scales.
template <uint32_t KIND>
struct RawK;
template <>
struct RawK<kQ2_K> {
    u32x2 c[4];
    u32x4 sc;
    uint32_t dm;
};
template <>
struct RawK<kPQ2> {
    u32x2 c[2][2];
    uint32_t d[2];
};
template <>
struct RawK<kQ8_0> {
    u32x4 c[8];    // codes 16h .. 16h+15 of the unit's eight blocks
    u32x2 sc[2];   // the eight binary16 block scales
};
template <>
struct RawK<kTQ2_0> {
    u32x2 c[4];  // bytes 8h .. 8h+7 of the four code pieces
    uint32_t d;  // binary16 scale
};
template <>
struct RawK<kTQ1_0> {
    u32x2 c[3];     // bytes 8h .. 8h+7 of the three 16-byte code pieces
    uint32_t tail;  // the 4-byte code piece (code bytes 48 .. 51)
    uint32_t d;
};
// Bytes per row of a tiled 256-element unit: the native block.
template <uint32_t KIND>
constexpr uint32_t unit_bytes_k() {
    return KIND == kQ2_K ? 84 : KIND == kQ8_0 ? 272 : KIND == kPQ2 ? 68 : KIND == kTQ2_0 ? 66 : 54;
}
template <uint32_t KIND>
__device__ __forceinline__ void load_unit_k(__amdgpu_buffer_rsrc_t rs, uint32_t u, uint32_t trp, uint32_t row,
                                            uint32_t h, RawK<KIND> &w) {
    if constexpr (KIND == kQ2_K) {
        const uint32_t seg = u * trp * 84u;
#pragma unroll
        for (uint32_t p = 0; p < 4; ++p) w.c[p] = bload2(rs, seg + 16u * p * trp + 16u * row + 8u * h);
        w.sc = bload4(rs, seg + 64u * trp + 16u * row);
        w.dm = bload1(rs, seg + 80u * trp + 4u * row);
    } else if constexpr (KIND == kQ8_0) {
#pragma unroll
        for (uint32_t b = 0; b < 2; ++b) {
            const uint32_t seg = (2 * u + b) * trp * 136u;
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) w.c[4 * b + j] = bload4(rs, seg + 16u * (2 * j + h) * trp + 16u * row);
            w.sc[b] = bload2(rs, seg + 128u * trp + 8u * row);
        }
    } else if constexpr (KIND == kTQ2_0 || KIND == kTQ1_0) {
        constexpr uint32_t P = KIND == kTQ2_0 ? 4 : 3, kScale = KIND == kTQ2_0 ? 64 : 52;
        const uint32_t seg = u * trp * unit_bytes_k<KIND>();
#pragma unroll
        for (uint32_t p = 0; p < P; ++p) w.c[p] = bload2(rs, seg + 16u * p * trp + 16u * row + 8u * h);
        if constexpr (KIND == kTQ1_0) w.tail = bload1(rs, seg + 48u * trp + 4u * row);
        w.d = __builtin_amdgcn_raw_buffer_load_b16(rs, static_cast<int>(seg + kScale * trp + 2u * row), 0, 0);
    } else {
#pragma unroll
        for (uint32_t b = 0; b < 2; ++b) {
            const uint32_t seg = (2 * u + b) * trp * 34u;
            w.c[b][0] = bload2(rs, seg + 16u * row + 8u * h);
            w.c[b][1] = bload2(rs, seg + 16u * trp + 16u * row + 8u * h);
            w.d[b] = __builtin_amdgcn_raw_buffer_load_b16(rs, static_cast<int>(seg + 32u * trp + 2u * row), 0, 0);
        }
    }
}

__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0F70); }
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// Workgroup barrier for LDS hand-offs: this wavefront's LDS traffic is complete, but global
// loads still in flight are not waited for, as __syncthreads() (a fence) would.
__device__ __forceinline__ void lds_barrier() {
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
}

// FUSED (PQ2 only): dot_pq2<true>'s fma(d, s, o) instead of o + d * s.
template <uint32_t KIND, int CT, bool FUSED>
__global__ __launch_bounds__(256) void k_prefill_kq(const uint8_t *__restrict__ W, uint32_t rows, uint32_t nu,
                                                    const uint8_t *__restrict__ xq, const float *__restrict__ as,
                                                    const _Float16 *__restrict__ bs, uint32_t M, uint32_t Mp,
                                                    uint32_t xcd_major, float *__restrict__ out,
                                                    int *__restrict__ err) {
    constexpr uint32_t NT = 32 * CT;
    constexpr bool kQ2 = KIND == kQ2_K, kQ8 = KIND == kQ8_0, kTQ = KIND == kTQ1_0 || KIND == kTQ2_0;
    constexpr uint32_t kSums = kQ2 ? 2 : 0;  // Q2_K: two runs of sub-block sums per unit
    constexpr uint32_t kScl = kQ8 ? 8 : 1;   // scale runs per unit (Q8_0: one per block)
    // Ring buffers (separate objects, named statically below, so the compiler can tell a
    // read of one from the direct-to-LDS loads in flight into the other): the codes
    // [s][h][token][16 bytes] (each half-wavefront's read covers 512 contiguous bytes),
    // the Q2_K sub-block sums [h][token][16 bytes] and the scales [token].
    __shared__ __attribute__((aligned(16))) uint8_t act0[8][2][NT * 16];
    __shared__ __attribute__((aligned(16))) uint8_t act1[8][2][NT * 16];
    __shared__ __attribute__((aligned(16))) uint8_t bsm0[kQ2 ? 2 : 1][kQ2 ? NT * 16 : 16];
    __shared__ __attribute__((aligned(16))) uint8_t bsm1[kQ2 ? 2 : 1][kQ2 ? NT * 16 : 16];
    __shared__ __attribute__((aligned(16))) float scl0[kScl][NT];
    __shared__ __attribute__((aligned(16))) float scl1[kScl][NT];
    using Bsm = uint8_t[kQ2 ? 2 : 1][kQ2 ? NT * 16 : 16];
    using Scl = float[kScl][NT];
    const uint32_t lane = threadIdx.x & 63, r32 = lane & 31, h = lane >> 5;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Workgroups go to the eight XCDs round-robin in dispatch order (x fastest), each with
    // its own L2.  With a multiple of eight token groups the grid is (8, row blocks, token
    // groups / 8): XCD x takes token groups x, x+8, ... and every row block of each, so a
    // token group's codes are read into one L2 only and the weights are shared there.
    const uint32_t bx = xcd_major ? blockIdx.y : blockIdx.x;
    const uint32_t by = xcd_major ? blockIdx.x + 8 * blockIdx.z : blockIdx.y;
    const uint32_t tile = 2 * bx + (wave >> 1), hw = wave & 1;
    const uint32_t tiles = (rows + kTile - 1) / kTile;
    const uint32_t t0 = by * NT;
    const uint32_t row_bytes = nu * unit_bytes_k<KIND>();
    uint32_t trows = 0;
    if (tile < tiles) {
        const uint32_t left = rows - tile * kTile;
        trows = left < kTile ? left : kTile;
    }
    const bool active = 32 * hw < trows;  // uniform per wavefront
    const uint32_t trp = (trows + 7u) & ~7u;
    const __amdgpu_buffer_rsrc_t rw =
        make_rsrc(W + static_cast<size_t>(active ? tile : 0) * kTile * row_bytes, active ? trp * row_bytes : 0u);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xq, nu * 256u * Mp);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(bs, kQ2 ? nu * 32u * Mp : 0u);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(as, nu * 4u * kScl * Mp);
    const uint32_t row = 32 * hw + r32, out0 = 32 * hw + 4 * h;  // tile rows

    // Unit u's token data -> LDS: 16 code runs (and Q2_K's 2 sum runs) of NT * 16 bytes and
    // NT scales, each contiguous in the prepared arrays; one wavefront instruction moves 64
    // tokens' 16 bytes (lanes past a short run idle).
    auto stage = [&](uint32_t u, uint8_t (&act)[8][2][NT * 16], Bsm &bsm, Scl &scl) {
        constexpr uint32_t per = (NT + 63) / 64;  // instructions per run
#pragma unroll
        for (uint32_t k = wave; k < (16 + kSums) * per; k += 4) {
            const uint32_t run = k / per, c = k % per;
            if (64 * c + lane < NT) {
                if (run < 16) {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void *)(&act[run >> 1][run & 1][1024 * c]), 16,
                                                             ((u * 16 + run) * Mp + t0 + 64 * c + lane) * 16u, 0, 0, 0);
                } else if constexpr (kQ2) {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void *)(&bsm[run - 16][1024 * c]), 16,
                                                             ((u * 2 + run - 16) * Mp + t0 + 64 * c + lane) * 16u, 0, 0,
                                                             0);
                }
            }
        }
        // Scale run r by wavefront 3 - r % 4.
#pragma unroll
        for (uint32_t r = 0; r < kScl; ++r) {
            if (wave != 3 - r % 4) continue;
#pragma unroll
            for (uint32_t c = 0; c < per; ++c)
                if (64 * c + lane < NT)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)(&scl[r][64 * c]), 4,
                                                             ((u * kScl + r) * Mp + t0 + 64 * c + lane) * 4u, 0, 0, 0);
        }
    };

    v16f o[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[ct][r] = 0.0f;

    RawK<KIND> w;
    stage(0, act0, bsm0, scl0);
    if (active) load_unit_k<KIND>(rw, 0, trp, row, h, w);
    wait_vmcnt0();
    lds_barrier();
    auto unit = [&](uint32_t u, const uint8_t (&act)[8][2][NT * 16], const Bsm &bsm, const Scl &scl,
                    uint8_t (&act_n)[8][2][NT * 16], Bsm &bsm_n, Scl &scl_n) {
        u32x4 aw[8];  // the weight operand of each K-step
        v8h mn;       // Q2_K: min_g of sub-blocks 8h .. 8h+7
        float d0 = 0.0f, d1 = 0.0f;  // Q2_K: d, dmin; PQ2: the two blocks' scales (half 0; zero in half 1)
        u32x2 wsc[2];                // Q8_0: the eight block scales
        if (active) {
            if constexpr (kQ2) {
                uint32_t m[16];  // sc_g in both 16-bit lanes
#pragma unroll
                for (int g = 0; g < 16; ++g) m[g] = ((w.sc[g >> 2] >> (8 * (g & 3))) & 15u) * 0x00010001u;
#pragma unroll
                for (uint32_t s = 0; s < 8; ++s) {
                    const uint32_t p = s >> 1;
#pragma unroll
                    for (uint32_t i = 0; i < 4; ++i) {
                        const uint32_t part = 2 * (s & 1) + (i >> 1), g = 8 * (p >> 1) + 2 * part + (p & 1);
                        const uint32_t q = (w.c[p][i & 1] >> (2 * part)) & 0x03030303u;
                        aw[s][i] =
                            __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, m[g]));
                    }
                }
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    mn[k] = static_cast<_Float16>(static_cast<float>((w.sc[2 * h + (k >> 2)] >> (8 * (k & 3) + 4)) & 15u));
                d0 = h ? 0.0f : h2f(w.dm & 0xffffu);
                d1 = h ? 0.0f : h2f(w.dm >> 16);
            } else if constexpr (kQ8) {
#pragma unroll
                for (uint32_t s = 0; s < 8; ++s) aw[s] = w.c[s];
                wsc[0] = w.sc[0];
                wsc[1] = w.sc[1];
            } else if constexpr (KIND == kTQ2_0) {
                // Fields c (0..3) -> signed bytes c - 1, as for PQ2.
#pragma unroll
                for (uint32_t s = 0; s < 8; ++s)
#pragma unroll
                    for (uint32_t i = 0; i < 4; ++i) {
                        const uint32_t k = 2 * (s & 1) + (i >> 1);
                        aw[s][i] = (((w.c[s >> 1][i & 1] >> (2 * k)) & 0x03030303u) + 0x7f7f7f7fu) ^ 0x80808080u;
                    }
                d0 = h ? 0.0f : h2f(w.d & 0xffffu);
            } else if constexpr (KIND == kTQ1_0) {
                // Base-3 digits of four code bytes at a time: with a byte y in each 16-bit lane,
                // y * 3 carries the next digit into the lane's high byte and leaves the rest of
                // the base-3 fraction (y * 3 mod 256) in its low byte.  The digits d (0..2)
                // then select d - 1 as a signed byte from {0xff, 0x00, 0x01}.
                uint32_t op[32];
                auto digits = [&](uint32_t x, int nd, uint32_t *dst) {
                    uint32_t L = x & 0x00ff00ffu, H = (x >> 8) & 0x00ff00ffu;
#pragma unroll
                    for (int k = 0; k < nd; ++k) {
                        const uint32_t mL = L * 3u, mH = H * 3u;  // no carry out of a lane: 255 * 3 < 2^16
                        dst[k] = perm(0u, 0x000100ffu, perm(mH, mL, 0x07030501u));  // high bytes, in byte order
                        L = mL & 0x00ff00ffu;
                        H = mH & 0x00ff00ffu;
                    }
                };
#pragma unroll
                for (uint32_t c = 0; c < 6; ++c) digits(w.c[c >> 1][c & 1], 5, op + 5 * c);
                uint32_t t4[4];
                digits(w.tail, 4, t4);
                const uint32_t pick = h ? 0x07060302u : 0x05040100u;  // bytes 2h, 2h+1 of two digit dwords
                op[30] = perm(t4[1], t4[0], pick);
                op[31] = perm(t4[3], t4[2], pick);
#pragma unroll
                for (uint32_t n = 0; n < 32; ++n) aw[n >> 2][n & 3] = op[n];
                d0 = h ? 0.0f : h2f(w.d & 0xffffu);
            } else {
                // Codes 0..2 -> signed bytes c - 1: +0x7f per byte (no carry out of a byte),
                // then the sign bit flipped.
#pragma unroll
                for (uint32_t s = 0; s < 8; ++s) {
                    const uint32_t cd = w.c[s >> 2][(s >> 1) & 1][s & 1];
#pragma unroll
                    for (uint32_t j = 0; j < 4; ++j)
                        aw[s][j] = (((cd >> (2 * j)) & 0x03030303u) + 0x7f7f7f7fu) ^ 0x80808080u;
                }
                d0 = h ? 0.0f : h2f(w.d[0] & 0xffffu);
                d1 = h ? 0.0f : h2f(w.d[1] & 0xffffu);
            }
        }
        // The next unit streams in while this one is multiplied.
        if (u + 1 < nu) {
            stage(u + 1, act_n, bsm_n, scl_n);
            if (active) load_unit_k<KIND>(rw, u + 1, trp, row, h, w);
        }
        if (active) {
            auto kstep = [&](int s, int ct, v16i acc) {
                const u32x4 bx = *reinterpret_cast<const u32x4 *>(&act[s][h][(32 * ct + r32) * 16]);
                return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i, aw[s]), __builtin_bit_cast(v4i, bx),
                                                             acc, 0, 0, 0);
            };
            if constexpr (kQ2 || kTQ) {
                // isum: each token group's chain of eight K-steps; the chains run side by side
                // (a dependent MFMA waits for its predecessor's result), and a single token
                // group splits its chain into even and odd K-steps, added at the end (exact).
                v16i is[CT];
                if constexpr (CT == 1) {
                    v16i odd = {};
                    is[0] = v16i{};
#pragma unroll
                    for (int s = 0; s < 8; s += 2) {
                        is[0] = kstep(s, 0, is[0]);
                        odd = kstep(s + 1, 0, odd);
                    }
                    is[0] += odd;
                } else {
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) is[ct] = v16i{};
#pragma unroll
                    for (int s = 0; s < 8; ++s)
#pragma unroll
                        for (int ct = 0; ct < CT; ++ct) is[ct] = kstep(s, ct, is[ct]);
                }
                if constexpr (kTQ) {
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) {
                        const float a = h ? 0.0f : scl[0][32 * ct + r32];
                        const v16f dd = __builtin_amdgcn_mfma_f32_32x32x2f32(d0, a, v16f{}, 0, 0, 0);  // fl(d * as)
#pragma unroll
                        for (int r = 0; r < 16; ++r) o[ct][r] = o[ct][r] + static_cast<float>(is[ct][r]) * dd[r];
                    }
                } else {
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) {
                        const uint32_t tok = 32 * ct + r32;
                        const float a = h ? 0.0f : scl[0][tok];
                        const v16f f1 = __builtin_amdgcn_mfma_f32_32x32x2f32(d0, a, v16f{}, 0, 0, 0);  // fl(as * d)
                        const v16f f2 = __builtin_amdgcn_mfma_f32_32x32x2f32(d1, a, v16f{}, 0, 0, 0);  // fl(as * dmin)
                        const v8h bsum = *reinterpret_cast<const v8h *>(&bsm[h][tok * 16]);
                        const v16f ms = __builtin_amdgcn_mfma_f32_32x32x16_f16(mn, bsum, v16f{}, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            o[ct][r] = o[ct][r] + (f1[r] * static_cast<float>(is[ct][r]) - f2[r] * ms[r]);
                    }
                }
            } else if constexpr (kQ8) {
                // dot_legacy's chain, block by block: Y = Y + fl(fl(ws_s * as_s) * float(I_s)),
                // I_s one K-step.
#pragma unroll
                for (int s = 0; s < 8; ++s) {
                    const float ws = h ? 0.0f : h2f((wsc[s >> 2][(s >> 1) & 1] >> (16 * (s & 1))) & 0xffffu);
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) {
                        // Read by every lane: a branch around the read (lanes of half 1 need
                        // none) lets the compiler sink the chain below all eight blocks' MFMAs,
                        // whose results then fill the registers.
                        const float sa = scl[s][32 * ct + r32];
                        const float a = h ? 0.0f : sa;
                        const v16f dd = __builtin_amdgcn_mfma_f32_32x32x2f32(ws, a, v16f{}, 0, 0, 0);
                        const v16i is = kstep(s, ct, v16i{});
#pragma unroll
                        for (int r = 0; r < 16; ++r) o[ct][r] = o[ct][r] + dd[r] * static_cast<float>(is[r]);
                    }
                    // One block's products at a time (measured: 2048 tokens 158.8 against 166.4 us
                    // with the scheduler free to issue later blocks' MFMAs early).
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
                // Per 128-element block b (K-steps 4b .. 4b+3): I_b and fl(ws_b * as).
                v16i ib[CT][2];
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) ib[ct][0] = ib[ct][1] = v16i{};
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct) {
                        ib[ct][0] = kstep(s, ct, ib[ct][0]);
                        ib[ct][1] = kstep(4 + s, ct, ib[ct][1]);
                    }
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    const float a = h ? 0.0f : scl[0][32 * ct + r32];
#pragma unroll
                    for (int b = 0; b < 2; ++b) {
                        const v16f dd = __builtin_amdgcn_mfma_f32_32x32x2f32(b ? d1 : d0, a, v16f{}, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const float sv = static_cast<float>(ib[ct][b][r]);
                            o[ct][r] = FUSED ? __builtin_fmaf(dd[r], sv, o[ct][r]) : o[ct][r] + dd[r] * sv;
                        }
                    }
                }
            }
        }
        wait_vmcnt0();  // unit u+1's token data and weights have landed
        lds_barrier();  // and every wavefront is done with unit u's buffers
    };
    for (uint32_t u = 0; u < nu; u += 2) {
        unit(u, act0, bsm0, scl0, act1, bsm1, scl1);
        if (u + 1 < nu) unit(u + 1, act1, bsm1, scl1, act0, bsm0, scl0);
    }
    if (!active) return;
    // Y[t][r]: the lane holds tokens t0 + 32ct + r32 and tile rows out0 + 8q + 0..3.
    bool bad = false;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        const uint32_t t = t0 + 32 * ct + r32;
        if (t >= M) continue;
        float *yr = out + static_cast<size_t>(t) * rows + static_cast<size_t>(tile) * kTile;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t r = out0 + 8 * q + e;
                if (r < trows) {
                    const float v = o[ct][4 * q + e];
                    yr[r] = v;
                    bad |= !finite(v);
                }
            }
        }
    }
    if (bad) raise_error(err, kErrNonfinite);
}

uint32_t padded_tokens(uint32_t M) { return (M + kTokAlign - 1) / kTokAlign * kTokAlign; }

// Scratch layout: codes | scales | sums, each 256-byte aligned.
size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

}  // namespace

size_t prefill_k_scratch_bytes(uint64_t cols, uint32_t tokens) {
    const size_t Mp = padded_tokens(tokens), nu = cols / kUnit;
    return align256(Mp * cols) + align256(nu * Mp * 4 * 8) + nu * Mp * 32;
}

// Tokens from which the GEMM takes over from the skinny kernel, which runs up to four
// 16-token chunks side by side per launch.  Measured (f32 input with its quantization, us,
// skinny / GEMM):
// - below 8192 rows the skinny kernel stays ahead to 64 tokens (6144 x 2048, 48 tokens: Q2_K
//   10.8 / 17.6, PQ2 14.1 / 15.6, Q8_0 16.8 / 23.7, TQ2_0 10.2 / 14.4; 64 tokens: Q2_K 12.1 /
//   17.3);
// - below 16384 rows to 48 tokens (12288 x 4096, 48 tokens: Q2_K 27.1 / 28.2, PQ2 26.1 /
//   24.0; 64 tokens: Q2_K 33.7 / 27.3, Q8_0 52.7 / 41.3);
// - from 16384 rows the GEMM wins from 17 tokens (17 / 32 tokens: Q2_K 32768 x 4096 38.4 /
//   26.9 and 38.3 / 28.3, PQ2 17408 x 5120 30.6 / 26.8 and 30.7 / 28.4, TQ2_0 17408 x 5120
//   26.5 / 23.6; Q8_0 17408 x 5120 48.3 / 47.6);
// - from 65536 rows from 16 (151936 x 4096: Q2_K 70.5 / 68.7, PQ2 74.1 / 57.8, Q8_0 169.5 /
//   144.5).
static uint32_t gemm_min_tokens(uint64_t rows) {
    return rows >= 65536 ? 16 : rows >= 16384 ? 17 : rows >= 8192 ? 48 : 65;
}

bool prefill_k_supported(uint32_t kind, uint64_t cols, uint64_t rows, uint32_t tokens) {
    // Codes, sums and scales are addressed with 32-bit buffer offsets.
    const uint64_t code_bytes = cols * padded_tokens(tokens);
    const bool kinds = kind == kQ2_K || kind == kPQ2 || kind == kQ8_0 || kind == kTQ1_0 || kind == kTQ2_0;
    return kinds && cols % kUnit == 0 && cols <= 65536 && rows > 0 && rows < (1ull << 31) &&
           code_bytes < (1ull << 31) && tokens >= gemm_min_tokens(rows);
}

// The prep (quantizing f32 input, or with BLOCKS copying prepared blocks of src_stride bytes
// per token) and the GEMM.
template <bool BLOCKS>
static int launch_k(uint32_t kind, const void *w_tiled, uint64_t cols, uint64_t rows, const void *src,
                    uint32_t src_stride, uint32_t M, int pinned, float *out, void *scratch, int *err, hipStream_t s) {
    if (!prefill_k_supported(kind, cols, rows, M)) return kLaunchUnsupported;
    const uint32_t K = static_cast<uint32_t>(cols), Mp = padded_tokens(M), nu = K / kUnit;
    uint8_t *base = static_cast<uint8_t *>(scratch);
    uint8_t *xq = base;
    float *as = reinterpret_cast<float *>(base + align256(static_cast<size_t>(Mp) * K));
    _Float16 *bs = reinterpret_cast<_Float16 *>(reinterpret_cast<uint8_t *>(as) + align256(static_cast<size_t>(nu) * Mp * 4 * 8));
    constexpr uint32_t kTok = 4;
    static_assert(kTokAlign % kTok == 0, "the prep takes whole token groups");
    const dim3 pgrid(Mp / kTok * ((K + 1023) / 1024)), pblock(64 * kTok);
    auto prep = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, pgrid, pblock, 0, s, src, src_stride, M, Mp, K, pinned, xq, as, bs, err);
    };
    switch (kind) {
        case kQ2_K: prep(k_prefill_k_prep<kQ2_K, kTok, BLOCKS>); break;
        case kQ8_0: prep(k_prefill_k_prep<kQ8_0, kTok, BLOCKS>); break;
        case kTQ1_0: prep(k_prefill_k_prep<kTQ1_0, kTok, BLOCKS>); break;
        case kTQ2_0: prep(k_prefill_k_prep<kTQ2_0, kTok, BLOCKS>); break;
        default: prep(k_prefill_k_prep<kPQ2, kTok, BLOCKS>);
    }
    if (const int e = launch_status()) return e;
    const uint32_t gx = static_cast<uint32_t>((rows + kRowsPerWg - 1) / kRowsPerWg);
    const auto W = static_cast<const uint8_t *>(w_tiled);
    const uint32_t R = static_cast<uint32_t>(rows);
    // Tokens per workgroup (measured, Q2_K 6144 x 2048, us): 64 from 1024 tokens (2048: 93.4
    // against 97.4 with 32; 4096: 184.3 / 200.4), 32 below (128 tokens: 18.0 / 22.3).
    // Q8_0 keeps 32 (2048 tokens: 158.8 us against 156.4 with 64, whose chain operands take
    // two wavefronts per SIMD instead of three).  Large matrices take 64 already while that
    // keeps 512 workgroups (their weights are re-read once per token group; Q2_K 151936 x
    // 4096, us: 128 tokens 273 -> 249, 512 tokens 987 -> 860; 32768 x 4096, 128 tokens 61.6
    // -> 53.8).  Only the token groups that hold real tokens are launched (the prep pads to Mp).
    const bool wide = M > 512 || (static_cast<uint64_t>(gx) * ((M + 63) / 64) >= 512 && M > 32);
    const uint32_t nt = wide && kind != kQ8_0 ? 64 : 32, groups = (M + nt - 1) / nt;
    const uint32_t xcd_major = groups % 8 == 0 && gx <= 65535;  // grid y and z limits
    const dim3 grid = xcd_major ? dim3(8, gx, groups / 8) : dim3(gx, groups);
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, W, R, nu, xq, as, bs, M, Mp, xcd_major, out, err);
    };
    if (kind == kQ2_K)
        nt == 64 ? go(k_prefill_kq<kQ2_K, 2, false>) : go(k_prefill_kq<kQ2_K, 1, false>);
    else if (kind == kTQ1_0)
        nt == 64 ? go(k_prefill_kq<kTQ1_0, 2, false>) : go(k_prefill_kq<kTQ1_0, 1, false>);
    else if (kind == kTQ2_0)
        nt == 64 ? go(k_prefill_kq<kTQ2_0, 2, false>) : go(k_prefill_kq<kTQ2_0, 1, false>);
    else if (kind == kQ8_0)
        go(k_prefill_kq<kQ8_0, 1, false>);
    else if (pinned)
        nt == 64 ? go(k_prefill_kq<kPQ2, 2, true>) : go(k_prefill_kq<kPQ2, 1, true>);
    else
        nt == 64 ? go(k_prefill_kq<kPQ2, 2, false>) : go(k_prefill_kq<kPQ2, 1, false>);
    return launch_status();
}

int launch_prefill_k(uint32_t kind, const void *w_tiled, uint64_t cols, uint64_t rows, const float *x, uint32_t M,
                     int pinned, float *out, void *scratch, int *err, hipStream_t s) {
    return launch_k<false>(kind, w_tiled, cols, rows, x, 0, M, pinned, out, scratch, err, s);
}

int launch_prefill_k_blocks(uint32_t kind, const void *w_tiled, uint64_t cols, uint64_t rows, const void *act,
                            uint32_t act_stride, uint32_t M, int pinned, float *out, void *scratch, int *err,
                            hipStream_t s) {
    return launch_k<true>(kind, w_tiled, cols, rows, act, act_stride, M, pinned, out, scratch, err, s);
}

}  // namespace prism
