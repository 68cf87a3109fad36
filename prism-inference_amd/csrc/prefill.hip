// prefill.hip -- tiled prefill GEMM for PTQ1 weights on the f16 matrix cores (gfx950).
//
// Y[t][r] = sum over 128-blocks b of fl(d_w[r][b] * T[t][r][b]), T built per block as
//     T = ((sc0*I0 + sc1*I1) + sc2*I2) + sc3*I3     (binary32, this order)
// where I_g is the exact integer dot of the 32-element group g and sc_g the token's
// binary16-exact Q8_0 scale: the public matvec order of dot_q8_groups
// (src/kernels.rs:1043-1064), so every token row equals its own project_f32 result
// bit for bit (the reference's tile invariant, src/kernels/prefill.rs:829-887).
//
// Why f16 MFMA for an integer dot: ternary weights and int8 codes are exact in
// binary16, their products and any partial sum (|I| <= 32*127) are exact in the
// f32 accumulator, so v_mfma_f32_32x32x16_f16 returns float(I_g) exactly, with no
// conversion.  sc_g is a binary16 value (11 significant bits) and |I_g| < 2^12, so
// sc_g*I_g is exact in binary32 and fl(T + fl(sc_g*I_g)) == fma(sc_g, I_g, T): one
// FMA per output per group.  The chain costs 6 VALU ops per (token, row, block)
// against 8 MFMA K-steps of 32 x 32; the VALU, not the matrix pipe, bounds the kernel.
//
// Work split: a workgroup of four wavefronts owns 128 weight rows and NT = 32*CT
// tokens.  Wavefront w owns 32 rows and decodes them itself, straight into the f16
// operand registers of the MFMA (no LDS, no barrier for weights): lane l supplies row
// l%32 and, per group, the 16 elements of "half" h = l/32 -- 8 for each of the group's
// two K=16 steps.  The tokens' codes, prepared once per call in exactly that order,
// stream block by block into a double-buffered LDS ring with direct-to-LDS buffer
// loads; one barrier per block hands a buffer from the loads to the readers and back.
//
// The activation side is prepared once per call by k_prefill_prep: Q8_0 quantization per
// token, the codes stored as binary16 in operand order and the f32 scales beside them.
//
// The pinned contract (dot_q8_groups_pinned) runs k_prefill_ptq1_pinned on the same
// tiles with its own operand order, four K=8 MFMAs per group (one per native lane) and
// four FMA chains per output; see there.
#include "device_common.hpp"
#include "kernels.hpp"
#include "quant_dev.hpp"
#include "tiled.hpp"

namespace prism {

namespace {

typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

typedef __attribute__((address_space(3))) void lds_void;

constexpr uint32_t kRowsPerWg = 128, kTokAlign = 128;

constexpr uint32_t sel_bytes(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
    return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

// Operand order.  Code dword D of a PTQ1 block, digit k, gives a "quad" of four
// consecutive elements (tools/ternary/src/lib.rs:202-250): A-piece dword w -> 16k+4w,
// B-piece dword v -> 80+8k+4v, and the two tail bytes repeated (b24 b25 b24 b25) with
// digits (k, k, k+1, k+1) -> 120+2k.  The 16-bit-lane decoder turns bytes (0, 2) and
// (1, 3) of a quad's dword into two f16 pairs: elements (b, b+2) and (b+1, b+3) of the
// quad at b.  Half h of the wavefront (lanes 32h..32h+31) supplies, for every quad, its
// pair h, i.e. elements (b+h, b+h+2): a lane decodes bytes h and h+2 of every code dword
// and tail byte 24+h, half of the block's elements, in PairDecoder.
//
// Source order: K-step j (K = 16) of group g takes, in half h, pair h of the group's
// quads 4j .. 4j+3 (dword i of the operand: quad 4j + i).
// Pinned order (dot_q8_groups_pinned, src/kernels.rs:1102-1147): the chain needs, per
// group, the sum over each native lane l's elements 4l..4l+3 and 16+4l..16+4l+3
// (q8_native_lanes, src/kernels.rs:1066-1076), i.e. quads l and l+4 of the group.  One
// v_mfma_f32_32x32x8_f16 per native lane sums exactly those eight: half h supplies pair
// h of quads l and l+4.
// Either way the operand dword for (group g, quad q) starts at this element:
__host__ __device__ constexpr uint32_t pair_base(uint32_t g, uint32_t q, uint32_t h) { return 32 * g + 4 * q + h; }

// ---- activation prep ------------------------------------------------------------------
// A workgroup of TOK wavefronts quantizes TOK consecutive tokens (one each, 1024 inputs;
// Q8_0 in the source contract, or the pinned PTQ1 native-scale contract), then writes
// their codes as binary16 in operand order, one 16-byte store per thread, so a slot's TOK
// tokens leave as one contiguous segment:
//   source xh[u][g][j][h][t][8]  (16 slots of 16 bytes per block and token),
//   pinned xh[u][g][l][h][t][4]  (32 slots of 8 bytes; a store covers two tokens),
// u = 128-block, tokens padded to Mp (a multiple of TOK) with zeros; 256 bytes per block
// and token either way.  Scales as sc[u][t][g].  The grid holds Mp / TOK * chunks
// workgroups.  A quantizer error is raised and the wavefront carries on (the call then
// reports it and clears the output).  TOK = 16 fills whole 128-byte lines per pinned slot;
// short prompts take TOK = 4, which spreads their few tokens over four times as many CUs.
// With BLOCKS the tokens' prepared Q8_0 blocks (src_stride bytes per token) are copied instead
// of quantizing f32 input.
template <bool PINNED, uint32_t TOK, bool BLOCKS>
__global__ __launch_bounds__(64 * TOK) void k_prefill_prep(const void *__restrict__ src, uint32_t src_stride,
                                                           uint32_t M, uint32_t Mp, uint32_t K,
                                                           _Float16 *__restrict__ xh, float *__restrict__ sc,
                                                           int *__restrict__ err) {
    __shared__ Q8Block blk[TOK][32];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t chunks = (K + 1023) / 1024;
    const uint32_t c = blockIdx.x % chunks, tb = blockIdx.x / chunks * TOK;
    const uint32_t k0 = c * 1024, n = K - k0 < 1024 ? K - k0 : 1024;  // multiple of 128
    const uint32_t t = tb + wave;
    if (t < M) {
        if constexpr (BLOCKS) {
            const uint32_t *from = reinterpret_cast<const uint32_t *>(
                static_cast<const uint8_t *>(src) + static_cast<size_t>(t) * src_stride + (k0 / 32) * sizeof(Q8Block));
            uint32_t *to = reinterpret_cast<uint32_t *>(&blk[wave]);
            for (uint32_t i = lane; i < n / 32 * sizeof(Q8Block) / 4; i += 64) to[i] = from[i];
        } else {
            // Contract 0: source (round half away); 2: pinned PTQ1 native scale (quant_dev.hpp).
            const float *x = static_cast<const float *>(src) + static_cast<size_t>(t) * K + k0;
            const int e = q8_0_blocks_wave(x, n / 32, PINNED ? 2 : 0, blk[wave], lane);
            if (e && lane == 0) raise_error(err, e);
        }
    }
    __syncthreads();
    if (lane < n / 32) {
        const uint32_t u = k0 / 128 + lane / 4;
        sc[(static_cast<size_t>(u) * Mp + t) * 4 + lane % 4] = t < M ? blk[wave][lane].scale : 0.0f;
    }
    // Operand dword of token tb + w: the f16 pair (e, e + 2).
    auto pair = [&](uint32_t w, uint32_t e) -> uint32_t {
        const bool real = tb + w < M;
        const int8_t v0 = real ? blk[w][e / 32].values[e % 32] : 0;
        const int8_t v1 = real ? blk[w][(e + 2) / 32].values[(e + 2) % 32] : 0;
        return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(v0))) |
               static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(v1))) << 16;
    };
    // 16 * TOK stores of 16 bytes per block: (slot, token) for the source order (16 slots),
    // (slot, token pair) for the pinned one (32 slots); consecutive threads take
    // consecutive tokens of one slot.
    for (uint32_t i = tid; i < n / 128 * 16 * TOK; i += 64 * TOK) {
        const uint32_t ub = i / (16 * TOK), u = k0 / 128 + ub, base = 128 * ub;
        if constexpr (PINNED) {
            constexpr uint32_t kPairs = TOK / 2;
            const uint32_t p = i % kPairs, s = (i / kPairs) % 32;
            const uint32_t g = s >> 3, l = (s >> 1) & 3u, h = s & 1u;
            const uint32_t e0 = base + pair_base(g, l, h), e1 = base + pair_base(g, l + 4, h);
            uint4 *dst = reinterpret_cast<uint4 *>(xh + ((static_cast<size_t>(u) * 32 + s) * Mp + tb + 2 * p) * 4);
            *dst = make_uint4(pair(2 * p, e0), pair(2 * p, e1), pair(2 * p + 1, e0), pair(2 * p + 1, e1));
        } else {
            const uint32_t w = i % TOK, s = (i / TOK) % 16;
            const uint32_t g = s >> 2, j = (s >> 1) & 1u, h = s & 1u;
            uint4 *dst = reinterpret_cast<uint4 *>(xh + ((static_cast<size_t>(u) * 16 + s) * Mp + tb + w) * 8);
            *dst = make_uint4(pair(w, base + pair_base(g, 4 * j, h)), pair(w, base + pair_base(g, 4 * j + 1, h)),
                              pair(w, base + pair_base(g, 4 * j + 2, h)), pair(w, base + pair_base(g, 4 * j + 3, h)));
        }
    }
}

// ---- weight decode ---------------------------------------------------------------------
// f16 pair (t_lo - 1, t_hi - 1) of the two digits sitting in byte 1 and byte 3 of m:
// the digits select bytes of the table {0xBC, 0x00, 0x3C} (the high bytes of -1, 0,
// +1 in binary16); selector 0x0c yields a zero low byte.
__device__ __forceinline__ uint32_t f16_pair(uint32_t m) {
    return perm(0u, 0x003C00BCu, (m & 0xff00ff00u) | 0x000c000cu);
}
__device__ __forceinline__ uint32_t pair_mul(uint32_t v, uint32_t m) {  // two 16-bit lanes times (m.lo, m.hi)
    typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, v) * __builtin_bit_cast(u16x2, m));
}

// Raw weight dwords of one block for a lane: the A piece (16 B), the B piece (8 B) and
// the tail dword (d in the high half) of the lane's row.
struct RawBlock {
    u32x4 a;
    u32x2 b;
    uint32_t tl;
};
__device__ __forceinline__ void load_block_codes(__amdgpu_buffer_rsrc_t rs, uint32_t seg, uint32_t trp, uint32_t row,
                                                 RawBlock &w) {
    w.a = bload4(rs, seg + 16u * row);
    w.b = bload2(rs, seg + 16u * trp + 8u * row);
    w.tl = bload1(rs, seg + 24u * trp + 4u * row);
}

// The weight side of the operand order (pair_base): half h needs pair h of every quad of
// the block.  Quad q of group g comes from (tools/ternary/src/lib.rs:202-250 element map;
// (D, k) = code dword D at digit k)
//   g0: q<4 (A_q, 0), else (A_{q-4}, 1)        g1: q<4 (A_q, 2), else (A_{q-4}, 3)
//   g2: q<4 (A_q, 4), else (B_{q%2}, (q-4)/2)  g3: q<4 (B_{q%2}, 2 + q/2), q = 4, 5 (B_{q-4}, 4),
//   q = 6, 7 the tail quads 120, 124,
// so a lane decodes bytes h and h + 2 of every code dword (digits 0..4) and byte 24 + h of
// the tail (digits 0..3): half of the block's elements.  Every dword's digits are used in
// order, so the decoder runs group by group: group(g, aw) yields aw[l][i] = pair h of quad
// l + 4i (l = 0..3, i = 0..1).
struct PairDecoder {
    uint32_t la[4], lb[2], tb;  // remaining 16-bit-lane byte pairs; the tail byte twice

    __device__ __forceinline__ PairDecoder(const RawBlock &w, uint32_t h) {
        const uint32_t sel = h ? sel_bytes(1, 12, 3, 12) : sel_bytes(0, 12, 2, 12);  // bytes h, h+2
        la[0] = perm(w.a.x, w.a.x, sel);
        la[1] = perm(w.a.y, w.a.y, sel);
        la[2] = perm(w.a.z, w.a.z, sel);
        la[3] = perm(w.a.w, w.a.w, sel);
        lb[0] = perm(w.b.x, w.b.x, sel);
        lb[1] = perm(w.b.y, w.b.y, sel);
        tb = perm(w.tl, w.tl, h ? sel_bytes(1, 12, 1, 12) : sel_bytes(0, 12, 0, 12));
    }
    // The next digit's f16 pair of a byte pair (remainder times 3).
    __device__ __forceinline__ static uint32_t next(uint32_t &L) {
        const uint32_t m = L * 3u;
        L = m & 0x00ff00ffu;
        return f16_pair(m);
    }
    __device__ __forceinline__ void group(int g, uint32_t aw[4][2]) {
        if (g < 2) {
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                aw[l][0] = next(la[l]);
                aw[l][1] = next(la[l]);
            }
        } else if (g == 2) {
#pragma unroll
            for (int l = 0; l < 4; ++l) aw[l][0] = next(la[l]);
#pragma unroll
            for (int l = 0; l < 4; ++l) aw[l][1] = next(lb[l % 2]);
        } else {
#pragma unroll
            for (int l = 0; l < 4; ++l) aw[l][0] = next(lb[l % 2]);
            aw[0][1] = next(lb[0]);
            aw[1][1] = next(lb[1]);
            // The tail byte at digit multipliers (3^k, 3^(k+1)): quads 120 (k = 0), 124 (k = 2).
            aw[2][1] = f16_pair((pair_mul(tb, 1u | (3u << 16)) & 0x00ff00ffu) * 3u);
            aw[3][1] = f16_pair((pair_mul(tb, 9u | (27u << 16)) & 0x00ff00ffu) * 3u);
        }
    }
};

// s_waitcnt through the builtin (gfx9 encoding, other counters left at their maxima),
// so the compiler's own wait bookkeeping sees it: vmcnt(0) / lgkmcnt(0).
__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0F70); }
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// Workgroup barrier for LDS hand-offs: this wavefront's LDS traffic is complete, but
// global loads still in flight are not waited for, as __syncthreads() (a fence) would.
__device__ __forceinline__ void lds_barrier() {
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
}

template <int CT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(CT == 4 ? 2 : 3))) void k_prefill_ptq1(const uint8_t *__restrict__ W, uint32_t rows, uint32_t nu,
                                                      const _Float16 *__restrict__ xh, const float *__restrict__ sc,
                                                      uint32_t M, uint32_t Mp, uint32_t xcd_major,
                                                      float *__restrict__ out, int *__restrict__ err) {
    constexpr uint32_t NT = 32 * CT;
    constexpr uint32_t kRun = NT * 16;  // bytes of one (g, j, h) run of one block
    // actN[g*2+j][h][token][16 bytes]: a lane's operand is 16 contiguous bytes, and
    // each half-wavefront of a read covers 512 contiguous bytes (no bank conflicts).
    // sclN holds the tokens' four group scales.  The two ring buffers are separate
    // objects, and the loop below names them statically, so the compiler can tell a
    // read of one from the direct-to-LDS loads in flight into the other and does not
    // wait for those loads before the current block's reads.
    __shared__ __attribute__((aligned(16))) uint8_t act0[8][2][kRun];
    __shared__ __attribute__((aligned(16))) uint8_t act1[8][2][kRun];
    __shared__ __attribute__((aligned(16))) float4 scl0[NT];
    __shared__ __attribute__((aligned(16))) float4 scl1[NT];
    const uint32_t lane = threadIdx.x & 63, r32 = lane & 31, h = lane >> 5;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Workgroups go to the eight XCDs round-robin in dispatch order (x fastest), each
    // XCD with its own L2.  With a multiple of eight token groups the grid is (8, row
    // blocks, token groups / 8): XCD x takes token groups x, x+8, ... and every row
    // block of each, so its tokens' codes are read into one L2 only and the whole
    // weight matrix is shared there by its token groups.  Otherwise (row blocks, token
    // groups).
    const uint32_t bx = xcd_major ? blockIdx.y : blockIdx.x;
    const uint32_t by = xcd_major ? blockIdx.x + 8 * blockIdx.z : blockIdx.y;
    const uint32_t tile = 2 * bx + (wave >> 1), hw = wave & 1;
    const uint32_t tiles = (rows + kTile - 1) / kTile;
    const uint32_t t0 = by * NT;
    const uint32_t row_bytes = nu * 28;
    uint32_t trows = 0;
    if (tile < tiles) {
        const uint32_t left = rows - tile * kTile;
        trows = left < kTile ? left : kTile;
    }
    const bool active = 32 * hw < trows;  // uniform per wavefront
    const uint32_t trp = (trows + 7u) & ~7u;
    const __amdgpu_buffer_rsrc_t rw =
        make_rsrc(W + static_cast<size_t>(active ? tile : 0) * kTile * row_bytes, active ? trp * row_bytes : 0u);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xh, nu * 8u * Mp * 32u);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(sc, nu * Mp * 16u);
    const uint32_t row = 32 * hw + r32, out0 = 32 * hw + 4 * h;  // tile rows

    // Block u's codes and scales of the workgroup's tokens -> act, scl: 16 runs of
    // NT*16 bytes and one of NT*16 bytes, each contiguous in xh / sc; one wavefront
    // instruction moves 64 tokens' 16 bytes (lanes past a short run idle).
    auto stage = [&](uint32_t u, uint8_t (&act)[8][2][kRun], float4 (&scl)[NT]) {
        constexpr uint32_t per = (NT + 63) / 64;  // instructions per run
#pragma unroll
        for (uint32_t k = wave; k < 16 * per; k += 4) {
            const uint32_t run = k / per, c = k % per;
            if (64 * c + lane < NT)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void *)(&act[run >> 1][run & 1][1024 * c]), 16,
                                                         ((u * 16 + run) * Mp + t0 + 64 * c + lane) * 16u, 0, 0, 0);
        }
        if (wave < per && 64 * wave + lane < NT)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)(&scl[64 * wave]), 16,
                                                     (u * Mp + t0 + 64 * wave + lane) * 16u, 0, 0, 0);
    };

    v16f o[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[ct][r] = 0.0f;

    RawBlock w;
    stage(0, act0, scl0);
    if (active) load_block_codes(rw, 0, trp, row, w);
    wait_vmcnt0();
    lds_barrier();
    // Block u from (act, scl) while block u+1 streams into (act_next, scl_next).
    auto block = [&](uint32_t u, const uint8_t (&act)[8][2][kRun], const float4 (&scl)[NT],
                     uint8_t (&act_next)[8][2][kRun], float4 (&scl_next)[NT]) {
        uint32_t aw[4][4][2];  // [g][i][j]: pair h of quad 4j + i of group g
        float dw = 0.0f;       // the lane's row scale in half 0, zero in half 1
        if (active) {
            PairDecoder dec(w, h);
#pragma unroll
            for (int g = 0; g < 4; ++g) dec.group(g, aw[g]);
            dw = h ? 0.0f : h2f(w.tl >> 16);
        }
        // The next block streams in while this one is multiplied.
        if (u + 1 < nu) {
            stage(u + 1, act_next, scl_next);
            if (active) load_block_codes(rw, (u + 1) * trp * 28u, trp, row, w);
        }
        if (active) {
            // The scales d_w of the lane's 16 output rows, in the MFMA output layout: the
            // outer product of the rows' scales with ones (exact).
            const v16f d = __builtin_amdgcn_mfma_f32_32x32x2f32(dw, h ? 0.0f : 1.0f, v16f{}, 0, 0, 0);
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const float4 sg4 = scl[32 * ct + r32];
                const float sg[4] = {sg4.x, sg4.y, sg4.z, sg4.w};
                v16f tt;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    v16f a = {};
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const v8h bx = *reinterpret_cast<const v8h *>(&act[2 * g + j][h][(32 * ct + r32) * 16]);
                        const v8h ax = __builtin_bit_cast(v8h, u32x4{aw[g][0][j], aw[g][1][j], aw[g][2][j], aw[g][3][j]});
                        a = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax, bx, a, 0, 0, 0);
                    }
                    // T = fl(T + sc_g * I_g): sc_g * I_g is exact, so one FMA (the first
                    // group's 0 + sc_0*I_0 is the product itself; a signed zero there
                    // never reaches Y).
#pragma unroll
                    for (int r = 0; r < 16; ++r) tt[r] = g == 0 ? sg[0] * a[r] : __builtin_fmaf(sg[g], a[r], tt[r]);
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) o[ct][r] = o[ct][r] + d[r] * tt[r];
            }
        }
        wait_vmcnt0();  // block u+1's codes, scales and weights have landed
        lds_barrier();  // and every wavefront is done with block u's buffers
    };
    for (uint32_t u = 0; u < nu; u += 2) {
        block(u, act0, scl0, act1, scl1);
        if (u + 1 < nu) block(u + 1, act1, scl1, act0, scl0);
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

// Short prompts on the same tiles: with few token groups the kernel above runs few
// workgroups, each through every block of its rows with one wavefront per SIMD (about 18 us
// of GEMM for 6144 x 2048 from 16 to 128 tokens).  Here a workgroup of sixteen wavefronts owns the
// same 128 rows and 32 tokens, and splits the blocks over four phases: wavefront w is row
// wavefront w % 4 (32 rows, as above) of phase w / 4, which takes blocks p, p + 4, ...
// Each phase stages its own block's codes (its four row wavefronts four runs each), so the
// codes still cross from L2 once per workgroup.  Per round of four blocks, phase 0 adds its
// own block's term fl(d_w * T) to the outputs it holds, phases 1..3 leave theirs in LDS, and
// after a barrier phase 0 adds them in block order: Y = Y + fl(d_w * T) block by block, the
// chain above, so every token row is again its own matvec.
constexpr uint32_t kPhases = 4;

__global__ __launch_bounds__(64 * 4 * kPhases) void k_prefill_ptq1_split(const uint8_t *__restrict__ W, uint32_t rows,
                                                                        uint32_t nu, const _Float16 *__restrict__ xh,
                                                                        const float *__restrict__ sc, uint32_t M,
                                                                        uint32_t Mp, uint32_t xcd_major,
                                                                        float *__restrict__ out, int *__restrict__ err) {
    constexpr uint32_t NT = 32;
    constexpr uint32_t kRun = NT * 16;  // bytes of one (g, j, h) run of one block
    // actN[phase][g*2+j][h][token][16 bytes], two ring buffers named statically (as above).
    __shared__ __attribute__((aligned(16))) uint8_t act0[kPhases][8][2][kRun];
    __shared__ __attribute__((aligned(16))) uint8_t act1[kPhases][8][2][kRun];
    __shared__ __attribute__((aligned(16))) float4 scl0[kPhases][NT];
    __shared__ __attribute__((aligned(16))) float4 scl1[kPhases][NT];
    // The terms of phases 1..3: [phase - 1][row wavefront][output register][lane].
    __shared__ float terms[kPhases - 1][4][16][64];
    const uint32_t lane = threadIdx.x & 63, r32 = lane & 31, h = lane >> 5;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t rw = wave & 3u, phase = wave >> 2;
    const uint32_t bx = xcd_major ? blockIdx.y : blockIdx.x;
    const uint32_t by = xcd_major ? blockIdx.x + 8 * blockIdx.z : blockIdx.y;
    const uint32_t tile = 2 * bx + (rw >> 1), hw = rw & 1;
    const uint32_t tiles = (rows + kTile - 1) / kTile;
    const uint32_t t0 = by * NT;
    const uint32_t row_bytes = nu * 28;
    uint32_t trows = 0;
    if (tile < tiles) {
        const uint32_t left = rows - tile * kTile;
        trows = left < kTile ? left : kTile;
    }
    const bool active = 32 * hw < trows;  // uniform per wavefront
    const uint32_t trp = (trows + 7u) & ~7u;
    const __amdgpu_buffer_rsrc_t rw_ =
        make_rsrc(W + static_cast<size_t>(active ? tile : 0) * kTile * row_bytes, active ? trp * row_bytes : 0u);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xh, nu * 8u * Mp * 32u);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(sc, nu * Mp * 16u);
    const uint32_t row = 32 * hw + r32, out0 = 32 * hw + 4 * h;  // tile rows

    // Block u's 16 runs (this phase's row wavefront rw moves runs rw, rw + 4, ...; one
    // instruction per run, lanes past the tokens idle) and the tokens' scales.
    auto stage = [&](uint32_t u, uint8_t (&act)[kPhases][8][2][kRun], float4 (&scl)[kPhases][NT]) {
#pragma unroll
        for (uint32_t k = rw; k < 16; k += 4)
            if (lane < NT)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void *)(&act[phase][k >> 1][k & 1][0]), 16,
                                                         ((u * 16 + k) * Mp + t0 + lane) * 16u, 0, 0, 0);
        if (rw == 0 && lane < NT)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)(&scl[phase][0]), 16, (u * Mp + t0 + lane) * 16u,
                                                     0, 0, 0);
    };

    v16f o;
#pragma unroll
    for (int r = 0; r < 16; ++r) o[r] = 0.0f;
    RawBlock w;
    if (phase < nu) {
        stage(phase, act0, scl0);
        if (active) load_block_codes(rw_, phase * trp * 28u, trp, row, w);
    }
    wait_vmcnt0();
    lds_barrier();
    // Round r (blocks 4r .. 4r+3) from (act, scl) while round r+1 streams into the others.
    auto round = [&](uint32_t r, const uint8_t (&act)[kPhases][8][2][kRun], const float4 (&scl)[kPhases][NT],
                     uint8_t (&act_next)[kPhases][8][2][kRun], float4 (&scl_next)[kPhases][NT]) {
        const uint32_t u = kPhases * r + phase, un = u + kPhases;
        const bool mine = u < nu && active;
        uint32_t aw[4][4][2];
        float dw = 0.0f;
        if (mine) {
            PairDecoder dec(w, h);
#pragma unroll
            for (int g = 0; g < 4; ++g) dec.group(g, aw[g]);
            dw = h ? 0.0f : h2f(w.tl >> 16);
        }
        if (un < nu) {
            stage(un, act_next, scl_next);
            if (active) load_block_codes(rw_, un * trp * 28u, trp, row, w);
        }
        if (mine) {
            const v16f d = __builtin_amdgcn_mfma_f32_32x32x2f32(dw, h ? 0.0f : 1.0f, v16f{}, 0, 0, 0);
            const float4 sg4 = scl[phase][r32];
            const float sg[4] = {sg4.x, sg4.y, sg4.z, sg4.w};
            v16f tt;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                v16f a = {};
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const v8h bx8 = *reinterpret_cast<const v8h *>(&act[phase][2 * g + j][h][r32 * 16]);
                    const v8h ax = __builtin_bit_cast(v8h, u32x4{aw[g][0][j], aw[g][1][j], aw[g][2][j], aw[g][3][j]});
                    a = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax, bx8, a, 0, 0, 0);
                }
#pragma unroll
                for (int k = 0; k < 16; ++k) tt[k] = g == 0 ? sg[0] * a[k] : __builtin_fmaf(sg[g], a[k], tt[k]);
            }
            if (phase == 0) {
#pragma unroll
                for (int k = 0; k < 16; ++k) o[k] = o[k] + d[k] * tt[k];
            } else {
#pragma unroll
                for (int k = 0; k < 16; ++k) terms[phase - 1][rw][k][lane] = d[k] * tt[k];
            }
        }
        wait_vmcnt0();  // round r+1's codes, scales and weights have landed
        lds_barrier();  // every term of round r is in LDS; round r's buffers are free
        if (phase == 0 && active) {
#pragma unroll
            for (uint32_t q = 1; q < kPhases; ++q)
                if (kPhases * r + q < nu)
#pragma unroll
                    for (int k = 0; k < 16; ++k) o[k] = o[k] + terms[q - 1][rw][k][lane];
        }
        lds_barrier();  // the terms are read before the next round writes them
    };
    const uint32_t rounds = (nu + kPhases - 1) / kPhases;
    for (uint32_t r = 0; r < rounds; r += 2) {
        round(r, act0, scl0, act1, scl1);
        if (r + 1 < rounds) round(r + 1, act1, scl1, act0, scl0);
    }
    if (phase != 0 || !active) return;
    // Y[t][r]: the lane holds token t0 + r32 and tile rows out0 + 8q + 0..3.
    const uint32_t t = t0 + r32;
    if (t >= M) return;
    bool bad = false;
    float *yr = out + static_cast<size_t>(t) * rows + static_cast<size_t>(tile) * kTile;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t r = out0 + 8 * q + e;
            if (r < trows) {
                const float v = o[4 * q + e];
                yr[r] = v;
                bad |= !finite(v);
            }
        }
    }
    if (bad) raise_error(err, kErrNonfinite);
}

// The pinned contract (dot_q8_groups_pinned, src/kernels.rs:1102-1147) on the same
// tiles: per (token, row) four binary32 lanes L[l] = fma(I_l, dd_g, L[l]) with
// dd_g = fl(d_w * A_g.scale), group by group, and (L0 + L1) + (L2 + L3) at the end.  In
// the pinned operand order one v_mfma_f32_32x32x8_f16 per (group, native lane) sums
// exactly that lane's eight elements, half h of the wavefront supplying four of them
// (binary16-exact operands, |I| <= 8*127): four MFMAs per group, each as long as one
// K=16 MFMA on gfx950, and no masking.  20 VALU per output and block instead of 6 (the
// four dd_g and sixteen FMAs): 32 tokens per workgroup keep the 64 lane accumulators of
// a wavefront in registers.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_prefill_ptq1_pinned(
    const uint8_t *__restrict__ W, uint32_t rows, uint32_t nu, const _Float16 *__restrict__ xh,
    const float *__restrict__ sc, uint32_t M, uint32_t Mp, uint32_t xcd_major, float *__restrict__ out,
    int *__restrict__ err) {
    constexpr uint32_t NT = 32;
    constexpr uint32_t kRun = NT * 8;  // bytes of one (g, l, h) run of one block
    __shared__ __attribute__((aligned(16))) uint8_t act0[32][kRun];
    __shared__ __attribute__((aligned(16))) uint8_t act1[32][kRun];
    __shared__ __attribute__((aligned(16))) float4 scl0[NT];
    __shared__ __attribute__((aligned(16))) float4 scl1[NT];
    const uint32_t lane = threadIdx.x & 63, r32 = lane & 31, h = lane >> 5;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t bx = xcd_major ? blockIdx.y : blockIdx.x;
    const uint32_t by = xcd_major ? blockIdx.x + 8 * blockIdx.z : blockIdx.y;
    const uint32_t tile = 2 * bx + (wave >> 1), hw = wave & 1;
    const uint32_t tiles = (rows + kTile - 1) / kTile;
    const uint32_t t0 = by * NT;
    const uint32_t row_bytes = nu * 28;
    uint32_t trows = 0;
    if (tile < tiles) {
        const uint32_t left = rows - tile * kTile;
        trows = left < kTile ? left : kTile;
    }
    const bool active = 32 * hw < trows;  // uniform per wavefront
    const uint32_t trp = (trows + 7u) & ~7u;
    const __amdgpu_buffer_rsrc_t rw =
        make_rsrc(W + static_cast<size_t>(active ? tile : 0) * kTile * row_bytes, active ? trp * row_bytes : 0u);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xh, nu * 8u * Mp * 32u);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(sc, nu * Mp * 16u);
    const uint32_t row = 32 * hw + r32, out0 = 32 * hw + 4 * h;  // tile rows

    // Block u's codes (32 runs of NT*8 bytes, each contiguous in xh and in LDS; one
    // instruction moves four runs, lane l tokens 2(l%16), 2(l%16)+1 of run l/16) and the
    // scales of the workgroup's tokens.
    auto stage = [&](uint32_t u, uint8_t (&act)[32][kRun], float4 (&scl)[NT]) {
        for (uint32_t i = wave; i < 8; i += 4)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void *)(&act[4 * i][0]), 16,
                                                     ((u * 32 + 4 * i + lane / 16) * Mp + t0 + 2 * (lane % 16)) * 8u, 0,
                                                     0, 0);
        if (wave == 0 && lane < NT)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)(&scl[0]), 16, (u * Mp + t0 + lane) * 16u, 0,
                                                     0, 0);
    };

    float L[4][16];
#pragma unroll
    for (int l = 0; l < 4; ++l)
#pragma unroll
        for (int r = 0; r < 16; ++r) L[l][r] = 0.0f;
    const v16f zero = {};

    RawBlock w = {};  // stays zero in an inactive wavefront
    stage(0, act0, scl0);
    if (active) load_block_codes(rw, 0, trp, row, w);
    wait_vmcnt0();
    lds_barrier();
    auto block = [&](uint32_t u, const uint8_t (&act)[32][kRun], const float4 (&scl)[NT],
                     uint8_t (&act_next)[32][kRun], float4 (&scl_next)[NT]) {
        PairDecoder dec(w, h);
        const float dw = h ? 0.0f : h2f(w.tl >> 16);  // the lane's row scale in half 0, zero in half 1
        if (u + 1 < nu) {
            stage(u + 1, act_next, scl_next);
            if (active) load_block_codes(rw, (u + 1) * trp * 28u, trp, row, w);
        }
        if (active) {
            const float4 sg4 = scl[r32];
            const float sg[4] = {sg4.x, sg4.y, sg4.z, sg4.w};
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                // dd[r] = fl(d_w * A_g.scale) for every (row, token) of the tile, as the
                // outer product of the rows' and tokens' scales on the matrix pipe: K = 2
                // with the second term zero, one rounding (no product is subnormal: both
                // scales are binary16 values).
                const v16f dd = __builtin_amdgcn_mfma_f32_32x32x2f32(dw, h ? 0.0f : sg[g], zero, 0, 0, 0);
                uint32_t aw[4][2];
                dec.group(g, aw);
#pragma unroll
                for (int l = 0; l < 4; ++l) {
                    const v4h b = *reinterpret_cast<const v4h *>(&act[(4 * g + l) * 2 + h][r32 * 8]);
                    const u32x2 a = {aw[l][0], aw[l][1]};
                    const v16f i = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, a), b, zero, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) L[l][r] = __builtin_fmaf(i[r], dd[r], L[l][r]);
                }
            }
        }
        wait_vmcnt0();
        lds_barrier();
    };
    for (uint32_t u = 0; u < nu; u += 2) {
        block(u, act0, scl0, act1, scl1);
        if (u + 1 < nu) block(u + 1, act1, scl1, act0, scl0);
    }
    if (!active) return;
    const uint32_t t = t0 + r32;
    if (t >= M) return;
    bool bad = false;
    float *yr = out + static_cast<size_t>(t) * rows + static_cast<size_t>(tile) * kTile;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t r = out0 + 8 * q + e;
            if (r < trows) {
                const int k = 4 * q + e;
                const float v = (L[0][k] + L[1][k]) + (L[2][k] + L[3][k]);
                yr[r] = v;
                bad |= !finite(v);
            }
        }
    }
    if (bad) raise_error(err, kErrNonfinite);
}

uint32_t padded_tokens(uint32_t M) { return (M + kTokAlign - 1) / kTokAlign * kTokAlign; }

// Source-contract prompts up to this many tokens take the block-split kernel.  Measured for
// 6144 x 2048 (prep + GEMM, us, split against the kernel above): 16 tokens 19.6 / 23.1, 64
// tokens 20.9 / 24.1, 128 tokens 21.3 / 24.6, 256 tokens 37.1 / 32.5, 512 tokens 55.4 / 44.9.
// Beyond 128 tokens the four-token-group workgroups of the kernel above fill more CUs.
constexpr uint32_t kSplitMaxTokens = 128;
// Workgroup rows (128 weight rows each) from which a matrix counts as large for the choice of
// tokens per workgroup (32768 rows).
constexpr uint32_t kLargeRowBlocks = 256;

}  // namespace

size_t prefill_scratch_bytes(uint32_t kind, uint64_t cols, uint32_t tokens) {
    if (kind != kPTQ1) return prefill_k_scratch_bytes(cols, tokens);
    const size_t Mp = padded_tokens(tokens);
    return ((Mp * cols * 2 + 255) & ~size_t(255)) + Mp * (cols / 32) * 4;
}

// Tokens from which PTQ1 takes the GEMM rather than the skinny kernel (up to four 16-token
// chunks side by side per launch, each unit decoded once per chunk).  Measured (f32 input
// with its quantization, GEMM / skinny, us): 16 tokens 6144 x 2048 18.9 / 13.9, 12288 x 4096
// 30.2 / 20.9, 151936 x 4096 139 / 93; 32 tokens source 6144 x 2048 20.0 / 17.3, 12288 x 4096
// 31.6 / 31.8, 17408 x 5120 38.2 / 46.6, 32768 x 4096 41.7 / 54.8; pinned 6144 x 2048 31.6 /
// 27.0, 12288 x 4096 56.7 / 73.7; 48 tokens source 6144 x 2048 20.3 / 21.4, pinned 32.3 / 42.4.
static uint32_t ptq1_gemm_min_tokens(uint64_t rows) { return rows < 8192 ? 33 : 32; }

bool prefill_supported(uint32_t kind, uint64_t cols, uint64_t rows, int pinned, uint32_t tokens) {
    if (kind != kPTQ1) return prefill_k_supported(kind, cols, rows, tokens);
    // The token codes are addressed with 32-bit buffer offsets.
    const uint64_t code_bytes = cols / 128 * 8u * padded_tokens(tokens) * 32u;
    if (tokens < ptq1_gemm_min_tokens(rows)) return false;
    return kind == kPTQ1 && cols % 128 == 0 && cols <= 65536 && rows > 0 &&
           (rows * (cols / 128) * 28) < (1ull << 40) && code_bytes < (1ull << 31);
}

// The prep (quantizing f32 input, or with BLOCKS copying prepared Q8_0 blocks of src_stride
// bytes per token) and the PTQ1 GEMM.
template <bool BLOCKS>
static int launch_ptq1(const void *w_tiled, uint64_t cols, uint64_t rows, const void *src, uint32_t src_stride,
                       uint32_t M, int pinned, float *out, void *scratch, int *err, hipStream_t s, uint32_t cus) {
    const uint32_t K = static_cast<uint32_t>(cols), Mp = padded_tokens(M);
    if (static_cast<uint64_t>(K / 128) * 8u * Mp * 32u >= (1ull << 31)) return kLaunchUnsupported;
    _Float16 *xh = static_cast<_Float16 *>(scratch);
    float *sc = reinterpret_cast<float *>(static_cast<uint8_t *>(scratch) + ((static_cast<size_t>(Mp) * K * 2 + 255) & ~size_t(255)));
    const uint32_t chunks = (K + 1023) / 1024;
    const uint64_t items = static_cast<uint64_t>(Mp) * chunks;
    static_assert(kTokAlign % 16 == 0, "the prep takes whole token groups");
    // Measured (prep alone, 2048 tokens): pinned 8.5 us with 16 tokens per workgroup, 13.4
    // with one token per wavefront and 8-byte stores; source 8.2 with 4 tokens, 10.6 with
    // 16, 9.3 with one token per wavefront.  Short prompts take 4 in both: 16 would leave
    // most CUs idle.
    const bool wide = pinned && Mp >= 1024;
    const dim3 pgrid(static_cast<uint32_t>(items / (wide ? 16 : 4))), pblock(wide ? 1024 : 256);
    if (wide)
        hipLaunchKernelGGL((k_prefill_prep<true, 16, BLOCKS>), pgrid, pblock, 0, s, src, src_stride, M, Mp, K, xh, sc,
                           err);
    else if (pinned)
        hipLaunchKernelGGL((k_prefill_prep<true, 4, BLOCKS>), pgrid, pblock, 0, s, src, src_stride, M, Mp, K, xh, sc,
                           err);
    else
        hipLaunchKernelGGL((k_prefill_prep<false, 4, BLOCKS>), pgrid, pblock, 0, s, src, src_stride, M, Mp, K, xh, sc,
                           err);
    if (const int e = launch_status()) return e;
    const uint32_t gx = static_cast<uint32_t>((rows + kRowsPerWg - 1) / kRowsPerWg);
    const auto W = static_cast<const uint8_t *>(w_tiled);
    const uint32_t R = static_cast<uint32_t>(rows), nu = K / 128;
    if (pinned) {
        const uint32_t groups = (M + 31) / 32;  // token groups holding real tokens
        const uint32_t xcd_major = groups % 8 == 0 && gx <= 65535;
        const dim3 grid = xcd_major ? dim3(8, gx, groups / 8) : dim3(gx, groups);
        hipLaunchKernelGGL(k_prefill_ptq1_pinned, grid, dim3(256), 0, s, W, R, nu, xh, sc, M, Mp, xcd_major, out, err);
        return launch_status();
    }
    // Tokens per workgroup (measured, 6144 x 2048): 64 keeps three wavefronts per SIMD
    // and beats 128 (two per SIMD, the decode shared by more tokens) up to about 4096
    // tokens (4096: 232 against 241-246 us); 32 (four wavefronts per SIMD) keeps CUs busy
    // on short prompts up to 512 tokens (512: 45.0 against 46.6 us; 768: 65.4 against 64.2).
    // Large matrices (at least kLargeRowBlocks workgroup rows) re-read their weights once per
    // token group, from HBM: there the workgroups take as many tokens as keep at least 512 of
    // them (1024 beyond 512 tokens) in the grid, and short prompts skip the block-split kernel.
    // Measured, 151936 x 4096 (us, the small-matrix choice -> this one): 32 tokens 145 -> 114,
    // 64 tokens 282 -> 168, 128 tokens 523 -> 312, 512 tokens 1365 -> 1065; 32768 x 4096: 64
    // tokens 62 -> 56, 128 tokens 119 -> 78, 256 tokens 180 -> 132.
    if (gx >= kLargeRowBlocks) {
        const uint32_t want = M > 512 ? 1024 : 512, mr = (M + 31) / 32 * 32;
        uint32_t nt = 32;
        for (uint32_t c : {128u, 64u})
            if (c <= mr && static_cast<uint64_t>(gx) * ((M + c - 1) / c) >= want) {
                nt = c;
                break;
            }
        const uint32_t groups = (M + nt - 1) / nt;
        const uint32_t xcd_major = groups % 8 == 0 && gx <= 65535;
        const dim3 grid = xcd_major ? dim3(8, gx, groups / 8) : dim3(gx, groups);
        if (nt == 128)
            hipLaunchKernelGGL(k_prefill_ptq1<4>, grid, dim3(256), 0, s, W, R, nu, xh, sc, M, Mp, xcd_major, out, err);
        else if (nt == 64)
            hipLaunchKernelGGL(k_prefill_ptq1<2>, grid, dim3(256), 0, s, W, R, nu, xh, sc, M, Mp, xcd_major, out, err);
        else
            hipLaunchKernelGGL(k_prefill_ptq1<1>, grid, dim3(256), 0, s, W, R, nu, xh, sc, M, Mp, xcd_major, out, err);
        return launch_status();
    }
    // The block-split kernel holds one workgroup per CU: with more workgroups than CUs its
    // grid runs in two rounds (17408 x 5120, 48 tokens: 69.1 us against 38.2 at 32 tokens).
    if (M <= kSplitMaxTokens && static_cast<uint64_t>(gx) * ((M + 31) / 32) <= cus) {
        const uint32_t groups = (M + 31) / 32;  // token groups holding real tokens
        const uint32_t xcd_major = groups % 8 == 0 && gx <= 65535;
        const dim3 grid = xcd_major ? dim3(8, gx, groups / 8) : dim3(gx, groups);
        hipLaunchKernelGGL(k_prefill_ptq1_split, grid, dim3(64 * 4 * kPhases), 0, s, W, R, nu, xh, sc, M, Mp, xcd_major,
                           out, err);
        return launch_status();
    }
    const uint32_t nt = M >= 4096 ? 128 : M > 512 ? 64 : 32, groups = (M + nt - 1) / nt;
    const uint32_t xcd_major = groups % 8 == 0 && gx <= 65535;  // grid y and z limits
    const dim3 grid = xcd_major ? dim3(8, gx, groups / 8) : dim3(gx, groups);
    if (nt == 128)
        hipLaunchKernelGGL(k_prefill_ptq1<4>, grid, dim3(256), 0, s, W, R, nu, xh, sc, M, Mp, xcd_major, out, err);
    else if (nt == 64)
        hipLaunchKernelGGL(k_prefill_ptq1<2>, grid, dim3(256), 0, s, W, R, nu, xh, sc, M, Mp, xcd_major, out, err);
    else
        hipLaunchKernelGGL(k_prefill_ptq1<1>, grid, dim3(256), 0, s, W, R, nu, xh, sc, M, Mp, xcd_major, out, err);
    return launch_status();
}

int launch_prefill(uint32_t kind, const void *w_tiled, uint64_t cols, uint64_t rows, const float *x, uint32_t M,
                   int pinned, float *out, void *scratch, int *err, hipStream_t s, uint32_t cus) {
    if (kind != kPTQ1) return launch_prefill_k(kind, w_tiled, cols, rows, x, M, pinned, out, scratch, err, s);
    return launch_ptq1<false>(w_tiled, cols, rows, x, 0, M, pinned, out, scratch, err, s, cus);
}

int launch_prefill_blocks(uint32_t kind, const void *w_tiled, uint64_t cols, uint64_t rows, const void *act,
                          uint32_t act_stride, uint32_t M, int pinned, float *out, void *scratch, int *err,
                          hipStream_t s, uint32_t cus) {
    if (kind != kPTQ1)
        return launch_prefill_k_blocks(kind, w_tiled, cols, rows, act, act_stride, M, pinned, out, scratch, err, s);
    return launch_ptq1<true>(w_tiled, cols, rows, act, act_stride, M, pinned, out, scratch, err, s, cus);
}

}  // namespace prism
