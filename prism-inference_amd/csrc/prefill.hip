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
// against 8 MFMA K-steps, so the kernel is bound by the matrix pipe.
//
// Work split: a workgroup owns one 64-row weight tile and 256 tokens.  Wavefronts
// 0..3 decode one group each of the tile's current block into LDS as f16
// (wavefront g = group g, lane = row; every weight load is contiguous thanks to the
// tiled layout); each of the eight wavefronts then multiplies the tile's 64 rows by
// its own 32 tokens: two MFMA tiles of 32 x 32, rows on the MFMA's M side.  Each
// wavefront's activation codes for the next block stream into its own LDS double
// buffer with direct-to-LDS buffer loads (no registers held), issued a whole block
// ahead; the raw weight dwords of the next block are fetched at the same time and
// decoded between two barriers once every wavefront is done with the current one.
//
// The activation side is prepared once per call by k_prefill_prep: Q8_0 source
// quantization per token, the codes stored as binary16 in the order the weight
// decoder emits a group's elements, and the f32 scales beside them.
#include "device_common.hpp"
#include "kernels.hpp"
#include "quant_dev.hpp"
#include "tiled.hpp"

namespace prism {

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

typedef __attribute__((address_space(3))) void lds_void;

constexpr uint32_t kRowPitch = 272;  // bytes per decoded row in LDS: 128 f16 + 16 pad
constexpr uint32_t kWBytes = kTile * kRowPitch + kTile * 4;  // decoded rows + d per row
constexpr uint32_t kTokPerWave = 32, kWaves = 8, kTokPerWg = kTokPerWave * kWaves;
constexpr uint32_t kActBytes = kTokPerWave * 128 * 2;  // one wavefront's f16 codes of one block

// Element (within a 128-block) held at decode position 32g + p.  Built from the
// decoder below: a dword of PTQ1 code bytes is split into 16-bit lanes
// (bytes 0,2 -> L; 1,3 -> H) and each digit step emits the f16 pair of L then of H.
struct PermTable {
    uint8_t e[128];
};
__host__ __device__ constexpr PermTable make_perm() {
    PermTable t{};
    const int swz[4] = {0, 2, 1, 3};  // L pair = bytes (0,2), H pair = bytes (1,3)
    // group 0 / 1: A-piece dwords w=0..3, digits k (0,1) / (2,3): element 16k + 4w + byte
    for (int g = 0; g < 2; ++g)
        for (int w = 0; w < 4; ++w)
            for (int kk = 0; kk < 2; ++kk)
                for (int j = 0; j < 4; ++j) t.e[32 * g + 8 * w + 4 * kk + j] = 16 * (2 * g + kk) + 4 * w + swz[j];
    // group 2: A-piece digit 4 (64 + 4w + byte), then B-piece dwords v=0,1 digits 0,1
    for (int w = 0; w < 4; ++w)
        for (int j = 0; j < 4; ++j) t.e[64 + 4 * w + j] = 64 + 4 * w + swz[j];
    for (int v = 0; v < 2; ++v)
        for (int kk = 0; kk < 2; ++kk)
            for (int j = 0; j < 4; ++j) t.e[80 + 8 * v + 4 * kk + j] = 80 + 8 * kk + 4 * v + swz[j];
    // group 3: B-piece dwords v=0,1 digits 2..4, then the two tail bytes digits 0..3
    for (int v = 0; v < 2; ++v)
        for (int kk = 2; kk < 5; ++kk)
            for (int j = 0; j < 4; ++j) t.e[96 + 12 * v + 4 * (kk - 2) + j] = 80 + 8 * kk + 4 * v + swz[j];
    for (int kk = 0; kk < 4; ++kk)
        for (int j = 0; j < 2; ++j) t.e[120 + 2 * kk + j] = 120 + 2 * kk + j;
    return t;
}
__constant__ PermTable kPerm = make_perm();

// ---- activation prep ------------------------------------------------------------------
// One wavefront per (token, 1024 inputs): Q8_0 source quantization into LDS, then the
// codes leave as binary16 in decode order and the scales as f32.
__global__ __launch_bounds__(256) void k_prefill_prep(const float *__restrict__ x, uint32_t M, uint32_t K,
                                                      _Float16 *__restrict__ xh, float *__restrict__ sc,
                                                      int *__restrict__ err) {
    __shared__ Q8Block blk[4][32];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t chunks = (K + 1023) / 1024;
    const uint32_t item = blockIdx.x * 4 + wave;
    if (item >= M * chunks) return;  // uniform per wavefront
    const uint32_t t = item / chunks, c = item % chunks;
    const uint32_t k0 = c * 1024, n = K - k0 < 1024 ? K - k0 : 1024;  // multiple of 128
    const float *xr = x + static_cast<size_t>(t) * K + k0;
    const int e = q8_0_blocks_wave(xr, n / 32, 0 /* source contract */, blk[wave], lane);
    if (e) {
        if (lane == 0) raise_error(err, e);
        return;
    }
    __builtin_amdgcn_wave_barrier();
    // Lane l emits decode positions 16l..16l+15 of the chunk.
    const uint32_t pos0 = 16 * lane;
    if (pos0 < n) {
        const uint32_t b = pos0 / 128, p0 = pos0 % 128;
        uint32_t packed[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t h2 = 0;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t el = 128 * b + kPerm.e[p0 + 2 * i + j];  // element within the chunk
                const int8_t q = blk[wave][el / 32].values[el % 32];
                const _Float16 f = static_cast<_Float16>(q);
                h2 |= static_cast<uint32_t>(__builtin_bit_cast(uint16_t, f)) << (16 * j);
            }
            packed[i] = h2;
        }
        uint4 *dst = reinterpret_cast<uint4 *>(xh + static_cast<size_t>(t) * K + k0 + pos0);
        dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
        dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    }
    if (lane < n / 32) sc[static_cast<size_t>(t) * (K / 32) + k0 / 32 + lane] = blk[wave][lane].scale;
}

// ---- weight decode -------------------------------------------------------------------
// f16 pair (t_lo - 1, t_hi - 1) of the two digits sitting in byte 1 and byte 3 of m:
// the digits select bytes of the table {0xBC, 0x00, 0x3C} (the high bytes of -1, 0,
// +1 in binary16); selector 0x0c yields a zero low byte.
__device__ __forceinline__ uint32_t f16_pair(uint32_t m) {
    return perm(0u, 0x003C00BCu, (m & 0xff00ff00u) | 0x000c000cu);
}

// Emits `nd` digit steps of the 16-bit-lane pair V (two code bytes), starting at
// digit `first`, one f16 pair per step into out[0..nd).
template <int FIRST, int ND>
__device__ __forceinline__ void digits(uint32_t V, uint32_t *out) {
    constexpr uint32_t pw[5] = {1, 3, 9, 27, 81};
    if constexpr (FIRST > 0) V = (V * pw[FIRST]) & 0x00ff00ffu;
#pragma unroll
    for (int k = 0; k < ND; ++k) {
        const uint32_t m = V * 3u;
        out[k] = f16_pair(m);
        V = m & 0x00ff00ffu;
    }
}

// Raw code dwords wavefront g needs for its group (lane = row): g < 2: the four
// A-piece dwords; g == 2: A-piece + both B-piece dwords; g == 3: B-piece + tail.
struct RawW {
    uint32_t v[7];
};
__device__ __forceinline__ void load_group(__amdgpu_buffer_rsrc_t rs, uint32_t seg, uint32_t trp, uint32_t g,
                                           uint32_t lane, RawW &w) {
    if (g <= 2) {
        const u32x4 a = bload4(rs, seg + 16u * lane);
        w.v[0] = a.x;
        w.v[1] = a.y;
        w.v[2] = a.z;
        w.v[3] = a.w;
    }
    if (g >= 2) {
        const u32x2 bb = bload2(rs, seg + 16u * trp + 8u * lane);
        w.v[4] = bb.x;
        w.v[5] = bb.y;
    }
    if (g == 3) w.v[6] = bload1(rs, seg + 24u * trp + 4u * lane);
}

// Wavefront g decodes group g for the 64 rows of the tile (lane = row) and writes 16
// f16 pairs at row*kRowPitch + 64*g; wavefront 3 also stores the row's d.
__device__ __forceinline__ void decode_group(const RawW &w, uint32_t g, uint32_t lane, uint8_t *buf) {
    uint32_t o[16];
    if (g < 2) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t L = w.v[q] & 0x00ff00ffu, H = (w.v[q] >> 8) & 0x00ff00ffu;
            uint32_t pl[2], ph[2];
            if (g == 0) {
                digits<0, 2>(L, pl);
                digits<0, 2>(H, ph);
            } else {
                digits<2, 2>(L, pl);
                digits<2, 2>(H, ph);
            }
            o[4 * q] = pl[0];
            o[4 * q + 1] = ph[0];
            o[4 * q + 2] = pl[1];
            o[4 * q + 3] = ph[1];
        }
    } else if (g == 2) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t pl, ph;
            digits<4, 1>(w.v[q] & 0x00ff00ffu, &pl);
            digits<4, 1>((w.v[q] >> 8) & 0x00ff00ffu, &ph);
            o[2 * q] = pl;
            o[2 * q + 1] = ph;
        }
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            uint32_t pl[2], ph[2];
            digits<0, 2>(w.v[4 + v] & 0x00ff00ffu, pl);
            digits<0, 2>((w.v[4 + v] >> 8) & 0x00ff00ffu, ph);
            o[8 + 4 * v] = pl[0];
            o[8 + 4 * v + 1] = ph[0];
            o[8 + 4 * v + 2] = pl[1];
            o[8 + 4 * v + 3] = ph[1];
        }
    } else {
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            uint32_t pl[3], ph[3];
            digits<2, 3>(w.v[4 + v] & 0x00ff00ffu, pl);
            digits<2, 3>((w.v[4 + v] >> 8) & 0x00ff00ffu, ph);
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                o[6 * v + 2 * k] = pl[k];
                o[6 * v + 2 * k + 1] = ph[k];
            }
        }
        // tail bytes 24, 25 in the two 16-bit lanes; the pair is (byte 24, byte 25)
        const uint32_t c = w.v[6];
        digits<0, 4>((c & 0xffu) | ((c & 0xff00u) << 8), o + 12);
        reinterpret_cast<float *>(buf + kTile * kRowPitch)[lane] = h2f(c >> 16);
    }
    uint4 *dst = reinterpret_cast<uint4 *>(buf + lane * kRowPitch + 64 * g);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
}

// LDS: decoded weights and the two activation buffers are distinct arrays, so the
// compiler can see that reading one never waits for the direct-to-LDS writes into
// another (a shared array would make every LDS read wait for all loads in flight).
__shared__ __attribute__((aligned(16))) uint8_t g_wl[kWBytes];

// s_waitcnt through the builtin (gfx9 encoding, other counters left at their maxima),
// so the compiler's own wait bookkeeping sees it: vmcnt(0) / lgkmcnt(0).
__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0F70); }
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// Workgroup barrier for LDS hand-offs only: this wavefront's LDS traffic is complete,
// but global loads still in flight (the next block's prefetch) are not waited for, as
// __syncthreads() (a memory fence) would.
__device__ __forceinline__ void lds_barrier() {
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
}
__shared__ __attribute__((aligned(16))) uint8_t g_act0[kWaves * kActBytes];
__shared__ __attribute__((aligned(16))) uint8_t g_act1[kWaves * kActBytes];

__global__ __launch_bounds__(512) void k_prefill_ptq1(const uint8_t *__restrict__ W, uint32_t rows, uint32_t nu,
                                                      const _Float16 *__restrict__ xh, const float *__restrict__ sc,
                                                      uint32_t M, float *__restrict__ out, int *__restrict__ err) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool decoder = wave < 4;  // wavefront g < 4 decodes group g
    const uint32_t tile = blockIdx.x;
    const uint32_t K = nu * 128, row_bytes = nu * 28;
    const uint32_t left = rows - tile * kTile;
    const uint32_t trows = left < kTile ? left : kTile;
    const uint32_t trp = (trows + 7u) & ~7u;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(W + static_cast<size_t>(tile) * kTile * row_bytes, trp * row_bytes);
    // This wavefront's 32 tokens; tokens >= M read zeros and are not stored.
    const uint32_t t0 = blockIdx.y * kTokPerWg + wave * kTokPerWave;
    const uint32_t tvalid = t0 < M ? (M - t0 < kTokPerWave ? M - t0 : kTokPerWave) : 0u;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xh + static_cast<size_t>(t0) * K, tvalid * K * 2u);
    const __amdgpu_buffer_rsrc_t rsc = make_rsrc(sc + static_cast<size_t>(t0) * (K / 32), tvalid * (K / 32) * 4u);
    const uint32_t half = lane >> 5, l32 = lane & 31;
    uint8_t *a0 = g_act0 + wave * kActBytes;
    uint8_t *a1 = g_act1 + wave * kActBytes;

    // Block u's codes of this wavefront's tokens -> dst, laid out [g][st][lane] x 16
    // bytes: each (g, st) is one 1 KiB direct-to-LDS load (lane l lands at +16 l).
    auto stream_act = [&](uint32_t u, uint8_t *dst) {
#pragma unroll
        for (int gs = 0; gs < 8; ++gs)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void *)(dst + 1024 * gs), 16,
                                                     (l32 * K + 128 * u + 16 * gs + 8 * half) * 2u, 0, 0, 0);
    };
    auto load_s = [&](uint32_t u) -> u32x4 { return bload4(rsc, (l32 * (K / 32) + 4 * u) * 4u); };

    v16f tt[2], o[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;

    // One block: multiply the decoded weights by the codes in `ab`, fold into Y.
    auto compute = [&](const uint8_t *ab, u32x4 s) {
        const float sg[4] = {__uint_as_float(s.x), __uint_as_float(s.y), __uint_as_float(s.z), __uint_as_float(s.w)};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            v8h bx[2];
#pragma unroll
            for (int st = 0; st < 2; ++st) bx[st] = *reinterpret_cast<const v8h *>(ab + 1024 * (2 * g + st) + 16 * lane);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                v8h aw[2];
#pragma unroll
                for (int st = 0; st < 2; ++st)
                    aw[st] = *reinterpret_cast<const v8h *>(g_wl + (32 * i + l32) * kRowPitch +
                                                             2 * (32 * g + 16 * st + 8 * half));
                v16f a = {};
                a = __builtin_amdgcn_mfma_f32_32x32x16_f16(aw[0], bx[0], a, 0, 0, 0);
                a = __builtin_amdgcn_mfma_f32_32x32x16_f16(aw[1], bx[1], a, 0, 0, 0);
                // T = fl(T + sc_g * I_g): sc_g * I_g is exact, so one FMA (the first
                // group's 0 + sc_0*I_0 is the product itself; a signed zero there never
                // reaches Y).
#pragma unroll
                for (int r = 0; r < 16; ++r) tt[i][r] = g == 0 ? sg[0] * a[r] : __builtin_fmaf(sg[g], a[r], tt[i][r]);
            }
        }
        // Y += fl(d * T); rows 8q + 4*half + 0..3 of each row tile hold the lane's values.
        const float *dv = reinterpret_cast<const float *>(g_wl + kTile * kRowPitch);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 d4 = *reinterpret_cast<const float4 *>(dv + 32 * i + 8 * q + 4 * half);
                o[i][4 * q] = o[i][4 * q] + d4.x * tt[i][4 * q];
                o[i][4 * q + 1] = o[i][4 * q + 1] + d4.y * tt[i][4 * q + 1];
                o[i][4 * q + 2] = o[i][4 * q + 2] + d4.z * tt[i][4 * q + 2];
                o[i][4 * q + 3] = o[i][4 * q + 3] + d4.w * tt[i][4 * q + 3];
            }
    };
    // Steps block u reading `cur`, streaming block u+1's codes into `nxt`; the raw
    // weights of block u+1 travel in registers and are decoded once every wavefront
    // is done with block u.
    auto step = [&](uint32_t u, const uint8_t *cur, uint8_t *nxt, u32x4 &s) {
        const bool more = u + 1 < nu;
        RawW wn;
        u32x4 sn = s;
        if (more) {
            if (decoder) load_group(rw, (u + 1) * trp * 28u, trp, wave, lane, wn);
            stream_act(u + 1, nxt);
            sn = load_s(u + 1);
        }
        compute(cur, s);
        s = sn;
        lds_barrier();  // every wavefront is done with block u's weights
        if (more && decoder) decode_group(wn, wave, lane, g_wl);
        wait_vmcnt0();  // block u+1's codes have landed
        lds_barrier();
    };

    stream_act(0, a0);
    if (decoder) {
        RawW w0;
        load_group(rw, 0, trp, wave, lane, w0);
        decode_group(w0, wave, lane, g_wl);
    }
    u32x4 s = load_s(0);
    wait_vmcnt0();
    lds_barrier();
    for (uint32_t u = 0; u < nu; u += 2) {
        step(u, a0, a1, s);
        if (u + 1 < nu) step(u + 1, a1, a0, s);
    }
    // Y[t][r]: the lane holds token t0 + l32 and rows 32i + 8q + 4*half + 0..3.
    if (l32 >= tvalid) return;
    float *yr = out + static_cast<size_t>(t0 + l32) * rows + static_cast<size_t>(tile) * kTile;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t r0 = 32 * i + 8 * q + 4 * half;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (r0 + e < trows) {
                    const float v = o[i][4 * q + e];
                    yr[r0 + e] = v;
                    bad |= !finite(v);
                }
            }
        }
    if (bad) raise_error(err, kErrNonfinite);
}

}  // namespace

size_t prefill_scratch_bytes(uint64_t cols, uint32_t tokens) {
    return static_cast<size_t>(tokens) * cols * 2 + static_cast<size_t>(tokens) * (cols / 32) * 4 + 256;
}

bool prefill_supported(uint32_t kind, uint64_t cols, uint64_t rows, int pinned) {
    return kind == kPTQ1 && !pinned && cols % 128 == 0 && cols <= 65536 && rows > 0 &&
           (rows * (cols / 128) * 28) < (1ull << 40);
}

int launch_prefill(const void *w_tiled, uint64_t cols, uint64_t rows, const float *x, uint32_t M, float *out,
                   void *scratch, int *err, hipStream_t s) {
    const uint32_t K = static_cast<uint32_t>(cols);
    _Float16 *xh = static_cast<_Float16 *>(scratch);
    float *sc = reinterpret_cast<float *>(static_cast<uint8_t *>(scratch) + ((static_cast<size_t>(M) * K * 2 + 255) & ~size_t(255)));
    const uint32_t chunks = (K + 1023) / 1024;
    const uint64_t items = static_cast<uint64_t>(M) * chunks;
    hipLaunchKernelGGL(k_prefill_prep, dim3(static_cast<uint32_t>((items + 3) / 4)), dim3(256), 0, s, x, M, K, xh, sc,
                       err);
    if (hipGetLastError() != hipSuccess) return -1;
    const dim3 grid(static_cast<uint32_t>((rows + kTile - 1) / kTile), (M + kTokPerWg - 1) / kTokPerWg);
    hipLaunchKernelGGL(k_prefill_ptq1, grid, dim3(64 * kWaves), 0, s, static_cast<const uint8_t *>(w_tiled),
                       static_cast<uint32_t>(rows), K / 128, xh, sc, M, out, err);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace prism
