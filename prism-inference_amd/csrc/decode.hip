// decode.hip -- the non-projection kernels of one full-attention decode step (gfx950):
// per-head q/k RMSNorm + RoPE + binary16 rounding, attention scores, softmax and the
// value reduction, the final norm + Q8_0 quantization ahead of the LM head, and the
// greedy choice + embedding of the next token.  The projections (q/k/v, o, the FFN
// chain, the LM head) run on the packed-matvec kernels.
//
// Position and token live in a device-resident DecodeState that the last kernel of
// a step advances, so one captured HIP graph replays every step unchanged.
//
// Arithmetic follows the reference's source order (src/graph.rs:4480-4911,
// src/kernels.rs:1256-1273,1344-1361,2971-3011,3679-3733,4431-4462): binary32
// products summed in binary64 for the dots and the value reduction, binary16
// rounding of q, k, v and of the probabilities.  Only the order of the binary64
// additions and the rare last-bit differences of exp/cos/sin (evaluated in
// binary64, device_common.hpp) differ from the reference.
#include "device_common.hpp"
#include "kernels.hpp"
#include "quant_dev.hpp"
#include "tiled.hpp"

namespace prism {

namespace {

constexpr uint32_t kHead = 128;        // head dimension the attention kernels are built for
constexpr uint32_t kScoreLanes = 4;    // lanes per scored position (kHead / 4 dimensions each)
constexpr uint32_t kScoreChunk = 256 / kScoreLanes;  // positions per score workgroup
constexpr uint32_t kValueDims = 16;     // dimensions per value workgroup
constexpr uint32_t kValueGroups = 256;  // position groups per value workgroup (x kValueDims/4 threads)
constexpr uint32_t kMaxTokens = 8192;   // KV cache positions the value kernel's LDS allows

// Score maxima slots per head: one per wavefront (16 positions) of each score workgroup.
__host__ __device__ constexpr uint32_t maxima_slots(uint32_t max_tokens) {
    return 4u * ((max_tokens + kScoreChunk - 1u) / kScoreChunk);
}

__device__ __forceinline__ uint16_t f16_bits(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// rope_frequencies_mrope (src/graph.rs:6406-6431) for text positions [pos, pos, pos, 0]:
// index i rotates by theta_sector * scale^i, the products rounded one by one; thread
// i < rope/2 writes pair i.
__device__ __forceinline__ void rope_freqs(DecodeState *st, uint32_t pos, const RopeArgs &r) {
    const uint32_t i = threadIdx.x;
    if (i >= r.rope / 2) return;
    float angle = i < 3 * r.sections[i % 3] ? static_cast<float>(pos) : 0.0f;
    for (uint32_t k = 0; k < i; ++k) angle = angle * r.theta_scale;
    st->cs[i] = cos_f32(angle);
    st->sn[i] = sin_f32(angle);
}

// rms_norm_rope_round_f16_into::<false> (src/kernels.rs:3679-3733) of two heads, one
// wavefront each: wavefront 0 takes the query head, wavefront 1 the KV head's key
// (wavefronts 2 and 3 only meet the closing barrier).  Lane l holds two elements of its
// head, the rotation pair (l, l + rope/2) when l < rope/2 and else (2l, 2l + 1), both past
// the rotated dimensions (x, the norm weights w and the pair's cos/sin already loaded), so
// the sum of squares is one wavefront butterfly and the rotation stays in the lane.  Per
// head: binary64 sum of the binary32 squares, mean rounded to binary32, 1/sqrt(mean + eps),
// (x * scale) * w, the rotation (x_a c - x_b s, x_a s + x_b c), rounding to binary16.  The
// results land in dst[0] (query) and dst[1] (key).  Returns the thread's error bits.
__device__ int norm_rope_wave(const float (&x)[2], const float (&w)[2], float c, float sn, bool rot, uint32_t ia,
                              uint32_t ib, float eps, float (*dst)[kHead]) {
    const uint32_t wave = threadIdx.x >> 6;
    int e = 0;
    if (wave < 2) {  // wave-uniform
        const double s = wave_sum(static_cast<double>(x[0] * x[0]) + static_cast<double>(x[1] * x[1]));
        const float mean = static_cast<float>(s / static_cast<double>(kHead));
        float scale = 1.0f / __builtin_sqrtf(mean + eps);
        scale = (finite(scale) && scale > 0.0f) ? scale : 0.0f;
        if (scale == 0.0f) e = kErrNonfinite;
        const float va = (x[0] * scale) * w[0], vb = (x[1] * scale) * w[1];
        if (!finite(va) || !finite(vb)) e |= kErrNonfinite;
        float ra = va, rb = vb;
        if (rot) {
            ra = va * c - vb * sn;
            rb = va * sn + vb * c;
        }
        if (!finite(ra) || !finite(rb)) e |= kErrNonfinite;
        ra = round_f16(ra);
        rb = round_f16(rb);
        if (!finite(ra) || !finite(rb)) e |= kErrNonfinite;
        dst[wave][ia] = ra;
        dst[wave][ib] = rb;
    }
    __syncthreads();
    return e;
}

// Workgroups go to the eight XCDs round-robin in dispatch order (x fastest), each XCD with
// its own L2.  Workgroups of one "unit" read the same cached rows (the query heads of a KV
// head, and the value slices that share a 128-byte row segment).  When the units divide
// by eight, workgroup b takes member (b/8) % members of unit b%8 + 8*((b/8)/members), so a
// unit's workgroups share one XCD and its rows are fetched into one L2; otherwise the
// plain order stands (false).  The grid holds units * members workgroups; members is a
// power of two (the shifts keep integer division off every workgroup's first steps).
__device__ __forceinline__ bool xcd_unit(uint32_t units, uint32_t lg_members, uint32_t &unit, uint32_t &member) {
    if (units % 8 != 0) return false;
    const uint32_t b = blockIdx.x + gridDim.x * blockIdx.y;
    const uint32_t k = b >> 3;
    unit = (b & 7u) + ((k >> lg_members) << 3);
    member = k & ((1u << lg_members) - 1u);
    return true;
}

__device__ __forceinline__ bool pow2(uint32_t v) { return v != 0 && (v & (v - 1u)) == 0; }

// Grid (heads, ceil(max_tokens / kScoreChunk)), 256 threads.  Each workgroup
// normalizes and rotates its query head and its KV head's current key, the first
// workgroup of every KV head appends the current key and value to the binary16
// caches, and the four lanes of quad t score position chunk*64 + t <= pos (a quarter
// of the dimensions each): f16_dot(q, k) * (1/sqrt(head)) with the current key taken
// from LDS.  Each wavefront also leaves the largest of its 16 scores (-inf for none) in
// maxima[head][4 * chunk + wavefront], so the softmax needs no workgroup-wide maximum.
// Every global
// read that does not depend on another (the cached key row, the head inputs, norm
// weights, RoPE factors, the value to append) is issued before the first is used.
__global__ __launch_bounds__(256) void k_attn_scores(AttnArgs p) {
    __shared__ float hv[2][kHead];  // [0] query, [1] current key
    const uint32_t tid = threadIdx.x, group = p.heads / p.kv_heads;
    uint32_t h = blockIdx.x, chunk = blockIdx.y, unit, member;
    const uint32_t lg_kv = __builtin_ctz(p.kv_heads), lg_group = __builtin_ctz(group);
    if (pow2(p.kv_heads) && pow2(group) && xcd_unit(p.kv_heads * gridDim.y, lg_group, unit, member)) {
        // unit: (KV head, chunk)
        h = ((unit & (p.kv_heads - 1u)) << lg_group) + member;
        chunk = unit >> lg_kv;
    }
    const uint32_t kh = h / group;
    const uint32_t qw = p.heads * kHead, kw = p.kv_heads * kHead;
    // Every load that does not need the position is issued before the position itself
    // is waited for: the normalization's inputs first (memory counters complete in issue
    // order, so the norm waits only for these), then the cached key row of this
    // thread's position (row 0 past the cache, never used).
    // The norm's two elements of this lane (norm_rope_wave; wavefronts 2 and 3 read
    // wavefront 0 and 1's and do not use them).
    const uint32_t lane = tid & 63u, which = (tid >> 6) & 1u, half = p.rope / 2;
    const bool rot = lane < half;
    const uint32_t ia = rot ? lane : 2u * lane, ib = rot ? lane + half : 2u * lane + 1u;
    const uint32_t base = which ? qw + kh * kHead : h * kHead;
    const float x[2] = {p.qkv[base + ia], p.qkv[base + ib]};
    // Both norm weights are read: selecting the pointer per thread would read it from
    // the kernel-argument memory with a vector load, one more round trip.
    const float qa = p.q_norm[ia], qb = p.q_norm[ib], ka = p.k_norm[ia], kb = p.k_norm[ib];
    const float nw[2] = {which ? ka : qa, which ? kb : qb};
    const float c = rot ? p.state->cs[lane] : 1.0f, sn = rot ? p.state->sn[lane] : 0.0f;
    const bool append = h % group == 0 && chunk == 0 && tid < kHead;
    const float vin = append ? p.qkv[qw + kw + kh * kHead + tid] : 0.0f;
    constexpr uint32_t kPart = kHead / kScoreLanes;  // dimensions per lane
    const uint32_t t = chunk * kScoreChunk + tid / kScoreLanes, part = tid % kScoreLanes;
    const uint32_t tr = t < p.max_tokens ? t : 0;
    uint4 kr[kPart / 8];
    const uint4 *krow =
        reinterpret_cast<const uint4 *>(p.kcache + static_cast<size_t>(tr) * kw + kh * kHead + part * kPart);
#pragma unroll
    for (uint32_t cc = 0; cc < kPart / 8; ++cc) kr[cc] = krow[cc];
    // The position last, through an address the compiler cannot prove uniform: a
    // uniform read becomes either a scalar load, which every later wait on the scalar
    // or LDS counter also waits for, or a vector load moved to a scalar register (and
    // so waited for) at once.  Read per lane, it is waited for where first used, after
    // the normalization.
    uint32_t lane0;
    asm volatile("v_mov_b32 %0, 0" : "=v"(lane0));
    const uint32_t pos = vector_load(&p.state->pos + lane0);

    // The norm needs no position; the exits come after it, so that no load above is
    // moved below them.
    int e = norm_rope_wave(x, nw, c, sn, rot, ia, ib, p.eps, hv);
    if (pos >= p.max_tokens) {  // uniform: every workgroup leaves
        if (tid == 0 && h == 0 && chunk == 0) raise_error(p.err, kErrInput);
        return;
    }
    if (chunk * kScoreChunk > pos) return;  // no position of this chunk is scored yet
    const float *qv = hv[0], *kv = hv[1];
    if (append) {
        const size_t at = static_cast<size_t>(pos) * kw + kh * kHead + tid;
        const float v = round_f16(vin);
        if (!finite(v)) e |= kErrNonfinite;
        p.kcache[at] = f16_bits(kv[tid]);
        p.vcache[at] = f16_bits(v);
    }
    const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(kHead));
    float smax = -__builtin_inff();
    if (t <= pos) {  // uniform over a quad
        // The terms are binary16 x binary16 products, exact in binary32, summed in
        // binary64: four partial sums per lane, then the quad's four lanes.  Only the
        // order of the binary64 additions differs from f16_dot's sequential sum.
        double s[4] = {0.0, 0.0, 0.0, 0.0};
        const float *q = qv + part * kPart;
        if (t == pos) {
            const float *k = kv + part * kPart;
#pragma unroll
            for (uint32_t dd = 0; dd < kPart; dd += 4)
#pragma unroll
                for (int j = 0; j < 4; ++j) s[j] += static_cast<double>(q[dd + j] * k[dd + j]);
        } else {
#pragma unroll
            for (uint32_t cc = 0; cc < kPart / 8; ++cc) {
                const uint32_t w4[4] = {kr[cc].x, kr[cc].y, kr[cc].z, kr[cc].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    s[j] += static_cast<double>(q[8 * cc + 2 * j] * h2f(w4[j] & 0xffffu));
                    s[j] += static_cast<double>(q[8 * cc + 2 * j + 1] * h2f(w4[j] >> 16));
                }
            }
        }
        double d = (s[0] + s[1]) + (s[2] + s[3]);
        d += dpp_d<kDppXor1>(d);
        d += dpp_d<kDppXor2>(d);
        smax = static_cast<float>(d) * scale;
        if (part == 0) p.scores[static_cast<size_t>(h) * p.max_tokens + t] = smax;
    }
    // Every lane of the workgroup is still here (the returns above are uniform).  fmaxf
    // passes over a NaN score; the softmax total then reports it.
    smax = wave_max(smax);
    if ((tid & 63u) == 0)
        p.maxima[static_cast<size_t>(h) * maxima_slots(p.max_tokens) + 4u * chunk + (tid >> 6)] = smax;
    if (e) raise_error(p.err, e);  // any element: an overflow can hit one element only
}

// Positions of the value reduction whose rows are loaded before the softmax (per
// thread: kValueAhead positions g, g + kValueGroups, ...), so that a context of up
// to kValueAhead * kValueGroups tokens costs one memory round trip.
constexpr uint32_t kValueAhead = 8;

// Grid (heads, kHead / kValueDims), 1024 threads; SPT scores per thread
// (SPT * 1024 >= max_tokens).  softmax_round_f16 (src/kernels.rs:4431-4462) of the
// head's pos+1 scores -- every workgroup recomputes it; each wavefront takes the maximum
// from the score kernel's per-wavefront maxima itself, and the reference's refusal of a
// NaN or +inf score or a -inf maximum shows as a non-finite total (each such case puts a
// NaN into the sum, and otherwise the total lies in [1, pos+1]) -- then source_value_tile
// (src/kernels.rs:2971-3011) for this workgroup's kValueDims dimensions:
// out[d] = sum_t p_t v_t[d] in binary64.  Each term is a binary16 x binary16
// product, exact in binary32, and a binary64 sum of such terms is exact unless they
// span more than 53 bits of magnitude (probabilities below 2^-24 are binary16
// zeros), so summing the positions in 256 interleaved groups and then the groups
// does not change the result.  The scores and the first value rows are read
// unconditionally (clamped to the cache, masked afterwards) before the position is
// waited for, so the kernel's inputs arrive in one memory round trip.
template <uint32_t SPT>
__global__ __launch_bounds__(1024) void k_attn_values(AttnArgs p) {
    __shared__ double redd[16];
    __shared__ float prob[kMaxTokens];
    __shared__ double acc[16][kValueDims];
    constexpr uint32_t nw = 16;  // wavefronts of the 1024-thread workgroup
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    // Unit: (KV head, 128-byte segment of its value rows), whose kLineSlices slices the
    // group's query heads all read.
    constexpr uint32_t kSlices = kHead / kValueDims, kLineSlices = 128 / (2 * kValueDims);
    static_assert((kSlices / kLineSlices) == 2 && kLineSlices == 4, "unit geometry below");
    const uint32_t group = p.heads / p.kv_heads;
    uint32_t h = blockIdx.x, slice = blockIdx.y, unit, member;
    const uint32_t lg_group = __builtin_ctz(group);
    if (pow2(group) && xcd_unit(p.kv_heads * 2u, lg_group + 2u, unit, member)) {
        h = ((unit >> 1) << lg_group) + (member & (group - 1u));
        slice = ((unit & 1u) << 2) + (member >> lg_group);
    }
    const uint32_t d0 = slice * kValueDims;
    const uint32_t kh = h / group, kw = p.kv_heads * kHead;
    const uint32_t last = p.max_tokens - 1;
    const float *sc = p.scores + static_cast<size_t>(h) * p.max_tokens;
    // Thread (g, q) sums positions g, g + kValueGroups, ... of dimensions d0+4q .. d0+4q+3, and
    // takes the softmax of positions g + kValueGroups * (q + kQuads * j): the probability of
    // its k-th value position is then held by lane q = k % kQuads of its own quad (register
    // k / kQuads) and reaches it by a DPP broadcast instead of an LDS round trip.
    constexpr uint32_t kQuads = kValueDims / 4;
    static_assert(kQuads == 4 && kValueAhead % kQuads == 0, "quad broadcast below");
    const uint32_t g = tid / kQuads, q = tid % kQuads;
    float sv[SPT];
#pragma unroll
    for (uint32_t k = 0; k < SPT; ++k) {
        const uint32_t i = g + kValueGroups * (q + kQuads * k);
        sv[k] = sc[i < last ? i : last];
    }
    // The head's score maxima: 4 per 64 positions, at most 64 * SPT; slots past the
    // position hold stale values and are masked below.
    const uint32_t slots = maxima_slots(p.max_tokens);
    const float *mxs = p.maxima + static_cast<size_t>(h) * slots;
    float mx[SPT];
#pragma unroll
    for (uint32_t k = 0; k < SPT; ++k) {
        const uint32_t i = lane + 64u * k;
        mx[k] = mxs[i < slots ? i : slots - 1u];
    }
    const uint32_t pos = vector_load(&p.state->pos);
    // Scores, maxima and position first: memory counters complete in issue order, and the
    // softmax must not wait for the value rows.
    __builtin_amdgcn_sched_barrier(0);
    const uint16_t *vb = p.vcache + kh * kHead + d0 + 4 * q;
    uint2 w[kValueAhead];
#pragma unroll
    for (uint32_t k = 0; k < kValueAhead; ++k) {
        const uint32_t i = g + k * kValueGroups;
        w[k] = *reinterpret_cast<const uint2 *>(vb + static_cast<size_t>(i < last ? i : last) * kw);
    }
    // A position past the cache is reported by the score kernel; this one then reduces
    // one position and writes nothing.  (No early return: the compiler would move the
    // value loads below it, after the wait for the position.)
    const bool ok = pos < p.max_tokens;
    const uint32_t n = ok ? pos + 1 : 1;
    const uint32_t live = 4u * ((n - 1u) / kScoreChunk + 1u);  // the slots of chunks 0 .. pos/64
    float m = -__builtin_inff();
#pragma unroll
    for (uint32_t k = 0; k < SPT; ++k)
        if (lane + 64u * k < live) m = fmaxf(m, mx[k]);
    m = wave_max(m);
    double tot = 0.0;
#pragma unroll
    for (uint32_t k = 0; k < SPT; ++k) {
        if (g + kValueGroups * (q + kQuads * k) < n) {
            const float e = exp_f32(sv[k] - m);
            sv[k] = e;
            tot += static_cast<double>(e);
        }
    }
    tot = wave_sum(tot);
    if (lane == 0) redd[wave] = tot;
    __syncthreads();
    tot = 0.0;
    for (uint32_t v = 0; v < nw; ++v) tot += redd[v];
    if (!__builtin_isfinite(tot)) {  // uniform
        if (tid == 0 && slice == 0 && ok) raise_error(p.err, kErrNonfinite);
        return;
    }
    const float inv = static_cast<float>(1.0 / tot);
    // Contexts past the kValueAhead * kValueGroups positions held in registers also stage
    // every probability in LDS for the loop below.
    constexpr bool kLong = SPT * 1024u > kValueAhead * kValueGroups;
    float pr[SPT];
#pragma unroll
    for (uint32_t k = 0; k < SPT; ++k) {
        const uint32_t i = g + kValueGroups * (q + kQuads * k);
        pr[k] = i < n ? round_f16(sv[k] * inv) : 0.0f;
        if constexpr (kLong)
            if (i < n) prob[i] = pr[k];
    }
    if constexpr (kLong) __syncthreads();
    double a[4] = {0.0, 0.0, 0.0, 0.0};
    auto accumulate = [&](const uint2 &r, float pr) {
        a[0] += static_cast<double>(pr * h2f(r.x & 0xffffu));
        a[1] += static_cast<double>(pr * h2f(r.x >> 16));
        a[2] += static_cast<double>(pr * h2f(r.y & 0xffffu));
        a[3] += static_cast<double>(pr * h2f(r.y >> 16));
    };
    // Rows past the position (stale cache rows) are zeroed here, where they are first
    // used: zeroing them earlier would wait for these loads before the softmax.
#pragma unroll
    for (uint32_t j = 0; j < kValueAhead / kQuads; ++j) {
        // Positions of register j >= SPT lie past the cache (>= SPT * 1024 > n - 1).
        const float v = j < SPT ? pr[j < SPT ? j : 0] : 0.0f;
        const float b[kQuads] = {dpp_f<0x00>(v), dpp_f<0x55>(v), dpp_f<0xAA>(v), dpp_f<0xFF>(v)};
#pragma unroll
        for (uint32_t qq = 0; qq < kQuads; ++qq) {
            const uint32_t k = kQuads * j + qq, i = g + k * kValueGroups;
            const bool in = i < n;
            accumulate(in ? w[k] : make_uint2(0, 0), in ? b[qq] : 0.0f);
        }
    }
    // Longer contexts: the remaining positions, eight rows loaded per batch before any
    // is used.
    if constexpr (kLong) {
        for (uint32_t i0 = g + kValueAhead * kValueGroups; i0 < n; i0 += 8 * kValueGroups) {
            uint2 r[8];
            float pv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t i = i0 + k * kValueGroups;
                const bool in = i < n;
                r[k] = in ? *reinterpret_cast<const uint2 *>(vb + static_cast<size_t>(i) * kw) : make_uint2(0, 0);
                pv[k] = in ? prob[i] : 0.0f;
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) accumulate(r[k], pv[k]);
        }
    }
    // A wavefront holds sixteen groups of the same four quads (lane = 4 * group + quad):
    // fold them with row rotations by 4 and 8 (DPP) and shuffles across rows, then the
    // wavefronts through LDS.
    constexpr int kDppRor4 = 0x124, kDppRor8 = 0x128;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        a[j] += dpp_d<kDppRor4>(a[j]);
        a[j] += dpp_d<kDppRor8>(a[j]);
        a[j] += __shfl_xor(a[j], 16);
        a[j] += __shfl_xor(a[j], 32);
    }
    if (lane < kValueDims / 4)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[wave][4 * q + j] = a[j];
    __syncthreads();
    if (tid < kValueDims && ok) {
        double t = acc[0][tid];
#pragma unroll
        for (uint32_t v = 1; v < nw; ++v) t += acc[v][tid];
        const float o = static_cast<float>(t);
        p.out[h * kHead + d0 + tid] = o;
        if (!finite(o)) raise_error(p.err, kErrNonfinite);
    }
}

// One workgroup: the final RMSNorm of the hidden state, quantized to Q8_0 in the
// source contract for the LM head (normalize_for_into + the public matvec's
// preparation, src/graph.rs:3992-3994).
__global__ __launch_bounds__(256) void k_lm_prep(const float *__restrict__ x, const float *__restrict__ w, uint32_t n,
                                                 float eps, Q8Block *__restrict__ out, int *err) {
    __shared__ double red[16];
    const float scale = rms_scale_wg(x, n, eps, red);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int e = scale == 0.0f ? kErrNonfinite
                          : quantize_prologue<false>(x, n, 0, out, wave, blockDim.x >> 6, lane, NormPre{w, scale});
    if (e && lane == 0) raise_error(err, e);
}

// Element i of row r of a Q8_0 matrix held in the 64-row tiled layout, dequantized
// as decode_row_into does (src/kernels.rs:303, d * q).  The Q8_0 unit (128 weights,
// 136 bytes) holds 16-byte code pieces p = 0..7 at p * 16 * TRP (element j in piece
// j / 16) and the four binary16 scales at 128 * TRP, 8 bytes per row; the offsets are
// written out so that nothing indexes a format table at run time (a table in private
// memory would cost a scratch round trip per element).
__device__ __forceinline__ float q8_0_tiled_at(const uint8_t *__restrict__ w, uint64_t rows, uint32_t cols, uint32_t r,
                                               uint32_t i) {
    constexpr uint32_t kUnitBytes = 136;
    const uint64_t row_bytes = static_cast<uint64_t>(cols) / 128 * kUnitBytes;
    const uint64_t tile = r / kTile;
    const uint32_t lr = r % kTile;
    const uint32_t trp = tile_rows_padded(rows, tile);
    const uint32_t u = i / 128, j = i % 128;
    const uint8_t *seg = w + tile * kTile * row_bytes + static_cast<uint64_t>(u) * trp * kUnitBytes;
    const int8_t q = static_cast<int8_t>(seg[(j / 16) * 16 * trp + lr * 16 + j % 16]);
    const uint8_t *sp = seg + 128 * trp + lr * 8 + 2 * (j / 32);
    const float d = h2f(static_cast<uint32_t>(sp[0]) | (static_cast<uint32_t>(sp[1]) << 8));
    return d * static_cast<float>(q);
}

// Row `token` of a tiled Q8_0 matrix, dequantized into out[0, cols) by the workgroup.  Each
// thread issues the loads of up to eight elements before its first store, so a row of up to
// 8 * blockDim.x elements costs one memory round trip rather than one per element.
__device__ __forceinline__ void embed_row(const uint8_t *__restrict__ emb, uint64_t rows, uint32_t cols,
                                          uint32_t token, float *__restrict__ out) {
    constexpr uint32_t kPer = 8;
    for (uint32_t i0 = threadIdx.x; i0 < cols; i0 += kPer * blockDim.x) {
        float v[kPer];
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) {
            const uint32_t i = i0 + k * blockDim.x;
            v[k] = i < cols ? q8_0_tiled_at(emb, rows, cols, token, i) : 0.0f;
        }
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) {
            const uint32_t i = i0 + k * blockDim.x;
            if (i < cols) out[i] = v[k];
        }
    }
}

__global__ __launch_bounds__(256) void k_embed(const uint8_t *__restrict__ emb, uint64_t rows, uint32_t cols,
                                               DecodeState *__restrict__ st, RopeArgs rope, float *__restrict__ out) {
    const uint32_t token = st->token;
    rope_freqs(st, st->pos, rope);
    embed_row(emb, rows, cols, token, out);
}

// Greedy choice: the first index of the largest logit.  The LM head's row-tile kernel
// leaves each 64-row tile's (largest value, first row); k_argmax_embed reduces them,
// records the token in the state and the token history, advances the position, and
// writes the chosen token's embedding (the tied LM head row) as the next step's hidden
// state.
constexpr uint32_t kArgmaxThreads = 1024, kArgmaxPer = 4;
constexpr uint32_t kArgmaxTiles = kArgmaxThreads * kArgmaxPer;
static_assert(static_cast<uint64_t>(kArgmaxTiles) * kTile == kGreedyMaxVocab, "greedy vocabulary limit");

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
    return bi == 0xffffffffu || (i != 0xffffffffu && (v > bv || (v == bv && i < bi)));
}

// Workgroup-wide (value, index) reduction; every thread returns the winner.
__device__ void reduce_best(float &best, uint32_t &idx, float *bv, uint32_t *bi) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) {
        const float ov = __shfl_xor(best, k);
        const uint32_t oi = __shfl_xor(idx, k);
        if (better(ov, oi, best, idx)) {
            best = ov;
            idx = oi;
        }
    }
    if (lane == 0) {
        bv[wave] = best;
        bi[wave] = idx;
    }
    __syncthreads();
    best = bv[0];
    idx = bi[0];
    for (uint32_t w = 1; w < nw; ++w)
        if (better(bv[w], bi[w], best, idx)) {
            best = bv[w];
            idx = bi[w];
        }
}

__global__ __launch_bounds__(kArgmaxThreads) void k_argmax_embed(const TileBest *__restrict__ tb, uint32_t ntiles,
                                                                 uint32_t vocab, const uint8_t *__restrict__ emb,
                                                                 uint32_t cols, DecodeState *__restrict__ st,
                                                                 RopeArgs rope, uint32_t *__restrict__ tokens,
                                                                 uint32_t max_steps, float *__restrict__ out) {
    __shared__ float bv[kArgmaxThreads / 64];
    __shared__ uint32_t bi[kArgmaxThreads / 64];
    const uint32_t tid = threadIdx.x;
    const uint32_t pos = st->pos;  // read before thread 0 advances it
    // Up to kArgmaxPer tiles per thread, every load issued before the first comparison;
    // the next position's RoPE frequencies are computed while they are in flight.
    TileBest t[kArgmaxPer];
#pragma unroll
    for (uint32_t k = 0; k < kArgmaxPer; ++k) {
        const uint32_t g = tid + k * kArgmaxThreads;
        t[k] = g < ntiles ? tb[g] : TileBest{0.0f, 0xffffffffu};
    }
    rope_freqs(st, pos + 1, rope);
    float best = -__builtin_inff();
    uint32_t idx = 0xffffffffu;
#pragma unroll
    for (uint32_t k = 0; k < kArgmaxPer; ++k)
        if (better(t[k].value, t[k].row, best, idx)) {
            best = t[k].value;
            idx = t[k].row;
        }
    reduce_best(best, idx, bv, bi);
    const uint32_t token = idx < vocab ? idx : 0;  // every tile holds a row
    if (tid == 0) {
        const uint32_t step = st->step;
        if (step < max_steps) tokens[step] = token;
        st->token = token;
        st->step = step + 1;
        st->pos = pos + 1;
    }
    embed_row(emb, vocab, cols, token, out);
}

}  // namespace

uint32_t attn_maxima_per_head(uint32_t max_tokens) { return maxima_slots(max_tokens); }

size_t argmax_scratch_bytes(uint64_t vocab) { return sizeof(TileBest) * ((vocab + kTile - 1) / kTile); }

namespace {
bool attention_supported(const AttnArgs &a) {
    return a.head_dim == kHead && a.rope <= kHead && a.rope % 2 == 0 && a.kv_heads != 0 && a.heads % a.kv_heads == 0 &&
           a.max_tokens != 0 && a.max_tokens <= kMaxTokens;
}
}  // namespace

int launch_attention(const AttnArgs &a) {
    const int rc = launch_attn_scores(a);
    return rc ? rc : launch_attn_values(a);
}

int launch_attn_scores(const AttnArgs &a) {
    if (!attention_supported(a)) return -2;
    const dim3 sg(a.heads, (a.max_tokens + kScoreChunk - 1) / kScoreChunk);
    hipLaunchKernelGGL(k_attn_scores, sg, dim3(256), 0, a.stream, a);
    return launch_status();
}

int launch_attn_values(const AttnArgs &a) {
    if (!attention_supported(a)) return -2;
    const dim3 vg(a.heads, kHead / kValueDims), vb(1024);
    if (a.max_tokens <= 1024)
        hipLaunchKernelGGL(k_attn_values<1>, vg, vb, 0, a.stream, a);
    else if (a.max_tokens <= 2048)
        hipLaunchKernelGGL(k_attn_values<2>, vg, vb, 0, a.stream, a);
    else if (a.max_tokens <= 4096)
        hipLaunchKernelGGL(k_attn_values<4>, vg, vb, 0, a.stream, a);
    else
        hipLaunchKernelGGL(k_attn_values<8>, vg, vb, 0, a.stream, a);
    return launch_status();
}

int launch_lm_prep(const float *x, const float *w, uint32_t n, float eps, void *q8_out, int *err, hipStream_t s) {
    if (n % 32) return -2;
    hipLaunchKernelGGL(k_lm_prep, dim3(1), dim3(256), 0, s, x, w, n, eps, static_cast<Q8Block *>(q8_out), err);
    return launch_status();
}

int launch_embed(const void *emb_tiled, uint64_t rows, uint32_t cols, DecodeState *st, const RopeArgs &rope,
                 float *out, hipStream_t s) {
    if (rope.rope > 2 * 64) return -2;
    hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), 0, s, static_cast<const uint8_t *>(emb_tiled), rows, cols, st,
                       rope, out);
    return launch_status();
}

int launch_argmax_embed(const TileBest *best, uint32_t vocab, const void *emb_tiled, uint32_t cols, DecodeState *st,
                        const RopeArgs &rope, uint32_t *tokens, uint32_t max_steps, float *out, hipStream_t s) {
    const uint32_t ntiles = (vocab + kTile - 1) / kTile;
    if (rope.rope > 2 * 64 || vocab == 0 || ntiles > kArgmaxTiles) return -2;
    hipLaunchKernelGGL(k_argmax_embed, dim3(1), dim3(kArgmaxThreads), 0, s, best, ntiles, vocab,
                       static_cast<const uint8_t *>(emb_tiled), cols, st, rope, tokens, max_steps, out);
    return launch_status();
}

}  // namespace prism
