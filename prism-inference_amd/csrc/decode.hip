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
constexpr uint32_t kScoreChunk = 256;  // positions per score workgroup
constexpr uint32_t kValueDims = 32;     // dimensions per value workgroup
constexpr uint32_t kValueGroups = 128;  // position groups per value workgroup (x kValueDims/4 threads)
constexpr uint32_t kMaxTokens = 8192;   // KV cache positions the value kernel's LDS allows

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

// rms_norm_rope_round_f16_into::<false> (src/kernels.rs:3679-3733) of one head
// (kHead values at src) into dst (LDS): (x * scale) * w, rotate the first `rope`
// dimensions (index i with i + rope/2), round to binary16.  Every thread of the
// workgroup calls it; returns error bits.
__device__ int norm_rope_head(const float *__restrict__ src, const float *__restrict__ w, float *dst, float *tmp,
                              double *red, const float *cs, const float *sn, uint32_t rope, float eps) {
    const uint32_t tid = threadIdx.x;
    const float scale = rms_scale_wg(src, kHead, eps, red);
    int e = scale == 0.0f ? kErrNonfinite : 0;
    if (tid < kHead) {
        const float v = (src[tid] * scale) * w[tid];
        tmp[tid] = v;
        if (!finite(v)) e |= kErrNonfinite;
    }
    __syncthreads();
    if (tid < kHead) {
        const uint32_t half = rope / 2;
        float r;
        if (tid < half)
            r = tmp[tid] * cs[tid] - tmp[tid + half] * sn[tid];
        else if (tid < rope)
            r = tmp[tid - half] * sn[tid - half] + tmp[tid] * cs[tid - half];
        else
            r = tmp[tid];
        if (!finite(r)) e |= kErrNonfinite;
        r = round_f16(r);
        if (!finite(r)) e |= kErrNonfinite;
        dst[tid] = r;
    }
    __syncthreads();
    return e;
}

// Grid (heads, ceil(max_tokens / kScoreChunk)), 256 threads.  Each workgroup
// normalizes and rotates its query head and its KV head's current key, the first
// workgroup of every KV head appends the current key and value to the binary16
// caches, and thread t scores position chunk*256 + t <= pos:
// f16_dot(q, k) * (1/sqrt(head)) with the current key taken from registers.
__global__ __launch_bounds__(256) void k_attn_scores(AttnArgs p) {
    __shared__ float qv[kHead], kv[kHead], tmp[kHead];
    __shared__ double red[16];
    const uint32_t tid = threadIdx.x, h = blockIdx.x, chunk = blockIdx.y;
    const uint32_t group = p.heads / p.kv_heads, kh = h / group;
    const uint32_t qw = p.heads * kHead, kw = p.kv_heads * kHead;
    const uint32_t pos = p.state->pos;
    if (pos >= p.max_tokens) {  // uniform: every workgroup leaves
        if (tid == 0 && h == 0 && chunk == 0) raise_error(p.err, kErrInput);
        return;
    }
    const float *cs = p.state->cs, *sn = p.state->sn;
    int e = norm_rope_head(p.qkv + h * kHead, p.q_norm, qv, tmp, red, cs, sn, p.rope, p.eps);
    e |= norm_rope_head(p.qkv + qw + kh * kHead, p.k_norm, kv, tmp, red, cs, sn, p.rope, p.eps);
    if (h % group == 0 && chunk == 0 && tid < kHead) {
        const size_t at = static_cast<size_t>(pos) * kw + kh * kHead + tid;
        const float v = round_f16(p.qkv[qw + kw + kh * kHead + tid]);
        if (!finite(v)) e |= kErrNonfinite;
        p.kcache[at] = f16_bits(kv[tid]);
        p.vcache[at] = f16_bits(v);
    }
    const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(kHead));
    const uint32_t t = chunk * kScoreChunk + tid;
    if (t <= pos) {
        // Four binary64 partial sums shorten the dependent chain; the terms are binary16
        // x binary16 products (exact in binary32) whose binary64 sums are exact, so the
        // split changes no bit of f16_dot's sequential sum.
        double s[4] = {0.0, 0.0, 0.0, 0.0};
        if (t == pos) {
            for (uint32_t d = 0; d < kHead; d += 4)
#pragma unroll
                for (int j = 0; j < 4; ++j) s[j] += static_cast<double>(qv[d + j] * kv[d + j]);
        } else {
            const uint4 *k = reinterpret_cast<const uint4 *>(p.kcache + static_cast<size_t>(t) * kw + kh * kHead);
            uint4 w[kHead / 8];
#pragma unroll
            for (uint32_t c = 0; c < kHead / 8; ++c) w[c] = k[c];
#pragma unroll
            for (uint32_t c = 0; c < kHead / 8; ++c) {
                const uint32_t w4[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    s[j] += static_cast<double>(qv[8 * c + 2 * j] * h2f(w4[j] & 0xffffu));
                    s[j] += static_cast<double>(qv[8 * c + 2 * j + 1] * h2f(w4[j] >> 16));
                }
            }
        }
        p.scores[static_cast<size_t>(h) * p.max_tokens + t] = static_cast<float>((s[0] + s[1]) + (s[2] + s[3])) * scale;
    }
    if (e && tid == 0) raise_error(p.err, e);
}

// Grid (heads, kHead / kValueDims), 1024 threads.  softmax_round_f16 (src/kernels.rs:
// 4431-4462) of the head's pos+1 scores -- every workgroup recomputes it -- then
// source_value_tile (src/kernels.rs:2971-3011) for this workgroup's kValueDims
// dimensions: out[d] = sum_t p_t v_t[d] in binary64.  Each term is a binary16 x
// binary16 product, exact in binary32, and a binary64 sum of such terms is exact
// unless they span more than 53 bits of magnitude (probabilities below 2^-24 are
// binary16 zeros), so summing the positions in 128 interleaved groups and then the
// groups does not change the result.
__global__ __launch_bounds__(1024) void k_attn_values(AttnArgs p) {
    __shared__ float redf[16];
    __shared__ double redd[16];
    __shared__ float prob[kMaxTokens];
    __shared__ double acc[16][kValueDims];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, nw = blockDim.x >> 6;
    const uint32_t h = blockIdx.x, d0 = blockIdx.y * kValueDims;
    const uint32_t kh = h / (p.heads / p.kv_heads), kw = p.kv_heads * kHead;
    const uint32_t pos = p.state->pos;
    if (pos >= p.max_tokens) return;  // reported by the score kernel
    const uint32_t n = pos + 1;
    const float *sc = p.scores + static_cast<size_t>(h) * p.max_tokens;
    float m = -__builtin_inff();
    bool bad = false;
    for (uint32_t i = tid; i < n; i += blockDim.x) {
        const float v = sc[i];
        bad |= (v != v) || v == __builtin_inff();
        m = fmaxf(m, v);
    }
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) m = fmaxf(m, __shfl_xor(m, k));
    if (lane == 0) redf[wave] = m;
    __syncthreads();
    m = redf[0];
    for (uint32_t w = 1; w < nw; ++w) m = fmaxf(m, redf[w]);
    if (__syncthreads_or(bad) || !finite(m)) {
        if (tid == 0 && blockIdx.y == 0) raise_error(p.err, kErrNonfinite);
        return;
    }
    double tot = 0.0;
    for (uint32_t i = tid; i < n; i += blockDim.x) {
        const float e = exp_f32(sc[i] - m);
        prob[i] = e;
        tot += static_cast<double>(e);
    }
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) tot += __shfl_xor(tot, k);
    if (lane == 0) redd[wave] = tot;
    __syncthreads();
    tot = 0.0;
    for (uint32_t w = 0; w < nw; ++w) tot += redd[w];
    const float inv = static_cast<float>(1.0 / tot);
    for (uint32_t i = tid; i < n; i += blockDim.x) prob[i] = round_f16(prob[i] * inv);
    __syncthreads();
    // Thread (g, q): positions g, g+128, ... of dimensions d0+4q .. d0+4q+3, eight rows
    // loaded per batch before any is used.
    const uint32_t g = tid / (kValueDims / 4), q = tid % (kValueDims / 4);
    double a[4] = {0.0, 0.0, 0.0, 0.0};
    const uint16_t *vb = p.vcache + kh * kHead + d0 + 4 * q;
    for (uint32_t i0 = g; i0 < n; i0 += 8 * kValueGroups) {
        uint2 w[8];
        float pr[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t i = i0 + k * kValueGroups;
            const bool in = i < n;
            w[k] = in ? *reinterpret_cast<const uint2 *>(vb + static_cast<size_t>(i) * kw) : make_uint2(0, 0);
            pr[k] = in ? prob[i] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            a[0] += static_cast<double>(pr[k] * h2f(w[k].x & 0xffffu));
            a[1] += static_cast<double>(pr[k] * h2f(w[k].x >> 16));
            a[2] += static_cast<double>(pr[k] * h2f(w[k].y & 0xffffu));
            a[3] += static_cast<double>(pr[k] * h2f(w[k].y >> 16));
        }
    }
    // A wavefront holds eight groups of the same eight quads (lane = 8 * group + quad):
    // fold them with lane shuffles, then the wavefronts through LDS.
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int k = 8; k <= 32; k <<= 1) a[j] += __shfl_xor(a[j], k);
    if (lane < kValueDims / 4)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[wave][4 * q + j] = a[j];
    __syncthreads();
    if (tid < kValueDims) {
        double t = acc[0][tid];
        for (uint32_t w = 1; w < nw; ++w) t += acc[w][tid];
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
// as decode_row_into does (src/kernels.rs:303, d * q).
__device__ __forceinline__ float q8_0_tiled_at(const uint8_t *__restrict__ w, uint64_t rows, uint32_t cols, uint32_t r,
                                               uint32_t i) {
    TiledFormat f;
    tiled_format(kQ8_0, &f);
    const uint64_t row_bytes = static_cast<uint64_t>(cols) / 128 * f.unit_bytes;
    const uint64_t tile = r / kTile;
    const uint32_t lr = r % kTile;
    const uint32_t trp = tile_rows_padded(rows, tile);
    const uint32_t u = i / 128, j = i % 128;
    const uint8_t *seg = w + tile * kTile * row_bytes + static_cast<uint64_t>(u) * trp * f.unit_bytes;
    const int8_t q = static_cast<int8_t>(seg[f.poff[j / 16] * trp + lr * 16 + j % 16]);
    const uint8_t *sp = seg + f.poff[8] * trp + lr * 8 + 2 * (j / 32);
    const float d = h2f(static_cast<uint32_t>(sp[0]) | (static_cast<uint32_t>(sp[1]) << 8));
    return d * static_cast<float>(q);
}

__global__ __launch_bounds__(256) void k_embed(const uint8_t *__restrict__ emb, uint64_t rows, uint32_t cols,
                                               DecodeState *__restrict__ st, RopeArgs rope, float *__restrict__ out) {
    const uint32_t token = st->token;
    rope_freqs(st, st->pos, rope);
    for (uint32_t i = threadIdx.x; i < cols; i += blockDim.x) out[i] = q8_0_tiled_at(emb, rows, cols, token, i);
}

// Greedy choice: the first index of the largest logit.  k_argmax_slices reduces
// contiguous slices to their (largest value, first index); k_argmax_embed reduces the
// slices in order, records the token in the state and the token history, advances
// the position, and writes the chosen token's embedding (the tied LM head row) as the
// next step's hidden state.
constexpr uint32_t kArgmaxGroups = 128;

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

__global__ __launch_bounds__(256) void k_argmax_slices(const float *__restrict__ logits, uint32_t vocab,
                                                       float *__restrict__ pval, uint32_t *__restrict__ pidx) {
    __shared__ float bv[4];
    __shared__ uint32_t bi[4];
    const uint32_t tid = threadIdx.x;
    const uint32_t span = (vocab + gridDim.x - 1) / gridDim.x;
    const uint32_t lo = blockIdx.x * span, hi = lo + span < vocab ? lo + span : vocab;
    float best = -__builtin_inff();
    uint32_t idx = 0xffffffffu;
    for (uint32_t i0 = lo + tid; i0 < hi; i0 += 8 * blockDim.x) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t i = i0 + k * blockDim.x;
            v[k] = i < hi ? logits[i] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t i = i0 + k * blockDim.x;
            if (i < hi && better(v[k], i, best, idx)) {
                best = v[k];
                idx = i;
            }
        }
    }
    reduce_best(best, idx, bv, bi);
    if (tid == 0) {
        pval[blockIdx.x] = best;
        pidx[blockIdx.x] = idx;
    }
}

__global__ __launch_bounds__(256) void k_argmax_embed(const float *__restrict__ pval, const uint32_t *__restrict__ pidx,
                                                      uint32_t vocab, const uint8_t *__restrict__ emb, uint32_t cols,
                                                      DecodeState *__restrict__ st, RopeArgs rope,
                                                      uint32_t *__restrict__ tokens, uint32_t max_steps,
                                                      float *__restrict__ out) {
    __shared__ float bv[4];
    __shared__ uint32_t bi[4];
    const uint32_t tid = threadIdx.x;
    const uint32_t pos = st->pos;  // read before thread 0 advances it
    float best = -__builtin_inff();
    uint32_t idx = 0xffffffffu;
    for (uint32_t g = tid; g < kArgmaxGroups; g += blockDim.x)
        if (better(pval[g], pidx[g], best, idx)) {
            best = pval[g];
            idx = pidx[g];
        }
    reduce_best(best, idx, bv, bi);
    const uint32_t token = idx < vocab ? idx : 0;  // a slice always holds a valid index
    if (tid == 0) {
        const uint32_t step = st->step;
        if (step < max_steps) tokens[step] = token;
        st->token = token;
        st->step = step + 1;
        st->pos = pos + 1;
    }
    rope_freqs(st, pos + 1, rope);
    for (uint32_t i = tid; i < cols; i += blockDim.x) out[i] = q8_0_tiled_at(emb, vocab, cols, token, i);
}

}  // namespace

size_t argmax_scratch_bytes() { return (sizeof(float) + sizeof(uint32_t)) * kArgmaxGroups; }

int launch_attention(const AttnArgs &a) {
    if (a.head_dim != kHead || a.rope > kHead || a.rope % 2 || a.kv_heads == 0 || a.heads % a.kv_heads ||
        a.max_tokens > kMaxTokens)
        return -2;
    const dim3 sg(a.heads, (a.max_tokens + kScoreChunk - 1) / kScoreChunk);
    hipLaunchKernelGGL(k_attn_scores, sg, dim3(256), 0, a.stream, a);
    hipLaunchKernelGGL(k_attn_values, dim3(a.heads, kHead / kValueDims), dim3(1024), 0, a.stream, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_lm_prep(const float *x, const float *w, uint32_t n, float eps, void *q8_out, int *err, hipStream_t s) {
    if (n % 32) return -2;
    hipLaunchKernelGGL(k_lm_prep, dim3(1), dim3(256), 0, s, x, w, n, eps, static_cast<Q8Block *>(q8_out), err);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_embed(const void *emb_tiled, uint64_t rows, uint32_t cols, DecodeState *st, const RopeArgs &rope,
                 float *out, hipStream_t s) {
    if (rope.rope > 2 * 64) return -2;
    hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), 0, s, static_cast<const uint8_t *>(emb_tiled), rows, cols, st,
                       rope, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_argmax_embed(const float *logits, uint32_t vocab, const void *emb_tiled, uint32_t cols, DecodeState *st,
                        const RopeArgs &rope, uint32_t *tokens, uint32_t max_steps, float *out, void *scratch,
                        hipStream_t s) {
    if (rope.rope > 2 * 64) return -2;
    float *pval = static_cast<float *>(scratch);
    uint32_t *pidx = reinterpret_cast<uint32_t *>(pval + kArgmaxGroups);
    hipLaunchKernelGGL(k_argmax_slices, dim3(kArgmaxGroups), dim3(256), 0, s, logits, vocab, pval, pidx);
    hipLaunchKernelGGL(k_argmax_embed, dim3(1), dim3(256), 0, s, pval, pidx, vocab,
                       static_cast<const uint8_t *>(emb_tiled), cols, st, rope, tokens, max_steps, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace prism
