// kernels.hpp -- host-side launchers of the gfx950 kernels (internal to libprism_hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prism {

// Device error bits raised by kernels, read back by prism_hip_sync.
constexpr int kErrNonfinite = 1;   // non-finite output / scale (PRISM_ERR_NONFINITE)
constexpr int kErrQuantRange = 2;  // activation quantizer overflow (PRISM_ERR_NONFINITE)
constexpr int kErrInput = 4;       // non-finite activation input (PRISM_ERR_NONFINITE)

// Launcher status: 0 on success, kLaunchUnsupported for a geometry the kernels do not
// cover, otherwise the hipError_t the launch left (positive).  hipGetLastError clears
// the error it returns, so a launcher reads it exactly once, here, and callers map the
// returned value instead of asking HIP again.
constexpr int kLaunchUnsupported = -2;
inline int launch_status() { return static_cast<int>(hipGetLastError()); }

// Activation-side formats consumed by the matvec kernels.  kActF32: f32 input the
// tiled kernels quantize in their prologue (contract in MatvecArgs::qcontract).
enum ActFormat : int { kActQ8K = 0, kActQ8 = 1, kActF32 = 2 };

// Which binary32 order a projection follows.
//   kind PTQ1 + Q8   : src (dot_q8_groups) or pinned (dot_q8_groups_pinned)
//   kind PTQ1 + Q8K  : dot_ptq1_q8k
//   kind PQ2  + Q8K  : unfused or fused (dot_pq2::<FUSED>)
//   kind PQ2  + Q8   : dot_q8_groups (odd group count)
//   kind Q2_K + Q8K  : kquants::dot
//   kind Q8_0 + Q8   : dot_legacy
struct MatvecArgs {
    uint32_t kind = 0;
    uint64_t cols = 0, rows = 0, row_bytes = 0;
    const uint8_t *w = nullptr;   // device, rows*row_bytes
    const uint8_t *w2 = nullptr;  // tiled only: FFN up matrix; out then receives SwiGLU(gate, up)
    const void *act = nullptr;    // device, token-major prepared blocks (or f32 rows)
    int act_format = kActQ8K;     // ActFormat
    int qcontract = 0;            // kActF32: Q8_K pinned flag, or Q8_0 contract (PRISM_Q8_*)
    bool qcontract_is_q8k = false;  // kActF32: the prologue quantizes to Q8_K
    uint32_t tokens = 1;
    int pinned = 0;               // pinned Q8 order (PTQ1) or fused FMA (PQ2 + Q8K); SwiGLU order
    float *out = nullptr;         // device, [tokens][rows]
    const float *residual = nullptr;  // tiled only: [tokens][rows], added to the outputs
    const float *norm_w = nullptr;    // tiled kActF32 only: RMSNorm weights applied before quantizing
    float eps = 0.0f;                 // RMSNorm epsilon
    void *q8_out = nullptr;           // tiled w2 only: the SwiGLU vector's Q8_0 blocks (rows % 32 == 0)
    int q8_contract = 0;              // their contract (PRISM_Q8_*)
    int *err = nullptr;           // device error flag
    // Tiled, one token, prepared activations, non-PTQ1 formats, row-tile kernel only: per
    // 64-row tile, the tile's largest output and the first row holding it, as
    // {float value, uint32_t row} pairs (TileBest), for the greedy choice.
    void *tile_best = nullptr;
    hipStream_t stream = nullptr;
    uint32_t cus = 256;           // compute units of the device
    void *scratch = nullptr;      // tiled only: tiled_scratch_bytes() of device memory
    size_t scratch_bytes = 0;
    // Scratch the caller can provide at most (a fixed buffer); kernel choices that need more
    // fall back to ones that need less.
    size_t scratch_cap = ~size_t(0);
};

// Return launch_status() values (0, kLaunchUnsupported, or a hipError_t).
// launch_matvec reads weights in the native row-major layout, launch_matvec_tiled in
// the 64-row tiled layout of tiled.hpp.
int launch_matvec(const MatvecArgs &a);
int launch_matvec_tiled(const MatvecArgs &a);
// Whether a kActF32 tiled call must be given prepared blocks instead (large matrices
// run a separate quantize kernel; the prologue would repeat it per workgroup).
bool tiled_needs_prepared(const MatvecArgs &a);
// Whether a kActF32 tiled call can quantize its input in the kernel's prologue at all (the
// split kernel's plan fits LDS); callers that always pass floats (the decoder) check it
// once instead of finding out at launch.
bool tiled_prologue_fits(const MatvecArgs &a);
// Device scratch a tiled call needs (the lane-ordered activations of a skinny batch).
size_t tiled_scratch_bytes(const MatvecArgs &a);
// Whether (kind, cols, rows) can be stored tiled on a device with `cus` compute units
// (every projection of it then has a tiled kernel), and the native -> tiled repack
// (the destination must hold tiled_bytes() and be zero-filled beforehand).
bool tiled_supported(uint32_t kind, uint64_t cols, uint64_t rows, uint32_t cus);
int launch_repack(const void *native, void *tiled, uint32_t kind, uint64_t cols, uint64_t rows, hipStream_t s);
// Tiled-prefill GEMM: quantizes x[M][cols] once and multiplies it by the tiled weights on
// the matrix cores; every output row is bit-identical to its own per-token matvec.  PTQ1
// in either contract on the f16 matrix cores (prefill.hip); Q2_K, PQ2, TQ1_0 and TQ2_0 (Q8_K
// activations) and Q8_0 on the int8 matrix cores (prefill_k.hip).
bool prefill_supported(uint32_t kind, uint64_t cols, uint64_t rows, int pinned, uint32_t tokens);
size_t prefill_scratch_bytes(uint32_t kind, uint64_t cols, uint32_t tokens);
// cus: the device's compute units (the block-split kernel runs one workgroup per CU).
int launch_prefill(uint32_t kind, const void *w_tiled, uint64_t cols, uint64_t rows, const float *x, uint32_t M,
                   int pinned, float *out, void *scratch, int *err, hipStream_t s, uint32_t cus);
// The same GEMMs on prepared activations (M tokens of act_stride bytes): Q8_0 blocks for PTQ1
// (pinned: the pinned chain) and Q8_0, Q8_K blocks for the other kinds (launch_prefill_k_blocks).
int launch_prefill_blocks(uint32_t kind, const void *w_tiled, uint64_t cols, uint64_t rows, const void *act,
                          uint32_t act_stride, uint32_t M, int pinned, float *out, void *scratch, int *err,
                          hipStream_t s, uint32_t cus);
bool prefill_k_supported(uint32_t kind, uint64_t cols, uint64_t rows, uint32_t tokens);
size_t prefill_k_scratch_bytes(uint64_t cols, uint32_t tokens);
int launch_prefill_k(uint32_t kind, const void *w_tiled, uint64_t cols, uint64_t rows, const float *x, uint32_t M,
                     int pinned, float *out, void *scratch, int *err, hipStream_t s);
// The same GEMM on prepared activations (M tokens of act_stride bytes): Q8_K blocks for
// Q2_K, PQ2 (pinned: the fused chain), TQ1_0 and TQ2_0, Q8_0 blocks for Q8_0; the blocks'
// codes, scales and sums are taken as they are.
int launch_prefill_k_blocks(uint32_t kind, const void *w_tiled, uint64_t cols, uint64_t rows, const void *act,
                            uint32_t act_stride, uint32_t M, int pinned, float *out, void *scratch, int *err,
                            hipStream_t s);
int launch_quantize_q8k(const float *x, uint64_t cols, uint32_t tokens, int pinned, void *out, int *err,
                        hipStream_t s);
int launch_quantize_q8_0(const float *x, uint64_t cols, uint32_t tokens, int contract, void *out, int *err,
                         hipStream_t s);
// h = SwiGLU(gate, up) elementwise (source or pinned order), n values per token.
int launch_swiglu(const float *gate, const float *up, float *h, uint64_t n, uint32_t tokens, int pinned, int *err,
                  hipStream_t s);
// out += residual, flagging non-finite sums.
int launch_add_residual(float *out, const float *residual, uint64_t n, int *err, hipStream_t s);
// Largest Hadamard block of the FFN chains (the block sits in one workgroup's LDS).
constexpr uint32_t kHadamardMaxBlock = 8192;
// The normalized blockwise Hadamard rotation of tokens rows of n values, in -> out.
int launch_hadamard(const float *in, float *out, uint64_t n, uint32_t tokens, uint32_t block, int *err,
                    hipStream_t s);
// lora_a_dot of a[0..n) with the SwiGLU vector h into *out (one workgroup).
int launch_lora_dot(const float *a, const float *h, uint32_t n, int pinned, float *out, int *err, hipStream_t s);
// p[0..n) = v with a kernel (safe inside captured graphs, unlike a memset node).
int launch_fill_i32(int *p, int v, uint32_t n, hipStream_t s);

// ---- decode step (decode.hip) ----
// Device-resident position / token / step counter of a decoder; the last kernel of a
// step advances it, so one captured graph serves every step.
struct DecodeState {
    uint32_t pos, token, step, pad;
    float cs[64], sn[64];  // RoPE cosines / sines of `pos` (rope_frequencies_mrope)
};
// RoPE geometry (src/graph.rs:6406-6431): rotated dimensions, M-RoPE sections and
// theta_scale = rope_base^(-2/rope) as binary32 powf.
struct RopeArgs {
    uint32_t rope;
    uint32_t sections[4];
    float theta_scale;
};
struct AttnArgs {
    const float *qkv;            // this token's projections: q [heads*D] | k [kv*D] | v [kv*D]
    const float *q_norm, *k_norm;  // per-head RMSNorm weights [D]
    uint16_t *kcache, *vcache;   // binary16 [max_tokens][kv*D]
    float *scores;               // [heads][max_tokens]
    float *maxima;               // [heads][attn_maxima_per_head(max_tokens)]: each score wavefront's largest
    float *out;                  // attended [heads*D]
    const DecodeState *state;
    uint32_t heads, kv_heads, head_dim, rope, max_tokens;
    float eps;                   // RMSNorm epsilon
    int *err;
    hipStream_t stream;
};
// q/k norm + RoPE + KV append + scores, then softmax + values: two launches
// (launch_attn_scores, then launch_attn_values).
int launch_attention(const AttnArgs &a);
// Slots of AttnArgs::maxima per head: one per 16-position wavefront of a 64-position score
// workgroup.
uint32_t attn_maxima_per_head(uint32_t max_tokens);
int launch_attn_scores(const AttnArgs &a);
int launch_attn_values(const AttnArgs &a);
// Final RMSNorm + Q8_0 (source) quantization of n values into q8_out.
int launch_lm_prep(const float *x, const float *w, uint32_t n, float eps, void *q8_out, int *err, hipStream_t s);
// out = dequantized row state->token of the tiled Q8_0 matrix [rows][cols]; the state's
// RoPE frequencies are set for state->pos.
int launch_embed(const void *emb_tiled, uint64_t rows, uint32_t cols, DecodeState *st, const RopeArgs &rope,
                 float *out, hipStream_t s);
// One 64-row tile's largest output and the first row that holds it.
struct TileBest {
    float value;
    uint32_t row;
};
// Greedy token from the LM head's TileBest pairs (MatvecArgs::tile_best, one per 64-row
// tile of the vocabulary), recorded and advanced in the state (with the RoPE frequencies
// of the new position), and its embedding (row of the tiled Q8_0 matrix [vocab][cols])
// written to out; one launch.
// Largest vocabulary the greedy launch reduces (4096 tiles of 64 rows).
constexpr uint64_t kGreedyMaxVocab = 262144;
size_t argmax_scratch_bytes(uint64_t vocab);
int launch_argmax_embed(const TileBest *best, uint32_t vocab, const void *emb_tiled, uint32_t cols, DecodeState *st,
                        const RopeArgs &rope, uint32_t *tokens, uint32_t max_steps, float *out, hipStream_t s);


}  // namespace prism
