/*
 * prism_hip.h -- C ABI of the MI355X (gfx950) packed quantized matmul path.
 *
 * This library replaces the device side of the reference's projection-executor
 * boundary (trait Pq2ProjectionExecutor, src/kernels/projection.rs:16-355) and the
 * GGML MUL_MAT backend op for packed weights (src/backend/ops.rs:444-466).  Every
 * entry point takes plain pointers and sizes; no C++ or torch type crosses it.
 *
 * Conventions (mirroring src/kernels/projection.rs:8-15,46-57,797-806,859-866):
 *  - Calls are synchronous unless the name ends in _device; host pointers are only
 *    read during the call and never retained.
 *  - Every projection writes exactly rows*tokens f32 values.  On any error the
 *    output is zero-filled (the reference clears its Vec) and a negative code is
 *    returned; nothing is replayed on the CPU.
 *  - A non-finite output, weight scale or activation is PRISM_ERR_NONFINITE.
 *  - A device fault latches: every later supports*() returns 0 and calls fail
 *    with PRISM_ERR_DEVICE_FAULT (tools/adreno-vulkan/src/executor.rs:1507-1530).
 *  - One context per host thread; contexts create no host threads.  Streams are
 *    internal (default priority).
 *
 * Arithmetic contract: results are bit-identical to the reference's scalar CPU
 * kernels for the same prepared activations and the same source/pinned choice
 * (src/kernels.rs:941-1248, src/kernels/kquants.rs:162-197,346-430).  SwiGLU
 * outputs follow libm exp and are compared with a tolerance.
 */
#ifndef PRISM_HIP_H
#define PRISM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Tensor kinds: GGML type ids (src/kernels.rs:75-87, src/backend.rs:99-141). */
#define PRISM_KIND_Q8_0 8u
#define PRISM_KIND_Q2_K 10u
#define PRISM_KIND_TQ1_0 34u /* 256 ternary weights in 54 bytes (src/kernels/tquants.rs:17-23) */
#define PRISM_KIND_TQ2_0 35u /* 256 ternary weights in 66 bytes */
#define PRISM_KIND_PQ2 142u
#define PRISM_KIND_PTQ1 143u

/* Error codes. */
#define PRISM_OK 0
#define PRISM_ERR_INVALID_INPUT (-1)
#define PRISM_ERR_RESOURCE (-2)
#define PRISM_ERR_NONFINITE (-3)
#define PRISM_ERR_DEVICE_FAULT (-4)
#define PRISM_ERR_UNSUPPORTED (-5)
#define PRISM_ERR_CANCELLED (-6)

/* Activation paths for prism_hip_supports (project / project_q8 / project_f32). */
#define PRISM_PATH_Q8K 0
#define PRISM_PATH_Q8 1
#define PRISM_PATH_F32 2

/* Q8_0 activation contracts (src/kernels.rs:552-617). */
#define PRISM_Q8_SOURCE 0        /* public matvec: d=max/127, round half away     */
#define PRISM_Q8_PINNED 1        /* pinned generic: same d, ties to even           */
#define PRISM_Q8_PINNED_NATIVE 2 /* pinned PTQ1: d=max*0x3c010204, inv=127/max, RNE */

/* Q8_K activation block, tools/ternary/src/lib.rs:27-39 (#[repr(C)], 292 bytes). */
typedef struct prism_q8k_block {
    float scale;
    int8_t values[256];
    int16_t sums[16];
} prism_q8k_block;

/* Prepared Q8_0 activation block, src/kernels.rs:528-535 (in-memory form, 40 bytes). */
typedef struct prism_q8_block {
    float scale; /* binary16-rounded */
    float sum;   /* binary16-rounded scaled code sum (unused by these dots) */
    int8_t values[32];
} prism_q8_block;

typedef struct prism_hip_ctx prism_hip_ctx;
typedef int64_t prism_weight_id; /* >= 1 on success, negative error code otherwise */

/* ---- lifecycle -------------------------------------------------------------- */

/* Opens device `device` (HIP ordinal).  max_resident_bytes bounds the weights the
 * context may own (0 = no bound).  flags must be 0.  Returns NULL on failure. */
prism_hip_ctx *prism_hip_create(int device, uint64_t max_resident_bytes, uint32_t flags);
void prism_hip_destroy(prism_hip_ctx *ctx);
/* Pq2ProjectionExecutor::identity (src/kernels/projection.rs:17-18). */
const char *prism_hip_identity(const prism_hip_ctx *ctx);
/* Message of the last failed call on this context ("" if none). */
const char *prism_hip_last_error(const prism_hip_ctx *ctx);
/* 1 once a device fault has latched. */
int prism_hip_faulted(const prism_hip_ctx *ctx);
/* Test hook with no counterpart in the reference's trait: latches the context's device
 * fault from the host, as a lost device or a failed wait would (the Vulkan executor's
 * latch, tools/adreno-vulkan/src/executor.rs:1507-1530), so that the latched behaviour
 * (every supports*() 0, operation_capacity 0, every call PRISM_ERR_DEVICE_FAULT with its
 * output cleared) can be tested without faulting a GPU.  Irreversible for this context;
 * other contexts are unaffected.  Returns PRISM_OK (PRISM_ERR_INVALID_INPUT for NULL). */
int prism_hip_inject_fault(prism_hip_ctx *ctx);
/* Pq2ProjectionExecutor::operation_capacity (projection.rs:20-28): 0 when faulted,
 * UINT64_MAX otherwise (submissions are not rationed). */
uint64_t prism_hip_operation_capacity(const prism_hip_ctx *ctx);
/* Pq2ProjectionExecutor::operation_count (projection.rs:30-36): cols*rows for a
 * supported projection, -1 (unknown) otherwise. */
int64_t prism_hip_operation_count(const prism_hip_ctx *ctx, uint32_t kind, uint64_t cols, uint64_t rows);

/* Work counted by one context over its lifetime, as MatvecStatistics counts it for one
 * scratch owner (src/kernels.rs:1792-1865).  Counts include failed work, saturate at
 * UINT64_MAX and survive errors, faults and weight releases; they describe dispatch,
 * not timing.
 *  - preparations: activation preparations attempted by the F32 entry points (one per
 *    call, shared by the call's matrices, as siblings share one prepared activation)
 *    and by the quantize entry points;
 *  - preparation_failures: those rejected before a matrix could be attempted (a null
 *    or empty input, an extent the quantizer cannot take); no matrix attempt is
 *    counted for them.  A non-finite input found by the device-side quantizer fails
 *    the dispatched call instead (it is counted as a failed device operation);
 *  - matrix_attempts / matrix_successes: matrices of every projection call, grouped
 *    matrices counted individually (a gate/up/down chain is three);
 *  - rejected_before_dispatch: attempts rejected before any launch (unknown weight,
 *    ineligible geometry, extent mismatch, latched fault);
 *  - device_operations: attempts dispatched to the GPU, including later failures (the
 *    reference's scalar_operations / neon_operations: this library has one backend);
 *  - grouped_dispatches: single calls submitting two or more matrices together
 *    (grouped_row_dispatches). */
typedef struct prism_hip_statistics {
    uint64_t preparations;
    uint64_t preparation_failures;
    uint64_t matrix_attempts;
    uint64_t matrix_successes;
    uint64_t rejected_before_dispatch;
    uint64_t device_operations;
    uint64_t grouped_dispatches;
} prism_hip_statistics;
/* The most recent projection call's record, as MatvecDiagnostics keeps it for the most
 * recent matrix attempt (src/kernels.rs:1725-1790): dispatched = launched after the
 * weight, activation and output checks; succeeded = complete, finite output returned.
 * Both 0 after a call rejected before dispatch. */
typedef struct prism_hip_diagnostics {
    int32_t dispatched;
    int32_t succeeded;
} prism_hip_diagnostics;
/* Copy the counters / the last record; PRISM_ERR_INVALID_INPUT for a null argument. */
int prism_hip_get_statistics(const prism_hip_ctx *ctx, prism_hip_statistics *out);
int prism_hip_get_diagnostics(const prism_hip_ctx *ctx, prism_hip_diagnostics *out);

/* Cancellation shared with the request owner (src/runtime.rs:35-60): registers a
 * caller-owned flag, read with acquire ordering, nonzero meaning cancelled; NULL
 * unregisters.  Every projection, quantize and decoder call checks it on entry and
 * prism_hip_decoder_generate between steps; with a flag registered a generate keeps at
 * most two steps in flight, so at most two complete after the flag is set (the
 * reference's "an executing scalar operation completes first").  A cancelled call waits
 * for the work it enqueued, zero-fills its outputs and returns PRISM_ERR_CANCELLED.  The
 * flag stays cancelled until its owner clears it, and must outlive the registration. */
int prism_hip_set_cancellation(prism_hip_ctx *ctx, const int32_t *flag);

/* ---- eligibility -------------------------------------------------------------- */

/* supports / supports_q8 / supports_f32 (projection.rs:38-44,59-66,89-92), decided
 * from geometry alone before any launch.  Returns 1 or 0. */
int prism_hip_supports(const prism_hip_ctx *ctx, uint32_t kind, uint64_t cols, uint64_t rows, int path);

/* A tensor as the trait's eligibility queries see it: Tensor's kind and dimensions
 * [cols, rows] (src/model.rs:184-193). */
typedef struct prism_tensor_desc {
    uint32_t kind;
    uint64_t cols, rows;
} prism_tensor_desc;
/* supports_f32_group (projection.rs:112-114): 1..8 siblings that can share one F32
 * input -- every member supports F32, one input width, and one activation contract
 * under both pinned settings.  Returns 1 or 0. */
int prism_hip_supports_f32_group(const prism_hip_ctx *ctx, const prism_tensor_desc *tensors, uint32_t n);
/* supports_f32_ffn_swiglu (projection.rs:212-214): gate and up of one packed kind and
 * one geometry [ffn][hidden]. */
int prism_hip_supports_f32_ffn_swiglu(const prism_hip_ctx *ctx, const prism_tensor_desc *gate,
                                      const prism_tensor_desc *up);
/* supports_f32_ffn_chain (projection.rs:261-263): tensors[3] = gate, up [ffn][hidden]
 * and down [hidden][ffn], one packed kind.  The chain has no Hadamard transform. */
int prism_hip_supports_f32_ffn_chain(const prism_hip_ctx *ctx, const prism_tensor_desc *tensors);
/* supports_f32_ffn_chain_lora (projection.rs:290-296; trait default false): the FFN
 * chain's own eligibility -- the rank-one A dot adds no geometry of its own. */
int prism_hip_supports_f32_ffn_chain_lora(const prism_hip_ctx *ctx, const prism_tensor_desc *tensors);
/* supports_tile_tokens (projection.rs:265-269; trait default false): multi-token tiles run batched on the
 * device (one weight read per batch of tokens).  1 unless faulted. */
int prism_hip_supports_tile_tokens(const prism_hip_ctx *ctx);

/* ---- weights ------------------------------------------------------------------ */

/* Upload-or-lookup of a packed row-major tensor [rows][cols] (bytes must equal
 * rows*cols/QK*block_bytes, src/kernels.rs:121-142).  `key` identifies the tensor
 * (the reference keys device copies by tensor identity,
 * tools/adreno-vulkan/src/executor.rs:686-760): acquiring an existing key with the
 * same geometry returns its id without copying. */
prism_weight_id prism_hip_weight_acquire(prism_hip_ctx *ctx, uint64_t key, uint32_t kind, uint64_t cols,
                                         uint64_t rows, const void *host, uint64_t bytes);
/* As prism_hip_weight_acquire, from native bytes already in device memory (read
 * only during the call; the context keeps its own copy). */
prism_weight_id prism_hip_weight_acquire_device(prism_hip_ctx *ctx, uint64_t key, uint32_t kind, uint64_t cols,
                                                uint64_t rows, const void *device_ptr, uint64_t bytes);
/* Registers caller-owned device memory holding the packed tensor (no copy).  The
 * caller keeps it alive until release. */
prism_weight_id prism_hip_weight_wrap_device(prism_hip_ctx *ctx, uint32_t kind, uint64_t cols, uint64_t rows,
                                             const void *device_ptr, uint64_t bytes);
/* The fast layout in caller-owned memory: the caller's allocator owns the device buffer
 * (BufferType{alignment, maximum} / GraphAllocator sizing, src/backend/allocator.rs:10-50)
 * and the context only references it.
 * prism_hip_weight_tiled_bytes: device bytes of the 64-row tiled image of a tensor, or 0
 *   when the tensor has no tiled layout on this device (it then runs on the native-layout
 *   kernels: use prism_hip_weight_wrap_device).
 * prism_hip_weight_repack_tiled: writes that image from native bytes in device memory
 *   (read only during the call) into tiled_dev, which holds exactly tiled_bytes; synchronous.
 * prism_hip_weight_wrap_tiled: registers a buffer holding that image (no copy); the caller
 *   keeps it alive until release.  Projections of it run the tiled kernels. */
uint64_t prism_hip_weight_tiled_bytes(const prism_hip_ctx *ctx, uint32_t kind, uint64_t cols, uint64_t rows);
int prism_hip_weight_repack_tiled(prism_hip_ctx *ctx, uint32_t kind, uint64_t cols, uint64_t rows,
                                  const void *native_dev, uint64_t native_bytes, void *tiled_dev, uint64_t tiled_bytes);
prism_weight_id prism_hip_weight_wrap_tiled(prism_hip_ctx *ctx, uint32_t kind, uint64_t cols, uint64_t rows,
                                            const void *tiled_dev, uint64_t tiled_bytes);
int prism_hip_weight_release(prism_hip_ctx *ctx, prism_weight_id w);
int prism_hip_weight_release_all(prism_hip_ctx *ctx);
uint64_t prism_hip_resident_bytes(const prism_hip_ctx *ctx);

/* ---- executor projections (host pointers, synchronous) ------------------------ */

/* Pq2ProjectionExecutor::project (projection.rs:46-57): PQ2 with cols%256==0 and
 * prepared Q8_K codes, `fused` selects mul_add accumulation.  Also accepts Q2_K
 * (kquants::dot) and PTQ1 (dot_ptq1_q8k, src/kernels.rs:999-1037).  act holds
 * tokens*cols/256 blocks, each with the sums of its codes in `sums` (as every Q8_K
 * quantizer writes them; Q2_K reads them); out receives [tokens][rows]. */
int prism_hip_project_q8k(prism_hip_ctx *ctx, prism_weight_id w, const prism_q8k_block *act, uint64_t nblocks,
                          uint32_t tokens, int fused, float *out);
/* Pq2ProjectionExecutor::project_q8 (projection.rs:68-87): PTQ1 or odd-group PQ2
 * with prepared Q8_0 codes; `pinned` selects the four-lane FMA order for PTQ1.
 * Also accepts Q8_0 weights (dot_legacy, src/kernels.rs:1204-1248). */
int prism_hip_project_q8(prism_hip_ctx *ctx, prism_weight_id w, const prism_q8_block *act, uint64_t nblocks,
                         uint32_t tokens, int pinned, float *out);
/* Pq2ProjectionExecutor::project_f32 (projection.rs:94-107) generalised to every
 * kind: quantizes on the GPU with the activation contract matvec_into would use
 * (ActivationContract::for_tensor, src/kernels.rs:1663-1673) then projects.
 * x holds tokens*cols floats. */
int prism_hip_project_f32(prism_hip_ctx *ctx, prism_weight_id w, const float *x, uint32_t tokens, int pinned,
                          float *out);
/* project_f32_group (projection.rs:115-130): n (1..8) siblings sharing one input. */
int prism_hip_project_f32_group(prism_hip_ctx *ctx, const prism_weight_id *ws, uint32_t n, const float *x,
                                int pinned, float *const *outs);
/* The group over a tile of tokens: x holds tokens*cols floats, outs[i] receives
 * [tokens][rows_i]; every row equals that token's own project_f32_group.
 * project_f32_pair_tokens / project_f32_triple_tokens (projection.rs:158-210) are the
 * n = 2 and n = 3 cases. */
int prism_hip_project_f32_group_tokens(prism_hip_ctx *ctx, const prism_weight_id *ws, uint32_t n, const float *x,
                                       uint32_t tokens, int pinned, float *const *outs);
int prism_hip_project_f32_pair_tokens(prism_hip_ctx *ctx, const prism_weight_id *ws, const float *x, uint32_t tokens,
                                      int pinned, float *out_a, float *out_b);
int prism_hip_project_f32_triple_tokens(prism_hip_ctx *ctx, const prism_weight_id *ws, const float *x,
                                        uint32_t tokens, int pinned, float *out_a, float *out_b, float *out_c);
/* project_f32_ffn_swiglu (projection.rs:206-222): out[ffn] = SwiGLU(gate(x), up(x)). */
int prism_hip_ffn_swiglu(prism_hip_ctx *ctx, prism_weight_id gate, prism_weight_id up, const float *x, int pinned,
                         float *out);
/* project_f32_ffn_chain (src/kernels/projection.rs:271-290):
 * out[hidden] = down(H(SwiGLU(gate(x), up(x)))) (+ residual if non-NULL).  Gate, up
 * and down share one packed kind (PQ2, PTQ1, Q2_K, Q8_0, TQ1_0 or TQ2_0).
 * hadamard_block is the call's hadamard_block_size: 0 (None) or 1 leaves H the identity;
 * otherwise H is the normalized Sylvester-Walsh-Hadamard transform of every
 * hadamard_block consecutive SwiGLU values (src/kernels.rs:3952-3987: butterflies with
 * half = 1, 2, 4, ..., (l, r) -> (l + r, l - r) in binary32, then each value times
 * 1/sqrt(block)), the rotation the decoder applies ahead of a rotated down projection
 * (src/graph.rs:1810-1831 picks the block, signs all +1).  A block that is not a power of
 * two up to 8192 dividing the FFN width is PRISM_ERR_INVALID_INPUT. */
int prism_hip_ffn_chain(prism_hip_ctx *ctx, prism_weight_id gate, prism_weight_id up, prism_weight_id down,
                        const float *x, const float *residual, uint32_t hadamard_block, int pinned, float *out);
/* project_f32_ffn_chain_lora (src/kernels/projection.rs:303-323, called from
 * matvec_ffn_chain_lora_with_executor :653-697): the chain of prism_hip_ffn_chain
 * (hadamard_block as there), plus *lora_dot = lora_a . SwiGLU(gate(x), up(x)) -- the
 * unrotated SwiGLU vector, as src/graph/prefill_ffn_tests.rs:554-590 orders it -- with lora_a[ffn]
 * (ffn = down's columns), in lora_a_dot's arithmetic (src/kernels.rs:2336-2357): pinned with
 * ffn % 16 == 0, sixteen binary32 FMA lanes combined as pinned_gdn::dot_scalar
 * (src/kernels/pinned_gdn.rs:205-230); otherwise the binary32 products summed in binary64
 * in index order (float_dot, src/kernels.rs:1256-1273).  A non-finite lora_a is rejected
 * before any launch (PRISM_ERR_INVALID_INPUT); a non-finite dot or output fails the call.
 * On any error out is zero-filled and *lora_dot is 0. */
int prism_hip_ffn_chain_lora(prism_hip_ctx *ctx, prism_weight_id gate, prism_weight_id up, prism_weight_id down,
                             const float *x, const float *residual, uint32_t hadamard_block, const float *lora_a,
                             int pinned, float *out, float *lora_dot);
/* project_f32_ffn_swiglu_tokens (projection.rs:239-259) and project_f32_ffn_chain_tokens
 * (projection.rs:328-355, hadamard_block as for prism_hip_ffn_chain): x [tokens][hidden], residual
 * (or NULL) and out [tokens][hidden] (SwiGLU: out [tokens][ffn]).  Gate and up run as
 * one sibling group over all tokens, so each weight is read once per batch of tokens;
 * every row equals that token's single-token chain. */
int prism_hip_ffn_swiglu_tokens(prism_hip_ctx *ctx, prism_weight_id gate, prism_weight_id up, const float *x,
                                uint32_t tokens, int pinned, float *out);
int prism_hip_ffn_chain_tokens(prism_hip_ctx *ctx, prism_weight_id gate, prism_weight_id up, prism_weight_id down,
                               const float *x, const float *residual, uint32_t tokens, uint32_t hadamard_block,
                               int pinned, float *out);
/* Tiled prefill (src/kernels/prefill.rs:200-725): X[tokens][cols] -> out[tokens][rows];
 * every token row is bit-identical to its own project_f32. */
int prism_hip_prefill(prism_hip_ctx *ctx, prism_weight_id w, const float *x, uint32_t tokens, int pinned,
                      float *out);

/* ---- backend op ----------------------------------------------------------------- */

/* ggml_mul_mat for a packed A (src/backend/call.rs:808-823, ops.rs:444-466): for each
 * of the ncols activation columns b[j][cols], out[j][rows] = kernels::matvec(A, b[j])
 * (public source contract). */
int prism_hip_mul_mat(prism_hip_ctx *ctx, prism_weight_id a, const float *b, uint32_t ncols, float *out);

/* ---- device-pointer dispatch (stream ordered; check with prism_hip_sync) -------- */

/* Quantize tokens*cols device floats into device Q8_K blocks / Q8_0 blocks. */
int prism_hip_quantize_q8k_device(prism_hip_ctx *ctx, const float *x, uint64_t cols, uint32_t tokens, int pinned,
                                  prism_q8k_block *out, void *stream);
int prism_hip_quantize_q8_device(prism_hip_ctx *ctx, const float *x, uint64_t cols, uint32_t tokens, int contract,
                                 prism_q8_block *out, void *stream);
/* Project device activations (path = PRISM_PATH_Q8K or PRISM_PATH_Q8 blocks, or
 * PRISM_PATH_F32 floats quantized on the fly) into device out[tokens][rows]. */
int prism_hip_project_device(prism_hip_ctx *ctx, prism_weight_id w, int path, const void *act, uint32_t tokens,
                             int pinned, float *out, void *stream);
/* FFN chain on device pointers (h may be NULL; when set it receives the unrotated SwiGLU
 * vector; hadamard_block as for prism_hip_ffn_chain).  down == 0 is project_f32_ffn_swiglu:
 * out receives the SwiGLU vector (ffn floats) and hadamard_block is ignored. */
int prism_hip_ffn_chain_device(prism_hip_ctx *ctx, prism_weight_id gate, prism_weight_id up, prism_weight_id down,
                               const float *x, const float *residual, uint32_t hadamard_block, int pinned,
                               float *out, float *h, void *stream);
/* prism_hip_project_device without any device allocation: every scratch buffer the
 * call's kernels use (the quantized activation, the skinny batch's lane-ordered copy,
 * the prefill token codes) is carved from one fixed, file-scope device array of
 * PRISM_NOALLOC_SCRATCH_BYTES per GPU, allocated with the code object when the library
 * first runs on that GPU and held until the process ends; the call itself never calls
 * hipMalloc or hipFree.  A call needing more scratch than that returns
 * PRISM_ERR_UNSUPPORTED before launching anything.  Every call on one GPU (from any
 * context) shares the array: calls that overlap on one GPU race, so order them on one
 * stream.  Nothing in the array needs to start at zero: each kernel reads only what an
 * earlier kernel of the same call wrote.  No counterpart in the reference: this is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops).  Arguments and results as prism_hip_project_device. */
#define PRISM_NOALLOC_SCRATCH_BYTES (16u << 20)
int prism_hip_project_device_noalloc(prism_hip_ctx *ctx, prism_weight_id w, int path, const void *act,
                                     uint32_t tokens, int pinned, float *out, void *stream);
/* Waits for `stream` (NULL = the context stream) and reports any error the
 * device-side checks raised since the last sync (non-finite values, scale
 * overflow).  Clears the device error flag. */
int prism_hip_sync(prism_hip_ctx *ctx, void *stream);
/* The context's internal stream (a hipStream_t), for ordering caller work. */
void *prism_hip_stream(prism_hip_ctx *ctx);

/* ---- full-attention decode step ---------------------------------------------------
 * A resident decoder over a context: the layer loop of the reference's Qwen35 graph
 * for full-attention layers (src/graph.rs:3870-3995) in the source arithmetic, with
 * every linear layer PTQ1 on the packed-matvec kernels and a tied Q8_0 LM head /
 * token embedding.  Per layer: RMSNorm fused into the q/k/v projection (one PTQ1
 * matrix of (heads + 2*kv_heads)*head_dim rows), per-head q/k RMSNorm + RoPE +
 * binary16 rounding, binary16 KV cache append, attention (f16 dots and value sums
 * in binary64, softmax_round_f16), o projection + residual, post-norm fused into the
 * gate/up/SwiGLU launch, down + residual; then the final norm, the LM head and the
 * greedy choice, whose embedding feeds the next step.  The geometry has no attention
 * output gate (the query projection is heads*head_dim wide).  No counterpart C API
 * exists in the reference: this is the reference's own graph code, restated around
 * the executor entry points above. */
typedef struct prism_hip_decoder prism_hip_decoder;
typedef struct {
    uint64_t hidden, ffn, heads, kv_heads, head_dim, rope, vocab, layers, max_tokens;
    uint64_t rope_sections[4]; /* M-RoPE sections; text positions use sectors 0..2 */
    float rope_base, eps;
} prism_decoder_geometry;

/* head_dim must be 128; hidden, ffn multiples of 128; max_tokens <= 8192; vocab <= 262144.
 * max_steps bounds one generate(). */
prism_hip_decoder *prism_hip_decoder_create(prism_hip_ctx *ctx, const prism_decoder_geometry *g, uint32_t max_steps);
void prism_hip_decoder_destroy(prism_hip_decoder *d);
/* Host tensors of layer l, native layouts: qkv PTQ1 [(heads+2kv)*head_dim][hidden]
 * (q rows, then k, then v), o PTQ1 [hidden][heads*head_dim], gate/up PTQ1
 * [ffn][hidden], down PTQ1 [hidden][ffn]; norm/post_norm [hidden], q_norm/k_norm
 * [head_dim] f32. */
int prism_hip_decoder_set_layer(prism_hip_decoder *d, uint32_t layer, const uint8_t *qkv, const uint8_t *o,
                                const uint8_t *gate, const uint8_t *up, const uint8_t *down, const float *norm,
                                const float *post_norm, const float *q_norm, const float *k_norm);
/* Binary16 cache rows [tokens][kv_heads*head_dim] of layer l (positions 0..tokens-1). */
int prism_hip_decoder_set_cache(prism_hip_decoder *d, uint32_t layer, const uint16_t *k, const uint16_t *v,
                                uint64_t tokens);
/* Tied LM head / embedding, Q8_0 [vocab][hidden] native rows, and the final norm. */
int prism_hip_decoder_set_head(prism_hip_decoder *d, const uint8_t *lm_head, const float *output_norm);
/* Runs `steps` greedy decode steps from `token` at position `pos`: tokens_out[steps]
 * receives the chosen tokens, logits_out (NULL or steps*vocab floats) every step's
 * logits, seconds (NULL allowed) the device time of the steps.  use_graph replays
 * one captured HIP graph per step. */
int prism_hip_decoder_generate(prism_hip_decoder *d, uint32_t token, uint64_t pos, uint32_t steps, int use_graph,
                               uint32_t *tokens_out, float *logits_out, double *seconds);

/* Measurement hooks of the decoder (no counterpart in the reference; for benchmarks and
 * profiles).  A step's launches form nine families, in step order: "qkv", "attn_scores",
 * "attn_values", "o", "gate_up", "down" (per layer), then "lm_prep", "lm_head", "greedy". */
#define PRISM_DECODER_FAMILIES 9
typedef struct {
    const char *name;  /* family name (static storage) */
    uint32_t launches; /* launches timed */
    double total_us;   /* their summed event-bracketed times */
    uint64_t bytes;    /* algorithmic bytes of one launch: packed weights at native size, f32 activations and
                          outputs, Q8_0 blocks at 34 bytes, binary16 cache rows read and appended */
} prism_decoder_launch_time;
/* Runs `steps` greedy steps from (token, pos) with launches issued one by one (no graph)
 * and a HIP event recorded on the context stream before every launch and after the
 * last; stats[PRISM_DECODER_FAMILIES] receives, per family, the launches timed, the
 * summed times between consecutive events (each launch with its dispatch gap) and the
 * bytes of one launch at position pos.  The decoder state advances as in generate. */
int prism_hip_decoder_profile(prism_hip_decoder *d, uint32_t token, uint64_t pos, uint32_t steps,
                              prism_decoder_launch_time *stats);
/* Launches one family (not "greedy") `reps` times per layer back to back at the
 * decoder's current position, cycling through the layers (the head's families run
 * `reps` times), with HIP events around the whole run: *avg_us receives the mean time
 * per launch and *bytes (may be NULL) the algorithmic bytes of one launch.  The
 * families other than "greedy" only recompute what a step at that position computes. */
int prism_hip_decoder_time_family(prism_hip_decoder *d, const char *family, uint32_t reps, double *avg_us,
                                  uint64_t *bytes);

/* ---- GGUF v3 weights (tools/gguf) --------------------------------------------------
 * A bounded reader of the GGUF header, metadata table and tensor index: the checks of
 * read_index (tools/gguf/src/stream.rs:349-657) -- magic, version, counts, unique keys
 * and names, UTF-8 without interior NUL, a power-of-two general.alignment (default 32),
 * 1..4 nonzero dimensions, known types (PQ2 142 / PTQ1 143 only in the Prism dialect),
 * block-complete first dimensions, aligned offsets, in-file non-overlapping extents and
 * the metadata budget.  Tensors and metadata keys enumerate in name order.  Host code:
 * none of these functions touches the GPU except prism_hip_weight_from_gguf. */
typedef struct prism_gguf prism_gguf;
/* IndexPolicy (stream.rs:44-131); prism_gguf_default_policy fills IndexPolicy::new(). */
typedef struct {
    int allow_v2, allow_zero_tensors, allow_zero_metadata;
    uint64_t max_file_bytes, max_tensors, max_metadata, metadata_budget;
    uint64_t max_key_bytes, max_string_bytes, max_array_string_bytes;
    uint64_t max_retained_string_array_bytes; /* 0 = unlimited */
    uint64_t max_array_items, max_alignment;
    int allow_positive_i32_alignment, reject_nonfinite_floats, reject_interior_nul_keys,
        reject_interior_nul_strings;
    uint64_t kv_overhead_bytes, string_overhead_bytes, tensor_overhead_bytes;
    int charge_skipped_scalar_arrays;
    int prism_dialect;        /* admit PQ2_0 (142) / PTQ1_0 (143) */
    int retain_string_arrays; /* keep string-array elements (else validated and skipped) */
    const uint32_t *allowed_types; /* optional allowlist of tensor type ids */
    size_t allowed_type_count;
} prism_gguf_policy;
/* IndexedTensor (stream.rs:185-199). */
typedef struct {
    uint32_t type_id, ndims;
    uint64_t dims[4]; /* GGML order: dims[0] is the packed (column) axis */
    uint64_t relative_offset, offset, bytes, elements;
} prism_gguf_tensor;

void prism_gguf_default_policy(prism_gguf_policy *policy);
/* policy NULL = defaults.  Errors: PRISM_ERR_INVALID_INPUT (message in prism_gguf_last_error). */
int prism_gguf_open(const char *path, const prism_gguf_policy *policy, prism_gguf **out);
void prism_gguf_close(prism_gguf *g);
const char *prism_gguf_last_error(void); /* this thread's last GGUF failure */
int prism_gguf_summary(const prism_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_offset,
                       uint64_t *tensor_count, uint64_t *metadata_count, uint64_t *remaining_budget);
int prism_gguf_tensor_at(const prism_gguf *g, uint64_t index, const char **name, prism_gguf_tensor *info);
int prism_gguf_find_tensor(const prism_gguf *g, const char *name, prism_gguf_tensor *info);
/* type_id: GGUF value type (8 string, 9 array); arrays report element type and count,
 * and retained = 0 when their elements were validated and skipped. */
int prism_gguf_metadata_at(const prism_gguf *g, uint64_t index, const char **key, uint32_t *type_id,
                           uint32_t *element_type_id, uint64_t *count, int *retained);
int prism_gguf_metadata_int(const prism_gguf *g, const char *key, int64_t *out);  /* any integer or bool scalar */
int prism_gguf_metadata_float(const prism_gguf *g, const char *key, double *out); /* F32 / F64 scalar */
/* A string scalar (element 0) or one element of a retained string array. */
int prism_gguf_metadata_string(const prism_gguf *g, const char *key, uint64_t element, const char **text,
                               uint64_t *len);
/* Copies a tensor's payload (exactly info.bytes) from the file. */
int prism_gguf_read_tensor(const prism_gguf *g, const char *name, void *dst, uint64_t dst_len);
/* Uploads a tensor as a weight (dims[0] = cols, dims[1] = rows, higher dims 1), through
 * prism_hip_weight_acquire with the given key (the residency cache's identity). */
prism_weight_id prism_hip_weight_from_gguf(prism_hip_ctx *ctx, const prism_gguf *g, const char *name, uint64_t key);
/* Lossless PQ2 -> PTQ1 export (tools/gguf/src/export.rs:130-318) into a new file (never
 * overwrites): requires a UINT32 general.file_type 141 or 142 and at least one PQ2
 * tensor; general.file_type becomes 143, PQ2 tensors become PTQ1 (each block packed and
 * re-expanded to its exact source bytes), other payloads are copied verbatim, extents
 * re-laid in offset order at the file's alignment.  receipt (optional) receives a JSON
 * summary with the output's SHA-256. */
int prism_gguf_export_ptq1(const char *src_path, const char *dst_path, char *receipt, size_t receipt_len);

#ifdef __cplusplus
}
#endif
#endif
