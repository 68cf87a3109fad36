/*
 * prism_oracle.h -- CPU restatement of the reference's scalar packed-matvec path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP kernels:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  The product library (libprism_hip.so) never links or calls it.
 *
 * Every function follows the reference's scalar Rust code; the file:line cited
 * beside each declaration is relative to the reference checkout
 * (symbiogenesis/prism-inference 0.1.33).  Arithmetic is plain IEEE binary32
 * with every rounding explicit: the library is compiled with
 * -ffp-contract=off and uses fmaf() exactly where the reference uses mul_add.
 *
 * Pinning of each function (golden vectors, closed forms) is listed in the
 * header comment of prism_oracle.c.
 */
#ifndef PRISM_ORACLE_H
#define PRISM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Tensor kinds (src/kernels.rs:75-87, src/backend.rs:99-141). */
#define PO_KIND_Q8_0 8u
#define PO_KIND_Q2_K 10u
#define PO_KIND_Q8_K 15u
#define PO_KIND_TQ1_0 34u
#define PO_KIND_TQ2_0 35u
#define PO_KIND_PQ2 142u
#define PO_KIND_PTQ1 143u

/* Error codes; identical values to the product C ABI (include/prism_hip.h). */
#define PO_OK 0
#define PO_ERR_INVALID_INPUT (-1)
#define PO_ERR_RESOURCE (-2)
#define PO_ERR_NONFINITE (-3)
#define PO_ERR_UNSUPPORTED (-5)

/* Q8_0 activation contracts (src/kernels.rs:552-617). */
#define PO_Q8_SOURCE 0        /* d = max/127, q = round-half-away(x*(1/d)) */
#define PO_Q8_PINNED 1        /* same scale, ties-to-even                   */
#define PO_Q8_PINNED_NATIVE 2 /* d = max*0x3c010204, inv = 127/max, RNE     */

/* In-memory Q8_K block, tools/ternary/src/lib.rs:27-39 (#[repr(C)], 292 B). */
typedef struct {
    float scale;
    int8_t values[256];
    int16_t sums[16];
} po_q8k_block;

/* In-memory prepared Q8_0 block, src/kernels.rs:528-535 (not the 34-B wire form). */
typedef struct {
    float scale; /* already binary16-rounded */
    float sum;   /* binary16-rounded scaled code sum */
    int8_t values[32];
} po_q8_block;

/* ---- codecs: tools/ternary/src/lib.rs ---- */
float po_half_to_float(uint16_t h);                          /* lib.rs:70-90 */
uint32_t po_half_to_float_bits(uint16_t h);                 /* same, as raw bits (keeps sNaN payloads) */
uint16_t po_float_to_half(float f);                          /* lib.rs:96-113 */
float po_round_f16(float f);                                 /* kernels.rs:2824-2830 */
void po_decode_ptq_trits(const uint8_t *blk, int16_t *out);  /* lib.rs:239-250 */
int po_pack_ptq(const uint8_t *pq2, uint8_t *ptq);           /* lib.rs:163-189 */
int po_unpack_ptq(const uint8_t *ptq, uint8_t *pq2);         /* lib.rs:260-290 */

/* ---- TQ1_0 / TQ2_0 (src/kernels/tquants.rs, tquants_oracle.c) ---- */
void po_tq_codes(uint32_t kind, const uint8_t *blk, int16_t *out);                  /* tquants.rs:145-190 */
int po_dot_tq(uint32_t kind, const uint8_t *row, size_t nblocks, const po_q8k_block *act,
              float *out);                                                            /* tquants.rs:255-273 */
int po_quantize_tq(uint32_t kind, const float *x, size_t n, uint8_t *out);          /* tquants.rs:275-324 */

/* ---- layout (src/kernels.rs:88-119) ---- */
int po_layout(uint32_t kind, size_t *group, size_t *block_bytes);

/* ---- activation quantizers ---- */
int po_quantize_q8k(const float *x, size_t n, int pinned, po_q8k_block *out);  /* kernels.rs:463-522 */
int po_quantize_q8_0(const float *x, size_t n, int contract, po_q8_block *out); /* kernels.rs:552-617 */

/* ---- weight / row quantizers (src/kernels.rs:640-711; kquants Q8_K layout) ---- */
int po_quantize_row(uint32_t kind, const float *x, size_t n, uint8_t *out, size_t out_len);

/* ---- row decode (src/kernels.rs:325-400, kquants.rs:53-78,139-158) ---- */
int po_decode_row(uint32_t kind, size_t count, const uint8_t *bytes, float *out);

/* ---- row dots ---- */
int po_dot_pq2(const uint8_t *row, size_t nblocks, const po_q8k_block *act, int fused,
               float *out);                                                      /* kernels.rs:941-955 */
int po_dot_q8_groups(uint32_t kind, const uint8_t *row, size_t nblocks, const po_q8_block *act,
                     float *out);                                                /* kernels.rs:1043-1064 */
int po_dot_q8_groups_pinned(uint32_t kind, const uint8_t *row, size_t nblocks,
                            const po_q8_block *act, float *out);                 /* kernels.rs:1066-1147 */
int po_dot_q2k(const uint8_t *row, size_t nblocks, const po_q8k_block *act, float *out); /* kquants.rs:162-197,346-430 */
int po_dot_q8_0(const uint8_t *row, size_t nblocks, const po_q8_block *act, float *out); /* kernels.rs:1204-1248 */
int po_dot_ptq1_q8k(const uint8_t *row, size_t nblocks, const po_q8k_block *act, float *out); /* kernels.rs:999-1037 */
int po_packed_dot(uint32_t kind, size_t count, const uint8_t *w, size_t wlen, const uint8_t *a,
                  size_t alen, float *out);                                      /* kernels.rs:1534-1617 */

/* ---- projections (MatvecScratch::prepare + PreparedMatvec::multiply) ----
 * Row partition follows CpuThreadPool: worker w of T owns rows [w*rows/T, (w+1)*rows/T)
 * (src/backend/threadpool.rs:190-196).  On error the output is zero-filled and the
 * first error in row order is returned. */
int po_activation_contract(uint32_t kind, size_t cols, int pinned); /* 0=Q8K 1=Q8 2=PinnedPtq1Q8 */
int po_matvec(uint32_t kind, size_t cols, size_t rows, const uint8_t *w, const float *x,
              int pinned, float *out, int threads);                   /* kernels.rs:1935-2122, 2565-2815 */
int po_project_q8k(uint32_t kind, size_t cols, size_t rows, const uint8_t *w,
                   const po_q8k_block *act, int fused, float *out, int threads);
int po_project_q8(uint32_t kind, size_t cols, size_t rows, const uint8_t *w, const po_q8_block *act,
                  int pinned, float *out, int threads);

/* ---- SwiGLU (src/graph.rs:121-131; src/kernels/pinned_activations.rs:26-62,141-178) ---- */
float po_vector_exp(float x);
void po_silu(float *x, size_t n, int pinned);
void po_swiglu(const float *gate, float *up, size_t n, int pinned);

/* ---- LoRA A dot beside the FFN chain (src/kernels.rs:2336-2357) ---- */
int po_lora_a_dot(const float *a, const float *input, size_t n, int pinned, float *out);

/* ---- FFN chain: gate/up -> SwiGLU -> down (+ residual) (src/graph.rs:3935-3956) ---- */
int po_ffn(uint32_t kind, size_t hidden, size_t ffn, const uint8_t *wg, const uint8_t *wu,
           const uint8_t *wd, const float *x, const float *residual, int pinned, float *out,
           float *h_out, int threads);

/* ---- blockwise normalized Walsh-Hadamard rotation (src/kernels.rs:3952-3987) and the chain
 * that rotates the SwiGLU vector ahead of down (src/kernels/projection.rs:271-290) ---- */
int po_hadamard(float *v, size_t n, uint32_t block);
int po_ffn_rotated(uint32_t kind, size_t hidden, size_t ffn, const uint8_t *wg, const uint8_t *wu,
                   const uint8_t *wd, const float *x, const float *residual, uint32_t hadamard_block,
                   int pinned, float *out, float *h_out, int threads);

/* ---- full-attention decode step, source order (decoder_oracle.c) ---- */
typedef struct {
    size_t hidden, ffn, heads, kv_heads, head_dim, rope, vocab, layers, max_tokens;
    size_t rope_sections[4];
    float rope_base, eps;
} po_decoder_geometry;

typedef struct {
    const uint8_t *qkv;   /* PTQ1 [(heads + 2 kv_heads) * head_dim][hidden]: q, k, v rows */
    const uint8_t *o;     /* PTQ1 [hidden][heads * head_dim] */
    const uint8_t *gate;  /* PTQ1 [ffn][hidden] */
    const uint8_t *up;    /* PTQ1 [ffn][hidden] */
    const uint8_t *down;  /* PTQ1 [hidden][ffn] */
    const float *norm, *post_norm, *q_norm, *k_norm;
    uint16_t *kcache, *vcache; /* binary16 [max_tokens][kv_heads * head_dim] */
} po_decoder_layer;

int po_rms_norm(const float *x, const float *w, size_t n, float eps, float *out); /* kernels.rs:3389-3418,3823-3878 */
void po_rope_frequencies(size_t rope, const size_t sections[4], const size_t positions[4], float base,
                         float *cosines, float *sines);                           /* graph.rs:6406-6431 */
int po_norm_rope_f16(float *v, const float *w, size_t head, size_t rope, const float *cosines,
                     const float *sines, float eps);                              /* kernels.rs:3679-3733 */
int po_softmax_round_f16(float *v, size_t n);                                     /* kernels.rs:4431-4462 */
int po_attention_head(const float *q, const uint16_t *kc, const uint16_t *vc, size_t stride, size_t offset,
                      size_t past, const float *kcur, const float *vcur, size_t head, float *scores,
                      float *out);                                                /* graph.rs:4884-4911 */
int po_decoder_step(const po_decoder_geometry *g, const po_decoder_layer *layers, const uint8_t *lm_head,
                    const float *output_norm, uint32_t token, size_t pos, float *logits,
                    int threads);                                                 /* graph.rs:3870-3995 */
size_t po_argmax(const float *v, size_t n);

#ifdef __cplusplus
}
#endif
#endif
