/*
 * decoder_oracle.c -- CPU restatement of one full-attention decode step of the
 * reference's Qwen35 graph in its source ("Arithmetic::Source") order.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP decode step.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * The layer composition follows src/graph.rs:3870-3995 (norm -> attention ->
 * residual add + post norm -> FFN -> residual add; final norm -> LM head); the
 * attention follows the single-head source path of full_attention_state
 * (src/graph.rs:4480-4911).  Every linear projection goes through po_matvec, the
 * restated public matvec (source activation contract).  The synthetic geometry has
 * no attention output gate: the query projection is heads*head wide.
 *
 * Pinning: rms_norm and the softmax are checked against float64 closed forms and
 * hand-computed cases in tests/test_decoder_oracle.py; RoPE against the rotation
 * matrix; the attention against a float64 evaluation of the same formulas; the
 * composition has no fixture in the reference and is parity unpinned beyond that.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "prism_oracle.h"

static inline int finite_f(float v) { return isfinite(v); }

/* rms_norm_scale_inner (src/kernels.rs:3823-3878): binary64 sum of the binary32
 * squares, mean rounded to binary32, scale = 1 / sqrt(mean + eps). */
static int rms_scale(const float *x, size_t n, float eps, float *scale) {
    double sum = 0.0;
    for (size_t i = 0; i < n; i++) {
        if (!finite_f(x[i])) return PO_ERR_NONFINITE;
        sum += (double)(x[i] * x[i]);
    }
    float mean = (float)(sum / (double)(uint32_t)n);
    float s = 1.0f / sqrtf(mean + eps);
    if (!finite_f(s) || s <= 0.0f) return PO_ERR_NONFINITE;
    *scale = s;
    return PO_OK;
}

/* rms_norm_into, source order (src/kernels.rs:3389-3418): (x * scale) * w. */
int po_rms_norm(const float *x, const float *w, size_t n, float eps, float *out) {
    float scale;
    int rc = rms_scale(x, n, eps, &scale);
    if (rc) return rc;
    for (size_t i = 0; i < n; i++) {
        out[i] = (x[i] * scale) * w[i];
        if (!finite_f(out[i])) return PO_ERR_NONFINITE;
    }
    return PO_OK;
}

/* rope_frequencies_mrope (src/graph.rs:6406-6431). */
void po_rope_frequencies(size_t rope, const size_t sections[4], const size_t positions[4], float base,
                         float *cosines, float *sines) {
    const float theta_scale = powf(base, -2.0f / (float)rope);
    float thetas[4] = {(float)positions[0], (float)positions[1], (float)positions[2], (float)positions[3]};
    for (size_t index = 0; index < rope / 2; index++) {
        size_t sector = index % 3;
        float angle = index < 3 * sections[sector] ? thetas[sector] : thetas[3];
        cosines[index] = cosf(angle);
        sines[index] = sinf(angle);
        for (int k = 0; k < 4; k++) thetas[k] *= theta_scale;
    }
}

/* rms_norm_rope_round_f16_into::<false> (src/kernels.rs:3679-3733) on one head,
 * in place: normalize, rotate the first `rope` dimensions (halves index and
 * index + rope/2), round to binary16. */
int po_norm_rope_f16(float *v, const float *w, size_t head, size_t rope, const float *cosines,
                     const float *sines, float eps) {
    float scale;
    int rc = rms_scale(v, head, eps, &scale);
    if (rc) return rc;
    for (size_t i = 0; i < head; i++) {
        v[i] = (v[i] * scale) * w[i];
        if (!finite_f(v[i])) return PO_ERR_NONFINITE;
    }
    for (size_t i = 0; i < rope / 2; i++) {
        float first = v[i], second = v[i + rope / 2];
        v[i] = first * cosines[i] - second * sines[i];
        v[i + rope / 2] = first * sines[i] + second * cosines[i];
    }
    for (size_t i = 0; i < head; i++) {
        if (!finite_f(v[i])) return PO_ERR_NONFINITE;
        v[i] = po_round_f16(v[i]);
        if (!finite_f(v[i])) return PO_ERR_NONFINITE;
    }
    return PO_OK;
}

/* softmax_round_f16 (src/kernels.rs:4431-4462). */
int po_softmax_round_f16(float *v, size_t n) {
    float maximum = -INFINITY;
    for (size_t i = 0; i < n; i++) {
        if (isnan(v[i]) || v[i] == INFINITY) return PO_ERR_INVALID_INPUT;
        maximum = fmaxf(maximum, v[i]);
    }
    if (!finite_f(maximum)) return PO_ERR_INVALID_INPUT;
    double total = 0.0;
    for (size_t i = 0; i < n; i++) {
        v[i] = expf(v[i] - maximum);
        total += (double)v[i];
    }
    float inverse = (float)(1.0 / total);
    for (size_t i = 0; i < n; i++) v[i] = po_round_f16(v[i] * inverse);
    return PO_OK;
}

/* One query head over `past` cached tokens plus the current one (src/graph.rs:
 * 4884-4911): scores by f16_dot / float_dot (binary32 products summed in binary64,
 * src/kernels.rs:1256-1273,1344-1361) times 1/sqrt(head), softmax_round_f16, then
 * source_value_tile (src/kernels.rs:2971-3011).  kc/vc: binary16 rows with `stride`
 * halves per token, this head's slice at `offset`. */
int po_attention_head(const float *q, const uint16_t *kc, const uint16_t *vc, size_t stride, size_t offset,
                      size_t past, const float *kcur, const float *vcur, size_t head, float *scores, float *out) {
    const float scale = 1.0f / sqrtf((float)head);
    for (size_t t = 0; t <= past; t++) {
        double s = 0.0;
        for (size_t d = 0; d < head; d++) {
            float k = t < past ? po_half_to_float(kc[t * stride + offset + d]) : kcur[d];
            s += (double)(q[d] * k);
        }
        scores[t] = (float)s * scale;
    }
    int rc = po_softmax_round_f16(scores, past + 1);
    if (rc) return rc;
    for (size_t d = 0; d < head; d++) {
        double s = 0.0;
        for (size_t t = 0; t < past; t++) s += (double)(scores[t] * po_half_to_float(vc[t * stride + offset + d]));
        out[d] = (float)(s + (double)(scores[past] * vcur[d]));
    }
    return PO_OK;
}

static int add_finite(float *h, const float *d, size_t n) {
    for (size_t i = 0; i < n; i++) {
        h[i] = h[i] + d[i];
        if (!finite_f(h[i])) return PO_ERR_NONFINITE;
    }
    return PO_OK;
}

/* One decode step: embed `token` (the tied Q8_0 LM head row, decode_row_into
 * src/kernels.rs:303), run every layer at position `pos` (appending its key and
 * value to the caches), final norm, LM head.  logits: vocab floats. */
int po_decoder_step(const po_decoder_geometry *g, const po_decoder_layer *layers, const uint8_t *lm_head,
                    const float *output_norm, uint32_t token, size_t pos, float *logits, int threads) {
    const size_t H = g->hidden, F = g->ffn, D = g->head_dim;
    const size_t QW = g->heads * D, KW = g->kv_heads * D, QKV = QW + 2 * KW;
    const size_t group = g->heads / g->kv_heads;
    const size_t row_bytes = H / 32 * 34;
    int rc = PO_OK;
    float *hidden = malloc(sizeof(float) * H), *xn = malloc(sizeof(float) * H);
    float *qkv = malloc(sizeof(float) * QKV), *att = malloc(sizeof(float) * QW);
    float *tmp = malloc(sizeof(float) * H), *scores = malloc(sizeof(float) * (pos + 1));
    float *cosines = malloc(sizeof(float) * (g->rope / 2)), *sines = malloc(sizeof(float) * (g->rope / 2));
    if (!hidden || !xn || !qkv || !att || !tmp || !scores || !cosines || !sines) rc = PO_ERR_RESOURCE;
    if (!rc && (token >= g->vocab || pos >= g->max_tokens)) rc = PO_ERR_INVALID_INPUT;
    if (!rc) rc = po_decode_row(PO_KIND_Q8_0, H, lm_head + (size_t)token * row_bytes, hidden);
    if (!rc) {
        const size_t positions[4] = {pos, pos, pos, 0};
        po_rope_frequencies(g->rope, g->rope_sections, positions, g->rope_base, cosines, sines);
    }
    for (size_t l = 0; !rc && l < g->layers; l++) {
        const po_decoder_layer *L = &layers[l];
        rc = po_rms_norm(hidden, L->norm, H, g->eps, xn);
        if (!rc) rc = po_matvec(PO_KIND_PTQ1, H, QKV, L->qkv, xn, 0, qkv, threads);
        float *q = qkv, *k = qkv + QW, *v = qkv + QW + KW;
        for (size_t h = 0; !rc && h < g->heads; h++)
            rc = po_norm_rope_f16(q + h * D, L->q_norm, D, g->rope, cosines, sines, g->eps);
        for (size_t h = 0; !rc && h < g->kv_heads; h++)
            rc = po_norm_rope_f16(k + h * D, L->k_norm, D, g->rope, cosines, sines, g->eps);
        for (size_t i = 0; !rc && i < KW; i++) {
            v[i] = po_round_f16(v[i]);
            if (!finite_f(v[i])) rc = PO_ERR_NONFINITE;
        }
        for (size_t h = 0; !rc && h < g->heads; h++) {
            size_t kh = h / group;
            rc = po_attention_head(q + h * D, L->kcache, L->vcache, KW, kh * D, pos, k + kh * D, v + kh * D, D,
                                   scores, att + h * D);
        }
        for (size_t i = 0; !rc && i < KW; i++) {
            L->kcache[pos * KW + i] = po_float_to_half(k[i]);
            L->vcache[pos * KW + i] = po_float_to_half(v[i]);
        }
        if (!rc) rc = po_matvec(PO_KIND_PTQ1, QW, H, L->o, att, 0, tmp, threads);
        if (!rc) rc = add_finite(hidden, tmp, H);
        if (!rc) rc = po_rms_norm(hidden, L->post_norm, H, g->eps, xn);
        if (!rc) rc = po_ffn(PO_KIND_PTQ1, H, F, L->gate, L->up, L->down, xn, hidden, 0, tmp, NULL, threads);
        if (!rc) memcpy(hidden, tmp, sizeof(float) * H);
    }
    if (!rc) rc = po_rms_norm(hidden, output_norm, H, g->eps, xn);
    if (!rc) rc = po_matvec(PO_KIND_Q8_0, H, g->vocab, lm_head, xn, 0, logits, threads);
    free(hidden); free(xn); free(qkv); free(att); free(tmp); free(scores); free(cosines); free(sines);
    return rc;
}

/* Greedy choice: the first index of the largest logit. */
size_t po_argmax(const float *v, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}
