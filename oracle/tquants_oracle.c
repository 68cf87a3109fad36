/*
 * tquants_oracle.c -- CPU restatement of the reference's native 256-element ternary
 * formats TQ1_0 (kind 34, 54 B per block) and TQ2_0 (kind 35, 66 B per block):
 * decode, the Q8_K row dot and the weight quantizer (src/kernels/tquants.rs:17-324,
 * themselves ports of ggml's ggml-quants.c / ggml-cpu/quants.c).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP TQ kernels.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Pinning: every function is checked against the ten records of the reference's
 * tests/fixtures/upstream-tquants.json (packed bytes, decoded values, the generic
 * dot's bits and the quantizer's output) in tests/test_tquants_oracle.py, and the
 * trit decoder against the closed form on all 256 bytes.
 */
#include <math.h>
#include <string.h>

#include "prism_oracle.h"

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline int finite_f(float f) { return (f2u(f) & 0x7f800000u) != 0x7f800000u; }

/* Digit k of a TQ1_0 byte, minus one: ((b * 3^k mod 256) * 3) / 256 - 1
 * (TQ1_BYTE_LUT, tquants.rs:25-41). */
static int tq1_digit(uint8_t b, int k) {
    static const uint8_t pw[5] = {1, 3, 9, 27, 81};
    const uint8_t m = (uint8_t)(b * pw[k]);
    return (int)m * 3 / 256 - 1;
}

/* codes(), tquants.rs:145-190: the 256 signed digits of one block in element order. */
void po_tq_codes(uint32_t kind, const uint8_t *blk, int16_t *out) {
    if (kind == PO_KIND_TQ2_0) {
        for (int half = 0; half < 2; half++)
            for (int col = 0; col < 32; col++) {
                const uint8_t b = blk[32 * half + col];
                for (int k = 0; k < 4; k++) out[128 * half + col + 32 * k] = (int16_t)(((b >> (2 * k)) & 3) - 1);
            }
        return;
    }
    for (int col = 0; col < 32; col++)
        for (int k = 0; k < 5; k++) out[col + 32 * k] = (int16_t)tq1_digit(blk[col], k);
    for (int col = 0; col < 16; col++)
        for (int k = 0; k < 5; k++) out[160 + col + 16 * k] = (int16_t)tq1_digit(blk[32 + col], k);
    for (int col = 0; col < 4; col++)
        for (int k = 0; k < 4; k++) out[240 + col + 4 * k] = (int16_t)tq1_digit(blk[48 + col], k);
}

static size_t tq_block_bytes(uint32_t kind) { return kind == PO_KIND_TQ2_0 ? 66 : 54; }

/* dot(), tquants.rs:255-273: per block the exact integer dot, then
 * sum = fl(sum + fl(float(I) * fl(d * a.scale))). */
int po_dot_tq(uint32_t kind, const uint8_t *row, size_t nblocks, const po_q8k_block *act, float *out) {
    const size_t bb = tq_block_bytes(kind);
    float sum = 0.0f;
    int16_t w[256];
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = row + b * bb;
        po_tq_codes(kind, blk, w);
        int32_t integer = 0;
        for (int i = 0; i < 256; i++) integer += (int32_t)w[i] * (int32_t)act[b].values[i];
        const uint16_t h = (uint16_t)(blk[bb - 2] | (blk[bb - 1] << 8));
        const float d = po_half_to_float(h);
        if (!finite_f(d) || !finite_f(act[b].scale)) return PO_ERR_NONFINITE;
        const float ds = d * act[b].scale;
        sum = sum + (float)integer * ds;
    }
    if (!finite_f(sum)) return PO_ERR_NONFINITE;
    *out = sum;
    return PO_OK;
}

/* quantize(), tquants.rs:275-324: d = max|x|, stored as binary16; levels
 * round-half-away(x * (1/d)) + 1; TQ2_0 packs 2-bit levels at stride 32, TQ1_0 packs
 * five base-3 digits (most significant first, the 4-digit tail times 3) into
 * ceil(code * 256 / 243). */
int po_quantize_tq(uint32_t kind, const float *x, size_t n, uint8_t *out) {
    const size_t bb = tq_block_bytes(kind);
    if (n == 0 || n % 256) return PO_ERR_INVALID_INPUT;
    for (size_t i = 0; i < n; i++)
        if (!finite_f(x[i])) return PO_ERR_INVALID_INPUT;
    memset(out, 0, n / 256 * bb);
    for (size_t b = 0; b < n / 256; b++) {
        const float *in = x + 256 * b;
        uint8_t *o = out + bb * b;
        float d = 0.0f;
        for (int i = 0; i < 256; i++) d = fmaxf(d, fabsf(in[i]));
        const uint16_t bits = po_float_to_half(d);
        if (!finite_f(po_half_to_float(bits))) return PO_ERR_NONFINITE;
        o[bb - 2] = (uint8_t)(bits & 255u);
        o[bb - 1] = (uint8_t)(bits >> 8);
        float inverse = 0.0f;
        if (d != 0.0f) {
            inverse = 1.0f / d;
            if (!finite_f(inverse)) return PO_ERR_NONFINITE;
        }
        uint8_t levels[256];
        for (int i = 0; i < 256; i++) levels[i] = (uint8_t)((int16_t)roundf(in[i] * inverse) + 1);
        if (kind == PO_KIND_TQ2_0) {
            for (int i = 0; i < 256; i++) o[i / 128 * 32 + i % 32] |= (uint8_t)(levels[i] << (2 * (i % 128 / 32)));
        } else {
            for (int byte = 0; byte < 52; byte++) {
                int first, stride, count;
                if (byte < 32) {
                    first = byte; stride = 32; count = 5;
                } else if (byte < 48) {
                    first = 160 + byte - 32; stride = 16; count = 5;
                } else {
                    first = 240 + byte - 48; stride = 4; count = 4;
                }
                uint32_t code = 0;
                for (int k = 0; k < count; k++) code = code * 3 + levels[first + k * stride];
                if (count == 4) code *= 3;
                o[byte] = (uint8_t)((code * 256 + 242) / 243);
            }
        }
    }
    return PO_OK;
}
