/*
 * prism_oracle.c -- CPU restatement of the reference's scalar packed-matvec path.
 *
 * TEST INFRASTRUCTURE ONLY: this is the checker for the HIP kernels, never the
 * product.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load it.  Build: oracle/Makefile (-O2 -ffp-contract=off -fno-fast-math).
 *
 * The reference is Rust (edition 2024, nightly toolchain) and cannot be built in
 * this environment, so there is no oracle/_ref build.  Each function below cites
 * the reference file:line it restates.  Pinning (what fixes each function beyond
 * retyping its formula; the tests live in tests/test_oracle_*.py):
 *
 *   half_to_float        ptq-reference.bin: 26 native binary16 cases + exhaustive
 *                        round trip over all finite halves.
 *   float_to_half        numpy RNE float16 over 2^20 random floats + all halves;
 *                        row-quantizers.json TypeId 1 (F16) records.
 *   decode_ptq_trits     ptq-reference.bin (161 native PQ2<->PTQ cases), the
 *                        20 000-block LCG(12345) element map with both upstream
 *                        traversals, exhaustive 256-byte closed form.
 *   pack/unpack_ptq      ptq-reference.bin byte-exact both directions.
 *   quantize_q8k         row-quantizers.json TypeId 15 (source);
 *                        swift-q8k-parity.bin (pinned, fused nearest-int boundary).
 *   quantize_q8_0        row-quantizers.json TypeId 8 (source); swift-q8-parity.bin
 *                        (pinned generic + native scale), swift-ptq1-q8-scale-parity.bin
 *                        (native scale halfway cases, codes -52/-77, generic -51).
 *   quantize_row PQ2/PTQ1 row-quantizers.json TypeId 142/143.
 *   dot_pq2              native capture KAT (fused 0xc1f90b01 / unfused 0xc1f90b02),
 *                        closed-form KATs [5.0], [-254.0], [0.0];
 *                        pq2-inputs.bin 15 shapes vs f64 (rel-RMS < 0.05).
 *   dot_q8_groups(+pinned) swift-ptq1-dot-parity.bin native pinned bits and source
 *                        bits; KATs [7.0], [0.99993896], odd-PQ2 [11.0], [19.25];
 *                        LCG(99) upstream integer group sums (5000 trials).
 *   dot_q2k / decode Q2_K upstream-kquants.json TypeId 10 (quantize, decode, GenericDot).
 *   dot_q8_0             no fixture: representable-exact chains equal the exact sum,
 *                        and hand-derived binary32 known answers separate the order
 *                        from a fused last step, a reordered chain and the scales
 *                        applied in the other order (tests/fixtures_util.py).
 *   dot_ptq1_q8k         equal to dot_pq2 unfused on pack_ptq'd PQ2 rows (lossless codec).
 *   silu/swiglu pinned   swift-activation-parity.json: all 45 native SiLU and SwiGLU
 *                        bits (vector body, libm tail, finite edges); bitwise parity of
 *                        the source path (libm exp) is unpinnable.
 *   matvec/ffn           compositions of the above; per-token == row dot loop.
 *   lora_a_dot           pinned: sixteen FMA lanes on inputs whose products and sums are
 *                        exact equal the exact dot, and a constructed input whose lane
 *                        sums differ from the ordered sum pins the lane combination;
 *                        source: constructed inputs where the ordered binary64 sum
 *                        absorbs a term (1e20 + 1 - 1e20 + 1 == 1, not 2) pin the order.
 */
#include "prism_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* small helpers                                                             */
/* ------------------------------------------------------------------------- */

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline int is_finite(float f) { return (f2u(f) & 0x7f800000u) != 0x7f800000u; }
static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* scale(): f16 -> f32 with a finite check (src/kernels.rs:152-154). */
static int scale_of(const uint8_t *p, float *out) {
    float v = po_half_to_float(rd16(p));
    if (!is_finite(v)) return PO_ERR_NONFINITE;
    *out = v;
    return PO_OK;
}

/* ------------------------------------------------------------------------- */
/* codecs                                                                    */
/* ------------------------------------------------------------------------- */

/* tools/ternary/src/lib.rs:70-90: every binary16 pattern to binary32, exact. */
float po_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t mant = h & 1023u;
    uint32_t exp = (h >> 10) & 31u;
    if (exp == 0) {
        if (mant == 0) return u2f(sign);
        exp = 113;
        while ((mant & 1024u) == 0) {
            mant <<= 1;
            exp -= 1;
        }
        mant &= 1023u;
    } else if (exp == 31) {
        exp = 255;
    } else {
        exp += 112;
    }
    return u2f(sign | (exp << 23) | (mant << 13));
}

/* tools/ternary/src/lib.rs:96-113: binary32 -> binary16, round-ties-to-even,
 * signed zero and subnormals kept, NaN -> sign|0x7e00.  Written from the IEEE
 * definition (integer mantissa rounding), not from the reference's bit trick. */
uint16_t po_float_to_half(float f) {
    uint32_t b = f2u(f);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    uint32_t a = b & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;
    if (a >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to infinity */
    if (a < 0x38800000u) {                        /* below 2^-14: subnormal half */
        if (a < 0x33000000u) return sign;         /* < 2^-25 (tie at 2^-25 -> 0) */
        uint32_t e = a >> 23;
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* value in units of 2^-24 is m >> shift */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (a >> 23) - 112u;
    uint32_t m = a & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

uint32_t po_half_to_float_bits(uint16_t h) { return f2u(po_half_to_float(h)); }

/* src/kernels.rs:2824-2830 */
float po_round_f16(float f) { return po_half_to_float(po_float_to_half(f)); }

/* Fractional trit k of byte x: ((x * 3^k mod 256) * 3) >> 8 (lib.rs:202-233). */
static inline int trit(uint32_t x, int k) {
    for (int i = 0; i < k; i++) x = (x * 3u) & 255u;
    return (int)((x * 3u) >> 8);
}

/* tools/ternary/src/lib.rs:239-250: element i -> (byte, digit). */
void po_decode_ptq_trits(const uint8_t *blk, int16_t *out) {
    for (int i = 0; i < 128; i++) {
        int lane, digit;
        if (i < 80) {
            lane = i % 16;
            digit = i / 16;
        } else if (i < 120) {
            lane = 16 + (i - 80) % 8;
            digit = (i - 80) / 8;
        } else {
            lane = 24 + (i - 120) % 2;
            digit = (i - 120) / 2;
        }
        out[i] = (int16_t)(trit(blk[lane], digit) - 1);
    }
}

static int check_scale_bytes(const uint8_t *p) {
    uint16_t s = rd16(p);
    if (s == 0 || s == 0x8000u || (s & 0x7c00u) == 0x7c00u) return PO_ERR_INVALID_INPUT;
    return PO_OK;
}

static inline uint8_t pq2_code(const uint8_t *b, int i) { return (b[2 + i / 4] >> (2 * (i % 4))) & 3u; }

/* tools/ternary/src/lib.rs:163-189 (with check_pq2 :147-156). */
int po_pack_ptq(const uint8_t *src, uint8_t *out) {
    if (check_scale_bytes(src)) return PO_ERR_INVALID_INPUT;
    for (int i = 2; i < 34; i++)
        if (src[i] & (src[i] >> 1) & 0x55u) return PO_ERR_INVALID_INPUT;
    memset(out, 0, 28);
    int pos = 0;
    const int widths[2] = {16, 8};
    for (int wi = 0; wi < 2; wi++) {
        int width = widths[wi];
        int start = pos / 5;
        for (int m = 0; m < width; m++) {
            uint32_t q = 0;
            for (int n = 0; n < 5; n++) q = q * 3u + pq2_code(src, pos + m + n * width);
            uint32_t v = (q * 256u + 242u) / 243u;
            if (v > 255u) return PO_ERR_INVALID_INPUT;
            out[start + m] = (uint8_t)v;
        }
        pos += width * 5;
    }
    for (int h = 0; h < 2; h++) {
        uint32_t q = 0;
        for (int n = 0; n < 4; n++) q = q * 3u + pq2_code(src, 120 + h + n * 2);
        uint32_t v = (q * 3u * 256u + 242u) / 243u;
        if (v > 255u) return PO_ERR_INVALID_INPUT;
        out[24 + h] = (uint8_t)v;
    }
    out[26] = src[0];
    out[27] = src[1];
    return PO_OK;
}

/* tools/ternary/src/lib.rs:207-233 (digit table) and :260-290 (unpack). */
static void ptq_digits(uint32_t byte, uint8_t digits[5], int *canon5, int *canon4) {
    uint32_t frac = byte, value = 0;
    for (int d = 0; d < 5; d++) {
        frac *= 3u;
        uint32_t t = frac >> 8;
        digits[d] = (uint8_t)t;
        value = value * 3u + t;
        frac &= 255u;
    }
    *canon5 = ((value * 256u + 242u) / 243u) == byte;
    *canon4 = ((value / 3u * 3u * 256u + 242u) / 243u) == byte;
}

int po_unpack_ptq(const uint8_t *src, uint8_t *out) {
    if (check_scale_bytes(src + 26)) return PO_ERR_INVALID_INPUT;
    memset(out, 0, 34);
    out[0] = src[26];
    out[1] = src[27];
    int pos = 0;
    const int widths[2] = {16, 8};
    for (int wi = 0; wi < 2; wi++) {
        int width = widths[wi];
        int start = pos / 5;
        for (int m = 0; m < width; m++) {
            uint8_t dg[5];
            int c5, c4;
            ptq_digits(src[start + m], dg, &c5, &c4);
            if (!c5) return PO_ERR_INVALID_INPUT;
            for (int n = 0; n < 5; n++) {
                int idx = pos + n * width + m;
                out[2 + idx / 4] |= (uint8_t)(dg[n] << (2 * (idx % 4)));
            }
        }
        pos += width * 5;
    }
    for (int h = 0; h < 2; h++) {
        uint8_t dg[5];
        int c5, c4;
        ptq_digits(src[24 + h], dg, &c5, &c4);
        if (!c4) return PO_ERR_INVALID_INPUT;
        for (int n = 0; n < 4; n++) {
            int idx = 120 + n * 2 + h;
            out[2 + idx / 4] |= (uint8_t)(dg[n] << (2 * (idx % 4)));
        }
    }
    return PO_OK;
}

/* ------------------------------------------------------------------------- */
/* layout                                                                    */
/* ------------------------------------------------------------------------- */

/* src/kernels.rs:88-119 (only the kinds on this path). */
int po_layout(uint32_t kind, size_t *group, size_t *bytes) {
    switch (kind) {
    case PO_KIND_Q8_0: *group = 32; *bytes = 34; return PO_OK;
    case PO_KIND_Q2_K: *group = 256; *bytes = 84; return PO_OK;
    case PO_KIND_Q8_K: *group = 256; *bytes = 292; return PO_OK;
    case PO_KIND_PQ2: *group = 128; *bytes = 34; return PO_OK;
    case PO_KIND_PTQ1: *group = 128; *bytes = 28; return PO_OK;
    case PO_KIND_TQ1_0: *group = 256; *bytes = 54; return PO_OK; /* tquants.rs:17-23 */
    case PO_KIND_TQ2_0: *group = 256; *bytes = 66; return PO_OK;
    default: return PO_ERR_UNSUPPORTED;
    }
}

/* ------------------------------------------------------------------------- */
/* activation quantizers                                                     */
/* ------------------------------------------------------------------------- */

/* src/kernels.rs:407-415: finite and within -127..=127, then truncating cast. */
static int quantized(float v, int8_t *q) {
    if (!is_finite(v) || !(v >= -127.0f && v <= 127.0f)) return PO_ERR_INVALID_INPUT;
    *q = (int8_t)v;
    return PO_OK;
}

/* src/kernels.rs:420-428: fused magic-number nearest integer. */
static int pinned_q8k_integer(float value, float inv, int8_t *q) {
    float rounded = fmaf(inv, value, 12582912.0f);
    if (!is_finite(rounded)) return PO_ERR_NONFINITE;
    int32_t integer = (int32_t)(f2u(rounded) & 0x7fffffu) - 0x400000;
    if (integer > 127) integer = 127;
    if (integer < -128) return PO_ERR_INVALID_INPUT;
    *q = (int8_t)integer;
    return PO_OK;
}

static int all_finite(const float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (!is_finite(x[i])) return 0;
    return 1;
}

/* src/kernels.rs:463-522 (FINITE_INPUT after the caller's preflight). */
int po_quantize_q8k(const float *x, size_t n, int pinned, po_q8k_block *out) {
    if (n % 256 != 0) return PO_ERR_INVALID_INPUT;
    if (!all_finite(x, n)) return PO_ERR_NONFINITE;
    for (size_t b = 0; b < n / 256; b++) {
        const float *c = x + b * 256;
        po_q8k_block *blk = out + b;
        float maximum = 0.0f;
        for (int i = 0; i < 256; i++)
            if (fabsf(c[i]) > fabsf(maximum)) maximum = c[i];
        memset(blk, 0, sizeof(*blk));
        if (maximum == 0.0f) continue;
        float inv = -127.0f / maximum;
        if (!is_finite(inv)) return PO_ERR_NONFINITE;
        blk->scale = 1.0f / inv;
        for (int i = 0; i < 256; i++) {
            int rc;
            if (pinned) {
                rc = pinned_q8k_integer(c[i], inv, &blk->values[i]);
            } else {
                float r = nearbyintf(c[i] * inv); /* ties to even */
                if (r > 127.0f) r = 127.0f;
                rc = quantized(r, &blk->values[i]);
            }
            if (rc) return rc;
        }
        for (int j = 0; j < 16; j++) {
            int s = 0;
            for (int i = 0; i < 16; i++) s += blk->values[16 * j + i];
            blk->sums[j] = (int16_t)s;
        }
    }
    return PO_OK;
}

/* src/kernels.rs:552-617. */
int po_quantize_q8_0(const float *x, size_t n, int contract, po_q8_block *out) {
    if (n % 32 != 0) return PO_ERR_INVALID_INPUT;
    if (!all_finite(x, n)) return PO_ERR_NONFINITE;
    const int pinned = contract != PO_Q8_SOURCE;
    const int native = contract == PO_Q8_PINNED_NATIVE;
    for (size_t b = 0; b < n / 32; b++) {
        const float *c = x + b * 32;
        po_q8_block *blk = out + b;
        float maximum = 0.0f;
        for (int i = 0; i < 32; i++) {
            float a = fabsf(c[i]);
            if (a > maximum) maximum = a;
        }
        float d = native ? maximum * u2f(0x3c010204u) : maximum / 127.0f;
        float inv = (d == 0.0f) ? 0.0f : (native ? 127.0f / maximum : 1.0f / d);
        blk->scale = po_round_f16(d);
        if (!is_finite(blk->scale)) return PO_ERR_NONFINITE;
        int32_t sum = 0;
        for (int i = 0; i < 32; i++) {
            float p = c[i] * inv;
            float r = pinned ? nearbyintf(p) : roundf(p);
            int rc = quantized(r, &blk->values[i]);
            if (rc) return rc;
            sum += blk->values[i];
        }
        blk->sum = po_round_f16((float)sum * d);
    }
    return PO_OK;
}

/* src/kernels.rs:617-636 quantize_ternary (PQ2 block from 128 floats). */
static int quantize_ternary(const float *x, uint8_t *blk) {
    float maximum = 0.0f;
    for (int i = 0; i < 128; i++) {
        float a = fabsf(x[i]);
        if (a > maximum) maximum = a;
    }
    float inv = 0.0f;
    if (maximum > 0.0f) {
        inv = 1.0f / maximum;
        if (!is_finite(inv)) return PO_ERR_NONFINITE;
    }
    uint16_t s = po_float_to_half(maximum);
    if (!is_finite(po_half_to_float(s))) return PO_ERR_NONFINITE;
    memset(blk, 0, 34);
    blk[0] = (uint8_t)(s & 255u);
    blk[1] = (uint8_t)(s >> 8);
    for (int i = 0; i < 128; i++) {
        int8_t q;
        int rc = quantized(roundf(x[i] * inv), &q);
        if (rc) return rc;
        int code = q + 1;
        if (code > 3) code = 3;
        blk[2 + i / 4] |= (uint8_t)(code << (2 * (i % 4)));
    }
    return PO_OK;
}

/* src/kernels.rs:640-711 for PQ2, PTQ1, Q8_0 and Q8_K. */
int po_quantize_row(uint32_t kind, const float *x, size_t n, uint8_t *out, size_t out_len) {
    size_t group, bytes;
    if (po_layout(kind, &group, &bytes) || kind == PO_KIND_Q2_K) return PO_ERR_UNSUPPORTED;
    if (kind == PO_KIND_TQ1_0 || kind == PO_KIND_TQ2_0) { /* kernels.rs:660, before the generic checks */
        if (n % 256 == 0 && out_len != n / 256 * bytes) return PO_ERR_INVALID_INPUT;
        return po_quantize_tq(kind, x, n, out);
    }
    if (n == 0 || n % group) return PO_ERR_INVALID_INPUT;
    if (!all_finite(x, n)) return PO_ERR_NONFINITE;
    if (out_len != n / group * bytes) return PO_ERR_INVALID_INPUT;
    switch (kind) {
    case PO_KIND_PQ2:
    case PO_KIND_PTQ1:
        for (size_t b = 0; b < n / 128; b++) {
            uint8_t blk[34];
            int rc = quantize_ternary(x + 128 * b, blk);
            if (rc) return rc;
            if (kind == PO_KIND_PQ2) {
                memcpy(out + 34 * b, blk, 34);
            } else {
                uint8_t s0 = blk[0], s1 = blk[1];
                blk[0] = 0x00;
                blk[1] = 0x3c;
                rc = po_pack_ptq(blk, out + 28 * b);
                if (rc) return rc;
                out[28 * b + 26] = s0;
                out[28 * b + 27] = s1;
            }
        }
        return PO_OK;
    case PO_KIND_Q8_0: {
        po_q8_block *q = (po_q8_block *)malloc(sizeof(po_q8_block) * (n / 32));
        if (!q) return PO_ERR_RESOURCE;
        int rc = po_quantize_q8_0(x, n, PO_Q8_SOURCE, q);
        if (!rc) {
            for (size_t b = 0; b < n / 32; b++) {
                uint16_t s = po_float_to_half(q[b].scale);
                out[34 * b] = (uint8_t)(s & 255u);
                out[34 * b + 1] = (uint8_t)(s >> 8);
                memcpy(out + 34 * b + 2, q[b].values, 32);
            }
        }
        free(q);
        return rc;
    }
    case PO_KIND_Q8_K: {
        po_q8k_block *q = (po_q8k_block *)malloc(sizeof(po_q8k_block) * (n / 256));
        if (!q) return PO_ERR_RESOURCE;
        int rc = po_quantize_q8k(x, n, 0, q);
        if (!rc) memcpy(out, q, sizeof(po_q8k_block) * (n / 256)); /* repr(C) == wire layout, LE */
        free(q);
        return rc;
    }
    default: return PO_ERR_UNSUPPORTED;
    }
}

/* ------------------------------------------------------------------------- */
/* row decode                                                                */
/* ------------------------------------------------------------------------- */

/* src/kernels.rs:325-400 and src/kernels/kquants.rs:53-78,139-158. */
int po_decode_row(uint32_t kind, size_t count, const uint8_t *bytes, float *out) {
    size_t group, bb;
    if (po_layout(kind, &group, &bb)) return PO_ERR_UNSUPPORTED;
    if (count == 0 || count % group) return PO_ERR_INVALID_INPUT;
    size_t nb = count / group;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *p = bytes + b * bb;
        float *o = out + b * group;
        float d, m;
        int16_t t[128];
        switch (kind) {
        case PO_KIND_PQ2:
            if (scale_of(p, &d)) return PO_ERR_NONFINITE;
            for (int i = 0; i < 128; i++) o[i] = (float)((int)pq2_code(p, i) - 1) * d;
            break;
        case PO_KIND_PTQ1:
            if (scale_of(p + 26, &d)) return PO_ERR_NONFINITE;
            po_decode_ptq_trits(p, t);
            for (int i = 0; i < 128; i++) o[i] = (float)t[i] * d;
            break;
        case PO_KIND_Q8_0:
            if (scale_of(p, &d)) return PO_ERR_NONFINITE;
            for (int i = 0; i < 32; i++) o[i] = (float)(int8_t)p[2 + i] * d;
            break;
        case PO_KIND_Q2_K:
            if (scale_of(p + 80, &d) || scale_of(p + 82, &m)) return PO_ERR_NONFINITE;
            for (int i = 0; i < 256; i++) {
                int g = i / 16;
                float sc = (float)(p[g] & 15), mn = (float)(p[g] >> 4);
                float q = (float)((p[16 + i / 128 * 32 + i % 32] >> (2 * (i % 128 / 32))) & 3);
                float v = (d * sc) * q - m * mn;
                if (!is_finite(v)) return PO_ERR_NONFINITE;
                o[i] = v;
            }
            break;
        case PO_KIND_TQ1_0:
        case PO_KIND_TQ2_0: { /* tquants.rs:240-253 */
            int16_t c[256];
            if (scale_of(p + bb - 2, &d)) return PO_ERR_NONFINITE;
            po_tq_codes(kind, p, c);
            for (int i = 0; i < 256; i++) o[i] = (float)c[i] * d;
            break;
        }
        case PO_KIND_Q8_K: {
            float s;
            memcpy(&s, p, 4);
            if (!is_finite(s)) return PO_ERR_NONFINITE;
            for (int i = 0; i < 256; i++) o[i] = (float)(int8_t)p[4 + i] * s;
            break;
        }
        default: return PO_ERR_UNSUPPORTED;
        }
        for (size_t i = 0; i < group; i++)
            if (!is_finite(o[i])) return PO_ERR_NONFINITE;
    }
    return PO_OK;
}

/* ------------------------------------------------------------------------- */
/* row dots                                                                  */
/* ------------------------------------------------------------------------- */

static void block_values(uint32_t kind, const uint8_t *blk, int16_t *w) {
    if (kind == PO_KIND_PQ2) {
        for (int i = 0; i < 128; i++) w[i] = (int16_t)((int)pq2_code(blk, i) - 1);
    } else {
        po_decode_ptq_trits(blk, w);
    }
}

static inline int32_t dot_i(const int16_t *w, const int8_t *a, int n) {
    int32_t s = 0;
    for (int i = 0; i < n; i++) s += (int32_t)w[i] * (int32_t)a[i];
    return s;
}

/* src/kernels.rs:941-955: out = fused ? fma(d,s,out) : out + d*s, d = scale*act.scale. */
int po_dot_pq2(const uint8_t *row, size_t nblocks, const po_q8k_block *act, int fused, float *out) {
    float o = 0.0f;
    int16_t w[128];
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = row + 34 * b;
        const po_q8k_block *a = act + b / 2;
        int start = (int)(b % 2) * 128;
        float ws;
        if (scale_of(blk, &ws)) return PO_ERR_NONFINITE;
        float d = ws * a->scale;
        block_values(PO_KIND_PQ2, blk, w);
        float s = (float)dot_i(w, a->values + start, 128);
        o = fused ? fmaf(d, s, o) : o + d * s;
    }
    if (!is_finite(o)) return PO_ERR_NONFINITE;
    *out = o;
    return PO_OK;
}

/* src/kernels.rs:1043-1064: t = sum_g fl(A.scale * I_g) in order; out += d*t. */
int po_dot_q8_groups(uint32_t kind, const uint8_t *row, size_t nblocks, const po_q8_block *act,
                     float *out) {
    const size_t bb = kind == PO_KIND_PQ2 ? 34 : 28;
    float o = 0.0f;
    int16_t w[128];
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = row + bb * b;
        float d;
        if (scale_of(kind == PO_KIND_PQ2 ? blk : blk + 26, &d)) return PO_ERR_NONFINITE;
        block_values(kind, blk, w);
        float t = 0.0f;
        for (int g = 0; g < 4; g++) {
            const po_q8_block *a = act + 4 * b + g;
            t = t + a->scale * (float)dot_i(w + 32 * g, a->values, 32);
        }
        o = o + d * t;
    }
    if (!is_finite(o)) return PO_ERR_NONFINITE;
    *out = o;
    return PO_OK;
}

/* src/kernels.rs:1066-1076: lane l sums positions 4l..4l+3 and 16+4l..16+4l+3. */
static void q8_native_lanes(const int16_t *w, const int8_t *a, int32_t lanes[4]) {
    for (int l = 0; l < 4; l++) {
        int32_t s = 0;
        for (int j = 0; j < 4; j++) {
            s += (int32_t)w[4 * l + j] * a[4 * l + j];
            s += (int32_t)w[16 + 4 * l + j] * a[16 + 4 * l + j];
        }
        lanes[l] = s;
    }
}

/* src/kernels.rs:1102-1147: four FMA lanes across the row, pairwise reduction. */
int po_dot_q8_groups_pinned(uint32_t kind, const uint8_t *row, size_t nblocks,
                            const po_q8_block *act, float *out) {
    if (kind != PO_KIND_PTQ1) return po_dot_q8_groups(kind, row, nblocks, act, out);
    float L[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int16_t w[128];
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = row + 28 * b;
        block_values(PO_KIND_PTQ1, blk, w);
        float ws;
        if (scale_of(blk + 26, &ws)) return PO_ERR_NONFINITE;
        for (int g = 0; g < 4; g++) {
            const po_q8_block *a = act + 4 * b + g;
            int32_t I[4];
            q8_native_lanes(w + 32 * g, a->values, I);
            float d = ws * a->scale;
            for (int l = 0; l < 4; l++) L[l] = fmaf((float)I[l], d, L[l]);
        }
    }
    float o = (L[0] + L[1]) + (L[2] + L[3]);
    if (!is_finite(o)) return PO_ERR_NONFINITE;
    *out = o;
    return PO_OK;
}

/* src/kernels/kquants.rs:162-197 (per block) and :346-430 (row). */
int po_dot_q2k(const uint8_t *row, size_t nblocks, const po_q8k_block *act, float *out) {
    float sum = 0.0f;
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t *p = row + 84 * b;
        const po_q8k_block *a = act + b;
        float as = a->scale;
        if (!is_finite(as)) return PO_ERR_NONFINITE;
        float d, dmin;
        if (scale_of(p + 80, &d) || scale_of(p + 82, &dmin)) return PO_ERR_NONFINITE;
        int32_t isum = 0, msum = 0;
        for (int half = 0; half < 2; half++) {
            const uint8_t *qh = p + 16 + half * 32;
            for (int part = 0; part < 4; part++) {
                for (int sub = 0; sub < 2; sub++) {
                    int g = half * 8 + part * 2 + sub;
                    int32_t sc = p[g] & 15, mn = p[g] >> 4;
                    msum += (int32_t)a->sums[g] * mn;
                    int32_t sd = 0;
                    for (int j = 0; j < 16; j++)
                        sd += (int32_t)((qh[sub * 16 + j] >> (2 * part)) & 3) * a->values[g * 16 + j];
                    isum += sc * sd;
                }
            }
        }
        sum = sum + ((as * d) * (float)isum - (as * dmin) * (float)msum);
    }
    if (!is_finite(sum)) return PO_ERR_NONFINITE;
    *out = sum;
    return PO_OK;
}

/* src/kernels.rs:1204-1248 (Q8_0 weights). */
int po_dot_q8_0(const uint8_t *row, size_t nblocks, const po_q8_block *act, float *out) {
    float o = 0.0f;
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t *p = row + 34 * b;
        float ws;
        if (scale_of(p, &ws)) return PO_ERR_NONFINITE;
        int32_t s = 0;
        for (int i = 0; i < 32; i++) s += (int32_t)(int8_t)p[2 + i] * act[b].values[i];
        o = o + (ws * act[b].scale) * (float)s;
    }
    if (!is_finite(o)) return PO_ERR_NONFINITE;
    *out = o;
    return PO_OK;
}

/* src/kernels.rs:999-1037 (scalar branch). */
int po_dot_ptq1_q8k(const uint8_t *row, size_t nblocks, const po_q8k_block *act, float *out) {
    float o = 0.0f;
    int16_t w[128];
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = row + 28 * b;
        const po_q8k_block *a = act + b / 2;
        float ws;
        if (scale_of(blk + 26, &ws) || !is_finite(a->scale)) return PO_ERR_NONFINITE;
        float d = ws * a->scale;
        po_decode_ptq_trits(blk, w);
        o = o + d * (float)dot_i(w, a->values + (b % 2) * 128, 128);
    }
    if (!is_finite(o)) return PO_ERR_NONFINITE;
    *out = o;
    return PO_OK;
}

/* src/kernels.rs:1534-1617 for PQ2, PTQ1, Q2_K and Q8_0 (wire-format activations). */
int po_packed_dot(uint32_t kind, size_t count, const uint8_t *w, size_t wlen, const uint8_t *a,
                  size_t alen, float *out) {
    size_t group, bb;
    if (kind == PO_KIND_Q8_K) return PO_ERR_INVALID_INPUT;
    if (po_layout(kind, &group, &bb)) return PO_ERR_UNSUPPORTED;
    if (count == 0 || count % group || count / group * bb != wlen) return PO_ERR_INVALID_INPUT;
    if (kind == PO_KIND_PQ2 || kind == PO_KIND_Q2_K || kind == PO_KIND_TQ1_0 || kind == PO_KIND_TQ2_0) {
        if (count % 256 || count / 256 * 292 != alen) return PO_ERR_INVALID_INPUT;
        size_t na = count / 256;
        po_q8k_block *q = (po_q8k_block *)malloc(sizeof(po_q8k_block) * na);
        if (!q) return PO_ERR_RESOURCE;
        memcpy(q, a, alen);
        int rc = PO_OK;
        for (size_t i = 0; i < na; i++)
            if (!is_finite(q[i].scale)) rc = PO_ERR_NONFINITE;
        if (!rc)
            rc = kind == PO_KIND_PQ2    ? po_dot_pq2(w, count / 128, q, 0, out)
                 : kind == PO_KIND_Q2_K ? po_dot_q2k(w, na, q, out)
                                        : po_dot_tq(kind, w, na, q, out);
        free(q);
        return rc;
    }
    if (count % 32 || count / 32 * 34 != alen) return PO_ERR_INVALID_INPUT;
    size_t na = count / 32;
    po_q8_block *q = (po_q8_block *)malloc(sizeof(po_q8_block) * na);
    if (!q) return PO_ERR_RESOURCE;
    int rc = PO_OK;
    for (size_t i = 0; i < na && !rc; i++) {
        rc = scale_of(a + 34 * i, &q[i].scale);
        q[i].sum = 0.0f;
        memcpy(q[i].values, a + 34 * i + 2, 32);
    }
    if (!rc)
        rc = kind == PO_KIND_PTQ1 ? po_dot_q8_groups(kind, w, count / 128, q, out)
                                  : po_dot_q8_0(w, na, q, out);
    free(q);
    return rc;
}

/* ------------------------------------------------------------------------- */
/* projections                                                               */
/* ------------------------------------------------------------------------- */

/* src/kernels.rs:1663-1673 ActivationContract::for_tensor. */
int po_activation_contract(uint32_t kind, size_t cols, int pinned) {
    if (kind == PO_KIND_PTQ1 && pinned) return 2;
    if (kind == PO_KIND_Q2_K || kind == PO_KIND_TQ1_0 || kind == PO_KIND_TQ2_0) return 0;
    if (kind == PO_KIND_PQ2 && cols % 256 == 0) return 0;
    return 1;
}

typedef struct {
    uint32_t kind;
    size_t cols, rows, row_bytes, first, last;
    const uint8_t *w;
    const po_q8k_block *q8k;
    const po_q8_block *q8;
    int pinned;
    float *out;
    int rc;
    size_t err_row;
} job_t;

static int row_dot(const job_t *j, size_t r, float *o) {
    const uint8_t *row = j->w + r * j->row_bytes;
    switch (j->kind) {
    case PO_KIND_Q2_K: return po_dot_q2k(row, j->cols / 256, j->q8k, o);
    case PO_KIND_TQ1_0:
    case PO_KIND_TQ2_0: return po_dot_tq(j->kind, row, j->cols / 256, j->q8k, o);
    case PO_KIND_Q8_0: return po_dot_q8_0(row, j->cols / 32, j->q8, o);
    case PO_KIND_PQ2:
        if (j->q8k) return po_dot_pq2(row, j->cols / 128, j->q8k, j->pinned, o);
        /* odd-group PQ2 uses Q8_0 */
        __attribute__((fallthrough));
    case PO_KIND_PTQ1:
        return j->pinned ? po_dot_q8_groups_pinned(j->kind, row, j->cols / 128, j->q8, o)
                         : po_dot_q8_groups(j->kind, row, j->cols / 128, j->q8, o);
    default: return PO_ERR_UNSUPPORTED;
    }
}

static void *run_job(void *arg) {
    job_t *j = (job_t *)arg;
    j->rc = PO_OK;
    for (size_t r = j->first; r < j->last; r++) {
        int rc = row_dot(j, r, j->out + r);
        if (rc) {
            j->rc = rc;
            j->err_row = r;
            return NULL;
        }
    }
    return NULL;
}

static int run_rows(job_t *proto, int threads) {
    if (threads < 1) threads = 1;
    if ((size_t)threads > proto->rows) threads = (int)proto->rows;
    job_t jobs[256];
    pthread_t tids[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; t++) {
        jobs[t] = *proto;
        jobs[t].first = (size_t)t * proto->rows / (size_t)threads;
        jobs[t].last = (size_t)(t + 1) * proto->rows / (size_t)threads;
    }
    for (int t = 1; t < threads; t++) pthread_create(&tids[t], NULL, run_job, &jobs[t]);
    run_job(&jobs[0]);
    for (int t = 1; t < threads; t++) pthread_join(tids[t], NULL);
    int rc = PO_OK;
    size_t best = (size_t)-1;
    for (int t = 0; t < threads; t++)
        if (jobs[t].rc && jobs[t].err_row < best) {
            best = jobs[t].err_row;
            rc = jobs[t].rc;
        }
    return rc;
}

static int check_geometry(uint32_t kind, size_t cols, size_t rows, size_t *row_bytes) {
    size_t group, bb;
    if (kind != PO_KIND_Q2_K && kind != PO_KIND_Q8_0 && kind != PO_KIND_PQ2 && kind != PO_KIND_PTQ1 &&
        kind != PO_KIND_TQ1_0 && kind != PO_KIND_TQ2_0)
        return PO_ERR_UNSUPPORTED;
    po_layout(kind, &group, &bb);
    if (cols == 0 || rows == 0 || cols % group) return PO_ERR_INVALID_INPUT;
    *row_bytes = cols / group * bb;
    return PO_OK;
}

int po_project_q8k(uint32_t kind, size_t cols, size_t rows, const uint8_t *w,
                   const po_q8k_block *act, int fused, float *out, int threads) {
    job_t j = {0};
    int rc = check_geometry(kind, cols, rows, &j.row_bytes);
    if (!rc && po_activation_contract(kind, cols, 0) != 0) rc = PO_ERR_INVALID_INPUT;
    if (!rc) {
        j.kind = kind; j.cols = cols; j.rows = rows; j.w = w; j.q8k = act; j.pinned = fused; j.out = out;
        rc = run_rows(&j, threads);
    }
    if (rc) memset(out, 0, sizeof(float) * rows);
    return rc;
}

int po_project_q8(uint32_t kind, size_t cols, size_t rows, const uint8_t *w, const po_q8_block *act,
                  int pinned, float *out, int threads) {
    job_t j = {0};
    int rc = check_geometry(kind, cols, rows, &j.row_bytes);
    if (!rc && po_activation_contract(kind, cols, 0) == 0 && kind != PO_KIND_PQ2) rc = PO_ERR_INVALID_INPUT;
    if (!rc) {
        j.kind = kind; j.cols = cols; j.rows = rows; j.w = w; j.q8 = act; j.pinned = pinned; j.out = out;
        rc = run_rows(&j, threads);
    }
    if (rc) memset(out, 0, sizeof(float) * rows);
    return rc;
}

/* kernels::matvec_into with a (pinned or source) MatvecScratch:
 * prepare (src/kernels.rs:1997-2122) then multiply (:2580-2815). */
int po_matvec(uint32_t kind, size_t cols, size_t rows, const uint8_t *w, const float *x,
              int pinned, float *out, int threads) {
    size_t row_bytes;
    int rc = check_geometry(kind, cols, rows, &row_bytes);
    if (rc) {
        memset(out, 0, sizeof(float) * rows);
        return rc;
    }
    int contract = po_activation_contract(kind, cols, pinned);
    if (contract == 0) {
        po_q8k_block *q = (po_q8k_block *)malloc(sizeof(po_q8k_block) * (cols / 256));
        if (!q) return PO_ERR_RESOURCE;
        rc = po_quantize_q8k(x, cols, pinned, q);
        if (!rc) rc = po_project_q8k(kind, cols, rows, w, q, pinned, out, threads);
        free(q);
    } else {
        po_q8_block *q = (po_q8_block *)malloc(sizeof(po_q8_block) * (cols / 32));
        if (!q) return PO_ERR_RESOURCE;
        int qc = contract == 2 ? PO_Q8_PINNED_NATIVE : (pinned ? PO_Q8_PINNED : PO_Q8_SOURCE);
        rc = po_quantize_q8_0(x, cols, qc, q);
        if (!rc) rc = po_project_q8(kind, cols, rows, w, q, pinned, out, threads);
        free(q);
    }
    if (rc) memset(out, 0, sizeof(float) * rows);
    return rc;
}

/* ------------------------------------------------------------------------- */
/* SwiGLU                                                                    */
/* ------------------------------------------------------------------------- */

/* src/kernels/pinned_activations.rs:26-62: ggml's vectorised expf (a published
 * polynomial method), with fmaf exactly where the reference uses mul_add. */
float po_vector_exp(float value) {
    float z = fmaf(value, u2f(0x3fb8aa3bu), 12582912.0f);
    float n = z - 12582912.0f;
    float r = fmaf(-n, u2f(0x3f317200u), value);
    r = fmaf(-n, u2f(0x35bfbe8eu), r);
    uint32_t e = f2u(z) << 23;
    float k = u2f(e + f2u(1.0f));
    float sq = r * r;
    float inner = fmaf(fmaf(u2f(0x3c072010u), r, u2f(0x3d2b9f17u)), sq,
                       fmaf(u2f(0x3e2aaf33u), r, u2f(0x3efffedbu)));
    float poly = fmaf(inner, sq, u2f(0x3f7ffff6u) * r);
    if (fabsf(n) > 126.0f) {
        uint32_t shift = n <= 0.0f ? 0x82000000u : 0u;
        float s1 = u2f(shift + 0x7f000000u);
        if (fabsf(n) > 192.0f) return s1 * s1;
        float s2 = u2f(e - shift);
        return fmaf(s2, poly, s2) * s1;
    }
    return fmaf(poly, k, k);
}

/* Pinned SiLU row (src/kernels/pinned_activations.rs:110-133): x / (1 + vexp(0 - x))
 * for the first len/4*4 values, libm exp for the tail; source SiLU
 * (src/kernels.rs:3365-3368): x / (1 + exp(-x)). */
void po_silu(float *x, size_t n, int pinned) {
    size_t vec = n / 4 * 4;
    for (size_t i = 0; i < n; i++) {
        float v = x[i];
        float den = 1.0f + ((pinned && i < vec) ? po_vector_exp(0.0f - v) : expf(-v));
        x[i] = v / den;
    }
}

/* source: src/graph.rs:121-131 with silu = x/(1+exp(-x)) (src/kernels.rs:3365-3368);
 * pinned: src/kernels/pinned_activations.rs:141-178 (vector exp for the first
 * len/4*4 elements, libm exp for the tail). */
void po_swiglu(const float *gate, float *up, size_t n, int pinned) {
    size_t vec = n / 4 * 4;
    for (size_t i = 0; i < n; i++) {
        float g = gate[i];
        if (pinned) {
            float den = 1.0f + (i < vec ? po_vector_exp(0.0f - g) : expf(-g));
            up[i] = (g * up[i]) / den;
        } else {
            float s = g / (1.0f + expf(-g));
            up[i] = up[i] * s;
        }
    }
}

/* lora_a_dot (src/kernels.rs:2336-2357): a . input with a finite input of matching
 * length.  Pinned with n % 16 == 0: pinned_gdn::dot_scalar (src/kernels/pinned_gdn.rs:
 * 205-230), sixteen binary32 fused multiply-add lanes, register r lane l holding
 * element offset + 4r + l, reduced as (s0 + s2) + (s1 + s3) per lane, then
 * (l0 + l1) + (l2 + l3).  Otherwise float_dot (src/kernels.rs:1256-1273): the binary32
 * products summed in binary64 in index order, rounded to binary32.  A non-finite result
 * is an error (finite, src/kernels.rs:152-163). */
int po_lora_a_dot(const float *a, const float *input, size_t n, int pinned, float *out) {
    *out = 0.0f;
    if (n == 0) return PO_ERR_INVALID_INPUT;
    for (size_t i = 0; i < n; i++)
        if (!is_finite(input[i])) return PO_ERR_INVALID_INPUT;
    float r;
    if (pinned && n % 16 == 0) {
        float sums[4][4] = {{0}};
        for (size_t off = 0; off < n; off += 16)
            for (int reg = 0; reg < 4; reg++)
                for (int lane = 0; lane < 4; lane++) {
                    const size_t i = off + (size_t)reg * 4 + (size_t)lane;
                    sums[reg][lane] = fmaf(a[i], input[i], sums[reg][lane]);
                }
        float lanes[4];
        for (int lane = 0; lane < 4; lane++)
            lanes[lane] = (sums[0][lane] + sums[2][lane]) + (sums[1][lane] + sums[3][lane]);
        r = (lanes[0] + lanes[1]) + (lanes[2] + lanes[3]);
    } else {
        double s = 0.0;
        for (size_t i = 0; i < n; i++) s += (double)(a[i] * input[i]);
        r = (float)s;
    }
    if (!is_finite(r)) return PO_ERR_NONFINITE;
    *out = r;
    return PO_OK;
}

/* gate/up projections sharing one preparation, SwiGLU into up, then down
 * (src/graph.rs:3935-3956); optional residual add as the executor chain does. */
/* hadamard (src/kernels.rs:3952-3987) over every `block` consecutive values: finite input,
 * butterflies with half = 1, 2, 4, ... turning (l, r) into (l + r, l - r) in binary32,
 * then each value times the binary32 1 / sqrt(block); a non-finite result fails. */
int po_hadamard(float *v, size_t n, uint32_t block) {
    if (block == 0 || (block & (block - 1)) || n % block) return PO_ERR_INVALID_INPUT;
    const float norm = 1.0f / sqrtf((float)block);
    for (size_t b = 0; b < n; b += block) {
        float *x = v + b;
        for (uint32_t i = 0; i < block; i++)
            if (!is_finite(x[i])) return PO_ERR_NONFINITE;
        for (uint32_t half = 1; half < block; half *= 2)
            for (uint32_t base = 0; base < block; base += 2 * half)
                for (uint32_t i = base; i < base + half; i++) {
                    const float l = x[i], r = x[i + half];
                    x[i] = l + r;
                    x[i + half] = l - r;
                }
        for (uint32_t i = 0; i < block; i++) {
            x[i] = x[i] * norm;
            if (!is_finite(x[i])) return PO_ERR_NONFINITE;
        }
    }
    return PO_OK;
}

/* The chain with hadamard_block_size (src/kernels/projection.rs:271-290): gate and up
 * matvecs, SwiGLU, then (block > 1) the blockwise Hadamard rotation of the SwiGLU vector
 * ahead of the down matvec (src/graph/prefill_ffn_tests.rs:517-547 rotates `mid` before
 * cpu_matvec(down, ...)); h_out receives the unrotated SwiGLU vector. */
int po_ffn_rotated(uint32_t kind, size_t hidden, size_t ffn, const uint8_t *wg, const uint8_t *wu,
                   const uint8_t *wd, const float *x, const float *residual, uint32_t hadamard_block,
                   int pinned, float *out, float *h_out, int threads) {
    float *g = (float *)malloc(sizeof(float) * ffn);
    float *u = (float *)malloc(sizeof(float) * ffn);
    int rc = (g && u) ? PO_OK : PO_ERR_RESOURCE;
    if (!rc) rc = po_matvec(kind, hidden, ffn, wu, x, pinned, u, threads);
    if (!rc) rc = po_matvec(kind, hidden, ffn, wg, x, pinned, g, threads);
    if (!rc) {
        po_swiglu(g, u, ffn, pinned);
        for (size_t i = 0; i < ffn; i++)
            if (!is_finite(u[i])) rc = PO_ERR_NONFINITE;
    }
    if (!rc && h_out) memcpy(h_out, u, sizeof(float) * ffn);
    if (!rc && hadamard_block > 1) rc = po_hadamard(u, ffn, hadamard_block);
    if (!rc) rc = po_matvec(kind, ffn, hidden, wd, u, pinned, out, threads);
    if (!rc && residual)
        for (size_t i = 0; i < hidden; i++) {
            out[i] = out[i] + residual[i];
            if (!is_finite(out[i])) rc = PO_ERR_NONFINITE;
        }
    if (rc) memset(out, 0, sizeof(float) * hidden);
    free(g);
    free(u);
    return rc;
}

int po_ffn(uint32_t kind, size_t hidden, size_t ffn, const uint8_t *wg, const uint8_t *wu,
           const uint8_t *wd, const float *x, const float *residual, int pinned, float *out,
           float *h_out, int threads) {
    return po_ffn_rotated(kind, hidden, ffn, wg, wu, wd, x, residual, 0, pinned, out, h_out, threads);
}
