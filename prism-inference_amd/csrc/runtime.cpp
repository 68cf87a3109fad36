// runtime.cpp -- context, weight residency, dispatch and the extern "C" ABI of
// libprism_hip.so (declared in include/prism_hip.h).
//
// The executor semantics follow the reference's projection boundary
// (src/kernels/projection.rs): eligibility is decided from geometry before any
// launch, outputs are complete and finite or the call fails with the output
// zero-filled, nothing is replayed elsewhere, and a device fault latches the
// context as unsupported (tools/adreno-vulkan/src/executor.rs:1507-1530).
#include "runtime_internal.hpp"

#include <cmath>

using namespace prism;
using namespace prism::rt;

namespace {

// Token count below which no f32 projection runs as a tiled-prefill GEMM (prefill_supported
// has the last word: its own thresholds per kind, contract and matrix size).
constexpr uint32_t kPrefillMinTokens = 16;

// Quantize device floats with the contract matvec_into would use, then project.  `role`
// is the grow-mode buffer of the quantized activation; sc == nullptr selects grow mode.
int project_f32_dev(prism_hip_ctx *c, const Weight &w, const float *x, uint32_t tokens, int pinned, float *out,
                    DevBuf &role, hipStream_t s, const float *residual = nullptr, Scratch *sc = nullptr) {
    Scratch grow{c};
    Scratch &scr = sc ? *sc : grow;
    if (w.tiled && tokens >= kPrefillMinTokens && prefill_supported(w.kind, w.cols, w.rows, pinned, tokens)) {
        void *pre = nullptr;
        int rc = scr.get(c->pre, prefill_scratch_bytes(w.kind, w.cols, tokens), &pre);
        if (rc) return rc;
        rc = launch_result(c, launch_prefill(w.kind, w.dev, w.cols, w.rows, x, tokens, pinned, out, pre, c->err, s, c->cus),
                           "prefill launch");
        // The residual joins after the projection, one binary32 add per output (as the
        // row kernels do in their epilogue).
        if (!rc && residual)
            rc = launch_result(c, launch_add_residual(out, residual, w.rows * tokens, c->err, s), "residual launch");
        return rc;
    }
    if (w.tiled) {
        MatvecArgs a = f32_args(c, w, x, tokens, pinned, out, residual, s);
        if (!tiled_needs_prepared(a)) return run_matvec(c, a, true, &scr);
    }
    const int contract = contract_for(w.kind, w.cols, pinned);
    void *act = nullptr;
    int rc = scr.get(role, act_bytes(contract, w.cols, tokens), &act);
    if (rc) return rc;
    rc = quantize(c, contract, x, w.cols, tokens, pinned, act, s);
    if (rc) return rc;
    MatvecArgs a = matvec_args(c, w, contract == 0 ? kActQ8K : kActQ8, act, tokens, pinned, out, s);
    if (w.tiled) a.residual = residual;
    rc = run_matvec(c, a, w.tiled, &scr);
    if (!rc && residual && !w.tiled)
        rc = launch_result(c, launch_add_residual(out, residual, w.rows * tokens, c->err, s), "residual launch");
    return rc;
}

bool eligible(uint32_t kind, uint64_t cols, uint64_t rows, int path) {
    uint64_t g, b;
    if (!layout(kind, &g, &b) || cols == 0 || rows == 0 || cols % g) return false;
    if (rows > 0xffffffffull || cols > 0xffffffffull) return false;
    switch (path) {
    case PRISM_PATH_Q8K:
        if (kind == PRISM_KIND_PQ2) return cols % 256 == 0;
        return kind == PRISM_KIND_Q2_K || kind == PRISM_KIND_PTQ1 || kind == PRISM_KIND_TQ1_0 ||
               kind == PRISM_KIND_TQ2_0;
    case PRISM_PATH_Q8: return kind == PRISM_KIND_PTQ1 || kind == PRISM_KIND_PQ2 || kind == PRISM_KIND_Q8_0;
    case PRISM_PATH_F32: return true;
    default: return false;
    }
}

// Whether two tensors take one activation contract under both pinned settings, so one
// quantized input serves both whatever the caller passes as `pinned`.
bool same_contract(uint32_t k0, uint64_t c0, uint32_t k1, uint64_t c1) {
    return c0 == c1 && contract_for(k0, c0, 0) == contract_for(k1, c1, 0) &&
           contract_for(k0, c0, 1) == contract_for(k1, c1, 1);
}

// supports_f32_group: 1..8 direct-F32 siblings sharing one input width and contract.
bool group_eligible(const prism_tensor_desc *t, uint32_t n) {
    if (!t || n == 0 || n > 8) return false;
    for (uint32_t i = 0; i < n; ++i) {
        if (!eligible(t[i].kind, t[i].cols, t[i].rows, PRISM_PATH_F32)) return false;
        if (!same_contract(t[0].kind, t[0].cols, t[i].kind, t[i].cols)) return false;
    }
    return true;
}

// The packed kinds the FFN chains run on, one kind for gate, up and down.
bool ffn_kind(uint32_t kind) {
    return kind == PRISM_KIND_PQ2 || kind == PRISM_KIND_Q2_K || kind == PRISM_KIND_PTQ1 || kind == PRISM_KIND_Q8_0 ||
           kind == PRISM_KIND_TQ1_0 || kind == PRISM_KIND_TQ2_0;
}

// supports_f32_ffn_swiglu / supports_f32_ffn_chain: gate and up [ffn][hidden] of one
// kind; down (if given) [hidden][ffn] of the same kind.
bool ffn_eligible(const prism_tensor_desc &g, const prism_tensor_desc &u, const prism_tensor_desc *d) {
    if (!ffn_kind(g.kind) || g.kind != u.kind || g.cols != u.cols || g.rows != u.rows) return false;
    if (!eligible(g.kind, g.cols, g.rows, PRISM_PATH_F32)) return false;
    if (!d) return true;
    return d->kind == g.kind && d->cols == g.rows && d->rows == g.cols &&
           eligible(d->kind, d->cols, d->rows, PRISM_PATH_F32);
}

prism_tensor_desc desc_of(const Weight &w) { return prism_tensor_desc{w.kind, w.cols, w.rows}; }

void zero(float *p, size_t n) {
    if (p) std::memset(p, 0, sizeof(float) * n);
}

// Shared front half of the projections.  *out is the weight whenever the id is known,
// also when the call then fails, so the caller can clear rows*tokens outputs.
int prepare_weight(prism_hip_ctx *c, prism_weight_id wid, int path, const Weight **out) {
    *out = nullptr;
    if (!c) return PRISM_ERR_INVALID_INPUT;
    const Weight *w = find(c, wid);
    *out = w;
    int rc = check_ready(c);
    if (rc) return rc;
    if (!w) return fail(c, PRISM_ERR_INVALID_INPUT, "unknown weight id");
    if (!eligible(w->kind, w->cols, w->rows, path))
        return fail(c, PRISM_ERR_UNSUPPORTED, "projection not supported for this tensor");
    return PRISM_OK;
}

int finish(prism_hip_ctx *c, float *host_out, const float *dev_out, size_t n) {
    hipError_t e = hipMemcpyAsync(host_out, dev_out, sizeof(float) * n, hipMemcpyDeviceToHost, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "copy output");
    return drain(c, c->stream);
}

// The Hadamard block of a rotated down projection (project_f32_ffn_chain's
// hadamard_block_size, src/kernels/projection.rs:277-301): 0 or 1 = none; otherwise a power
// of two from 2 to kHadamardMaxBlock dividing the SwiGLU width, as the GPU precedent accepts
// (tools/adreno-vulkan/src/executor.rs:2493-2507, there up to 1024).
bool hadamard_ok(uint32_t hb, uint64_t ffn) {
    return hb <= 1 || ((hb & (hb - 1)) == 0 && hb <= kHadamardMaxBlock && ffn % hb == 0);
}

// The down projection's input: the SwiGLU rows hv, or (hb > 1) their blockwise Hadamard
// rotation in c->hr (the reference rotates the SwiGLU vector ahead of the quantizer,
// src/graph.rs:4168-4276 with src/kernels.rs:3952-4021); hv itself stays unrotated.
int down_input(prism_hip_ctx *c, const float *hv, uint64_t ffn, uint32_t tokens, uint32_t hb, hipStream_t s,
               const float **in) {
    *in = hv;
    if (hb <= 1) return PRISM_OK;
    int rc = ensure(c, c->hr, sizeof(float) * ffn * tokens);
    if (rc) return rc;
    float *hr = static_cast<float *>(c->hr.p);
    rc = launch_result(c, launch_hadamard(hv, hr, ffn, tokens, hb, c->err, s), "hadamard launch");
    if (!rc) *in = hr;
    return rc;
}

int ffn_chain_impl(prism_hip_ctx *c, const Weight &g, const Weight &u, const Weight *d, const float *x,
                   const float *residual, int pinned, float *out, float *h, hipStream_t s, uint32_t hb = 0) {
    // Shapes: gate/up [ffn][hidden], down [hidden][ffn] (projection.rs:571-597).
    if (g.cols != u.cols || g.rows != u.rows || g.kind != u.kind)
        return fail(c, PRISM_ERR_INVALID_INPUT, "gate/up geometry differs");
    if (d && (d->cols != g.rows || d->rows != g.cols))
        return fail(c, PRISM_ERR_INVALID_INPUT, "down geometry does not match gate/up");
    if (!hadamard_ok(hb, g.rows))
        return fail(c, PRISM_ERR_INVALID_INPUT, "Hadamard block must be a power of two up to 8192 dividing the FFN width");
    if (!d) hb = 0;
    float *hv = h;
    int rc = PRISM_OK;
    if (!hv) {
        rc = ensure(c, c->h, sizeof(float) * g.rows);
        if (rc) return rc;
        hv = static_cast<float *>(c->h.p);
    }
    bool fused = false;
    if (g.tiled && u.tiled) {
        // gate, up and SwiGLU in one launch, x quantized in the prologue.
        MatvecArgs a = f32_args(c, g, x, 1, pinned, hv, nullptr, s);
        a.w2 = static_cast<const uint8_t *>(u.dev);
        // A tiled down matrix on Q8_0 activations takes the SwiGLU vector as blocks the
        // gate/up epilogue quantizes (its contract, per 32 rows), not as floats -- unless
        // the vector is rotated first.
        const int dc = d ? contract_for(d->kind, d->cols, pinned) : 0;
        if (d && d->tiled && dc != 0 && g.rows % 32 == 0 && hb <= 1) {
            rc = ensure(c, c->act2, act_bytes(dc, d->cols, 1));
            if (rc) return rc;
            a.q8_out = c->act2.p;
            a.q8_contract = dc == 2 ? PRISM_Q8_PINNED_NATIVE : (pinned ? PRISM_Q8_PINNED : PRISM_Q8_SOURCE);
            a.out = h;  // the floats only when the caller asked for them
        }
        if (!tiled_needs_prepared(a)) {
            rc = run_matvec(c, a, true);
            if (rc) return rc;
            fused = true;
            if (a.q8_out) {
                MatvecArgs da = matvec_args(c, *d, kActQ8, a.q8_out, 1, pinned, out, s);
                da.residual = residual;
                return run_matvec(c, da, true);
            }
        }
    }
    if (!fused) {
        rc = ensure(c, c->gate, sizeof(float) * g.rows);
        if (!rc) rc = ensure(c, c->up, sizeof(float) * g.rows);
        if (rc) return rc;
        const int contract = contract_for(g.kind, g.cols, pinned);
        rc = ensure(c, c->act, act_bytes(contract, g.cols, 1));
        if (!rc) rc = quantize(c, contract, x, g.cols, 1, pinned, c->act.p, s);
        if (!rc)
            rc = matvec(c, g, contract == 0 ? kActQ8K : kActQ8, c->act.p, 1, pinned, static_cast<float *>(c->gate.p), s);
        if (!rc)
            rc = matvec(c, u, contract == 0 ? kActQ8K : kActQ8, c->act.p, 1, pinned, static_cast<float *>(c->up.p), s);
        if (rc) return rc;
        rc = launch_result(c,
                           launch_swiglu(static_cast<float *>(c->gate.p), static_cast<float *>(c->up.p), hv, g.rows, 1,
                                         pinned, c->err, s),
                           "swiglu launch");
        if (rc) return rc;
    }
    if (!d) return PRISM_OK;
    const float *din = nullptr;
    rc = down_input(c, hv, g.rows, 1, hb, s, &din);
    if (rc) return rc;
    return project_f32_dev(c, *d, din, 1, pinned, out, c->act2, s, residual);
}

// Sibling projections of `tokens` token rows of one f32 input (device pointers):
// outs[i] receives [tokens][rows_i].  A member whose kernel prepares its own codes (the
// tiled-prefill GEMM, or a single token's quantizing prologue) takes x directly; the
// others share one quantization of x, as the reference's sibling groups share one
// prepared activation (src/kernels/siblings.rs:30, src/graph.rs:1880-2003).  The
// members share a contract (group_eligible), so every output is its own
// project_f32's.
int group_tokens_impl(prism_hip_ctx *c, const Weight *const *w, uint32_t n, const float *x, uint32_t tokens,
                      int pinned, float *const *outs, hipStream_t s) {
    const int contract = contract_for(w[0]->kind, w[0]->cols, pinned);
    bool prepared = false;
    for (uint32_t i = 0; i < n; ++i) {
        const Weight &wi = *w[i];
        bool own = wi.tiled && tokens >= kPrefillMinTokens && prefill_supported(wi.kind, wi.cols, wi.rows, pinned, tokens);
        if (!own && wi.tiled && tokens == 1) own = !tiled_needs_prepared(f32_args(c, wi, x, 1, pinned, outs[i], nullptr, s));
        int rc;
        if (own) {
            rc = project_f32_dev(c, wi, x, tokens, pinned, outs[i], c->act, s);
        } else {
            if (!prepared) {
                rc = ensure(c, c->act, act_bytes(contract, wi.cols, tokens));
                if (!rc) rc = quantize(c, contract, x, wi.cols, tokens, pinned, c->act.p, s);
                if (rc) return rc;
                prepared = true;
            }
            rc = matvec(c, wi, contract == 0 ? kActQ8K : kActQ8, c->act.p, tokens, pinned, outs[i], s);
        }
        if (rc) return rc;
    }
    return PRISM_OK;
}

// The FFN chain over `tokens` token rows (device pointers): x [tokens][hidden] ->
// SwiGLU [tokens][ffn] -> (down) out [tokens][hidden] (+ residual).  One token runs the
// fused single-token chain; more run gate and up as one sibling group over all tokens
// (multi-token kernels read each weight once per batch), one SwiGLU launch, and down
// over all tokens.  Every token row is its own single-token chain's result.  h, if not
// NULL, receives the SwiGLU rows; without a down projection `out` is that vector.
int ffn_tokens_impl(prism_hip_ctx *c, const Weight &g, const Weight &u, const Weight *d, const float *x,
                    const float *residual, uint32_t tokens, int pinned, float *out, float *h, hipStream_t s,
                    uint32_t hb = 0) {
    const prism_tensor_desc dd = d ? desc_of(*d) : prism_tensor_desc{};
    if (!ffn_eligible(desc_of(g), desc_of(u), d ? &dd : nullptr))
        return fail(c, PRISM_ERR_UNSUPPORTED, "FFN chain needs gate/up [ffn][hidden] and down [hidden][ffn] of one packed kind");
    if (!hadamard_ok(hb, g.rows))
        return fail(c, PRISM_ERR_INVALID_INPUT, "Hadamard block must be a power of two up to 8192 dividing the FFN width");
    if (tokens == 1) return ffn_chain_impl(c, g, u, d, x, residual, pinned, d ? out : nullptr, d ? h : out, s, hb);
    const size_t nh = sizeof(float) * g.rows * tokens;
    int rc = ensure(c, c->gate, nh);
    if (!rc) rc = ensure(c, c->up, nh);
    float *hv = d ? h : out;
    if (!rc && !hv) {
        rc = ensure(c, c->h, nh);
        hv = static_cast<float *>(c->h.p);
    }
    if (rc) return rc;
    const Weight *gu[2] = {&g, &u};
    float *gu_out[2] = {static_cast<float *>(c->gate.p), static_cast<float *>(c->up.p)};
    rc = group_tokens_impl(c, gu, 2, x, tokens, pinned, gu_out, s);
    if (!rc)
        rc = launch_result(c, launch_swiglu(gu_out[0], gu_out[1], hv, g.rows, tokens, pinned, c->err, s),
                           "swiglu launch");
    if (rc || !d) return rc;
    const float *din = nullptr;
    rc = down_input(c, hv, g.rows, tokens, hb, s, &din);
    if (rc) return rc;
    return project_f32_dev(c, *d, din, tokens, pinned, out, c->act2, s, residual);
}

}  // namespace

extern "C" {

prism_hip_ctx *prism_hip_create(int device, uint64_t max_resident_bytes, uint32_t flags) {
    if (flags != 0) return nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return nullptr;
    if (hipSetDevice(device) != hipSuccess) return nullptr;
    auto *c = new prism_hip_ctx();
    c->device = device;
    c->max_resident = max_resident_bytes;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess || hipStreamCreate(&c->stream) != hipSuccess ||
        hipMalloc(&c->err, sizeof(int)) != hipSuccess || hipMemset(c->err, 0, sizeof(int)) != hipSuccess) {
        delete c;
        return nullptr;
    }
    c->cus = static_cast<uint32_t>(prop.multiProcessorCount);
    // With `device` current: this GPU's copy of the no-allocation entry point's scratch.
    const hipError_t se = static_scratch_address(device, &c->noalloc, &c->noalloc_bytes);
    if (se != hipSuccess) {
        c->noalloc = nullptr;
        c->noalloc_bytes = 0;
        c->noalloc_error = std::string("static scratch lookup: ") + hipGetErrorString(se);
    }
    char buf[256];
    std::snprintf(buf, sizeof buf, "prism-hip/%s/%d-cu/exact-scalar-order", prop.gcnArchName, prop.multiProcessorCount);
    c->identity = buf;
    return c;
}

void prism_hip_destroy(prism_hip_ctx *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    prism_hip_weight_release_all(c);
    for (DevBuf *b : {&c->x, &c->act, &c->act2, &c->out, &c->gate, &c->up, &c->h, &c->hr, &c->res, &c->pre, &c->sk, &c->lora})
        if (b->p) (void)hipFree(b->p);
    if (c->err) (void)hipFree(c->err);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

const char *prism_hip_identity(const prism_hip_ctx *c) { return c ? c->identity.c_str() : ""; }
const char *prism_hip_last_error(const prism_hip_ctx *c) { return c ? c->last_error.c_str() : "null context"; }
int prism_hip_faulted(const prism_hip_ctx *c) { return c ? (c->faulted ? 1 : 0) : 1; }
int prism_hip_inject_fault(prism_hip_ctx *c) {
    if (!c) return PRISM_ERR_INVALID_INPUT;
    c->faulted = true;
    c->last_error = "device fault latched by prism_hip_inject_fault";
    return PRISM_OK;
}
uint64_t prism_hip_operation_capacity(const prism_hip_ctx *c) { return (!c || c->faulted) ? 0 : UINT64_MAX; }

int64_t prism_hip_operation_count(const prism_hip_ctx *c, uint32_t kind, uint64_t cols, uint64_t rows) {
    if (!c || c->faulted) return -1;
    if (!eligible(kind, cols, rows, PRISM_PATH_F32)) return -1;
    return static_cast<int64_t>(cols * rows);
}

int prism_hip_supports(const prism_hip_ctx *c, uint32_t kind, uint64_t cols, uint64_t rows, int path) {
    if (!c || c->faulted) return 0;
    return eligible(kind, cols, rows, path) ? 1 : 0;
}

int prism_hip_supports_f32_group(const prism_hip_ctx *c, const prism_tensor_desc *tensors, uint32_t n) {
    if (!c || c->faulted) return 0;
    return group_eligible(tensors, n) ? 1 : 0;
}

int prism_hip_supports_f32_ffn_swiglu(const prism_hip_ctx *c, const prism_tensor_desc *gate,
                                      const prism_tensor_desc *up) {
    if (!c || c->faulted || !gate || !up) return 0;
    return ffn_eligible(*gate, *up, nullptr) ? 1 : 0;
}

int prism_hip_supports_f32_ffn_chain(const prism_hip_ctx *c, const prism_tensor_desc *tensors) {
    if (!c || c->faulted || !tensors) return 0;
    return ffn_eligible(tensors[0], tensors[1], &tensors[2]) ? 1 : 0;
}

int prism_hip_supports_f32_ffn_chain_lora(const prism_hip_ctx *c, const prism_tensor_desc *tensors) {
    return prism_hip_supports_f32_ffn_chain(c, tensors);
}

int prism_hip_supports_tile_tokens(const prism_hip_ctx *c) { return (!c || c->faulted) ? 0 : 1; }

uint64_t prism_hip_weight_tiled_bytes(const prism_hip_ctx *c, uint32_t kind, uint64_t cols, uint64_t rows) {
    uint64_t g, b;
    if (!c || !layout(kind, &g, &b) || cols == 0 || rows == 0 || cols % g) return 0;
    if (!tiled_supported(kind, cols, rows, c->cus)) return 0;
    return tiled_bytes(rows, cols / g * b);
}

static prism_weight_id add_weight(prism_hip_ctx *c, uint64_t key, uint32_t kind, uint64_t cols, uint64_t rows,
                                  uint64_t bytes, bool owned, void *dev) {
    Weight w;
    w.key = key;
    w.kind = kind;
    w.cols = cols;
    w.rows = rows;
    uint64_t g, b;
    layout(kind, &g, &b);
    w.row_bytes = cols / g * b;
    w.bytes = bytes;
    w.dev = dev;
    w.owned = owned;
    const int64_t id = c->next_id++;
    c->weights[id] = w;
    if (owned) {
        c->resident += bytes;
        c->by_key[key] = id;
    }
    return id;
}

static int check_geometry(prism_hip_ctx *c, uint32_t kind, uint64_t cols, uint64_t rows, uint64_t bytes) {
    uint64_t g, b;
    if (!layout(kind, &g, &b)) return fail(c, PRISM_ERR_UNSUPPORTED, "unsupported tensor kind");
    if (cols == 0 || rows == 0 || cols % g) return fail(c, PRISM_ERR_INVALID_INPUT, "incomplete blocks");
    if (rows > 0xffffffffull || cols > 0xffffffffull) return fail(c, PRISM_ERR_INVALID_INPUT, "extent overflow");
    if (cols / g * b * rows != bytes) return fail(c, PRISM_ERR_INVALID_INPUT, "byte extent mismatch");
    return PRISM_OK;
}

// Copies native device bytes into a context-owned buffer, repacked into the tiled
// layout when the geometry allows it (the native copy serves every other shape).
static prism_weight_id store_weight(prism_hip_ctx *c, uint64_t key, uint32_t kind, uint64_t cols, uint64_t rows,
                                    const void *native, uint64_t bytes) {
    const bool tiled = tiled_supported(kind, cols, rows, c->cus);
    const uint64_t row_bytes = bytes / rows;
    const uint64_t dev_bytes = tiled ? tiled_bytes(rows, row_bytes) : bytes;
    void *dev = nullptr;
    hipError_t e = hipMalloc(&dev, dev_bytes);
    if (e != hipSuccess) return hip_fail(c, e, "hipMalloc(weights)");
    if (tiled) {
        e = hipMemsetAsync(dev, 0, dev_bytes, c->stream);
        if (e == hipSuccess) {
            const int lr = launch_repack(native, dev, kind, cols, rows, c->stream);
            if (lr < 0) {
                (void)hipFree(dev);
                return fail(c, PRISM_ERR_UNSUPPORTED, "no tiled layout for this tensor");
            }
            e = static_cast<hipError_t>(lr);
        }
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    } else {
        e = hipMemcpy(dev, native, bytes, hipMemcpyDeviceToDevice);
    }
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail(c, e, "store weights");
    }
    const prism_weight_id id = add_weight(c, key, kind, cols, rows, bytes, true, dev);
    c->weights[id].tiled = tiled;
    c->resident += dev_bytes - bytes;
    c->weights[id].bytes = dev_bytes;
    return id;
}

prism_weight_id prism_hip_weight_acquire(prism_hip_ctx *c, uint64_t key, uint32_t kind, uint64_t cols, uint64_t rows,
                                         const void *host, uint64_t bytes) {
    int rc = check_live(c);
    if (rc) return rc;
    if (!host) return fail(c, PRISM_ERR_INVALID_INPUT, "null weight bytes");
    rc = check_geometry(c, kind, cols, rows, bytes);
    if (rc) return rc;
    auto k = c->by_key.find(key);
    if (k != c->by_key.end()) {
        const Weight *w = find(c, k->second);
        if (w && w->kind == kind && w->cols == cols && w->rows == rows) return k->second;
        return fail(c, PRISM_ERR_INVALID_INPUT, "key already bound to a different tensor");
    }
    if (c->max_resident && c->resident + bytes > c->max_resident)
        return fail(c, PRISM_ERR_RESOURCE, "resident weight budget exceeded");
    void *staging = nullptr;
    hipError_t e = hipMalloc(&staging, bytes);
    if (e != hipSuccess) return hip_fail(c, e, "hipMalloc(weight staging)");
    e = hipMemcpy(staging, host, bytes, hipMemcpyHostToDevice);
    prism_weight_id id = e == hipSuccess ? store_weight(c, key, kind, cols, rows, staging, bytes)
                                         : hip_fail(c, e, "upload weights");
    (void)hipFree(staging);
    return id;
}

prism_weight_id prism_hip_weight_acquire_device(prism_hip_ctx *c, uint64_t key, uint32_t kind, uint64_t cols,
                                                uint64_t rows, const void *device_ptr, uint64_t bytes) {
    int rc = check_live(c);
    if (rc) return rc;
    if (!device_ptr) return fail(c, PRISM_ERR_INVALID_INPUT, "null weight bytes");
    rc = check_geometry(c, kind, cols, rows, bytes);
    if (rc) return rc;
    auto k = c->by_key.find(key);
    if (k != c->by_key.end()) {
        const Weight *w = find(c, k->second);
        if (w && w->kind == kind && w->cols == cols && w->rows == rows) return k->second;
        return fail(c, PRISM_ERR_INVALID_INPUT, "key already bound to a different tensor");
    }
    if (c->max_resident && c->resident + bytes > c->max_resident)
        return fail(c, PRISM_ERR_RESOURCE, "resident weight budget exceeded");
    return store_weight(c, key, kind, cols, rows, device_ptr, bytes);
}

prism_weight_id prism_hip_weight_wrap_device(prism_hip_ctx *c, uint32_t kind, uint64_t cols, uint64_t rows,
                                             const void *dev, uint64_t bytes) {
    int rc = check_live(c);
    if (rc) return rc;
    if (!dev) return fail(c, PRISM_ERR_INVALID_INPUT, "null device pointer");
    rc = check_geometry(c, kind, cols, rows, bytes);
    if (rc) return rc;
    return add_weight(c, 0, kind, cols, rows, bytes, false, const_cast<void *>(dev));
}

int prism_hip_weight_repack_tiled(prism_hip_ctx *c, uint32_t kind, uint64_t cols, uint64_t rows,
                                  const void *native_dev, uint64_t native_bytes, void *tiled_dev,
                                  uint64_t tiled_bytes_) {
    int rc = check_live(c);
    if (rc) return rc;
    if (!native_dev || !tiled_dev) return fail(c, PRISM_ERR_INVALID_INPUT, "null device pointer");
    rc = check_geometry(c, kind, cols, rows, native_bytes);
    if (rc) return rc;
    const uint64_t need = prism_hip_weight_tiled_bytes(c, kind, cols, rows);
    if (need == 0) return fail(c, PRISM_ERR_UNSUPPORTED, "no tiled layout for this tensor on this device");
    if (tiled_bytes_ != need) return fail(c, PRISM_ERR_INVALID_INPUT, "tiled buffer size differs from prism_hip_weight_tiled_bytes");
    // Padding rows of the last tile must read as zero weights: clear, then scatter the
    // native bytes.  (The call synchronizes, so it cannot sit inside a graph capture.)
    HIP_OR_FAIL(c, hipMemsetAsync(tiled_dev, 0, need, c->stream));
    rc = launch_result(c, launch_repack(native_dev, tiled_dev, kind, cols, rows, c->stream), "repack launch");
    if (rc) return rc;
    HIP_OR_FAIL(c, hipStreamSynchronize(c->stream));
    return PRISM_OK;
}

prism_weight_id prism_hip_weight_wrap_tiled(prism_hip_ctx *c, uint32_t kind, uint64_t cols, uint64_t rows,
                                            const void *tiled_dev, uint64_t tiled_bytes_) {
    int rc = check_live(c);
    if (rc) return rc;
    if (!tiled_dev) return fail(c, PRISM_ERR_INVALID_INPUT, "null device pointer");
    uint64_t g, b;
    if (!layout(kind, &g, &b)) return fail(c, PRISM_ERR_UNSUPPORTED, "unsupported tensor kind");
    if (cols == 0 || rows == 0 || cols % g) return fail(c, PRISM_ERR_INVALID_INPUT, "incomplete blocks");
    const uint64_t need = prism_hip_weight_tiled_bytes(c, kind, cols, rows);
    if (need == 0) return fail(c, PRISM_ERR_UNSUPPORTED, "no tiled layout for this tensor on this device");
    if (tiled_bytes_ != need) return fail(c, PRISM_ERR_INVALID_INPUT, "tiled buffer size differs from prism_hip_weight_tiled_bytes");
    const prism_weight_id id = add_weight(c, 0, kind, cols, rows, need, false, const_cast<void *>(tiled_dev));
    c->weights[id].tiled = true;
    return id;
}

int prism_hip_weight_release(prism_hip_ctx *c, prism_weight_id id) {
    if (!c) return PRISM_ERR_INVALID_INPUT;
    auto it = c->weights.find(id);
    if (it == c->weights.end()) return fail(c, PRISM_ERR_INVALID_INPUT, "unknown weight id");
    if (it->second.owned) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipFree(it->second.dev);
        c->resident -= it->second.bytes;
        c->by_key.erase(it->second.key);
    }
    c->weights.erase(it);
    return PRISM_OK;
}

int prism_hip_weight_release_all(prism_hip_ctx *c) {
    if (!c) return PRISM_ERR_INVALID_INPUT;
    (void)hipStreamSynchronize(c->stream);
    for (auto &kv : c->weights)
        if (kv.second.owned) (void)hipFree(kv.second.dev);
    c->weights.clear();
    c->by_key.clear();
    c->resident = 0;
    return PRISM_OK;
}

uint64_t prism_hip_resident_bytes(const prism_hip_ctx *c) { return c ? c->resident : 0; }

static int project_q8k_host(prism_hip_ctx *c, prism_weight_id wid, const prism_q8k_block *act, uint64_t nblocks,
                            uint32_t tokens, int fused, float *out, Tally &t) {
    const Weight *w = nullptr;
    int rc = prepare_weight(c, wid, PRISM_PATH_Q8K, &w);
    if (rc) {
        if (w) zero(out, w->rows * tokens);
        return rc;
    }
    const size_t n = w->rows * tokens;
    if (!act || !out || tokens == 0 || nblocks != (w->cols + 255) / 256 * tokens) {
        zero(out, n);
        return fail(c, PRISM_ERR_INVALID_INPUT, "Q8_K activation extent mismatch");
    }
    t.dispatch();
    const size_t ab = sizeof(prism_q8k_block) * nblocks;
    rc = ensure(c, c->act, ab);
    if (!rc) rc = ensure(c, c->out, sizeof(float) * n);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(c->act.p, act, ab, hipMemcpyHostToDevice, c->stream);
        rc = e == hipSuccess ? PRISM_OK : hip_fail(c, e, "upload activations");
    }
    if (!rc) rc = matvec(c, *w, kActQ8K, c->act.p, tokens, fused, static_cast<float *>(c->out.p), c->stream);
    if (!rc) rc = finish(c, out, static_cast<float *>(c->out.p), n);
    if (rc) zero(out, n);
    return rc;
}

int prism_hip_project_q8k(prism_hip_ctx *c, prism_weight_id wid, const prism_q8k_block *act, uint64_t nblocks,
                          uint32_t tokens, int fused, float *out) {
    Tally t(c, 1, false);
    return t(project_q8k_host(c, wid, act, nblocks, tokens, fused, out, t));
}

static int project_q8_host(prism_hip_ctx *c, prism_weight_id wid, const prism_q8_block *act, uint64_t nblocks,
                           uint32_t tokens, int pinned, float *out, Tally &t) {
    const Weight *w = nullptr;
    int rc = prepare_weight(c, wid, PRISM_PATH_Q8, &w);
    if (rc) {
        if (w) zero(out, w->rows * tokens);
        return rc;
    }
    const size_t n = w->rows * tokens;
    if (!act || !out || tokens == 0 || nblocks != w->cols / 32 * tokens) {
        zero(out, n);
        return fail(c, PRISM_ERR_INVALID_INPUT, "Q8_0 activation extent mismatch");
    }
    t.dispatch();
    const size_t ab = sizeof(prism_q8_block) * nblocks;
    rc = ensure(c, c->act, ab);
    if (!rc) rc = ensure(c, c->out, sizeof(float) * n);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(c->act.p, act, ab, hipMemcpyHostToDevice, c->stream);
        rc = e == hipSuccess ? PRISM_OK : hip_fail(c, e, "upload activations");
    }
    if (!rc) rc = matvec(c, *w, kActQ8, c->act.p, tokens, pinned, static_cast<float *>(c->out.p), c->stream);
    if (!rc) rc = finish(c, out, static_cast<float *>(c->out.p), n);
    if (rc) zero(out, n);
    return rc;
}

int prism_hip_project_q8(prism_hip_ctx *c, prism_weight_id wid, const prism_q8_block *act, uint64_t nblocks,
                         uint32_t tokens, int pinned, float *out) {
    Tally t(c, 1, false);
    return t(project_q8_host(c, wid, act, nblocks, tokens, pinned, out, t));
}

static int project_f32_checked(prism_hip_ctx *c, prism_weight_id wid, const float *x, uint32_t tokens, int pinned,
                               float *out, Tally &t) {
    const Weight *w = nullptr;
    int rc = prepare_weight(c, wid, PRISM_PATH_F32, &w);
    if (rc) {
        if (w) zero(out, w->rows * tokens);
        return rc;
    }
    const size_t n = w->rows * tokens;
    if (!x || !out || tokens == 0) {
        t.bad_input();
        zero(out, n);
        return fail(c, PRISM_ERR_INVALID_INPUT, "null input or output");
    }
    t.dispatch();
    rc = ensure(c, c->x, sizeof(float) * w->cols * tokens);
    if (!rc) rc = ensure(c, c->out, sizeof(float) * n);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(c->x.p, x, sizeof(float) * w->cols * tokens, hipMemcpyHostToDevice, c->stream);
        rc = e == hipSuccess ? PRISM_OK : hip_fail(c, e, "upload activations");
    }
    if (!rc)
        rc = project_f32_dev(c, *w, static_cast<float *>(c->x.p), tokens, pinned, static_cast<float *>(c->out.p),
                             c->act, c->stream);
    if (!rc) rc = finish(c, out, static_cast<float *>(c->out.p), n);
    if (rc) zero(out, n);
    return rc;
}

static int project_f32_host(prism_hip_ctx *c, prism_weight_id wid, const float *x, uint32_t tokens, int pinned,
                            float *out) {
    Tally t(c, 1, true);
    return t(project_f32_checked(c, wid, x, tokens, pinned, out, t));
}

int prism_hip_project_f32(prism_hip_ctx *c, prism_weight_id w, const float *x, uint32_t tokens, int pinned,
                          float *out) {
    return project_f32_host(c, w, x, tokens, pinned, out);
}

int prism_hip_prefill(prism_hip_ctx *c, prism_weight_id w, const float *x, uint32_t tokens, int pinned, float *out) {
    return project_f32_host(c, w, x, tokens, pinned, out);
}

int prism_hip_mul_mat(prism_hip_ctx *c, prism_weight_id a, const float *b, uint32_t ncols, float *out) {
    return project_f32_host(c, a, b, ncols, 0, out);
}

// Host-pointer sibling group over `tokens` token rows: outs[i] receives [tokens][rows_i].
static int group_checked(prism_hip_ctx *c, const prism_weight_id *ws, uint32_t n, const float *x, uint32_t tokens,
                         int pinned, float *const *outs, Tally &tally) {
    if (!c) return PRISM_ERR_INVALID_INPUT;
    if (!ws || !outs || n == 0 || n > 8) return fail(c, PRISM_ERR_INVALID_INPUT, "bad projection group");
    const Weight *w[8] = {};
    for (uint32_t i = 0; i < n; ++i) w[i] = find(c, ws[i]);
    // Clears every output whose weight is known (the others have no known length).
    auto clear = [&](int code) {
        for (uint32_t i = 0; i < n; ++i)
            if (w[i] && outs[i]) zero(outs[i], w[i]->rows * tokens);
        return code;
    };
    int rc = check_ready(c);
    if (rc) return clear(rc);
    if (!x || tokens == 0) {
        tally.bad_input();
        return clear(fail(c, PRISM_ERR_INVALID_INPUT, "null input or no tokens"));
    }
    prism_tensor_desc t[8];
    for (uint32_t i = 0; i < n; ++i) {
        if (!w[i] || !outs[i]) return clear(fail(c, PRISM_ERR_INVALID_INPUT, "unknown weight id in group"));
        t[i] = desc_of(*w[i]);
    }
    if (!group_eligible(t, n))
        return clear(fail(c, PRISM_ERR_UNSUPPORTED, "group members do not share an input width and activation contract"));
    tally.dispatch();
    uint64_t total = 0;
    for (uint32_t i = 0; i < n; ++i) total += w[i]->rows;
    const uint64_t cols = w[0]->cols;
    rc = ensure(c, c->x, sizeof(float) * cols * tokens);
    if (!rc) rc = ensure(c, c->out, sizeof(float) * total * tokens);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(c->x.p, x, sizeof(float) * cols * tokens, hipMemcpyHostToDevice, c->stream);
        rc = e == hipSuccess ? PRISM_OK : hip_fail(c, e, "upload activations");
    }
    float *dev_out[8];
    uint64_t off = 0;
    for (uint32_t i = 0; i < n; ++i) {
        dev_out[i] = static_cast<float *>(c->out.p) + off;
        off += w[i]->rows * tokens;
    }
    if (!rc) rc = group_tokens_impl(c, w, n, static_cast<const float *>(c->x.p), tokens, pinned, dev_out, c->stream);
    for (uint32_t i = 0; i < n && !rc; ++i) {
        hipError_t e = hipMemcpyAsync(outs[i], dev_out[i], sizeof(float) * w[i]->rows * tokens, hipMemcpyDeviceToHost,
                                      c->stream);
        if (e != hipSuccess) rc = hip_fail(c, e, "copy group output");
    }
    if (!rc) rc = drain(c, c->stream);
    return rc ? clear(rc) : rc;
}

static int group_host(prism_hip_ctx *c, const prism_weight_id *ws, uint32_t n, const float *x, uint32_t tokens,
                      int pinned, float *const *outs) {
    Tally t(c, ws && outs && n <= 8 ? n : 1, true);
    return t(group_checked(c, ws, n, x, tokens, pinned, outs, t));
}

int prism_hip_project_f32_group(prism_hip_ctx *c, const prism_weight_id *ws, uint32_t n, const float *x, int pinned,
                                float *const *outs) {
    return group_host(c, ws, n, x, 1, pinned, outs);
}

int prism_hip_project_f32_group_tokens(prism_hip_ctx *c, const prism_weight_id *ws, uint32_t n, const float *x,
                                       uint32_t tokens, int pinned, float *const *outs) {
    return group_host(c, ws, n, x, tokens, pinned, outs);
}

int prism_hip_project_f32_pair_tokens(prism_hip_ctx *c, const prism_weight_id *ws, const float *x, uint32_t tokens,
                                      int pinned, float *out_a, float *out_b) {
    float *const outs[2] = {out_a, out_b};
    return group_host(c, ws, 2, x, tokens, pinned, outs);
}

int prism_hip_project_f32_triple_tokens(prism_hip_ctx *c, const prism_weight_id *ws, const float *x, uint32_t tokens,
                                        int pinned, float *out_a, float *out_b, float *out_c) {
    float *const outs[3] = {out_a, out_b, out_c};
    return group_host(c, ws, 3, x, tokens, pinned, outs);
}

static int ffn_checked(prism_hip_ctx *c, prism_weight_id gid, prism_weight_id uid, prism_weight_id did,
                       const float *x, const float *residual, uint32_t tokens, int pinned, uint32_t hb, float *out,
                       Tally &t) {
    if (!c) return PRISM_ERR_INVALID_INPUT;
    const Weight *g = find(c, gid), *u = find(c, uid), *d = did ? find(c, did) : nullptr;
    // Output length: down's rows, or gate's for the SwiGLU vector; known when those ids are.
    const Weight *shape = did ? d : g;
    const uint64_t nout = shape ? shape->rows * tokens : 0;
    int rc = check_ready(c);
    if (rc) {
        zero(out, nout);
        return rc;
    }
    if (!g || !u || (did && !d)) {
        zero(out, nout);
        return fail(c, PRISM_ERR_INVALID_INPUT, "unknown weight id");
    }
    if (!x || !out || tokens == 0) {
        t.bad_input();
        zero(out, nout);
        return fail(c, PRISM_ERR_INVALID_INPUT, "null input or output, or no tokens");
    }
    const prism_tensor_desc dd = d ? desc_of(*d) : prism_tensor_desc{};
    if (!ffn_eligible(desc_of(*g), desc_of(*u), d ? &dd : nullptr)) {
        zero(out, nout);
        return fail(c, PRISM_ERR_UNSUPPORTED, "FFN chain needs gate/up [ffn][hidden] and down [hidden][ffn] of one packed kind");
    }
    t.dispatch();
    const uint64_t nx = g->cols * tokens;
    rc = ensure(c, c->x, sizeof(float) * nx);
    if (!rc) rc = ensure(c, c->out, sizeof(float) * nout);
    if (!rc && residual) rc = ensure(c, c->res, sizeof(float) * nout);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(c->x.p, x, sizeof(float) * nx, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess && residual)
            e = hipMemcpyAsync(c->res.p, residual, sizeof(float) * nout, hipMemcpyHostToDevice, c->stream);
        rc = e == hipSuccess ? PRISM_OK : hip_fail(c, e, "upload activations");
    }
    if (!rc)
        rc = ffn_tokens_impl(c, *g, *u, d, static_cast<float *>(c->x.p),
                             residual ? static_cast<float *>(c->res.p) : nullptr, tokens, pinned,
                             static_cast<float *>(c->out.p), nullptr, c->stream, hb);
    if (!rc) rc = finish(c, out, static_cast<float *>(c->out.p), nout);
    if (rc) zero(out, nout);
    return rc;
}

static int ffn_host(prism_hip_ctx *c, prism_weight_id gid, prism_weight_id uid, prism_weight_id did, const float *x,
                    const float *residual, uint32_t tokens, int pinned, float *out, uint32_t hb = 0) {
    Tally t(c, did ? 3 : 2, true);
    return t(ffn_checked(c, gid, uid, did, x, residual, tokens, pinned, hb, out, t));
}

int prism_hip_ffn_swiglu(prism_hip_ctx *c, prism_weight_id gate, prism_weight_id up, const float *x, int pinned,
                         float *out) {
    return ffn_host(c, gate, up, 0, x, nullptr, 1, pinned, out);
}

int prism_hip_ffn_swiglu_tokens(prism_hip_ctx *c, prism_weight_id gate, prism_weight_id up, const float *x,
                                uint32_t tokens, int pinned, float *out) {
    return ffn_host(c, gate, up, 0, x, nullptr, tokens, pinned, out);
}

int prism_hip_ffn_chain(prism_hip_ctx *c, prism_weight_id gate, prism_weight_id up, prism_weight_id down,
                        const float *x, const float *residual, uint32_t hadamard_block, int pinned, float *out) {
    if (!c) return PRISM_ERR_INVALID_INPUT;
    if (down == 0) return Tally(c, 3, true)(fail(c, PRISM_ERR_INVALID_INPUT, "down projection required"));
    return ffn_host(c, gate, up, down, x, residual, 1, pinned, out, hadamard_block);
}

int prism_hip_ffn_chain_tokens(prism_hip_ctx *c, prism_weight_id gate, prism_weight_id up, prism_weight_id down,
                               const float *x, const float *residual, uint32_t tokens, uint32_t hadamard_block,
                               int pinned, float *out) {
    if (!c) return PRISM_ERR_INVALID_INPUT;
    if (down == 0) return Tally(c, 3, true)(fail(c, PRISM_ERR_INVALID_INPUT, "down projection required"));
    return ffn_host(c, gate, up, down, x, residual, tokens, pinned, out, hadamard_block);
}

static int ffn_lora_checked(prism_hip_ctx *c, prism_weight_id gid, prism_weight_id uid, prism_weight_id did,
                            const float *x, const float *residual, uint32_t hb, const float *lora_a, int pinned,
                            float *out, float *lora_dot, Tally &t) {
    if (lora_dot) *lora_dot = 0.0f;
    if (!c) return PRISM_ERR_INVALID_INPUT;
    const Weight *g = find(c, gid), *u = find(c, uid), *d = find(c, did);
    const uint64_t nout = d ? d->rows : 0;
    int rc = check_ready(c);
    if (rc) {
        zero(out, nout);
        return rc;
    }
    if (!g || !u || !d) {
        zero(out, nout);
        return fail(c, PRISM_ERR_INVALID_INPUT, "unknown weight id");
    }
    const prism_tensor_desc dd = desc_of(*d);
    if (!ffn_eligible(desc_of(*g), desc_of(*u), &dd)) {
        zero(out, nout);
        return fail(c, PRISM_ERR_UNSUPPORTED, "FFN chain needs gate/up [ffn][hidden] and down [hidden][ffn] of one packed kind");
    }
    if (!x || !out || !lora_a || !lora_dot) {
        t.bad_input();
        zero(out, nout);
        return fail(c, PRISM_ERR_INVALID_INPUT, "null input, output, LoRA factor or dot");
    }
    // The caller's own check (matvec_ffn_chain_lora_with_executor, projection.rs:664-670):
    // a non-finite LoRA A factor never reaches a submission.
    const uint64_t nl = d->cols;
    for (uint64_t i = 0; i < nl; ++i) {
        if (!std::isfinite(lora_a[i])) {
            zero(out, nout);
            return fail(c, PRISM_ERR_INVALID_INPUT, "non-finite LoRA A factor");
        }
    }
    t.dispatch();
    rc = ensure(c, c->x, sizeof(float) * g->cols);
    if (!rc) rc = ensure(c, c->out, sizeof(float) * nout);
    if (!rc) rc = ensure(c, c->h, sizeof(float) * g->rows);
    if (!rc) rc = ensure(c, c->lora, sizeof(float) * (nl + 1));
    if (!rc && residual) rc = ensure(c, c->res, sizeof(float) * nout);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(c->x.p, x, sizeof(float) * g->cols, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(c->lora.p, lora_a, sizeof(float) * nl, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess && residual)
            e = hipMemcpyAsync(c->res.p, residual, sizeof(float) * nout, hipMemcpyHostToDevice, c->stream);
        rc = e == hipSuccess ? PRISM_OK : hip_fail(c, e, "upload activations");
    }
    float *hv = static_cast<float *>(c->h.p), *dot = static_cast<float *>(c->lora.p) + nl;
    if (!rc)
        rc = ffn_chain_impl(c, *g, *u, d, static_cast<const float *>(c->x.p),
                            residual ? static_cast<const float *>(c->res.p) : nullptr, pinned,
                            static_cast<float *>(c->out.p), hv, c->stream, hb);
    if (!rc)
        rc = launch_result(c, launch_lora_dot(static_cast<const float *>(c->lora.p), hv, static_cast<uint32_t>(nl),
                                              pinned, dot, c->err, c->stream),
                           "LoRA dot launch");
    if (!rc) {
        hipError_t e = hipMemcpyAsync(lora_dot, dot, sizeof(float), hipMemcpyDeviceToHost, c->stream);
        if (e != hipSuccess) rc = hip_fail(c, e, "copy LoRA dot");
    }
    if (!rc) rc = finish(c, out, static_cast<float *>(c->out.p), nout);
    if (!rc && !std::isfinite(*lora_dot)) rc = fail(c, PRISM_ERR_NONFINITE, "non-finite LoRA dot");
    if (rc) {
        zero(out, nout);
        *lora_dot = 0.0f;
    }
    return rc;
}

int prism_hip_ffn_chain_lora(prism_hip_ctx *c, prism_weight_id gate, prism_weight_id up, prism_weight_id down,
                             const float *x, const float *residual, uint32_t hadamard_block, const float *lora_a,
                             int pinned, float *out, float *lora_dot) {
    Tally t(c, 3, true);
    return t(ffn_lora_checked(c, gate, up, down, x, residual, hadamard_block, lora_a, pinned, out, lora_dot, t));
}

int prism_hip_quantize_q8k_device(prism_hip_ctx *c, const float *x, uint64_t cols, uint32_t tokens, int pinned,
                                  prism_q8k_block *out, void *stream) {
    Tally t(c, 0, true);
    int rc = check_ready(c);
    if (rc) return t(rc);
    if (!x || !out || cols == 0 || cols % 256) {
        t.bad_input();
        return t(fail(c, PRISM_ERR_INVALID_INPUT, "Q8_K needs cols % 256 == 0"));
    }
    hipStream_t s;
    rc = call_stream(c, stream, &s);
    return t(rc ? rc : quantize(c, 0, x, cols, tokens, pinned, out, s));
}

int prism_hip_quantize_q8_device(prism_hip_ctx *c, const float *x, uint64_t cols, uint32_t tokens, int contract,
                                 prism_q8_block *out, void *stream) {
    Tally t(c, 0, true);
    int rc = check_ready(c);
    if (rc) return t(rc);
    if (!x || !out || cols == 0 || cols % 32 || contract < 0 || contract > 2) {
        t.bad_input();
        return t(fail(c, PRISM_ERR_INVALID_INPUT, "Q8_0 needs cols % 32 == 0 and a known contract"));
    }
    hipStream_t s;
    rc = call_stream(c, stream, &s);
    if (rc) return t(rc);
    return t(launch_result(c, launch_quantize_q8_0(x, cols, tokens, contract, out, c->err, s), "quantize"));
}

static int project_device_checked(prism_hip_ctx *c, prism_weight_id wid, int path, const void *act, uint32_t tokens,
                                  int pinned, float *out, void *stream, Tally &t) {
    const Weight *w = nullptr;
    int rc = prepare_weight(c, wid, path, &w);
    if (rc) return rc;
    if (!act || !out || tokens == 0) {
        t.bad_input();
        return fail(c, PRISM_ERR_INVALID_INPUT, "null device pointer");
    }
    hipStream_t s;
    rc = call_stream(c, stream, &s);
    if (rc) return rc;
    t.dispatch();
    if (path == PRISM_PATH_F32)
        return project_f32_dev(c, *w, static_cast<const float *>(act), tokens, pinned, out, c->act, s);
    return matvec(c, *w, path == PRISM_PATH_Q8K ? kActQ8K : kActQ8, act, tokens, pinned, out, s);
}

int prism_hip_project_device(prism_hip_ctx *c, prism_weight_id wid, int path, const void *act, uint32_t tokens,
                             int pinned, float *out, void *stream) {
    Tally t(c, 1, path == PRISM_PATH_F32);
    return t(project_device_checked(c, wid, path, act, tokens, pinned, out, stream, t));
}

static int project_noalloc_checked(prism_hip_ctx *c, prism_weight_id wid, int path, const void *act,
                                   uint32_t tokens, int pinned, float *out, void *stream, Tally &t) {
    const Weight *w = nullptr;
    int rc = prepare_weight(c, wid, path, &w);
    if (rc) return rc;
    if (!act || !out || tokens == 0) {
        t.bad_input();
        return fail(c, PRISM_ERR_INVALID_INPUT, "null device pointer");
    }
    if (!c->noalloc) return fail(c, PRISM_ERR_UNSUPPORTED, c->noalloc_error);
    hipStream_t s;
    rc = call_stream(c, stream, &s);
    if (rc) return rc;
    t.dispatch();
    Scratch fixed{c, static_cast<uint8_t *>(c->noalloc), c->noalloc_bytes, 0};
    if (path == PRISM_PATH_F32)
        return project_f32_dev(c, *w, static_cast<const float *>(act), tokens, pinned, out, c->act, s, nullptr, &fixed);
    return matvec(c, *w, path == PRISM_PATH_Q8K ? kActQ8K : kActQ8, act, tokens, pinned, out, s, &fixed);
}

int prism_hip_project_device_noalloc(prism_hip_ctx *c, prism_weight_id wid, int path, const void *act,
                                     uint32_t tokens, int pinned, float *out, void *stream) {
    Tally t(c, 1, path == PRISM_PATH_F32);
    return t(project_noalloc_checked(c, wid, path, act, tokens, pinned, out, stream, t));
}

static int ffn_device_checked(prism_hip_ctx *c, prism_weight_id gid, prism_weight_id uid, prism_weight_id did,
                              const float *x, const float *residual, uint32_t hb, int pinned, float *out, float *h,
                              void *stream, Tally &t) {
    int rc = check_ready(c);
    if (rc) return rc;
    const Weight *g = find(c, gid), *u = find(c, uid), *d = did ? find(c, did) : nullptr;
    if (!g || !u || (did && !d) || !out) return fail(c, PRISM_ERR_INVALID_INPUT, "bad FFN chain arguments");
    if (!x) {
        t.bad_input();
        return fail(c, PRISM_ERR_INVALID_INPUT, "bad FFN chain arguments");
    }
    if (d && d->kind != g->kind) return fail(c, PRISM_ERR_UNSUPPORTED, "FFN chain needs one packed kind");
    hipStream_t s;
    rc = call_stream(c, stream, &s);
    if (rc) return rc;
    t.dispatch();
    // Without a down projection the call is project_f32_ffn_swiglu: out receives h.
    if (!d) return ffn_chain_impl(c, *g, *u, nullptr, x, nullptr, pinned, nullptr, out, s);
    return ffn_chain_impl(c, *g, *u, d, x, residual, pinned, out, h, s, hb);
}

int prism_hip_ffn_chain_device(prism_hip_ctx *c, prism_weight_id gid, prism_weight_id uid, prism_weight_id did,
                               const float *x, const float *residual, uint32_t hadamard_block, int pinned,
                               float *out, float *h, void *stream) {
    Tally t(c, did ? 3 : 2, true);
    return t(ffn_device_checked(c, gid, uid, did, x, residual, hadamard_block, pinned, out, h, stream, t));
}

int prism_hip_sync(prism_hip_ctx *c, void *stream) {
    if (!c) return PRISM_ERR_INVALID_INPUT;
    if (c->faulted) return fail(c, PRISM_ERR_DEVICE_FAULT, "device fault latched");
    hipStream_t s;
    const int rc = call_stream(c, stream, &s);
    return rc ? rc : drain(c, s);
}

void *prism_hip_stream(prism_hip_ctx *c) { return c ? static_cast<void *>(c->stream) : nullptr; }

int prism_hip_set_cancellation(prism_hip_ctx *c, const int32_t *flag) {
    if (!c) return PRISM_ERR_INVALID_INPUT;
    c->cancel = flag;
    return PRISM_OK;
}

int prism_hip_get_statistics(const prism_hip_ctx *c, prism_hip_statistics *out) {
    if (!c || !out) return PRISM_ERR_INVALID_INPUT;
    *out = c->stats;
    return PRISM_OK;
}

int prism_hip_get_diagnostics(const prism_hip_ctx *c, prism_hip_diagnostics *out) {
    if (!c || !out) return PRISM_ERR_INVALID_INPUT;
    *out = c->diag;
    return PRISM_OK;
}

}  // extern "C"
