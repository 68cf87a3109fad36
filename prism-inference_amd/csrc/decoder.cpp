// decoder.cpp -- the resident full-attention decoder of the C ABI (prism_hip_decoder_*):
// weights and KV caches on the device, one decode step as a fixed sequence of
// launches on the context stream, optionally captured once into a HIP graph and
// replayed per step (the position lives in device memory, so the graph never
// changes).
//
// Layer loop: src/graph.rs:3870-3995 (source arithmetic).  Per layer six launches:
//   q/k/v      PTQ1 split matvec, RMSNorm(norm) fused into its quantizing prologue
//   attention  q/k norm + RoPE + KV append + scores; softmax + values (decode.hip)
//   o          PTQ1 split matvec + residual                  -> hidden'
//   gate/up    PTQ1 split matvec pair, RMSNorm(post_norm) prologue, SwiGLU epilogue
//              that writes the SwiGLU vector as Q8_0 blocks (source contract)
//   down       PTQ1 split matvec on those blocks + residual  -> hidden''
// then the final norm + Q8_0 quantization, the Q8_0 LM head (row-tile kernel) and
// the greedy choice, which also writes the next step's embedding.
#include <cmath>

#include "runtime_internal.hpp"

using namespace prism;
using namespace prism::rt;

struct prism_hip_decoder {
    prism_hip_ctx *ctx = nullptr;
    prism_decoder_geometry g{};
    uint32_t max_steps = 0;
    struct Layer {
        prism_weight_id qkv = 0, o = 0, gate = 0, up = 0, down = 0;
        float *norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
        uint16_t *kc = nullptr, *vc = nullptr;
    };
    std::vector<Layer> layers;
    prism_weight_id lm_head = 0;
    float *output_norm = nullptr;
    float *hidden[2] = {nullptr, nullptr};
    float *qkv = nullptr, *att = nullptr, *scores = nullptr, *logits = nullptr;
    void *ffn_q8 = nullptr;  // the SwiGLU vector's Q8_0 blocks
    float *logits_all = nullptr;
    size_t logits_all_steps = 0;
    void *lm_act = nullptr;
    void *argmax_scratch = nullptr;  // zero-filled at creation
    DecodeState *state = nullptr;
    uint32_t *tokens = nullptr;
    std::vector<void *> owned;  // device allocations freed on destroy
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace {

template <typename T>
int dalloc(prism_hip_decoder *d, T **p, size_t bytes) {
    void *v = nullptr;
    hipError_t e = hipMalloc(&v, bytes);
    if (e != hipSuccess) return hip_fail(d->ctx, e, "hipMalloc(decoder)");
    d->owned.push_back(v);
    *p = static_cast<T *>(v);
    return PRISM_OK;
}

int upload(prism_hip_decoder *d, void *dst, const void *src, size_t bytes) {
    hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
    return e == hipSuccess ? PRISM_OK : hip_fail(d->ctx, e, "decoder upload");
}

// Uploads one PTQ1 / Q8_0 tensor into the context's tiled residency under a key
// private to this decoder (`slot` numbers its tensors), so no other caller's
// residency key can alias it and releasing it on destroy affects nobody else.
int weight(prism_hip_decoder *d, prism_weight_id *id, uint64_t slot, uint32_t kind, uint64_t cols, uint64_t rows,
           const uint8_t *host) {
    uint64_t group, block;
    layout(kind, &group, &block);
    const uint64_t bytes = rows * (cols / group) * block;
    if (*id) prism_hip_weight_release(d->ctx, *id);
    *id = 0;
    const uint64_t key = (1ull << 63) | (reinterpret_cast<uint64_t>(d) << 12) | slot;
    prism_weight_id w = prism_hip_weight_acquire(d->ctx, key, kind, cols, rows, host, bytes);
    if (w < 0) return static_cast<int>(w);
    const Weight *W = find(d->ctx, w);
    if (!W || !W->tiled) return fail(d->ctx, PRISM_ERR_UNSUPPORTED, "decoder weight not stored tiled");
    *id = w;
    return PRISM_OK;
}

// One projection of a resident weight on device floats: RMSNorm (when norm_w) and
// the source Q8_0 quantization in the prologue, optional residual, optional up
// matrix (SwiGLU epilogue, whose vector goes to q8_out as source-contract Q8_0 blocks).
int project(prism_hip_decoder *d, prism_weight_id wid, const float *x, float *out, const float *residual,
            const float *norm_w, prism_weight_id up = 0, void *q8_out = nullptr) {
    prism_hip_ctx *c = d->ctx;
    const Weight *w = find(c, wid);
    MatvecArgs a = f32_args(c, *w, x, 1, 0, out, residual, c->stream);
    a.norm_w = norm_w;
    a.eps = d->g.eps;
    if (up) a.w2 = static_cast<const uint8_t *>(find(c, up)->dev);
    a.q8_out = q8_out;
    a.q8_contract = PRISM_Q8_SOURCE;
    return run_matvec(c, a, true);
}

// A projection of prepared Q8_0 blocks (the source contract's dot_q8_groups) + residual.
int project_q8(prism_hip_decoder *d, prism_weight_id wid, const void *act, float *out, const float *residual) {
    prism_hip_ctx *c = d->ctx;
    const Weight *w = find(c, wid);
    MatvecArgs a = matvec_args(c, *w, kActQ8, act, 1, 0, out, c->stream);
    a.residual = residual;
    return run_matvec(c, a, true);
}

// rope_frequencies_mrope (src/graph.rs:6406-6431): theta_scale = rope_base.powf(-2 / rope).
RopeArgs rope_args(const prism_decoder_geometry &g) {
    RopeArgs r{};
    r.rope = static_cast<uint32_t>(g.rope);
    for (int i = 0; i < 4; ++i) r.sections[i] = static_cast<uint32_t>(g.rope_sections[i]);
    r.theta_scale = ::powf(g.rope_base, -2.0f / static_cast<float>(g.rope));
    return r;
}

// Enqueues one decode step on the context stream (also used under graph capture).
int enqueue_step(prism_hip_decoder *d) {
    prism_hip_ctx *c = d->ctx;
    const prism_decoder_geometry &g = d->g;
    hipStream_t s = c->stream;
    float *h0 = d->hidden[0], *h1 = d->hidden[1];
    AttnArgs at{};
    at.qkv = d->qkv;
    at.scores = d->scores;
    at.out = d->att;
    at.state = d->state;
    at.heads = static_cast<uint32_t>(g.heads);
    at.kv_heads = static_cast<uint32_t>(g.kv_heads);
    at.head_dim = static_cast<uint32_t>(g.head_dim);
    at.rope = static_cast<uint32_t>(g.rope);
    at.max_tokens = static_cast<uint32_t>(g.max_tokens);
    at.eps = g.eps;
    at.err = c->err;
    at.stream = s;
    for (const auto &L : d->layers) {
        int rc = project(d, L.qkv, h0, d->qkv, nullptr, L.norm);
        if (rc) return rc;
        at.q_norm = L.q_norm;
        at.k_norm = L.k_norm;
        at.kcache = L.kc;
        at.vcache = L.vc;
        rc = launch_result(c, launch_attention(at), "attention launch");
        if (rc) return rc;
        rc = project(d, L.o, d->att, h1, h0, nullptr);
        if (!rc) rc = project(d, L.gate, h1, nullptr, nullptr, L.post_norm, L.up, d->ffn_q8);
        if (!rc) rc = project_q8(d, L.down, d->ffn_q8, h0, h1);
        if (rc) return rc;
    }
    const Weight *lm = find(c, d->lm_head);
    int rc = launch_result(c, launch_lm_prep(h0, d->output_norm, static_cast<uint32_t>(g.hidden), g.eps, d->lm_act,
                                             c->err, s),
                           "final norm launch");
    if (!rc) rc = matvec(c, *lm, kActQ8, d->lm_act, 1, 0, d->logits, s);
    if (!rc)
        rc = launch_result(c,
                           launch_argmax_embed(d->logits, static_cast<uint32_t>(g.vocab), lm->dev,
                                               static_cast<uint32_t>(g.hidden), d->state, rope_args(g), d->tokens,
                                               d->max_steps, h0, d->argmax_scratch, s),
                           "argmax launch");
    return rc;
}

void drop_graph(prism_hip_decoder *d) {
    if (d->exec) (void)hipGraphExecDestroy(d->exec);
    if (d->graph) (void)hipGraphDestroy(d->graph);
    d->exec = nullptr;
    d->graph = nullptr;
}

// Every tensor set and still resident: prism_hip_weight_release_all (or a release of
// one of the decoder's ids) may have dropped weights the captured graph reads, in
// which case the graph is dropped too and the decoder must be given its tensors again.
bool ready(prism_hip_decoder *d) {
    bool ok = d->lm_head && d->output_norm && find(d->ctx, d->lm_head);
    for (const auto &L : d->layers)
        for (prism_weight_id w : {L.qkv, L.o, L.gate, L.up, L.down}) ok = ok && w && find(d->ctx, w);
    if (!ok) drop_graph(d);
    return ok;
}

}  // namespace

extern "C" {

prism_hip_decoder *prism_hip_decoder_create(prism_hip_ctx *c, const prism_decoder_geometry *g, uint32_t max_steps) {
    if (check_ready(c) || !g) return nullptr;
    const bool ok = g->head_dim == 128 && g->heads && g->kv_heads && g->heads % g->kv_heads == 0 && g->rope &&
                    g->rope <= g->head_dim && g->rope % 2 == 0 && g->hidden && g->hidden % 128 == 0 && g->ffn &&
                    g->ffn % 128 == 0 && (g->heads * g->head_dim) % 128 == 0 && g->vocab && g->layers && g->layers <= 500 &&
                    g->max_tokens && g->max_tokens <= 8192 && g->vocab < (1u << 31) && max_steps &&
                    std::isfinite(g->eps) && g->eps >= 0.0f && std::isfinite(g->rope_base) && g->rope_base > 0.0f;
    if (!ok) {
        fail(c, PRISM_ERR_INVALID_INPUT, "unsupported decoder geometry");
        return nullptr;
    }
    auto *d = new prism_hip_decoder;
    d->ctx = c;
    d->g = *g;
    d->max_steps = max_steps;
    d->layers.resize(g->layers);
    const size_t H = g->hidden, D = g->head_dim, KW = g->kv_heads * D, QKV = g->heads * D + 2 * KW;
    int rc = PRISM_OK;
    for (auto &L : d->layers) {
        if (!rc) rc = dalloc(d, &L.norm, sizeof(float) * H);
        if (!rc) rc = dalloc(d, &L.post_norm, sizeof(float) * H);
        if (!rc) rc = dalloc(d, &L.q_norm, sizeof(float) * D);
        if (!rc) rc = dalloc(d, &L.k_norm, sizeof(float) * D);
        if (!rc) rc = dalloc(d, &L.kc, sizeof(uint16_t) * g->max_tokens * KW);
        if (!rc) rc = dalloc(d, &L.vc, sizeof(uint16_t) * g->max_tokens * KW);
    }
    if (!rc) rc = dalloc(d, &d->output_norm, sizeof(float) * H);
    if (!rc) rc = dalloc(d, &d->hidden[0], sizeof(float) * H);
    if (!rc) rc = dalloc(d, &d->hidden[1], sizeof(float) * H);
    if (!rc) rc = dalloc(d, &d->qkv, sizeof(float) * QKV);
    if (!rc) rc = dalloc(d, &d->att, sizeof(float) * g->heads * D);
    if (!rc) rc = dalloc(d, &d->ffn_q8, sizeof(prism_q8_block) * (g->ffn / 32));
    if (!rc) rc = dalloc(d, &d->scores, sizeof(float) * g->heads * g->max_tokens);
    if (!rc) rc = dalloc(d, &d->logits, sizeof(float) * g->vocab);
    if (!rc) rc = dalloc(d, &d->lm_act, sizeof(prism_q8_block) * (H / 32));
    if (!rc) rc = dalloc(d, &d->state, sizeof(DecodeState));
    if (!rc) rc = dalloc(d, &d->tokens, sizeof(uint32_t) * max_steps);
    const size_t gs = argmax_scratch_bytes();
    if (!rc) rc = dalloc(d, &d->argmax_scratch, gs);
    if (!rc) {
        const hipError_t e = hipMemset(d->argmax_scratch, 0, gs);
        if (e != hipSuccess) rc = hip_fail(c, e, "decoder scratch reset");
    }
    if (rc) {
        prism_hip_decoder_destroy(d);
        return nullptr;
    }
    return d;
}

void prism_hip_decoder_destroy(prism_hip_decoder *d) {
    if (!d) return;
    drop_graph(d);
    if (d->ctx) {
        (void)hipStreamSynchronize(d->ctx->stream);
        for (const auto &L : d->layers)
            for (prism_weight_id w : {L.qkv, L.o, L.gate, L.up, L.down})
                if (w) prism_hip_weight_release(d->ctx, w);
        if (d->lm_head) prism_hip_weight_release(d->ctx, d->lm_head);
    }
    for (void *p : d->owned) (void)hipFree(p);
    if (d->logits_all) (void)hipFree(d->logits_all);
    delete d;
}

int prism_hip_decoder_set_layer(prism_hip_decoder *d, uint32_t layer, const uint8_t *qkv, const uint8_t *o,
                                const uint8_t *gate, const uint8_t *up, const uint8_t *down, const float *norm,
                                const float *post_norm, const float *q_norm, const float *k_norm) {
    if (!d) return PRISM_ERR_INVALID_INPUT;
    int rc = check_ready(d->ctx);
    if (rc) return rc;
    if (layer >= d->layers.size() || !qkv || !o || !gate || !up || !down || !norm || !post_norm || !q_norm || !k_norm)
        return fail(d->ctx, PRISM_ERR_INVALID_INPUT, "bad decoder layer arguments");
    drop_graph(d);
    const prism_decoder_geometry &g = d->g;
    const uint64_t H = g.hidden, D = g.head_dim, QW = g.heads * D, QKV = QW + 2 * g.kv_heads * D;
    auto &L = d->layers[layer];
    const uint64_t slot = 8ull * layer + 1;
    rc = weight(d, &L.qkv, slot, PRISM_KIND_PTQ1, H, QKV, qkv);
    if (!rc) rc = weight(d, &L.o, slot + 1, PRISM_KIND_PTQ1, QW, H, o);
    if (!rc) rc = weight(d, &L.gate, slot + 2, PRISM_KIND_PTQ1, H, g.ffn, gate);
    if (!rc) rc = weight(d, &L.up, slot + 3, PRISM_KIND_PTQ1, H, g.ffn, up);
    if (!rc) rc = weight(d, &L.down, slot + 4, PRISM_KIND_PTQ1, g.ffn, H, down);
    if (!rc) rc = upload(d, L.norm, norm, sizeof(float) * H);
    if (!rc) rc = upload(d, L.post_norm, post_norm, sizeof(float) * H);
    if (!rc) rc = upload(d, L.q_norm, q_norm, sizeof(float) * D);
    if (!rc) rc = upload(d, L.k_norm, k_norm, sizeof(float) * D);
    return rc;
}

int prism_hip_decoder_set_cache(prism_hip_decoder *d, uint32_t layer, const uint16_t *k, const uint16_t *v,
                                uint64_t tokens) {
    if (!d) return PRISM_ERR_INVALID_INPUT;
    int rc = check_ready(d->ctx);
    if (rc) return rc;
    if (layer >= d->layers.size() || tokens > d->g.max_tokens || (tokens && (!k || !v)))
        return fail(d->ctx, PRISM_ERR_INVALID_INPUT, "bad decoder cache arguments");
    const size_t n = sizeof(uint16_t) * tokens * d->g.kv_heads * d->g.head_dim;
    rc = upload(d, d->layers[layer].kc, k, n);
    if (!rc) rc = upload(d, d->layers[layer].vc, v, n);
    return rc;
}

int prism_hip_decoder_set_head(prism_hip_decoder *d, const uint8_t *lm_head, const float *output_norm) {
    if (!d) return PRISM_ERR_INVALID_INPUT;
    int rc = check_ready(d->ctx);
    if (rc) return rc;
    if (!lm_head || !output_norm) return fail(d->ctx, PRISM_ERR_INVALID_INPUT, "bad decoder head arguments");
    drop_graph(d);
    rc = weight(d, &d->lm_head, 0, PRISM_KIND_Q8_0, d->g.hidden, d->g.vocab, lm_head);
    if (!rc) rc = upload(d, d->output_norm, output_norm, sizeof(float) * d->g.hidden);
    return rc;
}

int prism_hip_decoder_generate(prism_hip_decoder *d, uint32_t token, uint64_t pos, uint32_t steps, int use_graph,
                               uint32_t *tokens_out, float *logits_out, double *seconds) {
    if (!d) return PRISM_ERR_INVALID_INPUT;
    prism_hip_ctx *c = d->ctx;
    int rc = check_ready(c);
    if (rc) return rc;
    if (!ready(d)) return fail(c, PRISM_ERR_INVALID_INPUT, "decoder weights not set");
    if (steps == 0 || steps > d->max_steps || token >= d->g.vocab || pos + steps > d->g.max_tokens || !tokens_out)
        return fail(c, PRISM_ERR_INVALID_INPUT, "bad generate arguments");
    hipStream_t s = c->stream;
    const size_t vocab = d->g.vocab;
    if (logits_out && d->logits_all_steps < steps) {
        if (d->logits_all) (void)hipFree(d->logits_all);
        d->logits_all = nullptr;
        d->logits_all_steps = 0;
        HIP_OR_FAIL(c, hipMalloc(&d->logits_all, sizeof(float) * vocab * steps));
        d->logits_all_steps = steps;
    }
    const DecodeState init{static_cast<uint32_t>(pos), token, 0, 0};
    HIP_OR_FAIL(c, hipMemcpyAsync(d->state, &init, sizeof(init), hipMemcpyHostToDevice, s));
    HIP_OR_FAIL(c, hipStreamSynchronize(s));
    const Weight *lm = find(c, d->lm_head);
    rc = launch_result(c,
                       launch_embed(lm->dev, d->g.vocab, static_cast<uint32_t>(d->g.hidden), d->state, rope_args(d->g),
                                    d->hidden[0], s),
                       "embed launch");
    if (rc) return rc;
    if (use_graph && !d->exec) {
        HIP_OR_FAIL(c, hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        rc = enqueue_step(d);
        hipGraph_t graph = nullptr;
        hipError_t e = hipStreamEndCapture(s, &graph);
        if (rc) {
            if (graph) (void)hipGraphDestroy(graph);
            return rc;
        }
        if (e != hipSuccess) return hip_fail(c, e, "hipStreamEndCapture");
        d->graph = graph;
        HIP_OR_FAIL(c, hipGraphInstantiate(&d->exec, d->graph, nullptr, nullptr, 0));
    }
    hipEvent_t t0 = nullptr, t1 = nullptr;
    HIP_OR_FAIL(c, hipEventCreate(&t0));
    HIP_OR_FAIL(c, hipEventCreate(&t1));
    HIP_OR_FAIL(c, hipEventRecord(t0, s));
    for (uint32_t i = 0; i < steps && !rc; ++i) {
        if (use_graph) {
            hipError_t e = hipGraphLaunch(d->exec, s);
            if (e != hipSuccess) rc = hip_fail(c, e, "hipGraphLaunch");
        } else {
            rc = enqueue_step(d);
        }
        if (!rc && logits_out) {
            hipError_t e = hipMemcpyAsync(d->logits_all + vocab * i, d->logits, sizeof(float) * vocab,
                                          hipMemcpyDeviceToDevice, s);
            if (e != hipSuccess) rc = hip_fail(c, e, "copy logits");
        }
    }
    if (!rc) {
        hipError_t e = hipEventRecord(t1, s);
        if (e != hipSuccess) rc = hip_fail(c, e, "hipEventRecord");
    }
    if (!rc) rc = drain(c, s);
    if (!rc && seconds) {
        float ms = 0.0f;
        hipError_t e = hipEventElapsedTime(&ms, t0, t1);
        if (e != hipSuccess) rc = hip_fail(c, e, "hipEventElapsedTime");
        *seconds = ms * 1e-3;
    }
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    if (!rc) {
        hipError_t e = hipMemcpy(tokens_out, d->tokens, sizeof(uint32_t) * steps, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = hip_fail(c, e, "copy tokens");
    }
    if (!rc && logits_out) {
        hipError_t e = hipMemcpy(logits_out, d->logits_all, sizeof(float) * vocab * steps, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = hip_fail(c, e, "copy logits");
    }
    if (rc) {
        std::memset(tokens_out, 0, sizeof(uint32_t) * steps);
        if (logits_out) std::memset(logits_out, 0, sizeof(float) * vocab * steps);
    }
    return rc;
}

}  // extern "C"
