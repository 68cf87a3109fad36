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
#include <cstring>
#include <vector>

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
    float *qkv = nullptr, *att = nullptr, *scores = nullptr, *maxima = nullptr, *logits = nullptr;
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

// Whether a projection the step gives floats (qkv, o, the gate/up pair) quantizes them in
// its kernel's prologue at these widths.
bool prologue_fits(prism_hip_decoder *d, prism_weight_id wid, prism_weight_id up = 0, void *q8_out = nullptr) {
    prism_hip_ctx *c = d->ctx;
    MatvecArgs a = f32_args(c, *find(c, wid), nullptr, 1, 0, nullptr, nullptr, c->stream);
    if (up) a.w2 = static_cast<const uint8_t *>(find(c, up)->dev);
    a.q8_out = q8_out;
    return tiled_prologue_fits(a);
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

// Launch families of one step, in step order (the measurement entry points report
// them by these names).
enum Family : int { kQkv, kScores, kValues, kO, kGateUp, kDown, kLmPrep, kLmHead, kGreedy, kFamilies };
const char *const kFamilyName[kFamilies] = {"qkv",     "attn_scores", "attn_values", "o",     "gate_up",
                                            "down",    "lm_prep",     "lm_head",     "greedy"};

// Called before every launch of a step (family, layer; layer 0 for the head); used to
// bracket launches with events.  nullptr in the step the graph captures.
struct StepHook {
    virtual int before(Family f, uint32_t layer) = 0;
    virtual ~StepHook() = default;
};

AttnArgs attn_args(prism_hip_decoder *d) {
    prism_hip_ctx *c = d->ctx;
    const prism_decoder_geometry &g = d->g;
    AttnArgs at{};
    at.qkv = d->qkv;
    at.scores = d->scores;
    at.maxima = d->maxima;
    at.out = d->att;
    at.state = d->state;
    at.heads = static_cast<uint32_t>(g.heads);
    at.kv_heads = static_cast<uint32_t>(g.kv_heads);
    at.head_dim = static_cast<uint32_t>(g.head_dim);
    at.rope = static_cast<uint32_t>(g.rope);
    at.max_tokens = static_cast<uint32_t>(g.max_tokens);
    at.eps = g.eps;
    at.err = c->err;
    at.stream = c->stream;
    return at;
}

// One launch family for one layer (the head's families ignore `layer`).
int launch_family(prism_hip_decoder *d, Family f, uint32_t layer) {
    prism_hip_ctx *c = d->ctx;
    const prism_decoder_geometry &g = d->g;
    float *h0 = d->hidden[0], *h1 = d->hidden[1];
    const auto &L = d->layers[layer < d->layers.size() ? layer : 0];
    AttnArgs at = attn_args(d);
    at.q_norm = L.q_norm;
    at.k_norm = L.k_norm;
    at.kcache = L.kc;
    at.vcache = L.vc;
    switch (f) {
    case kQkv: return project(d, L.qkv, h0, d->qkv, nullptr, L.norm);
    case kScores: return launch_result(c, launch_attn_scores(at), "attention scores launch");
    case kValues: return launch_result(c, launch_attn_values(at), "attention values launch");
    case kO: return project(d, L.o, d->att, h1, h0, nullptr);
    case kGateUp: return project(d, L.gate, h1, nullptr, nullptr, L.post_norm, L.up, d->ffn_q8);
    case kDown: return project_q8(d, L.down, d->ffn_q8, h0, h1);
    case kLmPrep:
        return launch_result(c, launch_lm_prep(h0, d->output_norm, static_cast<uint32_t>(g.hidden), g.eps, d->lm_act,
                                               c->err, c->stream),
                             "final norm launch");
    case kLmHead: {
        // The row-tile kernel also leaves each 64-row tile's largest logit and first row.
        const Weight &w = *find(c, d->lm_head);
        MatvecArgs a = matvec_args(c, w, kActQ8, d->lm_act, 1, 0, d->logits, c->stream);
        a.tile_best = d->argmax_scratch;
        return run_matvec(c, a, w.tiled);
    }
    case kGreedy:
        return launch_result(c,
                             launch_argmax_embed(static_cast<const TileBest *>(d->argmax_scratch),
                                                 static_cast<uint32_t>(g.vocab), find(c, d->lm_head)->dev,
                                                 static_cast<uint32_t>(g.hidden), d->state, rope_args(g), d->tokens,
                                                 d->max_steps, h0, c->stream),
                             "argmax launch");
    default: return fail(c, PRISM_ERR_INVALID_INPUT, "unknown launch family");
    }
}

// Enqueues one decode step on the context stream (also used under graph capture).
int enqueue_step(prism_hip_decoder *d, StepHook *hook = nullptr) {
    auto run = [&](Family f, uint32_t layer) {
        if (hook) {
            const int rc = hook->before(f, layer);
            if (rc) return rc;
        }
        return launch_family(d, f, layer);
    };
    for (uint32_t l = 0; l < d->layers.size(); ++l)
        for (Family f : {kQkv, kScores, kValues, kO, kGateUp, kDown}) {
            const int rc = run(f, l);
            if (rc) return rc;
        }
    for (Family f : {kLmPrep, kLmHead, kGreedy}) {
        const int rc = run(f, 0);
        if (rc) return rc;
    }
    return PRISM_OK;
}

// Algorithmic bytes of one launch of family f at decode position pos: packed weights
// at their native size, f32 activations and outputs, Q8_0 blocks at 34 bytes, binary16
// cache rows read (pos + 1 of them) and appended.
uint64_t family_bytes(const prism_hip_decoder *d, Family f, uint64_t pos) {
    const prism_decoder_geometry &g = d->g;
    const uint64_t H = g.hidden, F = g.ffn, D = g.head_dim, QW = g.heads * D, KW = g.kv_heads * D, QKV = QW + 2 * KW;
    auto ptq1 = [](uint64_t rows, uint64_t cols) { return rows * (cols / 128) * 28; };
    const uint64_t n = pos + 1;
    switch (f) {
    case kQkv: return ptq1(QKV, H) + 4 * H + 4 * H + 4 * QKV;
    case kScores: return 4 * QKV + 2 * 4 * D + n * KW * 2 + 2 * KW * 2 + 4 * g.heads * n;
    case kValues: return 4 * g.heads * n + n * KW * 2 + 4 * QW;
    case kO: return ptq1(H, QW) + 4 * QW + 4 * H + 4 * H;
    case kGateUp: return 2 * ptq1(F, H) + 4 * H + 4 * H + F / 32 * 34;
    case kDown: return ptq1(H, F) + F / 32 * 34 + 4 * H + 4 * H;
    case kLmPrep: return 4 * H + 4 * H + H / 32 * 34;
    // The LM head also writes each 64-row tile's (largest logit, first row) pair, which
    // the greedy launch reads back instead of the logits.
    case kLmHead: return g.vocab * (H / 32) * 34 + H / 32 * 34 + 4 * g.vocab + 8 * ((g.vocab + 63) / 64);
    case kGreedy: return 8 * ((g.vocab + 63) / 64) + H / 32 * 34 + 4 * H;
    default: return 0;
    }
}

// Destroys the captured step.  A replay may still be queued on the context stream, so the
// stream drains first: the executable is never freed under a launch in flight.
void drop_graph(prism_hip_decoder *d) {
    if (!d->exec && !d->graph) return;
    if (d->ctx && d->ctx->stream) (void)hipStreamSynchronize(d->ctx->stream);
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

// Resets the device state to (token, pos) and writes the token's embedding.
int start(prism_hip_decoder *d, uint32_t token, uint64_t pos) {
    prism_hip_ctx *c = d->ctx;
    hipStream_t s = c->stream;
    const DecodeState init{static_cast<uint32_t>(pos), token, 0, 0};
    HIP_OR_FAIL(c, hipMemcpyAsync(d->state, &init, sizeof(init), hipMemcpyHostToDevice, s));
    HIP_OR_FAIL(c, hipStreamSynchronize(s));
    const Weight *lm = find(c, d->lm_head);
    return launch_result(c,
                         launch_embed(lm->dev, d->g.vocab, static_cast<uint32_t>(d->g.hidden), d->state,
                                      rope_args(d->g), d->hidden[0], s),
                         "embed launch");
}

// Records an event on the context stream before every launch of a step.
struct EventHook final : StepHook {
    prism_hip_ctx *c;
    std::vector<hipEvent_t> ev;
    std::vector<Family> fam;
    size_t used = 0;
    explicit EventHook(prism_hip_ctx *ctx) : c(ctx) {}
    ~EventHook() override {
        for (hipEvent_t e : ev) (void)hipEventDestroy(e);
    }
    int mark() {
        if (used == ev.size()) {
            hipEvent_t e = nullptr;
            HIP_OR_FAIL(c, hipEventCreate(&e));
            ev.push_back(e);
        }
        HIP_OR_FAIL(c, hipEventRecord(ev[used], c->stream));
        ++used;
        return PRISM_OK;
    }
    int before(Family f, uint32_t) override {
        fam.push_back(f);
        return mark();
    }
};

int family_of(const char *name, Family *f) {
    if (!name) return PRISM_ERR_INVALID_INPUT;
    for (int i = 0; i < kFamilies; ++i)
        if (std::strcmp(name, kFamilyName[i]) == 0) {
            *f = static_cast<Family>(i);
            return PRISM_OK;
        }
    return PRISM_ERR_INVALID_INPUT;
}

}  // namespace

extern "C" {

prism_hip_decoder *prism_hip_decoder_create(prism_hip_ctx *c, const prism_decoder_geometry *g, uint32_t max_steps) {
    if (check_live(c) || !g) return nullptr;
    const bool ok = g->head_dim == 128 && g->heads && g->kv_heads && g->heads % g->kv_heads == 0 && g->rope &&
                    g->rope <= g->head_dim && g->rope % 2 == 0 && g->hidden && g->hidden % 128 == 0 && g->ffn &&
                    g->ffn % 128 == 0 && (g->heads * g->head_dim) % 128 == 0 && g->vocab && g->layers && g->layers <= 500 &&
                    g->max_tokens && g->max_tokens <= 8192 && g->vocab <= kGreedyMaxVocab && max_steps &&
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
    if (!rc)
        rc = dalloc(d, &d->maxima,
                    sizeof(float) * g->heads * attn_maxima_per_head(static_cast<uint32_t>(g->max_tokens)));
    if (!rc) rc = dalloc(d, &d->logits, sizeof(float) * g->vocab);
    if (!rc) rc = dalloc(d, &d->lm_act, sizeof(prism_q8_block) * (H / 32));
    if (!rc) rc = dalloc(d, &d->state, sizeof(DecodeState));
    if (!rc) rc = dalloc(d, &d->tokens, sizeof(uint32_t) * max_steps);
    const size_t gs = argmax_scratch_bytes(g->vocab);
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
    int rc = check_live(d->ctx);
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
    if (!rc && !(prologue_fits(d, L.qkv) && prologue_fits(d, L.o) && prologue_fits(d, L.gate, L.up, d->ffn_q8)))
        rc = fail(d->ctx, PRISM_ERR_UNSUPPORTED, "decoder projection too wide for the quantizing prologue");
    if (!rc) rc = upload(d, L.norm, norm, sizeof(float) * H);
    if (!rc) rc = upload(d, L.post_norm, post_norm, sizeof(float) * H);
    if (!rc) rc = upload(d, L.q_norm, q_norm, sizeof(float) * D);
    if (!rc) rc = upload(d, L.k_norm, k_norm, sizeof(float) * D);
    return rc;
}

int prism_hip_decoder_set_cache(prism_hip_decoder *d, uint32_t layer, const uint16_t *k, const uint16_t *v,
                                uint64_t tokens) {
    if (!d) return PRISM_ERR_INVALID_INPUT;
    int rc = check_live(d->ctx);
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
    int rc = check_live(d->ctx);
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
    rc = start(d, token, pos);
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
        e = hipGraphInstantiate(&d->exec, d->graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            d->exec = nullptr;
            drop_graph(d);  // the next call captures again
            return hip_fail(c, e, "hipGraphInstantiate");
        }
    }
    hipEvent_t t0 = nullptr, t1 = nullptr;
    HIP_OR_FAIL(c, hipEventCreate(&t0));
    HIP_OR_FAIL(c, hipEventCreate(&t1));
    HIP_OR_FAIL(c, hipEventRecord(t0, s));
    // With a cancellation flag registered, steps are checked between launches and at most
    // two are in flight: step i waits for step i - 2 before it is enqueued.
    hipEvent_t inflight[2] = {nullptr, nullptr};
    if (c->cancel) {
        for (hipEvent_t &e : inflight) {
            const hipError_t he = hipEventCreateWithFlags(&e, hipEventDisableTiming);
            if (he != hipSuccess && !rc) rc = hip_fail(c, he, "hipEventCreate");
        }
    }
    for (uint32_t i = 0; i < steps && !rc; ++i) {
        if (c->cancel) {
            if (i >= 2) {
                const hipError_t he = hipEventSynchronize(inflight[i % 2]);
                if (he != hipSuccess) {
                    rc = hip_fail(c, he, "hipEventSynchronize");
                    break;
                }
            }
            if (cancelled(c)) {
                rc = fail(c, PRISM_ERR_CANCELLED, "cancelled by the request owner");
                break;
            }
        }
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
        if (!rc && c->cancel) {
            const hipError_t he = hipEventRecord(inflight[i % 2], s);
            if (he != hipSuccess) rc = hip_fail(c, he, "hipEventRecord");
        }
    }
    if (rc == PRISM_ERR_CANCELLED) {  // the enqueued steps complete first (and report their errors)
        const int drc = drain(c, s);
        if (drc) rc = drc;
        else fail(c, PRISM_ERR_CANCELLED, "cancelled by the request owner");
    }
    for (hipEvent_t e : inflight)
        if (e) (void)hipEventDestroy(e);
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

extern "C" {

int prism_hip_decoder_profile(prism_hip_decoder *d, uint32_t token, uint64_t pos, uint32_t steps,
                              prism_decoder_launch_time *stats) {
    if (!d) return PRISM_ERR_INVALID_INPUT;
    prism_hip_ctx *c = d->ctx;
    int rc = check_ready(c);
    if (rc) return rc;
    if (!stats) return fail(c, PRISM_ERR_INVALID_INPUT, "stats required");
    for (int i = 0; i < kFamilies; ++i) {
        stats[i].name = kFamilyName[i];
        stats[i].launches = 0;
        stats[i].total_us = 0.0;
        stats[i].bytes = family_bytes(d, static_cast<Family>(i), pos);
    }
    if (!ready(d)) return fail(c, PRISM_ERR_INVALID_INPUT, "decoder weights not set");
    if (steps == 0 || steps > d->max_steps || token >= d->g.vocab || pos + steps > d->g.max_tokens)
        return fail(c, PRISM_ERR_INVALID_INPUT, "bad profile arguments");
    rc = start(d, token, pos);
    EventHook hook(c);
    for (uint32_t i = 0; i < steps && !rc; ++i) {
        hook.used = 0;
        hook.fam.clear();
        rc = enqueue_step(d, &hook);
        if (!rc) rc = hook.mark();  // end of the step's last launch
        if (!rc) rc = drain(c, c->stream);
        for (size_t k = 0; !rc && k + 1 < hook.used; ++k) {
            float ms = 0.0f;
            const hipError_t e = hipEventElapsedTime(&ms, hook.ev[k], hook.ev[k + 1]);
            if (e != hipSuccess) {
                rc = hip_fail(c, e, "hipEventElapsedTime");
                break;
            }
            prism_decoder_launch_time &st = stats[hook.fam[k]];
            st.launches += 1;
            st.total_us += 1e3 * ms;
        }
    }
    return rc;
}

int prism_hip_decoder_time_family(prism_hip_decoder *d, const char *family, uint32_t reps, double *avg_us,
                                  uint64_t *bytes) {
    if (!d) return PRISM_ERR_INVALID_INPUT;
    prism_hip_ctx *c = d->ctx;
    int rc = check_ready(c);
    if (rc) return rc;
    Family f;
    if (family_of(family, &f) || f == kGreedy || reps == 0 || !avg_us)
        return fail(c, PRISM_ERR_INVALID_INPUT, "bad family timing arguments");
    if (!ready(d)) return fail(c, PRISM_ERR_INVALID_INPUT, "decoder weights not set");
    DecodeState st{};
    HIP_OR_FAIL(c, hipMemcpy(&st, d->state, sizeof(st), hipMemcpyDeviceToHost));
    if (st.pos >= d->g.max_tokens) return fail(c, PRISM_ERR_INVALID_INPUT, "decoder position past the cache");
    const bool per_layer = f <= kDown;
    const uint32_t layers = per_layer ? static_cast<uint32_t>(d->layers.size()) : 1;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    HIP_OR_FAIL(c, hipEventCreate(&t0));
    hipError_t e = hipEventCreate(&t1);
    if (e != hipSuccess) {
        (void)hipEventDestroy(t0);
        return hip_fail(c, e, "hipEventCreate");
    }
    e = hipEventRecord(t0, c->stream);
    if (e != hipSuccess) rc = hip_fail(c, e, "hipEventRecord");
    for (uint32_t r = 0; r < reps && !rc; ++r)
        for (uint32_t l = 0; l < layers && !rc; ++l) rc = launch_family(d, f, l);
    if (!rc && (e = hipEventRecord(t1, c->stream)) != hipSuccess) rc = hip_fail(c, e, "hipEventRecord");
    if (!rc) rc = drain(c, c->stream);
    float ms = 0.0f;
    if (!rc && (e = hipEventElapsedTime(&ms, t0, t1)) != hipSuccess) rc = hip_fail(c, e, "hipEventElapsedTime");
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    if (rc) return rc;
    *avg_us = 1e3 * ms / (static_cast<double>(reps) * layers);
    if (bytes) *bytes = family_bytes(d, f, st.pos);
    return PRISM_OK;
}

}  // extern "C"
