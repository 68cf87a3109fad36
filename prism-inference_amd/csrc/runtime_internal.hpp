// runtime_internal.hpp -- state and helpers shared by the translation units that
// implement the extern "C" ABI of libprism_hip.so (runtime.cpp, decoder.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "prism_hip.h"
#include "kernels.hpp"
#include "tiled.hpp"

namespace prism::rt {

struct Weight {
    uint64_t key = 0;
    uint32_t kind = 0;
    uint64_t cols = 0, rows = 0, row_bytes = 0, bytes = 0;
    void *dev = nullptr;
    bool owned = false;
    bool tiled = false;  // 64-row tiled device layout (tiled.hpp) instead of native rows
};

// Grow-only device scratch buffer.
struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
};

inline bool layout(uint32_t kind, uint64_t *group, uint64_t *block) {
    switch (kind) {
    case PRISM_KIND_Q8_0: *group = 32; *block = 34; return true;
    case PRISM_KIND_Q2_K: *group = 256; *block = 84; return true;
    case PRISM_KIND_PQ2: *group = 128; *block = 34; return true;
    case PRISM_KIND_PTQ1: *group = 128; *block = 28; return true;
    case PRISM_KIND_TQ1_0: *group = 256; *block = 54; return true;
    case PRISM_KIND_TQ2_0: *group = 256; *block = 66; return true;
    default: return false;
    }
}

// ActivationContract::for_tensor (src/kernels.rs:1663-1673): 0 = Q8_K, 1 = Q8_0, 2 = pinned PTQ1 Q8_0.
inline int contract_for(uint32_t kind, uint64_t cols, int pinned) {
    if (kind == PRISM_KIND_PTQ1 && pinned) return 2;
    if (kind == PRISM_KIND_Q2_K || kind == PRISM_KIND_TQ1_0 || kind == PRISM_KIND_TQ2_0) return 0;
    if (kind == PRISM_KIND_PQ2 && cols % 256 == 0) return 0;
    return 1;
}

}  // namespace prism::rt

struct prism_hip_ctx {
    int device = 0;
    uint32_t cus = 256;
    uint64_t max_resident = 0, resident = 0;
    hipStream_t stream = nullptr;
    std::string identity, last_error;
    bool faulted = false;
    std::map<int64_t, prism::rt::Weight> weights;
    std::map<uint64_t, int64_t> by_key;
    int64_t next_id = 1;
    int *err = nullptr;  // device error flag
    prism::rt::DevBuf x, act, act2, out, gate, up, h, hr, res, pre, sk, lora;
    // This device's copy of the fixed scratch array (static_scratch.hip), looked up at
    // creation; nullptr if the lookup failed.
    void *noalloc = nullptr;
    size_t noalloc_bytes = 0;
    std::string noalloc_error;
    prism_hip_statistics stats = {};
    prism_hip_diagnostics diag = {};
    const int32_t *cancel = nullptr;  // the request owner's cancellation flag, if any
};

namespace prism {
hipError_t static_scratch_address(int device, void **ptr, size_t *bytes);
}

namespace prism::rt {

inline int fail(prism_hip_ctx *c, int code, const std::string &msg) {
    if (c) c->last_error = msg;
    return code;
}

// HIP errors after which the device or its queue can no longer be trusted: the
// context latches them.  The reference latches device loss, a submission timeout and
// a failed fence wait (tools/adreno-vulkan/src/device.rs:1450-1490); argument and
// launch-configuration errors return an error and leave the context usable.
inline bool device_fault(hipError_t e) {
    switch (e) {
    case hipErrorIllegalAddress:
    case hipErrorLaunchFailure:
    case hipErrorLaunchTimeOut:
    case hipErrorPriorLaunchFailure:
    case hipErrorECCNotCorrectable:
    case hipErrorAssert:
    case hipErrorNoDevice:
    case hipErrorContextIsDestroyed:
    case hipErrorDeinitialized:
    case hipErrorRuntimeMemory:
    case hipErrorRuntimeOther:
    case hipErrorUnknown: return true;
    default: return false;
    }
}

// Maps a HIP failure to an ABI code; only device faults latch.
inline int hip_fail(prism_hip_ctx *c, hipError_t e, const char *what) {
    std::string m = std::string(what) + ": " + hipGetErrorString(e);
    if (e == hipErrorOutOfMemory || e == hipErrorLaunchOutOfResources) return fail(c, PRISM_ERR_RESOURCE, m);
    if (device_fault(e)) {
        c->faulted = true;
        return fail(c, PRISM_ERR_DEVICE_FAULT, m);
    }
    if (e == hipErrorInvalidValue || e == hipErrorInvalidDevicePointer || e == hipErrorInvalidHandle)
        return fail(c, PRISM_ERR_INVALID_INPUT, m);
    return fail(c, PRISM_ERR_UNSUPPORTED, m);
}

// Maps a launcher's status (kernels.hpp launch_status) to an ABI code.
inline int launch_result(prism_hip_ctx *c, int rc, const char *what) {
    if (rc == 0) return PRISM_OK;
    if (rc < 0) return fail(c, PRISM_ERR_UNSUPPORTED, std::string(what) + ": geometry not supported by the kernels");
    return hip_fail(c, static_cast<hipError_t>(rc), what);
}

#define HIP_OR_FAIL(ctx, call)                                 \
    do {                                                       \
        hipError_t e_ = (call);                                \
        if (e_ != hipSuccess) return hip_fail(ctx, e_, #call); \
    } while (0)

// Grows a scratch buffer.  Work runs on the context stream only, so a capture in
// progress there means the buffer is about to be baked into a graph: growing it would
// free memory the graph already references, so that is refused (size the scratch with
// one uncaptured call first).
inline int ensure(prism_hip_ctx *c, DevBuf &b, size_t bytes) {
    if (bytes <= b.cap) return PRISM_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(c->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        return fail(c, PRISM_ERR_UNSUPPORTED, "scratch would grow during graph capture: run the call once uncaptured");
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr;
    b.cap = 0;
    size_t n = bytes < 4096 ? 4096 : bytes;
    hipError_t e = hipMalloc(&b.p, n);
    if (e != hipSuccess) return hip_fail(c, e, "hipMalloc(scratch)");
    b.cap = n;
    return PRISM_OK;
}

// The stream a device-pointer call runs on.  The context's scratch buffers and error
// flag are shared by all of its calls, so they are ordered on the one context stream;
// another stream would race on them and is rejected.
inline int call_stream(prism_hip_ctx *c, void *stream, hipStream_t *out) {
    if (stream && static_cast<hipStream_t>(stream) != c->stream)
        return fail(c, PRISM_ERR_INVALID_INPUT, "device calls run on the context stream (NULL or prism_hip_stream)");
    *out = c->stream;
    return PRISM_OK;
}

// Device scratch of one call.  Grow mode (base == nullptr): each role is one of the
// context's grow-only buffers.  Fixed mode: every request is carved, 256-byte aligned,
// from one region that is never grown or freed (the static per-device array of the
// no-allocation entry point); a call that needs more than the region fails cleanly.
struct Scratch {
    prism_hip_ctx *c = nullptr;
    uint8_t *base = nullptr;
    size_t cap = 0, used = 0;

    int get(DevBuf &role, size_t bytes, void **p, size_t *got = nullptr) {
        if (!base) {
            const int rc = ensure(c, role, bytes);
            if (rc) return rc;
            *p = role.p;
            if (got) *got = role.cap;
            return PRISM_OK;
        }
        const size_t at = (used + 255) & ~size_t(255);
        if (at > cap || bytes > cap - at) {
            char m[160];
            std::snprintf(m, sizeof m, "call needs %zu more bytes of scratch than the %zu-byte static scratch holds",
                          at + bytes - cap, cap);
            return fail(c, PRISM_ERR_UNSUPPORTED, m);
        }
        used = at + bytes;
        *p = base + at;
        if (got) *got = bytes;
        return PRISM_OK;
    }
};

inline bool cancelled(const prism_hip_ctx *c) { return c->cancel && __atomic_load_n(c->cancel, __ATOMIC_ACQUIRE) != 0; }

// Weight management: only a latched fault refuses it (cancellation concerns requests).
inline int check_live(prism_hip_ctx *c) {
    if (!c) return PRISM_ERR_INVALID_INPUT;
    if (c->faulted) return fail(c, PRISM_ERR_DEVICE_FAULT, "device fault latched");
    return PRISM_OK;
}

inline int check_ready(prism_hip_ctx *c) {
    if (!c) return PRISM_ERR_INVALID_INPUT;
    if (c->faulted) return fail(c, PRISM_ERR_DEVICE_FAULT, "device fault latched");
    if (cancelled(c)) return fail(c, PRISM_ERR_CANCELLED, "cancelled by the request owner");
    return PRISM_OK;
}

// One public call, recorded into the context's statistics and diagnostics when it ends
// (MatvecStatistics::record, src/kernels.rs:1798-1830): n matrices, and whether the call
// prepares (quantizes) its own F32 activation.  The call marks a rejected activation with
// bad_input() and the point past every check with dispatch(); operator() records the
// outcome and passes the return code through.
struct Tally {
    prism_hip_ctx *c;
    uint32_t n;
    bool prepares;
    bool input_ok = true, dispatched = false;
    Tally(prism_hip_ctx *ctx, uint32_t matrices, bool prep) : c(ctx), n(matrices), prepares(prep) {}
    void bad_input() { input_ok = false; }
    void dispatch() { dispatched = true; }
    static void add(uint64_t &v, uint64_t k) { v = v > UINT64_MAX - k ? UINT64_MAX : v + k; }
    int operator()(int rc) {
        if (!c) return rc;
        prism_hip_statistics &s = c->stats;
        const bool ok = rc == PRISM_OK && dispatched;
        if (prepares) {
            add(s.preparations, 1);
            if (!input_ok) add(s.preparation_failures, 1);
        }
        if (n == 0 || !input_ok) {  // a preparation alone, or no matrix could be attempted
            if (n) c->diag = prism_hip_diagnostics{0, 0};
            return rc;
        }
        add(s.matrix_attempts, n);
        if (ok) add(s.matrix_successes, n);
        if (!dispatched) {
            add(s.rejected_before_dispatch, n);
        } else {
            add(s.device_operations, n);
            if (n > 1) add(s.grouped_dispatches, 1);
        }
        c->diag = prism_hip_diagnostics{dispatched ? 1 : 0, ok ? 1 : 0};
        return rc;
    }
};

inline const Weight *find(prism_hip_ctx *c, prism_weight_id w) {
    auto it = c->weights.find(w);
    return it == c->weights.end() ? nullptr : &it->second;
}

// Reads and clears the device error flag after the stream drained.
inline int drain(prism_hip_ctx *c, hipStream_t s) {
    HIP_OR_FAIL(c, hipStreamSynchronize(s));
    int flag = 0;
    HIP_OR_FAIL(c, hipMemcpy(&flag, c->err, sizeof(int), hipMemcpyDeviceToHost));
    if (flag) {
        if (const int e = launch_fill_i32(c->err, 0, 1, s)) return launch_result(c, e, "reset error flag");
        HIP_OR_FAIL(c, hipStreamSynchronize(s));
        if (flag & kErrInput) return fail(c, PRISM_ERR_NONFINITE, "non-finite activation input");
        if (flag & kErrQuantRange) return fail(c, PRISM_ERR_NONFINITE, "activation quantization scale overflow");
        return fail(c, PRISM_ERR_NONFINITE, "non-finite value in projection output");
    }
    return PRISM_OK;
}

inline int quantize(prism_hip_ctx *c, int contract, const float *x, uint64_t cols, uint32_t tokens, int pinned, void *out,
             hipStream_t s) {
    int rc = contract == 0 ? launch_quantize_q8k(x, cols, tokens, pinned, out, c->err, s)
                           : launch_quantize_q8_0(x, cols, tokens, contract == 2 ? PRISM_Q8_PINNED_NATIVE
                                                                                : (pinned ? PRISM_Q8_PINNED
                                                                                          : PRISM_Q8_SOURCE),
                                                  out, c->err, s);
    return launch_result(c, rc, "quantize launch");
}

inline size_t act_bytes(int contract, uint64_t cols, uint32_t tokens) {
    return contract == 0 ? sizeof(prism_q8k_block) * ((cols + 255) / 256) * tokens
                         : sizeof(prism_q8_block) * (cols / 32) * tokens;
}

inline MatvecArgs matvec_args(prism_hip_ctx *c, const Weight &w, int act_format, const void *act, uint32_t tokens, int pinned,
                       float *out, hipStream_t s) {
    MatvecArgs a;
    a.kind = w.kind;
    a.cols = w.cols;
    a.rows = w.rows;
    a.row_bytes = w.row_bytes;
    a.w = static_cast<const uint8_t *>(w.dev);
    a.act = act;
    a.act_format = act_format;
    a.tokens = tokens;
    a.pinned = pinned;
    a.out = out;
    a.err = c->err;
    a.stream = s;
    a.cus = c->cus;
    return a;
}

// sc == nullptr: the context's grow-only buffers.
inline int run_matvec(prism_hip_ctx *c, const MatvecArgs &args, bool tiled, Scratch *sc = nullptr) {
    MatvecArgs a = args;
    if (tiled) {
        if (sc && sc->base) {  // a fixed buffer: what is left of it bounds the kernel choice
            const size_t at = (sc->used + 255) & ~size_t(255);
            a.scratch_cap = at < sc->cap ? sc->cap - at : 0;
        }
        const size_t need = tiled_scratch_bytes(a);
        if (need) {
            Scratch grow{c};
            const int e = (sc ? *sc : grow).get(c->sk, need, &a.scratch, &a.scratch_bytes);
            if (e) return e;
        }
    }
    return launch_result(c, tiled ? launch_matvec_tiled(a) : launch_matvec(a), "matvec launch");
}

inline int matvec(prism_hip_ctx *c, const Weight &w, int act_format, const void *act, uint32_t tokens, int pinned,
           float *out, hipStream_t s, Scratch *sc = nullptr) {
    return run_matvec(c, matvec_args(c, w, act_format, act, tokens, pinned, out, s), w.tiled, sc);
}

// f32 input for a tiled weight, quantized in the kernel prologue with the contract
// matvec_into would use; `residual` is added to every output row.
inline MatvecArgs f32_args(prism_hip_ctx *c, const Weight &w, const float *x, uint32_t tokens, int pinned, float *out,
                    const float *residual, hipStream_t s) {
    MatvecArgs a = matvec_args(c, w, kActF32, x, tokens, pinned, out, s);
    const int contract = contract_for(w.kind, w.cols, pinned);
    a.qcontract_is_q8k = contract == 0;
    a.qcontract = contract == 0 ? pinned : contract == 2 ? PRISM_Q8_PINNED_NATIVE : (pinned ? PRISM_Q8_PINNED : PRISM_Q8_SOURCE);
    a.residual = residual;
    return a;
}

}  // namespace prism::rt
