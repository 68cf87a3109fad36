// kernels.hpp -- host-side launchers of the gfx950 kernels (internal to libprism_hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prism {

// Device error bits raised by kernels, read back by prism_hip_sync.
constexpr int kErrNonfinite = 1;   // non-finite output / scale (PRISM_ERR_NONFINITE)
constexpr int kErrQuantRange = 2;  // activation quantizer overflow (PRISM_ERR_NONFINITE)
constexpr int kErrInput = 4;       // non-finite activation input (PRISM_ERR_NONFINITE)

// Activation-side formats consumed by the matvec kernels.
enum ActFormat : int { kActQ8K = 0, kActQ8 = 1 };

// Which binary32 order a projection follows.
//   kind PTQ1 + Q8   : src (dot_q8_groups) or pinned (dot_q8_groups_pinned)
//   kind PTQ1 + Q8K  : dot_ptq1_q8k
//   kind PQ2  + Q8K  : unfused or fused (dot_pq2::<FUSED>)
//   kind PQ2  + Q8   : dot_q8_groups (odd group count)
//   kind Q2_K + Q8K  : kquants::dot
//   kind Q8_0 + Q8   : dot_legacy
struct MatvecArgs {
    uint32_t kind;
    uint64_t cols, rows, row_bytes;
    const uint8_t *w;  // device, rows*row_bytes
    const void *act;   // device, token-major prepared blocks
    int act_format;    // ActFormat
    uint32_t tokens;
    int pinned;        // pinned Q8 order (PTQ1) or fused FMA (PQ2 + Q8K)
    float *out;        // device, [tokens][rows]
    int *err;          // device error flag
    hipStream_t stream;
};

// Returns 0 on success, -1 when the launch failed, -2 when the shape is unsupported.
// launch_matvec reads weights in the native row-major layout, launch_matvec_tiled in
// the 64-row tiled layout of tiled.hpp.
int launch_matvec(const MatvecArgs &a);
int launch_matvec_tiled(const MatvecArgs &a);
// Whether (kind, cols, rows) can be stored tiled, and the native -> tiled repack
// (the destination must hold tiled_bytes() and be zero-filled beforehand).
bool tiled_supported(uint32_t kind, uint64_t cols, uint64_t rows);
int launch_repack(const void *native, void *tiled, uint32_t kind, uint64_t cols, uint64_t rows, hipStream_t s);
int launch_quantize_q8k(const float *x, uint64_t cols, uint32_t tokens, int pinned, void *out, int *err,
                        hipStream_t s);
int launch_quantize_q8_0(const float *x, uint64_t cols, uint32_t tokens, int contract, void *out, int *err,
                         hipStream_t s);
// h = SwiGLU(gate, up) elementwise (source or pinned order), n values per token.
int launch_swiglu(const float *gate, const float *up, float *h, uint64_t n, uint32_t tokens, int pinned, int *err,
                  hipStream_t s);
// out += residual, flagging non-finite sums.
int launch_add_residual(float *out, const float *residual, uint64_t n, int *err, hipStream_t s);
// p[0..n) = v with a kernel (safe inside captured graphs, unlike a memset node).
int launch_fill_i32(int *p, int v, uint32_t n, hipStream_t s);

}  // namespace prism
