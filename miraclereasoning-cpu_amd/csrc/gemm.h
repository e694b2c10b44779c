// MFMA GEMM for batched prefill: C[m, n] = A[m, k] . W[n, k]^T with FP32
// activations, BF16/F16/FP32 weights and FP32-faithful products.
//
// The matrix cores multiply BF16 operands exactly into FP32 accumulators.  An
// FP32 activation is carried as the sum of three BF16 terms (hi + mid + lo,
// each rounded to nearest even from the remainder of the previous), which
// leaves about 2^-27 of its value behind; weights are BF16 (one term), F16
// (two terms, exact: 11 significant bits fit in hi + lo) or FP32 (three
// terms).  Products of terms whose orders sum to at most 2 are accumulated
// (3, 5 or 6 MFMAs per tile step), so the result carries FP32-level error.
#pragma once

#include "common.h"

namespace mr {

enum GemmEpilogue { GEMM_STORE = 0, GEMM_RESIDUAL = 1, GEMM_SWIGLU = 2 };

struct GemmArgs {
    const float *a = nullptr;    // [m, lda] FP32 activations
    int lda = 0;
    const void *w = nullptr;     // [n, k] weight rows (gate rows for GEMM_SWIGLU)
    const void *w2 = nullptr;    // GEMM_SWIGLU: up rows
    int dtype = MR_BF16;
    float *c = nullptr;          // [m, ldc] output; GEMM_RESIDUAL updates it in place
    int ldc = 0;
    int m = 0, n = 0, k = 0;     // GEMM_SWIGLU: n = output columns (FFN width)
    float scale = 1.0f;          // GEMM_RESIDUAL: c += scale * (A . W^T)
};

// STORE:    c = A . W^T
// RESIDUAL: c = c + scale * (A . W^T)
// SWIGLU:   c = silu(A . Wg^T) * (A . Wu^T), silu(g) = g / (1 + exp(-g))
// Requires k % 8 == 0, lda % 4 == 0 and 16-byte aligned a and weight rows.
int launch_gemm(hipStream_t s, int epilogue, const GemmArgs &g);

// Groups of rows with their own weights (the experts of a batched MoE), one
// launch: group z multiplies rows offset[z] .. offset[z] + count[z] of g.a by
// w[z] (and w2[z]) into the same rows of g.c; g.w, g.w2 and g.m are unused.
// Weight rows must be 16-byte aligned.  STORE and SWIGLU epilogues.
struct GemmGroups {
    const int *offset = nullptr;     // [groups] device
    const int *count = nullptr;      // [groups] device
    void *const *w = nullptr;        // [groups] device table of weight pointers
    void *const *w2 = nullptr;       // [groups] SWIGLU up rows
    int groups = 0;
    int max_rows = 0;                // bound on every count (sizes the grid)
};
int launch_gemm_grouped(hipStream_t s, int epilogue, const GemmArgs &g, const GemmGroups &gg);

}  // namespace mr
