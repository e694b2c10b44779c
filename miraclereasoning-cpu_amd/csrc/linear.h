// Projection kernels: bandwidth-bound GEMV for one row of activations (decode),
// a tiled FP32 GEMM for a few rows (op-level calls), shared by ops and engine.
#pragma once

#include "common.h"

namespace mr {

enum GemvPrologue { PRO_COPY = 0, PRO_RMS = 1 };
// EPI_GATED (copy prologue only): y += scale * ((0 + (*scale_ptr) * aux) + (*scale_ptr2) * acc),
// the parallel gated residual of flashlighting-2.0 (model.py:171-176) with acc its FFN branch;
// EPI_GATED_ATTN the same sum with acc the attention branch and aux the FFN branch:
// y += scale * ((0 + (*scale_ptr) * acc) + (*scale_ptr2) * aux).
enum GemvEpilogue {
    EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2, EPI_SCALE_ADD = 3, EPI_GATED = 4, EPI_GATED_ATTN = 5
};

struct GemvArgs {
    const void *w = nullptr;     // [n, k] weight rows (gate rows for EPI_SWIGLU)
    const void *w2 = nullptr;    // up rows for EPI_SWIGLU
    const float *x = nullptr;    // input vector [k]
    const float *gain = nullptr; // PRO_RMS gain [k]; null = non-affine
    float eps = 0.0f;
    int n = 0, k = 0;
    float *y = nullptr;          // [n] output (EPI_RESIDUAL: updated in place)
    float scale = 1.0f;          // EPI_RESIDUAL: y += scale * acc
    float *x_out = nullptr;      // PRO_RMS: block 0 also stores the normalized x here
    const int *done = nullptr;   // device flag; non-zero = skip (greedy loop finished)
    const float *scale_ptr = nullptr;  // EPI_SCALE_ADD: y += (*scale_ptr) * acc
    const float *aux = nullptr;        // EPI_GATED, EPI_GATED_ATTN: [n] the other branch
    const float *scale_ptr2 = nullptr; // EPI_GATED: gate of acc; EPI_GATED_ATTN: gate of aux
};

// Launch y = epilogue(W . prologue(x)) on stream s.  Chooses a vectorized
// 16-byte-load kernel when every row starts 16-byte aligned, else a scalar one.
int launch_gemv(hipStream_t s, int dtype, int prologue, int epilogue, const GemvArgs &a);

// y[rows, n] = x[rows, k] . W[n, k]^T (FP32 accumulation), rows >= 1.
int launch_linear(hipStream_t s, const float *x, const void *w, int dtype, float *y, int rows, int n, int k);

}  // namespace mr
