// MFMA GEMM for batched prefill: C[m, n] = A[m, k] . W[n, k]^T with FP32
// activations, BF16/F16/FP32 weights and FP32-faithful products.
//
// The matrix cores multiply BF16 or FP16 operands exactly into FP32
// accumulators.  BF16 scheme: an FP32 activation is carried as the sum of
// three BF16 terms (hi + mid + lo, each rounded to nearest even from the
// remainder of the previous), which leaves about 2^-27 of its value behind;
// weights are BF16 (one term), F16 (two terms, exact: 11 significant bits fit
// in hi + lo) or FP32 (three terms).  Products of terms whose orders sum to
// at most 2 are accumulated (3, 5 or 6 MFMAs per tile step), so the result
// carries FP32-level error.  FP16 scheme (BF16 weights): each activation row
// is scaled by a power of two into FP16 range and carried as hi + lo FP16
// terms (about 2^-23 of its value left behind), the weights scaled by a power
// of two are exact in FP16, and two MFMAs per tile step carry the product.
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
    // FP16 terms (BF16 weights only): wscale > 0 is the weights' power-of-two
    // scale into FP16 range (gemm_f16_weight_scale) and wh (wh2: SwiGLU up
    // rows) the weights converted with it; ascale (m floats) and ahl_ws
    // (2 m k halves) are device workspaces that receive A's row scales and its
    // hi and lo planes.  Otherwise (wscale 0) the BF16 scheme runs.
    float wscale = 0.0f;
    const void *wh = nullptr, *wh2 = nullptr;   // the weights times wscale in FP16 (gemm_f16_weight_copy)
    float *ascale = nullptr;
    _Float16 *ahl_ws = nullptr;
    bool a_split = false;            // FP16 terms: ascale and ahl_ws already hold A (a unused)
    const _Float16 *ahl = nullptr;   // set by launch_gemm for the kernel
    int64_t plane_stride = 0;        // halves from A's hi plane to its lo plane (0: m k)
    int ldw = 0;                     // elements between weight rows (0: k; set by the split GEMM)
    // GEMM_SWIGLU, FP16 terms: with c_hl the output is written as the next
    // FP16-term GEMM's A (a_split) instead of into c: row r times c_scale[r]
    // (a power of two that keeps every value of the row below 2^14) = hi + lo
    // into planes [hi: m x n | lo: m x n] of c_hl.
    _Float16 *c_hl = nullptr;
    const float *c_scale = nullptr;
};

// STORE:    c = A . W^T
// RESIDUAL: c = c + scale * (A . W^T)
// SWIGLU:   c = silu(A . Wg^T) * (A . Wu^T), silu(g) = g / (1 + exp(-g))
// Requires k % 8 == 0, lda % 4 == 0 and 16-byte aligned a and weight rows.
int launch_gemm(hipStream_t s, int epilogue, const GemmArgs &g);

// A's FP16 terms as the FP16-term GEMMs take them (a_split): row r's scale
// 2^t into scale[r], a[r][k] 2^t = hi + lo into planes [hi: m x k | lo: m x k].
int launch_row_split(hipStream_t s, const float *a, int lda, int m, int k, float *scale, _Float16 *planes);

// c = A . W^T (BF16-term scheme, no FP16 weights) with K cut into `slices`
// runs of whole k-steps, each its own workgroups' partial product in `part`
// (slices x m x n floats), then summed slice by slice in order: for a few
// output columns over many rows, where the plain GEMM has too few tiles.
int launch_gemm_split(hipStream_t s, const GemmArgs &g, int slices, float *part);

// The power of two 2^s that puts max |w| of a BF16 matrix of `count` values
// in [2^13, 2^14) (1 for an all-zero matrix), so that w 2^s is exact in FP16
// for every |w| >= 2^-31 max |w|; 0 for a matrix holding a non-finite value or
// another dtype (the FP16 scheme is then not used).  Synchronizes the stream.
int gemm_f16_weight_scale(hipStream_t s, const void *w, int dtype, int64_t count, float *scale);

// An upper bound on the largest row norm, max_r sqrt(sum_k w[r][k]^2), of a
// BF16 matrix of `rows` x `cols` values into *norm (0 for another dtype or a
// non-finite value).  Synchronizes the stream.
int gemm_row_norm_bound(hipStream_t s, const void *w, int dtype, int64_t rows, int64_t cols, float *norm);

// dst[i] = FP16(w[i] * scale) for `count` BF16 values (exact for a scale from
// gemm_f16_weight_scale, or a smaller power of two).
int gemm_f16_weight_copy(hipStream_t s, const void *w, int64_t count, float scale, void *dst);

// Groups of rows with their own weights (the experts of a batched MoE), one
// launch: group z multiplies rows offset[z] .. offset[z] + count[z] of g.a by
// w[z] (and w2[z]) into the same rows of g.c; g.w and g.w2 are unused.
// Weight rows must be 16-byte aligned.  STORE and SWIGLU epilogues.  With wh
// (BF16 weights), the FP16-term scheme: wh[z] (wh2[z]) are the groups' FP16
// copies with scales wscale[z] (SwiGLU: gate and up share it), and g.m rows
// of g.a (every row a group may hold) are split into g.ascale and g.ahl_ws
// first.  Otherwise g.m is unused and the BF16-term scheme runs.
struct GemmGroups {
    const int *offset = nullptr;     // [groups] device
    const int *count = nullptr;      // [groups] device
    void *const *w = nullptr;        // [groups] device table of weight pointers
    void *const *w2 = nullptr;       // [groups] SWIGLU up rows
    void *const *wh = nullptr, *const *wh2 = nullptr;   // [groups] FP16 copies
    const float *wscale = nullptr;   // [groups] their scales
    int groups = 0;
    int max_rows = 0;                // bound on every count (sizes the grid)
    // Optional: [groups + 1] device prefix sums of the groups' kGemmRowTile-row
    // tiles, and a bound on the last (total_rows / kGemmRowTile + groups): the
    // FP16-term kernel then runs only the groups' own row tiles, not
    // max_rows' worth in every group.
    const int *row_tile_start = nullptr;
    int row_tiles = 0;
};
constexpr int kGemmRowTile = 128;   // rows of a GEMM tile
int launch_gemm_grouped(hipStream_t s, int epilogue, const GemmArgs &g, const GemmGroups &gg);

}  // namespace mr
