// Batched prefill for the GQA families: a whole prompt chunk per kernel, with
// the projections on the matrix cores (gemm.h) and causal windowed attention
// over the chunk's own keys plus the ring (keys of earlier positions).
#pragma once

#include "gemm.h"

namespace mr {

struct PrefillAttnArgs {
    const float *qkv = nullptr;     // [rows, ld]: q (heads*d) | k (kvw) | v (kvw), normalized and rotated
    int ld = 0;
    const float *ring_k = nullptr;  // [cap, kvw]: position p < p0 at slot p % cap
    const float *ring_v = nullptr;
    int cap = 0;                    // ring rows = attention window (model.py:105)
    float *out = nullptr;           // [rows, ldo] attended values per query head
    int ldo = 0;
    int p0 = 0, rows = 0;           // position of row 0, rows in the chunk
    int heads = 0, kv_heads = 0, d = 0;
    float inv_root = 1.0f;          // 1 / sqrt(d)
    int window = 0;                 // keys a query sees (0: cap)
    int hole = 0;                   // > 0: the key at position p - hole is not seen (latent memory)
    const float *ext = nullptr;     // [rows][heads][d + 4]: m, l, 2 unused, o[d] of extra columns, merged at the end
    // Optional workspace (head dims 32/64/128): the keys and values of the
    // positions the chunk attends to, split once into FP16 terms (4 planes of
    // kv16_rows x kv_heads*d halves, in 32-row tiles from the first attended
    // position, so kv16_rows covers the attended rows rounded up to 32) with
    // per-KV-head scales (kv16_scale, 2 kv_heads floats; kv16_max, 2 kv_heads
    // words); without it (or with too few rows) every workgroup splits its
    // tiles itself.
    _Float16 *kv16 = nullptr;
    int kv16_rows = 0;
    float *kv16_scale = nullptr;
    unsigned *kv16_max = nullptr;
    // Optional with kv16: room for kv_part_blocks x 2 kv_heads words, the
    // per-block maxima of the K/V maxima pass, which the split then reduces
    // per head (no zeroing and no atomics on the same 2 kv_heads words).
    unsigned *kv_part = nullptr;
    int kv_part_blocks = 0;
    // With out_hl (the presplit form above, no ext): the attended values go
    // out as the O projection's FP16 terms (gemm.h, a_split) instead of into
    // out.  Every output is a convex combination of values, so the power of
    // two that maps the largest |v| of every KV head into [2^13, 2^14) serves
    // as every row's scale: into out_scale[r], and o 2^t = hi + lo into planes
    // [hi: rows x ldo | lo: rows x ldo] of out_hl.
    _Float16 *out_hl = nullptr;
    float *out_scale = nullptr;
};

// Blocks of the K/V maxima pass over n attended positions (kv_part's rows):
// kKvMaxRows positions each.
constexpr int kKvMaxRows = 32;
__host__ __device__ inline int prefill_kv_max_blocks(int n) { return (n + kKvMaxRows - 1) / kKvMaxRows; }

// Whether launch_prefill_attention takes the presplit form for a (head dims
// 32, 64 or 128, with the kv16 workspace and enough rows in it).
bool prefill_attention_presplit(const PrefillAttnArgs &a);

// out = softmax(q . k / sqrt(d)) . v per query head over the keys at
// positions max(0, p - window + 1) .. p of each query position p (but
// p - hole), keys before the chunk read from the ring at slot position % cap;
// with ext, the extra columns' partial joins the softmax.
int launch_prefill_attention(hipStream_t s, const PrefillAttnArgs &a);
// y[i] = 2^x[i] by the prefill attention's hardware exp2 (which 0) or
// e^x[i] by expf (which 1), for measuring their errors.
int launch_debug_exp(hipStream_t s, const float *x, float *y, int n, int which);

// flashnano-1.6's relay rows (keys pooled from completed chunks) as the
// attention's extra partial: ext[t][head] = (m, l, 0, 0, o[d]) over the first
// ((p0 + t) / chunk) * slots relay rows (d a multiple of 4, at most 128).
struct RelayPartialArgs {
    const float *qkv = nullptr;   // [rows, ld]: normalized, rotated queries at column 0
    int ld = 0;
    const float *relay_k = nullptr, *relay_v = nullptr;   // [relay rows, kv_heads * d]
    float *ext = nullptr;         // [rows][heads][d + 4]
    int p0 = 0, rows = 0, heads = 0, kv_heads = 0, d = 0, chunk = 0, slots = 0;
    float inv_root = 1.0f;
};
int launch_relay_partial(hipStream_t s, const RelayPartialArgs &a);

// y[r] = x[r] * (1 / sqrt(mean(x[r]^2) + eps)) * gain (gain may be null).
// k_rms_rows straight into an FP16-term GEMM's A workspace (row scales and
// hi / lo planes, see gemm.h): the GEMM then runs with a_split.  With
// oscale (width <= 2048), also the scales that put the rows' SwiGLU output
// (gemm.h c_hl) below 2^14, from the gate and up weights' row norm bounds ng
// and nu (gemm_row_norm_bound).
int launch_rms_rows_split(hipStream_t s, const float *x, int ldx, const float *gain, float eps, int width,
                          float *scale, _Float16 *planes, int rows, float ng = 0.0f, float nu = 0.0f,
                          float *oscale = nullptr);
// The widths launch_rms_rows_split takes: multiples of 8 up to 8192 (wider
// rows take launch_rms_rows and the GEMM's own split).
inline bool rms_split_fits(int width) { return width % 8 == 0 && width <= 8192; }
int launch_rms_rows(hipStream_t s, const float *x, int ldx, const float *gain, float eps, int width, float *y,
                    int ldy, int rows);

// Per-head RMSNorm (q_norm / k_norm, when `norm`) and RoPE at position p0 + r of
// the q and k heads of each qkv row, in place (model.py:100-103).
int launch_qk_rows(hipStream_t s, float *qkv, int ld, int rows, int p0, int heads, int kv_heads, int d,
                   const float *q_gain, const float *k_gain, float eps, int norm, const float *rope, int split_half);

// Key heads only (RMSNorm with k_gain, RoPE) of rows whose positions are
// positions[r] (rows of width ld, keys at column 0).
int launch_k_rows_at(hipStream_t s, float *k, int ld, int rows, const int *positions, int kv_heads, int d,
                     const float *k_gain, float eps, const float *rope, int split_half);

// Ring rows of the chunk's last min(rows, cap) positions (model.py:21-25).
int launch_ring_store(hipStream_t s, const float *qkv, int ld, int qd, int kvw, float *ring_k, float *ring_v, int cap,
                      int p0, int rows);

// x[r] = embed[ids[p0 + r]] widened to FP32 (model.py:259).
int launch_embed_rows(hipStream_t s, const void *table, int dtype, const int *ids, int p0, int rows, float *x, int h);

}  // namespace mr
