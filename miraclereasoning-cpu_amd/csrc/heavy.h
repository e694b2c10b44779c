// heavy-medium-2.0 token-step kernels (model.py:192-255): latent KV with
// block-mean sparse attention and grouped adaptive MoE, all control on device.
#pragma once

#include <algorithm>

#include "common.h"

namespace mr {

struct HeavyAttnArgs {
    const float *q = nullptr;        // [heads*d] raw projection (the Q rows of the packed Q/latent GEMV)
    const float *kv = nullptr;       // [2*kv_heads*d] kv_up output: keys then values
    const float *rope = nullptr;     // [positions][d/2][2] cos, sin
    const int *pos = nullptr, *done = nullptr;
    float *q_rot = nullptr;          // [heads*d] normalized, rotated queries
    float *ring_k = nullptr, *ring_v = nullptr;   // [context, kv_heads*d] of this inner loop
    float *bsum_k = nullptr, *bsum_v = nullptr;   // [blocks, kv_heads*d] running block sums
    float *out = nullptr;            // [heads*d] attended values
    float *part = nullptr;           // [heads][heavy_parts(window, context)][d + 2] split partials (or null)
    // With kv_w set, the K/V projection of the latent runs inside the
    // attention prologue (heavy_kv_fused geometries) and kv is not read.
    const void *kv_w = nullptr;      // [2*kv_heads*d, latent] kv_up weight
    const float *latent_x = nullptr; // [latent] the latent projection
    int kv_dtype = MR_BF16, latent = 0;
    int *choice = nullptr;           // choice record of this layer/loop at position 0 (or null)
    int choice_stride = 0;           // ints between the records of consecutive positions
    int choice_blocks = 0;           // offset of the block lists inside a record
    int heads = 0, kv_heads = 0, d = 0, window = 0, block = 0, slots = 0;
    float slope = 0.0f;              // alibi_slope_scale / sqrt(d), FP32
};

// Split form of the attention (head dims 32/64/128): one partial per 32 rows
// of the window and one for the chosen blocks.
constexpr int kHeavyRows = 32;
inline int heavy_window_splits(int window, int context) {
    return (std::min(window, context) + kHeavyRows - 1) / kHeavyRows;
}
inline int heavy_parts(int window, int context) { return heavy_window_splits(window, context) + 1; }
bool heavy_split_path(int d, int window, int context, int block, int slots);
bool heavy_kv_fused(int dtype, int latent);

int launch_heavy_attention(hipStream_t s, const HeavyAttnArgs &a, int context);

struct MoeArgs {
    const float *router = nullptr;   // [groups + experts] coarse then fine logits (no biases)
    const float *coarse_bias = nullptr, *group_bias = nullptr, *fine_bias = nullptr, *expert_bias = nullptr;
    const float *x = nullptr;        // [h] RMS-normalized input of the experts
    void *const *gate = nullptr;     // [experts + shared] weight pointers: routed, then shared
    void *const *up = nullptr;
    void *const *down = nullptr;
    int dtype = MR_BF16;
    const int *done = nullptr;
    const int *pos = nullptr;        // position of the token (or null: `position`)
    int position = 0;
    int *ids = nullptr;              // [kmax] chosen experts, descending probability
    float *weights = nullptr;        // [kmax] renormalized weights (0 beyond active)
    int *active = nullptr;           // adaptive width
    float *act = nullptr;            // [(kmax + shared) * ffn] SwiGLU activations per slot
    float *hidden = nullptr;         // residual stream, updated in place
    int *choice = nullptr;           // choice record of this layer/loop at position 0 (or null)
    int choice_stride = 0;
    int experts = 0, groups = 0, kmin = 0, kmax = 0, shared = 0, ffn = 0, h = 0;
    float inv_temperature_div = 1.0f;   // max(temperature, 1e-4), FP32 (logits are divided by it)
    float log_experts = 1.0f;           // max(float32(log(E)), 1)
    float shared_scale = 1.0f;          // residual_scale / shared, FP32
    float scale = 1.0f;                 // residual_scale / sqrt(inner_loop_steps), FP32
};

int launch_moe(hipStream_t s, const MoeArgs &a);

// ---- batched prefill of a chunk of rows (positions p0 .. p0 + rows - 1) ----

// Block sums of one inner-loop pass after its ring holds the chunk's keys and
// values: for every row, the running sum of its block up to the row (keys then
// values, [rows][2 kv_heads d]), in row order from the block's running sum
// before the chunk, as the token step adds them; bsum_k / bsum_v end holding
// the running sums after the chunk.
struct HeavyScanArgs {
    const float *ring_k = nullptr, *ring_v = nullptr;   // [context, kvw], rows p0 .. p0 + rows - 1 stored
    float *bsum_k = nullptr, *bsum_v = nullptr;         // [blocks, kvw]
    float *sums = nullptr;                              // [rows][2 kvw]
    int p0 = 0, rows = 0, kvw = 0, block = 0;
};
int launch_heavy_scan(hipStream_t s, const HeavyScanArgs &a);

// Per row and query head: the block columns scored as the token step scores
// them (block-sum quotients, sequential dot product, distance penalty), the
// stable top-k, the choice record, and the chosen blocks' softmax partial
// ext[row][head] = (m, l, -, -, o[d]) for launch_prefill_attention.
struct HeavySelectArgs {
    const float *qkv = nullptr;      // [rows, ld]: normalized, rotated queries at column 0
    int ld = 0;
    const float *bsum_k = nullptr, *bsum_v = nullptr;   // after the scan
    const float *sums = nullptr;     // [rows][2 kvw] from the scan
    float *ext = nullptr;            // [rows][heads][d + 4]
    int *choice = nullptr;           // choice record of this layer/loop at position 0 (or null)
    int choice_stride = 0, choice_blocks = 0;
    int p0 = 0, rows = 0, heads = 0, kv_heads = 0, d = 0, block = 0, slots = 0, context = 0;
    float slope = 0.0f;
};
int launch_heavy_select(hipStream_t s, const HeavySelectArgs &a);

// Routing of every row (the token step's arithmetic), then the expert-major
// gather: rows of expert e at offsets[e] .. + counts[e] of xg (routed experts,
// then one group of all rows per shared expert), map[row][slot] = gathered row.
// `a` is set up as for launch_moe with router = [rows][groups + experts]
// logits, ids / weights [rows][kmax], active [rows], x = [rows][h] input.
struct MoeRowsArgs {
    MoeArgs a;
    int rows = 0, p0 = 0;
    int *counts = nullptr, *offsets = nullptr, *fill = nullptr;   // [experts + shared]
    int *map = nullptr;              // [rows][kmax]
    int *tile_start = nullptr;       // optional [experts + shared + 1]: prefix sums of the groups' row tiles
    int tile_rows = 128;             // rows of such a tile
    float *xg = nullptr;             // [rows (kmax + shared)][h]
    // FP16 terms (h a multiple of 8): the rows' scales and planes from
    // launch_row_split over `rows` rows, gathered into the grouped GEMM's
    // workspace (planes [hi | lo] of capacity rows, one scale a row) in place
    // of xg: a row's split depends on the row alone, so the gathered split is
    // the split of the gathered rows.
    const float *x_scale = nullptr;
    const _Float16 *x_planes = nullptr;
    float *xg_scale = nullptr;
    _Float16 *xg_planes = nullptr;
    int capacity = 0;
};
int launch_moe_route_rows(hipStream_t s, const MoeRowsArgs &m);
// x[row] += scale * (sum of the routed experts' outputs by weight in chosen
// order, then the shared ones by shared_scale), y the grouped down outputs.
int launch_moe_combine_rows(hipStream_t s, const MoeRowsArgs &m, const float *y, float *x);

}  // namespace mr
