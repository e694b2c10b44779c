// flashlighting-2.0 token-step kernels (model.py:146-190): latent memory with
// per-row key/value caches, window masking of non-memory rows, and compaction
// (two oldest rows merged by their counts, or dropped without memory slots).
#pragma once

#include "common.h"
#include "linear.h"

namespace mr {

// Device state of one layer's latent memory: rows live in a ring of `cap`
// slots; logical row t is slot (start + t) % cap.
// skip_merged / merged_slot / merged_pos describe the row the last compaction
// merged (its cache row not yet computed); pending says the same for the fused
// row kernel, which computes it at the start of the next step.
struct LightState {
    int start, rows, memory, skip_merged, merged_slot, merged_pos, pending, pad;
};

struct LightArgs {
    const float *qlat = nullptr;     // [heads*d + latent] raw Q and latent projections
    const float *q_gain = nullptr, *k_gain = nullptr, *latent_gain = nullptr;
    float eps = 0.0f;
    const float *rope = nullptr;     // [positions][d/2][2] cos, sin
    int split_half = 0;
    const int *pos = nullptr, *done = nullptr;
    float *q_rot = nullptr;          // [heads*d]
    float *arena = nullptr;          // [cap, latent] latent rows
    float *positions = nullptr;      // [cap] row positions (integers)
    float *counts = nullptr;         // [cap] rows folded into each row
    float *kcache = nullptr, *vcache = nullptr;   // [cap, kv_heads*d] keys (normed, rotated) and values
    float *lat_new = nullptr;        // [latent] the row whose K/V the next projection computes
    const float *kv = nullptr;       // [2*kv_heads*d] that projection's output
    LightState *st = nullptr;
    float *out = nullptr;            // [heads*d] attended values
    float *part = nullptr;           // [heads][splits][d + 2] split partials (m, l, o)
    const void *kv_w = nullptr;      // [2*kv_heads*d, latent] packed [Wk; Wv] (fused row kernel)
    int kv_dtype = MR_BF16;
    // The FFN branch's gate/up + SwiGLU rows (they read the same normalized
    // input as the attention branch) in ffn_blocks more workgroups of the fused
    // row kernel, as a GEMV launch's workgroups would run them; 0 = apart.
    GemvArgs ffn;
    int ffn_blocks = 0, ffn_lpr = 0;
    // The FFN branch's down projection (EPI_STORE into its own vector) in
    // down_blocks more workgroups of the attention split kernel: its input is
    // ready once the fused row kernel has run the gate/up rows; 0 = apart.
    GemvArgs down;
    int down_blocks = 0, down_lpr = 0, down_dtype = MR_BF16;
    int heads = 0, kv_heads = 0, d = 0, latent = 0, window = 0, memory_slots = 0, cap = 0;
};

// Rows of the latent memory per attention split (head dims 32, 64, 128 take
// the split path; other dims the single-workgroup kernel).
constexpr int kLightRows = 64;
inline int light_splits(int cap) { return (cap + kLightRows - 1) / kLightRows; }
constexpr int kLightMaxSplits = 1024;   // split weights held in the merge kernel's LDS
// The split-key attention covers head dims 32/64/128 and up to 64 Ki memory rows.
inline bool light_split_path(int d, int cap) {
    return (d == 32 || d == 64 || d == 128) && light_splits(cap) <= kLightMaxSplits;
}

// Queries, the new latent row (appended), then - after the K/V projection of
// lat_new - its key/value cache row.
int launch_light_prep(hipStream_t s, const LightArgs &a);
int launch_light_store_kv(hipStream_t s, const LightArgs &a, bool merged);
// The same three steps in one launch (queries, the appended row, and the K/V
// projection with the cache row computed per KV head from the normalized
// latent), together with the cache row of the row the previous step's
// compaction merged (no step reads it before this one's attention); for the
// dtypes and latent widths light_kv_fused accepts.
bool light_kv_fused(int dtype, int latent, int d);
// Whether the gate/up GEMV g (weights of dtype) can ride in the fused row
// kernel (kv weights of kv_dtype); sets ffn, ffn_blocks and ffn_lpr of a.
bool light_ffn_in_row_kernel(LightArgs &a, const GemvArgs &g, int dtype);
int launch_light_kv(hipStream_t s, const LightArgs &a);
// Whether the down GEMV g (weights of dtype, EPI_STORE) can ride in the
// attention split kernel; sets down, down_blocks and down_lpr of a.
bool light_down_in_attend(LightArgs &a, const GemvArgs &g, int dtype);
// Attention over every row, then compaction (which leaves the merged row in
// lat_new and clears skip_merged when a merge happened).
int launch_light_attend(hipStream_t s, const LightArgs &a);

// ---- batched prefill of a chunk of rows (positions p0 .. p0 + rows - 1) ----
//
// Every query of the chunk sees a window of original rows (W + M positions
// ending at its own, the row at distance W masked as latent_mask does) plus,
// once the two oldest rows start folding, one extra row: logical row 0, the
// running merge.  The bookkeeping depends only on positions and is planned on
// the host; the merged row's latent follows the recurrence below.
struct LightRowsArgs {
    const float *lat = nullptr;         // [rows, latent] the chunk's normalized latents
    float *arena = nullptr, *positions = nullptr, *counts = nullptr;   // the token step's ring state
    float *slot0 = nullptr;             // [extra rows, latent] logical row 0 at each step that sees it as extra
    float *slot0_final = nullptr;       // [latent] logical row 0 after the chunk
    const int *flags = nullptr;         // [rows] 1: the step sees row 0 as extra (index extra_index[t]); 2: merge after it
    const int *extra_index = nullptr;   // [rows]
    const float *merge_count = nullptr; // [rows] count of row 0 before the step's merge
    const int *merge_row = nullptr;     // [rows] position of the row folded in (logical row 1)
    int init_from_arena = 0, init_slot = 0;   // row 0 before the chunk: arena slot, or the chunk's first row
    float *merged = nullptr;            // [rows, latent] scratch: the row a step's merge folds in, at its step
    float *row0_ws = nullptr;           // scratch of light_row0_ws_floats(rows, latent) floats
    int p0 = 0, rows = 0, latent = 0, cap = 0;
};
// Logical row 0's latent through the chunk: kernels.cl merge_rows
// (a x0 + b x1) / (a + b) with b = 1 at every merge, in step order (with a
// growing by 1 a merge, evaluated as a running sum over the count: equal to
// the step-by-step form up to rounding).
int launch_light_slot0(hipStream_t s, const LightRowsArgs &a);
inline size_t light_row0_ws_floats(int rows, int latent) {
    const size_t seg = (size_t)(rows + 127) / 128;   // segments of the recurrence
    return seg * latent + 4 + 2 * seg;
}
// ext[t][h] = (q . k0 / sqrt(d), 1, -, -, v0) for steps with an extra row,
// (-inf, 0, -, -, 0) otherwise; kv0 = [extra rows][k | v] (keys normed, rotated).
int launch_light_extra(hipStream_t s, const float *qkv, int ld, const float *kv0, const int *extra_index, float *ext,
                       int rows, int heads, int kv_heads, int d);
// The chunk's rows into the ring state (latent, position, count 1) for
// positions max(p0, p0 + rows - cap) .. p0 + rows - 1.
int launch_light_store_rows(hipStream_t s, const LightRowsArgs &a);
// Logical row 0 after the chunk (when it is a merged row) and the state.
int launch_light_finish(hipStream_t s, const LightRowsArgs &a, LightState *st, const LightState &fin, int write_slot0,
                        float slot0_position, float slot0_count);

// hidden += rs * ((0 + ag * o) + fg * f)  (model.py:171-176 parallel gated residual)
int launch_light_residual(hipStream_t s, float *hidden, const float *o, const float *f, const float *attention_gate,
                          const float *ffn_gate, float rs, int n, const int *done);

}  // namespace mr
