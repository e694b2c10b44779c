// Split-key decode attention over a ring window plus extra rows
// (kernels.cl:58-107 scores -> softmax -> mix, one pass, online softmax).
#pragma once

#include "common.h"

namespace mr {

// Op-level problem: queries already normalized and rotated.
struct AttnProblem {
    const float *q = nullptr;
    const float *ring_k = nullptr, *ring_v = nullptr;
    const float *extra_k = nullptr, *extra_v = nullptr;
    int heads = 0, kv_heads = 0, dim = 0, capacity = 0, start = 0, length = 0, extra_length = 0;
    float *out = nullptr;
};

int launch_attention_op(mr_ctx *ctx, const AttnProblem &p);
// Allocation-free variant: partials and counters in the device's static scratch.
int launch_attention_op_noalloc(mr_ctx *ctx, const AttnProblem &p);
int static_scratch_address(int device, void **out);
size_t static_scratch_bytes();

// Engine step: the kernel also RMS-normalizes (optional) and rotates the new
// query heads and key, writes the new key/value into the ring slot of this
// position, and takes the window geometry from the device position.
struct AttnStepArgs {
    const float *q = nullptr;          // [heads*dim] raw projection
    const float *k_new = nullptr;      // [kv_heads*dim] raw projection
    const float *v_new = nullptr;      // [kv_heads*dim]
    const float *q_gain = nullptr;     // per-head RMSNorm gains (null: no Q/K norm)
    const float *k_gain = nullptr;
    float eps = 0.0f;
    const float *rope = nullptr;       // [positions][dim/2][2] cos, sin of pos * inv_freq
    int split_half = 0;
    const int *pos = nullptr;          // device position of this token
    const int *done = nullptr;
    float *ring_k = nullptr, *ring_v = nullptr;   // [capacity, kv_heads*dim]
    int capacity = 0;
    const float *extra_k = nullptr, *extra_v = nullptr;  // relay rows
    int extra_chunk = 0, extra_slots = 0;  // extra rows = (pos / chunk) * slots
    int heads = 0, kv_heads = 0, dim = 0;
    float *part = nullptr;             // [kv_heads, splits, G, dim + 2]
    uint64_t *part_cells = nullptr;    // persistent kernel: the partials as cells [kv_heads, splits, G, dim + 2]
    unsigned *counters = nullptr;      // [kv_heads * head_groups]: zero between op-level launches; the step kernel's only grow
    float *out = nullptr;              // [heads*dim]
    int splits = 0, split_len = 0;
    // Query heads of a KV head split over this many units of each key range
    // (persistent kernel; 1 elsewhere): unit group v = kh * head_groups + hs
    // holds query heads [v * G, (v + 1) * G) with G = heads / (kv_heads *
    // head_groups), its counter, progress word and partials indexed by v.
    int head_groups = 1;
};

// Split geometry for at most `max_total` keys with kv_heads heads of `dim`, at
// most `max_units` (kv head, split) units.  The kernel divides the current key
// count over `splits`; `split_len` is the upper bound of keys per split.
void attention_plan(int max_total, int kv_heads, int dim, int max_units, int *splits, int *split_len);
size_t attention_part_floats(int heads, int kv_heads, int dim, int splits);
int launch_attention_step(hipStream_t s, const AttnStepArgs &a);

}  // namespace mr
