// Persistent step kernel: one launch (one workgroup per CU) runs a whole token step as a
// program of phases whose workgroups exchange activations as flag-in-data
// cells (ll.h) instead of meeting at grid barriers.
#pragma once

#include <vector>

#include "attention_tile.h"
#include "linear.h"

namespace mr {

enum PhaseKind : int { PH_EMBED = 0, PH_GEMV = 1, PH_ATTN = 2, PH_HEAD = 3 };

// What a step does after the last layer: nothing (prompt token), LM head
// (logits for the host), or LM head + greedy choice on device.
enum StepKind { STEP_PLAIN = 0, STEP_LOGITS = 1, STEP_GREEDY = 2, STEP_KINDS = 3 };

// One phase of the step program (device memory, built once per model).  Cell
// buffers (uint64_t) hold flag-in-data activations; a read of x expects the
// epoch of phase x_phase, a residual read of y the epoch of phase res_phase.
struct Phase {
    int kind = PH_GEMV;
    // PH_EMBED: y[j] = embedding row of the position's token, j < n
    // PH_GEMV / PH_HEAD: y = epilogue(W . prologue(x)), rows split over workgroups
    int dtype = MR_BF16, n = 0, k = 0, pro = PRO_COPY, epi = EPI_STORE;
    int x_phase = -1, res_phase = -1;
    const void *w = nullptr, *w2 = nullptr;
    const uint64_t *x = nullptr;
    const float *gain = nullptr;
    float eps = 0.0f, scale = 1.0f;
    uint64_t *y = nullptr;
    float *logits = nullptr;       // PH_HEAD: plain logits for the host
    // Progress words of x's producers when they are not the stream waves
    // (the O projection waits for the attention heads' words).
    const unsigned *ready = nullptr;
    int nready = 0;
    // PH_ATTN: at.s.q / k_new / v_new / out point at cells; x_phase = Q/K/V phase
    unsigned *heads_done = nullptr;   // [kv_heads] progress words of the merged heads
    att::Args at{};
    // Workgroups that take no rows of this GEMV phase (bit b of word b / 32;
    // grids of up to kSkipBits workgroups): the rows go to the others in
    // order.  The O projection skips the workgroups that merged attention
    // heads, which finish the attention phase last.
    unsigned skip[8] = {0, 0, 0, 0, 0, 0, 0, 0};
};
constexpr int kSkipBits = 256;

// Per-launch arguments (all pointers into the model's device state).
struct StepArgs {
    const Phase *phases = nullptr;
    int nphases = 0;
    int stride = 0;                     // epochs per position (>= phases of any program)
    int kind = 0;                       // StepKind
    int *pos = nullptr, *done = nullptr, *ids = nullptr, *gen = nullptr, *count = nullptr;
    const int *eos = nullptr;
    int *err = nullptr;                 // 1 = a wait timed out
    unsigned *progress = nullptr;       // [kWordCopies][kWordCopyStride] progress words, one per workgroup
    int nprogress = 0;
    unsigned *exits = nullptr;          // workgroups that left this launch (last one finishes)
    float *best_val = nullptr;          // [grid] per-workgroup argmax partials
    int *best_idx = nullptr, *bad = nullptr;
    const void *embed = nullptr;
    int embed_dtype = MR_F32;
    const void *dummy = nullptr;        // 16 readable bytes: target of loads past a matrix's end
    int xbuf = 0;                       // floats of one GEMV input staging buffer (two in LDS)
    unsigned long long *trace = nullptr;   // optional [nphases][grid][kTraceFields]
};

// Trace record of one (phase, workgroup): wall clock (100 MHz) at the phase's
// entry, when its input was staged, when its last stream wave stored its
// outputs and when its first stream wave did; the fifth field is unused.  In
// an attention phase: entry, the unit's Q/K/V cells staged, the phase's end
// for this workgroup (after its merge, for a merging unit), the unit's partial
// stored and, in a merging unit, its first partial cells seen.
constexpr int kTraceFields = 5;

// Waves 0..kControlWaves-1 of a workgroup wait for and stage phase inputs; the
// other (stream) waves load weights, compute and store outputs.
constexpr int kStepThreads = 512;
constexpr int kControlWaves = 4;
constexpr int kStreamWaves = kStepThreads / 64 - kControlWaves;

// Progress words are written in kWordCopies copies kWordCopyStride words apart
// (4 KB + 256 B, so the copies sit on different memory channels) and each
// workgroup polls copy blockIdx % kWordCopies: every copy is polled by an
// eighth of the grid.
constexpr int kWordCopies = 8;
constexpr int kWordCopyStride = 1088;

// Floats of one GEMV input staging buffer, and the dynamic LDS of the kernel.
int step_xbuf_floats(const std::vector<Phase> &program, int grid);
size_t step_lds_bytes(const std::vector<Phase> &program, int grid);
// Attention splits per KV head in the step kernel: enough units that each
// covers its keys in one round of its waves' loads, at most cus / kv_heads.
int step_attention_splits(int max_total, int kv_heads, int dim, int cus);
// Workgroups that merge attention heads in the step kernel (the merging unit
// of each (KV head, query-head group)), as a skip mask for the next phase.
void step_attention_mergers(const AttnStepArgs &a, int grid, unsigned *mask);
// Groups the query heads of a KV head are split into (AttnStepArgs::head_groups)
// so that the (KV head, group, split) units fill up to `cus` workgroups.
int step_attention_head_groups(int heads, int kv_heads, int splits, int cus);
// The kernel is instantiated per (weight dtype of every GEMV phase, head dim).
int step_blocks_per_cu(size_t lds, int dtype, int dim, int *blocks);
int launch_step(hipStream_t s, const StepArgs &a, int grid, size_t lds, int dtype, int dim);

}  // namespace mr
