// Step-level engine internals: model weights, sequence state and step launchers.
#pragma once

#include <array>
#include <vector>

#include "attention.h"
#include "heavy.h"
#include "lighting.h"
#include "linear.h"
#include "prefill.h"
#include "step.h"

namespace mr {

struct Weight {
    void *ptr = nullptr;
    int dtype = MR_F32;
    int64_t rows = 0, cols = 0;
    bool owned = true;
    // batched prefill GEMMs: power-of-two scale into FP16 range (0: the BF16
    // term scheme is used for this matrix)
    float f16_scale = 0.0f;
    void *f16 = nullptr;   // the matrix times f16_scale in FP16 (owned)
    float row_norm = 0.0f;  // SwiGLU gate and up: bound on the largest row norm (0: none)
    explicit operator bool() const { return ptr != nullptr; }
    const float *f() const { return (const float *)ptr; }
};

struct Mlp {
    Weight gate, up, down;
};

struct Layer {
    bool global = false;
    int kv_heads = 0;
    int capacity = 0;          // ring rows
    Weight a_norm, f_norm, qkv, q_norm, k_norm, o;
    Mlp ffn;
    Weight cbr;                // flashnano-1.6 learned queries [slots, h]
    float *cbr_queries = nullptr;  // RMS-normalized queries (fixed per model)
    // flashlighting-2.0
    Weight latent, latent_norm, k_up, v_up, attention_gate, ffn_gate;
    // heavy-medium-2.0: qkv packs [Wq; Wlatent], router packs [Wcoarse; Wfine]
    Weight kv_up, router, router_coarse_bias, router_fine_bias, group_bias, expert_bias;
    std::vector<Mlp> experts, shared;
    void **expert_tab = nullptr;       // device [3][experts + shared]: gate, up, down pointers
    // the batched prefill's FP16 copies of the experts (null when an expert has
    // none): device [3][experts + shared] pointers and their scales (an expert's
    // gate and up share one)
    void **expert_tab_h = nullptr;
    float *expert_scale = nullptr;
    float *bsum_k = nullptr, *bsum_v = nullptr;   // [inner][blocks, kvw] running block sums
    // flashlighting-2.0: qkv packs [Wq; Wlatent], kv_up packs [Wk; Wv]; latent
    // memory ring of light_cap rows with per-row key/value caches
    int light_cap = 0;
    float *arena = nullptr, *positions = nullptr, *counts = nullptr, *kcache = nullptr, *vcache = nullptr;
    LightState *light = nullptr;
    // caches
    float *ring_k = nullptr, *ring_v = nullptr;        // [capacity, kv_heads*dim] (per inner loop for heavy)
    float *relay_k = nullptr, *relay_v = nullptr;      // flashnano-1.6 relay
    int relay_capacity = 0;
    float *pending = nullptr;                          // flashnano-1.6 chunk rows
    int splits = 0, split_len = 0;                     // attention plan
    int step_splits = 0;                               // attention splits in the step kernel
    int step_head_groups = 1;                          // query-head groups per KV head in the step kernel
};

}  // namespace mr

struct mr_model {
    mr_ctx *ctx = nullptr;
    mr_model_desc d{};
    std::vector<mr::Layer> layers;
    mr::Weight embed, output, norm;
    float *freq = nullptr;       // [head_dim/2] inverse frequencies
    float *rope = nullptr;       // [context][head_dim/2][2] cos, sin per integer position
    bool finalized = false;
    int position = 0;            // host mirror of *pos_dev
    // device state (one allocation, see engine.hip)
    void *state = nullptr;
    int *pos_dev = nullptr;      // position of the next token
    int *done_dev = nullptr;     // 0 run; 1 greedy loop hit EOS; 2 non-finite logits
    int *ids_dev = nullptr;      // [context+1] token per position
    int *gen_dev = nullptr;      // [context+1] generated tokens; gen_dev[-1] is at count_dev
    int *count_dev = nullptr;    // number of generated tokens
    int *eos_dev = nullptr;      // EOS id for the greedy loop (-1 none)
    int *cbr_skip = nullptr;     // flashnano-1.6: non-zero = no chunk completes this step
    float *hidden = nullptr, *xnorm = nullptr, *qkv = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr;
    float *part = nullptr;
    unsigned *counters = nullptr;
    float *cbr_pooled = nullptr, *cbr_anchor = nullptr, *cbr_kv = nullptr;
    // heavy-medium-2.0 step buffers and the per-position choice log
    float *q_rot = nullptr, *kvbuf = nullptr, *router_out = nullptr, *moe_w = nullptr, *moe_act = nullptr;
    int *moe_ids = nullptr, *moe_active = nullptr;
    float *lat_new = nullptr, *branch_o = nullptr, *branch_f = nullptr;   // flashlighting-2.0
    float *split_part = nullptr;         // split decode attention partials (latent and block-sparse families)
    int *choices = nullptr;              // [context + 1][layers][inner][choice_rec]
    int choice_rec = 0;                  // ints per record: active, kmax ids, heads x slots blocks
    // step execution: persistent kernel (when the model fits its phases) or
    // per-layer kernels replayed from a hipGraph / launched eagerly
    int mode = MR_STEP_PERSISTENT;
    bool persistent_ok = false;
    int grid = 0;                        // persistent workgroups (one per CU)
    int step_dtype = MR_BF16;            // weight dtype of every GEMV phase
    size_t step_lds = 0;
    mr::Phase *prog_plain = nullptr, *prog_head = nullptr;
    int n_plain = 0, n_head = 0;
    // Persistent-kernel state, cleared on reset: flag-in-data activation cells
    // (hidden, qkv, attn, act) and the launch exit counter.
    uint64_t *cells = nullptr;
    size_t cell_count = 0;
    uint64_t *c_hidden = nullptr, *c_qkv = nullptr, *c_attn = nullptr, *c_act = nullptr;
    unsigned *sync = nullptr;
    size_t sync_count = 0;
    // progress words: one per workgroup [grid], then the merged
    // attention heads' [layers * query_heads]
    unsigned *words = nullptr;
    size_t word_count = 0;
    uint64_t *part_cells = nullptr;      // attention partials (m, l, o) as cells
    unsigned *merge_counts = nullptr;    // [layers][max kv heads] finished attention units (only grow)
    size_t merge_count_n = 0;
    size_t part_cell_count = 0;
    int xbuf = 0;                        // floats of one GEMV input staging buffer
    void *dummy = nullptr;               // 16 zero bytes for loads past a matrix's end
    int *err = nullptr;                  // wait timeout flag
    bool timed_out = false;              // a persistent step timed out: graph mode from the next reset
    bool inject_timeout = false;         // test hook: report the next step status as timed out
    float *best_val = nullptr;
    int *best_idx = nullptr, *bad = nullptr;
    float last_ms = 0.0f;                // device time of the last greedy loop
    // batched prefill workspace, grown on demand
    void *pf = nullptr;
    size_t pf_bytes = 0;
    std::array<hipGraphExec_t, mr::STEP_KINDS> exec{};
    std::array<int, mr::STEP_KINDS> eager_runs{};
};

namespace mr {
int record_step(mr_model *m, int kind);   // enqueue one step's kernels on the context stream
}
