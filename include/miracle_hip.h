/*
 * miracle_hip.h — C ABI of libmiracle_hip.so, the MI355X (gfx950) backend of the
 * Miracle per-token forward path.
 *
 * It replaces the reference's OpenCL binding (miracle_reasoning/opencl.py) and
 * kernel file (miracle_reasoning/kernels.cl).  Every function returns 0 on
 * success and a non-zero MR_ERR_* code otherwise; mr_last_error() then holds a
 * message naming the operation (thread-local).  No C++ exception crosses the
 * ABI.  Pointers named "device" are HBM addresses obtained from mr_alloc; all
 * other pointers are host memory.  A context owns one HIP stream; work on it
 * runs in order.  A context, and every model created on it, must be used by one
 * thread at a time (the reference's rule for a backend and its queue,
 * opencl.py:130-133).
 */
#ifndef MIRACLE_HIP_H
#define MIRACLE_HIP_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define MR_API __attribute__((visibility("default")))
#else
#define MR_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
enum {
    MR_OK = 0,
    MR_ERR_INVALID = 1,     /* bad argument or shape (reference: ValueError)            */
    MR_ERR_HIP = 2,         /* HIP runtime failure   (reference: OpenCLError)           */
    MR_ERR_NOMEM = 3,       /* allocation failed or above the device limit              */
    MR_ERR_STATE = 4,       /* model not finalized / weights missing                    */
    MR_ERR_NONFINITE = 5,   /* non-finite logits during device-side greedy generation   */
    MR_ERR_INJECTED = 6,    /* failure injected by mr_debug_fail_next (tests only)      */
    MR_ERR_TIMEOUT = 7      /* a persistent step's wait for another workgroup timed out */
};

/* Storage dtype of a weight tensor.  BF16/F16 stay in their stored bits in HBM
 * and are widened to FP32 in registers (reference widens on the host,
 * weights.py:64-74). */
enum { MR_F32 = 0, MR_BF16 = 1, MR_F16 = 2 };

/* Message for the last failing call on this thread. */
MR_API const char *mr_last_error(void);

/* ---- devices (reference: opencl.py:84-115 list_devices / Device) ------- */
typedef struct mr_device_info {
    char name[256];
    char arch[64];              /* e.g. "gfx950:sramecc+:xnack-" */
    int64_t memory_bytes;       /* reference Device.memory_bytes          */
    int64_t max_allocation_bytes; /* reference Device.max_allocation_bytes */
    int32_t compute_units;
    int32_t pci_bus_id;
    int32_t clock_khz;
    int32_t memory_clock_khz;
    int32_t memory_bus_width;
    int32_t reserved;
} mr_device_info;

MR_API int mr_device_count(int *count);
MR_API int mr_device_get_info(int device, mr_device_info *out);

/* ---- context (reference: OpenCLBackend.__init__/__del__/finish,
 *      opencl.py:136-176, 302-303) ------------------------------------- */
typedef struct mr_ctx mr_ctx;
MR_API int mr_ctx_create(int device, mr_ctx **out);
/* Drops the caller's reference.  Each model created on the context holds one
 * more, so the stream and the context's blocks are released when the last of
 * the context and its models is destroyed, in whichever order they go. */
MR_API int mr_ctx_destroy(mr_ctx *ctx);
MR_API int mr_sync(mr_ctx *ctx);

/* ---- memory (reference: OpenCLBackend.empty/upload/read/copy,
 *      opencl.py:178-217; Tensor.__del__ opencl.py:123-126) ------------- */
MR_API int mr_alloc(mr_ctx *ctx, size_t bytes, void **device_ptr);
MR_API int mr_free(mr_ctx *ctx, void *device_ptr);
MR_API int mr_h2d(mr_ctx *ctx, void *device_dst, const void *host_src, size_t bytes);  /* blocking */
MR_API int mr_d2h(mr_ctx *ctx, void *host_dst, const void *device_src, size_t bytes);  /* blocking */
MR_API int mr_d2d(mr_ctx *ctx, void *device_dst, const void *device_src, size_t bytes); /* enqueued */

/* ---- op-level kernels: one per reference kernel (kernels.cl), argument
 *      lists as the reference enqueues them, plus a weight dtype tag.
 *      All are enqueued on the context stream. ------------------------------ */
/* kernels.cl:5-17  (opencl.py:241-247 linear): y[rows,out] = x[rows,in] . w[out,in]^T */
MR_API int mr_linear(mr_ctx *ctx, const float *x, const void *w, int w_dtype, float *y, int rows, int out_dim,
              int in_dim);
/* kernels.cl:19-28 (opencl.py:249-255 norm): w == NULL means non-affine */
MR_API int mr_rms(mr_ctx *ctx, const float *x, const float *w, float *y, int rows, int width, float eps);
/* kernels.cl:30-44 (opencl.py:257-263 rotate) */
MR_API int mr_rope(mr_ctx *ctx, const float *x, const float *freq, const float *pos, float *y, int rows, int heads,
            int dim, int split_half);
/* kernels.cl:46-50 (opencl.py:272-277 swiglu) */
MR_API int mr_swiglu(mr_ctx *ctx, const float *g, const float *u, float *y, int n);
/* kernels.cl:52-56 (opencl.py:265-270 add): z = x + scale*y */
MR_API int mr_axpy(mr_ctx *ctx, const float *x, const float *y, float *z, int n, float scale);
/* kernels.cl:58-73 (scores, run by name at model.py:164, 215) */
MR_API int mr_scores(mr_ctx *ctx, const float *q, const float *k, const float *extra_k, float *s, int heads,
              int kv_heads, int dim, int capacity, int start, int length, int extra_length);
/* kernels.cl:75-84 (opencl.py:279-282 softmax) */
MR_API int mr_softmax(mr_ctx *ctx, const float *x, float *y, int rows, int width);
/* kernels.cl:86-91 (latent_mask, model.py:166) */
MR_API int mr_latent_mask(mr_ctx *ctx, float *scores, const float *positions, int heads, int length, int memory,
                   int earliest);
/* kernels.cl:93-107 (opencl.py:294-300 mix) */
MR_API int mr_mix(mr_ctx *ctx, const float *p, const float *v, const float *extra_v, float *y, int heads, int kv_heads,
           int dim, int capacity, int start, int length, int extra_length);
/* kernels.cl:110-117 (pool_scores, model.py:129) */
MR_API int mr_pool_scores(mr_ctx *ctx, const float *u, const float *q, float *s, int tokens, int slots, int width);
/* kernels.cl:119-130 (pool_mix, model.py:133) */
MR_API int mr_pool_mix(mr_ctx *ctx, const float *u, const float *p, float *z, float *anchors, int tokens, int slots,
                int width, int start_position);
/* kernels.cl:133-137 (merge_rows, model.py:180) */
MR_API int mr_merge_rows(mr_ctx *ctx, const float *x, float *y, int width, float a, float b);
/* kernels.cl:140-148 (block_means, model.py:213) */
MR_API int mr_block_means(mr_ctx *ctx, const float *x, float *y, int length, int width, int block);
/* opencl.py:284-292 attention = scores -> softmax -> mix, fused (one pass,
 * split over keys, online softmax). */
MR_API int mr_attention(mr_ctx *ctx, const float *q, const float *k, const float *v, const float *extra_k,
                 const float *extra_v, float *y, int heads, int kv_heads, int dim, int capacity, int start,
                 int length, int extra_length);
/* No counterpart in the reference.  mr_attention for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation): same arguments, kernels and results, but the split
 * partials and merge counters live in a static 8 MiB device array per GPU
 * (held until the process ends) instead of a context allocation, and the
 * counters are cleared by a kernel, not a memset.  A call needing more scratch
 * than 8 MiB (kv_heads * splits * (heads / kv_heads) * (dim + 2) floats,
 * splits <= 512 / kv_heads, plus kv_heads counters) fails with MR_ERR_INVALID.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other contexts, other threads) race. */
MR_API int mr_attention_noalloc(mr_ctx *ctx, const float *q, const float *k, const float *v, const float *extra_k,
                                const float *extra_v, float *y, int heads, int kv_heads, int dim, int capacity,
                                int start, int length, int extra_length);

/* ---- step-level engine: the whole of MiracleModel._step and the LM head
 *      (model.py:257-285, 303-308) for one sequence, device-resident. ------- */
enum {
    MR_FAMILY_FLASHNANO_15 = 0, MR_FAMILY_FLASHNANO_16 = 1, MR_FAMILY_FLASHNANO_17 = 2,
    MR_FAMILY_FLASHLITE_20 = 3, MR_FAMILY_FLASHLIGHTING_20 = 4, MR_FAMILY_HEAVY_MEDIUM_20 = 5
};

/* Geometry of one model (reference: ModelConfig, config.py:13-39). */
typedef struct mr_model_desc {
    int32_t family;
    int32_t vocab_size, hidden_size, layers, query_heads, kv_heads, global_kv_heads, head_dim, ffn_dim;
    int32_t context_length;     /* cache capacity bound (model.py:46-49)                 */
    int32_t window;             /* 0 = no window                                          */
    int32_t tie_embeddings, qk_norm, split_half_rope;
    int32_t latent_dim, memory_slots, cbr_chunk_size, cbr_slots, inner_loop_steps;
    float norm_eps, cbr_norm_eps, residual_scale;
    /* heavy-medium-2.0 (source fields, model.py:192-255) */
    int32_t routed_experts, router_groups, router_top_k_min, router_top_k_max, shared_experts;
    int32_t global_block_size, global_slots;
    float router_temperature, alibi_slope_scale;
    uint64_t global_layer_mask_lo, global_layer_mask_hi;   /* bit i = layer i is global (i < 128) */
    /* heavy-medium-2.0 scales, each computed by the host in double precision from
     * the config's floats and rounded to FP32 once, as the reference's host code
     * does before its kernel calls: residual_scale / sqrt(inner_loop_steps)
     * (model.py:262), residual_scale / shared_experts (model.py:255) and
     * alibi_slope_scale / sqrt(head_dim) (model.py:218). */
    float heavy_step_scale, heavy_shared_scale, block_slope, reserved0;
} mr_model_desc;

/* Weight kinds (canonical names of weights.py:211-245). */
enum {
    MR_W_EMBED = 0, MR_W_OUTPUT, MR_W_NORM,
    MR_W_A_NORM, MR_W_F_NORM, MR_W_Q, MR_W_K, MR_W_V, MR_W_O, MR_W_Q_NORM, MR_W_K_NORM,
    MR_W_GATE, MR_W_UP, MR_W_DOWN,
    MR_W_LATENT, MR_W_LATENT_NORM, MR_W_KV_UP, MR_W_ATTENTION_GATE, MR_W_FFN_GATE, MR_W_CBR,
    MR_W_ROUTER_COARSE, MR_W_ROUTER_COARSE_BIAS, MR_W_ROUTER_FINE, MR_W_ROUTER_FINE_BIAS,
    MR_W_ROUTER_GROUP_BIAS, MR_W_ROUTER_EXPERT_BIAS,
    MR_W_SHARED_GATE, MR_W_SHARED_UP, MR_W_SHARED_DOWN,
    MR_W_COUNT
};

typedef struct mr_model mr_model;

/* Reference: MiracleModel.__init__ (model.py:43-56). */
MR_API int mr_model_create(mr_ctx *ctx, const mr_model_desc *desc, mr_model **out);
MR_API int mr_model_destroy(mr_model *model);
/* Copies one host tensor into the model's HBM layout.  `layer` is -1 for model-
 * level tensors; `expert` indexes routed/shared experts (else -1).  1-D tensors
 * must be MR_F32.  (Reference: WeightCache.tensor, weights.py:266-280.) */
MR_API int mr_model_set_weight(mr_model *model, int kind, int layer, int expert, const void *host, int dtype,
                        int64_t rows, int64_t cols);
/* float32[head_dim/2] RoPE inverse frequencies (reference: model.py:55). */
MR_API int mr_model_set_rope(mr_model *model, const float *inv_freq, int count);
/* Checks every weight is present and allocates sequence state. */
MR_API int mr_model_finalize(mr_model *model);
/* Reference: MiracleModel.reset (model.py:74-77). */
MR_API int mr_model_reset(mr_model *model);
MR_API int mr_model_position(mr_model *model, int *position);

/* Append n tokens to the sequence (reference: prefill, model.py:295-312).
 * flags: MR_FWD_RETURN_ALL -> logits for every token ([n, vocab]); otherwise
 * only for the last token ([vocab]).  MR_FWD_BATCHED -> batched prefill for
 * every family: each layer runs once per chunk of up to 4096 prompt rows
 * (projections as MFMA GEMMs with FP32-faithful products, windowed attention
 * over the chunk plus the caches; flashnano-1.6's relay rows pooled for every
 * CBR chunk that ends in the chunk; the latent memory's compaction planned per
 * position; block sums scanned per row and blocks chosen per row as the token
 * step chooses them; experts as grouped GEMMs); results agree with the token
 * loop to FP32 rounding, not bit for bit.  A single token and geometries
 * outside the kernels' widths take the token loop.
 * logits may be NULL (no readback; the last token's logits stay on device). */
enum { MR_FWD_RETURN_ALL = 1, MR_FWD_BATCHED = 2 };
MR_API int mr_model_forward(mr_model *model, const int32_t *ids, int n, int flags, float *logits);

/* Greedy continuation on device (reference: generate with temperature 0,
 * model.py:338-356): starting from the argmax of the logits of the last
 * forward, emit up to max_new tokens, stopping after `eos` (eos < 0: never).
 * Only token ids cross to the host.  Returns MR_ERR_NONFINITE if a step's
 * logits were not all finite (tokens before it are still written). */
MR_API int mr_model_generate_greedy(mr_model *model, int max_new, int eos, int32_t *tokens, int *produced);

/* How a token step runs.  MR_STEP_PERSISTENT (default): one kernel launch per
 * step walks the whole layer stack, one workgroup per CU (used when every
 * phase fits it; otherwise the model runs MR_STEP_GRAPH).  Its workgroups wait
 * on each other's results, so they must all be resident at once: a plain
 * launch whose grid equals the CU count and whose registers fill a CU places
 * one on every CU when the GPU is otherwise idle.  If other work holds CUs and
 * a wait times out, the step fails with MR_ERR_TIMEOUT and the model switches to
 * MR_STEP_GRAPH at the next mr_model_reset (mr_model_get_step_mode reports it).
 * MR_STEP_GRAPH: five fused kernels per layer, replayed from a captured
 * hipGraph.  MR_STEP_EAGER: the same kernels launched one by one (for
 * profilers). */
enum { MR_STEP_PERSISTENT = 0, MR_STEP_GRAPH = 1, MR_STEP_EAGER = 2 };
MR_API int mr_model_set_step_mode(mr_model *model, int mode);
/* The mode steps actually run in (a persistent request may fall back). */
MR_API int mr_model_get_step_mode(mr_model *model, int *mode);
/* Routing decisions of every position so far (heavy-medium-2.0): per position,
 * layer and inner loop one record of 1 + router_top_k_max + query_heads *
 * global_slots ints: the adaptive width, the chosen experts in descending
 * probability (-1 past the width), then per query head the chosen global blocks
 * in ascending order (-1 padded).  The reference makes these choices on the host
 * (model.py:220-249); no reference function returns them, they are what its
 * trace records for parity checks.  *per_position receives the ints per
 * position. */
MR_API int mr_model_choices(mr_model *model, int32_t *out, int64_t capacity, int *per_position);

/* Phase timeline of the persistent step kernel (diagnostics; no counterpart in
 * the reference).  Runs one greedy decode step at the current position with
 * timestamps (100 MHz device wall clock) written per phase and workgroup:
 * out[(phase * grid + wg) * 5 + {0: phase entry, 1: input staged, 2: outputs
 * stored by the last stream wave, 3: by the first stream wave, 4: unused}]
 * (0 where not stamped); in attention phases 1 is the unit's Q/K/V cells
 * staged, 2 the workgroup's end of the phase, 3 the unit's partial stored and
 * 4 a merging unit's first partial cells seen.
 * `capacity` is the number of uint64 in `out`; *phases and *grid receive the
 * program size.  The step advances the sequence like any decode step. */
MR_API int mr_model_trace_step(mr_model *model, uint64_t *out, int64_t capacity, int *phases, int *grid);

/* Device milliseconds of the last mr_model_generate_greedy call (HIP events
 * around its decode steps). */
MR_API int mr_model_last_decode_ms(mr_model *model, float *ms);

/* Measurement: average device time of one launch of a step kernel, taken with
 * HIP events on the context stream.  `which` is an MR_KERNEL_* id; the kernel is
 * launched for every layer in turn (so a repeat never finds the previous
 * layer's weights in cache), `reps` times over, at the current position.  The
 * position and every cached key/value row the next step reads are left as they
 * were; the scratch activations and the last logits are not (call
 * mr_model_forward again before mr_model_generate_greedy).  No counterpart in
 * the reference (it has no timers); used by bench.py. */
enum { MR_KERNEL_QKV = 0, MR_KERNEL_ATTENTION = 1, MR_KERNEL_O = 2, MR_KERNEL_GATE_UP = 3, MR_KERNEL_DOWN = 4,
       MR_KERNEL_HEAD = 5 };
MR_API int mr_model_time_kernel(mr_model *model, int which, int reps, float *avg_ms);

/* Test hook: make the next model call on this context fail with
 * MR_ERR_INJECTED (the reference's failed-device-operation path,
 * model.py:298-311).  Not a counterpart of any reference function. */
MR_API int mr_debug_fail_next(mr_ctx *ctx);

/* Test hook: the status check after the model's next persistent step reports
 * MR_ERR_TIMEOUT as if a wait had given up (the host-side half of the
 * timeout path: the error, the poisoned model, the switch to MR_STEP_GRAPH at
 * reset).  No kernel is made to wait.  Not a counterpart of any reference
 * function. */
MR_API int mr_debug_step_timeout(mr_model *model);

/* Test hook: c[m, n] = a[m, k] . w[n, k]^T (device FP32 a and c, device BF16
 * w) through the batched-prefill MFMA GEMM in the BF16-term scheme
 * (scheme 0) or the FP16-term scheme (scheme 1, with the matrix's FP16 scale
 * computed here; `ascale` is a device workspace of m floats).  Synchronizes.
 * k must be a multiple of 8.  Not a counterpart of any reference function. */
MR_API int mr_debug_gemm(mr_ctx *ctx, const float *a, const void *w, float *c, float *ascale, int m, int n, int k,
                         int scheme);

/* Test hook: the batched prefill's grouped (expert) MFMA GEMM in the FP16-term
 * scheme.  Group z holds counts[z] (host, >= 0) consecutive rows of a
 * [rows, k] (device FP32, groups in order, rows = the sum of counts) and its
 * own weights, rows z n .. z n + n - 1 of w (device BF16 [groups, n, k]);
 * c [rows, n] receives a . w_z^T for each group's rows, or with swiglu the
 * SwiGLU of the gate (w) and up (w2, same layout) products (a group's gate
 * and up copies share one FP16 scale, as the model's do).  tile_list 1 runs
 * the kernel over the groups' own 128-row tiles (the prefix sums the prefill
 * takes from its routing), 0 the grid of max(counts) rows in every group.
 * Synchronizes; k must be a multiple of 8.  Not a counterpart of any
 * reference function. */
MR_API int mr_debug_gemm_grouped(mr_ctx *ctx, const float *a, const void *w, const void *w2, float *c,
                                 const int *counts, int groups, int n, int k, int swiglu, int tile_list);

/* Test hook: the batched-prefill attention over device FP32 buffers.  qkv
 * [rows, heads*d + 2*kv_heads*d] holds each row's (normalized, rotated)
 * query, key and value at positions p0 .. p0 + rows - 1; ring_k/ring_v
 * [cap, kv_heads*d] hold the keys and values of positions p < p0 at slot
 * p % cap; out [rows, heads*d] receives softmax(q.k / sqrt(d)).v over the
 * keys at positions max(0, p - window + 1) .. p (window 0: cap).  presplit
 * 1 splits the attended keys and values into FP16 terms once beforehand
 * (workspace allocated here), 0 lets every workgroup split its tiles.
 * Synchronizes.  Not a counterpart of any reference function. */
MR_API int mr_debug_prefill_attention(mr_ctx *ctx, const float *qkv, const float *ring_k, const float *ring_v,
                                      float *out, int rows, int p0, int heads, int kv_heads, int d, int cap,
                                      int window, int presplit);

/* Test hook: y[i] = 2^x[i] by the hardware exp2 the batched prefill's
 * softmax uses (which 0; log2 e is folded into its score scale), or
 * y[i] = e^x[i] by the expf of the token step's softmax (which 1), for device
 * x and y of n floats.  Synchronizes.  Not a counterpart of any reference
 * function. */
MR_API int mr_debug_exp(mr_ctx *ctx, const float *x, float *y, int n, int which);

#ifdef __cplusplus
}
#endif
#endif /* MIRACLE_HIP_H */
