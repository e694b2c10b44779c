// Step-level engine: MiracleModel._step + LM head (model.py:257-308) for one
// sequence, with weights and caches resident in HBM.
//
// One token step of a GQA family (flashnano-1.5/1.6/1.7, flashlite-2.0) is five
// fused kernels per layer:
//   1. RMSNorm(hidden, a_norm) -> [Wq;Wk;Wv] GEMV           (model.py:281, 98-99)
//   2. Q/K RMSNorm + RoPE + ring write + split-key attention (model.py:100-113)
//   3. Wo GEMV + residual                                    (model.py:116, 282)
//   4. RMSNorm(hidden, f_norm) -> gate/up GEMV + SwiGLU      (model.py:87-89, 283)
//   5. Wdown GEMV + residual                                 (model.py:283)
// plus, for flashnano-1.6, the chunk-end CBR pooling into the relay
// (model.py:118-144).  The position, the token ids and the greedy-loop state
// live in device memory, so one step is a fixed launch sequence that is
// captured once in a hipGraph and replayed for every token.
#include <cmath>
#include <cstring>
#include <initializer_list>

#include "engine.h"

using namespace mr;

namespace mr {
namespace {

bool is_gqa(int family) {
    return family == MR_FAMILY_FLASHNANO_15 || family == MR_FAMILY_FLASHNANO_16 ||
           family == MR_FAMILY_FLASHNANO_17 || family == MR_FAMILY_FLASHLITE_20;
}

// Families whose prompt can run as whole-chunk kernels: the GQA families
// (flashnano-1.6 with the relay rows of every CBR chunk that ends inside the
// prompt chunk built before its attention), heavy-medium-2.0, whose block sums
// and block choices are rebuilt per row from a scan of the chunk, and
// flashlighting-2.0, whose latent memory is planned per step.
bool batched_prefill_family(int family) {
    return is_gqa(family) || family == MR_FAMILY_HEAVY_MEDIUM_20 || family == MR_FAMILY_FLASHLIGHTING_20;
}

int dtype_bytes(int dt) { return dt == MR_F32 ? 4 : 2; }

__device__ __forceinline__ float widen_any(const void *p, int dt, int64_t i) {
    if (dt == MR_F32) return ((const float *)p)[i];
    uint32_t b = ((const uint16_t *)p)[i];
    return dt == MR_BF16 ? bf16_to_f32(b) : f16_to_f32(b);
}

// hidden = embed[ids[pos]] widened (model.py:259).
__global__ void k_embed(const void *table, int dt, const int *ids, const int *pos, const int *done, float *hidden,
                        int h) {
    if (*done) return;
    int tok = ids[*pos];
    for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < h; j += gridDim.x * blockDim.x)
        hidden[j] = widen_any(table, dt, (int64_t)tok * h + j);
}

__global__ void k_advance(int *pos, const int *done) {
    if (!*done) *pos += 1;
}

// Greedy token choice over logits (np.argmax: first maximum), the finiteness
// check of model.py:339-342, then optional position advance, token append and
// EOS stop.
__global__ void __launch_bounds__(1024) k_argmax(const float *logits, int n, int *pos, int *done, int *ids,
                                                 int *gen, int *count, const int *eos, int advance) {
    __shared__ float bv[1024];
    __shared__ int bi[1024];
    __shared__ int bad;
    if (*done) return;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    float best = -INFINITY;
    int idx = n;
    bool nonfinite = false;
    auto consider = [&](float v, int i) {
        if (!isfinite(v)) nonfinite = true;
        if (v > best || (v == best && i < idx)) {
            best = v;
            idx = i;
        }
    };
    // 16-byte loads, eight per thread issued together before any compare (a
    // load at a time made the pass 31 dependent round trips); the choice is
    // the largest value, lowest index among equals, in any visiting order.
    constexpr int U = 8;
    const int n4 = ((uintptr_t)logits & 15) == 0 ? n / 4 : 0;
    for (int base = threadIdx.x; base < n4; base += blockDim.x * U) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i4 = base + u * (int)blockDim.x;
            v[u] = i4 < n4 ? *(const float4 *)(logits + 4 * i4) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i4 = base + u * (int)blockDim.x;
            if (i4 < n4) {
                consider(v[u].x, 4 * i4);
                consider(v[u].y, 4 * i4 + 1);
                consider(v[u].z, 4 * i4 + 2);
                consider(v[u].w, 4 * i4 + 3);
            }
        }
    }
    for (int i = 4 * n4 + threadIdx.x; i < n; i += blockDim.x) consider(logits[i], i);
    if (nonfinite) atomicOr(&bad, 1);
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = idx;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            float ov = bv[threadIdx.x + s];
            int oi = bi[threadIdx.x + s];
            if (ov > bv[threadIdx.x] || (ov == bv[threadIdx.x] && oi < bi[threadIdx.x])) {
                bv[threadIdx.x] = ov;
                bi[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        int p = *pos;
        if (advance) *pos = ++p;
        if (bad) {
            *done = 2;
            return;
        }
        int tok = bi[0];
        ids[p] = tok;
        gen[*count] = tok;
        *count += 1;
        if (tok == *eos) *done = 1;
    }
}

// ---- flashnano-1.6 CBR (model.py:118-144) -----------------------------------
// Pools one chunk (row(t), t < chunk, at positions start_position + t) into one
// slot with its learned query q: scores u . q / sqrt(h), softmax over the
// chunk, the probability-weighted row and the rounded probability-weighted
// position as its anchor (kernels.cl:110-130).  sp holds chunk + 8 floats.
template <typename RowFn>
__device__ void cbr_pool_slot(RowFn row, const float *q, int chunk, int h, int start_position, float *sp,
                              float *pooled, float *anchor) {
    float *red = sp + chunk;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int t = wave; t < chunk; t += blockDim.x / 64) {
        const float *u = row(t);
        float acc = 0.0f;
        for (int j = lane; j < h; j += 64) acc = fmaf(u[j], q[j], acc);
        acc = wave_sum(acc);
        if (lane == 0) sp[t] = acc / sqrtf((float)h);
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int t = threadIdx.x; t < chunk; t += blockDim.x) mx = fmaxf(mx, sp[t]);
    mx = block_max(mx, red);
    float den = 0.0f;
    for (int t = threadIdx.x; t < chunk; t += blockDim.x) den += expf(sp[t] - mx);
    den = block_sum(den, red);
    __syncthreads();
    for (int t = threadIdx.x; t < chunk; t += blockDim.x) sp[t] = expf(sp[t] - mx) / den;
    __syncthreads();
    for (int j = threadIdx.x; j < h; j += blockDim.x) {
        float v = 0.0f;
        for (int t = 0; t < chunk; ++t) v = fmaf(sp[t], row(t)[j], v);
        pooled[j] = v;
    }
    if (threadIdx.x == 0) {
        float ps = 0.0f;
        for (int t = 0; t < chunk; ++t) ps = fmaf(sp[t], (float)(start_position + t), ps);
        *anchor = rintf(ps);
    }
}

// Token step: stores this step's normalized input in the pending chunk; at a
// chunk end pools it into `slots` rows.  Block m pools slot m.
__global__ void __launch_bounds__(256) k_cbr_pool(const float *xnorm, float *pending, const float *queries,
                                                  float *pooled, float *anchors, int *skip_flag, const int *pos_p,
                                                  const int *done, int chunk, int h) {
    extern __shared__ float sp[];   // [chunk] probabilities, then reduction scratch
    const int pos = *pos_p;
    const bool skip = *done || (pos % chunk != chunk - 1);
    if (blockIdx.x == 0) {
        if (threadIdx.x == 0) *skip_flag = skip ? 1 : 0;
        if (!*done)
            for (int j = threadIdx.x; j < h; j += blockDim.x) pending[(int64_t)(pos % chunk) * h + j] = xnorm[j];
    }
    if (skip) return;
    const int m = blockIdx.x;
    auto row = [&](int t) -> const float * { return t == chunk - 1 ? xnorm : pending + (int64_t)t * h; };
    cbr_pool_slot(row, queries + (int64_t)m * h, chunk, h, pos + 1 - chunk, sp, pooled + (int64_t)m * h,
                  anchors + m);
}

// Batched prefill, CBR pooling of the chunks first_chunk .. first_chunk + nc - 1
// (all ending inside the prompt rows at positions p0 ..): the row of position
// p is pending row p % chunk before p0, row p - p0 of xn after.
__device__ __forceinline__ const float *cbr_row(const float *xn, int ldx, const float *pending, int p0, int chunk,
                                                int h, int p) {
    return p < p0 ? pending + (int64_t)(p % chunk) * h : xn + (int64_t)(p - p0) * ldx;
}

// Pooling step 1, one block per row of the chunks: its scores against the
// learned queries, scores[(c * slots + m) * chunk + t] = u . q_m / sqrt(h),
// each summed as the token step sums it.
__global__ void __launch_bounds__(256) k_cbr_scores_rows(const float *xn, int ldx, const float *pending,
                                                         const float *queries, float *scores, int p0,
                                                         int first_chunk, int chunk, int slots, int h) {
    const int c = blockIdx.x / chunk, t = blockIdx.x % chunk;
    const float *u = cbr_row(xn, ldx, pending, p0, chunk, h, (first_chunk + c) * chunk + t);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int m = wave; m < slots; m += blockDim.x / 64) {
        const float *q = queries + (int64_t)m * h;
        float acc = 0.0f;
        for (int j = lane; j < h; j += 64) acc = fmaf(u[j], q[j], acc);
        acc = wave_sum(acc);
        if (lane == 0) scores[((int64_t)c * slots + m) * chunk + t] = acc / sqrtf((float)h);
    }
}

// Pooling step 2, block (c, m, b): the softmax of chunk c's scores for slot m
// (as the token step forms it), then columns 256 b .. 256 b + 255 of pooled
// row c * slots + m; column block 0 also writes its anchor.
__global__ void __launch_bounds__(256) k_cbr_mix_rows(const float *xn, int ldx, const float *pending,
                                                      const float *scores, float *pooled, float *anchors, int p0,
                                                      int first_chunk, int chunk, int slots, int h) {
    extern __shared__ float sp[];   // [chunk] probabilities, then reduction scratch
    float *red = sp + chunk;
    const int c = blockIdx.x, r = c * slots + blockIdx.y, start = (first_chunk + c) * chunk;
    const float *s = scores + (int64_t)r * chunk;
    float mx = -INFINITY;
    for (int t = threadIdx.x; t < chunk; t += blockDim.x) mx = fmaxf(mx, s[t]);
    mx = block_max(mx, red);
    float den = 0.0f;
    for (int t = threadIdx.x; t < chunk; t += blockDim.x) den += expf(s[t] - mx);
    den = block_sum(den, red);
    for (int t = threadIdx.x; t < chunk; t += blockDim.x) sp[t] = expf(s[t] - mx) / den;
    __syncthreads();
    const int j = blockIdx.z * blockDim.x + threadIdx.x;
    if (j < h) {
        float v = 0.0f;
        for (int t = 0; t < chunk; ++t) v = fmaf(sp[t], cbr_row(xn, ldx, pending, p0, chunk, h, start + t)[j], v);
        pooled[(int64_t)r * h + j] = v;
    }
    if (blockIdx.z == 0 && threadIdx.x == 0) {
        float ps = 0.0f;
        for (int t = 0; t < chunk; ++t) ps = fmaf(sp[t], (float)(start + t), ps);
        anchors[r] = rintf(ps);
    }
}

// Batched prefill: the pending buffer as the token loop leaves it after the
// rows at positions p0 .. p0 + rows - 1 (row position % chunk holds the
// latest position of that residue); block b stores row rows - gridDim.x + b.
__global__ void __launch_bounds__(256) k_cbr_pending_rows(const float *xn, int ldx, float *pending, int p0, int rows,
                                                          int chunk, int h) {
    const int t = rows - gridDim.x + blockIdx.x;
    const float *src = xn + (int64_t)t * ldx;
    float *dst = pending + (int64_t)((p0 + t) % chunk) * h;
    for (int j = threadIdx.x; j < h; j += blockDim.x) dst[j] = src[j];
}

// Pooled rows through Wk and Wv (model.py:135): one wave per output value.
__global__ void __launch_bounds__(256) k_cbr_project(const float *pooled, const void *wkv, int dt, float *out,
                                                     const int *skip_flag, int kvw2, int h) {
    if (*skip_flag) return;
    const int m = blockIdx.y, lane = threadIdx.x & 63;
    const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (o >= kvw2) return;
    const float *x = pooled + (int64_t)m * h;
    float acc = 0.0f;
    for (int j = lane; j < h; j += 64) acc = fmaf(widen_any(wkv, dt, (int64_t)o * h + j), x[j], acc);
    acc = wave_sum(acc);
    if (lane == 0) out[(int64_t)m * kvw2 + o] = acc;
}

// K-norm + RoPE at the pooled anchor of one pooled [K | V] row, then its relay
// row dst (model.py:136-144).  kr holds kv_heads * d floats.
__device__ void cbr_finish_row(const float *src, float anchor, const float *k_gain, float eps, const float *rope,
                               int split_half, float *relay_k, float *relay_v, int64_t dst, int kv_heads, int d,
                               float *kr) {
    const int kvw = kv_heads * d;
    for (int j = threadIdx.x; j < kvw; j += blockDim.x) kr[j] = src[j];
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int hh = wave; hh < kv_heads; hh += blockDim.x / 64) {
        float *row = kr + hh * d;
        float ss = 0.0f;
        for (int j = lane; j < d; j += 64) ss = fmaf(row[j], row[j], ss);
        ss = wave_sum(ss);
        float scale = 1.0f / sqrtf(ss / (float)d + eps);
        for (int j = lane; j < d; j += 64) row[j] = row[j] * scale * k_gain[j];
    }
    __syncthreads();
    const int half = d / 2;
    // anchors are rounded positions inside the chunk, so they index the table
    const float *cs = rope + (int64_t)anchor * half * 2;
    for (int i = threadIdx.x; i < kv_heads * half; i += blockDim.x) {
        int hh = i / half, p = i % half;
        float *row = kr + hh * d;
        int j = split_half ? p : 2 * p, k = split_half ? p + half : 2 * p + 1;
        float u = row[j], v = row[k];
        rope_rotate(u, v, cs[2 * p], cs[2 * p + 1]);
        row[j] = u;
        row[k] = v;
    }
    __syncthreads();
    for (int j = threadIdx.x; j < kvw; j += blockDim.x) {
        relay_k[dst * kvw + j] = kr[j];
        relay_v[dst * kvw + j] = src[kvw + j];
    }
}

// Token step: block m finishes slot m of the chunk that ends at this position.
__global__ void __launch_bounds__(256) k_cbr_finish(const float *kv, const float *anchors, const float *k_gain,
                                                    float eps, const float *rope, int split_half, float *relay_k,
                                                    float *relay_v, const int *skip_flag, const int *pos_p,
                                                    int chunk, int slots, int kv_heads, int d) {
    extern __shared__ float kr[];
    if (*skip_flag) return;
    const int m = blockIdx.x;
    cbr_finish_row(kv + (int64_t)m * 2 * kv_heads * d, anchors[m], k_gain, eps, rope, split_half, relay_k, relay_v,
                   (int64_t)(*pos_p / chunk) * slots + m, kv_heads, d, kr);
}

// Batched prefill: block r finishes pooled row r (relay row first_chunk * slots + r).
__global__ void __launch_bounds__(256) k_cbr_finish_rows(const float *kv, const float *anchors, const float *k_gain,
                                                         float eps, const float *rope, int split_half, float *relay_k,
                                                         float *relay_v, int first_chunk, int slots, int kv_heads,
                                                         int d) {
    extern __shared__ float kr[];
    const int r = blockIdx.x;
    cbr_finish_row(kv + (int64_t)r * 2 * kv_heads * d, anchors[r], k_gain, eps, rope, split_half, relay_k, relay_v,
                   (int64_t)first_chunk * slots + r, kv_heads, d, kr);
}

// Non-affine RMSNorm of the learned CBR queries, once per model (model.py:126-127).
__global__ void __launch_bounds__(256) k_rows_rms(const void *x, int dt, float *y, int width, float eps) {
    __shared__ float red[4];
    const int64_t base = (int64_t)blockIdx.x * width;
    float ss = 0.0f;
    for (int j = threadIdx.x; j < width; j += blockDim.x) {
        float v = widen_any(x, dt, base + j);
        ss = fmaf(v, v, ss);
    }
    ss = block_sum(ss, red);
    float scale = 1.0f / sqrtf(ss / (float)width + eps);
    for (int j = threadIdx.x; j < width; j += blockDim.x) y[base + j] = widen_any(x, dt, base + j) * scale;
}

// ------------------------------------------------------------------ host helpers
int device_alloc(mr_model *m, size_t bytes, void **p) {
    MR_HIP(hipMalloc(p, bytes ? bytes : 16), "allocate model buffer");
    (void)m;
    return MR_OK;
}

struct Expect {
    int64_t rows, cols;
};

int expected_shape(const mr_model *m, int kind, int layer, Expect *e) {
    const mr_model_desc &d = m->d;
    const int h = d.hidden_size, hd = d.head_dim, qd = d.query_heads * d.head_dim;
    int kvh = layer >= 0 ? m->layers[layer].kv_heads : d.kv_heads;
    int kvw = kvh * hd;
    int inner = d.latent_dim ? d.latent_dim : h;
    switch (kind) {
        case MR_W_EMBED: case MR_W_OUTPUT: *e = {d.vocab_size, h}; return MR_OK;
        case MR_W_NORM: case MR_W_A_NORM: case MR_W_F_NORM: *e = {h, 1}; return MR_OK;
        case MR_W_Q: *e = {qd, h}; return MR_OK;
        case MR_W_K: case MR_W_V: *e = {kvw, inner}; return MR_OK;
        case MR_W_O: *e = {h, qd}; return MR_OK;
        case MR_W_Q_NORM: case MR_W_K_NORM: *e = {hd, 1}; return MR_OK;
        case MR_W_GATE: case MR_W_UP: case MR_W_SHARED_GATE: case MR_W_SHARED_UP: *e = {d.ffn_dim, h}; return MR_OK;
        case MR_W_DOWN: case MR_W_SHARED_DOWN: *e = {h, d.ffn_dim}; return MR_OK;
        case MR_W_LATENT: *e = {d.latent_dim, h}; return MR_OK;
        case MR_W_LATENT_NORM: *e = {d.latent_dim, 1}; return MR_OK;
        case MR_W_KV_UP: *e = {2 * kvw, d.latent_dim}; return MR_OK;
        case MR_W_ATTENTION_GATE: case MR_W_FFN_GATE: *e = {1, 1}; return MR_OK;
        case MR_W_CBR: *e = {d.cbr_slots, h}; return MR_OK;
        case MR_W_ROUTER_COARSE: *e = {d.router_groups, h}; return MR_OK;
        case MR_W_ROUTER_FINE: *e = {d.routed_experts, h}; return MR_OK;
        case MR_W_ROUTER_COARSE_BIAS: case MR_W_ROUTER_GROUP_BIAS: *e = {d.router_groups, 1}; return MR_OK;
        case MR_W_ROUTER_FINE_BIAS: case MR_W_ROUTER_EXPERT_BIAS: *e = {d.routed_experts, 1}; return MR_OK;
    }
    return fail(MR_ERR_INVALID, "unknown weight kind " + std::to_string(kind));
}

bool is_vector_kind(int kind) {
    switch (kind) {
        case MR_W_NORM: case MR_W_A_NORM: case MR_W_F_NORM: case MR_W_Q_NORM: case MR_W_K_NORM:
        case MR_W_LATENT_NORM: case MR_W_ATTENTION_GATE: case MR_W_FFN_GATE: case MR_W_ROUTER_COARSE_BIAS:
        case MR_W_ROUTER_FINE_BIAS: case MR_W_ROUTER_GROUP_BIAS: case MR_W_ROUTER_EXPERT_BIAS:
            return true;
    }
    return false;
}

int upload_into(mr_model *m, Weight &w, const void *host, int dtype, int64_t rows, int64_t cols) {
    size_t bytes = (size_t)rows * cols * dtype_bytes(dtype);
    if (!w.ptr) MR_TRY(device_alloc(m, bytes, &w.ptr));
    w.dtype = dtype;
    w.rows = rows;
    w.cols = cols;
    MR_HIP(hipMemcpy(w.ptr, host, bytes, hipMemcpyHostToDevice), "upload weight");
    return MR_OK;
}

Weight *weight_slot(mr_model *m, int kind, int layer, int expert) {
    if (layer < 0) {
        switch (kind) {
            case MR_W_EMBED: return &m->embed;
            case MR_W_OUTPUT: return &m->output;
            case MR_W_NORM: return &m->norm;
        }
        return nullptr;
    }
    Layer &L = m->layers[layer];
    const bool heavy = m->d.family == MR_FAMILY_HEAVY_MEDIUM_20;
    switch (kind) {
        case MR_W_A_NORM: return &L.a_norm;
        case MR_W_F_NORM: return &L.f_norm;
        case MR_W_O: return &L.o;
        case MR_W_Q_NORM: return &L.q_norm;
        case MR_W_K_NORM: return &L.k_norm;
        case MR_W_LATENT: return &L.latent;
        case MR_W_LATENT_NORM: return &L.latent_norm;
        case MR_W_KV_UP: return &L.kv_up;
        case MR_W_ATTENTION_GATE: return &L.attention_gate;
        case MR_W_FFN_GATE: return &L.ffn_gate;
        case MR_W_CBR: return &L.cbr;
        case MR_W_ROUTER_COARSE_BIAS: return &L.router_coarse_bias;
        case MR_W_ROUTER_FINE_BIAS: return &L.router_fine_bias;
        case MR_W_ROUTER_GROUP_BIAS: return &L.group_bias;
        case MR_W_ROUTER_EXPERT_BIAS: return &L.expert_bias;
        case MR_W_GATE: case MR_W_UP: case MR_W_DOWN: {
            Mlp *mlp = &L.ffn;
            if (heavy) {
                if (expert < 0 || expert >= (int)L.experts.size()) return nullptr;
                mlp = &L.experts[expert];
            }
            return kind == MR_W_GATE ? &mlp->gate : kind == MR_W_UP ? &mlp->up : &mlp->down;
        }
        case MR_W_SHARED_GATE: case MR_W_SHARED_UP: case MR_W_SHARED_DOWN: {
            if (expert < 0 || expert >= (int)L.shared.size()) return nullptr;
            Mlp &mlp = L.shared[expert];
            return kind == MR_W_SHARED_GATE ? &mlp.gate : kind == MR_W_SHARED_UP ? &mlp.up : &mlp.down;
        }
    }
    return nullptr;
}

void free_weight(Weight &w) {
    if (w.ptr && w.owned) hipFree(w.ptr);
    if (w.f16) hipFree(w.f16);
    w.ptr = nullptr;
    w.f16 = nullptr;
}

// The five fused kernels of one GQA layer (plus the flashnano-1.6 CBR kernels,
// timed together with attention).
int launch_gqa_part(mr_model *m, Layer &L, int part) {
    const mr_model_desc &d = m->d;
    hipStream_t s = m->ctx->stream;
    const int h = d.hidden_size, hd = d.head_dim, qd = d.query_heads * hd, kvw = L.kv_heads * hd;
    switch (part) {
        case MR_KERNEL_QKV: {   // RMSNorm -> fused Q/K/V projection
            GemvArgs g;
            g.w = L.qkv.ptr; g.x = m->hidden; g.gain = L.a_norm.f(); g.eps = d.norm_eps;
            g.n = qd + 2 * kvw; g.k = h; g.y = m->qkv; g.done = m->done_dev;
            if (d.family == MR_FAMILY_FLASHNANO_16) g.x_out = m->xnorm;
            return launch_gemv(s, L.qkv.dtype, PRO_RMS, EPI_STORE, g);
        }
        case MR_KERNEL_ATTENTION: {   // Q/K norm + RoPE + ring write + attention
            AttnStepArgs a;
            a.q = m->qkv; a.k_new = m->qkv + qd; a.v_new = m->qkv + qd + kvw;
            if (d.qk_norm) { a.q_gain = L.q_norm.f(); a.k_gain = L.k_norm.f(); }
            a.eps = d.norm_eps; a.rope = m->rope; a.split_half = d.split_half_rope;
            a.pos = m->pos_dev; a.done = m->done_dev;
            a.ring_k = L.ring_k; a.ring_v = L.ring_v; a.capacity = L.capacity;
            if (d.family == MR_FAMILY_FLASHNANO_16) {
                a.extra_k = L.relay_k; a.extra_v = L.relay_v;
                a.extra_chunk = d.cbr_chunk_size; a.extra_slots = d.cbr_slots;
            }
            a.heads = d.query_heads; a.kv_heads = L.kv_heads; a.dim = hd;
            a.part = m->part; a.counters = m->counters; a.out = m->attn;
            a.splits = L.splits; a.split_len = L.split_len;
            MR_TRY(launch_attention_step(s, a));
            if (d.family != MR_FAMILY_FLASHNANO_16) return MR_OK;
            // flashnano-1.6: chunk pooling into the relay, after this step's attention.
            const int chunk = d.cbr_chunk_size, slots = d.cbr_slots;
            const int dt = L.qkv.dtype;
            size_t lds = (size_t)(chunk + 8) * sizeof(float);
            k_cbr_pool<<<slots, 256, lds, s>>>(m->xnorm, L.pending, L.cbr_queries, m->cbr_pooled, m->cbr_anchor,
                                                m->cbr_skip, m->pos_dev, m->done_dev, chunk, h);
            MR_LAUNCHED("enqueue cbr pool");
            const void *wkv = (const char *)L.qkv.ptr + (size_t)qd * h * dtype_bytes(dt);
            k_cbr_project<<<dim3(ceil_div(2 * kvw, 4), slots), 256, 0, s>>>(m->cbr_pooled, wkv, dt, m->cbr_kv,
                                                                             m->cbr_skip, 2 * kvw, h);
            MR_LAUNCHED("enqueue cbr project");
            k_cbr_finish<<<slots, 256, (size_t)kvw * sizeof(float), s>>>(
                m->cbr_kv, m->cbr_anchor, L.k_norm.f(), d.norm_eps, m->rope, d.split_half_rope, L.relay_k,
                L.relay_v, m->cbr_skip, m->pos_dev, chunk, slots, L.kv_heads, hd);
            MR_LAUNCHED("enqueue cbr finish");
            return MR_OK;
        }
        case MR_KERNEL_O: {   // o projection + residual
            GemvArgs o;
            o.w = L.o.ptr; o.x = m->attn; o.n = h; o.k = qd; o.y = m->hidden; o.scale = d.residual_scale;
            o.done = m->done_dev;
            return launch_gemv(s, L.o.dtype, PRO_COPY, EPI_RESIDUAL, o);
        }
        case MR_KERNEL_GATE_UP: {   // RMSNorm -> gate/up + SwiGLU
            GemvArgs gu;
            gu.w = L.ffn.gate.ptr; gu.w2 = L.ffn.up.ptr; gu.x = m->hidden; gu.gain = L.f_norm.f();
            gu.eps = d.norm_eps; gu.n = d.ffn_dim; gu.k = h; gu.y = m->act; gu.done = m->done_dev;
            return launch_gemv(s, L.ffn.gate.dtype, PRO_RMS, EPI_SWIGLU, gu);
        }
        case MR_KERNEL_DOWN: {   // down projection + residual
            GemvArgs dn;
            dn.w = L.ffn.down.ptr; dn.x = m->act; dn.n = h; dn.k = d.ffn_dim; dn.y = m->hidden;
            dn.scale = d.residual_scale; dn.done = m->done_dev;
            return launch_gemv(s, L.ffn.down.dtype, PRO_COPY, EPI_RESIDUAL, dn);
        }
    }
    return fail(MR_ERR_INVALID, "unknown layer kernel");
}

int record_gqa_layer(mr_model *m, Layer &L) {
    for (int part : {MR_KERNEL_QKV, MR_KERNEL_ATTENTION, MR_KERNEL_O, MR_KERNEL_GATE_UP, MR_KERNEL_DOWN})
        MR_TRY(launch_gqa_part(m, L, part));
    return MR_OK;
}

// One heavy-medium-2.0 layer: inner_loop_steps passes, each latent-KV sparse
// attention + residual, then grouped adaptive MoE + residual (model.py:259-263).
int record_heavy_layer(mr_model *m, Layer &L, int li) {
    const mr_model_desc &d = m->d;
    hipStream_t s = m->ctx->stream;
    const int h = d.hidden_size, hd = d.head_dim, qd = d.query_heads * hd, kvw = L.kv_heads * hd;
    const int inner = d.inner_loop_steps, blocks = ceil_div(d.context_length, d.global_block_size);
    const int kmax = d.router_top_k_max;
    for (int loop = 0; loop < inner; ++loop) {
        GemvArgs g;   // RMSNorm -> [Wq; Wlatent]
        g.w = L.qkv.ptr; g.x = m->hidden; g.gain = L.a_norm.f(); g.eps = d.norm_eps;
        g.n = qd + d.latent_dim; g.k = h; g.y = m->qkv; g.done = m->done_dev;
        MR_TRY(launch_gemv(s, L.qkv.dtype, PRO_RMS, EPI_STORE, g));
        const bool fused = heavy_kv_fused(L.kv_up.dtype, d.latent_dim);
        if (!fused) {
            GemvArgs u;   // latent -> [K; V]
            u.w = L.kv_up.ptr; u.x = m->qkv + qd; u.n = 2 * kvw; u.k = d.latent_dim; u.y = m->kvbuf;
            u.done = m->done_dev;
            MR_TRY(launch_gemv(s, L.kv_up.dtype, PRO_COPY, EPI_STORE, u));
        }
        HeavyAttnArgs a;
        if (fused) {   // the projection runs in the attention prologue
            a.kv_w = L.kv_up.ptr; a.kv_dtype = L.kv_up.dtype; a.latent_x = m->qkv + qd; a.latent = d.latent_dim;
        }
        a.q = m->qkv; a.kv = m->kvbuf; a.rope = m->rope; a.pos = m->pos_dev; a.done = m->done_dev;
        a.q_rot = m->q_rot;
        a.ring_k = L.ring_k + (size_t)loop * d.context_length * kvw;
        a.ring_v = L.ring_v + (size_t)loop * d.context_length * kvw;
        a.bsum_k = L.bsum_k + (size_t)loop * blocks * kvw;
        a.bsum_v = L.bsum_v + (size_t)loop * blocks * kvw;
        a.out = m->attn;
        a.part = m->split_part;
        a.choice = m->choices + ((size_t)li * inner + loop) * m->choice_rec;
        a.choice_stride = d.layers * inner * m->choice_rec;
        a.choice_blocks = 1 + kmax;
        a.heads = d.query_heads; a.kv_heads = L.kv_heads; a.d = hd; a.window = d.window;
        a.block = d.global_block_size; a.slots = d.global_slots; a.slope = d.block_slope;
        MR_TRY(launch_heavy_attention(s, a, d.context_length));
        GemvArgs o;   // hidden += step_scale * Wo . attended
        o.w = L.o.ptr; o.x = m->attn; o.n = h; o.k = qd; o.y = m->hidden; o.scale = d.heavy_step_scale;
        o.done = m->done_dev;
        MR_TRY(launch_gemv(s, L.o.dtype, PRO_COPY, EPI_RESIDUAL, o));
        GemvArgs r;   // RMSNorm -> [Wcoarse; Wfine]; the normalized input feeds the experts
        r.w = L.router.ptr; r.x = m->hidden; r.gain = L.f_norm.f(); r.eps = d.norm_eps;
        r.n = d.router_groups + d.routed_experts; r.k = h; r.y = m->router_out; r.x_out = m->xnorm;
        r.done = m->done_dev;
        MR_TRY(launch_gemv(s, L.router.dtype, PRO_RMS, EPI_STORE, r));
        MoeArgs e;
        const size_t n = d.routed_experts + d.shared_experts;
        e.router = m->router_out;
        e.coarse_bias = L.router_coarse_bias.f(); e.group_bias = L.group_bias.f();
        e.fine_bias = L.router_fine_bias.f(); e.expert_bias = L.expert_bias.f();
        e.x = m->xnorm; e.gate = L.expert_tab; e.up = L.expert_tab + n; e.down = L.expert_tab + 2 * n;
        e.dtype = L.experts[0].gate.dtype; e.done = m->done_dev; e.pos = m->pos_dev;
        e.ids = m->moe_ids; e.weights = m->moe_w; e.active = m->moe_active; e.act = m->moe_act; e.hidden = m->hidden;
        e.choice = a.choice; e.choice_stride = a.choice_stride;
        e.experts = d.routed_experts; e.groups = d.router_groups; e.kmin = d.router_top_k_min; e.kmax = kmax;
        e.shared = d.shared_experts; e.ffn = d.ffn_dim; e.h = h;
        e.inv_temperature_div = d.router_temperature;
        e.log_experts = std::max((float)std::log((double)d.routed_experts), 1.0f);
        e.shared_scale = d.heavy_shared_scale; e.scale = d.heavy_step_scale;
        MR_TRY(launch_moe(s, e));
    }
    return MR_OK;
}

// One flashlighting-2.0 layer (model.py:146-190, 271-279).
int record_light_layer(mr_model *m, Layer &L) {
    const mr_model_desc &d = m->d;
    hipStream_t s = m->ctx->stream;
    const int h = d.hidden_size, hd = d.head_dim, qd = d.query_heads * hd, kvw = L.kv_heads * hd;
    GemvArgs g;   // RMSNorm -> [Wq; Wlatent]; the normalized input also feeds the FFN
    g.w = L.qkv.ptr; g.x = m->hidden; g.gain = L.a_norm.f(); g.eps = d.norm_eps;
    g.n = qd + d.latent_dim; g.k = h; g.y = m->qkv; g.x_out = m->xnorm; g.done = m->done_dev;
    MR_TRY(launch_gemv(s, L.qkv.dtype, PRO_RMS, EPI_STORE, g));
    LightArgs a;
    a.qlat = m->qkv; a.q_gain = L.q_norm.f(); a.k_gain = L.k_norm.f(); a.latent_gain = L.latent_norm.f();
    a.eps = d.norm_eps; a.rope = m->rope; a.split_half = d.split_half_rope; a.pos = m->pos_dev;
    a.done = m->done_dev; a.q_rot = m->q_rot; a.arena = L.arena; a.positions = L.positions; a.counts = L.counts;
    a.kcache = L.kcache; a.vcache = L.vcache; a.lat_new = m->lat_new; a.kv = m->kvbuf; a.st = L.light;
    a.out = m->attn; a.heads = d.query_heads; a.kv_heads = L.kv_heads; a.d = hd; a.latent = d.latent_dim;
    a.window = d.window; a.memory_slots = d.memory_slots; a.cap = L.light_cap; a.part = m->split_part;
    a.kv_w = L.kv_up.ptr; a.kv_dtype = L.kv_up.dtype;
    // queries, the appended row and its cache row: one launch where the
    // geometry allows, else prologue, projection and cache row apart
    const bool fused = light_kv_fused(L.kv_up.dtype, d.latent_dim, hd);
    GemvArgs gu;   // the FFN branch's gate/up: in the fused row kernel where it fits, else after the O projection
    gu.w = L.ffn.gate.ptr; gu.w2 = L.ffn.up.ptr; gu.x = m->xnorm; gu.n = d.ffn_dim; gu.k = h; gu.y = m->act;
    gu.done = m->done_dev;
    const bool ffn_early = fused && light_ffn_in_row_kernel(a, gu, L.ffn.gate.dtype);
    GemvArgs dn;   // the FFN branch's down projection
    dn.w = L.ffn.down.ptr; dn.x = m->act; dn.n = h; dn.k = d.ffn_dim; dn.done = m->done_dev;
    // With gate/up in the fused row kernel, the down rows ride in the attention
    // split kernel (the FFN branch into branch_f) and the O projection's
    // epilogue adds the gated residual; else down's epilogue adds it.
    GemvArgs dn_early = dn;
    dn_early.y = m->branch_f;
    const bool down_early = ffn_early && light_down_in_attend(a, dn_early, L.ffn.down.dtype);
    GemvArgs u;   // [Wk; Wv] . new latent row
    u.w = L.kv_up.ptr; u.x = m->lat_new; u.n = 2 * kvw; u.k = d.latent_dim; u.y = m->kvbuf; u.done = m->done_dev;
    if (fused) {
        MR_TRY(launch_light_kv(s, a));
    } else {
        MR_TRY(launch_light_prep(s, a));
        MR_TRY(launch_gemv(s, L.kv_up.dtype, PRO_COPY, EPI_STORE, u));
        MR_TRY(launch_light_store_kv(s, a, false));
    }
    MR_TRY(launch_light_attend(s, a));
    if (!fused) {   // the merged row's cache row now (the fused row kernel does it at the next step's start)
        GemvArgs um = u;   // [Wk; Wv] . merged row, skipped unless compaction merged
        um.done = &L.light->skip_merged;
        MR_TRY(launch_gemv(s, L.kv_up.dtype, PRO_COPY, EPI_STORE, um));
        MR_TRY(launch_light_store_kv(s, a, true));
    }
    GemvArgs o;
    o.w = L.o.ptr; o.x = m->attn; o.n = h; o.k = qd; o.done = m->done_dev;
    if (down_early) {   // hidden += rs * ((0 + ag * O(attn)) + fg * f)
        o.y = m->hidden; o.aux = m->branch_f; o.scale = d.residual_scale; o.scale_ptr = L.attention_gate.f();
        o.scale_ptr2 = L.ffn_gate.f();
        return launch_gemv(s, L.o.dtype, PRO_COPY, EPI_GATED_ATTN, o);
    }
    o.y = m->branch_o;
    MR_TRY(launch_gemv(s, L.o.dtype, PRO_COPY, EPI_STORE, o));
    if (!ffn_early) MR_TRY(launch_gemv(s, L.ffn.gate.dtype, PRO_COPY, EPI_SWIGLU, gu));
    // hidden += rs * ((0 + ag * o) + fg * down(act)) in the down projection's epilogue
    dn.y = m->hidden; dn.scale = d.residual_scale; dn.aux = m->branch_o; dn.scale_ptr = L.attention_gate.f();
    dn.scale_ptr2 = L.ffn_gate.f();
    return launch_gemv(s, L.ffn.down.dtype, PRO_COPY, EPI_GATED, dn);
}

int launch_lm_head(mr_model *m) {
    const mr_model_desc &d = m->d;
    const Weight &head = d.tie_embeddings ? m->embed : m->output;
    GemvArgs g;
    g.w = head.ptr; g.x = m->hidden; g.gain = m->norm.f(); g.eps = d.norm_eps;
    g.n = d.vocab_size; g.k = d.hidden_size; g.y = m->logits; g.done = m->done_dev;
    return launch_gemv(m->ctx->stream, head.dtype, PRO_RMS, EPI_STORE, g);
}

int record_head(mr_model *m, int kind) {
    const mr_model_desc &d = m->d;
    hipStream_t s = m->ctx->stream;
    if (kind == STEP_PLAIN) {
        k_advance<<<1, 1, 0, s>>>(m->pos_dev, m->done_dev);
        MR_LAUNCHED("enqueue advance");
        return MR_OK;
    }
    MR_TRY(launch_lm_head(m));
    if (kind == STEP_LOGITS) {
        k_advance<<<1, 1, 0, s>>>(m->pos_dev, m->done_dev);
        MR_LAUNCHED("enqueue advance");
    } else {
        k_argmax<<<1, 1024, 0, s>>>(m->logits, d.vocab_size, m->pos_dev, m->done_dev, m->ids_dev, m->gen_dev,
                                    m->count_dev, m->eos_dev, 1);
        MR_LAUNCHED("enqueue argmax");
    }
    return MR_OK;
}

}  // namespace

int record_step(mr_model *m, int kind) {
    hipStream_t s = m->ctx->stream;
    const mr_model_desc &d = m->d;
    k_embed<<<ceil_div(d.hidden_size, 256), 256, 0, s>>>(m->embed.ptr, m->embed.dtype, m->ids_dev, m->pos_dev,
                                                         m->done_dev, m->hidden, d.hidden_size);
    MR_LAUNCHED("enqueue embed");
    for (int li = 0; li < d.layers; ++li)
        MR_TRY(d.family == MR_FAMILY_HEAVY_MEDIUM_20    ? record_heavy_layer(m, m->layers[li], li)
               : d.family == MR_FAMILY_FLASHLIGHTING_20 ? record_light_layer(m, m->layers[li])
                                                        : record_gqa_layer(m, m->layers[li]));
    return record_head(m, kind);
}

namespace {

int run_persistent(mr_model *m, int kind, unsigned long long *trace = nullptr) {
    StepArgs a;
    a.trace = trace;
    a.phases = kind == STEP_PLAIN ? m->prog_plain : m->prog_head;
    a.nphases = kind == STEP_PLAIN ? m->n_plain : m->n_head;
    a.stride = m->n_head;
    a.kind = kind;
    a.pos = m->pos_dev; a.done = m->done_dev; a.ids = m->ids_dev; a.gen = m->gen_dev; a.count = m->count_dev;
    a.eos = m->eos_dev; a.err = m->err; a.exits = m->sync + m->sync_count - 1;
    a.best_val = m->best_val; a.best_idx = m->best_idx; a.bad = m->bad;
    a.embed = m->embed.ptr; a.embed_dtype = m->embed.dtype; a.dummy = m->dummy; a.xbuf = m->xbuf;
    a.progress = m->words; a.nprogress = m->grid;
    return launch_step(m->ctx->stream, a, m->grid, m->step_lds, m->step_dtype, m->d.head_dim);
}

int run_step(mr_model *m, int kind) {
    hipStream_t s = m->ctx->stream;
    if (m->mode == MR_STEP_PERSISTENT && m->persistent_ok) return run_persistent(m, kind);
    if (m->mode == MR_STEP_EAGER) return record_step(m, kind);
    if (!m->exec[kind]) {
        // The first run of each step kind is eager (it also checks every launch
        // configuration); the second captures the same sequence.
        if (m->eager_runs[kind] == 0) {
            m->eager_runs[kind] = 1;
            return record_step(m, kind);
        }
        hipGraph_t graph = nullptr;
        MR_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin step capture");
        int rc = record_step(m, kind);
        hipError_t e = hipStreamEndCapture(s, &graph);
        if (rc != MR_OK) {
            if (graph) hipGraphDestroy(graph);
            return rc;
        }
        MR_HIP(e, "end step capture");
        hipError_t ie = hipGraphInstantiate(&m->exec[kind], graph, nullptr, nullptr, 0);
        hipGraphDestroy(graph);
        MR_HIP(ie, "instantiate step graph");
    }
    MR_HIP(hipGraphLaunch(m->exec[kind], s), "launch step graph");
    return MR_OK;
}

int check_ctx(mr_model *m, const char *what) {
    MR_REQUIRE(m, std::string(what) + ": null model");
    if (m->ctx->fail_next) {
        m->ctx->fail_next = false;
        return fail(MR_ERR_INJECTED, std::string(what) + ": injected failure");
    }
    if (!m->finalized) return fail(MR_ERR_STATE, std::string(what) + ": model not finalized");
    MR_HIP(hipSetDevice(m->ctx->device), "select device");
    return MR_OK;
}

// A persistent step whose wait timed out leaves err set; report it.  The
// kernel's workgroups wait on each other, so they must all be resident at
// once: a timeout means some never started while the others waited (other
// work held CUs).  The model then runs in graph mode from its next reset.
int check_step_error(mr_model *m) {
    if (!m->persistent_ok) return MR_OK;
    int err = 0;
    MR_HIP(hipMemcpy(&err, m->err, sizeof(int), hipMemcpyDeviceToHost), "read step status");
    if (m->inject_timeout && m->mode == MR_STEP_PERSISTENT) {
        m->inject_timeout = false;
        err = 1;
    }
    if (err) {
        m->timed_out = true;
        return fail(MR_ERR_TIMEOUT, "persistent step kernel: a wait for another workgroup timed out (its "
                                    "workgroups were not all resident); the model runs in graph mode after reset");
    }
    return MR_OK;
}

// Phase program of one step for the persistent kernel (GQA families).  Each
// read names the phase whose cells it expects: x_phase for the input,
// res_phase for a residual's previous value.
std::vector<Phase> build_program(mr_model *m, bool head) {
    const mr_model_desc &d = m->d;
    const int h = d.hidden_size, hd = d.head_dim, qd = d.query_heads * hd;
    std::vector<Phase> prog;
    auto last = [&]() { return (int)prog.size() - 1; };
    Phase e;
    e.kind = PH_EMBED;
    e.n = h;
    e.y = m->c_hidden;
    prog.push_back(e);
    int hidden_at = last();
    for (int li = 0; li < d.layers; ++li) {
        Layer &L = m->layers[li];
        const int kvw = L.kv_heads * hd;
        Phase g;
        g.kind = PH_GEMV; g.dtype = L.qkv.dtype; g.n = qd + 2 * kvw; g.k = h; g.pro = PRO_RMS; g.epi = EPI_STORE;
        g.w = L.qkv.ptr; g.x = m->c_hidden; g.x_phase = hidden_at; g.gain = L.a_norm.f(); g.eps = d.norm_eps;
        g.y = m->c_qkv;
        prog.push_back(g);
        const int qkv_at = last();
        Phase a;
        a.kind = PH_ATTN;
        a.x_phase = qkv_at;
        a.heads_done = m->words + (size_t)kWordCopies * kWordCopyStride + (size_t)li * d.query_heads;
        AttnStepArgs &t = a.at.s;
        t.q = (const float *)m->c_qkv;
        t.k_new = (const float *)(m->c_qkv + qd);
        t.v_new = (const float *)(m->c_qkv + qd + kvw);
        if (d.qk_norm) { t.q_gain = L.q_norm.f(); t.k_gain = L.k_norm.f(); }
        t.eps = d.norm_eps; t.rope = m->rope; t.split_half = d.split_half_rope;
        t.ring_k = L.ring_k; t.ring_v = L.ring_v; t.capacity = L.capacity;
        t.heads = d.query_heads; t.kv_heads = L.kv_heads; t.dim = hd;
        t.part = m->part; t.out = (float *)m->c_attn; t.splits = L.step_splits; t.split_len = 0;
        t.part_cells = m->part_cells;
        t.head_groups = L.step_head_groups;
        t.counters = m->merge_counts + (size_t)li * m->merge_count_n / d.layers;
        a.at.mode = 1;
        a.at.ring_k_ro = L.ring_k; a.at.ring_v_ro = L.ring_v;
        prog.push_back(a);
        const int attn_at = last();
        Phase o;
        o.kind = PH_GEMV; o.dtype = L.o.dtype; o.n = h; o.k = qd; o.pro = PRO_COPY; o.epi = EPI_RESIDUAL;
        o.w = L.o.ptr; o.x = m->c_attn; o.x_phase = attn_at; o.y = m->c_hidden; o.res_phase = hidden_at;
        o.ready = a.heads_done; o.nready = L.kv_heads * L.step_head_groups;
        o.scale = d.residual_scale;
        step_attention_mergers(a.at.s, m->grid, o.skip);
        prog.push_back(o);
        hidden_at = last();
        Phase gu;
        gu.kind = PH_GEMV; gu.dtype = L.ffn.gate.dtype; gu.n = d.ffn_dim; gu.k = h; gu.pro = PRO_RMS;
        gu.epi = EPI_SWIGLU; gu.w = L.ffn.gate.ptr; gu.w2 = L.ffn.up.ptr; gu.x = m->c_hidden; gu.x_phase = hidden_at;
        gu.gain = L.f_norm.f(); gu.eps = d.norm_eps; gu.y = m->c_act;
        prog.push_back(gu);
        const int act_at = last();
        Phase dn;
        dn.kind = PH_GEMV; dn.dtype = L.ffn.down.dtype; dn.n = h; dn.k = d.ffn_dim; dn.pro = PRO_COPY;
        dn.epi = EPI_RESIDUAL; dn.w = L.ffn.down.ptr; dn.x = m->c_act; dn.x_phase = act_at; dn.y = m->c_hidden;
        dn.res_phase = hidden_at; dn.scale = d.residual_scale;
        prog.push_back(dn);
        hidden_at = last();
    }
    if (head) {
        const Weight &w = d.tie_embeddings ? m->embed : m->output;
        Phase hp;
        hp.kind = PH_HEAD; hp.dtype = w.dtype; hp.n = d.vocab_size; hp.k = h; hp.pro = PRO_RMS; hp.epi = EPI_STORE;
        hp.w = w.ptr; hp.x = m->c_hidden; hp.x_phase = hidden_at; hp.gain = m->norm.f(); hp.eps = d.norm_eps;
        hp.logits = m->logits;
        prog.push_back(hp);
    }
    return prog;
}

// The persistent kernel covers GQA families whose head dim has a tiled
// attention unit and whose matrices all take 16-byte row vectors.
bool persistent_fits(mr_model *m) {
    const mr_model_desc &d = m->d;
    if (d.family == MR_FAMILY_FLASHNANO_16 || !is_gqa(d.family)) return false;
    if (d.head_dim != 32 && d.head_dim != 64 && d.head_dim != 128) return false;
    if (d.query_heads / d.kv_heads > 16) return false;
    auto vec_ok = [](const Weight &w, int k) {
        int e = w.dtype == MR_F32 ? 4 : 8;
        return k % e == 0 && ((uintptr_t)w.ptr % 16) == 0;
    };
    const int h = d.hidden_size;
    const Weight &head = d.tie_embeddings ? m->embed : m->output;
    if (!vec_ok(head, h)) return false;
    m->step_dtype = head.dtype;   // one weight dtype for every GEMV phase (the kernel's instantiation)
    for (Layer &L : m->layers) {
        if (d.query_heads / L.kv_heads > 16) return false;
        if (!vec_ok(L.qkv, h) || !vec_ok(L.o, d.query_heads * d.head_dim) || !vec_ok(L.ffn.gate, h) ||
            !vec_ok(L.ffn.up, h) || !vec_ok(L.ffn.down, d.ffn_dim))
            return false;
        for (const Weight *w : {&L.qkv, &L.o, &L.ffn.gate, &L.ffn.up, &L.ffn.down})
            if (w->dtype != m->step_dtype) return false;
    }
    return true;
}

int setup_persistent(mr_model *m) {
    m->persistent_ok = false;
    if (!persistent_fits(m)) return MR_OK;
    const mr_model_desc &d = m->d;
    hipDeviceProp_t p;
    MR_HIP(hipGetDeviceProperties(&p, m->ctx->device), "query device");
    m->grid = p.multiProcessorCount;
    if (m->grid < 8) return MR_OK;
    // Epochs are position * stride + phase + 1 in 32 bits.
    const int64_t stride = 2 + 5 * (int64_t)d.layers;
    if ((int64_t)(d.context_length + 1) * stride >= (int64_t)UINT32_MAX) return MR_OK;
    // Cells: hidden, qkv, attn, act, each region a multiple of two cells so
    // every region starts 16-byte aligned.
    int max_kvw = 0;
    for (Layer &L : m->layers) max_kvw = std::max(max_kvw, L.kv_heads * d.head_dim);
    auto even = [](size_t n) { return (n + 1) & ~(size_t)1; };
    const size_t qd = (size_t)d.query_heads * d.head_dim;
    const size_t n_hidden = even(d.hidden_size), n_qkv = even(qd + 2 * (size_t)max_kvw), n_attn = even(qd);
    m->cell_count = n_hidden + n_qkv + n_attn + even(d.ffn_dim);
    MR_TRY(device_alloc(m, m->cell_count * sizeof(uint64_t), (void **)&m->cells));
    m->c_hidden = m->cells;
    m->c_qkv = m->c_hidden + n_hidden;
    m->c_attn = m->c_qkv + n_qkv;
    m->c_act = m->c_attn + n_attn;
    m->sync_count = 1;   // the launch exit counter
    MR_TRY(device_alloc(m, m->sync_count * sizeof(unsigned), (void **)&m->sync));
    if (m->grid > kWordCopyStride) return MR_OK;   // more workgroups than a progress-word copy holds
    m->word_count = (size_t)kWordCopies * kWordCopyStride + (size_t)d.layers * d.query_heads;
    MR_TRY(device_alloc(m, m->word_count * sizeof(unsigned), (void **)&m->words));
    MR_HIP(hipMemset(m->words, 0, m->word_count * sizeof(unsigned)), "clear step progress");
    m->part_cell_count = 0;
    for (Layer &L : m->layers) {
        L.step_splits = step_attention_splits(L.capacity, L.kv_heads, d.head_dim, m->grid);
        L.step_head_groups = step_attention_head_groups(d.query_heads, L.kv_heads, L.step_splits, m->grid);
        m->part_cell_count = std::max(m->part_cell_count, (size_t)d.query_heads * L.step_splits * (d.head_dim + 2));
    }
    MR_TRY(device_alloc(m, m->part_cell_count * sizeof(uint64_t), (void **)&m->part_cells));
    MR_HIP(hipMemset(m->part_cells, 0, m->part_cell_count * sizeof(uint64_t)), "clear attention cells");
    int max_kvh = 1;   // counters per layer: one per (KV head, query-head group)
    for (Layer &L : m->layers) max_kvh = std::max(max_kvh, L.kv_heads * L.step_head_groups);
    m->merge_count_n = (size_t)d.layers * max_kvh;
    MR_TRY(device_alloc(m, m->merge_count_n * sizeof(unsigned), (void **)&m->merge_counts));
    MR_HIP(hipMemset(m->merge_counts, 0, m->merge_count_n * sizeof(unsigned)), "clear attention counters");
    MR_TRY(device_alloc(m, 256, &m->dummy));
    MR_TRY(device_alloc(m, sizeof(int), (void **)&m->err));
    MR_TRY(device_alloc(m, m->grid * sizeof(float), (void **)&m->best_val));
    MR_TRY(device_alloc(m, m->grid * sizeof(int), (void **)&m->best_idx));
    MR_TRY(device_alloc(m, m->grid * sizeof(int), (void **)&m->bad));
    MR_HIP(hipMemset(m->cells, 0, m->cell_count * sizeof(uint64_t)), "clear step cells");
    MR_HIP(hipMemset(m->sync, 0, m->sync_count * sizeof(unsigned)), "clear step counters");
    MR_HIP(hipMemset(m->dummy, 0, 256), "clear step dummy");
    MR_HIP(hipMemset(m->err, 0, sizeof(int)), "clear step status");

    std::vector<Phase> plain = build_program(m, false), head = build_program(m, true);
    if ((int64_t)head.size() != stride) return fail(MR_ERR_INVALID, "step program: unexpected phase count");
    m->xbuf = std::max(step_xbuf_floats(plain, m->grid), step_xbuf_floats(head, m->grid));
    m->step_lds = std::max(step_lds_bytes(plain, m->grid), step_lds_bytes(head, m->grid));
    if (m->step_lds > 64 * 1024) return MR_OK;
    int per_cu = 0;   // every workgroup must be resident at once (one per CU)
    MR_TRY(step_blocks_per_cu(m->step_lds, m->step_dtype, d.head_dim, &per_cu));
    if (per_cu < 1) return MR_OK;
    m->n_plain = (int)plain.size();
    m->n_head = (int)head.size();
    MR_TRY(device_alloc(m, plain.size() * sizeof(Phase), (void **)&m->prog_plain));
    MR_TRY(device_alloc(m, head.size() * sizeof(Phase), (void **)&m->prog_head));
    MR_HIP(hipMemcpy(m->prog_plain, plain.data(), plain.size() * sizeof(Phase), hipMemcpyHostToDevice),
           "upload step program");
    MR_HIP(hipMemcpy(m->prog_head, head.data(), head.size() * sizeof(Phase), hipMemcpyHostToDevice),
           "upload step program");
    m->persistent_ok = true;
    return MR_OK;
}

// heavy-medium-2.0 layer: packed projections present, experts complete,
// per-inner-loop rings (capacity = context) and block sums, expert table.
// FP16 copies of projection matrices for the batched prefill's FP16-term
// GEMMs (gemm.h), each with its power-of-two scale; the matrices in `shared`
// (a SwiGLU pair, one tile holds rows of both) take their smaller scale.
int f16_copies(mr_model *m, std::initializer_list<Weight *> ws, std::initializer_list<Weight *> shared) {
    for (Weight *w : ws)
        MR_TRY(gemm_f16_weight_scale(m->ctx->stream, w->ptr, w->dtype, w->rows * w->cols, &w->f16_scale));
    float common = INFINITY;
    for (Weight *w : shared) common = std::min(common, w->f16_scale);
    for (Weight *w : shared) w->f16_scale = common;
    for (Weight *w : ws)
        if (w->f16_scale > 0.0f) {
            MR_TRY(device_alloc(m, (size_t)w->rows * w->cols * 2, &w->f16));
            MR_TRY(gemm_f16_weight_copy(m->ctx->stream, w->ptr, w->rows * w->cols, w->f16_scale, w->f16));
        }
    return MR_OK;
}

// Bounds on the gate and up rows' norms where the batched prefill writes the
// SwiGLU output straight into the down projection's FP16 terms (every
// matrix of the FFN with an FP16 copy).  The FFN's input rows are RMSNorm
// outputs of `width` values with `gain` (1-D, float32), so |y|^2 <= width
// max gain^2 and every output of a row is at most width max gain^2 ng nu: the
// bounds are kept only where that stays finite, so that the row scales are.
int swiglu_row_norms(mr_model *m, Mlp &f, const Weight &gain, int width) {
    f.gate.row_norm = f.up.row_norm = 0.0f;
    if (!(f.gate.f16_scale > 0.0f && f.up.f16_scale > 0.0f && f.down.f16_scale > 0.0f)) return MR_OK;
    for (Weight *w : {&f.gate, &f.up})
        MR_TRY(gemm_row_norm_bound(m->ctx->stream, w->ptr, w->dtype, w->rows, w->cols, &w->row_norm));
    double gmax = 1.0;
    if (gain.ptr) {
        std::vector<float> g(width);
        MR_HIP(hipMemcpy(g.data(), gain.ptr, (size_t)width * sizeof(float), hipMemcpyDeviceToHost), "read norm gain");
        gmax = 0.0;
        for (float v : g) gmax = std::isfinite(v) ? std::max(gmax, (double)std::fabs(v)) : INFINITY;
    }
    const double bound = (double)width * gmax * gmax * f.gate.row_norm * f.up.row_norm;
    if (!(bound < 1.0e37)) f.gate.row_norm = f.up.row_norm = 0.0f;
    return MR_OK;
}

// The SwiGLU output of rows of `h` values straight into the down
// projection's FP16 terms (the row-norm bounds found at finalize).
bool act_split_fits(const Mlp &f, int h) {
    return h <= 2048 && f.down.f16_scale > 0.0f && f.gate.row_norm > 0.0f && f.up.row_norm > 0.0f;
}

int finalize_heavy_layer(mr_model *m, Layer &L, int i) {
    const mr_model_desc &d = m->d;
    const int hd = d.head_dim, qd = d.query_heads * hd, kvw = L.kv_heads * hd;
    const std::string at = " in layer " + std::to_string(i);
    for (const Weight *w : {&L.kv_up, &L.router_coarse_bias, &L.router_fine_bias, &L.group_bias, &L.expert_bias})
        if (!w->ptr) return fail(MR_ERR_STATE, "missing heavy-medium weight" + at);
    if (L.qkv.rows != 3) return fail(MR_ERR_STATE, "missing q/latent weight" + at);
    L.qkv.rows = qd + d.latent_dim;
    if (L.router.rows != 3) return fail(MR_ERR_STATE, "missing router weight" + at);
    L.router.rows = d.router_groups + d.routed_experts;
    // the batched prefill's FP16-term projections (the router keeps the exact
    // BF16-term GEMM: its logits choose the experts)
    MR_TRY(f16_copies(m, {&L.qkv, &L.kv_up, &L.o}, {}));
    const int dt = L.experts[0].gate.dtype;
    std::vector<void *> tab(3 * (size_t)(d.routed_experts + d.shared_experts));
    const size_t n = d.routed_experts + d.shared_experts;
    for (size_t e = 0; e < n; ++e) {
        const Mlp &mlp = e < (size_t)d.routed_experts ? L.experts[e] : L.shared[e - d.routed_experts];
        if (!mlp.gate.ptr || !mlp.up.ptr || !mlp.down.ptr) return fail(MR_ERR_STATE, "missing expert weight" + at);
        if (mlp.gate.dtype != dt || mlp.up.dtype != dt || mlp.down.dtype != dt)
            return fail(MR_ERR_INVALID, "experts must share one dtype" + at);
        tab[e] = mlp.gate.ptr;
        tab[n + e] = mlp.up.ptr;
        tab[2 * n + e] = mlp.down.ptr;
    }
    MR_TRY(device_alloc(m, tab.size() * sizeof(void *), (void **)&L.expert_tab));
    MR_HIP(hipMemcpy(L.expert_tab, tab.data(), tab.size() * sizeof(void *), hipMemcpyHostToDevice), "upload expert table");
    // FP16 copies for the batched prefill's grouped GEMMs (all experts or none)
    std::vector<void *> tab_h(tab.size());
    std::vector<float> scale(tab.size());
    bool all = true;
    for (size_t e = 0; e < n && all; ++e) {
        Mlp &mlp = e < (size_t)d.routed_experts ? L.experts[e] : L.shared[e - d.routed_experts];
        MR_TRY(f16_copies(m, {&mlp.gate, &mlp.up, &mlp.down}, {&mlp.gate, &mlp.up}));
        all = mlp.gate.f16 && mlp.up.f16 && mlp.down.f16;
        tab_h[e] = mlp.gate.f16;
        tab_h[n + e] = mlp.up.f16;
        tab_h[2 * n + e] = mlp.down.f16;
        scale[e] = mlp.gate.f16_scale;
        scale[n + e] = mlp.up.f16_scale;
        scale[2 * n + e] = mlp.down.f16_scale;
    }
    if (all) {
        MR_TRY(device_alloc(m, tab_h.size() * sizeof(void *), (void **)&L.expert_tab_h));
        MR_HIP(hipMemcpy(L.expert_tab_h, tab_h.data(), tab_h.size() * sizeof(void *), hipMemcpyHostToDevice),
               "upload expert table");
        MR_TRY(device_alloc(m, scale.size() * sizeof(float), (void **)&L.expert_scale));
        MR_HIP(hipMemcpy(L.expert_scale, scale.data(), scale.size() * sizeof(float), hipMemcpyHostToDevice),
               "upload expert scales");
    }
    const size_t ring = (size_t)d.inner_loop_steps * d.context_length * kvw * sizeof(float);
    const int blocks = ceil_div(d.context_length, d.global_block_size);
    const size_t bsum = (size_t)d.inner_loop_steps * blocks * kvw * sizeof(float);
    MR_TRY(device_alloc(m, ring, (void **)&L.ring_k));
    MR_TRY(device_alloc(m, ring, (void **)&L.ring_v));
    MR_TRY(device_alloc(m, bsum, (void **)&L.bsum_k));
    MR_TRY(device_alloc(m, bsum, (void **)&L.bsum_v));
    for (void *p : {(void *)L.ring_k, (void *)L.ring_v, (void *)L.bsum_k, (void *)L.bsum_v})
        MR_HIP(hipMemset(p, 0, p == L.ring_k || p == L.ring_v ? ring : bsum), "clear heavy caches");
    if (heavy_split_path(hd, d.window, d.context_length, d.global_block_size, d.global_slots) && !m->split_part) {
        // split partials, shared by the layers and inner-loop passes (one at a time)
        const size_t n = (size_t)d.query_heads * heavy_parts(d.window, d.context_length) * (hd + 2);
        MR_TRY(device_alloc(m, n * sizeof(float), (void **)&m->split_part));
    }
    return MR_OK;
}

// flashlighting-2.0 layer: packed projections, norms, gates and FFN present;
// latent ring of window + memory_slots + 1 rows with key/value caches.
int finalize_light_layer(mr_model *m, Layer &L, int i) {
    const mr_model_desc &d = m->d;
    const int hd = d.head_dim, qd = d.query_heads * hd, kvw = L.kv_heads * hd;
    const std::string at = " in layer " + std::to_string(i);
    for (const Weight *w : {&L.q_norm, &L.k_norm, &L.latent_norm, &L.attention_gate, &L.ffn_gate, &L.ffn.gate,
                            &L.ffn.up, &L.ffn.down})
        if (!w->ptr) return fail(MR_ERR_STATE, "missing flashlighting weight" + at);
    if (L.qkv.rows != 3) return fail(MR_ERR_STATE, "missing q/latent weight" + at);
    L.qkv.rows = qd + d.latent_dim;
    if (L.kv_up.rows != 3) return fail(MR_ERR_STATE, "missing k/v weight" + at);
    L.kv_up.rows = 2 * kvw;
    MR_REQUIRE(L.ffn.gate.dtype == L.ffn.up.dtype, "ffn gate and up must share one dtype");
    MR_TRY(f16_copies(m, {&L.qkv, &L.kv_up, &L.o, &L.ffn.gate, &L.ffn.up, &L.ffn.down}, {&L.ffn.gate, &L.ffn.up}));
    MR_TRY(swiglu_row_norms(m, L.ffn, L.a_norm, d.hidden_size));   // the FFN branch reads the attention's input
    L.light_cap = d.window + d.memory_slots + 1;
    const size_t cap = L.light_cap;
    MR_TRY(device_alloc(m, cap * d.latent_dim * sizeof(float), (void **)&L.arena));
    MR_TRY(device_alloc(m, cap * sizeof(float), (void **)&L.positions));
    MR_TRY(device_alloc(m, cap * sizeof(float), (void **)&L.counts));
    MR_TRY(device_alloc(m, cap * kvw * sizeof(float), (void **)&L.kcache));
    MR_TRY(device_alloc(m, cap * kvw * sizeof(float), (void **)&L.vcache));
    MR_TRY(device_alloc(m, sizeof(LightState), (void **)&L.light));
    MR_HIP(hipMemset(L.light, 0, sizeof(LightState)), "clear latent state");
    if (light_split_path(hd, L.light_cap) && !m->split_part) {   // split partials, shared by the layers (one at a time)
        const size_t n = (size_t)d.query_heads * light_splits(L.light_cap) * (hd + 2);
        MR_TRY(device_alloc(m, n * sizeof(float), (void **)&m->split_part));
    }
    return MR_OK;
}

void destroy_graphs(mr_model *m) {
    for (auto &e : m->exec)
        if (e) {
            hipGraphExecDestroy(e);
            e = nullptr;
        }
    m->eager_runs.fill(0);
}

}  // namespace
}  // namespace mr

extern "C" {

int mr_model_create(mr_ctx *ctx, const mr_model_desc *desc, mr_model **out) {
    MR_REQUIRE(ctx && desc && out, "mr_model_create: null argument");
    const mr_model_desc &d = *desc;
    MR_REQUIRE(d.family >= 0 && d.family <= MR_FAMILY_HEAVY_MEDIUM_20, "unsupported family");
    MR_REQUIRE(d.vocab_size > 0 && d.hidden_size > 0 && d.layers > 0 && d.layers <= 128 && d.query_heads > 0 &&
                   d.kv_heads > 0 && d.head_dim > 0 && d.head_dim % 2 == 0 && d.ffn_dim > 0 &&
                   d.context_length > 0 && d.query_heads % d.kv_heads == 0,
               "invalid model geometry");
    const bool heavy = d.family == MR_FAMILY_HEAVY_MEDIUM_20;
    if (d.family == MR_FAMILY_FLASHLIGHTING_20)
        MR_REQUIRE(d.latent_dim > 0 && d.window > 0 && d.memory_slots >= 0, "invalid flashlighting-2.0 geometry");
    if (heavy)
        MR_REQUIRE(d.latent_dim > 0 && d.inner_loop_steps >= 1 && d.routed_experts >= 1 &&
                       d.routed_experts <= 256 && d.router_groups >= 1 && d.router_groups <= d.routed_experts &&
                       d.router_top_k_min >= 1 && d.router_top_k_min <= d.router_top_k_max &&
                       d.router_top_k_max <= std::min(d.routed_experts, 16) && d.shared_experts >= 0 &&
                       d.global_block_size > 0 && d.global_slots > 0 && d.window > 0,
                   "invalid heavy-medium-2.0 geometry");
    if (d.family == MR_FAMILY_FLASHNANO_16)
        MR_REQUIRE(d.cbr_chunk_size > 0 && d.cbr_slots > 0, "FlashNano 1.6 requires CBR chunk size and slots");
    mr_model *m = new mr_model();
    m->ctx = ctx;
    m->d = d;
    m->layers.resize(d.layers);
    for (int i = 0; i < d.layers; ++i) {
        Layer &L = m->layers[i];
        uint64_t bit = i < 64 ? (d.global_layer_mask_lo >> i) & 1 : (d.global_layer_mask_hi >> (i - 64)) & 1;
        L.global = bit != 0;
        L.kv_heads = L.global && d.global_kv_heads ? d.global_kv_heads : d.kv_heads;
        // model.py:105 capacity = min(window or ctx, ctx)
        int win = L.global ? 0 : d.window;
        L.capacity = win > 0 ? std::min(win, d.context_length) : d.context_length;
        if (heavy) {   // model.py:203: each inner loop keeps every position
            L.global = false;
            L.kv_heads = d.kv_heads;
            L.capacity = d.context_length;
            L.experts.resize(d.routed_experts);
            L.shared.resize(d.shared_experts);
        }
        if (d.query_heads % L.kv_heads != 0) {
            delete m;
            return fail(MR_ERR_INVALID, "query heads must divide into KV groups");
        }
    }
    // The model keeps its context (device, stream) alive: destroying the
    // context first only drops the caller's reference.
    ctx_retain(ctx);
    *out = m;
    return MR_OK;
}

int mr_model_destroy(mr_model *m) {
    if (!m) return MR_OK;
    hipSetDevice(m->ctx->device);
    hipStreamSynchronize(m->ctx->stream);
    destroy_graphs(m);
    free_weight(m->embed);
    free_weight(m->output);
    free_weight(m->norm);
    for (Layer &L : m->layers) {
        for (Weight *w : {&L.a_norm, &L.f_norm, &L.qkv, &L.q_norm, &L.k_norm, &L.o, &L.ffn.gate, &L.ffn.up,
                          &L.ffn.down, &L.cbr, &L.latent, &L.latent_norm, &L.k_up, &L.v_up, &L.attention_gate,
                          &L.ffn_gate, &L.kv_up, &L.router, &L.router_coarse_bias, &L.router_fine_bias,
                          &L.group_bias, &L.expert_bias})
            free_weight(*w);
        for (Mlp &e : L.experts) { free_weight(e.gate); free_weight(e.up); free_weight(e.down); }
        for (Mlp &e : L.shared) { free_weight(e.gate); free_weight(e.up); free_weight(e.down); }
        for (float *p : {L.ring_k, L.ring_v, L.relay_k, L.relay_v, L.pending, L.cbr_queries, L.bsum_k, L.bsum_v,
                         L.arena, L.positions, L.counts, L.kcache, L.vcache})
            if (p) hipFree(p);
        if (L.light) hipFree(L.light);
        if (L.expert_tab) hipFree(L.expert_tab);
        if (L.expert_tab_h) hipFree(L.expert_tab_h);
        if (L.expert_scale) hipFree(L.expert_scale);
    }
    if (m->choices) hipFree(m->choices);
    if (m->freq) hipFree(m->freq);
    if (m->rope) hipFree(m->rope);
    if (m->state) hipFree(m->state);
    if (m->pf) hipFree(m->pf);
    if (m->split_part) hipFree(m->split_part);
    for (void *p : {(void *)m->prog_plain, (void *)m->prog_head, (void *)m->cells, (void *)m->sync, (void *)m->words, (void *)m->part_cells, (void *)m->merge_counts, m->dummy,
                    (void *)m->err, (void *)m->best_val, (void *)m->best_idx, (void *)m->bad})
        if (p) hipFree(p);
    mr_ctx *ctx = m->ctx;
    delete m;
    ctx_unref(ctx);
    return MR_OK;
}

int mr_model_set_weight(mr_model *m, int kind, int layer, int expert, const void *host, int dtype, int64_t rows,
                        int64_t cols) {
    MR_REQUIRE(m && host, "set_weight: null argument");
    MR_REQUIRE(dtype == MR_F32 || dtype == MR_BF16 || dtype == MR_F16, "set_weight: unknown dtype");
    MR_REQUIRE(layer >= -1 && layer < m->d.layers, "set_weight: layer out of range");
    MR_REQUIRE(!m->finalized, "set_weight: model already finalized");
    MR_HIP(hipSetDevice(m->ctx->device), "select device");
    Expect e;
    MR_TRY(expected_shape(m, kind, layer, &e));
    if (rows != e.rows || cols != e.cols)
        return fail(MR_ERR_INVALID, "weight kind " + std::to_string(kind) + " layer " + std::to_string(layer) +
                                        ": expected (" + std::to_string(e.rows) + ", " + std::to_string(e.cols) +
                                        "), got (" + std::to_string(rows) + ", " + std::to_string(cols) + ")");
    if (is_vector_kind(kind)) MR_REQUIRE(dtype == MR_F32, "set_weight: 1-D tensors must be float32");
    const bool model_level = kind == MR_W_EMBED || kind == MR_W_OUTPUT || kind == MR_W_NORM;
    MR_REQUIRE(model_level == (layer < 0), "set_weight: layer index does not match weight kind");
    if (is_gqa(m->d.family) && (kind == MR_W_Q || kind == MR_W_K || kind == MR_W_V)) {
        // Pack [Wq; Wk; Wv] so one GEMV produces the whole projection.
        Layer &L = m->layers[layer];
        const int64_t h = m->d.hidden_size, qd = (int64_t)m->d.query_heads * m->d.head_dim;
        const int64_t kvw = (int64_t)L.kv_heads * m->d.head_dim;
        const int64_t total = qd + 2 * kvw;
        if (!L.qkv.ptr) {
            MR_TRY(device_alloc(m, (size_t)total * h * dtype_bytes(dtype), &L.qkv.ptr));
            L.qkv.dtype = dtype;
            L.qkv.rows = 0;
            L.qkv.cols = h;
        }
        MR_REQUIRE(L.qkv.dtype == dtype, "set_weight: q, k and v must share one dtype");
        int64_t row0 = kind == MR_W_Q ? 0 : kind == MR_W_K ? qd : qd + kvw;
        char *dst = (char *)L.qkv.ptr + (size_t)row0 * h * dtype_bytes(dtype);
        MR_HIP(hipMemcpy(dst, host, (size_t)rows * cols * dtype_bytes(dtype), hipMemcpyHostToDevice),
               "upload weight");
        L.qkv.rows |= kind == MR_W_Q ? 1 : kind == MR_W_K ? 2 : 4;   // presence bits until finalize
        return MR_OK;
    }
    const bool lighting = m->d.family == MR_FAMILY_FLASHLIGHTING_20;
    if ((m->d.family == MR_FAMILY_HEAVY_MEDIUM_20 &&
         (kind == MR_W_Q || kind == MR_W_LATENT || kind == MR_W_ROUTER_COARSE || kind == MR_W_ROUTER_FINE)) ||
        (lighting && (kind == MR_W_Q || kind == MR_W_LATENT || kind == MR_W_K || kind == MR_W_V))) {
        // Pack [Wq; Wlatent], [Wcoarse; Wfine] and [Wk; Wv]: one GEMV each.
        Layer &L = m->layers[layer];
        const bool qpair = kind == MR_W_Q || kind == MR_W_LATENT;
        const bool kvpair = kind == MR_W_K || kind == MR_W_V;
        Weight &w = qpair ? L.qkv : kvpair ? L.kv_up : L.router;
        const int64_t kvw = (int64_t)L.kv_heads * m->d.head_dim;
        const int64_t h = kvpair ? m->d.latent_dim : m->d.hidden_size;
        const int64_t first = qpair ? (int64_t)m->d.query_heads * m->d.head_dim : kvpair ? kvw : m->d.router_groups;
        const int64_t second = qpair ? m->d.latent_dim : kvpair ? kvw : m->d.routed_experts;
        if (!w.ptr) {
            MR_TRY(device_alloc(m, (size_t)(first + second) * h * dtype_bytes(dtype), &w.ptr));
            w.dtype = dtype;
            w.rows = 0;
            w.cols = h;
        }
        MR_REQUIRE(w.dtype == dtype, "set_weight: packed projections must share one dtype");
        const bool lead = kind == MR_W_Q || kind == MR_W_ROUTER_COARSE || kind == MR_W_K;
        char *dst = (char *)w.ptr + (size_t)(lead ? 0 : first) * h * dtype_bytes(dtype);
        MR_HIP(hipMemcpy(dst, host, (size_t)rows * cols * dtype_bytes(dtype), hipMemcpyHostToDevice),
               "upload weight");
        w.rows |= lead ? 1 : 2;   // presence bits until finalize
        return MR_OK;
    }
    Weight *slot = weight_slot(m, kind, layer, expert);
    MR_REQUIRE(slot, "set_weight: weight kind not used by this family or expert index out of range");
    if (slot->ptr && slot->dtype != dtype) free_weight(*slot);
    return upload_into(m, *slot, host, dtype, rows, cols);
}

int mr_model_set_rope(mr_model *m, const float *inv_freq, int count) {
    MR_REQUIRE(m && inv_freq && count == m->d.head_dim / 2, "set_rope: expected head_dim/2 frequencies");
    MR_HIP(hipSetDevice(m->ctx->device), "select device");
    if (!m->freq) MR_TRY(device_alloc(m, count * sizeof(float), (void **)&m->freq));
    MR_HIP(hipMemcpy(m->freq, inv_freq, count * sizeof(float), hipMemcpyHostToDevice), "upload rope table");
    // cos/sin of every integer position: the angle is the FP32 product pos*freq
    // (kernels.cl:38), its cosine and sine are taken in double and rounded once.
    const int ctxn = m->d.context_length;
    std::vector<float> table((size_t)ctxn * count * 2);
    for (int pos = 0; pos < ctxn; ++pos)
        for (int p = 0; p < count; ++p) {
            float a = (float)pos * inv_freq[p];
            table[((size_t)pos * count + p) * 2] = (float)std::cos((double)a);
            table[((size_t)pos * count + p) * 2 + 1] = (float)std::sin((double)a);
        }
    if (!m->rope) MR_TRY(device_alloc(m, table.size() * sizeof(float), (void **)&m->rope));
    MR_HIP(hipMemcpy(m->rope, table.data(), table.size() * sizeof(float), hipMemcpyHostToDevice),
           "upload rope table");
    return MR_OK;
}

int mr_model_finalize(mr_model *m) {
    MR_REQUIRE(m, "finalize: null model");
    if (m->finalized) return MR_OK;
    MR_HIP(hipSetDevice(m->ctx->device), "select device");
    const mr_model_desc &d = m->d;
    int cus = 0;   // attention units per layer: at most one per CU
    MR_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, m->ctx->device), "query device");
    auto need = [&](const Weight &w, const char *name, int layer) -> int {
        if (!w.ptr)
            return fail(MR_ERR_STATE, std::string("missing weight ") + name +
                                          (layer >= 0 ? " in layer " + std::to_string(layer) : std::string()));
        return MR_OK;
    };
    MR_TRY(need(m->embed, "embed", -1));
    MR_TRY(need(m->norm, "norm", -1));
    if (!d.tie_embeddings) MR_TRY(need(m->output, "output", -1));
    MR_REQUIRE(m->freq, "finalize: RoPE table not set");
    const int h = d.hidden_size, hd = d.head_dim, qd = d.query_heads * hd;
    int max_kvw = 0, max_kvh = 0;
    size_t max_part = 0;
    const bool heavy = d.family == MR_FAMILY_HEAVY_MEDIUM_20;
    const bool lighting = d.family == MR_FAMILY_FLASHLIGHTING_20;
    const int inner = heavy ? d.inner_loop_steps : 1;
    for (int i = 0; i < d.layers; ++i) {
        Layer &L = m->layers[i];
        MR_TRY(need(L.a_norm, "a_norm", i));
        MR_TRY(need(L.o, "o", i));
        if (lighting) {
            MR_TRY(finalize_light_layer(m, L, i));
            max_kvw = std::max(max_kvw, L.kv_heads * hd);
            max_kvh = std::max(max_kvh, L.kv_heads);
            continue;
        }
        MR_TRY(need(L.f_norm, "f_norm", i));
        if (heavy) {
            MR_TRY(finalize_heavy_layer(m, L, i));
            max_kvw = std::max(max_kvw, L.kv_heads * hd);
            max_kvh = std::max(max_kvh, L.kv_heads);
            continue;
        }
        if (L.qkv.rows != 7) return fail(MR_ERR_STATE, "missing q/k/v weight in layer " + std::to_string(i));
        L.qkv.rows = qd + 2 * (int64_t)L.kv_heads * hd;
        if (d.qk_norm) {
            MR_TRY(need(L.q_norm, "q_norm", i));
            MR_TRY(need(L.k_norm, "k_norm", i));
        }
        MR_TRY(need(L.ffn.gate, "ffn.gate", i));
        MR_TRY(need(L.ffn.up, "ffn.up", i));
        MR_TRY(need(L.ffn.down, "ffn.down", i));
        MR_REQUIRE(L.ffn.gate.dtype == L.ffn.up.dtype, "ffn gate and up must share one dtype");
        MR_TRY(f16_copies(m, {&L.qkv, &L.o, &L.ffn.gate, &L.ffn.up, &L.ffn.down}, {&L.ffn.gate, &L.ffn.up}));
        MR_TRY(swiglu_row_norms(m, L.ffn, L.f_norm, h));
        const int kvw = L.kv_heads * hd;
        max_kvw = std::max(max_kvw, kvw);
        max_kvh = std::max(max_kvh, L.kv_heads);
        size_t ring = (size_t)L.capacity * kvw * sizeof(float);
        MR_TRY(device_alloc(m, ring, (void **)&L.ring_k));
        MR_TRY(device_alloc(m, ring, (void **)&L.ring_v));
        MR_HIP(hipMemset(L.ring_k, 0, ring), "clear ring");
        MR_HIP(hipMemset(L.ring_v, 0, ring), "clear ring");
        int extra_max = 0;
        if (d.family == MR_FAMILY_FLASHNANO_16) {
            MR_TRY(need(L.cbr, "cbr", i));
            L.relay_capacity = (d.context_length / d.cbr_chunk_size) * d.cbr_slots;
            extra_max = L.relay_capacity;
            size_t relay = (size_t)std::max(L.relay_capacity, 1) * kvw * sizeof(float);
            MR_TRY(device_alloc(m, relay, (void **)&L.relay_k));
            MR_TRY(device_alloc(m, relay, (void **)&L.relay_v));
            int prow = std::min(d.cbr_chunk_size, d.context_length);
            MR_TRY(device_alloc(m, (size_t)prow * h * sizeof(float), (void **)&L.pending));
            MR_TRY(device_alloc(m, (size_t)d.cbr_slots * h * sizeof(float), (void **)&L.cbr_queries));
            k_rows_rms<<<d.cbr_slots, 256, 0, m->ctx->stream>>>(L.cbr.ptr, L.cbr.dtype, L.cbr_queries, h,
                                                                d.cbr_norm_eps);
            MR_LAUNCHED("normalize cbr queries");
        }
        attention_plan(L.capacity + extra_max, L.kv_heads, hd, cus, &L.splits, &L.split_len);
        max_part = std::max(max_part, attention_part_floats(d.query_heads, L.kv_heads, hd, L.splits));
    }
    // One allocation for all per-sequence scalars and activation vectors.
    const int ctxn = d.context_length + 2;
    const int slots = std::max(d.cbr_slots, 1);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        size_t at = off;
        off += (bytes + 255) / 256 * 256;
        return at;
    };
    size_t o_ints = take(8 * sizeof(int));
    size_t o_ids = take((size_t)ctxn * sizeof(int));
    size_t o_gen = take((size_t)ctxn * sizeof(int));
    size_t o_hidden = take((size_t)h * sizeof(float));
    size_t o_xnorm = take((size_t)h * sizeof(float));
    size_t o_qkv = take((size_t)(qd + std::max(2 * max_kvw, d.latent_dim)) * sizeof(float));
    const int kmax = std::max(d.router_top_k_max, 1), moe_slots = kmax + d.shared_experts;
    const bool latent_family = heavy || lighting;
    size_t o_qrot = take(latent_family ? (size_t)qd * sizeof(float) : 0);
    size_t o_kvbuf = take(latent_family ? (size_t)2 * max_kvw * sizeof(float) : 0);
    size_t o_latnew = take(lighting ? (size_t)d.latent_dim * sizeof(float) : 0);
    size_t o_branch = take(lighting ? (size_t)2 * h * sizeof(float) : 0);
    size_t o_router = take(heavy ? (size_t)(d.router_groups + d.routed_experts) * sizeof(float) : 0);
    size_t o_moe_ids = take(heavy ? (size_t)(kmax + 1) * sizeof(int) : 0);
    size_t o_moe_w = take(heavy ? (size_t)kmax * sizeof(float) : 0);
    size_t o_moe_act = take(heavy ? (size_t)moe_slots * d.ffn_dim * sizeof(float) : 0);
    size_t o_attn = take((size_t)qd * sizeof(float));
    size_t o_act = take((size_t)d.ffn_dim * sizeof(float));
    size_t o_logits = take((size_t)d.vocab_size * sizeof(float));
    size_t o_part = take(max_part * sizeof(float));
    size_t o_cnt = take((size_t)std::max(max_kvh, 1) * sizeof(unsigned));
    size_t o_pool = take((size_t)slots * h * sizeof(float));
    size_t o_anchor = take((size_t)slots * sizeof(float));
    size_t o_cbrkv = take((size_t)slots * 2 * max_kvw * sizeof(float));
    MR_TRY(device_alloc(m, off, &m->state));
    MR_HIP(hipMemset(m->state, 0, off), "clear model state");
    char *base = (char *)m->state;
    int *ints = (int *)(base + o_ints);
    m->pos_dev = ints + 0;
    m->done_dev = ints + 1;
    m->count_dev = ints + 2;
    m->eos_dev = ints + 3;
    m->cbr_skip = ints + 4;
    m->ids_dev = (int *)(base + o_ids);
    m->gen_dev = (int *)(base + o_gen);
    m->hidden = (float *)(base + o_hidden);
    m->xnorm = (float *)(base + o_xnorm);
    m->qkv = (float *)(base + o_qkv);
    m->attn = (float *)(base + o_attn);
    m->act = (float *)(base + o_act);
    m->logits = (float *)(base + o_logits);
    m->part = (float *)(base + o_part);
    m->counters = (unsigned *)(base + o_cnt);
    m->cbr_pooled = (float *)(base + o_pool);
    m->cbr_anchor = (float *)(base + o_anchor);
    m->cbr_kv = (float *)(base + o_cbrkv);
    if (latent_family) {
        m->q_rot = (float *)(base + o_qrot);
        m->kvbuf = (float *)(base + o_kvbuf);
    }
    if (lighting) {
        m->lat_new = (float *)(base + o_latnew);
        m->branch_o = (float *)(base + o_branch);
        m->branch_f = m->branch_o + h;
    }
    if (heavy) {
        m->router_out = (float *)(base + o_router);
        m->moe_ids = (int *)(base + o_moe_ids);
        m->moe_active = m->moe_ids + kmax;
        m->moe_w = (float *)(base + o_moe_w);
        m->moe_act = (float *)(base + o_moe_act);
        m->choice_rec = 1 + kmax + d.query_heads * d.global_slots;
        const size_t n = (size_t)(d.context_length + 1) * d.layers * inner * m->choice_rec;
        MR_TRY(device_alloc(m, n * sizeof(int), (void **)&m->choices));
        MR_HIP(hipMemset(m->choices, 0xff, n * sizeof(int)), "clear choice log");
    }
    MR_HIP(hipDeviceSynchronize(), "finalize model");
    MR_TRY(setup_persistent(m));
    m->finalized = true;
    m->position = 0;
    return MR_OK;
}

int mr_model_reset(mr_model *m) {
    MR_REQUIRE(m, "reset: null model");
    if (!m->finalized) return MR_OK;
    MR_HIP(hipSetDevice(m->ctx->device), "select device");
    // Caches are overwritten before they are read (ring rows by position, the
    // relay by chunk), so a reset only rewinds the position.
    MR_HIP(hipMemsetAsync(m->pos_dev, 0, 4 * sizeof(int), m->ctx->stream), "reset position");
    for (mr::Layer &L : m->layers)   // latent memory starts empty
        if (L.light) MR_HIP(hipMemsetAsync(L.light, 0, sizeof(mr::LightState), m->ctx->stream), "reset latent memory");
    if (m->persistent_ok) {   // epochs restart with the position
        MR_HIP(hipMemsetAsync(m->cells, 0, m->cell_count * sizeof(uint64_t), m->ctx->stream), "reset step cells");
        MR_HIP(hipMemsetAsync(m->sync, 0, m->sync_count * sizeof(unsigned), m->ctx->stream), "reset step counters");
        MR_HIP(hipMemsetAsync(m->words, 0, m->word_count * sizeof(unsigned), m->ctx->stream), "reset step progress");
        MR_HIP(hipMemsetAsync(m->merge_counts, 0, m->merge_count_n * sizeof(unsigned), m->ctx->stream),
               "reset attention counters");
        MR_HIP(hipMemsetAsync(m->part_cells, 0, m->part_cell_count * sizeof(uint64_t), m->ctx->stream),
               "reset attention cells");
        MR_HIP(hipMemsetAsync(m->err, 0, sizeof(int), m->ctx->stream), "reset step status");
    }
    MR_HIP(hipStreamSynchronize(m->ctx->stream), "reset");
    m->position = 0;
    if (m->timed_out) {   // persistent steps timed out: fall back to the per-layer kernels
        m->timed_out = false;
        if (m->mode == MR_STEP_PERSISTENT) m->mode = MR_STEP_GRAPH;
    }
    return MR_OK;
}

int mr_model_position(mr_model *m, int *position) {
    MR_REQUIRE(m && position, "position: null argument");
    *position = m->position;
    return MR_OK;
}

int mr_model_set_step_mode(mr_model *m, int mode) {
    MR_REQUIRE(m, "set_step_mode: null model");
    MR_REQUIRE(mode >= MR_STEP_PERSISTENT && mode <= MR_STEP_EAGER, "set_step_mode: unknown mode");
    m->mode = mode;
    if (mode != MR_STEP_GRAPH) destroy_graphs(m);
    return MR_OK;
}

int mr_model_get_step_mode(mr_model *m, int *mode) {
    MR_REQUIRE(m && mode, "get_step_mode: null argument");
    *mode = m->mode == MR_STEP_PERSISTENT && !m->persistent_ok ? MR_STEP_GRAPH : m->mode;
    return MR_OK;
}

int mr_debug_step_timeout(mr_model *m) {
    MR_REQUIRE(m, "debug_step_timeout: null model");
    m->inject_timeout = true;
    return MR_OK;
}

int mr_model_last_decode_ms(mr_model *m, float *ms) {
    MR_REQUIRE(m && ms, "last_decode_ms: null argument");
    *ms = m->last_ms;
    return MR_OK;
}

namespace {

__global__ void k_set_int(int *p, int v) { *p = v; }

constexpr int kPrefillRows = 4096;   // prompt rows per batched prefill chunk
constexpr int kRouterSlices = 8;     // K slices of heavy-medium-2.0's router GEMM

// One chunk's activations (FP32, rows of the chunk): hidden, normalized input,
// q|k|v, attended values, SwiGLU activations and, with return_all, logits;
// for heavy-medium-2.0 also the latent rows, the block scan, the block
// partials, the router logits, the routing and the expert-major gather; for
// flashlighting-2.0 the latent rows, logical row 0 of each step, its keys and
// values and partials, both branches' outputs and the chunk's plan; for
// flashnano-1.6 the pooled CBR rows, their anchors and [K | V] projections,
// and the relay partials.
struct PrefillWs {
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *att = nullptr, *act = nullptr, *lg = nullptr;
    float *lat = nullptr, *sums = nullptr, *ext = nullptr, *router = nullptr, *mw = nullptr, *xg = nullptr,
          *y = nullptr;
    int *ids = nullptr, *active = nullptr, *counts = nullptr, *offsets = nullptr, *fill = nullptr, *map = nullptr;
    int *tile_start = nullptr;   // [groups + 1] prefix sums of the groups' GEMM row tiles
    float *slot0 = nullptr, *slot0_final = nullptr, *kv0 = nullptr, *obuf = nullptr, *fbuf = nullptr,
          *merge_count = nullptr;
    int *flags = nullptr, *extra_index = nullptr, *merge_row = nullptr, *extra_pos = nullptr;
    float *cbr_scores = nullptr, *cbr_pooled = nullptr, *cbr_anchor = nullptr, *cbr_kv = nullptr;   // flashnano-1.6
    float *router_part = nullptr;   // heavy-medium-2.0: the router GEMM's K slices
    float *xn_scale = nullptr;      // heavy-medium-2.0: the normalized rows' FP16 terms, split once
    _Float16 *xn_planes = nullptr;
    float *rowscale = nullptr;   // FP16-term GEMMs: scales of the rows of A
    float *act_scale = nullptr;  // row scales of the SwiGLU output written in FP16 terms (into act)
    float *att_scale = nullptr;  // row scales of the attended values written in FP16 terms (into att)
    _Float16 *planes = nullptr;  // and its hi and lo FP16 planes
    _Float16 *kv16 = nullptr;    // attention: the attended keys and values in FP16 terms
    int kv16_rows = 0;
    float *kv16_scale = nullptr;
    unsigned *kv16_max = nullptr;
    unsigned *kv_part = nullptr;   // the K/V maxima pass's per-block partials
    int kv_part_blocks = 0;
};

int prefill_workspace(mr_model *m, int rows, bool all, PrefillWs *w) {
    const mr_model_desc &d = m->d;
    const bool heavy = d.family == MR_FAMILY_HEAVY_MEDIUM_20, light = d.family == MR_FAMILY_FLASHLIGHTING_20;
    int max_kvw = 0;
    for (const Layer &L : m->layers) max_kvw = std::max(max_kvw, L.kv_heads * d.head_dim);
    const size_t r = (size_t)rows, h = d.hidden_size, qd = (size_t)d.query_heads * d.head_dim, kvw = max_kvw;
    const size_t slots = heavy ? (size_t)d.router_top_k_max + d.shared_experts : 1;
    const size_t groups = heavy ? (size_t)d.routed_experts + d.shared_experts : 0;
    const size_t kmax = heavy ? d.router_top_k_max : 0, lat = heavy || light ? d.latent_dim : 0;
    const bool cbr = d.family == MR_FAMILY_FLASHNANO_16;
    // pooled rows: cbr_slots per CBR chunk ending inside the rows
    const size_t pr = cbr ? (size_t)(rows / d.cbr_chunk_size + 1) * d.cbr_slots : 0;
    const size_t ext = heavy || light || cbr ? r * d.query_heads * (d.head_dim + 4) : 0;
    // rows split into FP16 terms at once: a chunk, its pooled CBR rows, or its
    // rows gathered for every expert slot
    const size_t split_rows = std::max({r, pr, heavy ? r * slots : 0});
    int max_cap = 0;
    for (const Layer &L : m->layers) max_cap = std::max(max_cap, L.capacity);
    for (const Layer &L : m->layers) max_cap = std::max(max_cap, L.light_cap);
    // the attended keys and values in FP16 terms, whole 32-row tiles: heavy-medium's window
    // attention sees the window, the others up to the ring
    const int attend = heavy && d.window > 0 ? d.window : max_cap;
    w->kv16_rows = ceil_div(rows + attend, 32) * 32;
    int max_kvh = 1;
    for (const Layer &L : m->layers) max_kvh = std::max(max_kvh, L.kv_heads);
    w->kv_part_blocks = prefill_kv_max_blocks(rows + attend);
    const size_t kv16 = (size_t)w->kv16_rows * kvw * 2;   // 4 planes of halves, in floats
    struct Piece { void **ptr; size_t floats; };
    const Piece pieces[] = {
        {(void **)&w->x, r * h}, {(void **)&w->xn, r * h}, {(void **)&w->qkv, r * (qd + 2 * kvw)},
        {(void **)&w->att, r * qd}, {(void **)&w->act, r * slots * d.ffn_dim}, {(void **)&w->lg, all ? r * d.vocab_size : 0},
        {(void **)&w->lat, r * lat}, {(void **)&w->ext, ext},
        // heavy-medium-2.0
        {(void **)&w->sums, heavy ? r * 2 * kvw : 0}, {(void **)&w->router, heavy ? r * (d.router_groups + groups) : 0},
        {(void **)&w->mw, r * kmax}, {(void **)&w->xg, heavy ? r * slots * h : 0},
        {(void **)&w->router_part, heavy ? r * kRouterSlices * (d.router_groups + groups) : 0},
        {(void **)&w->xn_scale, heavy ? r : 0}, {(void **)&w->xn_planes, heavy ? r * h : 0},
        {(void **)&w->y, heavy ? r * slots * h : 0}, {(void **)&w->ids, r * kmax}, {(void **)&w->active, heavy ? r : 0},
        {(void **)&w->counts, groups}, {(void **)&w->offsets, groups}, {(void **)&w->fill, groups},
        {(void **)&w->tile_start, heavy ? groups + 1 : 0},
        {(void **)&w->map, r * kmax},
        // flashlighting-2.0
        {(void **)&w->slot0, light ? r * lat : 0}, {(void **)&w->slot0_final, light ? lat : 0},
        {(void **)&w->kv0, light ? r * 2 * kvw : 0}, {(void **)&w->obuf, light ? r * h : 0},
        {(void **)&w->fbuf, light ? r * h : 0}, {(void **)&w->merge_count, light ? r : 0},
        {(void **)&w->flags, light ? r : 0}, {(void **)&w->extra_index, light ? r : 0},
        {(void **)&w->merge_row, light ? r : 0}, {(void **)&w->extra_pos, light ? r : 0},
        // flashnano-1.6
        {(void **)&w->cbr_scores, pr * (cbr ? d.cbr_chunk_size : 0)}, {(void **)&w->cbr_pooled, pr * h}, {(void **)&w->cbr_anchor, pr}, {(void **)&w->cbr_kv, pr * 2 * kvw},
        {(void **)&w->rowscale, split_rows}, {(void **)&w->act_scale, r}, {(void **)&w->att_scale, r},
        {(void **)&w->planes, split_rows * std::max({h, qd, (size_t)d.ffn_dim})},
        {(void **)&w->kv16, kv16}, {(void **)&w->kv16_scale, 2 * kvw}, {(void **)&w->kv16_max, 2 * kvw},
        {(void **)&w->kv_part, (size_t)w->kv_part_blocks * 2 * max_kvh}};
    auto up = [](size_t floats) { return (floats + 63) & ~(size_t)63; };   // 256-byte slices
    size_t total = 0;
    for (const Piece &pc : pieces) total += up(pc.floats);
    total *= sizeof(float);
    if (total > m->pf_bytes) {
        MR_HIP(hipStreamSynchronize(m->ctx->stream), "prefill workspace");
        if (m->pf) hipFree(m->pf);
        m->pf = nullptr;
        m->pf_bytes = 0;
        MR_TRY(device_alloc(m, total, &m->pf));
        m->pf_bytes = total;
    }
    float *p = (float *)m->pf;
    for (const Piece &pc : pieces) {
        *pc.ptr = pc.floats ? (void *)p : nullptr;
        p += up(pc.floats);
    }
    return MR_OK;
}

// The latent-memory bookkeeping of positions p0 .. p0 + rows - 1, planned on
// the host: the token step's compaction (k_light_compact) depends only on the
// positions, so it is replayed here from position 0 with logical row 0 kept as
// (position, count) and the original rows as a position range.  For each step
// of the chunk: whether it sees logical row 0 as an extra row (a merged row,
// or row 0 once the window has passed it) and at which position, whether a
// merge follows it, with row 0's count and the folded row; then the state
// after the chunk.
struct LightPlan {
    std::vector<int> flags, extra_index, merge_row, extra_pos;
    std::vector<float> merge_count;
    int extra = 0, window = 0, hole = 0, init_from_arena = 0, init_slot = 0;
    LightState fin{};
    int write_slot0 = 0;
    float slot0_position = 0.0f, slot0_count = 1.0f;
};

void plan_light_chunk(const mr_model_desc &d, int cap, int p0, int rows, LightPlan &pl) {
    const int W = d.window, M = d.memory_slots;
    pl.window = M > 0 ? W + M : W;
    pl.hole = M > 0 ? W : 0;
    pl.flags.assign(rows, 0);
    pl.extra_index.assign(rows, -1);
    pl.merge_row.assign(rows, 0);
    pl.merge_count.assign(rows, 0.0f);
    LightState st{};   // as after a reset
    int lo = 0;        // position of the oldest original row in the memory
    bool merged = false;
    float P0 = 0.0f, C0 = 1.0f;   // logical row 0 when merged
    bool merged_in_chunk = false;
    for (int p = 0; p < p0 + rows; ++p) {
        const int t = p - p0;
        if (t == 0) {
            pl.init_from_arena = p0 > 0;
            pl.init_slot = st.start;
        }
        if (t >= 0 && M > 0 && (merged || lo < p - pl.window + 1)) {
            pl.flags[t] |= 1;
            pl.extra_index[t] = pl.extra++;
            pl.extra_pos.push_back(merged ? (int)P0 : lo);
        }
        const int n = st.rows + 1, overflow = std::max(0, n - W);
        st.skip_merged = 1;
        st.pending = 0;
        if (M == 0 && overflow > 0) {
            st.start = (st.start + overflow) % cap;
            st.rows = n - overflow;
            st.memory = 0;
            lo += overflow;
        } else if (overflow > M) {
            float ca, pa;
            if (merged) {
                ca = C0;
                pa = P0;
            } else {
                ca = 1.0f;
                pa = (float)lo;
                ++lo;
            }
            const float cb = 1.0f, pb = (float)lo;   // logical row 1, an original row
            const float centre = (pa * ca + pb * cb) / (ca + cb);
            if (t >= 0) {
                pl.flags[t] |= 2;
                pl.merge_count[t] = ca;
                pl.merge_row[t] = lo;
                merged_in_chunk = true;
            }
            ++lo;
            P0 = rintf(centre);
            C0 = ca + cb;
            merged = true;
            st.start = (st.start + 1) % cap;
            st.memory = M;
            st.skip_merged = 0;
            st.pending = 1;
            st.merged_slot = st.start;
            st.merged_pos = (int)P0;
        } else {
            st.rows = n;
            st.memory = overflow;
        }
    }
    pl.fin = st;
    pl.write_slot0 = merged && merged_in_chunk;
    pl.slot0_position = P0;
    pl.slot0_count = C0;
}

// flashnano-1.6 over the chunk's rows (model.py:118-144): the relay rows of
// every CBR chunk that ends at a position p0 .. p0 + T - 1, all at once (a
// chunk's pooled rows depend only on its normalized layer inputs, w.xn here
// and the pending buffer before p0), then the pending buffer as the token
// loop leaves it.
int cbr_layer_rows(mr_model *m, Layer &L, const PrefillWs &w, int p0, int T) {
    const mr_model_desc &d = m->d;
    hipStream_t s = m->ctx->stream;
    const int h = d.hidden_size, hd = d.head_dim, qd = d.query_heads * hd, kvw = L.kv_heads * hd;
    const int chunk = d.cbr_chunk_size, slots = d.cbr_slots;
    const int first = p0 / chunk, nc = (p0 + T) / chunk - first;   // chunk c ends at (c + 1) * chunk - 1
    if (nc > 0) {
        k_cbr_scores_rows<<<nc * chunk, 256, 0, s>>>(w.xn, h, L.pending, L.cbr_queries, w.cbr_scores, p0, first,
                                                      chunk, slots, h);
        MR_LAUNCHED("enqueue cbr scores");
        k_cbr_mix_rows<<<dim3(nc, slots, ceil_div(h, 256)), 256, (size_t)(chunk + 8) * sizeof(float), s>>>(
            w.xn, h, L.pending, w.cbr_scores, w.cbr_pooled, w.cbr_anchor, p0, first, chunk, slots, h);
        MR_LAUNCHED("enqueue cbr pooling");
        GemmArgs kv;   // pooled rows through [Wk; Wv], the rows after Wq of the fused projection
        kv.a = w.cbr_pooled; kv.lda = h; kv.dtype = L.qkv.dtype;
        kv.w = (const char *)L.qkv.ptr + (size_t)qd * h * dtype_bytes(L.qkv.dtype);
        kv.c = w.cbr_kv; kv.ldc = 2 * kvw; kv.m = nc * slots; kv.n = 2 * kvw; kv.k = h;
        kv.wscale = L.qkv.f16_scale; kv.ascale = w.rowscale; kv.ahl_ws = w.planes;
        if (L.qkv.f16) kv.wh = (const _Float16 *)L.qkv.f16 + (size_t)qd * h;
        MR_TRY(launch_gemm(s, GEMM_STORE, kv));
        k_cbr_finish_rows<<<nc * slots, 256, (size_t)kvw * sizeof(float), s>>>(
            w.cbr_kv, w.cbr_anchor, L.k_norm.f(), d.norm_eps, m->rope, d.split_half_rope, L.relay_k, L.relay_v,
            first, slots, L.kv_heads, hd);
        MR_LAUNCHED("enqueue cbr finish rows");
    }
    k_cbr_pending_rows<<<std::min(T, chunk), 256, 0, s>>>(w.xn, h, L.pending, p0, T, chunk, h);
    MR_LAUNCHED("enqueue cbr pending rows");
    return MR_OK;
}

// One GQA layer over the chunk's rows (model.py:95-116, 264-266).
int gqa_layer_rows(mr_model *m, Layer &L, const PrefillWs &w, int p0, int T) {
    const mr_model_desc &d = m->d;
    hipStream_t s = m->ctx->stream;
    const int h = d.hidden_size, hd = d.head_dim, qd = d.query_heads * hd, ffn = d.ffn_dim;
    const int kvw = L.kv_heads * hd, ld = qd + 2 * kvw;
    GemmArgs g;
    g.a = w.xn; g.lda = h; g.w = L.qkv.ptr; g.dtype = L.qkv.dtype; g.c = w.qkv; g.ldc = ld;
    g.m = T; g.n = ld; g.k = h; g.wscale = L.qkv.f16_scale; g.wh = L.qkv.f16; g.ascale = w.rowscale; g.ahl_ws = w.planes;
    // the normalized rows go straight into the FP16-term GEMM's A workspace
    // (flashnano-1.6 pools them in FP32 first)
    const bool cbr = d.family == MR_FAMILY_FLASHNANO_16;
    g.a_split = g.wscale > 0.0f && !cbr && rms_split_fits(h);
    if (g.a_split) MR_TRY(launch_rms_rows_split(s, w.x, h, L.a_norm.f(), d.norm_eps, h, w.rowscale, w.planes, T));
    else MR_TRY(launch_rms_rows(s, w.x, h, L.a_norm.f(), d.norm_eps, h, w.xn, h, T));
    if (cbr) MR_TRY(cbr_layer_rows(m, L, w, p0, T));
    MR_TRY(launch_gemm(s, GEMM_STORE, g));
    MR_TRY(launch_qk_rows(s, w.qkv, ld, T, p0, d.query_heads, L.kv_heads, hd,
                          d.qk_norm ? L.q_norm.f() : nullptr, d.qk_norm ? L.k_norm.f() : nullptr,
                          d.norm_eps, d.qk_norm, m->rope, d.split_half_rope));
    PrefillAttnArgs a;
    a.qkv = w.qkv; a.ld = ld; a.ring_k = L.ring_k; a.ring_v = L.ring_v; a.cap = L.capacity;
    a.out = w.att; a.ldo = qd; a.p0 = p0; a.rows = T;
    a.heads = d.query_heads; a.kv_heads = L.kv_heads; a.d = hd; a.inv_root = 1.0f / sqrtf((float)hd);
    a.kv16 = w.kv16; a.kv16_rows = w.kv16_rows; a.kv16_scale = w.kv16_scale; a.kv16_max = w.kv16_max;
    a.kv_part = w.kv_part; a.kv_part_blocks = w.kv_part_blocks;
    if (cbr) {   // the relay rows join every row's softmax as its extra partial
        RelayPartialArgs r;
        r.qkv = w.qkv; r.ld = ld; r.relay_k = L.relay_k; r.relay_v = L.relay_v; r.ext = w.ext;
        r.p0 = p0; r.rows = T; r.heads = d.query_heads; r.kv_heads = L.kv_heads; r.d = hd;
        r.chunk = d.cbr_chunk_size; r.slots = d.cbr_slots; r.inv_root = a.inv_root;
        MR_TRY(launch_relay_partial(s, r));
        a.ext = w.ext;
    }
    // the attended values straight into the O projection's FP16 terms (att
    // holds T x qd floats, the same bytes as its two planes of halves)
    const bool att_split = !a.ext && L.o.dtype == MR_BF16 && L.o.f16_scale > 0.0f && prefill_attention_presplit(a);
    if (att_split) {
        a.out_hl = (_Float16 *)w.att;
        a.out_scale = w.att_scale;
    }
    MR_TRY(launch_prefill_attention(s, a));
    MR_TRY(launch_ring_store(s, w.qkv, ld, qd, kvw, L.ring_k, L.ring_v, L.capacity, p0, T));
    GemmArgs o;
    o.a = w.att; o.lda = qd; o.w = L.o.ptr; o.dtype = L.o.dtype; o.c = w.x; o.ldc = h;
    o.m = T; o.n = h; o.k = qd; o.scale = d.residual_scale; o.wscale = L.o.f16_scale; o.wh = L.o.f16;
    o.ascale = att_split ? w.att_scale : w.rowscale;
    o.ahl_ws = att_split ? (_Float16 *)w.att : w.planes;
    o.a_split = att_split;
    MR_TRY(launch_gemm(s, GEMM_RESIDUAL, o));
    GemmArgs gu;
    gu.a = w.xn; gu.lda = h; gu.w = L.ffn.gate.ptr; gu.w2 = L.ffn.up.ptr; gu.dtype = L.ffn.gate.dtype;
    gu.c = w.act; gu.ldc = ffn; gu.m = T; gu.n = ffn; gu.k = h;
    gu.wscale = L.ffn.gate.f16_scale; gu.wh = L.ffn.gate.f16; gu.wh2 = L.ffn.up.f16; gu.ascale = w.rowscale;
    gu.ahl_ws = w.planes;
    gu.a_split = gu.wscale > 0.0f && rms_split_fits(h);
    // the SwiGLU output straight into the down projection's FP16 terms (act
    // holds T x ffn floats, the same bytes as its two planes of halves)
    const bool act_split = gu.a_split && act_split_fits(L.ffn, h);
    if (act_split) {
        gu.c_hl = (_Float16 *)w.act;
        gu.c_scale = w.act_scale;
    }
    if (gu.a_split)
        MR_TRY(launch_rms_rows_split(s, w.x, h, L.f_norm.f(), d.norm_eps, h, w.rowscale, w.planes, T,
                                     L.ffn.gate.row_norm, L.ffn.up.row_norm, act_split ? w.act_scale : nullptr));
    else MR_TRY(launch_rms_rows(s, w.x, h, L.f_norm.f(), d.norm_eps, h, w.xn, h, T));
    MR_TRY(launch_gemm(s, GEMM_SWIGLU, gu));
    GemmArgs dn;
    dn.a = w.act; dn.lda = ffn; dn.w = L.ffn.down.ptr; dn.dtype = L.ffn.down.dtype; dn.c = w.x; dn.ldc = h;
    dn.m = T; dn.n = h; dn.k = ffn; dn.scale = d.residual_scale; dn.wscale = L.ffn.down.f16_scale;
    dn.wh = L.ffn.down.f16;
    dn.ascale = act_split ? w.act_scale : w.rowscale;
    dn.ahl_ws = act_split ? (_Float16 *)w.act : w.planes;
    dn.a_split = act_split;
    return launch_gemm(s, GEMM_RESIDUAL, dn);
}

// One heavy-medium-2.0 layer over the chunk's rows: every inner-loop pass's
// sparse attention and MoE (model.py:192-255, 259-263) with the token step's
// per-position semantics.  Keys and values go to the pass's ring first; the
// block scan gives every row its block sums as of its own position, so each
// row scores and chooses blocks exactly as its token step would; the window
// rows and the chosen blocks' partial meet in one softmax.  The experts run as
// two grouped GEMMs over the rows routed to them.
int heavy_layer_rows(mr_model *m, Layer &L, int li, const PrefillWs &w, int p0, int T) {
    const mr_model_desc &d = m->d;
    hipStream_t s = m->ctx->stream;
    const int h = d.hidden_size, hd = d.head_dim, qd = d.query_heads * hd, ffn = d.ffn_dim, lat = d.latent_dim;
    const int kvw = L.kv_heads * hd, ld = qd + 2 * kvw, inner = d.inner_loop_steps;
    const int blocks = ceil_div(d.context_length, d.global_block_size), kmax = d.router_top_k_max;
    const int E = d.routed_experts, S = d.shared_experts, groups = E + S, R = d.router_groups + E;
    for (int loop = 0; loop < inner; ++loop) {
        float *ring_k = L.ring_k + (size_t)loop * d.context_length * kvw;
        float *ring_v = L.ring_v + (size_t)loop * d.context_length * kvw;
        float *bsum_k = L.bsum_k + (size_t)loop * blocks * kvw, *bsum_v = L.bsum_v + (size_t)loop * blocks * kvw;
        int *choice = m->choices + ((size_t)li * inner + loop) * m->choice_rec;
        const int choice_stride = d.layers * inner * m->choice_rec;
        GemmArgs q;   // the Q rows of the packed [Wq; Wlatent]
        q.a = w.xn; q.lda = h; q.w = L.qkv.ptr; q.dtype = L.qkv.dtype; q.c = w.qkv; q.ldc = ld;
        q.m = T; q.n = qd; q.k = h;
        q.wscale = L.qkv.f16_scale; q.wh = L.qkv.f16; q.ascale = w.rowscale; q.ahl_ws = w.planes;
        // the normalized rows go straight into the FP16-term GEMMs' A workspace
        q.a_split = q.wscale > 0.0f && rms_split_fits(h);
        if (q.a_split) MR_TRY(launch_rms_rows_split(s, w.x, h, L.a_norm.f(), d.norm_eps, h, w.rowscale, w.planes, T));
        else MR_TRY(launch_rms_rows(s, w.x, h, L.a_norm.f(), d.norm_eps, h, w.xn, h, T));
        MR_TRY(launch_gemm(s, GEMM_STORE, q));
        GemmArgs lt = q;   // its latent rows (the same A)
        lt.w = (const char *)L.qkv.ptr + (size_t)qd * h * dtype_bytes(L.qkv.dtype); lt.c = w.lat; lt.ldc = lat;
        lt.n = lat;
        if (L.qkv.f16) lt.wh = (const _Float16 *)L.qkv.f16 + (size_t)qd * h;
        MR_TRY(launch_gemm(s, GEMM_STORE, lt));
        GemmArgs kv;   // latent -> [K | V] beside the queries
        kv.a = w.lat; kv.lda = lat; kv.w = L.kv_up.ptr; kv.dtype = L.kv_up.dtype; kv.c = w.qkv + qd; kv.ldc = ld;
        kv.m = T; kv.n = 2 * kvw; kv.k = lat;
        kv.wscale = L.kv_up.f16_scale; kv.wh = L.kv_up.f16; kv.ascale = w.rowscale; kv.ahl_ws = w.planes;
        MR_TRY(launch_gemm(s, GEMM_STORE, kv));
        MR_TRY(launch_qk_rows(s, w.qkv, ld, T, p0, d.query_heads, L.kv_heads, hd, nullptr, nullptr, 1e-6f, 1,
                              m->rope, d.split_half_rope));
        MR_TRY(launch_ring_store(s, w.qkv, ld, qd, kvw, ring_k, ring_v, d.context_length, p0, T));
        HeavyScanArgs sc;
        sc.ring_k = ring_k; sc.ring_v = ring_v; sc.bsum_k = bsum_k; sc.bsum_v = bsum_v; sc.sums = w.sums;
        sc.p0 = p0; sc.rows = T; sc.kvw = kvw; sc.block = d.global_block_size;
        MR_TRY(launch_heavy_scan(s, sc));
        HeavySelectArgs se;
        se.qkv = w.qkv; se.ld = ld; se.bsum_k = bsum_k; se.bsum_v = bsum_v; se.sums = w.sums; se.ext = w.ext;
        se.choice = choice; se.choice_stride = choice_stride; se.choice_blocks = 1 + kmax;
        se.p0 = p0; se.rows = T; se.heads = d.query_heads; se.kv_heads = L.kv_heads; se.d = hd;
        se.block = d.global_block_size; se.slots = d.global_slots; se.context = d.context_length;
        se.slope = d.block_slope;
        MR_TRY(launch_heavy_select(s, se));
        PrefillAttnArgs a;
        a.qkv = w.qkv; a.ld = ld; a.ring_k = ring_k; a.ring_v = ring_v; a.cap = d.context_length;
        a.window = d.window; a.ext = w.ext;
        a.out = w.att; a.ldo = qd; a.p0 = p0; a.rows = T;
        a.heads = d.query_heads; a.kv_heads = L.kv_heads; a.d = hd; a.inv_root = 1.0f / sqrtf((float)hd);
        a.kv16 = w.kv16; a.kv16_rows = w.kv16_rows; a.kv16_scale = w.kv16_scale; a.kv16_max = w.kv16_max;
        a.kv_part = w.kv_part; a.kv_part_blocks = w.kv_part_blocks;
        MR_TRY(launch_prefill_attention(s, a));
        GemmArgs o;   // hidden += step_scale * Wo . attended
        o.a = w.att; o.lda = qd; o.w = L.o.ptr; o.dtype = L.o.dtype; o.c = w.x; o.ldc = h;
        o.m = T; o.n = h; o.k = qd; o.scale = d.heavy_step_scale;
        o.wscale = L.o.f16_scale; o.wh = L.o.f16; o.ascale = w.rowscale; o.ahl_ws = w.planes;
        MR_TRY(launch_gemm(s, GEMM_RESIDUAL, o));
        MR_TRY(launch_rms_rows(s, w.x, h, L.f_norm.f(), d.norm_eps, h, w.xn, h, T));
        GemmArgs r;   // [Wcoarse; Wfine], K in slices: its R columns fill few tiles
        r.a = w.xn; r.lda = h; r.w = L.router.ptr; r.dtype = L.router.dtype; r.c = w.router; r.ldc = R;
        r.m = T; r.n = R; r.k = h;
        MR_TRY(launch_gemm_split(s, r, kRouterSlices, w.router_part));
        MoeRowsArgs mr_;
        MoeArgs &e = mr_.a;
        e.router = w.router;
        e.coarse_bias = L.router_coarse_bias.f(); e.group_bias = L.group_bias.f();
        e.fine_bias = L.router_fine_bias.f(); e.expert_bias = L.expert_bias.f();
        e.x = w.xn; e.dtype = L.experts[0].gate.dtype;
        e.ids = w.ids; e.weights = w.mw; e.active = w.active;
        e.choice = choice; e.choice_stride = choice_stride;
        e.experts = E; e.groups = d.router_groups; e.kmin = d.router_top_k_min; e.kmax = kmax;
        e.shared = S; e.ffn = ffn; e.h = h;
        e.inv_temperature_div = d.router_temperature;
        e.log_experts = std::max((float)std::log((double)E), 1.0f);
        e.shared_scale = d.heavy_shared_scale; e.scale = d.heavy_step_scale;
        mr_.rows = T; mr_.p0 = p0;
        mr_.counts = w.counts; mr_.offsets = w.offsets; mr_.fill = w.fill; mr_.map = w.map; mr_.xg = w.xg;
        mr_.tile_start = w.tile_start; mr_.tile_rows = kGemmRowTile;
        const bool f16 = L.expert_tab_h != nullptr;   // FP16 terms: the experts' copies and scales
        const int rows = T * (kmax + S);   // the gathered rows' capacity (routed slots, then shared)
        // FP16 terms: the T rows split once and their terms gathered, not the gathered rows split
        const bool gsplit = f16 && h % 8 == 0 && w.xn_planes;
        if (gsplit) {
            MR_TRY(launch_row_split(s, w.xn, h, T, h, w.xn_scale, w.xn_planes));
            mr_.x_scale = w.xn_scale; mr_.x_planes = w.xn_planes;
            mr_.xg_scale = w.rowscale; mr_.xg_planes = w.planes; mr_.capacity = rows;
        }
        MR_TRY(launch_moe_route_rows(s, mr_));
        GemmGroups gg;
        gg.offset = w.offsets; gg.count = w.counts; gg.groups = groups; gg.max_rows = T;
        // every gathered row is in one group: at most rows / 128 tiles plus a partial one a group
        gg.row_tile_start = w.tile_start; gg.row_tiles = ceil_div(T * (kmax + S), kGemmRowTile) + groups;
        gg.w = L.expert_tab; gg.w2 = L.expert_tab + groups;
        if (f16) { gg.wh = L.expert_tab_h; gg.wh2 = L.expert_tab_h + groups; gg.wscale = L.expert_scale; }
        GemmArgs gu;
        gu.a = w.xg; gu.lda = h; gu.dtype = e.dtype; gu.c = w.act; gu.ldc = ffn; gu.n = ffn; gu.k = h;
        gu.m = rows; gu.ascale = w.rowscale; gu.ahl_ws = w.planes; gu.a_split = gsplit;
        MR_TRY(launch_gemm_grouped(s, GEMM_SWIGLU, gu, gg));
        gg.w = L.expert_tab + 2 * groups;
        gg.w2 = nullptr;
        if (f16) { gg.wh = L.expert_tab_h + 2 * groups; gg.wh2 = nullptr; gg.wscale = L.expert_scale + 2 * groups; }
        GemmArgs dn;
        dn.a = w.act; dn.lda = ffn; dn.dtype = e.dtype; dn.c = w.y; dn.ldc = h; dn.n = h; dn.k = ffn;
        dn.m = rows; dn.ascale = w.rowscale; dn.ahl_ws = w.planes;
        MR_TRY(launch_gemm_grouped(s, GEMM_STORE, dn, gg));
        MR_TRY(launch_moe_combine_rows(s, mr_, w.y, w.x));
    }
    return MR_OK;
}

// One flashlighting-2.0 layer over the chunk's rows (model.py:146-190,
// 271-279).  The queries, the new latent rows and their keys and values come
// from GEMMs; logical row 0 of every step that sees it as an extra row comes
// from the merge recurrence, with its keys and values by a GEMM at its
// planned positions; the attention is the windowed one over the original
// rows (the ring caches for rows before the chunk) with the extra row's
// partial; the FFN branch and the gated residual follow; last, the chunk's
// rows and the planned state go to the token step's ring.
int light_layer_rows(mr_model *m, Layer &L, const PrefillWs &w, const LightPlan &pl, int p0, int T) {
    const mr_model_desc &d = m->d;
    hipStream_t s = m->ctx->stream;
    const int h = d.hidden_size, hd = d.head_dim, qd = d.query_heads * hd, ffn = d.ffn_dim, lat = d.latent_dim;
    const int kvw = L.kv_heads * hd, ld = qd + 2 * kvw;
    // the normalized rows straight into FP16 terms where the Q/latent and FFN
    // GEMMs take them (BF16 weights with FP16 copies), with the scales of the
    // SwiGLU output for the down projection's FP16 terms
    const bool xn_split = L.qkv.dtype == MR_BF16 && L.qkv.f16_scale > 0.0f && rms_split_fits(h);
    const bool gu_split = xn_split && L.ffn.gate.dtype == MR_BF16 && L.ffn.gate.f16_scale > 0.0f;
    const bool act_split = gu_split && act_split_fits(L.ffn, h);
    if (!gu_split) MR_TRY(launch_rms_rows(s, w.x, h, L.a_norm.f(), d.norm_eps, h, w.xn, h, T));
    if (xn_split)
        MR_TRY(launch_rms_rows_split(s, w.x, h, L.a_norm.f(), d.norm_eps, h, w.rowscale, w.planes, T,
                                     L.ffn.gate.row_norm, L.ffn.up.row_norm, act_split ? w.act_scale : nullptr));
    // FP16-term GEMMs where the weights have FP16 copies (BF16 weights)
    auto f16 = [&](GemmArgs &g, const Weight &wt, size_t row0 = 0) {
        g.wscale = wt.f16_scale;
        g.wh = wt.f16 ? (const void *)((const _Float16 *)wt.f16 + row0 * wt.cols) : nullptr;
        g.ascale = w.rowscale;
        g.ahl_ws = w.planes;
    };
    GemmArgs q;   // the Q rows of the packed [Wq; Wlatent]
    q.a = w.xn; q.lda = h; q.w = L.qkv.ptr; q.dtype = L.qkv.dtype; q.c = w.qkv; q.ldc = ld;
    q.m = T; q.n = qd; q.k = h;
    f16(q, L.qkv);
    q.a_split = xn_split;
    MR_TRY(launch_gemm(s, GEMM_STORE, q));
    GemmArgs lt = q;   // its latent rows, then RMSNorm with latent_norm in place
    lt.w = (const char *)L.qkv.ptr + (size_t)qd * h * dtype_bytes(L.qkv.dtype); lt.c = w.lat; lt.ldc = lat;
    lt.n = lat;
    f16(lt, L.qkv, qd);
    // the latent rows and the FFN branch (the same input) reuse the normalized
    // rows' FP16 terms before anything else splits
    lt.a_split = xn_split;
    MR_TRY(launch_gemm(s, GEMM_STORE, lt));
    GemmArgs gu;   // the FFN branch reads the same normalized input
    gu.a = w.xn; gu.lda = h; gu.w = L.ffn.gate.ptr; gu.w2 = L.ffn.up.ptr; gu.dtype = L.ffn.gate.dtype;
    gu.c = w.act; gu.ldc = ffn; gu.m = T; gu.n = ffn; gu.k = h;
    f16(gu, L.ffn.gate);
    gu.wh2 = L.ffn.up.f16;
    gu.a_split = gu_split;
    if (act_split) {
        gu.c_hl = (_Float16 *)w.act;
        gu.c_scale = w.act_scale;
    }
    MR_TRY(launch_gemm(s, GEMM_SWIGLU, gu));
    MR_TRY(launch_rms_rows(s, w.lat, lat, L.latent_norm.f(), d.norm_eps, lat, w.lat, lat, T));
    GemmArgs kv;   // [Wk; Wv] . latent beside the queries
    kv.a = w.lat; kv.lda = lat; kv.w = L.kv_up.ptr; kv.dtype = L.kv_up.dtype; kv.c = w.qkv + qd; kv.ldc = ld;
    kv.m = T; kv.n = 2 * kvw; kv.k = lat;
    f16(kv, L.kv_up);
    MR_TRY(launch_gemm(s, GEMM_STORE, kv));
    MR_TRY(launch_qk_rows(s, w.qkv, ld, T, p0, d.query_heads, L.kv_heads, hd, L.q_norm.f(), L.k_norm.f(), d.norm_eps,
                          1, m->rope, d.split_half_rope));
    LightRowsArgs r;
    r.lat = w.lat; r.arena = L.arena; r.positions = L.positions; r.counts = L.counts;
    r.slot0 = w.slot0; r.slot0_final = w.slot0_final; r.flags = w.flags; r.extra_index = w.extra_index;
    r.merge_count = w.merge_count; r.merge_row = w.merge_row; r.init_from_arena = pl.init_from_arena;
    r.init_slot = pl.init_slot; r.p0 = p0; r.rows = T; r.latent = lat; r.cap = L.light_cap;
    r.merged = w.obuf;   // free until the O projection
    r.row0_ws = w.fbuf;  // free until the FFN's down projection
    MR_REQUIRE(light_row0_ws_floats(T, d.latent_dim) <= (size_t)T * h, "latent rows: workspace too small");
    if (d.memory_slots > 0) MR_TRY(launch_light_slot0(s, r));   // reads the ring before this chunk writes it
    if (pl.extra > 0) {
        GemmArgs k0 = kv;   // logical row 0's keys and values
        k0.a = w.slot0; k0.c = w.kv0; k0.ldc = 2 * kvw; k0.m = pl.extra;
        MR_TRY(launch_gemm(s, GEMM_STORE, k0));
        MR_TRY(launch_k_rows_at(s, w.kv0, 2 * kvw, pl.extra, w.extra_pos, L.kv_heads, hd, L.k_norm.f(), d.norm_eps,
                                m->rope, d.split_half_rope));
        MR_TRY(launch_light_extra(s, w.qkv, ld, w.kv0, w.extra_index, w.ext, T, d.query_heads, L.kv_heads, hd));
    }
    PrefillAttnArgs a;
    a.qkv = w.qkv; a.ld = ld; a.ring_k = L.kcache; a.ring_v = L.vcache; a.cap = L.light_cap;
    a.window = pl.window; a.hole = pl.hole; a.ext = pl.extra > 0 ? w.ext : nullptr;
    a.out = w.att; a.ldo = qd; a.p0 = p0; a.rows = T;
    a.heads = d.query_heads; a.kv_heads = L.kv_heads; a.d = hd; a.inv_root = 1.0f / sqrtf((float)hd);
    a.kv16 = w.kv16; a.kv16_rows = w.kv16_rows; a.kv16_scale = w.kv16_scale; a.kv16_max = w.kv16_max;
    a.kv_part = w.kv_part; a.kv_part_blocks = w.kv_part_blocks;
    // without an extra partial, the attended values straight into the O projection's FP16 terms
    const bool att_split = !a.ext && L.o.dtype == MR_BF16 && L.o.f16_scale > 0.0f && prefill_attention_presplit(a);
    if (att_split) {
        a.out_hl = (_Float16 *)w.att;
        a.out_scale = w.att_scale;
    }
    MR_TRY(launch_prefill_attention(s, a));
    GemmArgs o;
    o.a = w.att; o.lda = qd; o.w = L.o.ptr; o.dtype = L.o.dtype; o.c = w.obuf; o.ldc = h; o.m = T; o.n = h; o.k = qd;
    f16(o, L.o);
    if (att_split) {
        o.ascale = w.att_scale;
        o.ahl_ws = (_Float16 *)w.att;
        o.a_split = true;
    }
    MR_TRY(launch_gemm(s, GEMM_STORE, o));
    GemmArgs dn;
    dn.a = w.act; dn.lda = ffn; dn.w = L.ffn.down.ptr; dn.dtype = L.ffn.down.dtype; dn.c = w.fbuf; dn.ldc = h;
    dn.m = T; dn.n = h; dn.k = ffn;
    f16(dn, L.ffn.down);
    if (act_split) {
        dn.ascale = w.act_scale;
        dn.ahl_ws = (_Float16 *)w.act;
        dn.a_split = true;
    }
    MR_TRY(launch_gemm(s, GEMM_STORE, dn));
    MR_TRY(launch_light_residual(s, w.x, w.obuf, w.fbuf, L.attention_gate.f(), L.ffn_gate.f(), d.residual_scale,
                                 T * h, nullptr));
    MR_TRY(launch_ring_store(s, w.qkv, ld, qd, kvw, L.kcache, L.vcache, L.light_cap, p0, T));
    MR_TRY(launch_light_store_rows(s, r));
    return launch_light_finish(s, r, L.light, pl.fin, pl.write_slot0, pl.slot0_position, pl.slot0_count);
}

// Whether a prompt of this model can take the batched path: its family, and
// the widths the GEMM tiles and row kernels take (other geometries, such as
// the reference's micro test models, take the token loop).
bool batched_prefill_ok(const mr_model *m) {
    const mr_model_desc &d = m->d;
    if (!batched_prefill_family(d.family)) return false;
    const int hd = d.head_dim, qd = d.query_heads * hd;
    if (d.hidden_size % 8 || d.ffn_dim % 8 || qd % 8 || hd % 4 || hd > 128) return false;
    if (d.family == MR_FAMILY_HEAVY_MEDIUM_20)
        return (hd == 32 || hd == 64 || hd == 128) && d.latent_dim % 8 == 0 && d.shared_experts <= 8 &&
               d.global_slots <= 32 && ceil_div(d.context_length, d.global_block_size) * 8 + hd * 4 <= 64 * 1024;
    if (d.family == MR_FAMILY_FLASHLIGHTING_20) return d.latent_dim % 8 == 0;
    return true;
}

int prefill_batched(mr_model *m, int n, bool all, float *logits) {
    const mr_model_desc &d = m->d;
    hipStream_t s = m->ctx->stream;
    const bool heavy = d.family == MR_FAMILY_HEAVY_MEDIUM_20, light = d.family == MR_FAMILY_FLASHLIGHTING_20;
    const int h = d.hidden_size, V = d.vocab_size;
    const int chunk = std::min(n, kPrefillRows);
    PrefillWs w;
    MR_TRY(prefill_workspace(m, chunk, all, &w));
    const Weight &head = d.tie_embeddings ? m->embed : m->output;
    for (int start = 0; start < n; start += chunk) {
        const int T = std::min(chunk, n - start), p0 = m->position + start;
        MR_TRY(launch_embed_rows(s, m->embed.ptr, m->embed.dtype, m->ids_dev, p0, T, w.x, h));
        LightPlan plan;
        if (light) {   // one plan serves every layer (the bookkeeping depends only on positions)
            plan = LightPlan();
            plan_light_chunk(d, m->layers[0].light_cap, p0, T, plan);
            MR_HIP(hipMemcpyAsync(w.flags, plan.flags.data(), T * sizeof(int), hipMemcpyHostToDevice, s), "upload plan");
            MR_HIP(hipMemcpyAsync(w.extra_index, plan.extra_index.data(), T * sizeof(int), hipMemcpyHostToDevice, s),
                   "upload plan");
            MR_HIP(hipMemcpyAsync(w.merge_row, plan.merge_row.data(), T * sizeof(int), hipMemcpyHostToDevice, s),
                   "upload plan");
            MR_HIP(hipMemcpyAsync(w.merge_count, plan.merge_count.data(), T * sizeof(float), hipMemcpyHostToDevice, s),
                   "upload plan");
            if (plan.extra)
                MR_HIP(hipMemcpyAsync(w.extra_pos, plan.extra_pos.data(), plan.extra * sizeof(int),
                                      hipMemcpyHostToDevice, s),
                       "upload plan");
            MR_HIP(hipStreamSynchronize(s), "upload plan");   // the host vectors go out of scope
        }
        for (int li = 0; li < d.layers; ++li) {
            Layer &L = m->layers[li];
            MR_TRY(heavy   ? heavy_layer_rows(m, L, li, w, p0, T)
                   : light ? light_layer_rows(m, L, w, plan, p0, T)
                           : gqa_layer_rows(m, L, w, p0, T));
        }
        if (all) {
            MR_TRY(launch_rms_rows(s, w.x, h, m->norm.f(), d.norm_eps, h, w.xn, h, T));
            GemmArgs lm;
            lm.a = w.xn; lm.lda = h; lm.w = head.ptr; lm.dtype = head.dtype; lm.c = w.lg; lm.ldc = V;
            lm.m = T; lm.n = V; lm.k = h;
            MR_TRY(launch_gemm(s, GEMM_STORE, lm));
            if (logits)
                MR_HIP(hipMemcpyAsync(logits + (size_t)start * V, w.lg, (size_t)T * V * sizeof(float),
                                      hipMemcpyDeviceToHost, s),
                       "read logits");
            if (start + T == n)
                MR_HIP(hipMemcpyAsync(m->logits, w.lg + (size_t)(T - 1) * V, (size_t)V * sizeof(float),
                                      hipMemcpyDeviceToDevice, s),
                       "keep last logits");
        } else if (start + T == n) {
            MR_HIP(hipMemcpyAsync(m->hidden, w.x + (size_t)(T - 1) * h, (size_t)h * sizeof(float),
                                  hipMemcpyDeviceToDevice, s),
                   "keep last hidden row");
            MR_TRY(launch_lm_head(m));
            if (logits)
                MR_HIP(hipMemcpyAsync(logits, m->logits, (size_t)V * sizeof(float), hipMemcpyDeviceToHost, s),
                       "read logits");
        }
    }
    k_set_int<<<1, 1, 0, s>>>(m->pos_dev, m->position + n);
    MR_LAUNCHED("enqueue position update");
    MR_HIP(hipStreamSynchronize(s), "batched prefill");
    MR_TRY(check_step_error(m));
    m->position += n;
    return MR_OK;
}

}  // namespace

int mr_model_forward(mr_model *m, const int32_t *ids, int n, int flags, float *logits) {
    MR_TRY(check_ctx(m, "forward"));
    MR_REQUIRE(ids && n > 0, "forward: input_ids must be a non-empty 1D integer sequence");
    const mr_model_desc &d = m->d;
    for (int i = 0; i < n; ++i)
        MR_REQUIRE(ids[i] >= 0 && ids[i] < d.vocab_size, "forward: input token is outside the vocabulary");
    if (m->position + n > d.context_length)
        return fail(MR_ERR_INVALID, "input would exceed context_length; reset or allocate a larger context");
    hipStream_t s = m->ctx->stream;
    MR_HIP(hipMemcpyAsync(m->ids_dev + m->position, ids, (size_t)n * sizeof(int), hipMemcpyHostToDevice, s),
           "upload token ids");
    MR_HIP(hipMemsetAsync(m->done_dev, 0, sizeof(int), s), "clear stop flag");
    const bool all = (flags & MR_FWD_RETURN_ALL) != 0;
    if ((flags & MR_FWD_BATCHED) && n > 1 && batched_prefill_ok(m)) return prefill_batched(m, n, all, logits);
    for (int i = 0; i < n; ++i) {
        const bool want = all || i == n - 1;
        MR_TRY(run_step(m, want ? STEP_LOGITS : STEP_PLAIN));
        if (want && logits) {
            float *dst = logits + (all ? (size_t)i * d.vocab_size : 0);
            MR_HIP(hipMemcpyAsync(dst, m->logits, (size_t)d.vocab_size * sizeof(float), hipMemcpyDeviceToHost, s),
                   "read logits");
        }
    }
    MR_HIP(hipStreamSynchronize(s), "forward");
    MR_TRY(check_step_error(m));
    m->position += n;
    return MR_OK;
}

int mr_model_generate_greedy(mr_model *m, int max_new, int eos, int32_t *tokens, int *produced) {
    MR_TRY(check_ctx(m, "generate"));
    MR_REQUIRE(tokens && produced && max_new >= 1, "generate: bad arguments");
    MR_REQUIRE(m->position >= 1, "generate: call forward first");
    MR_REQUIRE(m->position + max_new - 1 <= m->d.context_length, "generate: exceeds context_length");
    hipStream_t s = m->ctx->stream;
    int init[3] = {0, 0, eos};   // done, count, eos
    MR_HIP(hipMemcpyAsync(m->done_dev, init, sizeof(init), hipMemcpyHostToDevice, s), "arm greedy loop");
    // Choice from the logits of the last forward, without a step.
    k_argmax<<<1, 1024, 0, s>>>(m->logits, m->d.vocab_size, m->pos_dev, m->done_dev, m->ids_dev, m->gen_dev,
                                m->count_dev, m->eos_dev, 0);
    MR_LAUNCHED("enqueue argmax");
    hipEvent_t e0, e1;
    MR_HIP(hipEventCreate(&e0), "create event");
    MR_HIP(hipEventCreate(&e1), "create event");
    hipEventRecord(e0, s);
    int rc = MR_OK;
    for (int i = 1; i < max_new && rc == MR_OK; ++i) rc = run_step(m, STEP_GREEDY);
    hipEventRecord(e1, s);
    int host[3];
    hipError_t ce = hipMemcpyAsync(host, m->done_dev, sizeof(host), hipMemcpyDeviceToHost, s);
    hipError_t se = hipStreamSynchronize(s);
    float ms = 0.0f;
    if (se == hipSuccess && hipEventElapsedTime(&ms, e0, e1) == hipSuccess) m->last_ms = ms;
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (rc != MR_OK) return rc;
    MR_HIP(ce, "read greedy state");
    MR_HIP(se, "generate");
    MR_TRY(check_step_error(m));
    int count = host[1];
    MR_HIP(hipMemcpy(tokens, m->gen_dev, (size_t)count * sizeof(int), hipMemcpyDeviceToHost), "read tokens");
    int pos = 0;
    MR_HIP(hipMemcpy(&pos, m->pos_dev, sizeof(int), hipMemcpyDeviceToHost), "read position");
    m->position = pos;
    *produced = count;
    if (host[0] == 2) return fail(MR_ERR_NONFINITE, "non-finite output logits");
    return MR_OK;
}

int mr_model_time_kernel(mr_model *m, int which, int reps, float *avg_ms) {
    MR_TRY(check_ctx(m, "time_kernel"));
    MR_REQUIRE(avg_ms && reps >= 1 && which >= MR_KERNEL_QKV && which <= MR_KERNEL_HEAD, "time_kernel: bad arguments");
    MR_REQUIRE(is_gqa(m->d.family) || which == MR_KERNEL_HEAD,
               "time_kernel: the per-layer kernels are those of the GQA families");
    hipStream_t s = m->ctx->stream;
    hipEvent_t e0, e1;
    MR_HIP(hipEventCreate(&e0), "create event");
    MR_HIP(hipEventCreate(&e1), "create event");
    MR_HIP(hipMemsetAsync(m->done_dev, 0, sizeof(int), s), "clear stop flag");
    int launches = 0, rc = MR_OK;
    hipEventRecord(e0, s);
    for (int r = 0; r < reps && rc == MR_OK; ++r) {
        if (which == MR_KERNEL_HEAD) {
            rc = launch_lm_head(m);
            ++launches;
            continue;
        }
        for (Layer &L : m->layers) {
            rc = launch_gqa_part(m, L, which);
            if (rc != MR_OK) break;
            ++launches;
        }
    }
    hipEventRecord(e1, s);
    hipError_t e = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (rc != MR_OK) return rc;
    MR_HIP(e, "time kernel");
    *avg_ms = ms / (float)std::max(launches, 1);
    return MR_OK;
}

int mr_model_choices(mr_model *m, int32_t *out, int64_t capacity, int *per_position) {
    MR_TRY(check_ctx(m, "choices"));
    MR_REQUIRE(out && per_position, "choices: null argument");
    MR_REQUIRE(m->choices, "choices: the model makes no routing choices (heavy-medium-2.0 only)");
    const int64_t per = (int64_t)m->d.layers * m->d.inner_loop_steps * m->choice_rec;
    const int64_t n = per * m->position;
    MR_REQUIRE(n <= capacity, "choices: output too small");
    *per_position = (int)per;
    MR_HIP(hipStreamSynchronize(m->ctx->stream), "choices");
    if (n) MR_HIP(hipMemcpy(out, m->choices, (size_t)n * sizeof(int32_t), hipMemcpyDeviceToHost), "read choices");
    return MR_OK;
}

int mr_model_trace_step(mr_model *m, uint64_t *out, int64_t capacity, int *phases, int *grid) {
    MR_TRY(check_ctx(m, "trace_step"));
    MR_REQUIRE(out && phases && grid, "trace_step: null argument");
    if (!m->persistent_ok || m->mode != MR_STEP_PERSISTENT)
        return fail(MR_ERR_STATE, "trace_step: the model does not run the persistent step kernel");
    MR_REQUIRE(m->position >= 1 && m->position < m->d.context_length, "trace_step: call forward first");
    const size_t n = (size_t)m->n_head * m->grid * kTraceFields;
    MR_REQUIRE((int64_t)n <= capacity, "trace_step: output too small");
    *phases = m->n_head;
    *grid = m->grid;
    unsigned long long *buf = nullptr;
    MR_TRY(device_alloc(m, n * sizeof(unsigned long long), (void **)&buf));
    hipStream_t s = m->ctx->stream;
    hipMemsetAsync(buf, 0, n * sizeof(unsigned long long), s);
    int init[3] = {0, 0, -1};   // done, count, eos
    hipMemcpyAsync(m->done_dev, init, sizeof(init), hipMemcpyHostToDevice, s);
    int rc = run_persistent(m, STEP_GREEDY, buf);
    hipError_t e = hipStreamSynchronize(s);
    if (rc == MR_OK && e == hipSuccess) e = hipMemcpy(out, buf, n * sizeof(unsigned long long), hipMemcpyDeviceToHost);
    hipFree(buf);
    MR_TRY(rc);
    MR_HIP(e, "trace step");
    MR_TRY(check_step_error(m));
    m->position += 1;
    return MR_OK;
}

}  // extern "C"
