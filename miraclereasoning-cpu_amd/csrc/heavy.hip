// heavy-medium-2.0 token-step kernels (model.py:192-255).
//
// Attention of one inner-loop pass:
//   k_heavy_kv     the kv_up projection of the latent (one workgroup per KV
//                  head's K rows or V rows) with k_heavy_prep's work on the
//                  result, and the queries; the general path runs the
//                  projection as a GEMV and then:
//   k_heavy_prep   queries and the new key: RMSNorm without affine (eps 1e-6,
//                  kernels.cl:19-28 order) + interleaved RoPE; the key and value
//                  are appended to the pass's ring at the position and added to
//                  the running sums of their 64-row block, in row order, so the
//                  block means equal kernels.cl's block_means bit for bit.
//   k_heavy_attn_split + k_heavy_attn_merge (head dims 32/64/128): window
//                  rows in 32-row split partials; one workgroup per head
//                  scores the block columns (sequential dot products of the
//                  block means, kernels.cl:58-73), adds the distance penalty,
//                  takes the per-head stable top-k of blocks (descending score,
//                  ties to the lower block; model.py:220-226) and writes the
//                  chosen blocks' partial; the merge combines the partials.
//   k_heavy_attn / k_heavy_attn_lanes  one workgroup per query head, the
//                  same attention in kernels.cl's sequential orders (other head
//                  dims, and the path without a partial buffer).
// MoE:
//   k_moe_route    one wave: biases, group broadcast, temperature, softmax,
//                  stable top-k, confidence / entropy / adaptive width and
//                  renormalization in numpy's FP32 arithmetic (model.py:231-250;
//                  numpy float32 sums are pairwise).  With BF16 experts every
//                  routed-slot workgroup of the gate/up kernel routes the token
//                  itself instead.
//   k_moe_gate_up  SwiGLU activations of every active routed slot and every
//                  shared expert, weight pointers taken from a device table by
//                  the device-side expert ids.
//   k_moe_down     per output row: the routed experts accumulated in chosen
//                  order with their weights, then the shared experts with
//                  residual_scale / shared (kernels.cl:52-56 axpy chain), then
//                  the residual add.
#include "heavy.h"

#include "block_gemv.h"
#include "split_attention.h"

namespace mr {
namespace {

// ------------------------------------------------------------------ attention
// grid heads + kv_heads, 64 threads.  LDS: the row, its rotation angles and,
// for a key, the value and the old block sums, all loaded up front (none
// depends on the norm).
__global__ void __launch_bounds__(64) k_heavy_prep(HeavyAttnArgs a) {
    extern __shared__ float row[];
    __shared__ float scale;
    if (a.done && *a.done) return;
    const int pos = *a.pos, d = a.d, half = d / 2;
    const bool isq = (int)blockIdx.x < a.heads;
    const int hh = isq ? blockIdx.x : blockIdx.x - a.heads;
    const int kvw = a.kv_heads * d;
    const float *src = isq ? a.q + (int64_t)hh * d : a.kv + (int64_t)hh * d;
    const float *cs = a.rope + (int64_t)pos * half * 2;
    float *ang = row + d, *val = ang + d, *bk = val + d, *bv = bk + d;
    const int64_t slot = (int64_t)pos * kvw + (int64_t)hh * d;
    const int64_t bslot = (int64_t)(pos / a.block) * kvw + (int64_t)hh * d;
    const bool first = pos % a.block == 0;
#pragma unroll 4
    for (int j = threadIdx.x; j < d; j += blockDim.x) {
        row[j] = src[j];
        ang[j] = cs[j];
        if (!isq) {
            val[j] = a.kv[kvw + (int64_t)hh * d + j];
            bk[j] = first ? 0.0f : a.bsum_k[bslot + j];
            bv[j] = first ? 0.0f : a.bsum_v[bslot + j];
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {   // kernels.cl:19-28: one sequential sum of squares
        float v = 0.0f;
        for (int j = 0; j < d; ++j) {
            const float x = row[j];
            v += x * x;
        }
        scale = 1.0f / sqrtf(v / (float)d + 1e-6f);
    }
    __syncthreads();
    for (int p = threadIdx.x; p < half; p += blockDim.x) {   // interleaved pairs (kernels.cl:30-44)
        float u = row[2 * p] * scale * 1.0f, v = row[2 * p + 1] * scale * 1.0f;
        rope_rotate(u, v, ang[2 * p], ang[2 * p + 1]);
        row[2 * p] = u;
        row[2 * p + 1] = v;
    }
    __syncthreads();
    if (isq) {
        for (int j = threadIdx.x; j < d; j += blockDim.x) a.q_rot[(int64_t)hh * d + j] = row[j];
        return;
    }
    for (int j = threadIdx.x; j < d; j += blockDim.x) {
        const float k = row[j], v = val[j];
        a.ring_k[slot + j] = k;
        a.ring_v[slot + j] = v;
        a.bsum_k[bslot + j] = bk[j] + k;
        a.bsum_v[bslot + j] = bv[j] + v;
    }
}

// The K/V projection and the prologue in one launch: grid heads + 2 kv_heads,
// 256 threads.  Blocks < heads: query h as in k_heavy_prep.  The others: the
// K rows (first kv_heads blocks) or V rows of KV head kh, kv_up . latent
// (block_gemv), then k_heavy_prep's key and value work on them: the key's
// sequential sum of squares and interleaved rotation, the ring append and the
// block sums.
constexpr int kKvThreads = 256;

template <int DT>
__global__ void __launch_bounds__(kKvThreads) k_heavy_kv(HeavyAttnArgs a) {
    constexpr int EB = DT == MR_F32 ? 4 : 2;   // bytes per weight element
    extern __shared__ __align__(16) float sm[];
    __shared__ float scale;
    const int d = a.d, half = d / 2, tid = threadIdx.x;
    const int kvw = a.kv_heads * d;
    float *xs = sm, *row = sm + ((a.latent + 3) & ~3);
    const bool isq = (int)blockIdx.x < a.heads;
    const int b = isq ? blockIdx.x : blockIdx.x - a.heads;
    const bool isk = !isq && b < a.kv_heads;
    const int hh = isq ? b : (isk ? b : b - a.kv_heads);
    // The weight loads depend on nothing this step computes: they go out
    // before the flag and position loads.
    BlockGemv<DT> gemv;
    if (!isq)
        gemv.issue((const char *)a.kv_w + ((int64_t)(isk ? 0 : kvw) + (int64_t)hh * d) * a.latent * EB, d, a.latent);
    if (a.done && *a.done) return;
    const int pos = *a.pos;
    const float *cs = a.rope + (int64_t)pos * half * 2;
    float rc = 1.0f, rsn = 0.0f;   // this thread's rotation pair, loaded ahead of the norm
    if (tid < half) {
        rc = cs[2 * tid];
        rsn = cs[2 * tid + 1];
    }
    if (isq) {
        for (int j = tid; j < d; j += kKvThreads) row[j] = a.q[(int64_t)hh * d + j];
    } else {
        for (int j = tid; j < a.latent; j += kKvThreads) xs[j] = a.latent_x[j];
        __syncthreads();
        gemv.finish(xs, row);
    }
    __syncthreads();
    if (isq || isk) {
        if (tid == 0) {   // kernels.cl:19-28: one sequential sum of squares
            float v = 0.0f;
            for (int j = 0; j < d; ++j) {
                const float x = row[j];
                v += x * x;
            }
            scale = 1.0f / sqrtf(v / (float)d + 1e-6f);
        }
        __syncthreads();
        for (int p = tid; p < half; p += kKvThreads) {   // interleaved pairs (kernels.cl:30-44)
            float u = row[2 * p] * scale * 1.0f, v = row[2 * p + 1] * scale * 1.0f;
            rope_rotate(u, v, p == tid ? rc : cs[2 * p], p == tid ? rsn : cs[2 * p + 1]);
            row[2 * p] = u;
            row[2 * p + 1] = v;
        }
        __syncthreads();
    }
    if (isq) {
        for (int j = tid; j < d; j += kKvThreads) a.q_rot[(int64_t)hh * d + j] = row[j];
        return;
    }
    const int64_t slot = (int64_t)pos * kvw + (int64_t)hh * d;
    const int64_t bslot = (int64_t)(pos / a.block) * kvw + (int64_t)hh * d;
    const bool first = pos % a.block == 0;
    float *ring = isk ? a.ring_k : a.ring_v, *bsum = isk ? a.bsum_k : a.bsum_v;
    for (int j = tid; j < d; j += kKvThreads) {
        const float v = row[j];
        ring[slot + j] = v;
        bsum[bslot + j] = (first ? 0.0f : bsum[bslot + j]) + v;
    }
}

constexpr int kAttnThreads = 256;

__global__ void __launch_bounds__(kAttnThreads) k_heavy_attn(HeavyAttnArgs a) {
    extern __shared__ float sh[];
    if (a.done && *a.done) return;
    const int pos = *a.pos, d = a.d, tid = threadIdx.x;
    const int count = pos + 1, length = min(a.window, count), start = count - length;
    const int blocks = (count + a.block - 1) / a.block, total = length + blocks;
    const int h = blockIdx.x, kh = h / (a.heads / a.kv_heads), kvw = a.kv_heads * d;
    float *qs = sh;              // [d]
    float *sc = qs + d;          // [total] scores, then probabilities
    int *keep_flag = (int *)(sc + total);   // [blocks]
    __shared__ float red[kAttnThreads / 64];
    __shared__ float denom;
    for (int j = tid; j < d; j += kAttnThreads) qs[j] = a.q_rot[(int64_t)h * d + j];
    __syncthreads();
    const float root = sqrtf((float)d);
    for (int t = tid; t < total; t += kAttnThreads) {
        float v = 0.0f;
        if (t < length) {
            const float *kr = a.ring_k + (int64_t)(start + t) * kvw + (int64_t)kh * d;
            for (int j = 0; j < d; ++j) v += qs[j] * kr[j];
            sc[t] = v / root;
        } else {
            const int b = t - length;
            const float n = (float)min(a.block, count - b * a.block);
            const float *kb = a.bsum_k + (int64_t)b * kvw + (int64_t)kh * d;
            for (int j = 0; j < d; ++j) v += qs[j] * (kb[j] / n);
            const int end = min((b + 1) * a.block - 1, pos);
            sc[t] = v / root - a.slope * log1pf((float)(pos - end));
        }
    }
    __syncthreads();
    // Stable top-k of the block columns: rank = blocks scoring higher, or equal
    // with a lower index.
    const int keep = min(a.slots, blocks);
    for (int b = tid; b < blocks; b += kAttnThreads) {
        const float s = sc[length + b];
        int rank = 0;
        for (int c = 0; c < blocks; ++c) {
            const float o = sc[length + c];
            rank += o > s || (o == s && c < b);
        }
        keep_flag[b] = rank < keep;
    }
    __syncthreads();
    if (a.choice) {   // chosen blocks in ascending order, -1 padded
        int *rec = a.choice + (int64_t)pos * a.choice_stride + a.choice_blocks + h * a.slots;
        for (int b = tid; b < blocks; b += kAttnThreads)
            if (keep_flag[b]) {
                int at = 0;
                for (int c = 0; c < b; ++c) at += keep_flag[c];
                rec[at] = b;
            }
        for (int i = keep + tid; i < a.slots; i += kAttnThreads) rec[i] = -1;
    }
    for (int b = tid; b < blocks; b += kAttnThreads)
        if (!keep_flag[b]) sc[length + b] = -INFINITY;
    __syncthreads();
    // Softmax (kernels.cl:75-84): max, one sequential sum of exponentials, quotient.
    float mx = -INFINITY;
    for (int t = tid; t < total; t += kAttnThreads) mx = fmaxf(mx, sc[t]);
    mx = block_max(mx, red);
    if (tid == 0) {
        float den = 0.0f;
        for (int t = 0; t < total; ++t) den += expf(sc[t] - mx);
        denom = den;
    }
    __syncthreads();
    for (int t = tid; t < total; t += kAttnThreads) sc[t] = expf(sc[t] - mx) / denom;
    __syncthreads();
    // Mix (kernels.cl:93-107): one sequential sum over keys per output element.
    for (int j = tid; j < d; j += kAttnThreads) {
        float acc = 0.0f;
        for (int t = 0; t < total; ++t) {
            float v;
            if (t < length) {
                v = a.ring_v[(int64_t)(start + t) * kvw + (int64_t)kh * d + j];
            } else {
                const int b = t - length;
                const float n = (float)min(a.block, count - b * a.block);
                v = a.bsum_v[(int64_t)b * kvw + (int64_t)kh * d + j] / n;
            }
            acc += sc[t] * v;
        }
        a.out[(int64_t)h * d + j] = acc;
    }
}

// Head dims 32/64/128: the same attention with the window scores, the softmax
// sum and the value mix spread over the workgroup (a lane holds 16 dims of a
// key, D/16 lanes per key).  The block-mean scores keep the sequential
// per-thread order above, so the block choices are the same bit for bit; the
// window scores and the mix differ from the sequential orders by rounding.
template <int D>
__global__ void __launch_bounds__(kAttnThreads) k_heavy_attn_lanes(HeavyAttnArgs a) {
    constexpr int LPK = D / 16, KPW = kWave / LPK, NWV = kAttnThreads / kWave;
    extern __shared__ float sh[];
    __shared__ float red[NWV];
    __shared__ float wo[NWV][D];
    if (a.done && *a.done) return;
    const int pos = *a.pos, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, sub = lane % LPK, kg = lane / LPK;
    const int count = pos + 1, length = min(a.window, count), start = count - length;
    const int blocks = (count + a.block - 1) / a.block, total = length + blocks;
    const int h = blockIdx.x, kh = h / (a.heads / a.kv_heads), kvw = a.kv_heads * D;
    float *qs = sh;                          // [D]
    float *sc = qs + D;                      // [total] scores, then exponentials
    int *keep_flag = (int *)(sc + total);    // [blocks]
    for (int j = tid; j < D; j += kAttnThreads) qs[j] = a.q_rot[(int64_t)h * D + j];
    __syncthreads();
    const float root = sqrtf((float)D);
    float4 q[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) q[c] = *(const float4 *)(qs + 16 * sub + 4 * c);
    for (int r0 = wave * KPW; r0 < length; r0 += NWV * KPW) {   // window scores
        const int t = r0 + kg;
        float dot = 0.0f;
        if (t < length) {
            const float *kr = a.ring_k + (int64_t)(start + t) * kvw + (int64_t)kh * D + 16 * sub;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float4 k4 = load_f4(kr + 4 * c);
                dot = fmaf(q[c].x, k4.x, dot);
                dot = fmaf(q[c].y, k4.y, dot);
                dot = fmaf(q[c].z, k4.z, dot);
                dot = fmaf(q[c].w, k4.w, dot);
            }
        }
        dot = att::lanes_sum<LPK>(dot);
        if (t < length && sub == 0) sc[t] = dot / root;
    }
    for (int b = tid; b < blocks; b += kAttnThreads) {   // block-mean scores, sequential (kernels.cl:58-73)
        float v = 0.0f;
        const float n = (float)min(a.block, count - b * a.block);
        const float *kb = a.bsum_k + (int64_t)b * kvw + (int64_t)kh * D;
        for (int j = 0; j < D; ++j) v += qs[j] * (kb[j] / n);
        const int end = min((b + 1) * a.block - 1, pos);
        sc[length + b] = v / root - a.slope * log1pf((float)(pos - end));
    }
    __syncthreads();
    const int keep = min(a.slots, blocks);
    for (int b = tid; b < blocks; b += kAttnThreads) {   // stable top-k (model.py:220-226)
        const float s = sc[length + b];
        int rank = 0;
        for (int c = 0; c < blocks; ++c) {
            const float o = sc[length + c];
            rank += o > s || (o == s && c < b);
        }
        keep_flag[b] = rank < keep;
    }
    __syncthreads();
    if (a.choice) {
        int *rec = a.choice + (int64_t)pos * a.choice_stride + a.choice_blocks + h * a.slots;
        for (int b = tid; b < blocks; b += kAttnThreads)
            if (keep_flag[b]) {
                int at = 0;
                for (int c = 0; c < b; ++c) at += keep_flag[c];
                rec[at] = b;
            }
        for (int i = keep + tid; i < a.slots; i += kAttnThreads) rec[i] = -1;
    }
    for (int b = tid; b < blocks; b += kAttnThreads)
        if (!keep_flag[b]) sc[length + b] = -INFINITY;
    __syncthreads();
    float mx = -INFINITY;
    for (int t = tid; t < total; t += kAttnThreads) mx = fmaxf(mx, sc[t]);
    mx = block_max(mx, red);
    float den = 0.0f;
    for (int t = tid; t < total; t += kAttnThreads) {
        const float p = expf(sc[t] - mx);
        sc[t] = p;
        den += p;
    }
    den = block_sum(den, red);   // its barriers also publish sc
    float4 acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int r0 = wave * KPW; r0 < total; r0 += NWV * KPW) {   // weighted values
        const int t = r0 + kg;
        const float p = t < total ? sc[t] : 0.0f;
        if (p != 0.0f) {
            if (t < length) {
                const float *vr = a.ring_v + (int64_t)(start + t) * kvw + (int64_t)kh * D + 16 * sub;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float4 v = load_f4(vr + 4 * c);
                    acc[c].x = fmaf(p, v.x, acc[c].x);
                    acc[c].y = fmaf(p, v.y, acc[c].y);
                    acc[c].z = fmaf(p, v.z, acc[c].z);
                    acc[c].w = fmaf(p, v.w, acc[c].w);
                }
            } else {
                const int b = t - length;
                const float n = (float)min(a.block, count - b * a.block);
                const float *vb = a.bsum_v + (int64_t)b * kvw + (int64_t)kh * D + 16 * sub;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float4 v = load_f4(vb + 4 * c);
                    acc[c].x = fmaf(p, v.x / n, acc[c].x);
                    acc[c].y = fmaf(p, v.y / n, acc[c].y);
                    acc[c].z = fmaf(p, v.z / n, acc[c].z);
                    acc[c].w = fmaf(p, v.w / n, acc[c].w);
                }
            }
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const float ox = att::keygroups_sum_lanes<LPK>(acc[c].x);
        const float oy = att::keygroups_sum_lanes<LPK>(acc[c].y);
        const float oz = att::keygroups_sum_lanes<LPK>(acc[c].z);
        const float ow = att::keygroups_sum_lanes<LPK>(acc[c].w);
        if (kg == 0) *(float4 *)&wo[wave][16 * sub + 4 * c] = make_float4(ox, oy, oz, ow);
    }
    __syncthreads();
    for (int j = tid; j < D; j += kAttnThreads) {
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < NWV; ++w) o += wo[w][j];
        a.out[(int64_t)h * D + j] = o / den;
    }
}

// Split form for head dims 32/64/128, grid (window splits + 1, heads): the
// workgroups x < splits write the partial of window rows [32 x, 32 x + 32);
// the last one scores the block columns (the block-sum quotients of a chunk of
// blocks staged in LDS by every thread, then one sequential dot product per
// block in kernels.cl:58-73's order, so the block choices are the same bit for
// bit), takes the stable top-k and writes the chosen blocks' partial in
// ascending block order.  k_heavy_attn_merge combines the partials.
constexpr int kBlockChunkFloats = 4096;   // block-sum quotients staged per pass
constexpr int kHeavyMaxChosen = 32;       // chosen blocks per head
constexpr int kChosenBatch = 8;           // chosen blocks' value loads in flight together

inline size_t heavy_split_lds(int d, int blocks) {
    return (size_t)(d + 2 * blocks + kBlockChunkFloats + kBlockChunkFloats / d) * sizeof(float);
}

template <int D>
__global__ void __launch_bounds__(split::kThreads) k_heavy_attn_split(HeavyAttnArgs a) {
    constexpr int NT = split::kThreads;
    extern __shared__ float sh[];
    if (a.done && *a.done) return;
    const int pos = *a.pos, tid = threadIdx.x;
    const int count = pos + 1, length = min(a.window, count), start = count - length;
    const int h = blockIdx.y, kh = h / (a.heads / a.kv_heads), kvw = a.kv_heads * D;
    const int wsplits = gridDim.x - 1;
    float *part = a.part + ((int64_t)h * gridDim.x + blockIdx.x) * (D + 2);
    if ((int)blockIdx.x < wsplits) {
        const int t0 = blockIdx.x * kHeavyRows;
        if (t0 >= length) return;
        const auto rows = [&](int t, const float **k, const float **v) {
            *k = a.ring_k + (int64_t)(start + t) * kvw + (int64_t)kh * D;
            *v = a.ring_v + (int64_t)(start + t) * kvw + (int64_t)kh * D;
            return true;
        };
        split::partial<D>(a.q_rot + (int64_t)h * D, t0, min(length, t0 + kHeavyRows), rows, part);
        return;
    }
    __shared__ int chosen[kHeavyMaxChosen];
    const int blocks = (count + a.block - 1) / a.block;
    float *qs = sh, *sc = qs + D;            // [D] query, [blocks] block scores
    int *keep_flag = (int *)(sc + blocks);   // [blocks]
    float *quo = (float *)(keep_flag + blocks);
    for (int j = tid; j < D; j += NT) qs[j] = a.q_rot[(int64_t)h * D + j];
    const float root = sqrtf((float)D);
    constexpr int CB = kBlockChunkFloats / D;
    for (int b0 = 0; b0 < blocks; b0 += CB) {
        const int nb = min(CB, blocks - b0);
        float kv[kBlockChunkFloats / NT];   // every load of the chunk in flight before the quotients
#pragma unroll
        for (int k = 0; k < kBlockChunkFloats / NT; ++k) {   // unguarded (clamped) loads issue back to back
            const int i = min(tid + k * NT, nb * D - 1), b = b0 + i / D, j = i % D;
            kv[k] = a.bsum_k[(int64_t)b * kvw + (int64_t)kh * D + j];
        }
#pragma unroll
        for (int k = 0; k < kBlockChunkFloats / NT; ++k) {
            const int i = tid + k * NT, b = b0 + i / D;
            if (i < nb * D) quo[i + i / D] = kv[k] / (float)min(a.block, count - b * a.block);
        }
        __syncthreads();
        for (int b = b0 + tid; b < b0 + nb; b += NT) {
            const float *qb = quo + (b - b0) * (D + 1);   // rows padded by one float: no bank conflicts
            float v = 0.0f;
            for (int j = 0; j < D; ++j) v += qs[j] * qb[j];
            const int end = min((b + 1) * a.block - 1, pos);
            sc[b] = v / root - a.slope * log1pf((float)(pos - end));
        }
        __syncthreads();
    }
    const int keep = min(a.slots, blocks);
    for (int b = tid; b < blocks; b += NT) {   // stable top-k (model.py:220-226)
        const float s = sc[b];
        int rank = 0;
        for (int c = 0; c < blocks; ++c) {
            const float o = sc[c];
            rank += o > s || (o == s && c < b);
        }
        keep_flag[b] = rank < keep;
    }
    __syncthreads();
    for (int b = tid; b < blocks; b += NT)   // chosen blocks in ascending order
        if (keep_flag[b]) {
            int at = 0;
            for (int c = 0; c < b; ++c) at += keep_flag[c];
            chosen[at] = b;
        }
    __syncthreads();
    if (a.choice) {
        int *rec = a.choice + (int64_t)pos * a.choice_stride + a.choice_blocks + h * a.slots;
        for (int i = tid; i < a.slots; i += NT) rec[i] = i < keep ? chosen[i] : -1;
    }
    float m = -INFINITY;
    for (int i = 0; i < keep; ++i) m = fmaxf(m, sc[chosen[i]]);
    for (int j = tid; j < D; j += NT) {
        float o = 0.0f, l = 0.0f;
        for (int i0 = 0; i0 < keep; i0 += kChosenBatch) {
            float vals[kChosenBatch];
#pragma unroll
            for (int i = 0; i < kChosenBatch; ++i)
                vals[i] = a.bsum_v[(int64_t)chosen[min(i0 + i, keep - 1)] * kvw + (int64_t)kh * D + j];
#pragma unroll
            for (int i = 0; i < kChosenBatch; ++i) {
                if (i0 + i < keep) {
                    const int b = chosen[i0 + i];
                    const float p = expf(sc[b] - m);
                    const float n = (float)min(a.block, count - b * a.block);
                    o = fmaf(p, vals[i] / n, o);
                    l += p;
                }
            }
        }
        part[2 + j] = o;
        if (j == 0) {
            part[0] = m;
            part[1] = l;
        }
    }
}

// grid heads, split::kThreads: the active window partials and the block partial.
template <int D>
__global__ void __launch_bounds__(split::kThreads) k_heavy_attn_merge(HeavyAttnArgs a, int parts) {
    if (a.done && *a.done) return;
    const int length = min(a.window, *a.pos + 1);
    split::merge<D>(a.part + (int64_t)blockIdx.x * parts * (D + 2), (length + kHeavyRows - 1) / kHeavyRows, parts - 1,
                    a.out + (int64_t)blockIdx.x * D);
}

// ------------------------------------------------------------------ MoE
// numpy's float32 add.reduce: pairwise summation, blocks of 8 accumulators
// up to 128 elements, sequential below 8 elements; longer arrays split in two
// halves (a multiple of 8 first), which covers up to 256 elements here.
__device__ float np_block_sum(const float *a, int n) {
    if (n < 8) {
        float r = 0.0f;
        for (int i = 0; i < n; ++i) r += a[i];
        return r;
    }
    float r[8];
    for (int k = 0; k < 8; ++k) r[k] = a[k];
    int i = 8;
    for (; i < n - (n % 8); i += 8)
        for (int k = 0; k < 8; ++k) r[k] += a[i + k];
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) res += a[i];
    return res;
}

__device__ float np_pairwise_sum(const float *a, int n) {
    if (n <= 128) return np_block_sum(a, n);
    int n2 = n / 2;
    n2 -= n2 % 8;
    return np_block_sum(a, n2) + np_block_sum(a + n2, n - n2);
}

constexpr int kMaxExperts = 256;
constexpr int kMaxTopK = 16;

// Routing of one token by one wave (experts <= kMaxExperts, up to four per
// lane): biases, group broadcast, temperature, softmax, stable top-k, adaptive
// width and renormalized weights, left in r for the wave; with publish, also
// stored as the layer's ids, weights, width and choice record.  No workgroup
// barrier: the lanes exchange values through LDS, which a wave reads back in
// issue order.
struct RouteLds {
    float probs[kMaxExperts], terms[kMaxExperts];
    int chosen[kMaxTopK];
    float w[kMaxTopK];
    int active;
};

__device__ __forceinline__ void route_wave(const MoeArgs &a, RouteLds &r, bool publish) {
    constexpr int PER = kMaxExperts / kWave;
    const int lane = threadIdx.x & 63, E = a.experts, G = a.groups, size = (E + G - 1) / G;
    float logit[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {   // clamped indices: every load issues at once
        const int e = min(lane + kWave * i, E - 1), g = min(e / size, G - 1);
        const float fine = a.router[G + e] + (a.fine_bias[e] + a.expert_bias[e]);
        const float coarse = a.router[g] + (a.coarse_bias[g] + a.group_bias[g]);
        logit[i] = (fine + coarse) / a.inv_temperature_div;
    }
    // kernels.cl:75-84 softmax: the maximum (order-free), each exponent by its
    // own lane, the denominator summed in expert order by every lane
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; ++i)
        if (lane + kWave * i < E) m = fmaxf(m, logit[i]);
    m = wave_max(m);
    float ex[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        ex[i] = expf(logit[i] - m);
        if (lane + kWave * i < E) r.terms[lane + kWave * i] = ex[i];
    }
    __builtin_amdgcn_wave_barrier();
    float den = 0.0f;
    for (int e = 0; e < E; ++e) den += r.terms[e];
#pragma unroll
    for (int i = 0; i < PER; ++i)
        if (lane + kWave * i < E) r.probs[lane + kWave * i] = ex[i] / den;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < PER; ++i) {   // stable argsort of -probs (model.py:241)
        const int e = lane + kWave * i;
        if (e < E) {
            const float p = r.probs[e];
            int rank = 0;
            for (int f = 0; f < E; ++f) rank += r.probs[f] > p || (r.probs[f] == p && f < e);
            if (rank < a.kmax) r.chosen[rank] = e;
            r.terms[e] = p * logf(fmaxf(p, 1e-9f));
        }
    }
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {   // model.py:242-250; the weights stay in LDS (a private array would live in scratch memory)
        const int kmax = a.kmax;
        float *w = r.w;
        for (int k = 0; k < kmax; ++k) w[k] = r.probs[r.chosen[k]];
        const float confidence = w[0] - w[min(kmax - 1, 1)];
        const float entropy = -np_pairwise_sum(r.terms, E);
        const float spread = rintf((1.0f - confidence) * 2.0f + entropy / a.log_experts);
        const float width = fminf(fmaxf((float)a.kmin + spread, (float)a.kmin), (float)kmax);
        const int active = (int)width;
        for (int k = active; k < kmax; ++k) w[k] = 0.0f;
        const float wden = fmaxf(np_pairwise_sum(w, kmax), 1e-9f);
        for (int k = 0; k < kmax; ++k) w[k] = w[k] / wden;
        r.active = active;
    }
    __builtin_amdgcn_wave_barrier();
    if (publish) {
        const int active = r.active;
        if (lane < a.kmax) {
            a.ids[lane] = r.chosen[lane];
            a.weights[lane] = r.w[lane];
        }
        if (lane == 0) *a.active = active;
        if (a.choice) {
            int *rec = a.choice + (int64_t)(a.pos ? *a.pos : a.position) * a.choice_stride;
            if (lane == 0) rec[0] = active;
            if (lane < a.kmax) rec[1 + lane] = lane < active ? r.chosen[lane] : -1;
        }
    }
}

__global__ void __launch_bounds__(kWave) k_moe_route(MoeArgs a) {
    __shared__ RouteLds r;
    if (a.done && *a.done) return;
    route_wave(a, r, true);
}

constexpr int kMoeThreads = 512;
constexpr int kMoeRows = kMoeThreads / kWave;   // one wave per output row

__device__ __forceinline__ float dot_row(const void *w, int dt, int64_t row, int k, const float *xs) {
    const int lane = threadIdx.x & 63;
    float acc = 0.0f;
    if (dt == MR_BF16 && (k % 8) == 0) {
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 *r = (const u32x4 *)((const uint16_t *)w + row * k);
        for (int v = lane; v < k / 8; v += kWave) {
            const u32x4 q = __builtin_nontemporal_load(gmem(r + v));
            const float *x = xs + v * 8;
            acc = fmaf(__uint_as_float(q.x << 16), x[0], acc);
            acc = fmaf(__uint_as_float(q.x & 0xffff0000u), x[1], acc);
            acc = fmaf(__uint_as_float(q.y << 16), x[2], acc);
            acc = fmaf(__uint_as_float(q.y & 0xffff0000u), x[3], acc);
            acc = fmaf(__uint_as_float(q.z << 16), x[4], acc);
            acc = fmaf(__uint_as_float(q.z & 0xffff0000u), x[5], acc);
            acc = fmaf(__uint_as_float(q.w << 16), x[6], acc);
            acc = fmaf(__uint_as_float(q.w & 0xffff0000u), x[7], acc);
        }
    } else {
        for (int j = lane; j < k; j += kWave) {
            float wv;
            if (dt == MR_F32) wv = ((const float *)w)[row * k + j];
            else if (dt == MR_BF16) wv = bf16_to_f32(((const uint16_t *)w)[row * k + j]);
            else wv = f16_to_f32(((const uint16_t *)w)[row * k + j]);
            acc = fmaf(wv, xs[j], acc);
        }
    }
    return wave_sum(acc);
}

// grid (ceil(ffn / kMoeRows), kmax + shared)
__global__ void __launch_bounds__(kMoeThreads) k_moe_gate_up(MoeArgs a) {
    extern __shared__ float xs[];
    if (a.done && *a.done) return;
    const int slot = blockIdx.y;
    int e;
    if (slot < a.kmax) {
        if (slot >= *a.active) return;
        e = a.ids[slot];
    } else {
        e = a.experts + (slot - a.kmax);
    }
    for (int j = threadIdx.x; j < a.h; j += kMoeThreads) xs[j] = a.x[j];
    __syncthreads();
    const int row = blockIdx.x * kMoeRows + (threadIdx.x >> 6);
    if (row >= a.ffn) return;
    const float g = dot_row(a.gate[e], a.dtype, row, a.h, xs);
    const float u = dot_row(a.up[e], a.dtype, row, a.h, xs);
    if ((threadIdx.x & 63) == 0) a.act[(int64_t)slot * a.ffn + row] = (g / (1.0f + expf(-g))) * u;   // kernels.cl:46-50
}

// grid ceil(h / kMoeRows)
__global__ void __launch_bounds__(kMoeThreads) k_moe_down(MoeArgs a) {
    extern __shared__ float acts[];
    if (a.done && *a.done) return;
    const int slots = a.kmax + a.shared, active = *a.active;
    for (int i = threadIdx.x; i < slots * a.ffn; i += kMoeThreads) {
        const int s = i / a.ffn;
        acts[i] = (s < a.kmax && s >= active) ? 0.0f : a.act[i];
    }
    __syncthreads();
    const int row = blockIdx.x * kMoeRows + (threadIdx.x >> 6);
    if (row >= a.h) return;
    float total = 0.0f;
    for (int s = 0; s < active; ++s) {
        const float y = dot_row(a.down[a.ids[s]], a.dtype, row, a.ffn, acts + (int64_t)s * a.ffn);
        total = total + a.weights[s] * y;
    }
    for (int s = 0; s < a.shared; ++s) {
        const float y = dot_row(a.down[a.experts + s], a.dtype, row, a.ffn, acts + (int64_t)(a.kmax + s) * a.ffn);
        total = total + a.shared_scale * y;
    }
    if ((threadIdx.x & 63) == 0) a.hidden[row] = a.hidden[row] + a.scale * total;
}

// BF16 expert kernels (h and ffn multiples of 8).  A wave issues all of its
// 16-byte weight loads for a round (gate and up of two rows, or one row of
// every slot's down matrix) before the workgroup stages its input vector in
// LDS, so the weight latency and the staging overlap; the products keep the
// per-row wave sums and the accumulation order of the kernels above.
typedef unsigned moe_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kMoeGuRows = 2;        // rows per wave in the gate/up kernel
constexpr int kMoeGuVec = 4;         // 16-byte vectors per lane and matrix row in one round
constexpr int kMoeDnVec = 2;         // 16-byte vectors per lane and slot row in one round
constexpr int kMoeMaxSlots = 16;     // routed top-k + shared experts in the down kernel's slot chunk
constexpr int kMoeStage = 4;         // activation float4 loads per thread in flight while staging

__device__ __forceinline__ float dot8_bf16(moe_u32x4 q, const float *x, float acc) {
    const float4 x0 = *(const float4 *)x, x1 = *(const float4 *)(x + 4);
    acc = fmaf(__uint_as_float(q.x << 16), x0.x, acc);
    acc = fmaf(__uint_as_float(q.x & 0xffff0000u), x0.y, acc);
    acc = fmaf(__uint_as_float(q.y << 16), x0.z, acc);
    acc = fmaf(__uint_as_float(q.y & 0xffff0000u), x0.w, acc);
    acc = fmaf(__uint_as_float(q.z << 16), x1.x, acc);
    acc = fmaf(__uint_as_float(q.z & 0xffff0000u), x1.y, acc);
    acc = fmaf(__uint_as_float(q.w << 16), x1.z, acc);
    acc = fmaf(__uint_as_float(q.w & 0xffff0000u), x1.w, acc);
    return acc;
}

// grid (ceil(ffn / (kMoeRows * kMoeGuRows)), kmax + shared)
//
// The routed-slot workgroups route the token themselves (route_wave in wave
// 0: the same arithmetic in every workgroup, so the same experts) while the
// other waves stage the input; workgroup (0, 0) publishes the routing for
// k_moe_down and the choice log.
__global__ void __launch_bounds__(kMoeThreads) k_moe_gate_up_bf16(MoeArgs a) {
    extern __shared__ __align__(16) float xs[];
    __shared__ RouteLds route;
    if (a.done && *a.done) return;
    const int slot = blockIdx.y;
    int e;
    if (slot < a.kmax) {
        if (threadIdx.x < kWave) route_wave(a, route, blockIdx.x == 0 && slot == 0);
        for (int j = threadIdx.x * 4; j < a.h; j += kMoeThreads * 4) *(float4 *)&xs[j] = load_f4(a.x + j);
        __syncthreads();
        if (slot >= route.active) return;
        e = route.chosen[slot];
    } else {
        e = a.experts + (slot - a.kmax);
    }
    const int lane = threadIdx.x & 63, nv = a.h / 8;
    const int r0 = (blockIdx.x * kMoeRows + (threadIdx.x >> 6)) * kMoeGuRows;
    const moe_u32x4 *gw = (const moe_u32x4 *)a.gate[e], *uw = (const moe_u32x4 *)a.up[e];
    int64_t rb[kMoeGuRows];
#pragma unroll
    for (int r = 0; r < kMoeGuRows; ++r) rb[r] = (int64_t)min(r0 + r, a.ffn - 1) * nv;
    moe_u32x4 qg[kMoeGuRows][kMoeGuVec], qu[kMoeGuRows][kMoeGuVec];
#pragma unroll
    for (int i = 0; i < kMoeGuVec; ++i) {
        const int v = min(lane + kWave * i, nv - 1);
#pragma unroll
        for (int r = 0; r < kMoeGuRows; ++r) {
            qg[r][i] = __builtin_nontemporal_load(gmem(gw + rb[r] + v));
            qu[r][i] = __builtin_nontemporal_load(gmem(uw + rb[r] + v));
        }
    }
    if (slot >= a.kmax)
        for (int j = threadIdx.x * 4; j < a.h; j += kMoeThreads * 4) *(float4 *)&xs[j] = load_f4(a.x + j);
    __syncthreads();
    if (r0 >= a.ffn) return;
    float g[kMoeGuRows] = {}, u[kMoeGuRows] = {};
    for (int base = 0;;) {
#pragma unroll
        for (int i = 0; i < kMoeGuVec; ++i) {
            const int v = base + lane + kWave * i;
            if (v < nv) {
#pragma unroll
                for (int r = 0; r < kMoeGuRows; ++r) {
                    g[r] = dot8_bf16(qg[r][i], xs + 8 * v, g[r]);
                    u[r] = dot8_bf16(qu[r][i], xs + 8 * v, u[r]);
                }
            }
        }
        base += kWave * kMoeGuVec;
        if (base >= nv) break;
#pragma unroll
        for (int i = 0; i < kMoeGuVec; ++i) {
            const int v = min(base + lane + kWave * i, nv - 1);
#pragma unroll
            for (int r = 0; r < kMoeGuRows; ++r) {
                qg[r][i] = __builtin_nontemporal_load(gmem(gw + rb[r] + v));
                qu[r][i] = __builtin_nontemporal_load(gmem(uw + rb[r] + v));
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kMoeGuRows; ++r) {
        const float gs = wave_sum(g[r]), us = wave_sum(u[r]);
        if (lane == 0 && r0 + r < a.ffn)
            a.act[(int64_t)slot * a.ffn + r0 + r] = (gs / (1.0f + expf(-gs))) * us;   // kernels.cl:46-50
    }
}

// grid ceil(h / kMoeRows): one wave per output row over the active routed
// slots in chosen order, then the shared experts.
__global__ void __launch_bounds__(kMoeThreads) k_moe_down_bf16(MoeArgs a) {
    extern __shared__ __align__(16) float acts[];
    __shared__ const moe_u32x4 *wp[kMoeMaxSlots];
    __shared__ float wsc[kMoeMaxSlots];
    __shared__ int aoff[kMoeMaxSlots];
    if (a.done && *a.done) return;
    const int tid = threadIdx.x, lane = tid & 63, nv = a.ffn / 8;
    const int active = *a.active, n = active + a.shared;
    if (tid < n) {   // slot table: routed slots 0..active-1, then the shared experts
        const bool routed = tid < active;
        const int s = routed ? tid : a.kmax + (tid - active);
        const int id = a.ids[min(tid, a.kmax - 1)];   // loaded with the width, not after it
        const float w = a.weights[min(tid, a.kmax - 1)];
        wp[tid] = (const moe_u32x4 *)a.down[routed ? id : a.experts + (tid - active)];
        wsc[tid] = routed ? w : a.shared_scale;
        aoff[tid] = s * a.ffn;
    }
    __syncthreads();
    const int row = min((int)(blockIdx.x * kMoeRows + (tid >> 6)), a.h - 1);
    moe_u32x4 q[kMoeMaxSlots][kMoeDnVec];
#pragma unroll
    for (int k = 0; k < kMoeMaxSlots; ++k) {
        const moe_u32x4 *w = wp[min(k, n - 1)] + (int64_t)row * nv;
#pragma unroll
        for (int i = 0; i < kMoeDnVec; ++i)
            if (k < n) q[k][i] = __builtin_nontemporal_load(gmem(w + min(lane + kWave * i, nv - 1)));
    }
    const int total4 = (a.kmax + a.shared) * a.ffn;
    for (int j0 = 0; j0 < total4; j0 += kMoeThreads * 4 * kMoeStage) {   // kMoeStage loads in flight
        float4 t[kMoeStage];
#pragma unroll
        for (int k = 0; k < kMoeStage; ++k) t[k] = load_f4(a.act + min(j0 + (tid + k * kMoeThreads) * 4, total4 - 4));
#pragma unroll
        for (int k = 0; k < kMoeStage; ++k) {
            const int j = j0 + (tid + k * kMoeThreads) * 4;
            if (j < total4) *(float4 *)&acts[j] = t[k];
        }
    }
    __syncthreads();
    if ((int)(blockIdx.x * kMoeRows + (tid >> 6)) >= a.h) return;
    float acc[kMoeMaxSlots] = {};
    for (int base = 0;;) {
#pragma unroll
        for (int k = 0; k < kMoeMaxSlots; ++k) {
            if (k < n) {
#pragma unroll
                for (int i = 0; i < kMoeDnVec; ++i) {
                    const int v = base + lane + kWave * i;
                    if (v < nv) acc[k] = dot8_bf16(q[k][i], acts + aoff[k] + 8 * v, acc[k]);
                }
            }
        }
        base += kWave * kMoeDnVec;
        if (base >= nv) break;
#pragma unroll
        for (int k = 0; k < kMoeMaxSlots; ++k) {
            const moe_u32x4 *w = wp[min(k, n - 1)] + (int64_t)row * nv;
#pragma unroll
            for (int i = 0; i < kMoeDnVec; ++i)
                if (k < n) q[k][i] = __builtin_nontemporal_load(gmem(w + min(base + lane + kWave * i, nv - 1)));
        }
    }
    float total = 0.0f;
#pragma unroll
    for (int k = 0; k < kMoeMaxSlots; ++k) {
        if (k < n) {
            const float y = wave_sum(acc[k]);
            total = total + wsc[k] * y;
        }
    }
    if (lane == 0) a.hidden[row] = a.hidden[row] + a.scale * total;
}

// ------------------------------------------------------------------ batched prefill
// grid (blocks the chunk touches, ceil(2 kvw / 256)): one thread per column.
__global__ void __launch_bounds__(256) k_heavy_scan(HeavyScanArgs a) {
    const int c = blockIdx.y * 256 + threadIdx.x;
    if (c >= 2 * a.kvw) return;
    const bool isk = c < a.kvw;
    const int j = isk ? c : c - a.kvw;
    const float *ring = isk ? a.ring_k : a.ring_v;
    float *bsum = isk ? a.bsum_k : a.bsum_v;
    const int b = a.p0 / a.block + blockIdx.x, bstart = b * a.block;
    const int r0 = max(bstart, a.p0), r1 = min(bstart + a.block, a.p0 + a.rows);
    float v = bstart < a.p0 ? bsum[(int64_t)b * a.kvw + j] : 0.0f;
    for (int r = r0; r < r1; ++r) {
        v = v + ring[(int64_t)r * a.kvw + j];
        a.sums[(int64_t)(r - a.p0) * 2 * a.kvw + c] = v;
    }
    bsum[(int64_t)b * a.kvw + j] = v;
}

// grid (rows, heads), kSelThreads.  LDS: query, block scores, keep flags.
constexpr int kSelHeads = 4;   // query heads of one row per workgroup, a wave each
constexpr int kSelThreads = kSelHeads * kWave;

template <int D>
__global__ void __launch_bounds__(kSelThreads) k_heavy_select(HeavySelectArgs a) {
    extern __shared__ float sh[];
    __shared__ int chosen_all[kSelHeads][kHeavyMaxChosen];
    // wave w takes head kSelHeads y + w of row x; a wave past the last head
    // repeats the last head's work (every wave meets the same barriers: the
    // row's heads see the same blocks) and stores nothing
    const int t = blockIdx.x, wave = threadIdx.x >> 6, tid = threadIdx.x & 63;
    const bool live = (int)blockIdx.y * kSelHeads + wave < a.heads;
    const int h = min((int)blockIdx.y * kSelHeads + wave, a.heads - 1);
    const int pos = a.p0 + t, count = pos + 1, kh = h / (a.heads / a.kv_heads), kvw = a.kv_heads * D;
    const int blocks = (count + a.block - 1) / a.block, bt = pos / a.block;
    float *qs = sh + wave * (D + 2 * blocks), *sc = qs + D;
    int *keep_flag = (int *)(sc + blocks);
    int *chosen = chosen_all[wave];
    for (int j = tid; j < D; j += kWave) qs[j] = a.qkv[(int64_t)t * a.ld + (int64_t)h * D + j];
    __syncthreads();
    const float root = sqrtf((float)D);
    const float *row_sums = a.sums + (int64_t)t * 2 * kvw;
    for (int b = tid; b < blocks; b += kWave) {   // the token step's quotients and dot order
        const float *ks = b < bt ? a.bsum_k + (int64_t)b * kvw + (int64_t)kh * D : row_sums + (int64_t)kh * D;
        const float n = (float)min(a.block, count - b * a.block);
        float v = 0.0f;
        for (int j = 0; j < D; ++j) v += qs[j] * (ks[j] / n);
        const int end = min((b + 1) * a.block - 1, pos);
        sc[b] = v / root - a.slope * log1pf((float)(pos - end));
    }
    __syncthreads();
    const int keep = min(a.slots, blocks);
    for (int b = tid; b < blocks; b += kWave) {   // stable top-k (model.py:220-226)
        const float sv = sc[b];
        int rank = 0;
        for (int c = 0; c < blocks; ++c) {
            const float o = sc[c];
            rank += o > sv || (o == sv && c < b);
        }
        keep_flag[b] = rank < keep;
    }
    __syncthreads();
    for (int b = tid; b < blocks; b += kWave)
        if (keep_flag[b]) {
            int at = 0;
            for (int c = 0; c < b; ++c) at += keep_flag[c];
            chosen[at] = b;
        }
    __syncthreads();
    if (!live) return;   // no barrier follows
    if (a.choice) {
        int *rec = a.choice + (int64_t)pos * a.choice_stride + a.choice_blocks + h * a.slots;
        for (int i = tid; i < a.slots; i += kWave) rec[i] = i < keep ? chosen[i] : -1;
    }
    float m = -INFINITY;
    for (int i = 0; i < keep; ++i) m = fmaxf(m, sc[chosen[i]]);
    float *out = a.ext + ((int64_t)t * a.heads + h) * (D + 4);
    for (int j = tid; j < D; j += kWave) {
        float o = 0.0f, l = 0.0f;
        for (int i = 0; i < keep; ++i) {
            const int b = chosen[i];
            const float *vs = b < bt ? a.bsum_v + (int64_t)b * kvw : row_sums + kvw;
            const float p = expf(sc[b] - m);
            const float n = (float)min(a.block, count - b * a.block);
            o = fmaf(p, vs[(int64_t)kh * D + j] / n, o);
            l += p;
        }
        out[4 + j] = o;
        if (j == 0) {
            out[0] = m;
            out[1] = l;
            out[2] = out[3] = 0.0f;
        }
    }
}

// grid rows, one wave: route_wave with this row's logits, publishing its
// experts, weights, width and choice record; then its routed slots counted.
__global__ void __launch_bounds__(kWave) k_moe_route_rows(MoeRowsArgs m) {
    __shared__ RouteLds r;
    const int t = blockIdx.x;
    MoeArgs a = m.a;
    a.router += (int64_t)t * (a.groups + a.experts);
    a.ids += (int64_t)t * a.kmax;
    a.weights += (int64_t)t * a.kmax;
    a.active += t;
    a.pos = nullptr;
    a.position = m.p0 + t;
    route_wave(a, r, true);
    const int lane = threadIdx.x;
    if (lane < r.active) atomicAdd(&m.counts[r.chosen[lane]], 1);
}

__global__ void k_moe_zero(int *counts, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) counts[i] = 0;
}

// one thread: group offsets (routed experts in expert order, then one group
// of every row per shared expert), cleared fill cursors and, where asked,
// the prefix sums of the groups' row tiles
__global__ void k_moe_offsets(MoeRowsArgs m) {
    const int E = m.a.experts, S = m.a.shared;
    int at = 0, tiles = 0;
    for (int e = 0; e < E + S; ++e) {
        if (e >= E) m.counts[e] = m.rows;
        m.offsets[e] = at;
        at += m.counts[e];
        m.fill[e] = 0;
        if (m.tile_start) {
            m.tile_start[e] = tiles;
            tiles += (m.counts[e] + m.tile_rows - 1) / m.tile_rows;
        }
    }
    if (m.tile_start) m.tile_start[E + S] = tiles;
}

// grid rows, 256 threads: copy the row into each of its groups
__global__ void __launch_bounds__(256) k_moe_gather(MoeRowsArgs m) {
    __shared__ int dst[kMaxTopK + 8];
    const int t = blockIdx.x, E = m.a.experts, S = m.a.shared, kmax = m.a.kmax, h = m.a.h;
    const int active = m.a.active[t];
    if ((int)threadIdx.x < active) {
        const int e = m.a.ids[(int64_t)t * kmax + threadIdx.x];
        const int row = m.offsets[e] + atomicAdd(&m.fill[e], 1);
        dst[threadIdx.x] = row;
        m.map[(int64_t)t * kmax + threadIdx.x] = row;
    } else if ((int)threadIdx.x >= kmax && (int)threadIdx.x < kmax + S) {
        dst[threadIdx.x - kmax + active] = m.offsets[E + threadIdx.x - kmax] + t;
    }
    __syncthreads();
    if (m.x_planes) {
        const uint4 *hi = (const uint4 *)(m.x_planes + (int64_t)t * h);
        const uint4 *lo = (const uint4 *)(m.x_planes + ((int64_t)m.rows + t) * h);
        for (int i = 0; i < active + S; ++i) {
            const int64_t row = dst[i];
            if (threadIdx.x == 0) m.xg_scale[row] = m.x_scale[t];
            uint4 *yh = (uint4 *)(m.xg_planes + row * h), *yl = (uint4 *)(m.xg_planes + ((int64_t)m.capacity + row) * h);
            for (int j = threadIdx.x; j < h / 8; j += 256) {
                yh[j] = hi[j];
                yl[j] = lo[j];
            }
        }
        return;
    }
    const float *x = m.a.x + (int64_t)t * h;
    for (int i = 0; i < active + S; ++i) {
        float *y = m.xg + (int64_t)dst[i] * h;
        for (int j = threadIdx.x * 4; j < h; j += 256 * 4) *(float4 *)(y + j) = load_f4(x + j);
    }
}

// grid rows, 256 threads: k_moe_down's accumulation order per element
__global__ void __launch_bounds__(256) k_moe_combine(MoeRowsArgs m, const float *y, float *x) {
    const int t = blockIdx.x, E = m.a.experts, S = m.a.shared, kmax = m.a.kmax, h = m.a.h;
    const int active = m.a.active[t];
    float *xr = x + (int64_t)t * h;
    for (int j = threadIdx.x; j < h; j += 256) {
        float total = 0.0f;
        for (int i = 0; i < active; ++i)
            total = total + m.a.weights[(int64_t)t * kmax + i] * y[(int64_t)m.map[(int64_t)t * kmax + i] * h + j];
        for (int e = 0; e < S; ++e) total = total + m.a.shared_scale * y[(int64_t)(m.offsets[E + e] + t) * h + j];
        xr[j] = xr[j] + m.a.scale * total;
    }
}


}  // namespace

bool heavy_kv_fused(int dtype, int latent) {
    return dtype == MR_F32    ? block_gemv_fits<MR_F32>(latent)
           : dtype == MR_BF16 ? block_gemv_fits<MR_BF16>(latent)
           : dtype == MR_F16  ? block_gemv_fits<MR_F16>(latent)
                              : false;
}

bool heavy_split_path(int d, int window, int context, int block, int slots) {
    const int blocks = (context + block - 1) / block;
    return split::head_dim_ok(d) && heavy_parts(window, context) <= split::kMaxParts && slots <= kHeavyMaxChosen &&
           heavy_split_lds(d, blocks) <= 64 * 1024;
}

int launch_heavy_attention(hipStream_t s, const HeavyAttnArgs &a, int context) {
    MR_REQUIRE(a.heads % a.kv_heads == 0 && a.d % 2 == 0 && a.block > 0 && a.slots > 0, "heavy attention: bad geometry");
    if (a.kv_w) {
        MR_REQUIRE(heavy_kv_fused(a.kv_dtype, a.latent), "heavy attention: unsupported latent projection");
        const size_t lds = (size_t)(((a.latent + 3) & ~3) + a.d) * sizeof(float);
        const int grid = a.heads + 2 * a.kv_heads;
        if (a.kv_dtype == MR_BF16) k_heavy_kv<MR_BF16><<<grid, kKvThreads, lds, s>>>(a);
        else if (a.kv_dtype == MR_F16) k_heavy_kv<MR_F16><<<grid, kKvThreads, lds, s>>>(a);
        else k_heavy_kv<MR_F32><<<grid, kKvThreads, lds, s>>>(a);
    } else {
        k_heavy_prep<<<a.heads + a.kv_heads, 64, (size_t)5 * a.d * sizeof(float), s>>>(a);
    }
    MR_LAUNCHED("enqueue heavy attention prologue");
    const int blocks = (context + a.block - 1) / a.block;
    if (a.part && heavy_split_path(a.d, a.window, context, a.block, a.slots)) {
        const int parts = heavy_parts(a.window, context);
        const dim3 grid(parts, a.heads);
        const size_t lds = heavy_split_lds(a.d, blocks);
        switch (a.d) {
            case 128:
                k_heavy_attn_split<128><<<grid, split::kThreads, lds, s>>>(a);
                MR_LAUNCHED("enqueue heavy attention splits");
                k_heavy_attn_merge<128><<<a.heads, split::kThreads, 0, s>>>(a, parts);
                break;
            case 64:
                k_heavy_attn_split<64><<<grid, split::kThreads, lds, s>>>(a);
                MR_LAUNCHED("enqueue heavy attention splits");
                k_heavy_attn_merge<64><<<a.heads, split::kThreads, 0, s>>>(a, parts);
                break;
            default:
                k_heavy_attn_split<32><<<grid, split::kThreads, lds, s>>>(a);
                MR_LAUNCHED("enqueue heavy attention splits");
                k_heavy_attn_merge<32><<<a.heads, split::kThreads, 0, s>>>(a, parts);
                break;
        }
        MR_LAUNCHED("enqueue heavy attention merge");
        return MR_OK;
    }
    const size_t lds = (size_t)(a.d + std::min(a.window, context) + blocks) * sizeof(float) + (size_t)blocks * sizeof(int);
    MR_REQUIRE(lds <= 64 * 1024, "heavy attention: window and block count exceed shared memory");
    switch (a.d) {
        case 128: k_heavy_attn_lanes<128><<<a.heads, kAttnThreads, lds, s>>>(a); break;
        case 64: k_heavy_attn_lanes<64><<<a.heads, kAttnThreads, lds, s>>>(a); break;
        case 32: k_heavy_attn_lanes<32><<<a.heads, kAttnThreads, lds, s>>>(a); break;
        default: k_heavy_attn<<<a.heads, kAttnThreads, lds, s>>>(a); break;
    }
    MR_LAUNCHED("enqueue heavy attention");
    return MR_OK;
}

int launch_moe(hipStream_t s, const MoeArgs &a) {
    MR_REQUIRE(a.experts >= 1 && a.experts <= kMaxExperts && a.groups >= 1 && a.groups <= a.experts &&
                   a.kmin >= 1 && a.kmin <= a.kmax && a.kmax <= std::min(a.experts, kMaxTopK),
               "moe: routing geometry out of range");
    const int slots = a.kmax + a.shared;
    const size_t lds = (size_t)slots * a.ffn * sizeof(float);
    MR_REQUIRE(lds <= 64 * 1024, "moe: expert activations exceed shared memory");
    const bool fast = a.dtype == MR_BF16 && a.h % 8 == 0 && a.ffn % 8 == 0 && a.kmax + a.shared <= kMoeMaxSlots;
    if (!fast) {
        k_moe_route<<<1, kWave, 0, s>>>(a);
        MR_LAUNCHED("enqueue moe routing");
    }
    if (fast) {
        k_moe_gate_up_bf16<<<dim3(ceil_div(a.ffn, kMoeRows * kMoeGuRows), slots), kMoeThreads,
                             (size_t)a.h * sizeof(float), s>>>(a);
    } else {
        k_moe_gate_up<<<dim3(ceil_div(a.ffn, kMoeRows), slots), kMoeThreads, (size_t)a.h * sizeof(float), s>>>(a);
    }
    MR_LAUNCHED("enqueue moe gate/up");
    if (fast)
        k_moe_down_bf16<<<ceil_div(a.h, kMoeRows), kMoeThreads, lds, s>>>(a);
    else
        k_moe_down<<<ceil_div(a.h, kMoeRows), kMoeThreads, lds, s>>>(a);
    MR_LAUNCHED("enqueue moe down");
    return MR_OK;
}

int launch_heavy_scan(hipStream_t s, const HeavyScanArgs &a) {
    MR_REQUIRE(a.ring_k && a.ring_v && a.bsum_k && a.bsum_v && a.sums && a.rows > 0 && a.kvw > 0 && a.block > 0,
               "heavy scan: bad arguments");
    const int first = a.p0 / a.block, last = (a.p0 + a.rows - 1) / a.block;
    k_heavy_scan<<<dim3(last - first + 1, ceil_div(2 * a.kvw, 256)), 256, 0, s>>>(a);
    MR_LAUNCHED("enqueue heavy block scan");
    return MR_OK;
}

int launch_heavy_select(hipStream_t s, const HeavySelectArgs &a) {
    MR_REQUIRE(a.qkv && a.bsum_k && a.bsum_v && a.sums && a.ext && a.rows > 0 && a.slots <= kHeavyMaxChosen &&
                   a.kv_heads > 0 && a.heads % a.kv_heads == 0,
               "heavy select: bad arguments");
    const int blocks = ceil_div(a.p0 + a.rows, a.block);
    const size_t lds = (size_t)kSelHeads * (a.d + 2 * blocks) * sizeof(float);   // per wave: q, scores, flags
    MR_REQUIRE(lds <= 64 * 1024, "heavy select: too many blocks for shared memory");
    const dim3 grid(a.rows, ceil_div(a.heads, kSelHeads));
    switch (a.d) {
        case 128: k_heavy_select<128><<<grid, kSelThreads, lds, s>>>(a); break;
        case 64: k_heavy_select<64><<<grid, kSelThreads, lds, s>>>(a); break;
        case 32: k_heavy_select<32><<<grid, kSelThreads, lds, s>>>(a); break;
        default: return fail(MR_ERR_INVALID, "heavy select: head_dim must be 32, 64 or 128");
    }
    MR_LAUNCHED("enqueue heavy block selection");
    return MR_OK;
}

int launch_moe_route_rows(hipStream_t s, const MoeRowsArgs &m) {
    const MoeArgs &a = m.a;
    MR_REQUIRE(a.experts >= 1 && a.experts <= kMaxExperts && a.groups >= 1 && a.groups <= a.experts &&
                   a.kmin >= 1 && a.kmin <= a.kmax && a.kmax <= std::min(a.experts, kMaxTopK) && a.shared <= 8 &&
                   m.rows > 0 && a.h % 4 == 0,
               "moe rows: routing geometry out of range");
    const int groups = a.experts + a.shared;
    k_moe_zero<<<ceil_div(groups, 256), 256, 0, s>>>(m.counts, groups);
    MR_LAUNCHED("enqueue moe count clear");
    k_moe_route_rows<<<m.rows, kWave, 0, s>>>(m);
    MR_LAUNCHED("enqueue moe row routing");
    k_moe_offsets<<<1, 1, 0, s>>>(m);
    MR_LAUNCHED("enqueue moe group offsets");
    k_moe_gather<<<m.rows, 256, 0, s>>>(m);
    MR_LAUNCHED("enqueue moe gather");
    return MR_OK;
}

int launch_moe_combine_rows(hipStream_t s, const MoeRowsArgs &m, const float *y, float *x) {
    k_moe_combine<<<m.rows, 256, 0, s>>>(m, y, x);
    MR_LAUNCHED("enqueue moe combine");
    return MR_OK;
}

}  // namespace mr
