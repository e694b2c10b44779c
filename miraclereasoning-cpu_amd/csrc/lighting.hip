// flashlighting-2.0 token-step kernels (model.py:146-190).
//
// The reference recomputes, every step, the keys and values of every stored
// latent row (model.py:159-162).  A row's key depends only on its latent and
// its stored position, and its value only on its latent, so this build keeps a
// key and a value cache row per latent row and computes one only when a row is
// created: the new row of each step, and the row a merge produces.
//
// Per layer and step: k_light_prep (queries: RMSNorm with q_norm + RoPE; the
// new latent: RMSNorm with latent_norm, appended with its position and count
// 1), the K/V projection of the new latent, k_light_store (its K: RMSNorm with
// k_norm + RoPE at its position; its V), k_light_attend (scores over every row,
// latent_mask, softmax, mix: kernels.cl's sequential orders), k_light_compact
// (model.py:168-188: drop the overflow without memory slots; merge the two
// oldest rows by their counts when the overflow exceeds the slots; else mark
// the overflow as memory rows), then - when a merge happened - the K/V
// projection of the merged row and its cache row at its new position.
#include "lighting.h"

#include "attention_tile.h"

namespace mr {
namespace {

// RMSNorm of one row (kernels.cl:19-28) by one 64-lane workgroup: the row is
// staged in LDS, each lane sums the squares of its strided elements and a
// wave reduction adds the lanes (an FP32 reordering of the reference's
// sequential sum).
__device__ __forceinline__ void rms_row(const float *x, const float *gain, float eps, int width, float *y, float *scale) {
    float v = 0.0f;
    for (int j = threadIdx.x; j < width; j += blockDim.x) {
        const float t = x[j];
        y[j] = t;
        v = fmaf(t, t, v);
    }
    v = wave_sum(v);
    const float sc = 1.0f / sqrtf(v / (float)width + eps);
    if (threadIdx.x == 0) *scale = sc;
    for (int j = threadIdx.x; j < width; j += blockDim.x) y[j] = y[j] * sc * (gain ? gain[j] : 1.0f);
    __syncthreads();
}

// RoPE of one head row in LDS at integer position p (kernels.cl:30-44).
__device__ __forceinline__ void rope_row(float *row, const float *rope, int p, int d, int split_half) {
    const int half = d / 2;
    const float *cs = rope + (int64_t)p * half * 2;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const int j = split_half ? i : 2 * i, k = split_half ? i + half : 2 * i + 1;
        float u = row[j], v = row[k];
        rope_rotate(u, v, cs[2 * i], cs[2 * i + 1]);
        row[j] = u;
        row[k] = v;
    }
    __syncthreads();
}

// grid heads + 1, 64 threads: blocks < heads rotate queries, the last appends
// the new latent row.
__global__ void __launch_bounds__(64) k_light_prep(LightArgs a) {
    extern __shared__ float row[];
    __shared__ float scale;
    if (a.done && *a.done) return;
    const int pos = *a.pos;
    if ((int)blockIdx.x < a.heads) {
        const int h = blockIdx.x;
        rms_row(a.qlat + (int64_t)h * a.d, a.q_gain, a.eps, a.d, row, &scale);
        rope_row(row, a.rope, pos, a.d, a.split_half);
        for (int j = threadIdx.x; j < a.d; j += blockDim.x) a.q_rot[(int64_t)h * a.d + j] = row[j];
        return;
    }
    rms_row(a.qlat + (int64_t)a.heads * a.d, a.latent_gain, a.eps, a.latent, row, &scale);
    const LightState st = *a.st;
    const int slot = (st.start + st.rows) % a.cap;
    for (int j = threadIdx.x; j < a.latent; j += blockDim.x) {
        a.arena[(int64_t)slot * a.latent + j] = row[j];
        a.lat_new[j] = row[j];
    }
    if (threadIdx.x == 0) {
        a.positions[slot] = (float)pos;
        a.counts[slot] = 1.0f;
    }
}

// grid kv_heads, 64 threads: cache row of the new (merged = false) or merged row.
__global__ void __launch_bounds__(64) k_light_store(LightArgs a, int merged) {
    extern __shared__ float row[];
    __shared__ float scale;
    if (a.done && *a.done) return;
    const LightState st = *a.st;
    if (merged && st.skip_merged) return;
    const int slot = merged ? st.merged_slot : (st.start + st.rows) % a.cap;
    const int p = (int)a.positions[slot];
    const int kh = blockIdx.x, kvw = a.kv_heads * a.d;
    rms_row(a.kv + (int64_t)kh * a.d, a.k_gain, a.eps, a.d, row, &scale);
    rope_row(row, a.rope, p, a.d, a.split_half);
    for (int j = threadIdx.x; j < a.d; j += blockDim.x) {
        a.kcache[(int64_t)slot * kvw + (int64_t)kh * a.d + j] = row[j];
        a.vcache[(int64_t)slot * kvw + (int64_t)kh * a.d + j] = a.kv[kvw + (int64_t)kh * a.d + j];
    }
}

constexpr int kThreads = 256;

// grid heads, kThreads: attention of query head h over every row.
__global__ void __launch_bounds__(kThreads) k_light_attend(LightArgs a) {
    extern __shared__ float sh[];
    __shared__ float red[kThreads / 64];
    __shared__ float denom;
    if (a.done && *a.done) return;
    const int pos = *a.pos, d = a.d, tid = threadIdx.x;
    const LightState st = *a.st;
    const int n = st.rows + 1;   // with this step's row
    const int h = blockIdx.x, kh = h / (a.heads / a.kv_heads), kvw = a.kv_heads * d;
    const float earliest = (float)(pos - a.window + 1);
    float *qs = sh, *sc = sh + d;
    for (int j = tid; j < d; j += kThreads) qs[j] = a.q_rot[(int64_t)h * d + j];
    __syncthreads();
    const float root = sqrtf((float)d);
    for (int t = tid; t < n; t += kThreads) {   // kernels.cl:58-73, then latent_mask (86-91)
        const int slot = (st.start + t) % a.cap;
        const float *kr = a.kcache + (int64_t)slot * kvw + (int64_t)kh * d;
        float v = 0.0f;
        for (int j = 0; j < d; ++j) v += qs[j] * kr[j];
        v = v / root;
        if (t >= st.memory && a.positions[slot] < earliest) v = -INFINITY;
        sc[t] = v;
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int t = tid; t < n; t += kThreads) mx = fmaxf(mx, sc[t]);
    mx = block_max(mx, red);
    if (tid == 0) {   // kernels.cl:75-84
        float den = 0.0f;
        for (int t = 0; t < n; ++t) den += expf(sc[t] - mx);
        denom = den;
    }
    __syncthreads();
    for (int t = tid; t < n; t += kThreads) sc[t] = expf(sc[t] - mx) / denom;
    __syncthreads();
    for (int j = tid; j < d; j += kThreads) {   // kernels.cl:93-107
        float acc = 0.0f;
        for (int t = 0; t < n; ++t)
            acc += sc[t] * a.vcache[(int64_t)((st.start + t) % a.cap) * kvw + (int64_t)kh * d + j];
        a.out[(int64_t)h * d + j] = acc;
    }
}

// Split-key form of the same attention for head dims 32/64/128: workgroup
// (split s, head h) scores rows [64 s, 64 s + 64) of the memory with the
// latent mask and writes its partial (m, l, o); a second kernel merges the
// splits of each head.  A lane holds 16 dims of a row (D/16 lanes per row),
// each lane group keeps its own running max, sum and weighted values.
constexpr int kPartThreads = 256;

template <int D>
__global__ void __launch_bounds__(kPartThreads) k_light_attend_part(LightArgs a) {
    constexpr int LPK = D / 16;                 // lanes per row
    constexpr int KPW = kWave / LPK;            // rows side by side in a wave
    constexpr int NWV = kPartThreads / kWave;
    __shared__ float wm[NWV], wl[NWV], wo[NWV][D];
    if (a.done && *a.done) return;
    const LightState st = *a.st;
    const int n = st.rows + 1;                  // with this step's row
    const int t0 = blockIdx.x * kLightRows;
    if (t0 >= n) return;
    const int t1 = min(n, t0 + kLightRows);
    const int h = blockIdx.y, kh = h / (a.heads / a.kv_heads), kvw = a.kv_heads * D;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane % LPK, kg = lane / LPK;
    const float earliest = (float)(*a.pos - a.window + 1);
    const float inv_root = 1.0f / sqrtf((float)D);
    float4 q[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const float4 t = load_f4(a.q_rot + (int64_t)h * D + 16 * sub + 4 * c);
        q[c] = make_float4(t.x * inv_root, t.y * inv_root, t.z * inv_root, t.w * inv_root);
    }
    float m = -INFINITY, l = 0.0f;
    float4 acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int r0 = t0 + wave * KPW; r0 < t1; r0 += NWV * KPW) {
        const int t = r0 + kg;
        float s = -INFINITY;
        float4 v[4];
        if (t < t1) {
            const int slot = (st.start + t) % a.cap;
            // latent_mask (kernels.cl:86-91): non-memory rows older than the window
            if (!(t >= st.memory && a.positions[slot] < earliest)) {
                const float *kr = a.kcache + (int64_t)slot * kvw + (int64_t)kh * D + 16 * sub;
                const float *vr = a.vcache + (int64_t)slot * kvw + (int64_t)kh * D + 16 * sub;
                float dot = 0.0f;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float4 k4 = load_f4(kr + 4 * c);
                    v[c] = load_f4(vr + 4 * c);
                    dot = fmaf(q[c].x, k4.x, dot);
                    dot = fmaf(q[c].y, k4.y, dot);
                    dot = fmaf(q[c].z, k4.z, dot);
                    dot = fmaf(q[c].w, k4.w, dot);
                }
                s = dot;
            }
        }
        s = att::lanes_sum<LPK>(s == -INFINITY ? 0.0f : s) + (s == -INFINITY ? -INFINITY : 0.0f);
        const float m_new = fmaxf(m, s);
        if (m_new != -INFINITY) {
            const float alpha = m == -INFINITY ? 0.0f : __expf(m - m_new);
            const float p = s == -INFINITY ? 0.0f : __expf(s - m_new);
            l = l * alpha + p;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                acc[c].x = acc[c].x * alpha + (p != 0.0f ? p * v[c].x : 0.0f);
                acc[c].y = acc[c].y * alpha + (p != 0.0f ? p * v[c].y : 0.0f);
                acc[c].z = acc[c].z * alpha + (p != 0.0f ? p * v[c].z : 0.0f);
                acc[c].w = acc[c].w * alpha + (p != 0.0f ? p * v[c].w : 0.0f);
            }
            m = m_new;
        }
    }
    // fold the wave's row groups: common max, rescale, sum
    const float M = att::keygroups_max<LPK>(m);
    const float f = m == -INFINITY ? 0.0f : __expf(m - M);
    const float L = att::keygroups_sum<LPK>(l * f);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const float ox = att::keygroups_sum_lanes<LPK>(acc[c].x * f);
        const float oy = att::keygroups_sum_lanes<LPK>(acc[c].y * f);
        const float oz = att::keygroups_sum_lanes<LPK>(acc[c].z * f);
        const float ow = att::keygroups_sum_lanes<LPK>(acc[c].w * f);
        if (kg == 0) *(float4 *)&wo[wave][16 * sub + 4 * c] = make_float4(ox, oy, oz, ow);
    }
    if (lane == 0) {
        wm[wave] = M;
        wl[wave] = L;
    }
    __syncthreads();
    float *part = a.part + ((int64_t)h * gridDim.x + blockIdx.x) * (D + 2);
    float Mb = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWV; ++w) Mb = fmaxf(Mb, wm[w]);
    for (int j = threadIdx.x; j < D; j += kPartThreads) {
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < NWV; ++w)
            if (wm[w] != -INFINITY) o = fmaf(wo[w][j], __expf(wm[w] - Mb), o);
        part[2 + j] = o;
    }
    if (threadIdx.x == 0) {
        float Lb = 0.0f;
#pragma unroll
        for (int w = 0; w < NWV; ++w)
            if (wm[w] != -INFINITY) Lb = fmaf(wl[w], __expf(wm[w] - Mb), Lb);
        part[0] = Mb;
        part[1] = Lb;
    }
}

// grid heads, kMergeThreads: out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s.
// The split weights e^(m_s - M) go to LDS; lane quads cover D/4 float4
// columns and kMergeThreads / (D/4) split groups stride the splits, folded
// through LDS at the end.
constexpr int kMergeThreads = 256;

template <int D>
__global__ void __launch_bounds__(kMergeThreads) k_light_attend_merge(LightArgs a, int splits) {
    constexpr int Q = D / 4, G = kMergeThreads / Q;
    __shared__ float e[kLightMaxSplits], red[kMergeThreads / kWave];
    __shared__ float4 fold[G][Q];
    __shared__ float lsum[G];
    if (a.done && *a.done) return;
    const int n = a.st->rows + 1, active = min(splits, (n + kLightRows - 1) / kLightRows);
    const int h = blockIdx.x, tid = threadIdx.x;
    const float *part = a.part + (int64_t)h * splits * (D + 2);
    float mx = -INFINITY;
    for (int s = tid; s < active; s += kMergeThreads) {
        const float ms = part[(int64_t)s * (D + 2)];
        e[s] = ms;
        mx = fmaxf(mx, ms);
    }
    const float M = block_max(mx, red);
    for (int s = tid; s < active; s += kMergeThreads) e[s] = e[s] == -INFINITY ? 0.0f : __expf(e[s] - M);
    __syncthreads();
    const int g = tid / Q, c = tid % Q;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    float l = 0.0f;
#pragma unroll 4
    for (int s = g; s < active; s += G) {
        const float w = e[s];
        const float *ps = part + (int64_t)s * (D + 2);
        const float4 v = make_float4(ps[2 + 4 * c], ps[3 + 4 * c], ps[4 + 4 * c], ps[5 + 4 * c]);
        if (c == 0) l = fmaf(ps[1], w, l);
        o.x = fmaf(v.x, w, o.x);
        o.y = fmaf(v.y, w, o.y);
        o.z = fmaf(v.z, w, o.z);
        o.w = fmaf(v.w, w, o.w);
    }
    fold[g][c] = o;
    if (c == 0) lsum[g] = l;
    __syncthreads();
    if (tid < Q) {
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        float L = 0.0f;
#pragma unroll
        for (int k = 0; k < G; ++k) {
            t.x += fold[k][tid].x;
            t.y += fold[k][tid].y;
            t.z += fold[k][tid].z;
            t.w += fold[k][tid].w;
            L += lsum[k];
        }
        float *out = a.out + (int64_t)h * D + 4 * tid;
        out[0] = t.x / L;
        out[1] = t.y / L;
        out[2] = t.z / L;
        out[3] = t.w / L;
    }
}

// One workgroup: compaction after this step's attention (model.py:168-188).
__global__ void __launch_bounds__(64) k_light_compact(LightArgs a) {
    __shared__ LightState st;
    __shared__ int mode;   // 0 keep, 1 drop, 2 merge
    if (a.done && *a.done) return;
    if (threadIdx.x == 0) {
        st = *a.st;
        const int n = st.rows + 1, overflow = max(0, n - a.window);
        st.skip_merged = 1;
        if (a.memory_slots == 0 && overflow > 0) {
            mode = 1;
            st.start = (st.start + overflow) % a.cap;
            st.rows = n - overflow;
            st.memory = 0;
        } else if (overflow > a.memory_slots) {
            mode = 2;
        } else {
            mode = 0;
            st.rows = n;
            st.memory = overflow;
        }
    }
    __syncthreads();
    if (mode == 2) {
        const int s0 = st.start, s1 = (st.start + 1) % a.cap;
        const float ca = a.counts[s0], cb = a.counts[s1];
        for (int j = threadIdx.x; j < a.latent; j += blockDim.x) {   // kernels.cl merge_rows
            const float v = (ca * a.arena[(int64_t)s0 * a.latent + j] + cb * a.arena[(int64_t)s1 * a.latent + j]) /
                            (ca + cb);
            a.arena[(int64_t)s1 * a.latent + j] = v;
            a.lat_new[j] = v;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            const float centre = (a.positions[s0] * ca + a.positions[s1] * cb) / (ca + cb);
            a.positions[s1] = rintf(centre);
            a.counts[s1] = ca + cb;
            st.start = s1;
            st.rows = st.rows;   // n - 1 = previous rows
            st.memory = a.memory_slots;
            st.skip_merged = 0;
            st.merged_slot = s1;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) *a.st = st;
}

__global__ void k_light_residual(float *hidden, const float *o, const float *f, const float *ag, const float *fg,
                                 float rs, int n, const int *done) {
    if (done && *done) return;
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    const float branch = (0.0f + ag[0] * o[j]) + fg[0] * f[j];
    hidden[j] = hidden[j] + rs * branch;
}

}  // namespace

int launch_light_prep(hipStream_t s, const LightArgs &a) {
    k_light_prep<<<a.heads + 1, 64, (size_t)std::max(a.d, a.latent) * sizeof(float), s>>>(a);
    MR_LAUNCHED("enqueue latent prologue");
    return MR_OK;
}

int launch_light_store_kv(hipStream_t s, const LightArgs &a, bool merged) {
    k_light_store<<<a.kv_heads, 64, (size_t)a.d * sizeof(float), s>>>(a, merged ? 1 : 0);
    MR_LAUNCHED("enqueue latent key/value row");
    return MR_OK;
}

int launch_light_attend(hipStream_t s, const LightArgs &a) {
    if (light_split_path(a.d, a.cap) && a.part) {
        const int splits = light_splits(a.cap);
        const dim3 grid(splits, a.heads);
        switch (a.d) {
            case 128:
                k_light_attend_part<128><<<grid, kPartThreads, 0, s>>>(a);
                MR_LAUNCHED("enqueue latent attention splits");
                k_light_attend_merge<128><<<a.heads, kMergeThreads, 0, s>>>(a, splits);
                break;
            case 64:
                k_light_attend_part<64><<<grid, kPartThreads, 0, s>>>(a);
                MR_LAUNCHED("enqueue latent attention splits");
                k_light_attend_merge<64><<<a.heads, kMergeThreads, 0, s>>>(a, splits);
                break;
            default:
                k_light_attend_part<32><<<grid, kPartThreads, 0, s>>>(a);
                MR_LAUNCHED("enqueue latent attention splits");
                k_light_attend_merge<32><<<a.heads, kMergeThreads, 0, s>>>(a, splits);
                break;
        }
        MR_LAUNCHED("enqueue latent attention merge");
    } else {
        const size_t lds = (size_t)(a.d + a.cap) * sizeof(float);
        MR_REQUIRE(lds <= 64 * 1024, "latent attention: window and memory slots exceed shared memory");
        k_light_attend<<<a.heads, kThreads, lds, s>>>(a);
        MR_LAUNCHED("enqueue latent attention");
    }
    k_light_compact<<<1, 64, 0, s>>>(a);
    MR_LAUNCHED("enqueue latent compaction");
    return MR_OK;
}

int launch_light_residual(hipStream_t s, float *hidden, const float *o, const float *f, const float *attention_gate,
                          const float *ffn_gate, float rs, int n, const int *done) {
    k_light_residual<<<ceil_div(n, 256), 256, 0, s>>>(hidden, o, f, attention_gate, ffn_gate, rs, n, done);
    MR_LAUNCHED("enqueue gated residual");
    return MR_OK;
}

}  // namespace mr
