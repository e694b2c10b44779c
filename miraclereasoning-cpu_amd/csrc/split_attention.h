// Split-key decode attention of one query head: a workgroup scores a range of
// cached rows and writes its partial (m, l, o) = (max score, sum of e^(s - m),
// sum of e^(s - m) v); a second kernel merges the partials of each head,
// out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s.  Used by the
// latent-memory (flashlighting-2.0) and block-sparse (heavy-medium-2.0) step
// kernels for head dims 32/64/128.
#pragma once

#include "attention_tile.h"

namespace mr {
namespace split {

constexpr int kRows = 64;          // cached rows per split
constexpr int kThreads = 256;      // threads of a partial or merge workgroup
constexpr int kMaxParts = 1024;    // partials per head the merge holds in LDS

__host__ __device__ constexpr bool head_dim_ok(int d) { return d == 32 || d == 64 || d == 128; }

// Partial of the query head q (D floats, global) over rows [t0, t1).
// rows(t, &k, &v) returns the head slices of row t's key and value, or false
// for a masked row.  Scores are (q / sqrt(D)) . k.  A lane holds 16 dims of a
// row (D/16 lanes per row); each lane group keeps its own running max, sum and
// weighted values, folded over the wave and then the workgroup.  Every row
// masked gives (-inf, 0, 0).
template <int D, class Rows>
__device__ __forceinline__ void partial(const float *q_head, int t0, int t1, Rows rows, float *part) {
    constexpr int LPK = D / 16;            // lanes per row
    constexpr int KPW = kWave / LPK;       // rows side by side in a wave
    constexpr int NWV = kThreads / kWave;
    __shared__ float wm[NWV], wl[NWV], wo[NWV][D];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane % LPK, kg = lane / LPK;
    const float inv_root = 1.0f / sqrtf((float)D);
    float4 q[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const float4 t = load_f4(q_head + 16 * sub + 4 * c);
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
        const float *kr, *vr;
        if (t < t1 && rows(t, &kr, &vr)) {
            kr += 16 * sub;
            vr += 16 * sub;
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
        s = att::lanes_sum<LPK>(s == -INFINITY ? 0.0f : s) + (s == -INFINITY ? -INFINITY : 0.0f);
        const float m_new = fmaxf(m, s);
        if (m_new != -INFINITY) {
            const float alpha = m == -INFINITY ? 0.0f : expf(m - m_new);
            const float p = s == -INFINITY ? 0.0f : expf(s - m_new);
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
    const float f = m == -INFINITY ? 0.0f : expf(m - M);
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
    float Mb = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWV; ++w) Mb = fmaxf(Mb, wm[w]);
    for (int j = threadIdx.x; j < D; j += kThreads) {
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < NWV; ++w)
            if (wm[w] != -INFINITY) o = fmaf(wo[w][j], expf(wm[w] - Mb), o);
        part[2 + j] = o;
    }
    if (threadIdx.x == 0) {
        float Lb = 0.0f;
#pragma unroll
        for (int w = 0; w < NWV; ++w)
            if (wm[w] != -INFINITY) Lb = fmaf(wl[w], expf(wm[w] - Mb), Lb);
        part[0] = Mb;
        part[1] = Lb;
    }
}

// Merge of one head's partials part[0 .. n) and, when extra >= 0, part[extra]
// (each D + 2 floats apart) into out[0 .. D).  The split weights e^(m_s - M) go
// to LDS; lane quads cover D/4 float4 columns and kThreads / (D/4) split
// groups stride the partials, folded through LDS at the end.
// The first kPre column groups of each thread are loaded together with the
// maxima (clamped, so the loads issue at once), which saves the second round
// trip for up to kPre * G partials.
constexpr int kPre = 12;

template <int D>
__device__ __forceinline__ void merge(const float *part, int n, int extra, float *out) {
    constexpr int Q = D / 4, G = kThreads / Q;
    __shared__ float e[kMaxParts], red[kThreads / kWave];
    __shared__ float4 fold[G][Q];
    __shared__ float lsum[G];
    const int tid = threadIdx.x, total = n + (extra >= 0 ? 1 : 0);
    const int g = tid / Q, c = tid % Q;
    float4 pv[kPre];
    float pl[kPre];
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
        const int s = max(0, min(g + i * G, total - 1));
        const float *ps = part + (int64_t)(s < n ? s : extra) * (D + 2);
        pv[i] = make_float4(ps[2 + 4 * c], ps[3 + 4 * c], ps[4 + 4 * c], ps[5 + 4 * c]);
        pl[i] = ps[1];
    }
    float mx = -INFINITY;
    for (int s = tid; s < total; s += kThreads) {
        const float ms = part[(int64_t)(s < n ? s : extra) * (D + 2)];
        e[s] = ms;
        mx = fmaxf(mx, ms);
    }
    const float M = block_max(mx, red);
    for (int s = tid; s < total; s += kThreads) e[s] = e[s] == -INFINITY ? 0.0f : expf(e[s] - M);
    __syncthreads();
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    float l = 0.0f;
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
        const int s = g + i * G;
        if (s < total) {
            const float w = e[s];
            if (c == 0) l = fmaf(pl[i], w, l);
            o.x = fmaf(pv[i].x, w, o.x);
            o.y = fmaf(pv[i].y, w, o.y);
            o.z = fmaf(pv[i].z, w, o.z);
            o.w = fmaf(pv[i].w, w, o.w);
        }
    }
#pragma unroll 4
    for (int s = g + kPre * G; s < total; s += G) {
        const float w = e[s];
        const float *ps = part + (int64_t)(s < n ? s : extra) * (D + 2);
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
        float *dst = out + 4 * tid;
        dst[0] = t.x / L;
        dst[1] = t.y / L;
        dst[2] = t.z / L;
        dst[3] = t.w / L;
    }
}

}  // namespace split
}  // namespace mr
