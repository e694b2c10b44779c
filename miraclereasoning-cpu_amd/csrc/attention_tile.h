// Device code of the split-key attention unit, shared by the standalone
// attention kernel (attention.hip) and the persistent step kernel (step.hip).
//
// A unit (split, kh) owns the G = heads/kv_heads query heads that share KV head
// kh (kernels.cl:66 mapping) and a contiguous range of the logical keys
// [ring window, extra rows] (kernels.cl:67-68).  It scores them (dot /
// sqrt(dim), kernels.cl:72), keeps a running max m and l = sum exp(s - m),
// accumulates o = sum exp(s - m) v, and writes (m, l, o).  Merging the units of
// a head, out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s, gives the
// softmax-weighted value sum of kernels.cl:75-107 up to rounding.
//
// Keys and values stream through LDS in 16 KB tiles (4096 floats = 4096/dim
// keys), each thread loading 4 float4 of K and 4 of V per tile, coalesced along
// the row; the next tile is prefetched into registers while the current one is
// consumed (the tile loop's barriers order LDS only, so the prefetch stays in
// flight across them).  LL = true is the persistent kernel's mode: q/k/v arrive as
// flag-in-data cells (ll.h) of this step, the partials are exchanged between
// workgroups with agent-coherent accesses, and the merged output is written as
// cells.
#pragma once

#include "attention.h"
#include "ll.h"

namespace mr {
namespace att {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kTileFloats = 4096;
constexpr int kMaxG = 16;

struct Args {
    AttnStepArgs s;       // engine fields (mode 1)
    int mode;             // 0 = op-level, 1 = engine step
    int start, length, extra_length;   // mode 0 geometry
    const float *ring_k_ro, *ring_v_ro;
};

struct Geo {
    int pos, start, length, extra, total;
};

// LL-mode epochs: inputs (q/k/v cells) and output (merged cells); in that mode
// AttnStepArgs' q, k_new, v_new and out point at uint64_t cells.  The inputs'
// producers report progress in ready[0..nready) (ll.h progress words).
struct Io {
    unsigned ep_in, ep_out;
    int *err;
    const unsigned *ready;
    int nready;
};

template <bool COH>
__device__ __forceinline__ float ld(const float *p) {
    if constexpr (COH)
        return __hip_atomic_load(gmem(const_cast<float *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *gmem(p);
}

template <bool COH>
__device__ __forceinline__ void st(float *p, float v) {
    if constexpr (COH) __hip_atomic_store(gmem(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *gmem(p) = v;
}

// Window geometry at position `pos` (engine) or from the arguments (op level).
__device__ __forceinline__ Geo geometry(const Args &ka, int pos) {
    const AttnStepArgs &a = ka.s;
    Geo g;
    if (ka.mode == 1) {
        g.pos = pos;
        int count = pos + 1;
        g.length = min(count, a.capacity);
        g.start = (count - g.length) % a.capacity;
        g.extra = a.extra_chunk ? (pos / a.extra_chunk) * a.extra_slots : 0;
    } else {
        g.pos = 0;
        g.start = ka.start;
        g.length = ka.length;
        g.extra = ka.extra_length;
    }
    g.total = g.length + g.extra;
    return g;
}

// Engine mode: normalize (optional) and rotate the G queries and the new key in
// LDS, then store the new key/value in the ring slot of this position (done by
// the unit that holds the newest key).
// Returns false (block-uniform) when an LL wait gave up.
// hs: the unit's group of the KV head's query heads (AttnStepArgs::head_groups);
// group 0 stores the new key/value.
template <bool LL, int NT>
__device__ __forceinline__ bool prepare(const Args &ka, const Geo &g, int kh, int G, int d, float *qs, float *kn,
                                        float *vn, int t0, int t1, const Io &io, int hs = 0) {
    const AttnStepArgs &a = ka.s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int half = d / 2;
    // Loads that do not depend on this step's values go out first: the RoPE
    // row of this position (a thread rotates pairs p = tid % half only, as
    // NT is a multiple of half) and the Q/K norm gains of its lanes.
    float rc = 1.0f, rsn = 0.0f, gq[2] = {1.0f, 1.0f}, gk[2] = {1.0f, 1.0f};
    if (ka.mode == 1) {
        const float *cs = a.rope + ((int64_t)g.pos * half + tid % half) * 2;
        rc = gmem(cs)[0];
        rsn = gmem(cs)[1];
        if (a.q_gain)
#pragma unroll
            for (int t = 0; t < 2; ++t)
                if (lane + kWave * t < d) {
                    gq[t] = gmem(a.q_gain)[lane + kWave * t];
                    gk[t] = gmem(a.k_gain)[lane + kWave * t];
                }
    }
    if constexpr (LL) {
        // Q/K/V cells of this head (indices relative to q: the cells are one
        // buffer), each thread polling at most a few pairs.
        ll::Wait w = ll::waiter(io.err);
        const uint64_t *cells = (const uint64_t *)a.q;
        const int q0 = (kh * a.head_groups + hs) * G * d;
        const int k0 = (int)((const uint64_t *)a.k_new - cells) + kh * d;
        const int v0 = (int)((const uint64_t *)a.v_new - cells) + kh * d;
        for (int i = 2 * tid; i < G * d + 2 * d; i += 2 * NT) {
            const int src = i < G * d ? q0 + i : (i < G * d + d ? k0 + i - G * d : v0 + i - G * d - d);
            float *dst = i < G * d ? qs + i : (i < G * d + d ? kn + i - G * d : vn + i - G * d - d);
            const float2 v = ll::get2(cells, src, io.ep_in, w);
            dst[0] = v.x;
            dst[1] = v.y;
        }
        if (!ll::all_ok(w)) return false;
    } else {
        const float *q_src = a.q + (int64_t)(kh * a.head_groups + hs) * G * d;
        for (int i = tid; i < G * d; i += NT) qs[i] = *gmem(q_src + i);
        if (ka.mode != 1) {
            __syncthreads();
            return true;
        }
        for (int j = tid; j < d; j += NT) {
            kn[j] = *gmem(a.k_new + kh * d + j);
            vn[j] = *gmem(a.v_new + kh * d + j);
        }
        __syncthreads();
    }
    if (a.q_gain) {   // per-head RMSNorm, width = dim (kernels.cl:19-28)
        for (int r = wave; r < G + 1; r += (NT / kWave)) {
            float *row = r < G ? qs + r * d : kn;
            float ss = 0.0f;
            for (int j = lane; j < d; j += kWave) ss = fmaf(row[j], row[j], ss);
            ss = wave_sum(ss);
            const float scale = 1.0f / sqrtf(ss / (float)d + a.eps);
            const float *gain = r < G ? a.q_gain : a.k_gain;
            for (int j = lane, t = 0; j < d; j += kWave, ++t)
                row[j] = row[j] * scale * (t < 2 ? (r < G ? gq[t] : gk[t]) : gmem(gain)[j]);
        }
        __syncthreads();
    }
    for (int i = tid; i < (G + 1) * half; i += NT) {   // RoPE at this position (kernels.cl:30-44)
        const int r = i / half, p = i % half;
        float *row = r < G ? qs + r * d : kn;
        const int j = a.split_half ? p : 2 * p, k = a.split_half ? p + half : 2 * p + 1;
        float u = row[j], v = row[k];
        if (NT % half == 0) rope_rotate(u, v, rc, rsn);
        else rope_rotate(u, v, gmem(a.rope)[((int64_t)g.pos * half + p) * 2], gmem(a.rope)[((int64_t)g.pos * half + p) * 2 + 1]);
        row[j] = u;
        row[k] = v;
    }
    __syncthreads();
    const int newest = g.length - 1;
    if (hs == 0 && t0 <= newest && newest < t1) {
        const int kvw = a.kv_heads * d;
        int64_t slot = (int64_t)(g.pos % a.capacity) * kvw + (int64_t)kh * d;
        for (int j = tid; j < d; j += NT) {
            gmem(a.ring_k)[slot + j] = kn[j];
            gmem(a.ring_v)[slot + j] = vn[j];
        }
    }
    return true;
}

// Key range of `split` for the current total (the split length follows the
// window so every split of the fixed grid has work).
template <int D>
__device__ __forceinline__ void split_range(const Geo &g, int splits, int split, int *t0, int *t1, int *len) {
    constexpr int T = kTileFloats / D;
    int split_len = (g.total + splits - 1) / splits;
    split_len = (split_len + T - 1) / T * T;
    *len = split_len;
    *t0 = min(split * split_len, g.total);
    *t1 = min(*t0 + split_len, g.total);
}

template <int D>
__host__ __device__ constexpr int unit_lds_floats(int G) {
    return 2 * (kTileFloats / D) * D + G * D + 2 * D + G * (kTileFloats / D) + 3 * kMaxG + 4;
}

// One (split, kh) unit: writes its partial (m, l, o) for the G heads.  Returns
// false (block-uniform) when an LL wait gave up.
template <int D, bool LL, int NT = kThreads>
__device__ __forceinline__ bool attn_unit(const Args &ka, const Geo &g, int kh, int split, float *lds, const Io &io) {
    const AttnStepArgs &a = ka.s;
    constexpr int T = kTileFloats / D;          // keys per tile
    constexpr int C4 = D / 4;                   // float4 per row
    constexpr int LPK = C4 < 16 ? C4 : 16;      // lanes per key in the score pass
    constexpr int VPL = C4 / LPK;               // float4 per lane per key
    constexpr int NWV = NT / kWave;
    constexpr int FPT = kTileFloats / 4 / NT;   // float4 of K (and of V) per thread per tile
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.heads / a.kv_heads, kvw = a.kv_heads * D;
    int t0, t1, split_len;
    split_range<D>(g, a.splits, split, &t0, &t1, &split_len);

    float *Ks = lds;                           // [T][D]
    float *Vs = Ks + T * D;                    // [T][D]
    float *qs = Vs + T * D;                    // [G][D]
    float *kn = qs + G * D;                    // [D]
    float *vn = kn + D;                        // [D]
    float *sc = vn + D;                        // [G][T]
    float *stt = sc + G * T;                   // [G] running max, [G] running sum, [G] rescale

    const float *rk = ka.mode == 1 ? a.ring_k : ka.ring_k_ro;
    const float *rv = ka.mode == 1 ? a.ring_v : ka.ring_v_ro;
    const int newest = ka.mode == 1 ? g.length - 1 : -1;

    // Output ownership in the PV pass: thread -> column j, heads pg, pg+GS, ...
    constexpr int GS = NT / D > 0 ? NT / D : 1;
    const int pj = tid % D, pg = tid / D;
    constexpr int NACC = kMaxG / GS > 0 ? kMaxG / GS : 1;
    float acc[NACC];
    const int nacc = (G + GS - 1) / GS;
#pragma unroll
    for (int i = 0; i < NACC; ++i) acc[i] = 0.0f;

    // Tile loader: float4 index f = tid + 256*i -> (row f / C4, column f % C4).
    float4 pk[FPT], pv[FPT];
    auto fetch = [&](int c0) {
#pragma unroll
        for (int i = 0; i < FPT; ++i) {
            int f = tid + NT * i, r = f / C4, c = f % C4;
            int t = c0 + r;
            if (t < t1 && t != newest) {
                const float *kr, *vr;
                if (t < g.length) {
                    int64_t off = (int64_t)((g.start + t) % a.capacity) * kvw + (int64_t)kh * D;
                    kr = rk + off;
                    vr = rv + off;
                } else {
                    int64_t off = (int64_t)(t - g.length) * kvw + (int64_t)kh * D;
                    kr = a.extra_k + off;
                    vr = a.extra_v + off;
                }
                pk[i] = load_f4(kr + 4 * c);
                pv[i] = load_f4(vr + 4 * c);
            }
        }
    };
    auto stash = [&](int c0) {
#pragma unroll
        for (int i = 0; i < FPT; ++i) {
            int f = tid + NT * i, r = f / C4, c = f % C4;
            int t = c0 + r;
            float4 kk = make_float4(0.f, 0.f, 0.f, 0.f), vv = kk;
            if (t == newest) {
                kk = *(const float4 *)(kn + 4 * c);
                vv = *(const float4 *)(vn + 4 * c);
            } else if (t < t1) {
                kk = pk[i];
                vv = pv[i];
            }
            *(float4 *)(Ks + r * D + 4 * c) = kk;
            *(float4 *)(Vs + r * D + 4 * c) = vv;
        }
    };

    const float inv_norm = sqrtf((float)D);
    // The first tile holds keys of earlier steps only (the newest key comes
    // from the prepared row), so it is in flight while the inputs are awaited.
    if (t0 < t1) fetch(t0);
    if (!prepare<LL, NT>(ka, g, kh, G, D, qs, kn, vn, t0, t1, io)) return false;
    if (tid < G) {
        stt[tid] = -INFINITY;
        stt[kMaxG + tid] = 0.0f;
    }
    for (int c0 = t0; c0 < t1; c0 += T) {
        const int n = min(T, t1 - c0);
        stash(c0);
        lds_barrier();
        if (c0 + T < t1) fetch(c0 + T);   // in flight while this tile is consumed
        {   // scores: LPK lanes per key
            const int sub = lane % LPK, ks = lane / LPK;
            constexpr int KPW = kWave / LPK;
            for (int r0 = wave * KPW; r0 < n; r0 += NWV * KPW) {
                int r = r0 + ks;
                const float *kr = Ks + min(r, T - 1) * D;
                float4 kv[VPL];
#pragma unroll
                for (int v = 0; v < VPL; ++v) kv[v] = *(const float4 *)(kr + 4 * (sub + LPK * v));
                for (int gh = 0; gh < G; ++gh) {
                    float part = 0.0f;
#pragma unroll
                    for (int v = 0; v < VPL; ++v) {
                        float4 q4 = *(const float4 *)(qs + gh * D + 4 * (sub + LPK * v));
                        part = fmaf(q4.x, kv[v].x, part);
                        part = fmaf(q4.y, kv[v].y, part);
                        part = fmaf(q4.z, kv[v].z, part);
                        part = fmaf(q4.w, kv[v].w, part);
                    }
                    part = group_sum(part, LPK);
                    if (sub == 0 && r < n) sc[gh * T + r] = part / inv_norm;
                }
            }
        }
        lds_barrier();
        // Online softmax statistics per head (one wave per head).
        for (int gh = wave; gh < G; gh += NWV) {
            float mx = -INFINITY;
            for (int r = lane; r < n; r += kWave) mx = fmaxf(mx, sc[gh * T + r]);
            mx = wave_max(mx);
            const float m_old = stt[gh];
            const float m_new = fmaxf(m_old, mx);
            const float alpha = m_old == -INFINITY ? 0.0f : expf(m_old - m_new);
            float sum = 0.0f;
            for (int r = lane; r < n; r += kWave) {
                float p = expf(sc[gh * T + r] - m_new);
                sc[gh * T + r] = p;
                sum += p;
            }
            sum = wave_sum(sum);
            if (lane == 0) {
                stt[gh] = m_new;
                stt[kMaxG + gh] = stt[kMaxG + gh] * alpha + sum;
                stt[2 * kMaxG + gh] = alpha;
            }
        }
        lds_barrier();
        // Weighted values.
#pragma unroll
        for (int i = 0; i < NACC; ++i) {
            int gh = pg + GS * i;
            if (i < nacc && gh < G) {
                float v = acc[i] * stt[2 * kMaxG + gh];
                const float *p = sc + gh * T;
#pragma unroll 8
                for (int r = 0; r < n; ++r) v = fmaf(p[r], Vs[r * D + pj], v);
                acc[i] = v;
            }
        }
        lds_barrier();
    }

    // Partial (m, l, o) of this split; in LL mode as cells of this phase's
    // epoch (a merger reads them without any ordering between the stores).
    if constexpr (LL) {
        if (t0 < t1) {
            uint64_t *part = a.part_cells + ((int64_t)(kh * a.splits + split) * G) * (D + 2);
#pragma unroll
            for (int i = 0; i < NACC; ++i) {
                int gh = pg + GS * i;
                if (i < nacc && gh < G) ll::put(part + gh * (D + 2) + 2 + pj, acc[i], io.ep_out);
            }
            if (tid < G) {
                ll::put(part + tid * (D + 2), stt[tid], io.ep_out);
                ll::put(part + tid * (D + 2) + 1, stt[kMaxG + tid], io.ep_out);
            }
        }
        return true;
    }
    float *part = a.part + ((int64_t)(kh * a.splits + split) * G) * (D + 2);
    if (t0 < t1) {
#pragma unroll
        for (int i = 0; i < NACC; ++i) {
            int gh = pg + GS * i;
            if (i < nacc && gh < G) st<LL>(part + gh * (D + 2) + 2 + pj, acc[i]);
        }
        if (tid < G) {
            st<LL>(part + tid * (D + 2), stt[tid]);
            st<LL>(part + tid * (D + 2) + 1, stt[kMaxG + tid]);
        }
    }
    return true;
}

// Split weights of a merge, one wave per head: M = max_s m_s, then
// w_s = e^(m_s - M) (0 for a split without keys) and L = sum_s w_s l_s.
template <int NT>
__device__ __forceinline__ void merge_weights(float *w, const float *lv, float *L, int G, int active) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int gh = wave; gh < G; gh += NT / kWave) {
        float mx = -INFINITY;
        for (int s = lane; s < active; s += kWave) mx = fmaxf(mx, w[s * G + gh]);
        const float M = wave_max(mx);
        float sum = 0.0f;
        for (int s = lane; s < active; s += kWave) {
            const float l = lv[s * G + gh];
            const float e = l == 0.0f ? 0.0f : expf(w[s * G + gh] - M);
            w[s * G + gh] = e;
            sum = fmaf(e, l, sum);
        }
        sum = wave_sum(sum);
        if (lane == 0) L[gh] = sum;
    }
    __syncthreads();
}

// Merge the `active` splits of KV head kh into out[(kh*G + g)*D + j].
// LL = true: partials come from other workgroups of the same launch and the
// output is written as cells of epoch io.ep_out.
// Returns false (block-uniform) when an LL wait gave up.
template <int D, bool LL, int NT = kThreads>
__device__ __forceinline__ bool combine(const AttnStepArgs &a, int kh, int active, float *lds, const Io &io) {
    const int tid = threadIdx.x;
    const int G = a.heads / a.kv_heads;
    const float *base = a.part + (int64_t)kh * a.splits * G * (D + 2);
    float *w = lds;                      // [active][G] split maxima, then weights e^(m_s - M)
    float *lv = w + active * G;          // [active][G] split sums
    float *L = lv + active * G;          // [G]
    float *red = L + G;                  // [SG][G*D] partial sums
    for (int i = tid; i < active * G; i += NT) {
        w[i] = ld<LL>(base + (int64_t)i * (D + 2));
        lv[i] = ld<LL>(base + (int64_t)i * (D + 2) + 1);
    }
    __syncthreads();
    merge_weights<NT>(w, lv, L, G, active);
    // Thread (sg, j4): float4 column j4 of every head over splits sg, sg+SG, ...
    constexpr int C4 = D / 4;
    constexpr int SG = NT / C4;
    const int j4 = tid % C4, sg = tid / C4;
    for (int gh = 0; gh < G; ++gh) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
        for (int s = sg; s < active; s += SG) {
            const int off = (s * G + gh) * (D + 2) + 2 + 4 * j4;
            const float4 o = load_f4(base + off);
            const float e = w[s * G + gh];
            acc.x = fmaf(e, o.x, acc.x);
            acc.y = fmaf(e, o.y, acc.y);
            acc.z = fmaf(e, o.z, acc.z);
            acc.w = fmaf(e, o.w, acc.w);
        }
        *(float4 *)(red + (sg * G + gh) * D + 4 * j4) = acc;
    }
    __syncthreads();
    for (int i = tid; i < G * D; i += NT) {
        int gh = i / D, j = i % D;
        float sum = 0.0f;
        for (int q = 0; q < SG; ++q) sum += red[(q * G + gh) * D + j];
        const int64_t o = (int64_t)(kh * G + gh) * D + j;
        if constexpr (LL) ll::put((uint64_t *)a.out + o, sum / L[gh], io.ep_out);
        else *gmem(a.out + o) = sum / L[gh];
    }
    return true;
}

template <int D, int NT = kThreads>
__host__ __device__ constexpr int combine_lds_floats(int G, int splits) {
    return 2 * splits * G + G + (NT / (D / 4)) * G * D;
}

// The persistent kernel's merge: the partials of the `active` splits of unit
// group v (AttnStepArgs::head_groups) are cells of epoch io.ep_out.  Thread
// (gh, j4, sg) sums float4
// column j4 of head gh over splits sg, sg + SG, ...; each thread issues its
// o cells (up to kChunk float4 per round) together with one (m, l) pair and
// polls until all carry the epoch, so a merge that starts after its splits
// finished costs one round trip.  Writes out[(v*G + g)*D + j] as cells.
// Returns false (block-uniform) when a wait gave up.
template <int D, int NT>
__device__ __forceinline__ bool combine_cells(const AttnStepArgs &a, int v, int active, float *lds, const Io &io,
                                              unsigned long long *seen = nullptr) {
    constexpr int C4 = D / 4;
    constexpr int kChunk = 8;
    const int tid = threadIdx.x;
    const int G = a.heads / (a.kv_heads * a.head_groups);
    const uint64_t *base = a.part_cells + (int64_t)v * a.splits * G * (D + 2);
    const int SG = max(1, NT / (G * C4));               // split groups per (gh, j4)
    const bool owner = tid < G * C4 * SG;
    const int gh = owner ? tid / (C4 * SG) : 0, j4 = tid % C4, sg = owner ? (tid / C4) % SG : 0;
    float *w = lds;                      // [active][G] split maxima, then weights e^(m_s - M)
    float *lv = w + active * G;          // [active][G] split sums
    float *L = lv + active * G;          // [G]
    float *red = L + G;                  // [SG][G*D] partial sums
    ll::Wait wt = ll::waiter(io.err);
    ll::u64x2 c[kChunk][2];
    // Loads of splits past `active` (and of non-owner threads) fall outside
    // the head's partials and read zero without touching memory.
    const int limit = active * G * (D + 2);
    auto arrived = [&](const ll::u64x2 (&p)[2]) {
        return (unsigned)(p[0].x >> 32) == io.ep_out && (unsigned)(p[0].y >> 32) == io.ep_out &&
               (unsigned)(p[1].x >> 32) == io.ep_out && (unsigned)(p[1].y >> 32) == io.ep_out;
    };
    // The first chunk of o and this thread's (m, l) pair, polled until they are
    // all there.  Cells that arrived are kept: each poll re-reads only what is
    // still missing.
    {
        const int i = tid < active * G ? tid : active * G;
        ll::u64x2 ml{0ull, 0ull};
        unsigned pending = tid < active * G ? 1u << kChunk : 0u;   // bit q: chunk q, bit kChunk: (m, l)
#pragma unroll
        for (int q = 0; q < kChunk; ++q) {
            c[q][0] = c[q][1] = ll::u64x2{0ull, 0ull};
            if (owner && sg + q * SG < active) pending |= 1u << q;
        }
        for (;;) {
#pragma unroll
            for (int q = 0; q < kChunk; ++q)
                if (pending & (1u << q)) {
                    const int off = ((sg + q * SG) * G + gh) * (D + 2) + 2 + 4 * j4;
                    c[q][0] = ll::peek2(base, off, limit);
                    c[q][1] = ll::peek2(base, off + 2, limit);
                }
            if (pending & (1u << kChunk)) ml = ll::peek2(base, i * (D + 2), limit);
#pragma unroll
            for (int q = 0; q < kChunk; ++q)
                if (arrived(c[q])) pending &= ~(1u << q);
            if ((unsigned)(ml.x >> 32) == io.ep_out && (unsigned)(ml.y >> 32) == io.ep_out)
                pending &= ~(1u << kChunk);
            if (!pending || !ll::backoff(wt)) break;
        }
        if (seen && tid == 0) *seen = wall_clock64();   // trace: thread 0's first cells in
        if (tid < active * G) {
            w[tid] = __uint_as_float((unsigned)ml.x);
            lv[tid] = __uint_as_float((unsigned)ml.y);
        }
    }
    for (int i = tid + NT; i < active * G; i += NT) {   // more (m, l) pairs than threads
        const float2 v = ll::get2(base, i * (D + 2), io.ep_out, wt);
        w[i] = v.x;
        lv[i] = v.y;
    }
    if (!ll::all_ok(wt)) return false;
    merge_weights<NT>(w, lv, L, G, active);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < active; s0 += kChunk * SG) {
        if (s0 > 0) {   // further chunks (more than kChunk splits per thread)
            unsigned pending = 0;
#pragma unroll
            for (int q = 0; q < kChunk; ++q) {
                c[q][0] = c[q][1] = ll::u64x2{0ull, 0ull};
                if (owner && s0 + sg + q * SG < active) pending |= 1u << q;
            }
            for (;;) {
#pragma unroll
                for (int q = 0; q < kChunk; ++q)
                    if (pending & (1u << q)) {
                        const int off = ((s0 + sg + q * SG) * G + gh) * (D + 2) + 2 + 4 * j4;
                        c[q][0] = ll::peek2(base, off, limit);
                        c[q][1] = ll::peek2(base, off + 2, limit);
                    }
#pragma unroll
                for (int q = 0; q < kChunk; ++q)
                    if (arrived(c[q])) pending &= ~(1u << q);
                if (!pending || !ll::backoff(wt)) break;
            }
        }
#pragma unroll
        for (int q = 0; q < kChunk; ++q) {
            const int s = s0 + sg + q * SG;
            if (owner && s < active) {
                const float e = w[s * G + gh];
                acc.x = fmaf(e, __uint_as_float((unsigned)c[q][0].x), acc.x);
                acc.y = fmaf(e, __uint_as_float((unsigned)c[q][0].y), acc.y);
                acc.z = fmaf(e, __uint_as_float((unsigned)c[q][1].x), acc.z);
                acc.w = fmaf(e, __uint_as_float((unsigned)c[q][1].y), acc.w);
            }
        }
    }
    if (!ll::all_ok(wt)) return false;
    if (owner) *(float4 *)(red + (sg * G + gh) * D + 4 * j4) = acc;
    __syncthreads();
    for (int i = tid; i < G * D; i += NT) {
        const int h = i / D, j = i % D;
        float sum = 0.0f;
        for (int q = 0; q < SG; ++q) sum += red[(q * G + h) * D + j];
        ll::put((uint64_t *)a.out + (int64_t)(v * G + h) * D + j, sum / L[h], io.ep_out);
    }
    return true;
}

// Persistent-kernel unit with no barrier per tile: every wave scores and mixes
// its own keys of the split, keeping a running max, sum and weighted values
// per head; the waves' (m, l, o) are then combined in LDS into the unit's
// partial.  A lane holds 16 dims of a key (kWaveVec float4 of K and of V), so
// D/16 lanes share a key: a dot product is 16 FMAs and at most three in-row
// lane steps.  A round is kWaveKeys keys per lane; the first round's K/V
// loads (keys of earlier steps only) go out before the Q/K/V cells are
// awaited.  The unit scores G = heads / (kv_heads * head_groups) <=
// kWaveUnitMaxG query heads (group hs of KV head kh): with head_groups > 1 the
// groups of one KV head read the same keys, and the cost of a unit (its
// rounds run the heads one after another, then its partial and merge) falls
// with G.
constexpr int kWaveVec = 4;          // float4 per lane per key (16 dims)
constexpr int kWaveKeys = 1;         // keys per lane per round
constexpr int kWaveUnitMaxG = 4;

template <int D>
__host__ __device__ constexpr int keys_per_wave_round() {
    return kWaveKeys * (kWave / (D / (4 * kWaveVec)));
}

template <int D, int NT>
__host__ __device__ constexpr int unit_waves_lds_floats(int G) {
    return G * D + 2 * D + 2 * (NT / kWave) * G + (NT / kWave) * G * D;
}

// Sum over aligned groups of LPK <= 16 lanes (every lane of a group receives it).
template <int LPK>
__device__ __forceinline__ float lanes_sum(float v) {
    if constexpr (LPK >= 2) v += dpp_f<0xB1>(v);    // lane ^ 1
    if constexpr (LPK >= 4) v += dpp_f<0x4E>(v);    // lane ^ 2
    if constexpr (LPK >= 8) v += dpp_f<0x141>(v);   // the other half of the 8 (values uniform per quad)
    if constexpr (LPK >= 16) v += dpp_f<0x140>(v);  // the other half of the row (uniform per 8)
    return v;
}

// Sum / max over the key groups of a wave (lanes l, l ^ LPK, l ^ 2 LPK, ...);
// the value is uniform within each group of LPK lanes.
template <int LPK>
__device__ __forceinline__ float keygroups_sum(float v) {
    if constexpr (LPK < 2) v += dpp_f<0xB1>(v);
    if constexpr (LPK < 4) v += dpp_f<0x4E>(v);
    if constexpr (LPK < 8) v += dpp_f<0x141>(v);
    if constexpr (LPK < 16) v += dpp_f<0x140>(v);
    return xor32_sum(xor16_sum(v));
}
// Sum over lanes l, l ^ LPK, l ^ 2 LPK, ... for values that differ within a
// key group (lane l ^ 8 in a row is row_ror:8; smaller strides go through
// LDS swizzles).
template <int LPK>
__device__ __forceinline__ float keygroups_sum_lanes(float v) {
#pragma unroll
    for (int off = LPK; off < 8; off <<= 1) v += __shfl_xor(v, off, kWave);
    if constexpr (LPK <= 8) v += dpp_f<0x128>(v);
    return xor32_sum(xor16_sum(v));
}
template <int LPK>
__device__ __forceinline__ float keygroups_max(float v) {
    if constexpr (LPK < 2) v = fmaxf(v, dpp_f<0xB1>(v));
    if constexpr (LPK < 4) v = fmaxf(v, dpp_f<0x4E>(v));
    if constexpr (LPK < 8) v = fmaxf(v, dpp_f<0x141>(v));
    if constexpr (LPK < 16) v = fmaxf(v, dpp_f<0x140>(v));
    return xor32_max(xor16_max(v));
}

template <int D, int NT>
__device__ __forceinline__ bool attn_unit_waves(const Args &ka, const Geo &g, int kh, int hs, int split, float *lds,
                                                const Io &io, unsigned long long *staged = nullptr) {
    const AttnStepArgs &a = ka.s;
    constexpr int LPK = D / (4 * kWaveVec);   // lanes per key: 8, 4, 2
    constexpr int KPI = kWave / LPK;          // keys side by side in a wave
    constexpr int NWV = NT / kWave;
    constexpr int RK = kWaveKeys * KPI;       // keys per wave per round
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = lane % LPK, kg = lane / LPK;
    const int G = a.heads / (a.kv_heads * a.head_groups), kvw = a.kv_heads * D;
    int t0, t1, split_len;
    split_range<D>(g, a.splits, split, &t0, &t1, &split_len);
    float *qs = lds;                  // [G][D]
    float *kn = qs + G * D;           // [D] newest key (normalized, rotated)
    float *vn = kn + D;               // [D] newest value
    float *wm = vn + D;               // [NWV][G] per-wave max
    float *wl = wm + NWV * G;         // [NWV][G] per-wave sum
    float *wo = wl + NWV * G;         // [NWV][G][D] per-wave weighted values
    const int newest = g.length - 1;
    // The lane's float4 c holds dims 4 (sub + LPK c) .. + 3: the LPK lanes of a
    // key read one contiguous 16 LPK-byte span of its row per load.
    auto dim = [&](int c) { return 4 * (sub + LPK * c); };

    typedef float4 KeyRegs[kWaveKeys][kWaveVec];
    KeyRegs kr, vr;
    auto key_of = [&](int round, int i) { return t0 + (round * NWV + wave) * RK + i * KPI + kg; };
    auto fetch = [&](int round, KeyRegs &kd, KeyRegs &vd) {
#pragma unroll
        for (int i = 0; i < kWaveKeys; ++i) {
            const int t = key_of(round, i);
            const float *kb = nullptr, *vb = nullptr;
            if (t < t1 && t != newest) {
                if (t < g.length) {
                    const int64_t off = (int64_t)((g.start + t) % a.capacity) * kvw + (int64_t)kh * D;
                    kb = a.ring_k + off;
                    vb = a.ring_v + off;
                } else {
                    const int64_t off = (int64_t)(t - g.length) * kvw + (int64_t)kh * D;
                    kb = a.extra_k + off;
                    vb = a.extra_v + off;
                }
            }
#pragma unroll
            for (int c = 0; c < kWaveVec; ++c) {
                kd[i][c] = kb ? load_f4(kb + dim(c)) : make_float4(0.f, 0.f, 0.f, 0.f);
                vd[i][c] = vb ? load_f4(vb + dim(c)) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    };
    if (t0 >= t1) return true;   // no keys at this position (the newest key is in another split)
    const int per_round = NWV * RK;
    const int rounds = (t1 - t0 + per_round - 1) / per_round;
    fetch(0, kr, vr);
    if (!prepare<true, NT>(ka, g, kh, G, D, qs, kn, vn, t0, t1, io, hs)) return false;
    if (staged && tid == 0) *staged = wall_clock64();   // trace: Q/K/V cells in

    // scores carry the 1/sqrt(D) of kernels.cl:72 through the queries
    const float inv_root = 1.0f / sqrtf((float)D);
    float m_run[kWaveUnitMaxG], l_run[kWaveUnitMaxG];
    float4 acc[kWaveUnitMaxG][kWaveVec];
#pragma unroll
    for (int h = 0; h < kWaveUnitMaxG; ++h) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.0f;
#pragma unroll
        for (int c = 0; c < kWaveVec; ++c) acc[h][c] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int round = 0; round < rounds; ++round) {
        if (round > 0) fetch(round, kr, vr);
#pragma unroll
        for (int i = 0; i < kWaveKeys; ++i)
            if (key_of(round, i) == newest)
#pragma unroll
                for (int c = 0; c < kWaveVec; ++c) {
                    kr[i][c] = *(const float4 *)(kn + dim(c));
                    vr[i][c] = *(const float4 *)(vn + dim(c));
                }
#pragma unroll
        for (int h = 0; h < kWaveUnitMaxG; ++h) {
            if (h >= G) break;
            float4 q[kWaveVec];
#pragma unroll
            for (int c = 0; c < kWaveVec; ++c) {
                const float4 t = *(const float4 *)(qs + h * D + dim(c));
                q[c] = make_float4(t.x * inv_root, t.y * inv_root, t.z * inv_root, t.w * inv_root);
            }
            float sc[kWaveKeys];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < kWaveKeys; ++i) {
                float d = 0.0f;
#pragma unroll
                for (int c = 0; c < kWaveVec; ++c) {
                    d = fmaf(q[c].x, kr[i][c].x, d);
                    d = fmaf(q[c].y, kr[i][c].y, d);
                    d = fmaf(q[c].z, kr[i][c].z, d);
                    d = fmaf(q[c].w, kr[i][c].w, d);
                }
                d = lanes_sum<LPK>(d);
                sc[i] = key_of(round, i) < t1 ? d : -INFINITY;
                mx = fmaxf(mx, sc[i]);
            }
            mx = keygroups_max<LPK>(mx);
            const float m_new = fmaxf(m_run[h], mx);   // -inf while this wave has seen no key
            const float m_ref = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = m_run[h] == -INFINITY ? 0.0f : expf(m_run[h] - m_ref);
            float sum = 0.0f;
#pragma unroll
            for (int c = 0; c < kWaveVec; ++c)
                acc[h][c] = make_float4(acc[h][c].x * alpha, acc[h][c].y * alpha, acc[h][c].z * alpha,
                                        acc[h][c].w * alpha);
#pragma unroll
            for (int i = 0; i < kWaveKeys; ++i) {
                const float p = expf(sc[i] - m_ref);
                sum += p;
#pragma unroll
                for (int c = 0; c < kWaveVec; ++c) {
                    acc[h][c].x = fmaf(p, vr[i][c].x, acc[h][c].x);
                    acc[h][c].y = fmaf(p, vr[i][c].y, acc[h][c].y);
                    acc[h][c].z = fmaf(p, vr[i][c].z, acc[h][c].z);
                    acc[h][c].w = fmaf(p, vr[i][c].w, acc[h][c].w);
                }
            }
            // each key group holds a part of the sum (its own keys)
            sum = keygroups_sum<LPK>(sum);
            m_run[h] = m_new;
            l_run[h] = l_run[h] * alpha + sum;
        }
    }
    // Waves without keys of this unit keep m = -inf, l = 0, o = 0.
#pragma unroll
    for (int h = 0; h < kWaveUnitMaxG; ++h) {
        if (h >= G) break;
#pragma unroll
        for (int c = 0; c < kWaveVec; ++c) {
            float4 o = acc[h][c];
            o.x = keygroups_sum_lanes<LPK>(o.x);
            o.y = keygroups_sum_lanes<LPK>(o.y);
            o.z = keygroups_sum_lanes<LPK>(o.z);
            o.w = keygroups_sum_lanes<LPK>(o.w);
            if (kg == 0) *(float4 *)(wo + (wave * G + h) * D + dim(c)) = o;
        }
        if (lane == 0) {
            wm[wave * G + h] = m_run[h];
            wl[wave * G + h] = l_run[h];
        }
    }
    __syncthreads();
    uint64_t *part = a.part_cells + ((int64_t)((kh * a.head_groups + hs) * a.splits + split) * G) * (D + 2);
    for (int e = tid; e < G * D; e += NT) {
        const int h = e / D, j = e % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NWV; ++w) M = fmaxf(M, wm[w * G + h]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < NWV; ++w) {
            const float m = wm[w * G + h];
            const float f = m == -INFINITY ? 0.0f : expf(m - M);
            L = fmaf(wl[w * G + h], f, L);
            O = fmaf(wo[(w * G + h) * D + j], f, O);
        }
        ll::put(part + h * (D + 2) + 2 + j, O, io.ep_out);
        if (j == 0) {
            ll::put(part + h * (D + 2), M, io.ep_out);
            ll::put(part + h * (D + 2) + 1, L, io.ep_out);
        }
    }
    return true;
}

template <int D, int NT>
__host__ __device__ constexpr int combine_cells_lds_floats(int G, int splits) {
    return 2 * splits * G + G + (NT / (G * (D / 4)) > 0 ? NT / (G * (D / 4)) : 1) * G * D;
}

}  // namespace att
}  // namespace mr
