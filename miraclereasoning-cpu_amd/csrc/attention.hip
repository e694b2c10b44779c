// Split-key attention for one query token.
//
// Grid: (splits, kv_heads).  Workgroup (split, kh) owns the G = heads/kv_heads
// query heads that share KV head kh (kernels.cl:66 mapping) and a contiguous
// range of the logical keys [ring window, extra rows] (kernels.cl:67-68).  It
// scores them (dot / sqrt(dim), kernels.cl:72), keeps a running max m and
// l = sum exp(s - m), accumulates o = sum exp(s - m) v, and writes (m, l, o).
// The last workgroup of each KV head to finish (a device counter) merges the
// splits: out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s -- the softmax-
// weighted value sum of kernels.cl:75-107, up to rounding.
//
// Fast path (head dim 32/64/128): keys and values stream through LDS in 16 KB
// tiles (4096 floats = 4096/dim keys), each thread loading 4 float4 of K and 4
// of V per tile, coalesced along the row; the next tile is prefetched into
// registers while the current one is consumed.  The split length follows the
// current window, so every workgroup of the fixed grid has work.  Other head
// dims take a plain per-element path (micro models only).
#include "attention.h"

namespace mr {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kTileFloats = 4096;
constexpr int kMaxG = 16;

struct KernelArgs {
    AttnStepArgs s;       // engine fields (mode 1)
    int mode;             // 0 = op-level, 1 = engine step
    int start, length, extra_length;   // mode 0 geometry
    const float *ring_k_ro, *ring_v_ro;
};

struct Geo {
    int pos, start, length, extra, total;
};

__device__ __forceinline__ Geo geometry(const KernelArgs &ka) {
    const AttnStepArgs &a = ka.s;
    Geo g;
    if (ka.mode == 1) {
        g.pos = *a.pos;
        int count = g.pos + 1;
        g.length = min(count, a.capacity);
        g.start = (count - g.length) % a.capacity;
        g.extra = a.extra_chunk ? (g.pos / a.extra_chunk) * a.extra_slots : 0;
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
// LDS, then store the new key/value in the ring slot of this position (by the
// split that holds the newest key).  Ends with a barrier.
__device__ void prepare(const KernelArgs &ka, const Geo &g, int kh, int G, int d, float *qs, float *kn, float *vn,
                        int t0, int t1) {
    const AttnStepArgs &a = ka.s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *q_src = a.q + (int64_t)kh * G * d;
    for (int i = tid; i < G * d; i += kThreads) qs[i] = q_src[i];
    if (ka.mode != 1) {
        __syncthreads();
        return;
    }
    for (int j = tid; j < d; j += kThreads) {
        kn[j] = a.k_new[kh * d + j];
        vn[j] = a.v_new[kh * d + j];
    }
    __syncthreads();
    if (a.q_gain) {   // per-head RMSNorm, width = dim (kernels.cl:19-28)
        for (int r = wave; r < G + 1; r += kWaves) {
            float *row = r < G ? qs + r * d : kn;
            const float *gain = r < G ? a.q_gain : a.k_gain;
            float ss = 0.0f;
            for (int j = lane; j < d; j += kWave) ss = fmaf(row[j], row[j], ss);
            ss = wave_sum(ss);
            float scale = 1.0f / sqrtf(ss / (float)d + a.eps);
            for (int j = lane; j < d; j += kWave) row[j] = row[j] * scale * gain[j];
        }
        __syncthreads();
    }
    const int half = d / 2;   // RoPE at this position (kernels.cl:30-44)
    const float fpos = (float)g.pos;
    for (int i = tid; i < (G + 1) * half; i += kThreads) {
        int r = i / half, p = i % half;
        float *row = r < G ? qs + r * d : kn;
        int j = a.split_half ? p : 2 * p, k = a.split_half ? p + half : 2 * p + 1;
        float u = row[j], v = row[k];
        rope_pair(u, v, fpos, a.freq[p]);
        row[j] = u;
        row[k] = v;
    }
    __syncthreads();
    const int newest = g.length - 1;
    if (t0 <= newest && newest < t1) {
        const int kvw = a.kv_heads * d;
        int64_t slot = (int64_t)(g.pos % a.capacity) * kvw + (int64_t)kh * d;
        for (int j = tid; j < d; j += kThreads) {
            a.ring_k[slot + j] = kn[j];
            a.ring_v[slot + j] = vn[j];
        }
    }
}

// Merge the splits of KV head kh (run by the last workgroup to finish).
template <int D>
__device__ void combine(const AttnStepArgs &a, int kh, int G, int active, float *lds) {
    const int tid = threadIdx.x;
    const float *base = a.part + (int64_t)kh * a.splits * G * (D + 2);
    float *w = lds;                      // [active][G] split maxima, then weights e^(m_s - M)
    float *lv = w + active * G;          // [active][G] split sums
    float *L = lv + active * G;          // [G]
    float *red = L + G;                  // [SG][G*D] partial sums
    for (int i = tid; i < active * G; i += kThreads) {
        w[i] = base[(int64_t)i * (D + 2)];
        lv[i] = base[(int64_t)i * (D + 2) + 1];
    }
    __syncthreads();
    if (tid < G) {
        float M = -INFINITY;
        for (int s = 0; s < active; ++s) M = fmaxf(M, w[s * G + tid]);
        float sum = 0.0f;
        for (int s = 0; s < active; ++s) {
            float l = lv[s * G + tid];
            float e = l == 0.0f ? 0.0f : expf(w[s * G + tid] - M);
            w[s * G + tid] = e;
            sum = fmaf(e, l, sum);
        }
        L[tid] = sum;
    }
    __syncthreads();
    // Thread (sg, j4): float4 column j4 of every head, splits sg, sg+8, ...
    constexpr int C4 = D / 4;
    constexpr int SG = kThreads / C4;
    const int j4 = tid % C4, sg = tid / C4;
    for (int gh = 0; gh < G; ++gh) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
        for (int s = sg; s < active; s += SG) {
            const float4 o = *(const float4 *)(base + (int64_t)(s * G + gh) * (D + 2) + 2 + 4 * j4);
            const float e = w[s * G + gh];
            acc.x = fmaf(e, o.x, acc.x);
            acc.y = fmaf(e, o.y, acc.y);
            acc.z = fmaf(e, o.z, acc.z);
            acc.w = fmaf(e, o.w, acc.w);
        }
        *(float4 *)(red + (sg * G + gh) * D + 4 * j4) = acc;
    }
    __syncthreads();
    for (int i = tid; i < G * D; i += kThreads) {
        int gh = i / D, j = i % D;
        float sum = 0.0f;
        for (int q = 0; q < SG; ++q) sum += red[(q * G + gh) * D + j];
        a.out[(int64_t)(kh * G + gh) * D + j] = sum / L[gh];
    }
}

template <int D>
__global__ void __launch_bounds__(kThreads) k_attn_tiled(KernelArgs ka) {
    extern __shared__ float lds[];
    const AttnStepArgs &a = ka.s;
    if (ka.mode == 1 && a.done && *a.done) return;
    constexpr int T = kTileFloats / D;          // keys per tile
    constexpr int C4 = D / 4;                   // float4 per row
    constexpr int LPK = C4 < 16 ? C4 : 16;      // lanes per key in the score pass
    constexpr int VPL = C4 / LPK;               // float4 per lane per key
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kh = blockIdx.y, split = blockIdx.x;
    const int G = a.heads / a.kv_heads, kvw = a.kv_heads * D;

    const Geo g = geometry(ka);
    int split_len = (g.total + a.splits - 1) / a.splits;
    split_len = (split_len + T - 1) / T * T;
    const int t0 = min(split * split_len, g.total);
    const int t1 = min(t0 + split_len, g.total);

    float *Ks = lds;                           // [T][D]
    float *Vs = Ks + T * D;                    // [T][D]
    float *qs = Vs + T * D;                    // [G][D]
    float *kn = qs + G * D;                    // [D]
    float *vn = kn + D;                        // [D]
    float *sc = vn + D;                        // [G][T]
    float *st = sc + G * T;                    // [G] running max, [G] running sum, [G] rescale
    int *flag = (int *)(st + 3 * kMaxG);

    prepare(ka, g, kh, G, D, qs, kn, vn, t0, t1);
    if (tid < G) {
        st[tid] = -INFINITY;
        st[kMaxG + tid] = 0.0f;
    }

    const float *rk = ka.mode == 1 ? a.ring_k : ka.ring_k_ro;
    const float *rv = ka.mode == 1 ? a.ring_v : ka.ring_v_ro;
    const int newest = ka.mode == 1 ? g.length - 1 : -1;

    // Output ownership in the PV pass: thread -> column j, heads gs, gs+GS, ...
    constexpr int GS = kThreads / D > 0 ? kThreads / D : 1;
    const int pj = tid % D, pg = tid / D;
    float acc[kMaxG / GS > 0 ? kMaxG / GS : 1];
    const int nacc = (G + GS - 1) / GS;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(acc) / sizeof(float)); ++i) acc[i] = 0.0f;

    // Tile loader: float4 index f = tid + 256*i -> (row f / C4, column f % C4).
    float4 pk[4], pv[4];
    auto fetch = [&](int c0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int f = tid + kThreads * i, r = f / C4, c = f % C4;
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
                pk[i] = *(const float4 *)(kr + 4 * c);
                pv[i] = *(const float4 *)(vr + 4 * c);
            }
        }
    };
    auto stash = [&](int c0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int f = tid + kThreads * i, r = f / C4, c = f % C4;
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
    if (t0 < t1) fetch(t0);
    for (int c0 = t0; c0 < t1; c0 += T) {
        const int n = min(T, t1 - c0);
        stash(c0);
        __syncthreads();
        if (c0 + T < t1) fetch(c0 + T);   // in flight while this tile is consumed
        // Scores: LPK lanes per key.
        {
            const int sub = lane % LPK, ks = lane / LPK;
            constexpr int KPW = kWave / LPK;
            for (int r0 = wave * KPW; r0 < n; r0 += kWaves * KPW) {
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
        __syncthreads();
        // Online softmax statistics per head (one wave per head).
        for (int gh = wave; gh < G; gh += kWaves) {
            float mx = -INFINITY;
            for (int r = lane; r < n; r += kWave) mx = fmaxf(mx, sc[gh * T + r]);
            mx = wave_max(mx);
            const float m_old = st[gh];
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
                st[gh] = m_new;
                st[kMaxG + gh] = st[kMaxG + gh] * alpha + sum;
                st[2 * kMaxG + gh] = alpha;
            }
        }
        __syncthreads();
        // Weighted values.
        for (int i = 0; i < nacc; ++i) {
            int gh = pg + GS * i;
            if (gh < G) {
                float v = acc[i] * st[2 * kMaxG + gh];
                const float *p = sc + gh * T;
                for (int r = 0; r < n; ++r) v = fmaf(p[r], Vs[r * D + pj], v);
                acc[i] = v;
            }
        }
        __syncthreads();
    }

    // Partial (m, l, o) of this split.
    float *part = a.part + ((int64_t)(kh * a.splits + split) * G) * (D + 2);
    if (t0 < t1) {
        for (int i = 0; i < nacc; ++i) {
            int gh = pg + GS * i;
            if (gh < G) part[gh * (D + 2) + 2 + pj] = acc[i];
        }
        if (tid < G) {
            part[tid * (D + 2)] = st[tid];
            part[tid * (D + 2) + 1] = st[kMaxG + tid];
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) *flag = atomicAdd(&a.counters[kh], 1u) == (unsigned)(a.splits - 1);
    __syncthreads();
    const bool last = *flag;
    __syncthreads();   // the combine reuses this LDS
    if (!last) return;
    __threadfence();
    const int active = (g.total + split_len - 1) / split_len;
    combine<D>(a, kh, G, active, lds);
    if (tid == 0) a.counters[kh] = 0u;
}

// ---------------------------------------------------------------- generic path
// Any head dim (micro models, op-level tests with dim 6): per-element loops.
__global__ void __launch_bounds__(kThreads) k_attn_generic(KernelArgs ka) {
    extern __shared__ float lds[];
    const AttnStepArgs &a = ka.s;
    if (ka.mode == 1 && a.done && *a.done) return;
    const int tid = threadIdx.x;
    const int kh = blockIdx.y, split = blockIdx.x;
    const int d = a.dim, G = a.heads / a.kv_heads, kvw = a.kv_heads * d;
    const Geo g = geometry(ka);
    int split_len = (g.total + a.splits - 1) / a.splits;
    const int t0 = min(split * split_len, g.total);
    const int t1 = min(t0 + split_len, g.total);
    const int cap_len = a.split_len;   // LDS score rows sized for the plan's maximum
    float *qs = lds, *kn = qs + G * d, *vn = kn + d, *sc = vn + d;
    int *flag = (int *)(sc + G * cap_len);
    prepare(ka, g, kh, G, d, qs, kn, vn, t0, t1);
    const float *rk = ka.mode == 1 ? a.ring_k : ka.ring_k_ro;
    const float *rv = ka.mode == 1 ? a.ring_v : ka.ring_v_ro;
    const int newest = ka.mode == 1 ? g.length - 1 : -1;
    auto row = [&](const float *ring, const float *extra, const float *fresh, int t) -> const float * {
        if (t == newest) return fresh;
        if (t < g.length) return ring + (int64_t)((g.start + t) % a.capacity) * kvw + (int64_t)kh * d;
        return extra + (int64_t)(t - g.length) * kvw + (int64_t)kh * d;
    };
    const int n = t1 - t0;
    for (int i = tid; i < G * n; i += kThreads) {
        int gh = i / n, r = i % n;
        const float *kr = row(rk, a.extra_k, kn, t0 + r);
        float v = 0.0f;
        for (int j = 0; j < d; ++j) v = fmaf(qs[gh * d + j], kr[j], v);
        sc[gh * cap_len + r] = v / sqrtf((float)d);
    }
    __syncthreads();
    float *part = a.part + ((int64_t)(kh * a.splits + split) * G) * (d + 2);
    if (tid < G && n > 0) {
        float m = -INFINITY;
        for (int r = 0; r < n; ++r) m = fmaxf(m, sc[tid * cap_len + r]);
        float l = 0.0f;
        for (int r = 0; r < n; ++r) {
            float p = expf(sc[tid * cap_len + r] - m);
            sc[tid * cap_len + r] = p;
            l += p;
        }
        part[tid * (d + 2)] = m;
        part[tid * (d + 2) + 1] = l;
    }
    __syncthreads();
    if (n > 0)
        for (int i = tid; i < G * d; i += kThreads) {
            int gh = i / d, j = i % d;
            float acc = 0.0f;
            for (int r = 0; r < n; ++r) acc = fmaf(sc[gh * cap_len + r], row(rv, a.extra_v, vn, t0 + r)[j], acc);
            part[gh * (d + 2) + 2 + j] = acc;
        }
    __threadfence();
    __syncthreads();
    if (tid == 0) *flag = atomicAdd(&a.counters[kh], 1u) == (unsigned)(a.splits - 1);
    __syncthreads();
    if (!*flag) return;
    __threadfence();
    const int active = split_len ? (g.total + split_len - 1) / split_len : 0;
    const float *base = a.part + (int64_t)kh * a.splits * G * (d + 2);
    for (int i = tid; i < G * d; i += kThreads) {
        int gh = i / d, j = i % d;
        float M = -INFINITY;
        for (int s = 0; s < active; ++s) M = fmaxf(M, base[(s * G + gh) * (d + 2)]);
        float L = 0.0f, O = 0.0f;
        for (int s = 0; s < active; ++s) {
            const float *ps = base + (s * G + gh) * (d + 2);
            float w = expf(ps[0] - M);
            L = fmaf(w, ps[1], L);
            O = fmaf(w, ps[2 + j], O);
        }
        a.out[(int64_t)(kh * G + gh) * d + j] = O / L;
    }
    if (tid == 0) a.counters[kh] = 0u;
}

bool tiled_dim(int d) { return d == 32 || d == 64 || d == 128; }

size_t lds_tiled(int G, int d, int splits) {
    const int T = kTileFloats / d;
    size_t main = (size_t)(2 * T * d + G * d + 2 * d + G * T + 3 * kMaxG + 4);
    size_t comb = (size_t)(2 * splits * G + G + (kThreads / (d / 4)) * G * d);
    return std::max(main, comb) * sizeof(float);
}

size_t lds_generic(int G, int d, int split_len) { return (size_t)(G * d + 2 * d + G * split_len + 4) * sizeof(float); }

int launch(hipStream_t s, const KernelArgs &ka) {
    const AttnStepArgs &a = ka.s;
    const int G = a.heads / a.kv_heads;
    dim3 grid(a.splits, a.kv_heads);
    if (tiled_dim(a.dim) && G <= kMaxG) {
        size_t lds = lds_tiled(G, a.dim, a.splits);
        if (lds > 64 * 1024) return fail(MR_ERR_INVALID, "attention: workgroup LDS need above 64 KiB");
        switch (a.dim) {
            case 32: k_attn_tiled<32><<<grid, kThreads, lds, s>>>(ka); break;
            case 64: k_attn_tiled<64><<<grid, kThreads, lds, s>>>(ka); break;
            default: k_attn_tiled<128><<<grid, kThreads, lds, s>>>(ka); break;
        }
    } else {
        size_t lds = lds_generic(G, a.dim, a.split_len);
        if (lds > 64 * 1024) return fail(MR_ERR_INVALID, "attention: workgroup LDS need above 64 KiB");
        k_attn_generic<<<grid, kThreads, lds, s>>>(ka);
    }
    MR_LAUNCHED("enqueue attention");
    return MR_OK;
}

}  // namespace

void attention_plan(int max_total, int kv_heads, int dim, int *splits, int *split_len) {
    // One tile of keys per split at the full window, at most ~512 workgroups.
    const int T = tiled_dim(dim) ? kTileFloats / dim : 64;
    int want = std::max(1, 512 / std::max(kv_heads, 1));
    int n = std::max(1, std::min(want, ceil_div(max_total, T)));
    *splits = n;
    *split_len = ceil_div(max_total, n);   // upper bound of the per-split key count
}

size_t attention_part_floats(int heads, int kv_heads, int dim, int splits) {
    return (size_t)kv_heads * splits * (heads / kv_heads) * (dim + 2);
}

int launch_attention_step(hipStream_t s, const AttnStepArgs &a) {
    KernelArgs ka;
    ka.s = a;
    ka.mode = 1;
    ka.start = ka.length = ka.extra_length = 0;
    ka.ring_k_ro = a.ring_k;
    ka.ring_v_ro = a.ring_v;
    return launch(s, ka);
}

int launch_attention_op(mr_ctx *ctx, const AttnProblem &p) {
    int total = p.length + p.extra_length;
    KernelArgs ka;
    AttnStepArgs &a = ka.s;
    a.q = p.q;
    a.extra_k = p.extra_k;
    a.extra_v = p.extra_v;
    a.heads = p.heads;
    a.kv_heads = p.kv_heads;
    a.dim = p.dim;
    a.capacity = p.capacity;
    a.out = p.out;
    attention_plan(total, p.kv_heads, p.dim, &a.splits, &a.split_len);
    ka.mode = 0;
    ka.start = p.start;
    ka.length = p.length;
    ka.extra_length = p.extra_length;
    ka.ring_k_ro = p.ring_k;
    ka.ring_v_ro = p.ring_v;
    void *ws = nullptr;
    size_t part = attention_part_floats(p.heads, p.kv_heads, p.dim, a.splits) * sizeof(float);
    size_t cnt = (size_t)p.kv_heads * sizeof(unsigned);
    MR_TRY(ctx_alloc(ctx, part + cnt + 256, &ws));
    a.part = (float *)ws;
    a.counters = (unsigned *)((char *)ws + (part + 255) / 256 * 256);
    MR_HIP(hipMemsetAsync(a.counters, 0, cnt, ctx->stream), "attention: clear counters");
    int rc = launch(ctx->stream, ka);
    ctx_release(ctx, ws);   // stream-ordered: later work on this stream reuses it safely
    return rc;
}

}  // namespace mr
