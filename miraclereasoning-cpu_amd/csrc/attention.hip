// Split-key attention for one query token.
//
// Grid: (splits, kv_heads).  Workgroup (split, kh) owns the G = heads/kv_heads
// query heads that share KV head kh (kernels.cl:66 mapping) and the logical keys
// [split*split_len, (split+1)*split_len) of the order [ring window, extra rows]
// (kernels.cl:67-68).  It scores those keys (dot / sqrt(dim), kernels.cl:72),
// takes a local max m and l = sum exp(s - m), accumulates o = sum exp(s - m) v,
// and writes (m, l, o).  The last workgroup of each KV head to finish (a device
// counter) merges the splits: out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s,
// the same softmax-weighted value sum as kernels.cl:75-107 up to rounding.
//
// Key rows are read once from HBM by a group of lanes per key (16-byte loads
// when dim % 4 == 0); value rows are read once, coalesced across the dim.
#include "attention.h"

namespace mr {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

struct Geo {
    int start, length, extra, total, pos;
};

struct KernelArgs {
    AttnStepArgs s;       // engine fields (mode 1)
    int mode;             // 0 = op-level, 1 = engine step
    int start, length, extra_length;   // mode 0 geometry
    const float *ring_k_ro, *ring_v_ro;
};

template <int VEC>
__device__ __forceinline__ float dot_part(const float *q, const float *k, int sub, int lpk, int nv) {
    float acc = 0.0f;
    if constexpr (VEC == 4) {
        for (int v = sub; v < nv; v += lpk) {
            float4 a = *(const float4 *)(q + 4 * v);
            float4 b = *(const float4 *)(k + 4 * v);
            acc = fmaf(a.x, b.x, acc);
            acc = fmaf(a.y, b.y, acc);
            acc = fmaf(a.z, b.z, acc);
            acc = fmaf(a.w, b.w, acc);
        }
    } else {
        for (int v = sub; v < nv; v += lpk) acc = fmaf(q[v], k[v], acc);
    }
    return acc;
}

template <int VEC>
__global__ void __launch_bounds__(kThreads) k_attn_split(KernelArgs ka) {
    extern __shared__ float lds[];
    const AttnStepArgs &a = ka.s;
    if (ka.mode == 1 && a.done && *a.done) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kh = blockIdx.y, split = blockIdx.x;
    const int d = a.dim, G = a.heads / a.kv_heads, kvw = a.kv_heads * d;
    const int split_len = a.split_len;

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
    const int t0 = split * split_len;
    const int t1 = min(t0 + split_len, g.total);

    float *qs = lds;                       // [G*d]
    float *kn = qs + G * d;                // [d]
    float *vn = kn + d;                    // [d]
    float *sc = vn + d;                    // [G*split_len]
    float *stat = sc + G * split_len;      // [2*G]
    float *red = stat + 2 * G;             // [kWaves]
    int *flag = (int *)(red + kWaves);

    const float *q_src = a.q + (int64_t)kh * G * d;
    for (int i = tid; i < G * d; i += kThreads) qs[i] = q_src[i];
    if (ka.mode == 1) {
        for (int j = tid; j < d; j += kThreads) {
            kn[j] = a.k_new[kh * d + j];
            vn[j] = a.v_new[kh * d + j];
        }
        __syncthreads();
        // Per-head RMSNorm of the G queries and the key (kernels.cl:19-28, width = dim).
        if (a.q_gain) {
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
        // RoPE at this position (kernels.cl:30-44).
        const int half = d / 2;
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
        // The split holding the newest key stores it in the ring slot of this position.
        const int newest = g.length - 1;
        if (t0 <= newest && newest < t1) {
            int64_t slot = (int64_t)(g.pos % a.capacity) * kvw + (int64_t)kh * d;
            for (int j = tid; j < d; j += kThreads) {
                a.ring_k[slot + j] = kn[j];
                a.ring_v[slot + j] = vn[j];
            }
        }
    }
    __syncthreads();

    const float *rk = ka.mode == 1 ? a.ring_k : ka.ring_k_ro;
    const float *rv = ka.mode == 1 ? a.ring_v : ka.ring_v_ro;
    const int newest_from_lds = ka.mode == 1 ? g.length - 1 : -1;
    auto key_row = [&](int t) -> const float * {
        if (t == newest_from_lds) return kn;
        if (t < g.length) return rk + (int64_t)((g.start + t) % a.capacity) * kvw + (int64_t)kh * d;
        return a.extra_k + (int64_t)(t - g.length) * kvw + (int64_t)kh * d;
    };
    auto value_row = [&](int t) -> const float * {
        if (t == newest_from_lds) return vn;
        if (t < g.length) return rv + (int64_t)((g.start + t) % a.capacity) * kvw + (int64_t)kh * d;
        return a.extra_v + (int64_t)(t - g.length) * kvw + (int64_t)kh * d;
    };

    // Scores: lpk lanes per key.
    const int nv = d / VEC;
    int lpk = 1;
    while (lpk * 2 <= nv && lpk < 16) lpk *= 2;
    const int sub = lane & (lpk - 1), kslot = lane / lpk, kper_wave = kWave / lpk;
    const float inv_norm = sqrtf((float)d);
    for (int base = t0 + wave * kper_wave; base < t1; base += kWaves * kper_wave) {
        int t = base + kslot;
        bool ok = t < t1;
        const float *kr = key_row(ok ? t : t0);
        for (int gh = 0; gh < G; ++gh) {
            float part = dot_part<VEC>(qs + gh * d, kr, sub, lpk, nv);
            part = group_sum(part, lpk);
            if (ok && sub == 0) sc[gh * split_len + (t - t0)] = part / inv_norm;
        }
    }
    __syncthreads();

    // Local softmax statistics per head.
    const int n = max(t1 - t0, 0);
    for (int gh = wave; gh < G; gh += kWaves) {
        float m = -INFINITY;
        for (int i = lane; i < n; i += kWave) m = fmaxf(m, sc[gh * split_len + i]);
        m = wave_max(m);
        float l = 0.0f;
        for (int i = lane; i < n; i += kWave) {
            float p = expf(sc[gh * split_len + i] - m);
            sc[gh * split_len + i] = p;
            l += p;
        }
        l = wave_sum(l);
        if (lane == 0) {
            stat[2 * gh] = m;
            stat[2 * gh + 1] = l;
        }
    }
    __syncthreads();

    // Weighted values.
    float *part = a.part + ((int64_t)(kh * a.splits + split) * G) * (d + 2);
    for (int idx = tid; idx < G * d; idx += kThreads) {
        int gh = idx / d, j = idx % d;
        float acc = 0.0f;
        const float *p = sc + gh * split_len;
        for (int i = 0; i < n; ++i) acc = fmaf(p[i], value_row(t0 + i)[j], acc);
        part[gh * (d + 2) + 2 + j] = acc;
    }
    if (tid < G) {
        part[tid * (d + 2)] = n ? stat[2 * tid] : -INFINITY;
        part[tid * (d + 2) + 1] = n ? stat[2 * tid + 1] : 0.0f;
    }

    // Last workgroup of this KV head merges all splits.
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        unsigned prev = atomicAdd(&a.counters[kh], 1u);
        *flag = prev == (unsigned)(a.splits - 1);
    }
    __syncthreads();
    if (!*flag) return;
    __threadfence();
    const float *base = a.part + (int64_t)kh * a.splits * G * (d + 2);
    for (int idx = tid; idx < G * d; idx += kThreads) {
        int gh = idx / d, j = idx % d;
        float M = -INFINITY;
        for (int s = 0; s < a.splits; ++s) M = fmaxf(M, base[(s * G + gh) * (d + 2)]);
        float L = 0.0f, O = 0.0f;
        for (int s = 0; s < a.splits; ++s) {
            const float *ps = base + (s * G + gh) * (d + 2);
            float l = ps[1];
            if (l == 0.0f) continue;
            float w = expf(ps[0] - M);
            L = fmaf(w, l, L);
            O = fmaf(w, ps[2 + j], O);
        }
        a.out[(int64_t)(kh * G + gh) * d + j] = O / L;
    }
    if (tid == 0) a.counters[kh] = 0u;
}

size_t lds_bytes(int G, int d, int split_len) {
    return (size_t)(G * d + 2 * d + G * split_len + 2 * G + kWaves + 4) * sizeof(float);
}

int launch(hipStream_t s, const KernelArgs &ka) {
    const AttnStepArgs &a = ka.s;
    int G = a.heads / a.kv_heads;
    dim3 grid(a.splits, a.kv_heads);
    size_t lds = lds_bytes(G, a.dim, a.split_len);
    if (lds > 160 * 1024) return fail(MR_ERR_INVALID, "attention: workgroup LDS need above 160 KiB");
    if (a.dim % 4 == 0)
        k_attn_split<4><<<grid, kThreads, lds, s>>>(ka);
    else
        k_attn_split<1><<<grid, kThreads, lds, s>>>(ka);
    MR_LAUNCHED("enqueue attention");
    return MR_OK;
}

}  // namespace

void attention_plan(int max_total, int kv_heads, int *splits, int *split_len) {
    // Aim for ~512 workgroups over the KV heads, at least 16 keys per split.
    int want = std::max(1, 512 / std::max(kv_heads, 1));
    int len = std::max(16, ceil_div(max_total, want));
    len = (len + 15) / 16 * 16;
    *split_len = len;
    *splits = std::max(1, ceil_div(max_total, len));
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
    attention_plan(total, p.kv_heads, &a.splits, &a.split_len);
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
