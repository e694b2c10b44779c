// Split-key attention for one query token: the standalone kernels.
//
// Grid: (splits, kv_heads).  Each workgroup runs one (split, kh) unit
// (attention_tile.h); the last workgroup of each KV head to finish (a device
// counter) merges that head's splits.  Head dims 32/64/128 take the tiled
// unit; other head dims (micro models, op-level calls with dim 6) take a plain
// per-element path.
#include <mutex>
#include <string>
#include <vector>

#include "attention_tile.h"

// Scratch of the allocation-free entry point (mr_attention_noalloc): the split
// partials and the per-KV-head merge counters of one call.  Each GPU holds its
// own copy for the life of the process.  Host code never passes `scratch`
// itself to a kernel (on the host the name is only a stand-in): it uses the
// device address looked up once per device by mr::static_scratch_address().
static constexpr size_t kStaticScratchBytes = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace mr {
namespace {

using namespace att;
using KernelArgs = att::Args;

template <int D>
__global__ void __launch_bounds__(kThreads) k_attn_tiled(KernelArgs ka) {
    extern __shared__ float lds[];
    const AttnStepArgs &a = ka.s;
    if (ka.mode == 1 && a.done && *a.done) return;
    const int tid = threadIdx.x;
    const int kh = blockIdx.y, split = blockIdx.x;
    const Geo g = geometry(ka, ka.mode == 1 ? *a.pos : 0);
    attn_unit<D, false>(ka, g, kh, split, lds, Io{0u, 0u, nullptr, nullptr, 0});
    int *flag = (int *)(lds + unit_lds_floats<D>(a.heads / a.kv_heads) - 4);
    __threadfence();
    __syncthreads();
    if (tid == 0) *flag = atomicAdd(&a.counters[kh], 1u) == (unsigned)(a.splits - 1);
    __syncthreads();
    const bool last = *flag;
    __syncthreads();   // the merge reuses this LDS
    if (!last) return;
    __threadfence();
    int t0, t1, split_len;
    split_range<D>(g, a.splits, 0, &t0, &t1, &split_len);
    const int active = (g.total + split_len - 1) / split_len;
    combine<D, false>(a, kh, active, lds, Io{0u, 0u, nullptr, nullptr, 0});
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
    const Geo g = geometry(ka, ka.mode == 1 ? *a.pos : 0);
    int split_len = (g.total + a.splits - 1) / a.splits;
    const int t0 = min(split * split_len, g.total);
    const int t1 = min(t0 + split_len, g.total);
    const int cap_len = a.split_len;   // LDS score rows sized for the plan's maximum
    float *qs = lds, *kn = qs + G * d, *vn = kn + d, *sc = vn + d;
    int *flag = (int *)(sc + G * cap_len);
    prepare<false, kThreads>(ka, g, kh, G, d, qs, kn, vn, t0, t1, Io{0u, 0u, nullptr, nullptr, 0});
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
    int main = 0, comb = 0;
    switch (d) {
        case 32: main = unit_lds_floats<32>(G); comb = combine_lds_floats<32>(G, splits); break;
        case 64: main = unit_lds_floats<64>(G); comb = combine_lds_floats<64>(G, splits); break;
        default: main = unit_lds_floats<128>(G); comb = combine_lds_floats<128>(G, splits); break;
    }
    return (size_t)std::max(main, comb) * sizeof(float);
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

void attention_plan(int max_total, int kv_heads, int dim, int max_units, int *splits, int *split_len) {
    // One tile of keys per split at the full window, at most max_units units.
    const int T = tiled_dim(dim) ? kTileFloats / dim : 64;
    int want = std::max(1, max_units / std::max(kv_heads, 1));
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

namespace {

std::mutex g_scratch_mutex;
std::vector<void *> g_scratch_address;   // per device ordinal

__global__ void k_zero_words(unsigned *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

}  // namespace

size_t static_scratch_bytes() { return kStaticScratchBytes; }

// Called by mr_ctx_create with `device` current.
int static_scratch_address(int device, void **out) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if ((int)g_scratch_address.size() <= device) g_scratch_address.resize(device + 1, nullptr);
    if (!g_scratch_address[device]) {
        void *p = nullptr;
        MR_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch)), "look up the static attention scratch");
        g_scratch_address[device] = p;
    }
    *out = g_scratch_address[device];
    return MR_OK;
}

// The same plan and kernels as launch_attention_op, with the partials and
// counters in the device's static scratch: no allocation of any kind.  The
// counters are cleared by a kernel (not a memset), so the call can be
// captured in a graph.
int launch_attention_op_noalloc(mr_ctx *ctx, const AttnProblem &p) {
    MR_REQUIRE(ctx->scratch, "attention_noalloc: the context has no static scratch");
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
    attention_plan(p.length + p.extra_length, p.kv_heads, p.dim, 512, &a.splits, &a.split_len);
    ka.mode = 0;
    ka.start = p.start;
    ka.length = p.length;
    ka.extra_length = p.extra_length;
    ka.ring_k_ro = p.ring_k;
    ka.ring_v_ro = p.ring_v;
    const size_t part = (attention_part_floats(p.heads, p.kv_heads, p.dim, a.splits) * sizeof(float) + 255) /
                        256 * 256;
    const size_t need = part + (size_t)p.kv_heads * sizeof(unsigned);
    if (need > kStaticScratchBytes)
        return fail(MR_ERR_INVALID, "attention_noalloc: needs " + std::to_string(need) +
                                        " bytes of scratch, above its static " +
                                        std::to_string(kStaticScratchBytes) + " (use mr_attention)");
    a.part = (float *)ctx->scratch;
    a.counters = (unsigned *)((char *)ctx->scratch + part);
    k_zero_words<<<ceil_div(p.kv_heads, 256), 256, 0, ctx->stream>>>(a.counters, p.kv_heads);
    MR_LAUNCHED("attention_noalloc: clear counters");
    return launch(ctx->stream, ka);
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
    attention_plan(total, p.kv_heads, p.dim, 512, &a.splits, &a.split_len);
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
