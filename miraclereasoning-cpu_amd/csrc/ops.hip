// Op-level ABI: one entry point per reference kernel (kernels.cl), with the
// reference's argument lists.  These serve HIPBackend's op surface (the drop-in
// for OpenCLBackend); the fused decode step lives in engine.hip.
#include <algorithm>

#include "attention.h"
#include "gemm.h"
#include "linear.h"
#include "prefill.h"

namespace mr {
namespace {

constexpr int kThreads = 256;

inline int grid_for(int64_t n) { return (int)ceil_div64(n, kThreads); }

// kernels.cl:19-28: one block per row.
__global__ void __launch_bounds__(256) k_rms(const float *x, const float *w, float *y, int width, float eps) {
    __shared__ float red[kThreads / kWave];
    const float *xr = x + (int64_t)blockIdx.x * width;
    float ss = 0.0f;
    for (int j = threadIdx.x; j < width; j += blockDim.x) ss = fmaf(xr[j], xr[j], ss);
    ss = block_sum(ss, red);
    float scale = 1.0f / sqrtf(ss / (float)width + eps);
    for (int j = threadIdx.x; j < width; j += blockDim.x)
        y[(int64_t)blockIdx.x * width + j] = xr[j] * scale * (w ? w[j] : 1.0f);
}

// kernels.cl:30-44: one thread per rotated pair.
__global__ void k_rope(const float *x, const float *freq, const float *pos, float *y, int rows, int heads, int dim,
                       int split_half) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int half = dim / 2;
    if (i >= (int64_t)rows * heads * half) return;
    int p = (int)(i % half);
    int64_t head_row = i / half, base = head_row * dim;
    int j = split_half ? p : 2 * p;
    int k = split_half ? p + half : 2 * p + 1;
    float u = x[base + j], v = x[base + k];
    rope_pair(u, v, pos[head_row / heads], freq[p]);
    y[base + j] = u;
    y[base + k] = v;
}

__global__ void k_swiglu(const float *g, const float *u, float *y, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

__global__ void k_axpy(const float *x, const float *y, float *z, int n, float scale) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) z[i] = x[i] + scale * y[i];
}

__device__ __forceinline__ const float *row_of(const float *ring, const float *extra, int t, int kvw, int capacity,
                                               int start, int length, int kh, int dim) {
    if (t < length) return ring + (int64_t)((start + t) % capacity) * kvw + (int64_t)kh * dim;
    return extra + (int64_t)(t - length) * kvw + (int64_t)kh * dim;
}

// kernels.cl:58-73: one thread per (key, head).
__global__ void k_scores(const float *q, const float *k, const float *extra_k, float *s, int heads, int kv_heads,
                         int dim, int capacity, int start, int length, int extra_length) {
    int total = length + extra_length;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)total * heads) return;
    int h = (int)(i / total), t = (int)(i % total);
    int kh = h / (heads / kv_heads);
    const float *kr = row_of(k, extra_k, t, kv_heads * dim, capacity, start, length, kh, dim);
    float v = 0.0f;
    for (int j = 0; j < dim; ++j) v = fmaf(q[h * dim + j], kr[j], v);
    s[(int64_t)h * total + t] = v / sqrtf((float)dim);
}

// kernels.cl:75-84: one block per row.
__global__ void __launch_bounds__(256) k_softmax(const float *x, float *y, int width) {
    __shared__ float red[kThreads / kWave];
    const float *xr = x + (int64_t)blockIdx.x * width;
    float *yr = y + (int64_t)blockIdx.x * width;
    float m = -INFINITY;
    for (int j = threadIdx.x; j < width; j += blockDim.x) m = fmaxf(m, xr[j]);
    m = block_max(m, red);
    float den = 0.0f;
    for (int j = threadIdx.x; j < width; j += blockDim.x) den += expf(xr[j] - m);
    den = block_sum(den, red);
    for (int j = threadIdx.x; j < width; j += blockDim.x) yr[j] = expf(xr[j] - m) / den;
}

__global__ void k_latent_mask(float *scores, const float *positions, int heads, int length, int memory,
                              int earliest) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)heads * length) return;
    int t = (int)(i % length);
    if (t >= memory && positions[t] < (float)earliest) scores[i] = -INFINITY;
}

// kernels.cl:93-107: one thread per output element, keys in order.
__global__ void k_mix(const float *p, const float *v, const float *extra_v, float *y, int heads, int kv_heads,
                      int dim, int capacity, int start, int length, int extra_length) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= heads * dim) return;
    int h = i / dim, j = i % dim, kh = h / (heads / kv_heads), total = length + extra_length;
    float acc = 0.0f;
    for (int t = 0; t < total; ++t)
        acc = fmaf(p[(int64_t)h * total + t], row_of(v, extra_v, t, kv_heads * dim, capacity, start, length, kh, dim)[j],
                   acc);
    y[i] = acc;
}

__global__ void k_pool_scores(const float *u, const float *q, float *s, int tokens, int slots, int width) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= tokens * slots) return;
    int m = i / tokens, t = i % tokens;
    float v = 0.0f;
    for (int j = 0; j < width; ++j) v = fmaf(u[(int64_t)t * width + j], q[(int64_t)m * width + j], v);
    s[(int64_t)m * tokens + t] = v / sqrtf((float)width);
}

__global__ void k_pool_mix(const float *u, const float *p, float *z, float *anchors, int tokens, int slots,
                           int width, int start_position) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= width * slots) return;
    int m = i / width, j = i % width;
    float v = 0.0f, pos = 0.0f;
    for (int t = 0; t < tokens; ++t) {
        float w = p[(int64_t)m * tokens + t];
        v = fmaf(w, u[(int64_t)t * width + j], v);
        pos = fmaf(w, (float)(start_position + t), pos);
    }
    z[(int64_t)m * width + j] = v;
    if (j == 0) anchors[m] = rintf(pos);
}

__global__ void k_merge_rows(const float *x, float *y, int width, float a, float b) {
    int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j < width) y[j] = (a * x[j] + b * x[width + j]) / (a + b);
}

__global__ void k_block_means(const float *x, float *y, int length, int width, int block) {
    int blocks = (length + block - 1) / block;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)blocks * width) return;
    int b = (int)(i / width), j = (int)(i % width);
    int start = b * block, stop = min(start + block, length);
    float v = 0.0f;
    for (int t = start; t < stop; ++t) v += x[(int64_t)t * width + j];
    y[(int64_t)b * width + j] = v / (float)(stop - start);
}

}  // namespace
}  // namespace mr

using namespace mr;

#define OP_BEGIN(name)                                                      \
    MR_REQUIRE(ctx, name ": null context");                                \
    if (ctx->fail_next) {                                                   \
        ctx->fail_next = false;                                             \
        return fail(MR_ERR_INJECTED, name ": injected failure");            \
    }                                                                       \
    hipStream_t s = ctx->stream;

extern "C" {

int mr_linear(mr_ctx *ctx, const float *x, const void *w, int w_dtype, float *y, int rows, int out_dim, int in_dim) {
    OP_BEGIN("linear");
    MR_REQUIRE(x && w && y && rows > 0 && out_dim > 0 && in_dim > 0, "linear needs x[rows,in] and weight[out,in]");
    return launch_linear(s, x, w, w_dtype, y, rows, out_dim, in_dim);
}

int mr_rms(mr_ctx *ctx, const float *x, const float *w, float *y, int rows, int width, float eps) {
    OP_BEGIN("rms");
    MR_REQUIRE(x && y && rows > 0 && width > 0, "RMSNorm shape mismatch");
    k_rms<<<rows, kThreads, 0, s>>>(x, w, y, width, eps);
    MR_LAUNCHED("enqueue rms");
    return MR_OK;
}

int mr_rope(mr_ctx *ctx, const float *x, const float *freq, const float *pos, float *y, int rows, int heads, int dim,
            int split_half) {
    OP_BEGIN("rope");
    MR_REQUIRE(x && freq && pos && y && rows > 0 && heads > 0 && dim > 0 && dim % 2 == 0, "RoPE shape mismatch");
    k_rope<<<grid_for((int64_t)rows * heads * (dim / 2)), kThreads, 0, s>>>(x, freq, pos, y, rows, heads, dim,
                                                                            split_half);
    MR_LAUNCHED("enqueue rope");
    return MR_OK;
}

int mr_swiglu(mr_ctx *ctx, const float *g, const float *u, float *y, int n) {
    OP_BEGIN("swiglu");
    MR_REQUIRE(g && u && y && n > 0, "SwiGLU shapes differ");
    k_swiglu<<<grid_for(n), kThreads, 0, s>>>(g, u, y, n);
    MR_LAUNCHED("enqueue swiglu");
    return MR_OK;
}

int mr_axpy(mr_ctx *ctx, const float *x, const float *y, float *z, int n, float scale) {
    OP_BEGIN("axpy");
    MR_REQUIRE(x && y && z && n > 0, "residual shapes differ");
    k_axpy<<<grid_for(n), kThreads, 0, s>>>(x, y, z, n, scale);
    MR_LAUNCHED("enqueue axpy");
    return MR_OK;
}

int mr_scores(mr_ctx *ctx, const float *q, const float *k, const float *extra_k, float *sc, int heads, int kv_heads,
              int dim, int capacity, int start, int length, int extra_length) {
    OP_BEGIN("scores");
    MR_REQUIRE(q && k && sc && heads > 0 && kv_heads > 0 && heads % kv_heads == 0 && dim > 0 && capacity > 0 &&
                   length >= 0 && extra_length >= 0 && (extra_length == 0 || extra_k),
               "scores: bad arguments");
    int64_t n = (int64_t)(length + extra_length) * heads;
    if (n == 0) return MR_OK;
    k_scores<<<grid_for(n), kThreads, 0, s>>>(q, k, extra_k, sc, heads, kv_heads, dim, capacity, start, length,
                                              extra_length);
    MR_LAUNCHED("enqueue scores");
    return MR_OK;
}

int mr_softmax(mr_ctx *ctx, const float *x, float *y, int rows, int width) {
    OP_BEGIN("softmax");
    MR_REQUIRE(x && y && rows > 0 && width > 0, "softmax: bad shape");
    k_softmax<<<rows, kThreads, 0, s>>>(x, y, width);
    MR_LAUNCHED("enqueue softmax");
    return MR_OK;
}

int mr_latent_mask(mr_ctx *ctx, float *scores, const float *positions, int heads, int length, int memory,
                   int earliest) {
    OP_BEGIN("latent_mask");
    MR_REQUIRE(scores && positions && heads > 0 && length > 0, "latent_mask: bad arguments");
    k_latent_mask<<<grid_for((int64_t)heads * length), kThreads, 0, s>>>(scores, positions, heads, length, memory,
                                                                         earliest);
    MR_LAUNCHED("enqueue latent_mask");
    return MR_OK;
}

int mr_mix(mr_ctx *ctx, const float *p, const float *v, const float *extra_v, float *y, int heads, int kv_heads,
           int dim, int capacity, int start, int length, int extra_length) {
    OP_BEGIN("mix");
    MR_REQUIRE(p && v && y && heads > 0 && kv_heads > 0 && heads % kv_heads == 0 && dim > 0 && capacity > 0 &&
                   (extra_length == 0 || extra_v),
               "mix: bad arguments");
    k_mix<<<grid_for(heads * dim), kThreads, 0, s>>>(p, v, extra_v, y, heads, kv_heads, dim, capacity, start, length,
                                                      extra_length);
    MR_LAUNCHED("enqueue mix");
    return MR_OK;
}

int mr_pool_scores(mr_ctx *ctx, const float *u, const float *q, float *sc, int tokens, int slots, int width) {
    OP_BEGIN("pool_scores");
    MR_REQUIRE(u && q && sc && tokens > 0 && slots > 0 && width > 0, "pool_scores: bad arguments");
    k_pool_scores<<<grid_for(tokens * slots), kThreads, 0, s>>>(u, q, sc, tokens, slots, width);
    MR_LAUNCHED("enqueue pool_scores");
    return MR_OK;
}

int mr_pool_mix(mr_ctx *ctx, const float *u, const float *p, float *z, float *anchors, int tokens, int slots,
                int width, int start_position) {
    OP_BEGIN("pool_mix");
    MR_REQUIRE(u && p && z && anchors && tokens > 0 && slots > 0 && width > 0, "pool_mix: bad arguments");
    k_pool_mix<<<grid_for(width * slots), kThreads, 0, s>>>(u, p, z, anchors, tokens, slots, width, start_position);
    MR_LAUNCHED("enqueue pool_mix");
    return MR_OK;
}

int mr_merge_rows(mr_ctx *ctx, const float *x, float *y, int width, float a, float b) {
    OP_BEGIN("merge_rows");
    MR_REQUIRE(x && y && width > 0, "merge_rows: bad arguments");
    k_merge_rows<<<grid_for(width), kThreads, 0, s>>>(x, y, width, a, b);
    MR_LAUNCHED("enqueue merge_rows");
    return MR_OK;
}

int mr_block_means(mr_ctx *ctx, const float *x, float *y, int length, int width, int block) {
    OP_BEGIN("block_means");
    MR_REQUIRE(x && y && length > 0 && width > 0 && block > 0, "block_means: bad arguments");
    int blocks = (length + block - 1) / block;
    k_block_means<<<grid_for((int64_t)blocks * width), kThreads, 0, s>>>(x, y, length, width, block);
    MR_LAUNCHED("enqueue block_means");
    return MR_OK;
}

int mr_attention(mr_ctx *ctx, const float *q, const float *k, const float *v, const float *extra_k,
                 const float *extra_v, float *y, int heads, int kv_heads, int dim, int capacity, int start,
                 int length, int extra_length) {
    OP_BEGIN("attention");
    (void)s;
    MR_REQUIRE(q && k && v && y && heads > 0 && kv_heads > 0 && heads % kv_heads == 0 && dim > 0 && capacity > 0 &&
                   length >= 0 && extra_length >= 0 && length + extra_length > 0 &&
                   (extra_length == 0 || (extra_k && extra_v)),
               "attention: bad arguments");
    AttnProblem pr;
    pr.q = q; pr.ring_k = k; pr.ring_v = v; pr.extra_k = extra_k; pr.extra_v = extra_v;
    pr.heads = heads; pr.kv_heads = kv_heads; pr.dim = dim; pr.capacity = capacity;
    pr.start = start; pr.length = length; pr.extra_length = extra_length; pr.out = y;
    return launch_attention_op(ctx, pr);
}

int mr_attention_noalloc(mr_ctx *ctx, const float *q, const float *k, const float *v, const float *extra_k,
                         const float *extra_v, float *y, int heads, int kv_heads, int dim, int capacity, int start,
                         int length, int extra_length) {
    OP_BEGIN("attention_noalloc");
    (void)s;
    MR_REQUIRE(q && k && v && y && heads > 0 && kv_heads > 0 && heads % kv_heads == 0 && dim > 0 && capacity > 0 &&
                   length >= 0 && extra_length >= 0 && length + extra_length > 0 &&
                   (extra_length == 0 || (extra_k && extra_v)),
               "attention_noalloc: bad arguments");
    AttnProblem pr;
    pr.q = q; pr.ring_k = k; pr.ring_v = v; pr.extra_k = extra_k; pr.extra_v = extra_v;
    pr.heads = heads; pr.kv_heads = kv_heads; pr.dim = dim; pr.capacity = capacity;
    pr.start = start; pr.length = length; pr.extra_length = extra_length; pr.out = y;
    return launch_attention_op_noalloc(ctx, pr);
}

int mr_debug_gemm(mr_ctx *ctx, const float *a, const void *w, float *c, float *ascale, int m, int n, int k,
                  int scheme) {
    OP_BEGIN("debug gemm");
    MR_REQUIRE(a && w && c && m > 0 && n > 0 && k > 0 && k % 8 == 0 && (scheme == 0 || (scheme == 1 && ascale)),
               "debug gemm: bad arguments");
    GemmArgs g;
    g.a = a; g.lda = k; g.w = w; g.dtype = MR_BF16; g.c = c; g.ldc = n; g.m = m; g.n = n; g.k = k;
    if (scheme == 1) {
        MR_TRY(gemm_f16_weight_scale(s, w, MR_BF16, (int64_t)n * k, &g.wscale));
        MR_REQUIRE(g.wscale > 0.0f, "debug gemm: weights not eligible for FP16 terms");
        g.ascale = ascale;
        MR_HIP(hipMalloc((void **)&g.ahl_ws, (size_t)2 * m * k * sizeof(_Float16)), "debug gemm workspace");
        void *wh = nullptr;
        const hipError_t ea = hipMalloc(&wh, (size_t)n * k * 2);
        if (ea != hipSuccess) {
            (void)hipFree(g.ahl_ws);
            MR_HIP(ea, "debug gemm workspace");
        }
        g.wh = wh;
        const int rc = gemm_f16_weight_copy(s, w, (int64_t)n * k, g.wscale, wh);
        if (rc != MR_OK) {
            (void)hipFree(g.ahl_ws);
            (void)hipFree(wh);
            return rc;
        }
    }
    int rc = launch_gemm(s, GEMM_STORE, g);
    const hipError_t e = hipStreamSynchronize(s);
    if (g.ahl_ws) (void)hipFree(g.ahl_ws);
    if (g.wh) (void)hipFree(const_cast<void *>(g.wh));
    MR_TRY(rc);
    MR_HIP(e, "debug gemm");
    return MR_OK;
}

int mr_debug_gemm_grouped(mr_ctx *ctx, const float *a, const void *w, const void *w2, float *c, const int *counts,
                          int groups, int n, int k, int swiglu, int tile_list) {
    OP_BEGIN("debug grouped gemm");
    MR_REQUIRE(a && w && c && counts && groups > 0 && groups <= 1024 && n > 0 && k > 0 && k % 8 == 0 &&
                   (!swiglu || w2),
               "debug grouped gemm: bad arguments");
    std::vector<int> offset(groups), start(groups + 1);
    int rows = 0, max_rows = 0;
    start[0] = 0;
    for (int z = 0; z < groups; ++z) {
        MR_REQUIRE(counts[z] >= 0, "debug grouped gemm: negative group size");
        offset[z] = rows;
        rows += counts[z];
        max_rows = std::max(max_rows, counts[z]);
        start[z + 1] = start[z] + ceil_div(counts[z], kGemmRowTile);
    }
    MR_REQUIRE(rows > 0, "debug grouped gemm: no rows");
    std::vector<void *> owned;   // freed on every return
    auto alloc = [&](size_t bytes, void **p) {
        const hipError_t e = hipMalloc(p, bytes);
        if (e == hipSuccess) owned.push_back(*p);
        return e;
    };
    struct Free {   // after the stream's work on them
        std::vector<void *> &v;
        hipStream_t s;
        ~Free() {
            (void)hipStreamSynchronize(s);
            for (void *p : v) (void)hipFree(p);
        }
    } release{owned, s};
    const int mats = swiglu ? 2 : 1;
    const int64_t nk = (int64_t)n * k;
    std::vector<void *> tab_w(mats * groups), tab_h(mats * groups);
    std::vector<float> scale(mats * groups);
    _Float16 *wh = nullptr;
    MR_HIP(alloc((size_t)mats * groups * nk * 2, (void **)&wh), "debug grouped gemm workspace");
    // a scale per matrix; a group's gate and up rows share the smaller, as
    // the model's expert copies do (the SwiGLU kernel unscales both by one)
    for (int t = 0; t < mats; ++t)
        for (int z = 0; z < groups; ++z) {
            const void *src = (const char *)(t ? w2 : w) + (size_t)z * nk * 2;
            float sc = 0.0f;
            MR_TRY(gemm_f16_weight_scale(s, src, MR_BF16, nk, &sc));
            MR_REQUIRE(sc > 0.0f, "debug grouped gemm: weights not eligible for FP16 terms");
            tab_w[t * groups + z] = const_cast<void *>(src);
            scale[t * groups + z] = sc;
        }
    for (int z = 0; z < groups && mats == 2; ++z)
        scale[z] = scale[groups + z] = std::min(scale[z], scale[groups + z]);
    for (int t = 0; t < mats; ++t)
        for (int z = 0; z < groups; ++z) {
            _Float16 *dst = wh + ((size_t)t * groups + z) * nk;
            MR_TRY(gemm_f16_weight_copy(s, tab_w[t * groups + z], nk, scale[t * groups + z], dst));
            tab_h[t * groups + z] = dst;
        }
    void **d_w = nullptr, **d_h = nullptr;
    float *d_scale = nullptr, *ascale = nullptr;
    int *d_off = nullptr, *d_cnt = nullptr, *d_start = nullptr;
    _Float16 *planes = nullptr;
    MR_HIP(alloc(tab_w.size() * sizeof(void *), (void **)&d_w), "debug grouped gemm workspace");
    MR_HIP(alloc(tab_h.size() * sizeof(void *), (void **)&d_h), "debug grouped gemm workspace");
    MR_HIP(alloc(scale.size() * sizeof(float), (void **)&d_scale), "debug grouped gemm workspace");
    MR_HIP(alloc((size_t)groups * sizeof(int), (void **)&d_off), "debug grouped gemm workspace");
    MR_HIP(alloc((size_t)groups * sizeof(int), (void **)&d_cnt), "debug grouped gemm workspace");
    MR_HIP(alloc((size_t)(groups + 1) * sizeof(int), (void **)&d_start), "debug grouped gemm workspace");
    MR_HIP(alloc((size_t)rows * sizeof(float), (void **)&ascale), "debug grouped gemm workspace");
    MR_HIP(alloc((size_t)2 * rows * k * sizeof(_Float16), (void **)&planes), "debug grouped gemm workspace");
    MR_HIP(hipMemcpy(d_w, tab_w.data(), tab_w.size() * sizeof(void *), hipMemcpyHostToDevice), "debug grouped gemm");
    MR_HIP(hipMemcpy(d_h, tab_h.data(), tab_h.size() * sizeof(void *), hipMemcpyHostToDevice), "debug grouped gemm");
    MR_HIP(hipMemcpy(d_scale, scale.data(), scale.size() * sizeof(float), hipMemcpyHostToDevice), "debug grouped gemm");
    MR_HIP(hipMemcpy(d_off, offset.data(), groups * sizeof(int), hipMemcpyHostToDevice), "debug grouped gemm");
    MR_HIP(hipMemcpy(d_cnt, counts, groups * sizeof(int), hipMemcpyHostToDevice), "debug grouped gemm");
    MR_HIP(hipMemcpy(d_start, start.data(), (groups + 1) * sizeof(int), hipMemcpyHostToDevice), "debug grouped gemm");
    GemmArgs g;
    g.a = a; g.lda = k; g.dtype = MR_BF16; g.c = c; g.ldc = n; g.m = rows; g.n = n; g.k = k;
    g.ascale = ascale; g.ahl_ws = planes;
    GemmGroups gg;
    gg.offset = d_off; gg.count = d_cnt; gg.groups = groups; gg.max_rows = max_rows;
    gg.w = d_w; gg.w2 = swiglu ? d_w + groups : nullptr;
    gg.wh = d_h; gg.wh2 = swiglu ? d_h + groups : nullptr; gg.wscale = d_scale;
    if (tile_list) {
        gg.row_tile_start = d_start;
        gg.row_tiles = start[groups];
    }
    MR_TRY(launch_gemm_grouped(s, swiglu ? GEMM_SWIGLU : GEMM_STORE, g, gg));
    MR_HIP(hipStreamSynchronize(s), "debug grouped gemm");
    return MR_OK;
}

int mr_debug_exp(mr_ctx *ctx, const float *x, float *y, int n, int which) {
    OP_BEGIN("debug exp");
    MR_TRY(launch_debug_exp(s, x, y, n, which));
    MR_HIP(hipStreamSynchronize(s), "debug exp");
    return MR_OK;
}

int mr_debug_prefill_attention(mr_ctx *ctx, const float *qkv, const float *ring_k, const float *ring_v, float *out,
                               int rows, int p0, int heads, int kv_heads, int d, int cap, int window, int presplit) {
    OP_BEGIN("debug prefill attention");
    MR_REQUIRE(qkv && ring_k && ring_v && out && rows > 0 && p0 >= 0 && heads > 0 && kv_heads > 0 && d > 0 &&
                   cap > 0 && window >= 0,
               "debug prefill attention: bad arguments");
    PrefillAttnArgs a;
    a.qkv = qkv; a.ld = (heads + 2 * kv_heads) * d; a.ring_k = ring_k; a.ring_v = ring_v; a.cap = cap;
    a.out = out; a.ldo = heads * d; a.p0 = p0; a.rows = rows; a.heads = heads; a.kv_heads = kv_heads; a.d = d;
    a.inv_root = 1.0f / sqrtf((float)d); a.window = window;
    void *ws = nullptr;
    if (presplit) {
        const int n = ceil_div(rows + std::min(p0, (window ? window : cap) - 1), 32) * 32;   // whole 32-row tiles
        const size_t planes = (size_t)4 * n * kv_heads * d * sizeof(_Float16);
        MR_HIP(hipMalloc(&ws, planes + 4 * kv_heads * sizeof(float)), "debug prefill attention workspace");
        a.kv16 = (_Float16 *)ws;
        a.kv16_rows = n;
        a.kv16_scale = (float *)((char *)ws + planes);
        a.kv16_max = (unsigned *)(a.kv16_scale + 2 * kv_heads);
    }
    const int rc = launch_prefill_attention(s, a);
    const hipError_t e = hipStreamSynchronize(s);
    if (ws) (void)hipFree(ws);
    MR_TRY(rc);
    MR_HIP(e, "debug prefill attention");
    return MR_OK;
}

}  // extern "C"
