/*
 * ORACLE — test infrastructure only. Nothing in the shipped library calls this.
 *
 * A plain-C restatement of the work-item arithmetic of the reference's 13 OpenCL
 * kernels (miracle_reasoning/kernels.cl).  Each function walks the same NDRange
 * the reference enqueues (miracle_reasoning/opencl.py:241-300) and performs, for
 * each work-item, the same operations in the same order.  It is compiled with
 * -ffp-contract=off, the counterpart of `#pragma OPENCL FP_CONTRACT OFF`
 * (kernels.cl:3), and without fast-math, so every product is rounded before it is
 * added.  Work-items are independent, so OpenMP over them changes nothing in the
 * results.
 *
 * Transcendentals: the reference takes cos/sin/exp/sqrt from whichever OpenCL
 * runtime is installed (unpinned at the ulp level).  Here sqrt and division are
 * IEEE correctly rounded; cos and sin are evaluated in double and rounded once
 * (correctly rounded except for rare double-rounding cases); exp is glibc expf.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

#define EXPORT __attribute__((visibility("default")))

/* kernels.cl:5-17. y[r,o] = x[r,:] . w[o,:] with four interleaved lane sums
 * (lane l sums j = l mod 4, j < in_dim rounded down to a multiple of 4), the lanes
 * folded as ((x+y)+z)+w, then a sequential tail. */
EXPORT void oc_linear(const float *x, const float *w, float *y, int rows, int out_dim, int in_dim) {
    long total = (long)rows * out_dim;
#pragma omp parallel for schedule(static)
    for (long i = 0; i < total; ++i) {
        long r = i / out_dim, o = i % out_dim;
        const float *xr = x + r * (long)in_dim, *wr = w + o * (long)in_dim;
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
        int j = 0;
        for (; j + 3 < in_dim; j += 4) {
            s0 += xr[j] * wr[j];
            s1 += xr[j + 1] * wr[j + 1];
            s2 += xr[j + 2] * wr[j + 2];
            s3 += xr[j + 3] * wr[j + 3];
        }
        float v = s0 + s1 + s2 + s3;
        for (; j < in_dim; ++j) v += xr[j] * wr[j];
        y[r * (long)out_dim + o] = v;
    }
}

/* Same arithmetic with BF16 weights (raw bits).  Widening BF16 to FP32 is exact
 * (weights.py:70), so this equals oc_linear on the widened matrix; it only saves
 * the oracle from holding an FP32 copy of a large model. */
EXPORT void oc_linear_bf16(const float *x, const uint16_t *w, float *y, int rows, int out_dim, int in_dim) {
    long total = (long)rows * out_dim;
#pragma omp parallel for schedule(static)
    for (long i = 0; i < total; ++i) {
        long r = i / out_dim, o = i % out_dim;
        const float *xr = x + r * (long)in_dim;
        const uint16_t *wr = w + o * (long)in_dim;
        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        int j = 0;
        for (; j + 3 < in_dim; j += 4) {
            for (int l = 0; l < 4; ++l) {
                union { uint32_t u; float f; } c;
                c.u = (uint32_t)wr[j + l] << 16;
                s[l] += xr[j + l] * c.f;
            }
        }
        float v = s[0] + s[1] + s[2] + s[3];
        for (; j < in_dim; ++j) {
            union { uint32_t u; float f; } c;
            c.u = (uint32_t)wr[j] << 16;
            v += xr[j] * c.f;
        }
        y[r * (long)out_dim + o] = v;
    }
}

/* kernels.cl:19-28. Sequential sum of squares, scale = 1/sqrt(mean + eps),
 * y = (x * scale) * (affine ? w : 1). */
EXPORT void oc_rms(const float *x, const float *w, float *y, int rows, int width, float eps, int affine) {
#pragma omp parallel for schedule(static) if (rows > 1)
    for (int r = 0; r < rows; ++r) {
        const float *xr = x + (long)r * width;
        float v = 0.0f;
        for (int j = 0; j < width; ++j) { float a = xr[j]; v += a * a; }
        float scale = 1.0f / sqrtf(v / (float)width + eps);
        for (int j = 0; j < width; ++j)
            y[(long)r * width + j] = xr[j] * scale * (affine ? w[j] : 1.0f);
    }
}

/* kernels.cl:30-44. The angle is the FP32 product pos*freq; pairs are (2p, 2p+1)
 * (interleaved) or (p, p+dim/2) (split half). */
EXPORT void oc_rope(const float *x, const float *freq, const float *pos, float *y,
                    int rows, int heads, int dim, int split_half) {
    int half = dim / 2;
    long total = (long)rows * heads * half;
#pragma omp parallel for schedule(static) if (total > 4096)
    for (long i = 0; i < total; ++i) {
        int p = (int)(i % half);
        long head_row = i / half, base = head_row * dim;
        float a = pos[head_row / heads] * freq[p];
        float c = (float)cos((double)a), s = (float)sin((double)a);
        int j = split_half ? p : 2 * p;
        int k = split_half ? p + half : 2 * p + 1;
        float u = x[base + j], v = x[base + k];
        y[base + j] = u * c - v * s;
        y[base + k] = u * s + v * c;
    }
}

/* kernels.cl:46-50. */
EXPORT void oc_swiglu(const float *g, const float *u, float *y, int n) {
#pragma omp parallel for schedule(static) if (n > 4096)
    for (int i = 0; i < n; ++i) y[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

/* kernels.cl:52-56. */
EXPORT void oc_axpy(const float *x, const float *y, float *z, int n, float scale) {
    for (int i = 0; i < n; ++i) z[i] = x[i] + scale * y[i];
}

/* Row of a key/value inside the logical order [ring window, extra rows]
 * (kernels.cl:67-68 and :102-103). */
static inline const float *kv_row(const float *ring, const float *extra, int t, int kv_heads, int dim,
                                  int capacity, int start, int length, int kh) {
    if (t < length) return ring + ((long)((start + t) % capacity) * kv_heads * dim + (long)kh * dim);
    return extra + ((long)(t - length) * kv_heads * dim + (long)kh * dim);
}

/* kernels.cl:58-73. */
EXPORT void oc_scores(const float *q, const float *k, const float *extra_k, float *s,
                      int heads, int kv_heads, int dim, int capacity, int start, int length, int extra_length) {
    int total = length + extra_length;
    int group = heads / kv_heads;
    long n = (long)total * heads;
#pragma omp parallel for schedule(static) if (n > 1024)
    for (long i = 0; i < n; ++i) {
        int h = (int)(i / total), t = (int)(i % total);
        const float *kr = kv_row(k, extra_k, t, kv_heads, dim, capacity, start, length, h / group);
        float v = 0.0f;
        for (int j = 0; j < dim; ++j) v += q[(long)h * dim + j] * kr[j];
        s[(long)h * total + t] = v / sqrtf((float)dim);
    }
}

/* kernels.cl:75-84. Three sequential passes per row. */
EXPORT void oc_softmax(const float *x, float *y, int rows, int width) {
#pragma omp parallel for schedule(static) if (rows > 1)
    for (int r = 0; r < rows; ++r) {
        const float *xr = x + (long)r * width;
        float m = -INFINITY;
        for (int j = 0; j < width; ++j) m = fmaxf(m, xr[j]);
        float denom = 0.0f;
        for (int j = 0; j < width; ++j) denom += expf(xr[j] - m);
        for (int j = 0; j < width; ++j) y[(long)r * width + j] = expf(xr[j] - m) / denom;
    }
}

/* kernels.cl:86-91. */
EXPORT void oc_latent_mask(float *scores, const float *positions, int heads, int length, int memory, int earliest) {
    for (int h = 0; h < heads; ++h)
        for (int t = 0; t < length; ++t)
            if (t >= memory && positions[t] < (float)earliest) scores[(long)h * length + t] = -INFINITY;
}

/* kernels.cl:93-107. One sequential sum over keys per output element. */
EXPORT void oc_mix(const float *p, const float *v, const float *extra_v, float *y,
                   int heads, int kv_heads, int dim, int capacity, int start, int length, int extra_length) {
    int total = length + extra_length, group = heads / kv_heads;
    long n = (long)heads * dim;
#pragma omp parallel for schedule(static) if (n > 256)
    for (long i = 0; i < n; ++i) {
        int h = (int)(i / dim), j = (int)(i % dim);
        float acc = 0.0f;
        for (int t = 0; t < total; ++t) {
            const float *vr = kv_row(v, extra_v, t, kv_heads, dim, capacity, start, length, h / group);
            acc += p[(long)h * total + t] * vr[j];
        }
        y[i] = acc;
    }
}

/* kernels.cl:110-117. */
EXPORT void oc_pool_scores(const float *u, const float *q, float *s, int tokens, int slots, int width) {
    for (int m = 0; m < slots; ++m)
        for (int t = 0; t < tokens; ++t) {
            float v = 0.0f;
            for (int j = 0; j < width; ++j) v += u[(long)t * width + j] * q[(long)m * width + j];
            s[(long)m * tokens + t] = v / sqrtf((float)width);
        }
}

/* kernels.cl:119-130. Anchors are rint (ties to even) of the probability-weighted
 * mean position. */
EXPORT void oc_pool_mix(const float *u, const float *p, float *z, float *anchors,
                        int tokens, int slots, int width, int start_position) {
    for (int m = 0; m < slots; ++m)
        for (int j = 0; j < width; ++j) {
            float v = 0.0f, pos = 0.0f;
            for (int t = 0; t < tokens; ++t) {
                float w = p[(long)m * tokens + t];
                v += w * u[(long)t * width + j];
                pos += w * (float)(start_position + t);
            }
            z[(long)m * width + j] = v;
            if (j == 0) anchors[m] = rintf(pos);
        }
}

/* kernels.cl:133-137. */
EXPORT void oc_merge_rows(const float *x, float *y, int width, float a, float b) {
    for (int j = 0; j < width; ++j) y[j] = (a * x[j] + b * x[width + j]) / (a + b);
}

/* kernels.cl:140-148. The last block averages only the rows it has. */
EXPORT void oc_block_means(const float *x, float *y, int length, int width, int block) {
    int blocks = (length + block - 1) / block;
#pragma omp parallel for schedule(static) if ((long)blocks * width > 4096)
    for (long i = 0; i < (long)blocks * width; ++i) {
        int b = (int)(i / width), j = (int)(i % width);
        int start = b * block, stop = start + block < length ? start + block : length;
        float v = 0.0f;
        for (int t = start; t < stop; ++t) v += x[(long)t * width + j];
        y[(long)b * width + j] = v / (float)(stop - start);
    }
}
