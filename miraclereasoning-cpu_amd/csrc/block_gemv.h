// y[r] = W[r] . x for the rows r < n of a small weight block, by one
// workgroup: x (k floats) in LDS, a lane group of lpr lanes per row holding
// 16-byte weight vectors, every weight load of a batch in flight before the
// products.  For the per-token projections whose rows a single workgroup
// post-processes (normalization, rotation, cache append) itself.  The first
// batch is issued apart (issue) so a kernel can send it before the loads its
// input depends on; finish waits for it, takes the products and runs any
// further batches.
#pragma once

#include "common.h"

namespace mr {

constexpr int kBlockGemvBatch = 16;   // weight vectors per thread in flight

// k % (elements per 16-byte vector) == 0 and k / (elements per vector) <= 64.
template <int DT>
__host__ __device__ constexpr bool block_gemv_fits(int k) {
    return k % (DT == MR_F32 ? 4 : 8) == 0 && k / (DT == MR_F32 ? 4 : 8) <= 64;
}

template <int DT>
struct BlockGemv {
    static constexpr int E = DT == MR_F32 ? 4 : 8;   // elements per 16-byte vector
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    v4u q[kBlockGemvBatch];
    const v4u *wv;
    int n, nvec, lpr, rpp, sub, passes;

    __device__ __forceinline__ void load(int p0) {
#pragma unroll
        for (int i = 0; i < kBlockGemvBatch; ++i) {   // clamped, unguarded: every load issues at once
            const int r = min((p0 + i) * rpp + (int)threadIdx.x / lpr, n - 1);
            q[i] = __builtin_nontemporal_load(wv + (int64_t)r * nvec + min(sub, nvec - 1));
        }
    }

    __device__ __forceinline__ void issue(const void *w, int rows, int k) {
        wv = (const v4u *)w;
        n = rows;
        nvec = k / E;
        lpr = 1;
        while (lpr < nvec) lpr *= 2;
        rpp = (int)blockDim.x / lpr;
        sub = (int)threadIdx.x % lpr;
        passes = (n + rpp - 1) / rpp;
        load(0);
    }

    __device__ __forceinline__ void finish(const float *xs, float *ys) {
        for (int p0 = 0; p0 < passes; p0 += kBlockGemvBatch) {
            if (p0 > 0) load(p0);
#pragma unroll
            for (int i = 0; i < kBlockGemvBatch; ++i) {
                const int r = (p0 + i) * rpp + (int)threadIdx.x / lpr;
                float acc = 0.0f;
                if (sub < nvec) {
                    const float *x = xs + sub * E;
                    const unsigned u[4] = {q[i].x, q[i].y, q[i].z, q[i].w};
                    if constexpr (DT == MR_F32) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc = fmaf(__uint_as_float(u[e]), x[e], acc);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float lo = DT == MR_BF16 ? __uint_as_float(u[e] << 16) : f16_to_f32(u[e] & 0xffffu);
                            const float hi =
                                DT == MR_BF16 ? __uint_as_float(u[e] & 0xffff0000u) : f16_to_f32(u[e] >> 16);
                            acc = fmaf(lo, x[2 * e], acc);
                            acc = fmaf(hi, x[2 * e + 1], acc);
                        }
                    }
                }
                acc = group_sum(acc, lpr);
                if (sub == 0 && p0 + i < passes && r < n) ys[r] = acc;
            }
        }
    }
};

}  // namespace mr
