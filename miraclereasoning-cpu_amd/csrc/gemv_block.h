// Vectorized GEMV rows (decode projections): the device code of k_gemv_vec,
// shared with kernels that run projection rows in some of their workgroups.
//
// GEMV layout: the weight matrix stays in its stored dtype, row-major [n, k]
// (the reference's [out, in] layout, weights.py:211-245).  The input vector is
// staged in LDS as FP32 (after an optional RMSNorm prologue computed by every
// workgroup from the same values, so all workgroups see identical x).  A group
// of `lpr` lanes owns R output rows; each lane streams 16-byte weight vectors
// (8 BF16/F16 or 4 FP32 values) at a stride of lpr vectors, widens them in
// registers and accumulates with FMA in FP32, then the group reduces by lane
// shuffles.
#pragma once

#include <type_traits>

#include "linear.h"

namespace mr {
namespace gemv {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;

template <int DT>
struct Vec16;
template <>
struct Vec16<MR_F32> {
    static constexpr int E = 4;
    __device__ static void widen(const u32x4 &v, float *o) {
        o[0] = __uint_as_float(v.x); o[1] = __uint_as_float(v.y);
        o[2] = __uint_as_float(v.z); o[3] = __uint_as_float(v.w);
    }
};
template <>
struct Vec16<MR_BF16> {
    static constexpr int E = 8;
    __device__ static void widen(const u32x4 &v, float *o) {
        o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xffff0000u);
        o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xffff0000u);
        o[4] = __uint_as_float(v.z << 16); o[5] = __uint_as_float(v.z & 0xffff0000u);
        o[6] = __uint_as_float(v.w << 16); o[7] = __uint_as_float(v.w & 0xffff0000u);
    }
};
template <>
struct Vec16<MR_F16> {
    static constexpr int E = 8;
    __device__ static void widen(const u32x4 &v, float *o) {
        o[0] = f16_to_f32(v.x & 0xffffu); o[1] = f16_to_f32(v.x >> 16);
        o[2] = f16_to_f32(v.y & 0xffffu); o[3] = f16_to_f32(v.y >> 16);
        o[4] = f16_to_f32(v.z & 0xffffu); o[5] = f16_to_f32(v.z >> 16);
        o[6] = f16_to_f32(v.w & 0xffffu); o[7] = f16_to_f32(v.w >> 16);
    }
};

template <int DT>
__device__ __forceinline__ u32x4 load16(const void *base, int64_t elem) {
    constexpr int bytes = DT == MR_F32 ? 4 : 2;
    return __builtin_nontemporal_load((const u32x4 *)((const char *)base + elem * bytes));
}

// Stage x into LDS, applying the RMSNorm prologue (kernels.cl:19-28 arithmetic:
// scale = 1/sqrt(sum/k + eps), x * scale * gain).  With k a multiple of 4 and
// 16-byte aligned vectors, each thread has kStageBatch float4 loads of x (and
// of the gain, parked in LDS after xs until the scale is known) in flight at
// once; otherwise element by element.
constexpr int kStageBatch = 8;

__host__ __device__ inline int gemv_xs_floats(int k) { return (k + 3) & ~3; }

template <int PRO>
__device__ __forceinline__ void stage_x(const GemvArgs &a, float *xs, float *red) {
    const int tid = threadIdx.x;
    const float *gain = PRO == PRO_RMS ? a.gain : nullptr;
    float *gs = xs + gemv_xs_floats(a.k);   // PRO_RMS with a gain: the gain (red follows it)
    float ss = 0.0f;
    const bool vec = (a.k & 3) == 0 && ((uintptr_t)a.x & 15) == 0 && ((uintptr_t)gain & 15) == 0;
    // One loop per gain case: a load guarded by a runtime test inside the
    // batch makes the compiler wait for each load in turn (measured: the RMS
    // prologue took 8.6 µs of a 2304 x 2048 GEMV instead of 4.6).
    auto batches = [&](auto with_gain) {
        constexpr bool G = decltype(with_gain)::value;
        const int n4 = a.k / 4;
        for (int base = tid; base < n4; base += kGemvThreads * kStageBatch) {
            float4 xv[kStageBatch], gv[kStageBatch];
#pragma unroll
            for (int i = 0; i < kStageBatch; ++i) {   // clamped, unguarded: the loads issue together
                const int j = min(base + i * kGemvThreads, n4 - 1);
                xv[i] = *(const float4 *)(a.x + 4 * j);
                if constexpr (G) gv[i] = *(const float4 *)(gain + 4 * j);
            }
#pragma unroll
            for (int i = 0; i < kStageBatch; ++i) {
                const int j = base + i * kGemvThreads;
                if (j < n4) {
                    *(float4 *)(xs + 4 * j) = xv[i];
                    if constexpr (G) *(float4 *)(gs + 4 * j) = gv[i];
                    ss = fmaf(xv[i].x, xv[i].x, ss);
                    ss = fmaf(xv[i].y, xv[i].y, ss);
                    ss = fmaf(xv[i].z, xv[i].z, ss);
                    ss = fmaf(xv[i].w, xv[i].w, ss);
                }
            }
        }
    };
    if (vec) {
        if (gain) batches(std::true_type{});
        else batches(std::false_type{});
    } else {
        for (int j = tid; j < a.k; j += blockDim.x) {
            const float v = a.x[j];
            xs[j] = v;
            if (gain) gs[j] = gain[j];
            ss = fmaf(v, v, ss);
        }
    }
    if constexpr (PRO == PRO_RMS) {
        ss = block_sum(ss, red);   // its barriers also publish xs and gs
        const float scale = 1.0f / sqrtf(ss / (float)a.k + a.eps);
        for (int j = tid; j < a.k; j += blockDim.x) {
            const float v = xs[j] * scale * (gain ? gs[j] : 1.0f);
            xs[j] = v;
            if (a.x_out && blockIdx.x == 0) a.x_out[j] = v;   // (the first workgroup of the launch)
        }
    }
    __syncthreads();
}

// LDS of a GEMV workgroup: xs, the gain (RMS prologue with a gain), then the
// reduction scratch.
__host__ __device__ inline int gemv_red_offset(const GemvArgs &a, int pro) {
    return gemv_xs_floats(a.k) * (pro == PRO_RMS && a.gain ? 2 : 1);
}

template <int EPI>
__device__ __forceinline__ void finish_row(const GemvArgs &a, int row, float acc, float acc2) {
    if constexpr (EPI == EPI_STORE) {
        a.y[row] = acc;
    } else if constexpr (EPI == EPI_RESIDUAL) {
        // hidden + scale * projected, each product rounded (kernels.cl:52-56)
        a.y[row] = a.y[row] + a.scale * acc;
    } else if constexpr (EPI == EPI_SCALE_ADD) {
        a.y[row] = a.y[row] + (*a.scale_ptr) * acc;
    } else if constexpr (EPI == EPI_GATED) {
        const float branch = (0.0f + (*a.scale_ptr) * a.aux[row]) + (*a.scale_ptr2) * acc;
        a.y[row] = a.y[row] + a.scale * branch;
    } else if constexpr (EPI == EPI_GATED_ATTN) {
        const float branch = (0.0f + (*a.scale_ptr) * acc) + (*a.scale_ptr2) * a.aux[row];
        a.y[row] = a.y[row] + a.scale * branch;
    } else {
        // SwiGLU (kernels.cl:46-50): (g / (1 + exp(-g))) * u
        a.y[row] = (acc / (1.0f + expf(-acc))) * acc2;
    }
}

// The rows of workgroup `block` of a k_gemv_vec launch; smem holds
// gemv_lds_floats(a, PRO) floats.  Also run by other kernels' workgroups
// that carry a projection alongside their own work.
template <int DT, int R, int U, int PRO, int EPI>
__device__ __forceinline__ void gemv_vec_block(const GemvArgs &a, int lpr, int block, float *smem) {
    using V = Vec16<DT>;
    constexpr int E = V::E;
    constexpr int M = EPI == EPI_SWIGLU ? 2 : 1;   // matrices read per row
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane & (lpr - 1), slot = lane / lpr;
    const int slots = kWave / lpr;
    const int row0 = ((block * kGemvWaves + wave) * slots + slot) * R;
    const int nvec = a.k / E;
    const int64_t k = a.k;
    int64_t rowoff[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rowoff[r] = (int64_t)min(row0 + r, a.n - 1) * k;

    // Weight vectors of one batch: U vectors per row per matrix, lane-strided.
    u32x4 wv[U][R][M];
    auto issue = [&](int b) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int v = sub + (b * U + u) * lpr;
            if (v < nvec) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    wv[u][r][0] = load16<DT>(a.w, rowoff[r] + (int64_t)v * E);
                    if constexpr (M == 2) wv[u][r][1] = load16<DT>(a.w2, rowoff[r] + (int64_t)v * E);
                }
            }
        }
    };
    // The first batch is in flight while the flag is read and the prologue
    // stages x.
    issue(0);
    if (a.done && *a.done) return;
    float *xs = smem;
    float *red = smem + gemv_red_offset(a, PRO);
    stage_x<PRO>(a, xs, red);

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
    for (int b = 0;; ++b) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int v = sub + (b * U + u) * lpr;
            if (v < nvec) {
                float xv[E];
#pragma unroll
                for (int e = 0; e < E; e += 4) {
                    float4 t = *(const float4 *)(xs + v * E + e);
                    xv[e] = t.x; xv[e + 1] = t.y; xv[e + 2] = t.z; xv[e + 3] = t.w;
                }
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        float wf[E];
                        V::widen(wv[u][r][m], wf);
#pragma unroll
                        for (int e = 0; e < E; ++e) acc[r][m] = fmaf(wf[e], xv[e], acc[r][m]);
                    }
            }
        }
        if (sub + (b + 1) * U * lpr >= nvec) break;
        issue(b + 1);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = group_sum(acc[r][m], lpr);
    if (sub == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + r < a.n) finish_row<EPI>(a, row0 + r, acc[r][0], acc[r][M - 1]);
    }
}


// LDS floats of one GEMV workgroup.
__host__ __device__ inline int gemv_lds_floats(const GemvArgs &a, int pro) { return gemv_red_offset(a, pro) + kGemvWaves; }

}  // namespace gemv
}  // namespace mr
