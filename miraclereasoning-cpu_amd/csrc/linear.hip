// GEMV (decode) and small GEMM (op-level) projection kernels; the GEMV rows'
// device code (layout, staging, epilogues) is in gemv_block.h.
#include "linear.h"

#include "gemv_block.h"

namespace mr {

namespace {

using namespace gemv;

template <int DT, int R, int U, int PRO, int EPI>
__global__ void __launch_bounds__(kGemvThreads) k_gemv_vec(GemvArgs a, int lpr) {
    extern __shared__ float smem[];
    gemv_vec_block<DT, R, U, PRO, EPI>(a, lpr, blockIdx.x, smem);
}

// Any k, any alignment: one wave per row, lanes stride over elements.
template <int DT, int PRO, int EPI>
__global__ void __launch_bounds__(kGemvThreads) k_gemv_scalar(GemvArgs a) {
    extern __shared__ float smem[];
    if (a.done && *a.done) return;
    float *xs = smem;
    float *red = smem + gemv_red_offset(a, PRO);
    stage_x<PRO>(a, xs, red);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = blockIdx.x * kGemvWaves + wave;
    if (row >= a.n) return;
    float acc = 0.0f, acc2 = 0.0f;
    for (int j = lane; j < a.k; j += kWave) {
        acc = fmaf(load_w<DT>(a.w, (int64_t)row * a.k + j), xs[j], acc);
        if constexpr (EPI == EPI_SWIGLU) acc2 = fmaf(load_w<DT>(a.w2, (int64_t)row * a.k + j), xs[j], acc2);
    }
    acc = wave_sum(acc);
    if constexpr (EPI == EPI_SWIGLU) acc2 = wave_sum(acc2);
    if (lane == 0) finish_row<EPI>(a, row, acc, acc2);
}

template <int DT, int PRO, int EPI>
int launch_gemv_t(hipStream_t s, const GemvArgs &a) {
    constexpr int E = Vec16<DT>::E;
    const int bytes = DT == MR_F32 ? 4 : 2;
    size_t lds = (size_t)(gemv_red_offset(a, PRO) + kGemvWaves) * sizeof(float);
    bool aligned = (a.k % E) == 0 && ((uintptr_t)a.w % 16) == 0 &&
                   (EPI != EPI_SWIGLU || ((uintptr_t)a.w2 % 16) == 0) && ((int64_t)a.k * bytes) % 16 == 0;
    if (aligned) {
        int nvec = a.k / E;
        int lpr = 1;
        while (lpr * 2 <= nvec && lpr < kWave) lpr *= 2;
        const int slots = kWave / lpr;
        const int per_lane = ceil_div(nvec, lpr);   // vectors per lane per row
        constexpr int R = EPI == EPI_SWIGLU ? 1 : 2;
        int grid = ceil_div(a.n, kGemvWaves * slots * R);
        if (per_lane <= 2)
            k_gemv_vec<DT, R, 2, PRO, EPI><<<grid, kGemvThreads, lds, s>>>(a, lpr);
        else if (per_lane <= 4)
            k_gemv_vec<DT, R, 4, PRO, EPI><<<grid, kGemvThreads, lds, s>>>(a, lpr);
        else
            k_gemv_vec<DT, R, 6, PRO, EPI><<<grid, kGemvThreads, lds, s>>>(a, lpr);
    } else {
        int grid = ceil_div(a.n, kGemvWaves);
        k_gemv_scalar<DT, PRO, EPI><<<grid, kGemvThreads, lds, s>>>(a);
    }
    MR_LAUNCHED("gemv launch");
    return MR_OK;
}

template <int DT>
int launch_gemv_dt(hipStream_t s, int pro, int epi, const GemvArgs &a) {
    if (pro == PRO_COPY) {
        switch (epi) {
            case EPI_STORE: return launch_gemv_t<DT, PRO_COPY, EPI_STORE>(s, a);
            case EPI_RESIDUAL: return launch_gemv_t<DT, PRO_COPY, EPI_RESIDUAL>(s, a);
            case EPI_SWIGLU: return launch_gemv_t<DT, PRO_COPY, EPI_SWIGLU>(s, a);
            case EPI_SCALE_ADD: return launch_gemv_t<DT, PRO_COPY, EPI_SCALE_ADD>(s, a);
            case EPI_GATED: return launch_gemv_t<DT, PRO_COPY, EPI_GATED>(s, a);
            case EPI_GATED_ATTN: return launch_gemv_t<DT, PRO_COPY, EPI_GATED_ATTN>(s, a);
        }
    } else {
        switch (epi) {
            case EPI_STORE: return launch_gemv_t<DT, PRO_RMS, EPI_STORE>(s, a);
            case EPI_RESIDUAL: return launch_gemv_t<DT, PRO_RMS, EPI_RESIDUAL>(s, a);
            case EPI_SWIGLU: return launch_gemv_t<DT, PRO_RMS, EPI_SWIGLU>(s, a);
            case EPI_SCALE_ADD: return launch_gemv_t<DT, PRO_RMS, EPI_SCALE_ADD>(s, a);
        }
    }
    return fail(MR_ERR_INVALID, "gemv: bad prologue/epilogue");
}

// ------------------------------------------------------------------ small GEMM
// 64x64 output tile per 256-thread block, 16-wide k slices through LDS, 4x4
// outputs per thread, FP32 FMA.  For op-level calls with a handful of rows.
template <int DT>
__global__ void __launch_bounds__(256) k_gemm_small(const float *x, const void *w, float *y, int rows, int n,
                                                    int k) {
    __shared__ float xs[16][65];
    __shared__ float ws[16][65];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    float acc[4][4] = {};
    for (int kk = 0; kk < k; kk += 16) {
        for (int i = threadIdx.x; i < 64 * 16; i += 256) {
            int rr = i / 16, cc = i % 16;
            int gr = r0 + rr, gk = kk + cc;
            xs[cc][rr] = (gr < rows && gk < k) ? x[(int64_t)gr * k + gk] : 0.0f;
            int gn = c0 + rr;
            ws[cc][rr] = (gn < n && gk < k) ? load_w<DT>(w, (int64_t)gn * k + gk) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            float xv[4], wv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) { xv[i] = xs[c][ty * 4 + i]; wv[i] = ws[c][tx * 4 + i]; }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(xv[i], wv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int gr = r0 + ty * 4 + i, gn = c0 + tx * 4 + j;
            if (gr < rows && gn < n) y[(int64_t)gr * n + gn] = acc[i][j];
        }
}

}  // namespace

int launch_gemv(hipStream_t s, int dtype, int pro, int epi, const GemvArgs &a) {
    if (a.n <= 0 || a.k <= 0) return fail(MR_ERR_INVALID, "gemv: empty shape");
    switch (dtype) {
        case MR_F32: return launch_gemv_dt<MR_F32>(s, pro, epi, a);
        case MR_BF16: return launch_gemv_dt<MR_BF16>(s, pro, epi, a);
        case MR_F16: return launch_gemv_dt<MR_F16>(s, pro, epi, a);
    }
    return fail(MR_ERR_INVALID, "gemv: unknown weight dtype");
}

int launch_linear(hipStream_t s, const float *x, const void *w, int dtype, float *y, int rows, int n, int k) {
    if (rows <= 0 || n <= 0 || k <= 0) return fail(MR_ERR_INVALID, "linear: empty shape");
    if (rows == 1) {
        GemvArgs a;
        a.w = w; a.x = x; a.y = y; a.n = n; a.k = k;
        return launch_gemv(s, dtype, PRO_COPY, EPI_STORE, a);
    }
    dim3 grid(ceil_div(n, 64), ceil_div(rows, 64));
    switch (dtype) {
        case MR_F32: k_gemm_small<MR_F32><<<grid, 256, 0, s>>>(x, w, y, rows, n, k); break;
        case MR_BF16: k_gemm_small<MR_BF16><<<grid, 256, 0, s>>>(x, w, y, rows, n, k); break;
        case MR_F16: k_gemm_small<MR_F16><<<grid, 256, 0, s>>>(x, w, y, rows, n, k); break;
        default: return fail(MR_ERR_INVALID, "linear: unknown weight dtype");
    }
    MR_LAUNCHED("linear launch");
    return MR_OK;
}

}  // namespace mr
