// MFMA GEMM with FP32-faithful BF16 term products (batched prefill projections).
//
// Workgroup tile 128 x 128 outputs, k-steps of 32, four waves each owning a
// 64 x 64 quadrant as 4 x 4 tiles of v_mfma_f32_16x16x32_bf16.  Each k-step the
// workgroup loads its A rows (FP32) and W rows (BF16/F16/FP32) into registers,
// splits them into BF16 terms while writing LDS, and prefetches the next
// k-step's rows while the matrix cores work on this one.
//
// Operand layout of v_mfma_f32_16x16x32_bf16 (wave64): lane l supplies
// A[l % 16][8 (l / 16) + i] and B[8 (l / 16) + i][l % 16] for i < 8, and holds
// C[4 (l / 16) + j][l % 16] for j < 4.  Both operands are k-contiguous rows
// here (A rows are tokens, B "columns" are weight rows), so each lane reads 16
// bytes of one LDS row.
#include "gemm.h"

namespace mr {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 128, kBK = 32;
constexpr int kPitch = kBK + 8;   // BF16 elements per LDS row (80 bytes: rows stay 16-byte aligned)
constexpr int kThreads = 256;

template <int DT>
constexpr int planes() {
    return DT == MR_BF16 ? 1 : DT == MR_F16 ? 2 : 3;
}

// x = hi + mid + lo; every remainder is exact in FP32.
__device__ __forceinline__ void split3(float x, __bf16 &hi, __bf16 &mid, __bf16 &lo) {
    hi = (__bf16)x;
    float r = x - (float)hi;
    mid = (__bf16)r;
    r -= (float)mid;
    lo = (__bf16)r;
}

// One thread's share of a k-step: A rows tid/8 + 32 i, columns 4 (tid % 8)..+3.
struct ARegs {
    float4 v[4];
};

// W share: 16-bit weights as two 8-element chunks (rows idx/4, columns 8 (idx % 4));
// FP32 weights as four float4 (same mapping as A).
template <int DT>
struct WRegs {
    static constexpr int kN = DT == MR_F32 ? 4 : 2;
    u32x4 v[kN];
};

// Weight row r of this workgroup's tile.  For SWIGLU the 128 tile rows are two
// 64-row halves (one per wave column); in each half rows 0..31 are gate rows
// and rows 32..63 the up rows of the same 32 FFN columns.
template <int EPI>
__device__ __forceinline__ const char *w_row(const GemmArgs &g, int n0, int r, int esize, bool &ok) {
    int f;
    const void *base = g.w;
    if constexpr (EPI == GEMM_SWIGLU) {
        const int q = r & 63;
        f = n0 + (r >> 6) * 32 + (q & 31);
        if (q >= 32) base = g.w2;
    } else {
        f = n0 + r;
    }
    ok = f < g.n;
    return (const char *)base + (int64_t)(ok ? f : 0) * g.k * esize;
}

__device__ __forceinline__ void load_a(const GemmArgs &g, int m0, int k0, ARegs &r) {
    const int tid = threadIdx.x;
    const int col = k0 + (tid & 7) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = m0 + (tid >> 3) + 32 * i;
        if (row < g.m && col < g.k) r.v[i] = load_f4(g.a + (int64_t)row * g.lda + col);
        else r.v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

template <int DT, int EPI>
__device__ __forceinline__ void load_w(const GemmArgs &g, int n0, int k0, WRegs<DT> &r) {
    const int tid = threadIdx.x;
    if constexpr (DT == MR_F32) {
        const int col = k0 + (tid & 7) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            bool ok;
            const char *row = w_row<EPI>(g, n0, (tid >> 3) + 32 * i, 4, ok);
            if (ok && col < g.k) r.v[i] = *gmem((const u32x4 *)(row + (int64_t)col * 4));
            else r.v[i] = u32x4{0u, 0u, 0u, 0u};
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + kThreads * i;
            const int col = k0 + (idx & 3) * 8;
            bool ok;
            const char *row = w_row<EPI>(g, n0, idx >> 2, 2, ok);
            if (ok && col < g.k) r.v[i] = *gmem((const u32x4 *)(row + (int64_t)col * 2));
            else r.v[i] = u32x4{0u, 0u, 0u, 0u};
        }
    }
}

__device__ __forceinline__ void store_a(__bf16 (*as)[kBM][kPitch], const ARegs &r) {
    const int tid = threadIdx.x;
    const int col = (tid & 7) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = (tid >> 3) + 32 * i;
        const float x[4] = {r.v[i].x, r.v[i].y, r.v[i].z, r.v[i].w};
        bf16x4 h, m, l;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            __bf16 th, tm, tl;
            split3(x[e], th, tm, tl);
            h[e] = th;
            m[e] = tm;
            l[e] = tl;
        }
        *(bf16x4 *)&as[0][row][col] = h;
        *(bf16x4 *)&as[1][row][col] = m;
        *(bf16x4 *)&as[2][row][col] = l;
    }
}

template <int DT>
__device__ __forceinline__ void store_w(__bf16 (*bs)[kBN][kPitch], const WRegs<DT> &r) {
    const int tid = threadIdx.x;
    if constexpr (DT == MR_BF16) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + kThreads * i;
            *(u32x4 *)&bs[0][idx >> 2][(idx & 3) * 8] = r.v[i];
        }
    } else if constexpr (DT == MR_F16) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + kThreads * i;
            const f16x8 f = __builtin_bit_cast(f16x8, r.v[i]);
            bf16x8 h, l;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = (float)f[e];
                h[e] = (__bf16)x;
                l[e] = (__bf16)(x - (float)h[e]);
            }
            *(bf16x8 *)&bs[0][idx >> 2][(idx & 3) * 8] = h;
            *(bf16x8 *)&bs[1][idx >> 2][(idx & 3) * 8] = l;
        }
    } else {
        const int col = (tid & 7) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = (tid >> 3) + 32 * i;
            const f32x4 v = __builtin_bit_cast(f32x4, r.v[i]);
            const float x[4] = {v[0], v[1], v[2], v[3]};
            bf16x4 h, m, l;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                __bf16 th, tm, tl;
                split3(x[e], th, tm, tl);
                h[e] = th;
                m[e] = tm;
                l[e] = tl;
            }
            *(bf16x4 *)&bs[0][row][col] = h;
            *(bf16x4 *)&bs[1][row][col] = m;
            *(bf16x4 *)&bs[2][row][col] = l;
        }
    }
}

__device__ __forceinline__ f32x4 mfma(const bf16x8 &a, const bf16x8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// One 128 x 128 output tile (rows m0.., columns n0..) of g.
template <int DT, int EPI>
__device__ __forceinline__ void gemm_tile(const GemmArgs &g, int m0, int n0) {
    constexpr int PB = planes<DT>();
    __shared__ __attribute__((aligned(16))) __bf16 as[3][kBM][kPitch];
    __shared__ __attribute__((aligned(16))) __bf16 bs[PB][kBN][kPitch];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 15, lk = (lane >> 4) * 8;
    const int nk = (g.k + kBK - 1) / kBK;

    f32x4 acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

    ARegs ar;
    WRegs<DT> wr;
    load_a(g, m0, 0, ar);
    load_w<DT, EPI>(g, n0, 0, wr);
    for (int kt = 0; kt < nk; ++kt) {
        if (kt) lds_barrier();   // every wave is done with the previous k-step's LDS
        store_a(as, ar);
        store_w<DT>(bs, wr);
        lds_barrier();
        if (kt + 1 < nk) {
            load_a(g, m0, (kt + 1) * kBK, ar);
            load_w<DT, EPI>(g, n0, (kt + 1) * kBK, wr);
        }
        bf16x8 bf[PB][4];
#pragma unroll
        for (int q = 0; q < PB; ++q)
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) bf[q][ni] = *(const bf16x8 *)&bs[q][wn * 64 + ni * 16 + lr][lk];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            bf16x8 af[3];
#pragma unroll
            for (int p = 0; p < 3; ++p) af[p] = *(const bf16x8 *)&as[p][wm * 64 + mi * 16 + lr][lk];
            // term pairs (A order, W order) with orders summing to <= 2, smallest first
            if constexpr (PB >= 3) {
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma(af[0], bf[2][ni], acc[mi][ni]);
            }
            if constexpr (PB >= 2) {
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma(af[1], bf[1][ni], acc[mi][ni]);
            }
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma(af[2], bf[0][ni], acc[mi][ni]);
            if constexpr (PB >= 2) {
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma(af[0], bf[1][ni], acc[mi][ni]);
            }
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma(af[1], bf[0][ni], acc[mi][ni]);
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma(af[0], bf[0][ni], acc[mi][ni]);
        }
    }

    // C[4 (lane / 16) + j][lane % 16] of each 16 x 16 tile
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = m0 + wm * 64 + mi * 16 + (lane >> 4) * 4 + j;
            if (row >= g.m) continue;
            float *crow = g.c + (int64_t)row * g.ldc;
            if constexpr (EPI == GEMM_SWIGLU) {
#pragma unroll
                for (int ni = 0; ni < 2; ++ni) {
                    const int f = n0 + wn * 32 + ni * 16 + lr;
                    if (f >= g.n) continue;
                    const float gt = acc[mi][ni][j], up = acc[mi][ni + 2][j];
                    crow[f] = (gt / (1.0f + expf(-gt))) * up;
                }
            } else {
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) {
                    const int col = n0 + wn * 64 + ni * 16 + lr;
                    if (col >= g.n) continue;
                    if constexpr (EPI == GEMM_RESIDUAL) crow[col] = crow[col] + g.scale * acc[mi][ni][j];
                    else crow[col] = acc[mi][ni][j];
                }
            }
        }
    }
}

template <int DT, int EPI>
__global__ void __launch_bounds__(kThreads) k_gemm(GemmArgs g) {
    gemm_tile<DT, EPI>(g, blockIdx.y * kBM, blockIdx.x * (EPI == GEMM_SWIGLU ? kBN / 2 : kBN));
}

// grid (column tiles, row tiles of the largest group, groups): group z is
// rows offset[z] .. + count[z] of a and c with its own weight rows.
template <int DT, int EPI>
__global__ void __launch_bounds__(kThreads) k_gemm_grouped(GemmArgs g, GemmGroups gg) {
    const int z = blockIdx.z, m0 = blockIdx.y * kBM, rows = gg.count[z];
    if (m0 >= rows) return;
    const int64_t first = gg.offset[z];
    g.a += first * g.lda;
    g.c += first * g.ldc;
    g.m = rows;
    g.w = gg.w[z];
    if (EPI == GEMM_SWIGLU) g.w2 = gg.w2[z];
    gemm_tile<DT, EPI>(g, m0, blockIdx.x * (EPI == GEMM_SWIGLU ? kBN / 2 : kBN));
}

template <int DT>
int launch_grouped_dt(hipStream_t s, int epi, const GemmArgs &g, const GemmGroups &gg) {
    const int cols = epi == GEMM_SWIGLU ? kBN / 2 : kBN;
    const dim3 grid(ceil_div(g.n, cols), ceil_div(gg.max_rows, kBM), gg.groups);
    switch (epi) {
        case GEMM_STORE: k_gemm_grouped<DT, GEMM_STORE><<<grid, kThreads, 0, s>>>(g, gg); break;
        case GEMM_SWIGLU: k_gemm_grouped<DT, GEMM_SWIGLU><<<grid, kThreads, 0, s>>>(g, gg); break;
        default: return fail(MR_ERR_INVALID, "grouped gemm: epilogue must be STORE or SWIGLU");
    }
    MR_LAUNCHED("enqueue grouped MFMA GEMM");
    return MR_OK;
}

template <int DT>
int launch_dt(hipStream_t s, int epi, const GemmArgs &g) {
    const int cols = epi == GEMM_SWIGLU ? kBN / 2 : kBN;
    const dim3 grid(ceil_div(g.n, cols), ceil_div(g.m, kBM));
    switch (epi) {
        case GEMM_STORE: k_gemm<DT, GEMM_STORE><<<grid, kThreads, 0, s>>>(g); break;
        case GEMM_RESIDUAL: k_gemm<DT, GEMM_RESIDUAL><<<grid, kThreads, 0, s>>>(g); break;
        case GEMM_SWIGLU: k_gemm<DT, GEMM_SWIGLU><<<grid, kThreads, 0, s>>>(g); break;
        default: return fail(MR_ERR_INVALID, "gemm: unknown epilogue");
    }
    MR_LAUNCHED("enqueue MFMA GEMM");
    return MR_OK;
}

}  // namespace

int launch_gemm_grouped(hipStream_t s, int epilogue, const GemmArgs &g, const GemmGroups &gg) {
    MR_REQUIRE(g.a && g.c && g.n > 0 && g.k > 0 && gg.offset && gg.count && gg.w && gg.groups > 0 &&
                   gg.groups <= 65535 && gg.max_rows > 0 && (epilogue != GEMM_SWIGLU || gg.w2),
               "grouped gemm: bad arguments");
    MR_REQUIRE(g.k % 8 == 0 && g.lda % 4 == 0 && g.lda >= g.k && g.ldc >= g.n && ((uintptr_t)g.a & 15) == 0,
               "grouped gemm: k must be a multiple of 8 and rows 16-byte aligned");
    MR_REQUIRE(ceil_div(gg.max_rows, kBM) <= 65535, "grouped gemm: too many rows");
    switch (g.dtype) {
        case MR_BF16: return launch_grouped_dt<MR_BF16>(s, epilogue, g, gg);
        case MR_F16: return launch_grouped_dt<MR_F16>(s, epilogue, g, gg);
        case MR_F32: return launch_grouped_dt<MR_F32>(s, epilogue, g, gg);
    }
    return fail(MR_ERR_INVALID, "grouped gemm: unknown weight dtype");
}

int launch_gemm(hipStream_t s, int epilogue, const GemmArgs &g) {
    MR_REQUIRE(g.a && g.w && g.c && g.m > 0 && g.n > 0 && g.k > 0, "gemm: bad arguments");
    MR_REQUIRE(epilogue != GEMM_SWIGLU || g.w2, "gemm: SwiGLU needs gate and up weights");
    MR_REQUIRE(g.k % 8 == 0 && g.lda % 4 == 0 && g.lda >= g.k, "gemm: k must be a multiple of 8");
    MR_REQUIRE(((uintptr_t)g.a & 15) == 0 && ((uintptr_t)g.w & 15) == 0 && ((uintptr_t)g.w2 & 15) == 0,
               "gemm: operands must be 16-byte aligned");
    MR_REQUIRE(g.ldc >= g.n, "gemm: output rows too short");
    MR_REQUIRE(ceil_div(g.m, kBM) <= 65535, "gemm: too many rows");
    switch (g.dtype) {
        case MR_BF16: return launch_dt<MR_BF16>(s, epilogue, g);
        case MR_F16: return launch_dt<MR_F16>(s, epilogue, g);
        case MR_F32: return launch_dt<MR_F32>(s, epilogue, g);
    }
    return fail(MR_ERR_INVALID, "gemm: unknown weight dtype");
}

}  // namespace mr
