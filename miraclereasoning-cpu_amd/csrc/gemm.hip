// MFMA GEMM with FP32-faithful term products (batched prefill projections).
//
// Workgroup tile 128 x 128 outputs, k-steps of 32, four waves each owning a
// 64 x 64 quadrant as 4 x 4 tiles of v_mfma_f32_16x16x32_{bf16,f16}.  Each
// k-step the workgroup loads its A rows (FP32) and W rows (BF16/F16/FP32) into
// registers, splits them into terms while writing LDS, and prefetches the next
// k-step's rows while the matrix cores work on this one.
//
// Two term schemes.  BF16 terms: A as hi + mid + lo (three MFMAs against BF16
// weights).  FP16 terms (BF16 weights with a scale, gemm.h): A row r scaled by
// a power of two 2^t_r into FP16 range is hi + lo (11 + 11 significant bits),
// the weights scaled by 2^s are exact in FP16, so two MFMAs per tile step
// carry the product; the epilogue multiplies by 2^-t_r 2^-s (exact).
//
// Operand layout of v_mfma_f32_16x16x32_bf16 (wave64): lane l supplies
// A[l % 16][8 (l / 16) + i] and B[8 (l / 16) + i][l % 16] for i < 8, and holds
// C[4 (l / 16) + j][l % 16] for j < 4.  Both operands are k-contiguous rows
// here (A rows are tokens, B "columns" are weight rows), so each lane reads 16
// bytes of one LDS row.
#include "gemm.h"

#include <algorithm>
#include <cstring>

namespace mr {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 128, kBK = 32;
static_assert(kBM == kGemmRowTile, "the row tiles the grouped GEMM's tile list counts");
constexpr int kPitch = kBK + 8;   // BF16 elements per LDS row (80 bytes: rows stay 16-byte aligned)
constexpr int kThreads = 256;
constexpr int kSwigluNI = 4;   // 16-column MFMA tiles per wave in the SwiGLU FP16-term GEMM
constexpr int kKBH = 64;       // k-step of the register-staged FP16-term GEMM (halves)

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
    return (const char *)base + (int64_t)(ok ? f : 0) * (g.ldw ? g.ldw : g.k) * esize;
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

// x (already scaled into FP16 range) = hi + lo; x - hi is exact in FP32.
__device__ __forceinline__ void split2h(float x, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
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
__device__ __forceinline__ f32x4 mfma(const f16x8 &a, const f16x8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// The epilogue of both schemes: rows m0.., columns n0.. of the tile from the
// accumulators times `unscale` (per output row; 1 for the BF16 scheme).  A
// wave holds NI 16-column tiles; with SwiGLU the first NI / 2 are gate
// columns and the others the up columns of the same FFN columns.  The waves
// of a tile are two rows of WN.
template <int EPI, int NI = 4, int WN = 2, typename Unscale>
__device__ __forceinline__ void gemm_store(const GemmArgs &g, int m0, int n0, const f32x4 (&acc)[4][NI],
                                           Unscale unscale) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN, lr = lane & 15;
    // C[4 (lane / 16) + j][lane % 16] of each 16 x 16 tile
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = m0 + wm * 64 + mi * 16 + (lane >> 4) * 4 + j;
            if (row >= g.m) continue;
            const float u = unscale(row);
            float *crow = g.c + (int64_t)row * g.ldc;
            if constexpr (EPI == GEMM_SWIGLU) {
                const float cs = g.c_hl ? g.c_scale[row] : 1.0f;
                _Float16 *hrow = g.c_hl + (int64_t)row * g.n;
#pragma unroll
                for (int ni = 0; ni < NI / 2; ++ni) {
                    const int f = n0 + wn * 8 * NI + ni * 16 + lr;
                    if (f >= g.n) continue;
                    const float gt = acc[mi][ni][j] * u, up = acc[mi][ni + NI / 2][j] * u;
                    const float v = (gt / (1.0f + expf(-gt))) * up;
                    if (g.c_hl) {
                        _Float16 th, tl;
                        split2h(v * cs, th, tl);
                        hrow[f] = th;
                        hrow[(int64_t)g.m * g.n + f] = tl;
                    } else {
                        crow[f] = v;
                    }
                }
            } else {
#pragma unroll
                for (int ni = 0; ni < NI; ++ni) {
                    const int col = n0 + wn * 16 * NI + ni * 16 + lr;
                    if (col >= g.n) continue;
                    const float v = acc[mi][ni][j] * u;
                    if constexpr (EPI == GEMM_RESIDUAL) crow[col] = crow[col] + g.scale * v;
                    else crow[col] = v;
                }
            }
        }
    }
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

    gemm_store<EPI>(g, m0, n0, acc, [](int) { return 1.0f; });
}

// A's FP16 planes of a k-step of KB halves: per plane 128 rows of KB / 8
// chunks of 16 bytes; thread t holds chunks t + 256 j of each plane (row
// (t + 256 j) / (KB / 8), halves 8 ((t + 256 j) % (KB / 8)) .. + 7).
template <int KB>
struct AHRegs {
    u32x4 v[2][KB / 16];
};

template <int KB>
__device__ __forceinline__ void load_a_h(const GemmArgs &g, int m0, int k0, AHRegs<KB> &r) {
    constexpr int CPR = KB / 8;
    const int tid = threadIdx.x;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int j = 0; j < KB / 16; ++j) {
            const int q = tid + kThreads * j, row = m0 + q / CPR, col = k0 + (q % CPR) * 8;
            const _Float16 *plane = g.ahl + p * (g.plane_stride ? g.plane_stride : (int64_t)g.m * g.k);
            if (row < g.m && col < g.k) r.v[p][j] = *gmem((const u32x4 *)(plane + (int64_t)row * g.k + col));
            else r.v[p][j] = u32x4{0u, 0u, 0u, 0u};
        }
}

template <int KB>
__device__ __forceinline__ void store_a_h(_Float16 (*as)[kBM][KB + 8], const AHRegs<KB> &r) {
    constexpr int CPR = KB / 8;
    const int tid = threadIdx.x;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int j = 0; j < KB / 16; ++j) {
            const int q = tid + kThreads * j;
            *(u32x4 *)&as[p][q / CPR][(q % CPR) * 8] = r.v[p][j];
        }
}

// Weight row r of an FP16-term tile of 32 NI rows: two halves of 16 NI rows
// (one per wave column); with SwiGLU the first 8 NI rows of a half are gate
// rows and the rest the up rows of the same FFN columns.
template <int EPI, int NI>
__device__ __forceinline__ const char *w_row_h(const GemmArgs &g, int n0, int r, bool &ok) {
    int f;
    const void *base = g.w;
    if constexpr (EPI == GEMM_SWIGLU) {
        const int half = r / (16 * NI), q = r % (16 * NI);
        f = n0 + half * 8 * NI + q % (8 * NI);
        if (q >= 8 * NI) base = g.w2;
    } else {
        f = n0 + r;
    }
    ok = f < g.n;
    return (const char *)base + (int64_t)(ok ? f : 0) * g.k * 2;
}

// The FP16 weight rows of a k-step: 32 NI rows of KB / 8 chunks of 16 bytes,
// NI KB / 64 chunks per thread (row q / (KB / 8), halves 8 (q % (KB / 8))).
template <int EPI, int NI, int KB>
__device__ __forceinline__ void load_w_h(const GemmArgs &g, int n0, int k0, u32x4 (&r)[NI * KB / 64]) {
    constexpr int CPR = KB / 8;
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NI * KB / 64; ++i) {
        const int q = tid + kThreads * i;
        const int col = k0 + (q % CPR) * 8;
        bool ok;
        const char *row = w_row_h<EPI, NI>(g, n0, q / CPR, ok);
        if (ok && col < g.k) r[i] = *gmem((const u32x4 *)(row + (int64_t)col * 2));
        else r[i] = u32x4{0u, 0u, 0u, 0u};
    }
}

// Buffer addressing for K a multiple of the k-step and matrices under 2^31
// bytes: a thread's byte offsets into A's planes and the weight rows are
// computed once per tile, a k-step only moves the scalar offset, and a row
// past M or N addresses past its buffer's end, where the bounds check returns
// zeros (no per-load address arithmetic, no 64-bit pointers).
constexpr unsigned kPastEnd = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t half_rsrc(const void *p, int64_t halves) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)(halves * 2), 0x00020000);
}

// One 128 x 32 NI output tile in FP16 terms (BF16 weights, g.wscale > 0, A's
// planes and row scales from k_row_split, the weights' FP16 copy), k-steps
// of KB halves; each wave owns 64 x 16 NI outputs.  The operands pass through
// registers on their way to LDS; gemm_tile_hd below is the form for K a
// multiple of its k-step.
template <int EPI, int NI, int KB>
__device__ __forceinline__ void gemm_tile_h(const GemmArgs &g, int m0, int n0) {
    constexpr int CPR = KB / 8;
    __shared__ __attribute__((aligned(16))) _Float16 as[2][kBM][KB + 8];
    __shared__ __attribute__((aligned(16))) _Float16 bs[32 * NI][KB + 8];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 15, lk = (lane >> 4) * 8;
    const int nk = (g.k + KB - 1) / KB;

    f32x4 acc[4][NI];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

    AHRegs<KB> ar;
    u32x4 wr[NI * KB / 64];
    load_a_h<KB>(g, m0, 0, ar);
    load_w_h<EPI, NI, KB>(g, n0, 0, wr);
    for (int kt = 0; kt < nk; ++kt) {
        if (kt) lds_barrier();   // every wave is done with the previous k-step's LDS
        store_a_h<KB>(as, ar);
#pragma unroll
        for (int i = 0; i < NI * KB / 64; ++i) {
            const int q = tid + kThreads * i;
            *(u32x4 *)&bs[q / CPR][(q % CPR) * 8] = wr[i];
        }
        lds_barrier();
        if (kt + 1 < nk) {
            load_a_h<KB>(g, m0, (kt + 1) * KB, ar);
            load_w_h<EPI, NI, KB>(g, n0, (kt + 1) * KB, wr);
        }
#pragma unroll
        for (int kk = 0; kk < KB / 32; ++kk) {
            f16x8 bf[NI];
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) bf[ni] = *(const f16x8 *)&bs[wn * 16 * NI + ni * 16 + lr][32 * kk + lk];
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) {
                const f16x8 lo = *(const f16x8 *)&as[1][wm * 64 + mi * 16 + lr][32 * kk + lk];
                const f16x8 hi = *(const f16x8 *)&as[0][wm * 64 + mi * 16 + lr][32 * kk + lk];
                // the smaller term first
#pragma unroll
                for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = mfma(lo, bf[ni], acc[mi][ni]);
#pragma unroll
                for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = mfma(hi, bf[ni], acc[mi][ni]);
            }
        }
    }
    const float inv_w = 1.0f / g.wscale;
    gemm_store<EPI, NI>(g, m0, n0, acc, [&](int row) { return (1.0f / g.ascale[row]) * inv_w; });
}

// gemm_tile_h with its operands copied into LDS by the buffer unit
// (buffer_load_dwordx4 ... lds): no register staging and no LDS write
// instructions.  A stage holds A's hi and lo planes and the weight rows of a
// k-step of KB halves, rows unpadded (one copy fills 1 KB in lane order) with
// the 16-byte chunks of a row at swizzled positions, so that the operand reads
// of 16 consecutive rows fall on distinct banks.  S = 1: the next k-step is
// copied once every wave has read the stage (other workgroups on the CU cover
// the copy); S = 2: the copy of k-step kt + 1 runs while the waves compute kt.
// The same MFMAs in the same order as gemm_tile_h, so the same results.
// K a multiple of KB, every operand under 2^31 bytes.  The waves are two
// rows of WN, each with 64 x 16 NI outputs: WN = 2 gives 128 x 32 NI tiles
// of four waves, WN = 4 128 x 64 NI tiles of eight (fewer copied bytes per
// MFMA, since A's two planes serve twice the weight rows).  The kernels use
// KB = 64 with S = 1 where the grid has more tiles than the device has CUs
// (48 KB of LDS and three workgroups per CU, or 64 KB and two for WN = 4)
// and S = 2 where it has no more.  Measured slower on the prefill GEMMs:
// S = 2 on the large grids, KB = 32 with one or two stages, three stages of
// KB = 32 (two workgroups per CU), and 128 x 64 tiles of four waves (four
// workgroups per CU).
template <int KB>
__device__ __forceinline__ constexpr int chunk_swizzle(int r) {
    return KB == 64 ? (r >> 1) & 7 : (r >> 2) & 3;
}

// One copy: 16 bytes a lane from byte voff + so of the buffer into LDS at
// dst + 16 lane.  (Outside a lambda: the host pass of hipcc rejects the
// builtin inside one whose enclosing template is instantiated twice.)
__device__ __forceinline__ void copy_to_lds(__amdgpu_buffer_rsrc_t r, void *dst, unsigned voff, int so) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)dst, 16, voff, so, 0, 0);
}

template <int EPI, int NI, int KB, int S, int WN = 2>
__device__ __forceinline__ void gemm_tile_hd(const GemmArgs &g, int m0, int n0) {
    static_assert(KB == 32 || KB == 64, "k-step");
    constexpr int CPR = KB / 8;                    // 16-byte chunks per row
    constexpr int RPB = 1024 / (KB * 2);           // rows per 1 KB copy
    constexpr int NR = 16 * NI * WN;               // weight rows of a tile
    constexpr int BA = kBM / RPB, BW = NR / RPB;   // copies per A plane, for the weights
    constexpr int NW = 2 * WN;                     // waves: two rows of WN
    constexpr int NB = 2 * BA + BW;                // copies per stage
    static_assert(NB % NW == 0 && (8 * NI) % RPB == 0, "a copy per wave and row run");
    constexpr int NQ = NB / NW;                    // copies per wave per stage
    constexpr int SA = kBM * KB;                   // halves of an A plane in a stage
    __shared__ __attribute__((aligned(16))) _Float16 st[S][2 * SA + NR * KB];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 15, lq = lane >> 4;
    const int nk = g.k / KB;
    const int64_t mk = (int64_t)g.m * g.k, nkw = (int64_t)g.n * g.k;
    const __amdgpu_buffer_rsrc_t ra0 = half_rsrc(g.ahl, mk),
                                 ra1 = half_rsrc(g.ahl + (g.plane_stride ? g.plane_stride : mk), mk);

    // Copy i of this wave fills block b = wave + NW i of a stage: rows
    // RPB b' .. of A's hi plane (b < BA), lo plane (b < 2 BA) or the weights;
    // the lane's 16 bytes land at chunk lane % CPR of its row, so it reads the
    // logical chunk that the swizzle puts there.  Rows past M or N read zeros.
    unsigned voff[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        const int b = wave + NW * i;
        const int rb = (b < 2 * BA ? b % BA : b - 2 * BA) * RPB + lane / CPR;
        const int c = (lane % CPR) ^ chunk_swizzle<KB>(rb);
        if (b < 2 * BA) {
            const int row = m0 + rb;
            voff[i] = row < g.m ? (unsigned)(((int64_t)row * g.k + c * 8) * 2) : kPastEnd;
        } else {
            int f = n0 + rb;
            if constexpr (EPI == GEMM_SWIGLU) f = n0 + (rb / (16 * NI)) * 8 * NI + (rb % (16 * NI)) % (8 * NI);
            voff[i] = f < g.n ? (unsigned)(((int64_t)f * g.k + c * 8) * 2) : kPastEnd;
        }
    }
    // Copy i of a wave lies in A's hi plane for i < BA / NW, its lo plane
    // below 2 BA / NW, the weights above, whatever the wave, so the A buffers
    // are chosen at compile time; a weight copy builds its buffer from a
    // wave-uniform base (gate or up rows).  A choice among descriptors at run
    // time made the compiler loop over its lanes' values for every copy.
    static_assert(BA % NW == 0, "A copies per wave");
    const auto uniform = [](const void *p) {
        const uint64_t v = (uint64_t)p;
        return (const void *)(((uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((unsigned)(v >> 32)) << 32) |
                              (uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((unsigned)v));
    };
    const auto issue = [&](int kt, int stage) {
        const int so = kt * KB * 2;
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const int b = wave + NW * i;
            void *dst = &st[stage][b * 512];
            if (i < BA / NW) {
                copy_to_lds(ra0, dst, voff[i], so);
            } else if (i < 2 * BA / NW) {
                copy_to_lds(ra1, dst, voff[i], so);
            } else {
                const bool up = EPI == GEMM_SWIGLU && ((b - 2 * BA) * RPB) % (16 * NI) >= 8 * NI;
                copy_to_lds(half_rsrc(uniform(up ? g.w2 : g.w), nkw), dst, voff[i], so);
            }
        }
    };

    f32x4 acc[4][NI];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};
    static_assert(S == 1 || S == 2, "stages");
    issue(0, 0);
    int stage = 0;
    for (int kt = 0; kt < nk; ++kt) {
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's copies of k-step kt are in LDS
        lds_barrier();   // every wave's are (S = 2: and every wave is done with the other stage)
        if (S == 2 && kt + 1 < nk) issue(kt + 1, stage ^ 1);
        const _Float16 *ah = &st[stage][0], *al = ah + SA, *ws = ah + 2 * SA;
#pragma unroll
        for (int kk = 0; kk < KB / 32; ++kk) {
            const int c = 4 * kk + lq;
            f16x8 bf[NI];
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) {
                const int r = wn * 16 * NI + ni * 16 + lr;
                bf[ni] = *(const f16x8 *)(ws + r * KB + (c ^ chunk_swizzle<KB>(r)) * 8);
            }
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) {
                const int r = wm * 64 + mi * 16 + lr, off = r * KB + (c ^ chunk_swizzle<KB>(r)) * 8;
                const f16x8 lo = *(const f16x8 *)(al + off);
                const f16x8 hi = *(const f16x8 *)(ah + off);
                // the smaller term first
#pragma unroll
                for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = mfma(lo, bf[ni], acc[mi][ni]);
#pragma unroll
                for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = mfma(hi, bf[ni], acc[mi][ni]);
            }
        }
        if (S == 1 && kt + 1 < nk) {
            lds_barrier();   // every wave has read the stage
            issue(kt + 1, 0);
        }
        stage ^= S - 1;
    }
    const float inv_w = 1.0f / g.wscale;
    gemm_store<EPI, NI, WN>(g, m0, n0, acc, [&](int row) { return (1.0f / g.ascale[row]) * inv_w; });
}

constexpr int kDmaKB = 64, kDmaBlocksPerCU = 3;

// The FP16-term GEMMs take the LDS-copy tile when K is a multiple of its
// k-step and every operand is under 2^31 bytes (the buffer offsets), else
// the tile that loads through registers.
__host__ __device__ inline bool dma_tile_fits(const GemmArgs &g) {
    return g.k % kDmaKB == 0 && (int64_t)g.m * g.k * 2 < (1ll << 31) && (int64_t)g.n * g.k * 2 < (1ll << 31);
}

// Workgroups per CU that S stages of k-steps of KB halves leave room for in
// the CU's 160 KB of LDS (a stage: 2 x 128 A rows + 64 WN weight rows of KB
// halves), at most three.
constexpr int dma_blocks(int kb, int s, int wn) {
    return 160 * 1024 / (s * kb * 2 * (256 + 64 * wn)) < 3 ? 160 * 1024 / (s * kb * 2 * (256 + 64 * wn)) : 3;
}

// The tile (row ty, column tx) a workgroup of a k_gemm_hd grid computes.
// Workgroups go to the 8 XCDs in turn (linear id mod 8), each XCD with its
// own L2; in launch order an XCD takes every eighth column tile of every
// row, which, where a grid is resident at once, shares the weight columns
// but none of A's rows.  Here XCD k takes the k-th contiguous share of an
// order that walks groups of kTileGroup row tiles column by column, so the
// workgroups an XCD runs together share a few A row blocks and a few weight
// column blocks (groups of 4 measured faster than 2, 8 or 16, and than the
// launch order for the multi-round grids too).
constexpr int kTileGroup = 4;
__device__ __forceinline__ void xcd_tile(int &ty, int &tx) {
    const int gx = gridDim.x, gy = gridDim.y, total = gx * gy;
    const int lin = blockIdx.x + gx * blockIdx.y;
    const int k = lin % 8, q = total / 8, r = total % 8;
    const int t = k * q + min(k, r) + lin / 8;   // XCD k: tiles [k q + min(k, r), ...)
    const int grp = t / (kTileGroup * gx), within = t % (kTileGroup * gx);
    const int rows = min(kTileGroup, gy - grp * kTileGroup);
    ty = grp * kTileGroup + within % rows;
    tx = within / rows;
}

template <int EPI, int NI, int KB, int S, int WN>
__global__ void __launch_bounds__(128 * WN, dma_blocks(KB, S, WN)) k_gemm_hd(GemmArgs g) {
    int ty, tx;
    xcd_tile(ty, tx);
    gemm_tile_hd<EPI, NI, KB, S, WN>(g, ty * kBM, tx * (EPI == GEMM_SWIGLU ? 8 : 16) * NI * WN);
}

// Compute units of the current device, queried once per device.
int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    }
    return cus[dev];
}

template <int EPI, int NI>
__global__ void __launch_bounds__(kThreads) k_gemm_h(GemmArgs g) {
    gemm_tile_h<EPI, NI, kKBH>(g, blockIdx.y * kBM, blockIdx.x * (EPI == GEMM_SWIGLU ? 16 * NI : 32 * NI));
}

// A in FP16 terms, once per GEMM: row r's scale 2^t (max_k |a[r][k]| 2^t in
// [2^13, 2^14); 1 for an all-zero or non-finite row) into scale[r], and
// a[r][k] 2^t = hi + lo into planes hl[0][r][k], hl[1][r][k].  One wave per
// row (k a multiple of 4).
__global__ void __launch_bounds__(256) k_row_split(const float *a, int lda, int m, int k, float *scale,
                                                   _Float16 *hl) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= m) return;
    const float *r = a + (int64_t)row * lda;
    float mx = 0.0f;
    for (int c = 4 * lane; c < k; c += 4 * kWave) {
        const float4 v = load_f4(r + c);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    mx = wave_max(mx);
    int e = 0;
    if (mx > 0.0f && mx <= 3.0e38f) {
        frexpf(mx, &e);                     // mx = f 2^e, f in [0.5, 1)
        e = min(max(14 - e, -126), 126);    // mx 2^(14 - e) in [2^13, 2^14)
    }
    const float sc = ldexpf(1.0f, e);
    if (lane == 0) scale[row] = sc;
    _Float16 *hi = hl + (int64_t)row * k, *lo = hl + (int64_t)m * k + (int64_t)row * k;
    for (int c = 4 * lane; c < k; c += 4 * kWave) {
        const float4 v = load_f4(r + c);
        const float x[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};
        f16x4 h, l;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            _Float16 th, tl;
            split2h(x[i], th, tl);
            h[i] = th;
            l[i] = tl;
        }
        *(f16x4 *)(hi + c) = h;
        *(f16x4 *)(lo + c) = l;
    }
}

// k_row_split with the row kept in registers (NV 16-byte vectors per lane,
// k <= 256 NV): every load of the row in flight at once and the row read
// once; the same maximum (an exact operation in any order), scale and planes.
template <int NV>
__global__ void __launch_bounds__(256) k_row_split_reg(const float *a, int lda, int m, int k, float *scale,
                                                       _Float16 *hl) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= m) return;
    const float *r = a + (int64_t)row * lda;
    float4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = 4 * lane + 4 * kWave * i;
        v[i] = c < k ? load_f4(r + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    mx = wave_max(mx);
    int e = 0;
    if (mx > 0.0f && mx <= 3.0e38f) {
        frexpf(mx, &e);                     // mx = f 2^e, f in [0.5, 1)
        e = min(max(14 - e, -126), 126);    // mx 2^(14 - e) in [2^13, 2^14)
    }
    const float sc = ldexpf(1.0f, e);
    if (lane == 0) scale[row] = sc;
    _Float16 *hi = hl + (int64_t)row * k, *lo = hl + (int64_t)m * k + (int64_t)row * k;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = 4 * lane + 4 * kWave * i;
        if (c >= k) break;
        const float x[4] = {v[i].x * sc, v[i].y * sc, v[i].z * sc, v[i].w * sc};
        f16x4 h, l;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            _Float16 th, tl;
            split2h(x[j], th, tl);
            h[j] = th;
            l[j] = tl;
        }
        *(f16x4 *)(hi + c) = h;
        *(f16x4 *)(lo + c) = l;
    }
}

// A's FP16 planes and row scales (k_row_split, or its register form).
void row_split(hipStream_t s, const float *a, int lda, int m, int k, float *scale, _Float16 *hl) {
    if (k <= 4 * kWave * 8) k_row_split_reg<8><<<ceil_div(m, 4), 256, 0, s>>>(a, lda, m, k, scale, hl);
    else if (k <= 4 * kWave * 24) k_row_split_reg<24><<<ceil_div(m, 4), 256, 0, s>>>(a, lda, m, k, scale, hl);
    else k_row_split<<<ceil_div(m, 4), 256, 0, s>>>(a, lda, m, k, scale, hl);
}

__global__ void __launch_bounds__(256) k_bf16_to_f16(const uint16_t *w, int64_t count, float scale, _Float16 *dst) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = (_Float16)(__uint_as_float((unsigned)w[i] << 16) * scale);
}

// max |w| over a BF16 array as the bits of a non-negative float (atomic max
// on the bit patterns, which order like the values).
__global__ void __launch_bounds__(256) k_abs_max_bf16(const uint16_t *w, int64_t count, unsigned *out) {
    unsigned mx = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        mx = max(mx, (unsigned)(w[i] & 0x7fffu) << 16);
    for (int off = 32; off > 0; off >>= 1) mx = max(mx, (unsigned)__shfl_xor((int)mx, off));
    if ((threadIdx.x & 63) == 0) atomicMax(out, mx);
}

// max over rows of the row's L2 norm, one wave per row, as the bits of a
// non-negative float (atomic max on the bit patterns).
__global__ void __launch_bounds__(256) k_row_norm_max_bf16(const uint16_t *w, int64_t rows, int64_t cols,
                                                           unsigned *out) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint16_t *r = w + row * cols;
    float ss = 0.0f;
    for (int64_t c = lane; c < cols; c += kWave) {
        const float v = __uint_as_float((unsigned)r[c] << 16);
        ss += v * v;
    }
    ss = wave_sum(ss);
    if (lane == 0) atomicMax(out, __float_as_uint(sqrtf(ss)));
}

template <int DT, int EPI>
__global__ void __launch_bounds__(kThreads) k_gemm(GemmArgs g) {
    gemm_tile<DT, EPI>(g, blockIdx.y * kBM, blockIdx.x * (EPI == GEMM_SWIGLU ? kBN / 2 : kBN));
}

// grid (column tiles, row tiles, slices): slice z multiplies columns
// z ks .. of A by the same columns of W into its own partial product
// part[z] (STORE epilogue, BF16-term scheme), summed by k_sum_slices.
template <int DT>
__global__ void __launch_bounds__(kThreads) k_gemm_split(GemmArgs g, int ks, float *part) {
    const int z = blockIdx.z, lo = z * ks;
    const int esize = DT == MR_F32 ? 4 : 2;
    g.a += lo;
    g.w = (const char *)g.w + (int64_t)lo * esize;
    g.ldw = g.k;
    g.k = min(ks, g.k - lo);
    g.c = part + (int64_t)z * g.m * g.ldc;
    gemm_tile<DT, GEMM_STORE>(g, blockIdx.y * kBM, blockIdx.x * kBN);
}

// c[r][j] = sum over z of part[z][r][j], slices in order.
__global__ void __launch_bounds__(256) k_sum_slices(const float *part, int slices, int m, int n, int ldp, float *c,
                                                    int ldc) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)m * n) return;
    const int r = (int)(i / n), j = (int)(i % n);
    float v = 0.0f;
    for (int z = 0; z < slices; ++z) v += part[((int64_t)z * m + r) * ldp + j];
    c[(int64_t)r * ldc + j] = v;
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

// The FP16-term form: group z's rows are rows offset[z] .. of the planes and
// row scales split for all g.m rows.
template <int EPI>
__device__ __forceinline__ bool group_args(GemmArgs &g, const GemmGroups &gg, int z, int m0) {
    const int rows = gg.count[z];
    if (m0 >= rows) return false;
    const int64_t first = gg.offset[z];
    g.plane_stride = (int64_t)g.m * g.k;
    g.ahl += first * g.k;
    g.ascale += first;
    g.c += first * g.ldc;
    g.m = rows;
    g.w = gg.wh[z];
    if (EPI == GEMM_SWIGLU) g.w2 = gg.wh2[z];
    g.wscale = gg.wscale[z];
    return true;
}

template <int EPI, int NI>
__global__ void __launch_bounds__(kThreads) k_gemm_grouped_h(GemmArgs g, GemmGroups gg) {
    const int m0 = blockIdx.y * kBM;
    if (!group_args<EPI>(g, gg, blockIdx.z, m0)) return;
    gemm_tile_h<EPI, NI, kKBH>(g, m0, blockIdx.x * (EPI == GEMM_SWIGLU ? 16 * NI : 32 * NI));
}

template <int EPI, int NI>
__global__ void __launch_bounds__(kThreads, kDmaBlocksPerCU) k_gemm_grouped_hd(GemmArgs g, GemmGroups gg) {
    const int m0 = blockIdx.y * kBM;
    if (!group_args<EPI>(g, gg, blockIdx.z, m0)) return;
    gemm_tile_hd<EPI, NI, kDmaKB, 1, 2>(g, m0, blockIdx.x * (EPI == GEMM_SWIGLU ? 16 * NI : 32 * NI));
}

// The same over the groups' own row tiles only: grid (column tiles,
// row_tiles); row tile t belongs to the group z with row_tile_start[z] <= t
// < row_tile_start[z + 1], and those past the last group's end exit.  (The
// launch order, in which an expert's row tiles are neighbours, measured
// faster here than the XCD-aware order of the plain GEMMs.)
constexpr int kMaxTileGroups = 1024;   // groups the tile list's search holds in LDS
// The launcher takes WN = 4, 128 x 256 tiles of eight waves (measured faster
// than 128 x 128 for both the experts' gate/up and down).
template <int EPI, int NI, int WN>
__global__ void __launch_bounds__(128 * WN, dma_blocks(kDmaKB, 1, WN)) k_gemm_grouped_hd_list(GemmArgs g, GemmGroups gg) {
    const int ty = blockIdx.y, tx = blockIdx.x;
    // the prefix sums in LDS with one round of loads, then the search there
    __shared__ int start[kMaxTileGroups + 1];
    for (int i = threadIdx.x; i <= gg.groups; i += 128 * WN) start[i] = gg.row_tile_start[i];
    __syncthreads();
    if (ty >= start[gg.groups]) return;
    int lo = 0, hi = gg.groups - 1;   // the last z with start[z] <= ty
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (start[mid] <= ty) lo = mid;
        else hi = mid - 1;
    }
    const int m0 = (ty - start[lo]) * kBM;
    if (!group_args<EPI>(g, gg, lo, m0)) return;
    gemm_tile_hd<EPI, NI, kDmaKB, 1, WN>(g, m0, tx * (EPI == GEMM_SWIGLU ? 8 : 16) * NI * WN);
}

template <int DT>
int launch_grouped_dt(hipStream_t s, int epi, const GemmArgs &g, const GemmGroups &gg) {
    const int cols = epi == GEMM_SWIGLU ? kBN / 2 : kBN;
    const dim3 grid(ceil_div(g.n, cols), ceil_div(gg.max_rows, kBM), gg.groups);
    if (DT == MR_BF16 && gg.wh) {
        MR_REQUIRE(g.m > 0 && g.ascale && g.ahl_ws && gg.wscale && (epi != GEMM_SWIGLU || gg.wh2),
                   "grouped gemm: FP16 terms need the rows to split, their workspaces and the weights' scales");
        GemmArgs h = g;
        h.ahl = g.ahl_ws;
        if (!g.a_split) row_split(s, g.a, g.lda, g.m, g.k, g.ascale, g.ahl_ws);
        const bool dma = dma_tile_fits(g);
        // the groups' own row tiles where their prefix sums are given
        const bool list = dma && gg.row_tile_start && gg.row_tiles > 0 &&
                          gg.groups <= kMaxTileGroups;
        switch (epi) {
            case GEMM_STORE: {
                const dim3 gs(ceil_div(g.n, 32 * 4), ceil_div(gg.max_rows, kBM), gg.groups);
                const dim3 gl(ceil_div(g.n, 256), gg.row_tiles);
                if (list) k_gemm_grouped_hd_list<GEMM_STORE, 4, 4><<<gl, 512, 0, s>>>(h, gg);
                else if (dma) k_gemm_grouped_hd<GEMM_STORE, 4><<<gs, kThreads, 0, s>>>(h, gg);
                else k_gemm_grouped_h<GEMM_STORE, 4><<<gs, kThreads, 0, s>>>(h, gg);
                break;
            }
            case GEMM_SWIGLU: {
                const dim3 gs(ceil_div(g.n, 16 * kSwigluNI), ceil_div(gg.max_rows, kBM), gg.groups);
                const dim3 gl(ceil_div(g.n, 8 * kSwigluNI * 4), gg.row_tiles);
                if (list) k_gemm_grouped_hd_list<GEMM_SWIGLU, kSwigluNI, 4><<<gl, 512, 0, s>>>(h, gg);
                else if (dma) k_gemm_grouped_hd<GEMM_SWIGLU, kSwigluNI><<<gs, kThreads, 0, s>>>(h, gg);
                else k_gemm_grouped_h<GEMM_SWIGLU, kSwigluNI><<<gs, kThreads, 0, s>>>(h, gg);
                break;
            }
            default: return fail(MR_ERR_INVALID, "grouped gemm: epilogue must be STORE or SWIGLU");
        }
        MR_LAUNCHED("enqueue grouped MFMA GEMM (FP16 terms)");
        return MR_OK;
    }
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
    if (DT == MR_BF16 && g.wscale > 0.0f) {
        GemmArgs h = g;
        h.ahl = g.ahl_ws;
        h.w = g.wh;   // 16-bit rows: the BF16 loaders read them as they are
        h.w2 = g.wh2;
        if (!g.a_split) row_split(s, g.a, g.lda, g.m, g.k, g.ascale, g.ahl_ws);
        // 128 x 128 tiles (wider SwiGLU tiles, 192 or 256 columns, measured
        // slower: the accumulators leave one or two waves per SIMD)
        const bool dma = dma_tile_fits(g);
        const dim3 sgrid(ceil_div(g.n, 16 * kSwigluNI), grid.y);
        const int cus = device_cus();
        // 128 x 256 tiles of eight waves (fewer LDS bytes per MFMA) for the
        // projections whose grid of them still covers every CU; the SwiGLU
        // GEMM's large grids keep three 128 x 128 workgroups per CU
        const bool wide = epi != GEMM_SWIGLU && (int64_t)ceil_div(g.n, 256) * grid.y >= cus;
        const int wn = wide ? 4 : 2;
        const dim3 wgrid(ceil_div(g.n, (epi == GEMM_SWIGLU ? 8 : 16) * 4 * wn), grid.y);
        // A grid of at most one tile per CU leaves no other workgroup to
        // cover a k-step's copy: two LDS stages overlap it with the MFMAs.
        const bool two = (int64_t)wgrid.x * wgrid.y <= cus;
        const int threads = 128 * wn;
#define MR_HD(E, NI_)                                                                                  \
    do {                                                                                               \
        if (wn == 4) {                                                                                 \
            if (two) k_gemm_hd<E, NI_, 64, 2, 4><<<wgrid, threads, 0, s>>>(h);                         \
            else k_gemm_hd<E, NI_, 64, 1, 4><<<wgrid, threads, 0, s>>>(h);                             \
        } else {                                                                                       \
            if (two) k_gemm_hd<E, NI_, 64, 2, 2><<<wgrid, threads, 0, s>>>(h);                         \
            else k_gemm_hd<E, NI_, 64, 1, 2><<<wgrid, threads, 0, s>>>(h);                             \
        }                                                                                              \
    } while (0)
        switch (epi) {
            case GEMM_STORE:
                if (dma) MR_HD(GEMM_STORE, 4);
                else k_gemm_h<GEMM_STORE, 4><<<grid, kThreads, 0, s>>>(h);
                break;
            case GEMM_RESIDUAL:
                if (dma) MR_HD(GEMM_RESIDUAL, 4);
                else k_gemm_h<GEMM_RESIDUAL, 4><<<grid, kThreads, 0, s>>>(h);
                break;
            case GEMM_SWIGLU:
                if (dma) MR_HD(GEMM_SWIGLU, kSwigluNI);
                else k_gemm_h<GEMM_SWIGLU, kSwigluNI><<<sgrid, kThreads, 0, s>>>(h);
                break;
#undef MR_HD
            default: return fail(MR_ERR_INVALID, "gemm: unknown epilogue");
        }
        MR_LAUNCHED("enqueue MFMA GEMM (FP16 terms)");
        return MR_OK;
    }
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

int launch_gemm_split(hipStream_t s, const GemmArgs &g, int slices, float *part) {
    MR_REQUIRE(g.a && g.w && g.c && part && g.m > 0 && g.n > 0 && g.k > 0 && slices >= 1 && g.wscale <= 0.0f,
               "split gemm: bad arguments");
    MR_REQUIRE(g.k % 8 == 0 && g.lda % 4 == 0 && g.lda >= g.k && g.ldc >= g.n && ((uintptr_t)g.a & 15) == 0 &&
                   ((uintptr_t)g.w & 15) == 0,
               "split gemm: k must be a multiple of 8 and rows 16-byte aligned");
    const int ks = ceil_div(ceil_div(g.k, slices), kBK) * kBK;   // whole k-steps per slice
    const int n_slices = ceil_div(g.k, ks);
    GemmArgs h = g;
    h.ldc = g.n;   // partial products are packed rows of n
    const dim3 grid(ceil_div(g.n, kBN), ceil_div(g.m, kBM), n_slices);
    switch (g.dtype) {
        case MR_BF16: k_gemm_split<MR_BF16><<<grid, kThreads, 0, s>>>(h, ks, part); break;
        case MR_F16: k_gemm_split<MR_F16><<<grid, kThreads, 0, s>>>(h, ks, part); break;
        case MR_F32: k_gemm_split<MR_F32><<<grid, kThreads, 0, s>>>(h, ks, part); break;
        default: return fail(MR_ERR_INVALID, "split gemm: unknown weight dtype");
    }
    MR_LAUNCHED("enqueue split MFMA GEMM");
    k_sum_slices<<<(int)(((int64_t)g.m * g.n + 255) / 256), 256, 0, s>>>(part, n_slices, g.m, g.n, g.n, g.c, g.ldc);
    MR_LAUNCHED("enqueue split GEMM sum");
    return MR_OK;
}

int launch_row_split(hipStream_t s, const float *a, int lda, int m, int k, float *scale, _Float16 *planes) {
    MR_REQUIRE(a && scale && planes && m > 0 && k > 0 && k % 4 == 0 && lda % 4 == 0, "row split: bad arguments");
    row_split(s, a, lda, m, k, scale, planes);
    MR_LAUNCHED("enqueue row split");
    return MR_OK;
}

int launch_gemm_grouped(hipStream_t s, int epilogue, const GemmArgs &g, const GemmGroups &gg) {
    MR_REQUIRE(g.a && g.c && g.n > 0 && g.k > 0 && gg.offset && gg.count && gg.w && gg.groups > 0 &&
                   gg.groups <= 65535 && gg.max_rows > 0 && (epilogue != GEMM_SWIGLU || gg.w2) && !g.c_hl,
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

int gemm_f16_weight_scale(hipStream_t s, const void *w, int dtype, int64_t count, float *scale) {
    MR_REQUIRE(scale && (w || count == 0) && count >= 0, "f16 weight scale: bad arguments");
    *scale = 0.0f;
    if (dtype != MR_BF16 || count == 0) return MR_OK;
    unsigned *dev = nullptr;
    MR_HIP(hipMalloc((void **)&dev, sizeof(unsigned)), "f16 weight scale");
    unsigned bits = 0;
    hipError_t e = hipMemsetAsync(dev, 0, sizeof(unsigned), s);
    if (e == hipSuccess) {
        const int64_t blocks = std::min<int64_t>(ceil_div(count, (int64_t)256 * 16), 4096);
        k_abs_max_bf16<<<(int)std::max<int64_t>(blocks, 1), 256, 0, s>>>((const uint16_t *)w, count, dev);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpyAsync(&bits, dev, sizeof(unsigned), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(dev);
    MR_HIP(e, "f16 weight scale");
    float mx;
    memcpy(&mx, &bits, sizeof(mx));
    if (!(mx <= 3.0e38f)) return MR_OK;   // inf or NaN: not eligible
    int ex = 0;
    if (mx > 0.0f) {
        frexpf(mx, &ex);
        ex = std::min(std::max(14 - ex, -126), 126);
    }
    *scale = ldexpf(1.0f, ex);
    return MR_OK;
}

int gemm_row_norm_bound(hipStream_t s, const void *w, int dtype, int64_t rows, int64_t cols, float *norm) {
    MR_REQUIRE(norm && (w || rows * cols == 0) && rows >= 0 && cols >= 0, "row norm bound: bad arguments");
    *norm = 0.0f;
    if (dtype != MR_BF16 || rows == 0 || cols == 0) return MR_OK;
    MR_REQUIRE(ceil_div(rows, (int64_t)4) <= INT32_MAX, "row norm bound: too many rows");
    unsigned *dev = nullptr;
    MR_HIP(hipMalloc((void **)&dev, sizeof(unsigned)), "row norm bound");
    unsigned bits = 0;
    hipError_t e = hipMemsetAsync(dev, 0, sizeof(unsigned), s);
    if (e == hipSuccess) {
        k_row_norm_max_bf16<<<(int)ceil_div(rows, (int64_t)4), 256, 0, s>>>((const uint16_t *)w, rows, cols, dev);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpyAsync(&bits, dev, sizeof(unsigned), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(dev);
    MR_HIP(e, "row norm bound");
    float mx;
    memcpy(&mx, &bits, sizeof(mx));
    if (!(mx <= 1.0e30f)) return MR_OK;   // inf or NaN: no bound
    // the FP32 sums of squares carry a relative error below cols 2^-24
    *norm = mx * (1.0f + 1.0e-3f + (float)cols * 0x1p-24f);
    return MR_OK;
}

int gemm_f16_weight_copy(hipStream_t s, const void *w, int64_t count, float scale, void *dst) {
    MR_REQUIRE(w && dst && count > 0 && scale > 0.0f, "f16 weight copy: bad arguments");
    const int64_t blocks = std::min<int64_t>(ceil_div(count, (int64_t)256 * 8), 8192);
    k_bf16_to_f16<<<(int)blocks, 256, 0, s>>>((const uint16_t *)w, count, scale, (_Float16 *)dst);
    MR_LAUNCHED("enqueue f16 weight copy");
    return MR_OK;
}

int launch_gemm(hipStream_t s, int epilogue, const GemmArgs &g) {
    MR_REQUIRE((g.a || (g.a_split && g.wscale > 0.0f)) && g.w && g.c && g.m > 0 && g.n > 0 && g.k > 0,
               "gemm: bad arguments");
    MR_REQUIRE(epilogue != GEMM_SWIGLU || g.w2, "gemm: SwiGLU needs gate and up weights");
    MR_REQUIRE(g.k % 8 == 0 && g.lda % 4 == 0 && g.lda >= g.k, "gemm: k must be a multiple of 8");
    MR_REQUIRE(((uintptr_t)g.a & 15) == 0 && ((uintptr_t)g.w & 15) == 0 && ((uintptr_t)g.w2 & 15) == 0,
               "gemm: operands must be 16-byte aligned");
    MR_REQUIRE(g.ldc >= g.n, "gemm: output rows too short");
    MR_REQUIRE(g.wscale <= 0.0f || (g.dtype == MR_BF16 && g.ascale && g.ahl_ws && g.wh &&
                                     (epilogue != GEMM_SWIGLU || g.wh2) && ((uintptr_t)g.wh & 15) == 0 &&
                                     ((uintptr_t)g.wh2 & 15) == 0),
               "gemm: FP16 terms need BF16 weights, their FP16 copies and the row-scale and plane workspaces");
    MR_REQUIRE(ceil_div(g.m, kBM) <= 65535, "gemm: too many rows");
    MR_REQUIRE(!g.c_hl || (epilogue == GEMM_SWIGLU && g.wscale > 0.0f && g.c_scale && ((uintptr_t)g.c_hl & 15) == 0),
               "gemm: an output in FP16 terms needs the FP16-term SwiGLU GEMM and its row scales");
    switch (g.dtype) {
        case MR_BF16: return launch_dt<MR_BF16>(s, epilogue, g);
        case MR_F16: return launch_dt<MR_F16>(s, epilogue, g);
        case MR_F32: return launch_dt<MR_F32>(s, epilogue, g);
    }
    return fail(MR_ERR_INVALID, "gemm: unknown weight dtype");
}

}  // namespace mr
