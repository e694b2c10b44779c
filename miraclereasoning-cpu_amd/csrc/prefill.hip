// Batched prefill kernels for the GQA families (model.py:95-116, 257-285 over a
// prompt chunk): row RMSNorm, per-head norm + RoPE, causal windowed attention
// on the matrix cores, ring fill, embedding gather.
//
// Attention (k_attn_prefill) works in transposed form so that no operand ever
// changes lanes: with v_mfma_f32_16x16x4f32 (lane l supplies A[l % 16][l / 16]
// and B[l / 16][l % 16], and holds C[4 (l / 16) + j][l % 16]),
//   S^T = K . Q^T     leaves lane l the scores of query l % 16 against keys
//                     4 (l / 16) + j of each 16-key tile;
//   O^T += V^T . P^T  takes exactly those probabilities as its B operand when
//                     k-step s of a 16-key tile covers keys 4 (l / 16) + s,
// and O^T's C layout again gives lane l query l % 16 (dims 4 (l / 16) + j), so
// the running max, sum and rescale of the online softmax are per lane.
#include "prefill.h"

#include <algorithm>

namespace mr {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kKeys = 32;        // keys per LDS tile
constexpr int kAttnThreads = 256;

__device__ __forceinline__ f32x4 mfma4(float a, float b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma16(const f16x8 &a, const f16x8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// x = hi + lo in FP16 (x within FP16 range); x - hi is exact in FP32.
__device__ __forceinline__ void split2h(float x, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

constexpr float kLog2e = 1.4426950408889634f;

// 2^x by the hardware's exp2 (v_exp_f32, about 1 ulp; results below the
// normal range flush to 0, which a softmax weight that small is anyway).
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// The power of two 2^t with mx 2^t in [2^13, 2^14) (1 for 0 or a non-finite mx).
__device__ __forceinline__ float f16_range_scale(float mx) {
    if (!(mx > 0.0f) || !(mx <= 3.0e38f)) return 1.0f;
    int e;
    frexpf(mx, &e);
    return ldexpf(1.0f, min(max(14 - e, -126), 126));
}

// grid (ceil(rows / (64 / gb)), kv_heads * G / gb), 256 threads.  A workgroup
// serves gb query heads of one KV group (gb = 4, 2 or 1) on 64 / gb query
// rows: wave w takes head (w % gb) and rows 16 (w / gb) .. +15.
template <int D>
__global__ void __launch_bounds__(kAttnThreads) k_attn_prefill(PrefillAttnArgs a, int gb) {
    constexpr int NG = D / 16;                                   // 16-dim groups
    constexpr int KP = D + 4;                                    // LDS pitch of key rows (floats)
    constexpr int VP = kKeys + 4;                                // LDS pitch of value columns
    constexpr int NL = (kKeys * (D / 4) + kAttnThreads - 1) / kAttnThreads;   // float4 per thread
    __shared__ __attribute__((aligned(16))) float ks[kKeys * KP];   // ks[key][dim]
    __shared__ __attribute__((aligned(16))) float vt[D * VP];       // vt[dim][key]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lq = lane >> 4;
    const int G = a.heads / a.kv_heads, sub_groups = G / gb, tile_rows = 64 / gb;
    const int kh = blockIdx.y / sub_groups, hsub = blockIdx.y % sub_groups;
    const int t0 = (gridDim.x - 1 - blockIdx.x) * tile_rows;   // latest rows (most keys) first
    const int h = kh * G + hsub * gb + wave % gb;
    const int tq = t0 + (wave / gb) * 16 + lr;                  // this lane's query row
    const bool qvalid = tq < a.rows;
    const int qp = a.p0 + tq;
    const int d = a.d, kvw = a.kv_heads * d, qd = a.heads * d;

    float4 q[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int dim = g * 16 + 4 * lq;
        q[g] = qvalid && dim < d ? load_f4(a.qkv + (int64_t)tq * a.ld + h * d + dim) : make_float4(0.f, 0.f, 0.f, 0.f);
    }

    const int win = a.window ? a.window : a.cap;
    const int last = min(t0 + tile_rows, a.rows) - 1;
    const int klo = max(0, a.p0 + t0 - win + 1), khi = a.p0 + last;
    const int ntiles = (khi - klo) / kKeys + 1;

    float4 kr[NL], vr[NL];
    auto fetch = [&](int kb) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int e = tid + kAttnThreads * i;
            kr[i] = vr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            const int r = e / (D / 4), c = (e % (D / 4)) * 4, kp = kb + r;
            if (e < kKeys * (D / 4) && kp <= khi && c < d) {
                const float *kbase, *vbase;
                if (kp >= a.p0) {
                    kbase = a.qkv + (int64_t)(kp - a.p0) * a.ld + qd + kh * d;
                    vbase = kbase + kvw;
                } else {
                    const int64_t slot = kp % a.cap;
                    kbase = a.ring_k + slot * kvw + kh * d;
                    vbase = a.ring_v + slot * kvw + kh * d;
                }
                kr[i] = load_f4(kbase + c);
                vr[i] = load_f4(vbase + c);
            }
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int e = tid + kAttnThreads * i;
            if (e < kKeys * (D / 4)) {
                const int r = e / (D / 4), c = (e % (D / 4)) * 4;
                *(float4 *)&ks[r * KP + c] = kr[i];
                vt[(c + 0) * VP + r] = vr[i].x;
                vt[(c + 1) * VP + r] = vr[i].y;
                vt[(c + 2) * VP + r] = vr[i].z;
                vt[(c + 3) * VP + r] = vr[i].w;
            }
        }
    };

    float m_run = -INFINITY, l_run = 0.0f;
    f32x4 o[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) o[g] = f32x4{0.f, 0.f, 0.f, 0.f};

    fetch(klo);
    for (int it = 0; it < ntiles; ++it) {
        const int kb = klo + it * kKeys;
        if (it) lds_barrier();
        stash();
        lds_barrier();
        if (it + 1 < ntiles) fetch(kb + kKeys);

        f32x4 sc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            sc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                const float4 kk = *(const float4 *)&ks[(t * 16 + lr) * KP + g * 16 + 4 * lq];
                sc[t] = mfma4(kk.x, q[g].x, sc[t]);
                sc[t] = mfma4(kk.y, q[g].y, sc[t]);
                sc[t] = mfma4(kk.z, q[g].z, sc[t]);
                sc[t] = mfma4(kk.w, q[g].w, sc[t]);
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int kp = kb + t * 16 + 4 * lq + j;
                const bool ok = qvalid && kp <= qp && kp > qp - win && (a.hole == 0 || kp != qp - a.hole);
                const float v = ok ? sc[t][j] * a.inv_root : -INFINITY;
                sc[t][j] = v;
                tmax = fmaxf(tmax, v);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
        const float m_new = fmaxf(m_run, tmax);
        const float m_ref = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = expf(m_run - m_ref);
        float psum = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float p = expf(sc[t][j] - m_ref);
                sc[t][j] = p;
                psum += p;
            }
        psum += __shfl_xor(psum, 16, kWave);
        psum += __shfl_xor(psum, 32, kWave);
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int g = 0; g < NG; ++g) o[g] *= alpha;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                const float4 vv = *(const float4 *)&vt[(g * 16 + lr) * VP + t * 16 + 4 * lq];
                o[g] = mfma4(vv.x, sc[t][0], o[g]);
                o[g] = mfma4(vv.y, sc[t][1], o[g]);
                o[g] = mfma4(vv.z, sc[t][2], o[g]);
                o[g] = mfma4(vv.w, sc[t][3], o[g]);
            }
    }
    if (!qvalid) return;
    float wo = 1.0f, we = 0.0f;   // weights of the window's and the extra columns' partials
    const float *ext = nullptr;
    if (a.ext) {   // the extra partial (m, l, o) joins the softmax
        ext = a.ext + ((int64_t)tq * a.heads + h) * (d + 4);
        const float m_e = ext[0], m = fmaxf(m_run, m_e);
        wo = m_run == -INFINITY ? 0.0f : expf(m_run - m);
        we = m_e == -INFINITY ? 0.0f : expf(m_e - m);
        l_run = l_run * wo + ext[1] * we;
    }
    const float inv = 1.0f / l_run;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int dim = g * 16 + 4 * lq;
        if (dim < d) {
            float4 r = make_float4(o[g][0] * wo, o[g][1] * wo, o[g][2] * wo, o[g][3] * wo);
            if (ext) {
                const float4 e = load_f4(ext + 4 + dim);
                r = make_float4(r.x + e.x * we, r.y + e.y * we, r.z + e.z * we, r.w + e.w * we);
            }
            *(float4 *)(a.out + (int64_t)tq * a.ldo + h * d + dim) = make_float4(r.x * inv, r.y * inv, r.z * inv,
                                                                               r.w * inv);
        }
    }
}

// FP16-term form of k_attn_prefill for d = D in {32, 64, 128}, on
// v_mfma_f32_16x16x32_f16 (lane l supplies A[l % 16][8 (l / 16) + i] and
// B[8 (l / 16) + i][l % 16], i < 8, and holds C[4 (l / 16) + j][l % 16]).
// Every operand is scaled by a power of two into FP16 range and carried as
// hi + lo FP16 terms (11 + 11 significant bits); a product takes the three
// term products hi hi + hi lo + lo hi, and the scales are undone exactly in
// FP32: the queries per row, the keys and the values per 32-key tile (a
// workgroup-wide maximum).  Softmax weights in [0, 1] need no scale.
//   S^T = K . Q^T: A = key rows (16 keys x 32 dims), B = the lane's query
//                  dims, so lane l again holds the scores of query l % 16
//                  against keys 4 (l / 16) + j of each 16-key tile.
//   O^T += V^T . P^T: the 32 keys of a tile enter the contraction in the
//                  order that puts k-slot 8 g + i of lane group g on key
//                  4 g + i (i < 4) or 16 + 4 g + i - 4 (i >= 4), the keys whose
//                  weights the lane already holds; A reads V^T (values stored
//                  transposed in LDS) at those keys.
// Slot of key k (< 32) of a tile in the value contraction: lane group g's
// slots 8 g .. 8 g + 7 hold keys 4 g .. 4 g + 3 and 16 + 4 g .. 16 + 4 g + 3
// (the keys whose weights the group's lanes hold); runs of 4 keys stay runs.
__device__ __forceinline__ int vslot(int k) { return k < 16 ? 8 * (k >> 2) + (k & 3) : 8 * ((k - 16) >> 2) + 4 + (k & 3); }

template <int D>
__global__ void __launch_bounds__(kAttnThreads) k_attn_prefill_h(PrefillAttnArgs a, int gb) {
    constexpr int NC = D / 32;            // 32-dim chunks (QK contraction steps)
    constexpr int ND = D / 16;            // 16-dim output tiles
    constexpr int KP = D + 8;             // LDS pitch of key rows (halves; rows stay 16-byte aligned)
    constexpr int VP = kKeys + 8;         // LDS pitch of transposed value rows (halves)
    constexpr int NL = kKeys * (D / 4) / kAttnThreads;   // float4 of K (and of V) per thread per tile
    static_assert(NL >= 1 && NL <= 4 && kKeys * (D / 4) % kAttnThreads == 0, "tile split");
    __shared__ __attribute__((aligned(16))) _Float16 ks[2][kKeys * KP];   // [term][key][dim]
    __shared__ __attribute__((aligned(16))) _Float16 vt[2][D * VP];       // [term][dim][key]
    __shared__ float tile_max[2][kAttnThreads / kWave];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lq = lane >> 4;
    const int G = a.heads / a.kv_heads, sub_groups = G / gb, tile_rows = 64 / gb;
    const int kh = blockIdx.y / sub_groups, hsub = blockIdx.y % sub_groups;
    const int t0 = (gridDim.x - 1 - blockIdx.x) * tile_rows;   // latest rows (most keys) first
    const int h = kh * G + hsub * gb + wave % gb;
    const int tq = t0 + (wave / gb) * 16 + lr;                  // this lane's query row
    const bool qvalid = tq < a.rows;
    const int qp = a.p0 + tq;
    const int kvw = a.kv_heads * D, qd = a.heads * D;

    // The lane's query dims 32 c + 8 lq .. + 7, scaled by the row's power of
    // two (the row's maximum over the four lane groups that hold it).
    float qf[NC][8];
    float qmax = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        float4 u = make_float4(0.f, 0.f, 0.f, 0.f), v = u;
        if (qvalid) {
            const float *src = a.qkv + (int64_t)tq * a.ld + h * D + 32 * c + 8 * lq;
            u = load_f4(src);
            v = load_f4(src + 4);
        }
        const float t[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            qf[c][i] = t[i];
            qmax = fmaxf(qmax, fabsf(t[i]));
        }
    }
    qmax = fmaxf(qmax, __shfl_xor(qmax, 16, kWave));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32, kWave));
    const float sq = f16_range_scale(qmax);
    f16x8 qh[NC], ql[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            _Float16 th, tl;
            split2h(qf[c][i] * sq, th, tl);
            qh[c][i] = th;
            ql[c][i] = tl;
        }

    const int win = a.window ? a.window : a.cap;
    const int last = min(t0 + tile_rows, a.rows) - 1;
    const int klo = max(0, a.p0 + t0 - win + 1), khi = a.p0 + last;
    const int ntiles = (khi - klo) / kKeys + 1;

    // Thread e loads keys NL kg .. + NL - 1 (kg = e / (D / 4)) at dims c4 .. + 3,
    // and values NL kv .. + NL - 1 (kv = e % (kKeys / NL)) at dims v4 .. + 3:
    // the values go into LDS transposed, and with this mapping the lanes of a
    // write group store whole rows of V^T (the tile's key groups at one dim),
    // where the keys' mapping would put every lane on the same two banks.
    const int kg = tid / (D / 4), c4 = (tid % (D / 4)) * 4;
    const int kv = tid % (kKeys / NL), v4 = (tid / (kKeys / NL)) * 4;
    float4 kr[NL], vr[NL];
    auto fetch = [&](int kb) {
        const int kb_slot = kb < a.p0 ? kb % a.cap : 0;   // ring slot of the tile's first key (uniform)
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            kr[u] = vr[u] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int x = 0; x < 2; ++x) {   // the key row, then the value row
                const int r = NL * (x ? kv : kg) + u, kp = kb + r;
                if (kp <= khi) {
                    const float *base;
                    if (kp >= a.p0) {
                        base = a.qkv + (int64_t)(kp - a.p0) * a.ld + qd + x * kvw + kh * D;
                    } else {
                        int slot = kb_slot + r;
                        while (slot >= a.cap) slot -= a.cap;
                        base = (x ? a.ring_v : a.ring_k) + (int64_t)slot * kvw + kh * D;
                    }
                    if (x) vr[u] = load_f4(base + v4);
                    else kr[u] = load_f4(base + c4);
                }
            }
        }
    };
    // Tile scales (workgroup maxima of |K| and |V|) and the split into LDS.
    auto stash = [&](float &sk, float &sv) {
        float mk = 0.0f, mv = 0.0f;
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            mk = fmaxf(mk, fmaxf(fmaxf(fabsf(kr[u].x), fabsf(kr[u].y)), fmaxf(fabsf(kr[u].z), fabsf(kr[u].w))));
            mv = fmaxf(mv, fmaxf(fmaxf(fabsf(vr[u].x), fabsf(vr[u].y)), fmaxf(fabsf(vr[u].z), fabsf(vr[u].w))));
        }
        mk = wave_max(mk);
        mv = wave_max(mv);
        if (lane == 0) {
            tile_max[0][wave] = mk;
            tile_max[1][wave] = mv;
        }
        lds_barrier();
#pragma unroll
        for (int w = 0; w < kAttnThreads / kWave; ++w) {
            mk = fmaxf(mk, tile_max[0][w]);
            mv = fmaxf(mv, tile_max[1][w]);
        }
        sk = f16_range_scale(mk);
        sv = f16_range_scale(mv);
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            const int r = NL * kg + u;
            const float x[4] = {kr[u].x * sk, kr[u].y * sk, kr[u].z * sk, kr[u].w * sk};
            f16x4 hi, lo;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                _Float16 th, tl;
                split2h(x[i], th, tl);
                hi[i] = th;
                lo[i] = tl;
            }
            *(f16x4 *)&ks[0][r * KP + c4] = hi;
            *(f16x4 *)&ks[1][r * KP + c4] = lo;
        }
        // values transposed: dim v4 + i of keys NL kv .. + NL - 1
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            _Float16 hv[NL], lv[NL];
#pragma unroll
            for (int u = 0; u < NL; ++u) {
                const float x = (i == 0 ? vr[u].x : i == 1 ? vr[u].y : i == 2 ? vr[u].z : vr[u].w) * sv;
                split2h(x, hv[u], lv[u]);
            }
            const int at = (v4 + i) * VP + vslot(NL * kv);   // NL consecutive keys and slots
            if constexpr (NL == 4) {
                *(f16x4 *)&vt[0][at] = f16x4{hv[0], hv[1], hv[2], hv[3]};
                *(f16x4 *)&vt[1][at] = f16x4{lv[0], lv[1], lv[2], lv[3]};
            } else if constexpr (NL == 2) {
                *(f16x2 *)&vt[0][at] = f16x2{hv[0], hv[1]};
                *(f16x2 *)&vt[1][at] = f16x2{lv[0], lv[1]};
            } else {
                vt[0][at] = hv[0];
                vt[1][at] = lv[0];
            }
        }
    };

    float m_run = -INFINITY, l_run = 0.0f;
    f32x4 o[ND];
#pragma unroll
    for (int t = 0; t < ND; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    float sk = 1.0f, sv = 1.0f;
    fetch(klo);
    for (int it = 0; it < ntiles; ++it) {
        const int kb = klo + it * kKeys;
        if (it) lds_barrier();
        stash(sk, sv);
        lds_barrier();
        if (it + 1 < ntiles) fetch(kb + kKeys);

        f32x4 sc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            sc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int off = (t * 16 + lr) * KP + 32 * c + 8 * lq;
                const f16x8 kl = *(const f16x8 *)&ks[1][off];
                const f16x8 khh = *(const f16x8 *)&ks[0][off];
                sc[t] = mfma16(kl, qh[c], sc[t]);
                sc[t] = mfma16(khh, ql[c], sc[t]);
                sc[t] = mfma16(khh, qh[c], sc[t]);
            }
        }
        // scores in base-2 units: e^(s - m) = 2^(s log2 e - m log2 e), with
        // log2 e folded into the unscale product (one rounding, as for s)
        const float unscale = a.inv_root * kLog2e / (sq * sk);
        // a tile inside every row's window (and no hole) needs no mask
        const bool full = a.hole == 0 && kb + kKeys - 1 <= a.p0 + t0 && kb > a.p0 + last - win;
        float tmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float v = sc[t][j] * unscale;
                if (!full) {
                    const int kp = kb + t * 16 + 4 * lq + j;
                    const bool ok = qvalid && kp <= qp && kp > qp - win && (a.hole == 0 || kp != qp - a.hole);
                    v = ok ? v : -INFINITY;
                }
                sc[t][j] = v;
                tmax = fmaxf(tmax, v);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
        const float m_new = fmaxf(m_run, tmax);
        const float m_ref = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = exp2_hw(m_run - m_ref);
        float psum = 0.0f;
        f16x8 ph, pl;   // the lane's 8 weights in contraction order: tile 0's j, then tile 1's j
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float p = exp2_hw(sc[t][j] - m_ref);
                psum += p;
                _Float16 hh, ll;
                split2h(p, hh, ll);
                ph[4 * t + j] = hh;
                pl[4 * t + j] = ll;
            }
        psum += __shfl_xor(psum, 16, kWave);
        psum += __shfl_xor(psum, 32, kWave);
        l_run = l_run * alpha + psum;
        m_run = m_new;
        const float vun = 1.0f / sv;
#pragma unroll
        for (int t = 0; t < ND; ++t) {
            // the lane group's 8 slots, stored in contraction order by the stash
            const int row = (t * 16 + lr) * VP + 8 * lq;
            const f16x8 vh = *(const f16x8 *)&vt[0][row], vl = *(const f16x8 *)&vt[1][row];
            f32x4 pv = mfma16(vl, ph, f32x4{0.f, 0.f, 0.f, 0.f});
            pv = mfma16(vh, pl, pv);
            pv = mfma16(vh, ph, pv);
#pragma unroll
            for (int j = 0; j < 4; ++j) o[t][j] = fmaf(pv[j], vun, o[t][j] * alpha);
        }
    }
    if (!qvalid) return;
    float wo = 1.0f, we = 0.0f;   // weights of the window's and the extra columns' partials
    const float *ext = nullptr;
    if (a.ext) {   // the extra partial (m, l, o; m in natural units) joins the softmax
        ext = a.ext + ((int64_t)tq * a.heads + h) * (D + 4);
        const float m_e = ext[0] * kLog2e, m = fmaxf(m_run, m_e);
        wo = m_run == -INFINITY ? 0.0f : exp2_hw(m_run - m);
        we = m_e == -INFINITY ? 0.0f : exp2_hw(m_e - m);
        l_run = l_run * wo + ext[1] * we;
    }
    const float inv = 1.0f / l_run;
#pragma unroll
    for (int t = 0; t < ND; ++t) {
        const int dim = t * 16 + 4 * lq;
        float4 r = make_float4(o[t][0] * wo, o[t][1] * wo, o[t][2] * wo, o[t][3] * wo);
        if (ext) {
            const float4 e = load_f4(ext + 4 + dim);
            r = make_float4(r.x + e.x * we, r.y + e.y * we, r.z + e.z * we, r.w + e.w * we);
        }
        *(float4 *)(a.out + (int64_t)tq * a.ldo + h * D + dim) = make_float4(r.x * inv, r.y * inv, r.z * inv, r.w * inv);
    }
}

// The chunk's presplit form (the kv16 planes in k_kv_split_tiles' layout):
// the same arithmetic as k_attn_prefill_h with the keys' and values' terms
// and scales fixed for the chunk, and the tiles copied into LDS by the
// buffer unit (buffer_load_dwordx4 ... lds) with no register staging.  Two
// LDS stages: after the barrier that publishes tile it, the copy of tile
// it + 1 runs while the waves compute on tile it.  A stage is
// [K hi | K lo | V^T hi | V^T lo], 32 x D halves each, rows unpadded (one DMA
// instruction fills 1 KB in lane order); the 16-byte chunks of a row sit at
// swizzled positions so that the operand reads of 8 consecutive rows fall on
// distinct banks.
template <int D>
__device__ __forceinline__ int key_swizzle(int r) { return D / 8 >= 8 ? (r & 7) : ((r >> 1) & 3); }
__device__ __forceinline__ int vt_swizzle(int r) { return (r >> 1) & 3; }   // V^T rows: 4 chunks of 8 slots

// 16 bytes a lane from the buffer at voff + soff into LDS at lds + 16 lane
// (lds wave-uniform).
__device__ __forceinline__ void copy_to_lds16(__amdgpu_buffer_rsrc_t rs, void *lds, unsigned voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)lds, 16, voff, soff, 0, 0);
}

template <int D, int R>
__global__ void __launch_bounds__(kAttnThreads) k_attn_prefill_t(PrefillAttnArgs a, int gb, int first) {
    constexpr int NC = D / 32, ND = D / 16;
    constexpr int SUB = kKeys * D;                      // halves per sub-tile
    constexpr int NQ = 4 * SUB * 2 / 1024 / (kAttnThreads / kWave);   // 1 KB copies per wave per tile
    static_assert(NQ >= 1 && (4 * SUB * 2) % (1024 * (kAttnThreads / kWave)) == 0, "stage split");
    __shared__ __attribute__((aligned(16))) _Float16 st[2][4 * SUB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lq = lane >> 4;
    // A wave takes R sets of 16 query rows: every key and value operand read
    // from LDS feeds R products.
    const int G = a.heads / a.kv_heads, sub_groups = G / gb, tile_rows = 64 * R / gb;
    // Workgroups go to the 8 XCDs in turn (linear id mod 8), each XCD with its
    // own L2.  Neighbouring row blocks of a head read the same key tiles a
    // couple of iterations apart, so XCD x takes the x-th eighth of the
    // (head, row block) order, row blocks fastest.
    const int nwg = gridDim.x * gridDim.y, lin = blockIdx.x + gridDim.x * blockIdx.y;
    const int wg = nwg % 8 == 0 ? (lin % 8) * (nwg / 8) + lin / 8 : lin;
    const int rb = wg % gridDim.x, by = wg / gridDim.x;
    const int kh = by / sub_groups, hsub = by % sub_groups;
    const int t0 = (gridDim.x - 1 - rb) * tile_rows;   // latest rows (most keys) first
    const int h = kh * G + hsub * gb + wave % gb;
    int tq[R], qp[R];
    bool qvalid[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        tq[r] = t0 + (wave / gb) * 16 * R + 16 * r + lr;
        qvalid[r] = tq[r] < a.rows;
        qp[r] = a.p0 + tq[r];
    }
    const int kvw = a.kv_heads * D;

    // The lane's query dims 32 c + 8 lq .. + 7 per row set, scaled by the
    // row's power of two.
    f16x8 qh[R][NC], ql[R][NC];
    float sq[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float qf[NC][8];
        float qmax = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            float4 u = make_float4(0.f, 0.f, 0.f, 0.f), v = u;
            if (qvalid[r]) {
                const float *src = a.qkv + (int64_t)tq[r] * a.ld + h * D + 32 * c + 8 * lq;
                u = load_f4(src);
                v = load_f4(src + 4);
            }
            const float t[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                qf[c][i] = t[i];
                qmax = fmaxf(qmax, fabsf(t[i]));
            }
        }
        qmax = fmaxf(qmax, __shfl_xor(qmax, 16, kWave));
        qmax = fmaxf(qmax, __shfl_xor(qmax, 32, kWave));
        sq[r] = f16_range_scale(qmax);
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                _Float16 th, tl;
                split2h(qf[c][i] * sq[r], th, tl);
                qh[r][c][i] = th;
                ql[r][c][i] = tl;
            }
    }

    const int win = a.window ? a.window : a.cap;
    const int last = min(t0 + tile_rows, a.rows) - 1;
    const int klo = max(0, a.p0 + t0 - win + 1), khi = a.p0 + last;
    const int j0 = (klo - first) / kKeys;               // the planes' tiles start at position first
    const int ntiles = (khi - first) / kKeys - j0 + 1;

    // Copy q of a wave (q = wave + 4 i) fills stage chunks 64 q .. 64 q + 63;
    // lane l's chunk f = 64 q + l reads the plane chunk that belongs there.
    // Byte offsets within tile 0; tile j adds j * 32 kvw * 2 (a K tile is 32
    // rows of kvw halves, a V^T tile the kv heads' [dim][slot] blocks).
    const unsigned plane = (unsigned)a.kv16_rows * (unsigned)kvw * 2u;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)a.kv16, (short)0, (int)(4u * plane), 0x00020000);
    unsigned voff[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        const int f = (wave + 4 * i) * kWave + lane, sub = f / (SUB / 8), idx = f % (SUB / 8);
        if (sub < 2) {
            const int r = idx / (D / 8), pos = idx % (D / 8);
            voff[i] = sub * plane + (unsigned)((r * kvw + kh * D) * 2 + (pos ^ key_swizzle<D>(r)) * 16);
        } else {
            const int r = idx / 4, pos = idx % 4;
            voff[i] = sub * plane + (unsigned)(kh * D * kKeys * 2 + r * kKeys * 2 + (pos ^ vt_swizzle(r)) * 16);
        }
    }
    auto issue = [&](int j, int stage) {
        const int soff = j * kKeys * kvw * 2;
#pragma unroll
        for (int i = 0; i < NQ; ++i) copy_to_lds16(rs, &st[stage][(wave + 4 * i) * 512], voff[i], soff);
    };
    // the lane's operand chunks (half offsets within a stage)
    int koff[2][NC], voffl[ND];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int r = t * 16 + lr;
            koff[t][c] = r * D + ((4 * c + lq) ^ key_swizzle<D>(r)) * 8;
        }
#pragma unroll
    for (int t = 0; t < ND; ++t) {
        const int r = t * 16 + lr;
        voffl[t] = 2 * SUB + r * kKeys + (lq ^ vt_swizzle(r)) * 8;
    }

    float m_run[R], l_run[R], unscale[R];
    f32x4 o[R][ND];
    const float sk = a.kv16_scale[kh], sv = a.kv16_scale[a.kv_heads + kh];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        m_run[r] = -INFINITY;
        l_run[r] = 0.0f;
        unscale[r] = a.inv_root * kLog2e / (sq[r] * sk);
#pragma unroll
        for (int t = 0; t < ND; ++t) o[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    issue(j0, 0);
    for (int it = 0; it < ntiles; ++it) {
        const int kb = first + (j0 + it) * kKeys;
        const _Float16 *cur = st[it & 1];
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's copies of tile it are in LDS
        lds_barrier();                          // every wave's are; stage (it + 1) & 1 is read
        if (it + 1 < ntiles) issue(j0 + it + 1, (it + 1) & 1);

        f32x4 sc[R][2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < R; ++r) sc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const f16x8 kl = *(const f16x8 *)&cur[SUB + koff[t][c]];
                const f16x8 khh = *(const f16x8 *)&cur[koff[t][c]];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    sc[r][t] = mfma16(kl, qh[r][c], sc[r][t]);
                    sc[r][t] = mfma16(khh, ql[r][c], sc[r][t]);
                    sc[r][t] = mfma16(khh, qh[r][c], sc[r][t]);
                }
            }
        }
        const bool full = a.hole == 0 && kb + kKeys - 1 <= a.p0 + t0 && kb > a.p0 + last - win;
        f16x8 ph[R], pl[R];
        bool moved = false;
        float alpha[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float tmax = -INFINITY;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float v = sc[r][t][j] * unscale[r];
                    if (!full) {
                        const int kp = kb + t * 16 + 4 * lq + j;
                        const bool ok = qvalid[r] & (kp <= qp[r]) & (kp > qp[r] - win) &
                                        ((a.hole == 0) | (kp != qp[r] - a.hole));
                        v = ok ? v : -INFINITY;
                    }
                    sc[r][t][j] = v;
                    tmax = fmaxf(tmax, v);
                }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
            const float m_new = fmaxf(m_run[r], tmax);
            const float m_ref = m_new == -INFINITY ? 0.0f : m_new;
            alpha[r] = exp2_hw(m_run[r] - m_ref);
            moved |= alpha[r] != 1.0f;
            float psum = 0.0f;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float p = exp2_hw(sc[r][t][j] - m_ref);
                    psum += p;
                    _Float16 hh, ll;
                    split2h(p, hh, ll);
                    ph[r][4 * t + j] = hh;
                    pl[r][4 * t + j] = ll;
                }
            psum += __shfl_xor(psum, 16, kWave);
            psum += __shfl_xor(psum, 32, kWave);
            l_run[r] = l_run[r] * alpha[r] + psum;
            m_run[r] = m_new;
        }
        // o * 1 is o: the rescale only runs while some row's maximum moves
        if (__any(moved)) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int t = 0; t < ND; ++t) o[r][t] *= alpha[r];
        }
#pragma unroll
        for (int t = 0; t < ND; ++t) {
            const f16x8 vh = *(const f16x8 *)&cur[voffl[t]], vl = *(const f16x8 *)&cur[SUB + voffl[t]];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                o[r][t] = mfma16(vl, ph[r], o[r][t]);
                o[r][t] = mfma16(vh, pl[r], o[r][t]);
                o[r][t] = mfma16(vh, ph[r], o[r][t]);
            }
        }
    }
    const float vun = 1.0f / sv;
    float so = 1.0f;   // out_hl: the rows' scale, from every KV head's max |v|
    if (a.out_hl) {
        unsigned mb = 0;
        for (int kh = 0; kh < a.kv_heads; ++kh) mb = max(mb, a.kv16_max[a.kv_heads + kh]);
        so = f16_range_scale(__uint_as_float(mb));
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (!qvalid[r]) continue;
        float wo = 1.0f, we = 0.0f;
        const float *ext = nullptr;
        float l = l_run[r];
        if (a.ext) {   // the extra partial (m, l, o; m in natural units) joins the softmax
            ext = a.ext + ((int64_t)tq[r] * a.heads + h) * (D + 4);
            const float m_e = ext[0] * kLog2e, m = fmaxf(m_run[r], m_e);
            wo = m_run[r] == -INFINITY ? 0.0f : exp2_hw(m_run[r] - m);
            we = m_e == -INFINITY ? 0.0f : exp2_hw(m_e - m);
            l = l * wo + ext[1] * we;
        }
        const float inv = 1.0f / l;
#pragma unroll
        for (int t = 0; t < ND; ++t) {
            const int dim = t * 16 + 4 * lq;
            const f32x4 ov = o[r][t] * vun;
            float4 x = make_float4(ov[0] * wo, ov[1] * wo, ov[2] * wo, ov[3] * wo);
            if (ext) {
                const float4 e = load_f4(ext + 4 + dim);
                x = make_float4(x.x + e.x * we, x.y + e.y * we, x.z + e.z * we, x.w + e.w * we);
            }
            const float y[4] = {x.x * inv, x.y * inv, x.z * inv, x.w * inv};
            if (a.out_hl) {
                f16x4 hh, hl;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    _Float16 th, tl;
                    split2h(y[i] * so, th, tl);
                    hh[i] = th;
                    hl[i] = tl;
                }
                _Float16 *po = a.out_hl + (int64_t)tq[r] * a.ldo + h * D + dim;
                *(f16x4 *)po = hh;
                *(f16x4 *)(po + (int64_t)a.rows * a.ldo) = hl;
                if (h == 0 && t == 0 && lq == 0) a.out_scale[tq[r]] = so;
            } else {
                *(float4 *)(a.out + (int64_t)tq[r] * a.ldo + h * D + dim) = make_float4(y[0], y[1], y[2], y[3]);
            }
        }
    }
}

// The keys and values of positions first .. first + n - 1 (ring slot p % cap
// before p0, chunk row p - p0 after): per-KV-head maxima of |K| and |V| into
// mx[2][kv_heads] (bit patterns of non-negative floats, which order like the
// values; zeroed before).  A block takes kMaxRows positions, a thread 4 dims,
// their loads in flight kMaxBatch positions at a time (positions past the
// range read the last one again, which leaves a maximum as it is; more blocks
// with fewer positions measured slower, their atomics queueing on the same
// words); the D / 4 threads of a head combine their maxima before one atomic
// each.
constexpr int kMaxRows = kKvMaxRows;
constexpr int kMaxBatch = 8;

__global__ void k_kv_max(PrefillAttnArgs a, int first, int n) {
    const int kvw = a.kv_heads * a.d, qd = a.heads * a.d, c4 = 4 * threadIdx.x;
    const bool on = c4 < kvw;
    float mk = 0.0f, mv = 0.0f;
    for (int i0 = 0; i0 < kMaxRows && on; i0 += kMaxBatch) {
        if (first + (int)blockIdx.x * kMaxRows + i0 >= first + n) break;
        float4 x[kMaxBatch], y[kMaxBatch];
#pragma unroll
        for (int i = 0; i < kMaxBatch; ++i) {
            const int p = min(first + (int)blockIdx.x * kMaxRows + i0 + i, first + n - 1);
            const float *k = p >= a.p0 ? a.qkv + (int64_t)(p - a.p0) * a.ld + qd : a.ring_k + (int64_t)(p % a.cap) * kvw;
            const float *v = p >= a.p0 ? k + kvw : a.ring_v + (int64_t)(p % a.cap) * kvw;
            x[i] = load_f4(k + c4);
            y[i] = load_f4(v + c4);
        }
#pragma unroll
        for (int i = 0; i < kMaxBatch; ++i) {
            mk = fmaxf(mk, fmaxf(fmaxf(fabsf(x[i].x), fabsf(x[i].y)), fmaxf(fabsf(x[i].z), fabsf(x[i].w))));
            mv = fmaxf(mv, fmaxf(fmaxf(fabsf(y[i].x), fabsf(y[i].y)), fmaxf(fabsf(y[i].z), fabsf(y[i].w))));
        }
    }
    // the head's threads are a run of D / 4 <= 32 lanes starting at a multiple of D / 4
    for (int off = 1; off < a.d / 4; off <<= 1) {
        mk = fmaxf(mk, __shfl_xor(mk, off, kWave));
        mv = fmaxf(mv, __shfl_xor(mv, off, kWave));
    }
    if (on && c4 % a.d == 0) {
        const int head = c4 / a.d;
        if (a.kv_part) {   // this block's maxima, reduced by k_kv_split_tiles
            unsigned *part = a.kv_part + (size_t)blockIdx.x * 2 * a.kv_heads;
            part[head] = __float_as_uint(mk);
            part[a.kv_heads + head] = __float_as_uint(mv);
        } else {
            atomicMax(a.kv16_max + head, __float_as_uint(mk));
            atomicMax(a.kv16_max + a.kv_heads + head, __float_as_uint(mv));
        }
    }
}

// The same positions split into FP16 terms with the per-head scales, as the
// kv16 planes [K hi, K lo, V hi, V lo] in 32-row tiles from position first
// (kv16_rows x kv_heads d halves each): a K tile is its 32 rows as they are;
// a V tile holds each KV head's block transposed, [head][dim][slot], the key
// at row k of the tile in slot vslot(k).  Rows at first + n and beyond are
// zeros.  Grid (tiles, kv_heads), 256 threads; block (0, head) also stores
// the head's scales for the attention kernel.
template <int D>
__global__ void __launch_bounds__(256) k_kv_split_tiles(PrefillAttnArgs a, int first, int n) {
    constexpr int PER = kKeys * D / 4 / 256;   // float4 of K (and of V) per thread
    static_assert(PER >= 1 && kKeys * D / 4 % 256 == 0, "tile split");
    __shared__ __attribute__((aligned(16))) _Float16 vt[2][D * kKeys];
    const int kvw = a.kv_heads * D, qd = a.heads * D, head = blockIdx.y, j = blockIdx.x;
    unsigned mk, mv;
    if (a.kv_part) {   // the head's maxima over k_kv_max's blocks (an exact operation in any order)
        __shared__ unsigned red[2][256 / kWave];
        mk = 0;
        mv = 0;
        const unsigned *part = a.kv_part;
        for (int b = threadIdx.x, nb = prefill_kv_max_blocks(n); b < nb; b += 256) {
            mk = max(mk, part[(size_t)b * 2 * a.kv_heads + head]);
            mv = max(mv, part[(size_t)b * 2 * a.kv_heads + a.kv_heads + head]);
        }
        for (int off = 32; off > 0; off >>= 1) {
            mk = max(mk, (unsigned)__shfl_xor((int)mk, off));
            mv = max(mv, (unsigned)__shfl_xor((int)mv, off));
        }
        if ((threadIdx.x & 63) == 0) {
            red[0][threadIdx.x >> 6] = mk;
            red[1][threadIdx.x >> 6] = mv;
        }
        __syncthreads();
        mk = max(max(red[0][0], red[0][1]), max(red[0][2], red[0][3]));
        mv = max(max(red[1][0], red[1][1]), max(red[1][2], red[1][3]));
        if (j == 0 && threadIdx.x == 0) {   // for the attention's FP16-term output
            a.kv16_max[head] = mk;
            a.kv16_max[a.kv_heads + head] = mv;
        }
    } else {
        mk = a.kv16_max[head];
        mv = a.kv16_max[a.kv_heads + head];
    }
    const float sk = f16_range_scale(__uint_as_float(mk));
    const float sv = f16_range_scale(__uint_as_float(mv));
    if (j == 0 && threadIdx.x == 0) {
        a.kv16_scale[head] = sk;
        a.kv16_scale[a.kv_heads + head] = sv;
    }
    const int64_t plane = (int64_t)a.kv16_rows * kvw;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int e = threadIdx.x + 256 * u, r = e / (D / 4), c4 = (e % (D / 4)) * 4;
        const int p = first + j * kKeys + r;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f), y = x;
        if (p < first + n) {
            const float *k = p >= a.p0 ? a.qkv + (int64_t)(p - a.p0) * a.ld + qd : a.ring_k + (int64_t)(p % a.cap) * kvw;
            const float *v = p >= a.p0 ? k + kvw : a.ring_v + (int64_t)(p % a.cap) * kvw;
            x = load_f4(k + head * D + c4);
            y = load_f4(v + head * D + c4);
        }
        const float xs[4] = {x.x * sk, x.y * sk, x.z * sk, x.w * sk}, ys[4] = {y.x * sv, y.y * sv, y.z * sv, y.w * sv};
        f16x4 kh4, kl4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            _Float16 hi, lo;
            split2h(xs[i], hi, lo);
            kh4[i] = hi;
            kl4[i] = lo;
            split2h(ys[i], hi, lo);
            vt[0][(c4 + i) * kKeys + vslot(r)] = hi;
            vt[1][(c4 + i) * kKeys + vslot(r)] = lo;
        }
        const int64_t at = (int64_t)(j * kKeys + r) * kvw + head * D + c4;
        *(f16x4 *)(a.kv16 + at) = kh4;
        *(f16x4 *)(a.kv16 + plane + at) = kl4;
    }
    __syncthreads();
    constexpr int CH = D * kKeys / 8;   // 16-byte chunks of a V^T block
    const int64_t vbase = (int64_t)j * kKeys * kvw + (int64_t)head * D * kKeys;
    for (int e = threadIdx.x; e < 2 * CH; e += 256) {
        const int t = e / CH, c = e % CH;
        *(f16x8 *)(a.kv16 + (2 + t) * plane + vbase + c * 8) = *(const f16x8 *)&vt[t][c * 8];
    }
}

__global__ void __launch_bounds__(256) k_rms_rows(const float *x, int ldx, const float *gain, float eps, int width,
                                                  float *y, int ldy) {
    __shared__ float red[4];
    const float *xr = x + (int64_t)blockIdx.x * ldx;
    float *yr = y + (int64_t)blockIdx.x * ldy;
    float ss = 0.0f;
    for (int j = threadIdx.x; j < width; j += blockDim.x) ss += xr[j] * xr[j];
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)width + eps);
    for (int j = threadIdx.x; j < width; j += blockDim.x) yr[j] = xr[j] * scale * (gain ? gain[j] : 1.0f);
}

// k_rms_rows feeding an FP16-term GEMM directly: y = RMSNorm(x) gain (the
// same arithmetic), then y's row scale 2^t (max |y| 2^t in [2^13, 2^14)) into
// scale[row] and y 2^t = hi + lo into planes hl[0][row][.], hl[1][row][.]
// (rows of `width` halves; `rows` planes apart), as the GEMM's own split
// would write them.
// A thread holds up to kSplitChunks runs of 8 values of its row in registers
// (width a multiple of 8, at most 256 * 8 * kSplitChunks) through the three
// passes (sum of squares, maximum, split) and stores 8 halves at a time.
constexpr int kSplitChunks = 4;

__global__ void __launch_bounds__(256) k_rms_rows_split(const float *x, int ldx, const float *gain, float eps,
                                                        int width, float *scale, _Float16 *hl, int rows) {
    __shared__ float red[4];
    const float *xr = x + (int64_t)blockIdx.x * ldx;
    const int runs = width / 8;
    float4 v[kSplitChunks][2];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < kSplitChunks; ++c) {
        const int r = threadIdx.x + c * blockDim.x;
        v[c][0] = v[c][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < runs) {
            v[c][0] = load_f4(xr + 8 * r);
            v[c][1] = load_f4(xr + 8 * r + 4);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
            ss += v[c][t].x * v[c][t].x + v[c][t].y * v[c][t].y + v[c][t].z * v[c][t].z + v[c][t].w * v[c][t].w;
    }
    ss = block_sum(ss, red);
    const float rs = 1.0f / sqrtf(ss / (float)width + eps);
    float mx = 0.0f;
#pragma unroll
    for (int c = 0; c < kSplitChunks; ++c) {
        const int r = threadIdx.x + c * blockDim.x;
        if (r >= runs) continue;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const float4 g = gain ? load_f4(gain + 8 * r + 4 * t) : make_float4(1.f, 1.f, 1.f, 1.f);
            v[c][t] = make_float4(v[c][t].x * rs * g.x, v[c][t].y * rs * g.y, v[c][t].z * rs * g.z,
                                  v[c][t].w * rs * g.w);
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[c][t].x), fabsf(v[c][t].y)), fmaxf(fabsf(v[c][t].z), fabsf(v[c][t].w))));
        }
    }
    mx = block_max(mx, red);
    const float sc = f16_range_scale(mx);
    if (threadIdx.x == 0) scale[blockIdx.x] = sc;
    _Float16 *hi = hl + (int64_t)blockIdx.x * width, *lo = hl + (int64_t)rows * width + (int64_t)blockIdx.x * width;
#pragma unroll
    for (int c = 0; c < kSplitChunks; ++c) {
        const int r = threadIdx.x + c * blockDim.x;
        if (r >= runs) continue;
        const float y[8] = {v[c][0].x, v[c][0].y, v[c][0].z, v[c][0].w, v[c][1].x, v[c][1].y, v[c][1].z, v[c][1].w};
        f16x8 h, l;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            _Float16 th, tl;
            split2h(y[i] * sc, th, tl);
            h[i] = th;
            l[i] = tl;
        }
        *(f16x8 *)(hi + 8 * r) = h;
        *(f16x8 *)(lo + 8 * r) = l;
    }
}

// grid (rows, ceil((heads + kv_heads) / 4)), 256 threads: one wave per head.
__global__ void __launch_bounds__(256) k_qk_rows(float *qkv, int ld, int p0, int heads, int kv_heads, int d,
                                                 const float *q_gain, const float *k_gain, float eps, int norm,
                                                 const float *rope, int split_half, const int *positions) {
    const int lane = threadIdx.x & 63, hh = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (hh >= heads + kv_heads) return;
    float *row = qkv + (int64_t)blockIdx.x * ld + (int64_t)hh * d;   // k heads follow the q heads
    const float *gain = hh < heads ? q_gain : k_gain;
    float scale = 1.0f;
    if (norm) {
        float ss = 0.0f;
        for (int j = lane; j < d; j += kWave) ss += row[j] * row[j];
        scale = 1.0f / sqrtf(wave_sum(ss) / (float)d + eps);
    }
    const int half = d / 2;
    const int p = positions ? positions[blockIdx.x] : p0 + (int)blockIdx.x;
    const float *cs = rope + (int64_t)p * half * 2;
    for (int i = lane; i < half; i += kWave) {
        const int j = split_half ? i : 2 * i, k = split_half ? i + half : 2 * i + 1;
        float u = row[j], v = row[k];
        if (norm) {
            u = u * scale * (gain ? gain[j] : 1.0f);
            v = v * scale * (gain ? gain[k] : 1.0f);
        }
        rope_rotate(u, v, cs[2 * i], cs[2 * i + 1]);
        row[j] = u;
        row[k] = v;
    }
}

// k_qk_rows for head dims up to 128 with R rows per wave: every load of the
// R rows (the pair of lane l, the norm's elements l and l + 64, the RoPE row)
// in flight before any arithmetic, then each row exactly as k_qk_rows takes it.
template <int R>
__global__ void __launch_bounds__(256) k_qk_rows_r(float *qkv, int ld, int p0, int heads, int kv_heads, int d,
                                                   const float *q_gain, const float *k_gain, float eps, int norm,
                                                   const float *rope, int split_half, const int *positions,
                                                   int rows) {
    const int lane = threadIdx.x & 63, hh = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (hh >= heads + kv_heads) return;
    const float *gain = hh < heads ? q_gain : k_gain;
    const int half = d / 2;
    const bool pair = lane < half;
    const int j = split_half ? lane : 2 * lane, k = split_half ? lane + half : 2 * lane + 1;
    float u[R], v[R], c[R], sn[R], x0[R], x1[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = blockIdx.x * R + r;
        const bool live = row < rows;
        const float *rp = qkv + (int64_t)(live ? row : 0) * ld + (int64_t)hh * d;
        const int p = positions ? positions[live ? row : 0] : p0 + row;
        const float *cs = rope + ((int64_t)p * half + lane) * 2;
        u[r] = live && pair ? rp[j] : 0.0f;
        v[r] = live && pair ? rp[k] : 0.0f;
        c[r] = live && pair ? cs[0] : 1.0f;
        sn[r] = live && pair ? cs[1] : 0.0f;
        x0[r] = norm && live && lane < d ? rp[lane] : 0.0f;
        x1[r] = norm && live && lane + kWave < d ? rp[lane + kWave] : 0.0f;
    }
    const float gj = norm && gain && pair ? gain[j] : 1.0f, gk = norm && gain && pair ? gain[k] : 1.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = blockIdx.x * R + r;
        float scale = 1.0f;
        if (norm) {
            float ss = 0.0f;
            if (lane < d) ss += x0[r] * x0[r];
            if (lane + kWave < d) ss += x1[r] * x1[r];
            scale = 1.0f / sqrtf(wave_sum(ss) / (float)d + eps);
        }
        if (row >= rows || !pair) continue;
        float a = u[r], b = v[r];
        if (norm) {
            a = a * scale * gj;
            b = b * scale * gk;
        }
        rope_rotate(a, b, c[r], sn[r]);
        float *rp = qkv + (int64_t)row * ld + (int64_t)hh * d;
        rp[j] = a;
        rp[k] = b;
    }
}

__global__ void k_ring_store(const float *qkv, int ld, int qd, int kvw, float *ring_k, float *ring_v, int cap,
                             int first, int p0) {
    const int p = first + blockIdx.x;
    const float4 *src = (const float4 *)(qkv + (int64_t)(p - p0) * ld + qd);
    const int64_t slot = p % cap;
    float4 *dk = (float4 *)(ring_k + slot * kvw), *dv = (float4 *)(ring_v + slot * kvw);
    const int n4 = kvw / 4;   // 16-byte copies (ld, qd and kvw multiples of 4)
    for (int j = threadIdx.x; j < n4; j += blockDim.x) {
        dk[j] = src[j];
        dv[j] = src[n4 + j];
    }
}

__global__ void k_embed_rows(const void *table, int dt, const int *ids, int p0, float *x, int h) {
    const int64_t base = (int64_t)ids[p0 + blockIdx.x] * h;
    float *xr = x + (int64_t)blockIdx.x * h;
    for (int j = threadIdx.x; j < h; j += blockDim.x) {
        if (dt == MR_F32) xr[j] = ((const float *)table)[base + j];
        else if (dt == MR_BF16) xr[j] = bf16_to_f32(((const uint16_t *)table)[base + j]);
        else xr[j] = f16_to_f32(((const uint16_t *)table)[base + j]);
    }
}

// The relay columns of flashnano-1.6 (attention's extra keys, model.py:104-110)
// as a partial per row and query head, for the attention's ext input: row t
// (position p0 + t) sees the first (position / chunk) * slots relay rows, those
// of the chunks completed before it; m = the largest score (natural units),
// l = sum of exp(score - m), o = the exp-weighted sum of values (no relay
// row: m = -inf, l = 0, o = 0).
//
// Block (x, y) takes 32 (row, query head) pairs of KV head y (rows_per_block
// consecutive rows times its G query heads), 8 per wave, and streams the
// relay rows it sees through LDS in tiles of TR rows (64 for d <= 64, 32 for
// d <= 128, so a tile of keys and values stays under 34 KB; the pairs'
// queries take 16 KB more).  Scores: SPLIT
// lanes per relay row (lane % TR the row, lane / TR half of the dims), the
// lane's part of the key row held in registers across the wave's pairs, one
// online-softmax update per pair and tile; values: lanes over dims, each value
// read from LDS once for all the pairs, the probabilities read lane by lane.
constexpr int kRelayPairs = 32, kRelayPairsPerWave = kRelayPairs / 4;

template <int SPLIT>
__global__ void __launch_bounds__(256) k_relay_partial(RelayPartialArgs a, int rows_per_block) {
    constexpr int TR = kWave / SPLIT;   // relay rows per tile
    constexpr int DL = SPLIT;           // dims per lane in the value sum (d <= 64 * SPLIT)
    extern __shared__ __align__(16) float rl[];
    const int d = a.d, KP = d + 4, kvw = a.kv_heads * d, G = a.heads / a.kv_heads, kvh = blockIdx.y;
    // [TR][d + 4] keys, [TR][d] values, [kRelayPairs][d] queries
    float *ks = rl, *vs = rl + TR * KP, *qs = vs + TR * d;
    const int r0 = blockIdx.x * rows_per_block, nrows = min(rows_per_block, a.rows - r0), pairs = nrows * G;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int jr = lane % TR, part = lane / TR, dp = d / SPLIT;   // score lanes: relay row, dims part
    const int n_max = ((a.p0 + r0 + nrows - 1) / a.chunk) * a.slots;
    // pair pi is row r0 + pi / G, query head kvh * G + pi % G; pairs past the
    // last row repeat the last pair and are not stored
    for (int i = threadIdx.x; i < kRelayPairs * (d / 4); i += blockDim.x) {
        const int pi = min(i / (d / 4), pairs - 1), c = (i % (d / 4)) * 4;
        const float4 q = load_f4(a.qkv + (int64_t)(r0 + pi / G) * a.ld + (kvh * G + pi % G) * d + c);
        *(float4 *)(qs + (i / (d / 4)) * d + c) = q;
    }
    int seen[kRelayPairsPerWave];   // relay rows each pair sees
    float m[kRelayPairsPerWave], l[kRelayPairsPerWave], o[kRelayPairsPerWave][DL];
#pragma unroll
    for (int k = 0; k < kRelayPairsPerWave; ++k) {
        const int pi = min(wave * kRelayPairsPerWave + k, pairs - 1);
        seen[k] = ((a.p0 + r0 + pi / G) / a.chunk) * a.slots;
        m[k] = -INFINITY;
        l[k] = 0.0f;
#pragma unroll
        for (int x = 0; x < DL; ++x) o[k][x] = 0.0f;
    }
    const float *kb = a.relay_k + kvh * d, *vb = a.relay_v + kvh * d;
    for (int base = 0; base < n_max; base += TR) {
        const int cnt = min(TR, n_max - base);
        __syncthreads();   // the previous tile is read (the first: the queries are staged)
        for (int i = threadIdx.x; i < TR * (d / 4); i += blockDim.x) {   // rows past cnt: zeros
            const int j = i / (d / 4), c = (i % (d / 4)) * 4;
            const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            *(float4 *)(ks + j * KP + c) = j < cnt ? load_f4(kb + (int64_t)(base + j) * kvw + c) : z;
            *(float4 *)(vs + j * d + c) = j < cnt ? load_f4(vb + (int64_t)(base + j) * kvw + c) : z;
        }
        __syncthreads();
        // The lane's key row (its dims part) stays in registers for the
        // wave's pairs, and each value read from LDS serves all of them.  No
        // branches per pair: a pair that sees none of the tile scores -inf
        // everywhere and keeps its state (alpha 1, or 0 with nothing summed).
        float4 kr4[16];   // dp <= 64
#pragma unroll
        for (int i = 0; i < 16; ++i)
            kr4[i] = 4 * i < dp ? *(const float4 *)(ks + jr * KP + part * dp + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
        float p[kRelayPairsPerWave];
#pragma unroll
        for (int k = 0; k < kRelayPairsPerWave; ++k) {
            const int n = min(seen[k] - base, cnt);   // rows of the tile it sees (may be <= 0)
            const float *q = qs + (wave * kRelayPairsPerWave + k) * d + part * dp;
            float sc = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (4 * i < dp) {
                    const float4 qq = *(const float4 *)(q + 4 * i);
                    sc = fmaf(qq.x, kr4[i].x, sc);
                    sc = fmaf(qq.y, kr4[i].y, sc);
                    sc = fmaf(qq.z, kr4[i].z, sc);
                    sc = fmaf(qq.w, kr4[i].w, sc);
                }
            }
            if constexpr (SPLIT == 2) sc += __shfl_xor(sc, TR, kWave);
            sc = jr < n ? sc * a.inv_root : -INFINITY;
            const float mn = fmaxf(m[k], wave_max(sc));
            const float alpha = m[k] == -INFINITY ? 0.0f : expf(m[k] - mn);
            p[k] = jr < n ? expf(sc - mn) : 0.0f;
            l[k] = l[k] * alpha + wave_sum(p[k]) / SPLIT;   // each row's probability sits in SPLIT lanes
            m[k] = mn;
#pragma unroll
            for (int x = 0; x < DL; ++x) o[k][x] *= alpha;
        }
        // 8 relay rows a round over the staged rows (past a pair's n:
        // probability 0; past cnt: zero values)
        for (int jj = 0; jj < cnt; jj += 8) {
            float vv[8][DL];
#pragma unroll
            for (int u = 0; u < 8; ++u)
#pragma unroll
                for (int x = 0; x < DL; ++x) vv[u][x] = lane + x * kWave < d ? vs[(jj + u) * d + lane + x * kWave] : 0.0f;
#pragma unroll
            for (int k = 0; k < kRelayPairsPerWave; ++k)
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p[k]), jj + u));
#pragma unroll
                    for (int x = 0; x < DL; ++x) o[k][x] = fmaf(pj, vv[u][x], o[k][x]);
                }
        }
    }
#pragma unroll
    for (int k = 0; k < kRelayPairsPerWave; ++k) {
        const int pi = wave * kRelayPairsPerWave + k;
        if (pi >= pairs) break;
        const int t = r0 + pi / G, h = kvh * G + pi % G;
        float *out = a.ext + ((int64_t)t * a.heads + h) * (d + 4);
        if (lane == 0) *(float4 *)out = make_float4(m[k], l[k], 0.0f, 0.0f);
#pragma unroll
        for (int x = 0; x < DL; ++x)
            if (lane + x * kWave < d) out[4 + lane + x * kWave] = o[k][x];
    }
}

// y = 2^x by exp2_hw (which 0) or e^x by the library expf (which 1): the
// softmax exponential of the batched prefill and the token step's.
__global__ void __launch_bounds__(256) k_debug_exp(const float *x, float *y, int n, int which) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = which == 0 ? exp2_hw(x[i]) : expf(x[i]);
}

}  // namespace

int launch_debug_exp(hipStream_t s, const float *x, float *y, int n, int which) {
    MR_REQUIRE(x && y && n > 0 && (which == 0 || which == 1), "debug exp: bad arguments");
    k_debug_exp<<<ceil_div(n, 256), 256, 0, s>>>(x, y, n, which);
    MR_LAUNCHED("enqueue debug exp");
    return MR_OK;
}

bool prefill_attention_presplit(const PrefillAttnArgs &a) {
    const int win = a.window ? a.window : a.cap;
    const int first = std::max(0, a.p0 - win + 1), n = a.p0 + a.rows - first;
    const bool h = a.d == 128 || a.d == 64 || a.d == 32;
    return h && a.kv16 && a.kv16_scale && a.kv16_max && ceil_div(n, kKeys) * kKeys <= a.kv16_rows &&
           a.kv_heads * a.d <= 4096 && (int64_t)4 * a.kv16_rows * a.kv_heads * a.d * 2 < ((int64_t)1 << 31);
}

int launch_prefill_attention(hipStream_t s, const PrefillAttnArgs &a) {
    MR_REQUIRE(a.qkv && a.ring_k && a.ring_v && a.out && a.rows > 0 && a.cap > 0, "prefill attention: bad arguments");
    MR_REQUIRE(a.kv_heads > 0 && a.heads % a.kv_heads == 0, "prefill attention: heads must be a multiple of kv_heads");
    MR_REQUIRE(a.d % 4 == 0 && a.d <= 128 && a.ld % 4 == 0 && a.ldo % 4 == 0,
               "prefill attention: head_dim must be a multiple of 4 and at most 128");
    const int G = a.heads / a.kv_heads;
    const int gb = G % 4 == 0 ? 4 : G % 2 == 0 ? 2 : 1;
    const dim3 grid(ceil_div(a.rows, 64 / gb), a.kv_heads * (G / gb));
    const int win = a.window ? a.window : a.cap;
    const int first = std::max(0, a.p0 - win + 1), n = a.p0 + a.rows - first;
    const int n_tiles = ceil_div(n, kKeys);
    const bool planes = prefill_attention_presplit(a);
    MR_REQUIRE(!a.out_hl || (planes && !a.ext && a.out_scale && ((uintptr_t)a.out_hl & 7) == 0),
               "prefill attention: FP16-term output needs the presplit form, no extra partial and row scales");
    if (planes) {   // split the attended keys and values once
        PrefillAttnArgs b = a;   // the maxima's per-block partials where they fit, else atomics
        if (!(b.kv_part && prefill_kv_max_blocks(n) <= b.kv_part_blocks)) {
            b.kv_part = nullptr;
            MR_HIP(hipMemsetAsync(a.kv16_max, 0, 2 * a.kv_heads * sizeof(unsigned), s), "prefill attention");
        }
        const int threads = ceil_div(a.kv_heads * a.d / 4, kWave) * kWave;
        k_kv_max<<<prefill_kv_max_blocks(n), threads, 0, s>>>(b, first, n);
        const dim3 tiles(n_tiles, a.kv_heads);
        if (a.d == 128) k_kv_split_tiles<128><<<tiles, 256, 0, s>>>(b, first, n);
        else if (a.d == 64) k_kv_split_tiles<64><<<tiles, 256, 0, s>>>(b, first, n);
        else k_kv_split_tiles<32><<<tiles, 256, 0, s>>>(b, first, n);
    }
    // Two row sets a wave where that still leaves two workgroups per CU and
    // the rows' key counts are about even (at most a quarter of the rows see
    // less than a whole window) or the grid still fills the CUs twice; a
    // causal chunk keeps the twice as many one-set workgroups, latest rows
    // first, so that the short ones fill in behind the long ones.
    const dim3 grid2(ceil_div(a.rows, 128 / gb), a.kv_heads * (G / gb));
    const int wg2 = grid2.x * grid2.y;
    const bool two = wg2 >= 512 && (wg2 >= 1024 || (int64_t)(win - a.p0) * 4 <= a.rows);
    if (a.d == 128) {
        if (planes && two) k_attn_prefill_t<128, 2><<<grid2, kAttnThreads, 0, s>>>(a, gb, first);
        else if (planes) k_attn_prefill_t<128, 1><<<grid, kAttnThreads, 0, s>>>(a, gb, first);
        else k_attn_prefill_h<128><<<grid, kAttnThreads, 0, s>>>(a, gb);
    } else if (a.d == 64) {
        if (planes && two) k_attn_prefill_t<64, 2><<<grid2, kAttnThreads, 0, s>>>(a, gb, first);
        else if (planes) k_attn_prefill_t<64, 1><<<grid, kAttnThreads, 0, s>>>(a, gb, first);
        else k_attn_prefill_h<64><<<grid, kAttnThreads, 0, s>>>(a, gb);
    } else if (a.d == 32) {
        if (planes && two) k_attn_prefill_t<32, 2><<<grid2, kAttnThreads, 0, s>>>(a, gb, first);
        else if (planes) k_attn_prefill_t<32, 1><<<grid, kAttnThreads, 0, s>>>(a, gb, first);
        else k_attn_prefill_h<32><<<grid, kAttnThreads, 0, s>>>(a, gb);
    } else if (a.d <= 16) k_attn_prefill<16><<<grid, kAttnThreads, 0, s>>>(a, gb);
    else if (a.d <= 32) k_attn_prefill<32><<<grid, kAttnThreads, 0, s>>>(a, gb);
    else if (a.d <= 64) k_attn_prefill<64><<<grid, kAttnThreads, 0, s>>>(a, gb);
    else k_attn_prefill<128><<<grid, kAttnThreads, 0, s>>>(a, gb);
    MR_LAUNCHED("enqueue prefill attention");
    return MR_OK;
}

int launch_relay_partial(hipStream_t s, const RelayPartialArgs &a) {
    MR_REQUIRE(a.qkv && a.relay_k && a.relay_v && a.ext && a.rows > 0 && a.chunk > 0 && a.slots > 0,
               "relay partial: bad arguments");
    MR_REQUIRE(a.kv_heads > 0 && a.heads % a.kv_heads == 0 && a.heads / a.kv_heads <= kRelayPairs && a.d % 4 == 0 &&
                   a.d <= 2 * kWave && (a.d <= kWave || a.d % 8 == 0) && a.ld % 4 == 0,
               "relay partial: unsupported geometry");
    const int G = a.heads / a.kv_heads, rows_per_block = kRelayPairs / G;
    const dim3 grid(ceil_div(a.rows, rows_per_block), a.kv_heads);
    const size_t q_lds = (size_t)kRelayPairs * a.d * sizeof(float);
    if (a.d <= kWave)
        k_relay_partial<1><<<grid, 256, (size_t)kWave * (2 * a.d + 4) * sizeof(float) + q_lds, s>>>(a, rows_per_block);
    else
        k_relay_partial<2><<<grid, 256, (size_t)(kWave / 2) * (2 * a.d + 4) * sizeof(float) + q_lds, s>>>(
            a, rows_per_block);
    MR_LAUNCHED("enqueue relay partial");
    return MR_OK;
}

int launch_rms_rows(hipStream_t s, const float *x, int ldx, const float *gain, float eps, int width, float *y,
                    int ldy, int rows) {
    k_rms_rows<<<rows, 256, 0, s>>>(x, ldx, gain, eps, width, y, ldy);
    MR_LAUNCHED("enqueue row RMSNorm");
    return MR_OK;
}

// k_rms_rows_split for rows of at most 2048 values, one wave per row and four
// rows per workgroup, with no barrier: lane l holds the runs that threads l,
// l + 64, l + 128 and l + 192 of the one-workgroup-per-row form hold, keeps
// their sums of squares apart and adds their wave sums in that form's order,
// so the scale, the planes and the row scales are the same bits.
//
// With oscale, also the row scale of the SwiGLU output that a GEMM computes
// from these rows (gemm.h, c_hl): |silu(g)| <= |g| and, by Cauchy-Schwarz,
// |g| <= |y| ng and |u| <= |y| nu for the gate and up weights' largest row
// norms ng and nu, so |y|^2 ng nu bounds every value of the output row.
__global__ void __launch_bounds__(256) k_rms_rows_split_w(const float *x, int ldx, const float *gain, float eps,
                                                          int width, float *scale, _Float16 *hl, int rows,
                                                          float ng, float nu, float *oscale) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + (int64_t)row * ldx;
    const int runs = width / 8;   // <= 256
    float4 v[4][2], g[4][2];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const int r = lane + 64 * w;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            v[w][t] = r < runs ? load_f4(xr + 8 * r + 4 * t) : make_float4(0.f, 0.f, 0.f, 0.f);
            g[w][t] = gain && r < runs ? load_f4(gain + 8 * r + 4 * t) : make_float4(1.f, 1.f, 1.f, 1.f);
        }
    }
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        float ss = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
            ss += v[w][t].x * v[w][t].x + v[w][t].y * v[w][t].y + v[w][t].z * v[w][t].z + v[w][t].w * v[w][t].w;
        total += wave_sum(ss);
    }
    const float rs = 1.0f / sqrtf(total / (float)width + eps);
    float mx = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        if (lane + 64 * w >= runs) continue;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            v[w][t] = make_float4(v[w][t].x * rs * g[w][t].x, v[w][t].y * rs * g[w][t].y, v[w][t].z * rs * g[w][t].z,
                                  v[w][t].w * rs * g[w][t].w);
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[w][t].x), fabsf(v[w][t].y)), fmaxf(fabsf(v[w][t].z), fabsf(v[w][t].w))));
        }
    }
    mx = wave_max(mx);
    const float sc = f16_range_scale(mx);
    if (lane == 0) scale[row] = sc;
    if (oscale) {
        float ss = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            if (lane + 64 * w >= runs) continue;
#pragma unroll
            for (int t = 0; t < 2; ++t)
                ss += v[w][t].x * v[w][t].x + v[w][t].y * v[w][t].y + v[w][t].z * v[w][t].z + v[w][t].w * v[w][t].w;
        }
        ss = wave_sum(ss);
        if (lane == 0) oscale[row] = f16_range_scale(ss * 1.001f * ng * nu);
    }
    _Float16 *hi = hl + (int64_t)row * width, *lo = hl + (int64_t)rows * width + (int64_t)row * width;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const int r = lane + 64 * w;
        if (r >= runs) continue;
        const float y[8] = {v[w][0].x, v[w][0].y, v[w][0].z, v[w][0].w, v[w][1].x, v[w][1].y, v[w][1].z, v[w][1].w};
        f16x8 h, l;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            _Float16 th, tl;
            split2h(y[i] * sc, th, tl);
            h[i] = th;
            l[i] = tl;
        }
        *(f16x8 *)(hi + 8 * r) = h;
        *(f16x8 *)(lo + 8 * r) = l;
    }
}

int launch_rms_rows_split(hipStream_t s, const float *x, int ldx, const float *gain, float eps, int width,
                          float *scale, _Float16 *planes, int rows, float ng, float nu, float *oscale) {
    static_assert(256 * 8 * kSplitChunks == 8192, "rms_split_fits");
    MR_REQUIRE(rms_split_fits(width) && ldx % 4 == 0,
               "row RMSNorm into FP16 terms: width must be a multiple of 8 and at most 8192");
    MR_REQUIRE(!oscale || (width <= 2048 && ng > 0.0f && nu > 0.0f),
               "row RMSNorm into FP16 terms: the SwiGLU output scale needs rows of at most 2048 and weight norms");
    if (width <= 2048)
        k_rms_rows_split_w<<<ceil_div(rows, 4), 256, 0, s>>>(x, ldx, gain, eps, width, scale, planes, rows, ng, nu,
                                                             oscale);
    else k_rms_rows_split<<<rows, 256, 0, s>>>(x, ldx, gain, eps, width, scale, planes, rows);
    MR_LAUNCHED("enqueue row RMSNorm into FP16 terms");
    return MR_OK;
}

int launch_qk_rows(hipStream_t s, float *qkv, int ld, int rows, int p0, int heads, int kv_heads, int d,
                   const float *q_gain, const float *k_gain, float eps, int norm, const float *rope, int split_half) {
    if (d <= 128)
        k_qk_rows_r<8><<<dim3(ceil_div(rows, 8), ceil_div(heads + kv_heads, 4)), 256, 0, s>>>(
            qkv, ld, p0, heads, kv_heads, d, q_gain, k_gain, eps, norm, rope, split_half, nullptr, rows);
    else
        k_qk_rows<<<dim3(rows, ceil_div(heads + kv_heads, 4)), 256, 0, s>>>(qkv, ld, p0, heads, kv_heads, d, q_gain,
                                                                           k_gain, eps, norm, rope, split_half, nullptr);
    MR_LAUNCHED("enqueue q/k norm and RoPE");
    return MR_OK;
}

int launch_k_rows_at(hipStream_t s, float *k, int ld, int rows, const int *positions, int kv_heads, int d,
                     const float *k_gain, float eps, const float *rope, int split_half) {
    if (d <= 128)
        k_qk_rows_r<8><<<dim3(ceil_div(rows, 8), ceil_div(kv_heads, 4)), 256, 0, s>>>(
            k, ld, 0, 0, kv_heads, d, nullptr, k_gain, eps, 1, rope, split_half, positions, rows);
    else
        k_qk_rows<<<dim3(rows, ceil_div(kv_heads, 4)), 256, 0, s>>>(k, ld, 0, 0, kv_heads, d, nullptr, k_gain, eps, 1,
                                                                   rope, split_half, positions);
    MR_LAUNCHED("enqueue key norm and RoPE at row positions");
    return MR_OK;
}

int launch_ring_store(hipStream_t s, const float *qkv, int ld, int qd, int kvw, float *ring_k, float *ring_v, int cap,
                      int p0, int rows) {
    MR_REQUIRE(ld % 4 == 0 && qd % 4 == 0 && kvw % 4 == 0 && (((uintptr_t)qkv | (uintptr_t)ring_k | (uintptr_t)ring_v) & 15) == 0,
               "ring fill: rows must be 16-byte aligned");
    const int first = std::max(p0, p0 + rows - cap);
    k_ring_store<<<p0 + rows - first, 256, 0, s>>>(qkv, ld, qd, kvw, ring_k, ring_v, cap, first, p0);
    MR_LAUNCHED("enqueue ring fill");
    return MR_OK;
}

int launch_embed_rows(hipStream_t s, const void *table, int dtype, const int *ids, int p0, int rows, float *x, int h) {
    k_embed_rows<<<rows, 256, 0, s>>>(table, dtype, ids, p0, x, h);
    MR_LAUNCHED("enqueue embedding rows");
    return MR_OK;
}

}  // namespace mr
