// Persistent step kernel.
//
// One launch of one workgroup per CU runs a whole token step: the
// host builds, once per model, a program of phases (embedding row; per layer:
// Q/K/V GEMV, attention units with the split merge, O GEMV + residual, gate/up
// GEMV + SwiGLU, down GEMV + residual; LM head + greedy choice) and every
// workgroup walks it.
//
// Why one kernel: at bs = 1 a step streams 2.3-2.6 GB through ~120 dependent
// phases of 8-50 MB.  Separate launches pay a launch gap and a ramp-up each;
// here a workgroup issues the weight loads of its share of a phase (weights
// never depend on activations) before it waits for that phase's input, so the
// weights are in flight while the previous phase finishes elsewhere.
//
// No grid barriers: activations travel as flag-in-data cells (ll.h), and a
// workgroup waits only for the cells it reads.  The split merge of a group of
// query heads is done by one of its units (merger_split), which polls the other splits'
// partial cells (by the last unit to count itself when units outnumber the
// workgroups), and the step's closing work (greedy choice, position) by the
// last workgroup to leave the launch.  Every wait is bounded (ll.h).
//
// Reuse of a cell buffer within a step is ordered by the data dependencies
// themselves: a phase that rewrites a buffer consumes, directly or through the
// phases between, the outputs of every workgroup that read the previous
// contents, and those reads precede the reader's own outputs.
#include "step.h"

namespace mr {
namespace {

using namespace att;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int NT = kStepThreads;
constexpr int NW = NT / kWave;
constexpr int kXcds = 8;   // MI355X's XCDs, each with its own L2; the dispatcher deals workgroups round-robin

// Program descriptors are read through the constant address space: uniform
// loads from it become scalar loads, made where a field is used.
#define MR_CONST __attribute__((address_space(4)))

__device__ __forceinline__ unsigned epoch(const StepArgs &s, int pos, int phase) {
    return (unsigned)pos * (unsigned)s.stride + (unsigned)phase + 1u;
}

__device__ __forceinline__ float ldc(const float *p) {
    return __hip_atomic_load(gmem(const_cast<float *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc(float *p, float v) {
    __hip_atomic_store(gmem(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ldci(const int *p) {
    return __hip_atomic_load(gmem(const_cast<int *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stci(int *p, int v) {
    __hip_atomic_store(gmem(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void stamp(unsigned long long *tr, int i) {
    if (tr && threadIdx.x == 0) tr[i] = wall_clock64();
}

// ------------------------------------------------------------------ GEMV phase
// Rows [r0, r1) of each workgroup, in groups of `slots` rows (lpr lanes per
// row) dealt round-robin to the stream waves.  A job is kVC 16-byte vectors per
// lane of one row group of one matrix; a stream wave keeps kDepth jobs in
// flight (64 KB per CU in all), and issues
// its first kDepth before the phase's input is staged.  Loads past a matrix's
// end read a 16-byte dummy so every job issues the same number of loads and
// the compiler's waits stay exact.
//
// The control waves wait for the input's producers, read the input cells into
// one of two LDS buffers (a phase's stream waves read one while the control
// waves fill the other for the next phase) and take the RMSNorm sum.
constexpr int NC = kControlWaves;
constexpr int NS = kStreamWaves;

// Stream waves of this workgroup that have finished a phase (an LDS count):
// the last of them to finish marks the workgroup's progress word, so a
// consumer polls one word per workgroup.  Polls of shared words and cells all
// land on a few memory channels, and every weight load that touches those
// channels queues behind them: fewer, rarer polls keep the streams fast.
__shared__ unsigned finished_waves;

__device__ __forceinline__ bool wg_mark(const StepArgs &s, unsigned ep) {
    const unsigned old = atomicAdd(&finished_waves, 1u);
    if ((old + 1) % NS != 0) return false;
#pragma unroll
    for (int c = 0; c < kWordCopies; ++c) ll::mark(s.progress + c * kWordCopyStride + blockIdx.x, ep);
    return true;
}

// Rows [r0, r1) of this workgroup in a phase of n rows: equal blocks in
// workgroup order, over the workgroups the phase does not skip.
__device__ __forceinline__ void wg_rows(const Phase &ph, int &r0, int &r1) {
    const int n = ph.n, b = blockIdx.x;
    int workers = gridDim.x, rank = b;
    bool skipped = false;
    if (gridDim.x <= kSkipBits) {
        int total = 0, below = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const unsigned m = ph.skip[i];
            total += __builtin_popcount(m);
            if (32 * i + 32 <= b) below += __builtin_popcount(m);
            else if (32 * i <= b) below += __builtin_popcount(m & ((1u << (b - 32 * i)) - 1u));
        }
        skipped = (ph.skip[b >> 5] >> (b & 31)) & 1u;
        workers -= total;
        rank -= below;
    }
    const int rpw = (n + workers - 1) / workers;
    r0 = skipped ? n : min(rank * rpw, n);
    r1 = skipped ? n : min(r0 + rpw, n);
}
constexpr int kVC = 4;
constexpr int kDepth = 4;   // jobs in flight per stream wave when a job is one matrix (M = 1)
// Of them, the jobs issued before the phase's input is staged: the rest go
// out once it is (a CU returns loads in issue order, so the control waves'
// polls wait behind whatever the stream waves have in flight; two of four
// measured fastest, none much slower).
constexpr int kEntryDepth = 2;

struct GemvGeo {
    int r0, r1;      // rows of this workgroup
    int nvec;        // 16-byte vectors per row
    int lpr, slots;  // lanes per row, rows per job
    int cpr;         // jobs per row
    int groups;      // row groups of this stream wave
    int jobs;        // jobs of this stream wave
    int64_t rowbytes;
};

template <int M>
__device__ __forceinline__ GemvGeo gemv_geo(const Phase &ph) {
    GemvGeo g;
    const int eb = ph.dtype == MR_F32 ? 4 : 2;
    g.rowbytes = (int64_t)ph.k * eb;
    g.nvec = ph.k / (16 / eb);
    g.lpr = 1;
    while (g.lpr * 2 <= g.nvec && g.lpr < kWave) g.lpr *= 2;
    g.slots = kWave / g.lpr;
    const int vpl = (g.nvec + g.lpr - 1) / g.lpr;
    g.cpr = (vpl + kVC - 1) / kVC;
    wg_rows(ph, g.r0, g.r1);
    const int ngroups = (g.r1 - g.r0 + g.slots - 1) / g.slots;
    const int sw = (int)(threadIdx.x >> 6) - NC;
    g.groups = sw >= 0 && ngroups > sw ? (ngroups - sw + NS - 1) / NS : 0;
    g.jobs = g.groups * g.cpr;
    return g;
}

// A job: chunk c of row group j, for all M matrices (the gate and up rows of
// SwiGLU travel together, so no job selects a matrix at run time).
struct Cursor {
    int j, c;
};

__device__ __forceinline__ void advance(Cursor &u, int cpr) {
    if (++u.c == cpr) {
        u.c = 0;
        ++u.j;
    }
}

__device__ __forceinline__ int job_row(const GemvGeo &g, int j) {
    const int lane = threadIdx.x & 63, sw = (int)(threadIdx.x >> 6) - NC;
    return g.r0 + (sw + NS * j) * g.slots + lane / g.lpr;
}

template <int M>
__device__ __forceinline__ void issue(u32x4 (&b)[M][kVC], const Cursor &u, const char *w0, const char *w1,
                                      const GemvGeo &g, const void *dummy) {
    const int sub = (threadIdx.x & 63) & (g.lpr - 1);
    const int row = job_row(g, u.j);
    const bool live = u.j < g.groups && row < g.r1;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const char *base = (m == 0 ? w0 : w1) + (int64_t)row * g.rowbytes;
#pragma unroll
        for (int i = 0; i < kVC; ++i) {
            const int v = sub + (u.c * kVC + i) * g.lpr;
            const char *p = live && v < g.nvec ? base + (int64_t)v * 16 : (const char *)dummy;
            b[m][i] = __builtin_nontemporal_load(gmem((const u32x4 *)p));
        }
    }
}

template <int DT>
__device__ __forceinline__ void widen16(const u32x4 &v, float *o) {
    if constexpr (DT == MR_F32) {
        o[0] = __uint_as_float(v.x); o[1] = __uint_as_float(v.y);
        o[2] = __uint_as_float(v.z); o[3] = __uint_as_float(v.w);
    } else if constexpr (DT == MR_BF16) {
        o[0] = __uint_as_float(v.x << 16); o[1] = __uint_as_float(v.x & 0xffff0000u);
        o[2] = __uint_as_float(v.y << 16); o[3] = __uint_as_float(v.y & 0xffff0000u);
        o[4] = __uint_as_float(v.z << 16); o[5] = __uint_as_float(v.z & 0xffff0000u);
        o[6] = __uint_as_float(v.w << 16); o[7] = __uint_as_float(v.w & 0xffff0000u);
    } else {
        o[0] = f16_to_f32(v.x & 0xffffu); o[1] = f16_to_f32(v.x >> 16);
        o[2] = f16_to_f32(v.y & 0xffffu); o[3] = f16_to_f32(v.y >> 16);
        o[4] = f16_to_f32(v.z & 0xffffu); o[5] = f16_to_f32(v.z >> 16);
        o[6] = f16_to_f32(v.w & 0xffffu); o[7] = f16_to_f32(v.w >> 16);
    }
}

// The input values of chunk c for this lane, from the staged input in LDS.
template <int E>
__device__ __forceinline__ void load_x(float (&xr)[kVC][E], const GemvGeo &g, const float *xs, int c) {
    const int sub = (threadIdx.x & 63) & (g.lpr - 1);
#pragma unroll
    for (int i = 0; i < kVC; ++i) {
        const int v = min(sub + (c * kVC + i) * g.lpr, g.nvec - 1);
#pragma unroll
        for (int e = 0; e < E; e += 4) {
            const float4 t = *(const float4 *)(xs + v * E + e);
            xr[i][e] = t.x; xr[i][e + 1] = t.y; xr[i][e + 2] = t.z; xr[i][e + 3] = t.w;
        }
    }
}

template <int DT, int M, int E>
__device__ __forceinline__ void consume(const u32x4 (&b)[M][kVC], const Cursor &u, const GemvGeo &g,
                                        const float (&xr)[kVC][E], float (&acc)[M]) {
    const int sub = (threadIdx.x & 63) & (g.lpr - 1);
#pragma unroll
    for (int i = 0; i < kVC; ++i) {
        const int v = sub + (u.c * kVC + i) * g.lpr;
        if (v < g.nvec) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float wf[E];
                widen16<DT>(b[m][i], wf);
#pragma unroll
                for (int e = 0; e < E; ++e) acc[m] = fmaf(wf[e], xr[i][e], acc[m]);
            }
        }
    }
}

// Greedy choice bookkeeping of the LM head phase (per lane).
struct Best {
    float v;
    int i;
    int bad;
};

__device__ __forceinline__ void best_merge(Best &a, float v, int i) {
    if (v > a.v || (v == a.v && i < a.i)) {
        a.v = v;
        a.i = i;
    }
}

// Control waves: wait for the producers of the input (epoch ep_x), read it into
// xs, and read the residual inputs of this workgroup's rows (epoch ep_res) into
// res.  With the RMSNorm prologue (kernels.cl:19-28) xs holds input x gain and
// red[wave] the wave's sum of squares of the raw input: the 1/rms scale is
// applied to the dot products, y = scale * W (x * gain).
constexpr int kStartWords = 32;   // a phase reads its input cells once 1/kStartWords of the producers are done

__device__ __forceinline__ void stage_input(const Phase &ph, const GemvGeo &g, const StepArgs &s, unsigned ep_x,
                                            unsigned ep_res, float *xs, float *res, float *red, ll::Wait &w) {
    const int me = threadIdx.x, lanes = NC * kWave;
    // The first control wave waits until the producers start finishing (a
    // 32nd of their progress words), then releases the others through an LDS
    // word (ep_x, or ~0 when its wait gave up); the cell reads below wait for
    // the rest cell by cell.  Reading the cells from the first word on saves a
    // memory round trip per phase over waiting for every word; polling them
    // from the phase's start loads the memory with polls and is slower.
    __shared__ unsigned released;
    if (me < kWave) {
        if (ph.ready)
            ll::wait_words(ph.ready, ph.nready, ep_x, me, ph.nready - max(1, ph.nready / kStartWords), w);
        else
            ll::wait_words(s.progress + (blockIdx.x % kWordCopies) * kWordCopyStride, s.nprogress, ep_x, me,
                           s.nprogress - max(1, s.nprogress / kStartWords), w);
        const bool ok = __all(w.ok);
        if (me == 0) __hip_atomic_store(&released, ok ? ep_x : ~0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    } else {
        unsigned r;
        while ((r = __hip_atomic_load(&released, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) != ep_x && r != ~0u)
            __builtin_amdgcn_s_sleep(1);
        if (r == ~0u) w.ok = false;
    }
    const float *gain = ph.pro == PRO_RMS ? ph.gain : nullptr;
    const int n2 = ph.k / 2;
    float ss = 0.0f;
    constexpr int B = 8;
    for (int base = me; base < n2; base += lanes * B) {
        float2 gv[B];
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const int gi = 2 * min(base + i * lanes, n2 - 1);
            gv[i] = gain ? make_float2(gmem(gain)[gi], gmem(gain)[gi + 1]) : make_float2(1.0f, 1.0f);
        }
        // A poll round re-reads only the pairs still missing (late rounds carry
        // few bytes and return quickly); an arrived pair goes to xs as read,
        // and the sum of squares and gains follow in a fixed order.
        unsigned pending = 0;
#pragma unroll
        for (int i = 0; i < B; ++i)
            if (base + i * lanes < n2) pending |= 1u << i;
        for (;;) {
            ll::u64x2 c[B];
#pragma unroll
            for (int i = 0; i < B; ++i)
                c[i] = pending & (1u << i) ? ll::peek2(ph.x, 2 * (base + i * lanes), 2 * n2) : ll::u64x2{0ull, 0ull};
#pragma unroll
            for (int i = 0; i < B; ++i)
                if ((pending & (1u << i)) && (unsigned)(c[i].x >> 32) == ep_x && (unsigned)(c[i].y >> 32) == ep_x) {
                    const int idx = base + i * lanes;
                    *(float2 *)(xs + 2 * idx) =
                        make_float2(__uint_as_float((unsigned)c[i].x), __uint_as_float((unsigned)c[i].y));
                    pending &= ~(1u << i);
                }
            if (!pending || !ll::backoff(w)) break;
        }
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const int idx = base + i * lanes;
            if (idx < n2) {
                const float2 v = *(const float2 *)(xs + 2 * idx);
                ss = fmaf(v.x, v.x, ss);
                ss = fmaf(v.y, v.y, ss);
                *(float2 *)(xs + 2 * idx) = make_float2(v.x * gv[i].x, v.y * gv[i].y);
            }
        }
    }
    if ((ph.k & 1) && me == 0) {
        const float v = ll::get(ph.x + ph.k - 1, ep_x, w);
        xs[ph.k - 1] = v * (gain ? gmem(gain)[ph.k - 1] : 1.0f);
        ss = fmaf(v, v, ss);
    }
    if (ph.epi == EPI_RESIDUAL)
        for (int r = g.r0 + me; r < g.r1; r += lanes) res[r - g.r0] = ll::get(ph.y + r, ep_res, w);
    ss = wave_sum(ss);
    if ((me & 63) == 0) red[me >> 6] = ss;
}

template <int DT, int M, bool HEAD>
__device__ __forceinline__ bool gemv_phase(const Phase &ph, const StepArgs &s, unsigned ep_x, unsigned ep_res,
                                           unsigned ep_y, float *xs, unsigned long long *tr) {
    constexpr int E = DT == MR_F32 ? 4 : 8;
    __shared__ unsigned status[NC];   // per control wave: ep_x, or ~0 when a wait gave up
    const GemvGeo g = gemv_geo<M>(ph);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool ctl = wave < NC;
    float *res = xs + ((ph.k + 3) & ~3);
    float *red = res + ((g.r1 - g.r0 + 3) & ~3);
    float *outs = red + ((NC + 3) & ~3);
    const bool mine = g.r0 < g.r1;
    constexpr int DEPTH = kDepth / M;
    const char *w0 = (const char *)ph.w, *w1 = M == 2 ? (const char *)ph.w2 : w0;
    u32x4 buf[DEPTH][M][kVC];
    Cursor is{0, 0};
    if (ctl) {
        ll::Wait w = ll::waiter(s.err);
        if (mine) stage_input(ph, g, s, ep_x, ep_res, xs, res, red, w);
        const bool ok = __all(w.ok);
        if (lane == 0) status[wave] = ok ? ep_x : ~0u;
    } else {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            if (d >= kEntryDepth) break;
            issue<M>(buf[d], is, w0, w1, g, s.dummy);
            advance(is, g.cpr);
        }
    }
    lds_barrier();   // the weights stay in flight
#pragma unroll
    for (int i = 0; i < NC; ++i)
        if (status[i] == ~0u) return false;
    if (!ctl) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            if (d < kEntryDepth) continue;
            issue<M>(buf[d], is, w0, w1, g, s.dummy);
            advance(is, g.cpr);
        }
    }
    float scale = 1.0f;
    if (mine && ph.pro == PRO_RMS) {
        float ss = red[0];
#pragma unroll
        for (int i = 1; i < NC; ++i) ss += red[i];
        scale = 1.0f / sqrtf(ss / (float)ph.k + ph.eps);
    }
    stamp(tr, 1);

    Best best{-INFINITY, 0x7fffffff, 0};
    if (!ctl) {
        const int sub = lane & (g.lpr - 1);
        float xr[kVC][E];
        if (g.cpr == 1) load_x<E>(xr, g, xs, 0);   // one chunk per row: the lane's inputs stay in registers
        float acc[M];
#pragma unroll
        for (int i = 0; i < M; ++i) acc[i] = 0.0f;
        Cursor cs{0, 0};
        for (int t0 = 0; t0 < g.jobs; t0 += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                if (t0 + d < g.jobs) {
                    if (g.cpr != 1) load_x<E>(xr, g, xs, cs.c);
                    consume<DT, M, E>(buf[d], cs, g, xr, acc);
                    if (cs.c == g.cpr - 1) {   // row group complete
                        const float a0 = scale * group_sum(acc[0], g.lpr);
                        const float a1 = M == 2 ? scale * group_sum(acc[M - 1], g.lpr) : a0;
                        const int row = job_row(g, cs.j);
                        if (sub == 0 && row < g.r1) {
                            float out;
                            if (M == 2) out = (a0 / (1.0f + expf(-a0))) * a1;   // SwiGLU (kernels.cl:46-50)
                            else if (ph.epi == EPI_RESIDUAL) out = res[row - g.r0] + ph.scale * a0;
                            else out = a0;
                            outs[row - g.r0] = out;
                            if (HEAD) {
                                if (!isfinite(out)) best.bad = 1;
                                best_merge(best, out, row);
                            }
                        }
#pragma unroll
                        for (int i = 0; i < M; ++i) acc[i] = 0.0f;
                    }
                    advance(cs, g.cpr);
                }
                issue<M>(buf[d], is, w0, w1, g, s.dummy);
                advance(is, g.cpr);
            }
        }
        // Output cells are stored after the loop: a store holds the wave's
        // in-order memory counter until it is acknowledged, so stores inside
        // the loop would stall the weight loads behind them.
        for (int j = 0; j < g.groups; ++j) {
            const int row = job_row(g, j);
            if (sub == 0 && row < g.r1) {
                if (HEAD) gmem(ph.logits)[row] = outs[row - g.r0];
                else ll::put(ph.y + row, outs[row - g.r0], ep_y);
            }
        }
        if (!HEAD && lane == 0 && wg_mark(s, ep_y) && tr) tr[2] = wall_clock64();   // last stream wave done
        if (tr && tid == NC * kWave) tr[3] = wall_clock64();   // first stream wave done
    }
    if (HEAD) {   // per-workgroup greedy partial
        __shared__ float bv[NW];
        __shared__ int bi[NW], bb[NW];
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(best.v, off);
            const int oi = __shfl_xor(best.i, off);
            best.bad |= __shfl_xor(best.bad, off);
            best_merge(best, ov, oi);
        }
        if (lane == 0) {
            bv[wave] = best.v;
            bi[wave] = best.i;
            bb[wave] = best.bad;
        }
        __syncthreads();
        if (tid == 0) {
            Best r{bv[0], bi[0], bb[0]};
            for (int i = 1; i < NW; ++i) {
                r.bad |= bb[i];
                best_merge(r, bv[i], bi[i]);
            }
            stc(s.best_val + blockIdx.x, r.v);
            stci(s.best_idx + blockIdx.x, r.i);
            stci(s.bad + blockIdx.x, r.bad);
            if (tr) tr[2] = wall_clock64();
        }
    }
    return true;
}

template <int DT, bool HEAD>
__device__ __forceinline__ bool gemv_dispatch(const Phase &ph, const StepArgs &s, unsigned ep_x, unsigned ep_res,
                                              unsigned ep_y, float *xs, unsigned long long *tr) {
    if (!HEAD && ph.epi == EPI_SWIGLU) return gemv_phase<DT, 2, false>(ph, s, ep_x, ep_res, ep_y, xs, tr);
    return gemv_phase<DT, 1, HEAD>(ph, s, ep_x, ep_res, ep_y, xs, tr);
}

// ------------------------------------------------------------------ other phases
// Embedding row of the position's token (stream waves), as cells.
__device__ __forceinline__ void embed_phase(const Phase &ph, const StepArgs &s, int pos, unsigned ep_y) {
    const int wave = threadIdx.x >> 6;
    if (wave < NC) return;
    const int h = ph.n;
    const int rpw = (h + gridDim.x - 1) / gridDim.x;
    const int j0 = blockIdx.x * rpw, j1 = min(j0 + rpw, h);
    const int tok = gmem(s.ids)[pos];
    for (int j = j0 + (int)threadIdx.x - NC * kWave; j < j1; j += NS * kWave) {
        const int64_t i = (int64_t)tok * h + j;
        float v;
        if (s.embed_dtype == MR_F32) v = gmem((const float *)s.embed)[i];
        else if (s.embed_dtype == MR_BF16) v = bf16_to_f32(gmem((const uint16_t *)s.embed)[i]);
        else v = f16_to_f32(gmem((const uint16_t *)s.embed)[i]);
        ll::put(ph.y + j, v, ep_y);
    }
    if ((threadIdx.x & 63) == 0) wg_mark(s, ep_y);
}

// The split whose unit merges unit group v (KV head, query-head group).
// Split 0 for every group puts a layer's mergers on one XCD; spreading them
// (split v % splits, two per XCD) measured 4 % slower per step.
__host__ __device__ __forceinline__ int merger_split(int, int) { return 0; }

// Attention units (kv head, group of its query heads, split) dealt to the
// workgroups write their partials; one unit per group merges the group's
// splits (kernels.cl:58-107) and reports it in the group's progress word.
// With more units than workgroups, units count themselves in the group's
// counter and the one that completes the count merges.  The counters only grow (one
// count per unit per step), so "last" is the count reaching a multiple of the
// split count.  A unit counts itself once its partial's stores are
// acknowledged, so the merger finds them in one read (it still checks the
// cells' epochs).
template <int D>
__device__ __forceinline__ bool attn_phase(const Phase &ph, const StepArgs &s, int pos, unsigned ep_in,
                                           unsigned ep_out, float *lds, unsigned long long *tr) {
    const AttnStepArgs &a = ph.at.s;
    const int splits = a.splits, hg = a.head_groups, pairs = a.kv_heads * splits, units = pairs * hg;
    if ((int)blockIdx.x >= units) return true;
    __shared__ int merge_it;
    __syncthreads();   // the previous phase's readers of this LDS are done
    const Geo g = geometry(ph.at, pos);
    const Io io{ep_in, ep_out, s.err, nullptr, 0};
    int t0, t1, split_len;
    split_range<D>(g, splits, 0, &t0, &t1, &split_len);
    const int active = (g.total + split_len - 1) / split_len;
    // With one unit per workgroup, the head groups of a (KV head, split) pair
    // run on workgroups of one XCD (workgroup i runs on XCD i % 8), so their
    // reads of the same keys and values meet in that XCD's L2.
    const bool xcd_map = hg > 1 && pairs % kXcds == 0 && units <= (int)gridDim.x;
    for (int u = blockIdx.x; u < units; u += gridDim.x) {
        const int pair = xcd_map ? u % kXcds + kXcds * (u / kXcds / hg) : u / hg;
        const int hs = xcd_map ? (u / kXcds) % hg : u % hg;
        const int kh = pair / splits, split = pair % splits, v = kh * hg + hs;
        // head_groups > 1 is set only where a group fits the wave unit
        const bool ok = a.heads / (a.kv_heads * hg) <= kWaveUnitMaxG
                            ? attn_unit_waves<D, NT>(ph.at, g, kh, hs, split, lds, io, tr ? tr + 1 : nullptr)
                            : attn_unit<D, true, NT>(ph.at, g, kh, split, lds, io);
        if (!ok) return false;
        stamp(tr, 3);   // the unit's partial is stored
        // One unit per workgroup: the unit of split merger_split merges its group,
        // polling the other splits' partial cells as they land (no counter,
        // and no unit waits for its stores to be acknowledged).  With more
        // units than workgroups a workgroup runs several units in turn, and a
        // merger could wait on a unit queued behind it, so there the last
        // unit to count itself merges.  (Written as below, this measured 2 %
        // faster than with the test hoisted out of the loop.)
        if (units <= (int)gridDim.x) {
            if (split == merger_split(v, splits)) {
                // the unit's LDS reads fed its stores, so its LDS is free once
                // every wave is here; the fence keeps the merge's LDS accesses
                // below the barrier
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
                if (!combine_cells<D, NT>(a, v, active, lds, io, tr ? tr + 4 : nullptr)) return false;
                // the word is a hint (readers check the cells' epochs): it
                // need not wait for the merged cells' stores
                if (threadIdx.x == 0) ll::mark(ph.heads_done + v, ep_out);
            }
            continue;
        }
        // Every partial store of the unit is acknowledged (visible to the
        // merger) before the unit counts itself.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            const unsigned old =
                __hip_atomic_fetch_add(gmem(a.counters + v), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            merge_it = (old + 1) % (unsigned)splits == 0;
        }
        __syncthreads();
        if (merge_it) {
            if (!combine_cells<D, NT>(a, v, active, lds, io)) return false;
            __syncthreads();
            if (threadIdx.x == 0) ll::mark(ph.heads_done + v, ep_out);
        }
    }
    return true;
}

// One instantiation per (weight dtype, head dim): a step executes only its
// model's variants, so the code a layer runs stays small enough for the
// instruction cache (a kernel holding every variant is several times larger,
// and each phase then starts with a run of instruction fetches from L2).
template <int DT, int D>
__global__ void __launch_bounds__(NT) k_step(StepArgs s) {
    extern __shared__ float lds[];
    __shared__ int last;
    if (ldci(s.done) || ldci(s.err)) return;
    if (threadIdx.x == 0) finished_waves = 0;
    __syncthreads();
    const int pos = *s.pos;
    const MR_CONST Phase *prog = (const MR_CONST Phase *)s.phases;
    int gemvs = 0;   // GEMV phases so far: their inputs alternate between two LDS buffers
    for (int p = 0; p < s.nphases; ++p) {
        const Phase &ph = *(const Phase *)(prog + p);
        unsigned long long *tr = s.trace ? s.trace + ((size_t)p * gridDim.x + blockIdx.x) * kTraceFields : nullptr;
        stamp(tr, 0);
        const unsigned ep_y = epoch(s, pos, p);
        const unsigned ep_x = epoch(s, pos, ph.x_phase), ep_res = epoch(s, pos, ph.res_phase);
        float *xs = lds + (gemvs & 1) * s.xbuf;
        bool ok = true;
        switch (ph.kind) {
            case PH_EMBED:
                embed_phase(ph, s, pos, ep_y);
                stamp(tr, 1);
                break;
            case PH_GEMV:
                ok = gemv_dispatch<DT, false>(ph, s, ep_x, ep_res, ep_y, xs, tr);
                ++gemvs;
                break;
            case PH_HEAD:
                ok = gemv_dispatch<DT, true>(ph, s, ep_x, ep_res, ep_y, xs, tr);
                ++gemvs;
                break;
            case PH_ATTN:
                ok = attn_phase<D>(ph, s, pos, ep_x, ep_y, lds, tr);
                break;
        }
        if (!ok) return;
        if (ph.kind != PH_GEMV && ph.kind != PH_HEAD) stamp(tr, 2);
    }
    // The last workgroup to leave finishes the step: greedy choice, EOS, position.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(gmem(s.exits), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               gridDim.x - 1;
    __syncthreads();
    if (!last || threadIdx.x != 0) return;
    __hip_atomic_store(gmem(s.exits), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int next = pos + 1;
    *s.pos = next;
    if (s.kind == STEP_GREEDY) {
        Best w{-INFINITY, 0x7fffffff, 0};
        for (int i = 0; i < (int)gridDim.x; ++i) {
            w.bad |= ldci(s.bad + i);
            best_merge(w, ldc(s.best_val + i), ldci(s.best_idx + i));
        }
        if (w.bad) {
            *s.done = 2;
        } else {
            s.ids[next] = w.i;
            s.gen[*s.count] = w.i;
            *s.count += 1;
            if (w.i == *s.eos) *s.done = 1;
        }
    }
}

}  // namespace

int step_xbuf_floats(const std::vector<Phase> &program, int grid) {
    int need = 0;
    for (const Phase &ph : program)
        if (ph.kind == PH_GEMV || ph.kind == PH_HEAD) {
            int skipped = 0;
            if (grid <= kSkipBits)
                for (unsigned m : ph.skip) skipped += __builtin_popcount(m);
            const int workers = std::max(1, grid - skipped);
            const int rpw = (ph.n + workers - 1) / workers;
            need = std::max(need, ((ph.k + 3) & ~3) + 2 * ((rpw + 3) & ~3) + ((NC + 3) & ~3));
        }
    return (need + 3) & ~3;
}

size_t step_lds_bytes(const std::vector<Phase> &program, int grid) {
    size_t need = 2 * (size_t)step_xbuf_floats(program, grid);
    for (const Phase &ph : program) {
        if (ph.kind != PH_ATTN) continue;
        const int G = ph.at.s.heads / (ph.at.s.kv_heads * ph.at.s.head_groups), d = ph.at.s.dim,
                  sp = ph.at.s.splits;
        size_t f;
        const bool waves = G <= kWaveUnitMaxG;
        if (d == 128)
            f = std::max(waves ? unit_waves_lds_floats<128, NT>(G) : unit_lds_floats<128>(G),
                         combine_cells_lds_floats<128, NT>(G, sp));
        else if (d == 64)
            f = std::max(waves ? unit_waves_lds_floats<64, NT>(G) : unit_lds_floats<64>(G),
                         combine_cells_lds_floats<64, NT>(G, sp));
        else
            f = std::max(waves ? unit_waves_lds_floats<32, NT>(G) : unit_lds_floats<32>(G),
                         combine_cells_lds_floats<32, NT>(G, sp));
        need = std::max(need, f);
    }
    return need * sizeof(float);
}

namespace {

template <int DT>
const void *step_kernel_dim(int dim) {
    if (dim == 128) return (const void *)k_step<DT, 128>;
    if (dim == 64) return (const void *)k_step<DT, 64>;
    return (const void *)k_step<DT, 32>;
}

const void *step_kernel(int dtype, int dim) {
    if (dtype == MR_BF16) return step_kernel_dim<MR_BF16>(dim);
    if (dtype == MR_F16) return step_kernel_dim<MR_F16>(dim);
    return step_kernel_dim<MR_F32>(dim);
}

}  // namespace

void step_attention_mergers(const AttnStepArgs &a, int grid, unsigned *mask) {
    // the unit -> (pair, split) deal of attn_phase; with one unit per
    // workgroup, the unit of split merger_split of each (KV head, group)
    // merges it
    const int splits = a.splits, hg = a.head_groups, pairs = a.kv_heads * splits, units = pairs * hg;
    if (units > grid || grid > kSkipBits) return;
    const bool xcd_map = hg > 1 && pairs % kXcds == 0;
    unsigned m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int mergers = 0;
    for (int u = 0; u < units; ++u) {
        const int pair = xcd_map ? u % kXcds + kXcds * (u / kXcds / hg) : u / hg;
        const int hs = xcd_map ? (u / kXcds) % hg : u % hg;
        const int kh = pair / splits, split = pair % splits;
        if (split == merger_split(kh * hg + hs, splits)) {
            m[u >> 5] |= 1u << (u & 31);
            ++mergers;
        }
    }
    // Mergers on every workgroup (one split per group and as many groups as
    // workgroups) would leave the next phase no workers (wg_rows divides its
    // rows among the workgroups it does not skip): skip none then.
    if (mergers >= grid) return;
    for (int i = 0; i < 8; ++i) mask[i] |= m[i];
}

int step_attention_splits(int max_total, int kv_heads, int dim, int cus) {
    const int per_unit = (NT / kWave) * (dim == 128   ? keys_per_wave_round<128>()
                                         : dim == 64 ? keys_per_wave_round<64>()
                                                     : keys_per_wave_round<32>());
    const int want = std::max(1, cus / std::max(kv_heads, 1));
    return std::max(1, std::min(want, ceil_div(max_total, per_unit)));
}

// Doubling while the units still fit the grid: a unit of G heads runs its
// heads one after another, so spare workgroups are best spent on fewer heads
// per unit (the groups of a KV head read the same keys, through one L2).
int step_attention_head_groups(int heads, int kv_heads, int splits, int cus) {
    const int G = heads / std::max(kv_heads, 1);
    int hg = 1;
    while (G % (2 * hg) == 0 && kv_heads * splits * 2 * hg <= cus) hg *= 2;
    return G / hg <= kWaveUnitMaxG ? hg : 1;
}

int step_blocks_per_cu(size_t lds, int dtype, int dim, int *blocks) {
    MR_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks, step_kernel(dtype, dim), NT, lds),
           "query step kernel occupancy");
    return MR_OK;
}

// A plain launch of exactly one workgroup per CU: the kernel's registers fill
// a CU, so the dispatcher places one workgroup on every CU at once (the setup
// checks the occupancy).  Should a workgroup not start, the others' bounded
// waits end the step with an error rather than hanging.
int launch_step(hipStream_t s, const StepArgs &a, int grid, size_t lds, int dtype, int dim) {
    void *args[] = {(void *)&a};
    MR_HIP(hipLaunchKernel(step_kernel(dtype, dim), dim3(grid), dim3(NT), args, lds, s), "launch step kernel");
    return MR_OK;
}

}  // namespace mr
