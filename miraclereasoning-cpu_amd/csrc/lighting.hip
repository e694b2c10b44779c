// flashlighting-2.0 token-step kernels (model.py:146-190).
//
// The reference recomputes, every step, the keys and values of every stored
// latent row (model.py:159-162).  A row's key depends only on its latent and
// its stored position, and its value only on its latent, so this build keeps a
// key and a value cache row per latent row and computes one only when a row is
// created: the new row of each step, and the row a merge produces.
//
// Per layer and step: the queries (RMSNorm with q_norm + RoPE), the new latent
// (RMSNorm with latent_norm, appended with its position and count 1) and its
// cache rows (the K/V projection; K: RMSNorm with k_norm + RoPE at its
// position; V as projected) - one launch of k_light_kv, or k_light_prep, a
// GEMV and k_light_store where its geometry does not fit; the attention over
// every row with latent_mask (split partials and a merge for head dims
// 32/64/128, else k_light_attend in kernels.cl's sequential orders);
// k_light_compact (model.py:168-188: drop the overflow without memory slots;
// merge the two oldest rows by their counts when the overflow exceeds the
// slots; else mark the overflow as memory rows); then - when a merge happened
// - the merged row's cache rows at its new position.
#include "lighting.h"

#include "block_gemv.h"
#include "gemv_block.h"
#include "split_attention.h"

namespace mr {
static_assert(kLightRows == split::kRows && kLightMaxSplits == split::kMaxParts, "latent split geometry");
namespace {

// RMSNorm of one row (kernels.cl:19-28) by one 64-lane workgroup: the row is
// staged in LDS, each lane sums the squares of its strided elements and a
// wave reduction adds the lanes (an FP32 reordering of the reference's
// sequential sum).
__device__ __forceinline__ void rms_row(const float *x, const float *gain, float eps, int width, float *y, float *scale) {
    float v = 0.0f;
    for (int j = threadIdx.x; j < width; j += blockDim.x) {
        const float t = x[j];
        y[j] = t;
        v = fmaf(t, t, v);
    }
    v = wave_sum(v);
    const float sc = 1.0f / sqrtf(v / (float)width + eps);
    if (threadIdx.x == 0) *scale = sc;
    for (int j = threadIdx.x; j < width; j += blockDim.x) y[j] = y[j] * sc * (gain ? gain[j] : 1.0f);
    __syncthreads();
}

// RoPE of one head row in LDS at integer position p (kernels.cl:30-44).
__device__ __forceinline__ void rope_row(float *row, const float *rope, int p, int d, int split_half) {
    const int half = d / 2;
    const float *cs = rope + (int64_t)p * half * 2;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const int j = split_half ? i : 2 * i, k = split_half ? i + half : 2 * i + 1;
        float u = row[j], v = row[k];
        rope_rotate(u, v, cs[2 * i], cs[2 * i + 1]);
        row[j] = u;
        row[k] = v;
    }
    __syncthreads();
}

// grid heads + 1, 64 threads: blocks < heads rotate queries, the last appends
// the new latent row.
__global__ void __launch_bounds__(64) k_light_prep(LightArgs a) {
    extern __shared__ float row[];
    __shared__ float scale;
    if (a.done && *a.done) return;
    const int pos = *a.pos;
    if ((int)blockIdx.x < a.heads) {
        const int h = blockIdx.x;
        rms_row(a.qlat + (int64_t)h * a.d, a.q_gain, a.eps, a.d, row, &scale);
        rope_row(row, a.rope, pos, a.d, a.split_half);
        for (int j = threadIdx.x; j < a.d; j += blockDim.x) a.q_rot[(int64_t)h * a.d + j] = row[j];
        return;
    }
    rms_row(a.qlat + (int64_t)a.heads * a.d, a.latent_gain, a.eps, a.latent, row, &scale);
    const LightState st = *a.st;
    const int slot = (st.start + st.rows) % a.cap;
    for (int j = threadIdx.x; j < a.latent; j += blockDim.x) {
        a.arena[(int64_t)slot * a.latent + j] = row[j];
        a.lat_new[j] = row[j];
    }
    if (threadIdx.x == 0) {
        a.positions[slot] = (float)pos;
        a.counts[slot] = 1.0f;
    }
}

// grid kv_heads, 64 threads: cache row of the new (merged = false) or merged row.
__global__ void __launch_bounds__(64) k_light_store(LightArgs a, int merged) {
    extern __shared__ float row[];
    __shared__ float scale;
    if (a.done && *a.done) return;
    const LightState st = *a.st;
    if (merged && st.skip_merged) return;
    const int slot = merged ? st.merged_slot : (st.start + st.rows) % a.cap;
    const int p = (int)a.positions[slot];
    const int kh = blockIdx.x, kvw = a.kv_heads * a.d;
    rms_row(a.kv + (int64_t)kh * a.d, a.k_gain, a.eps, a.d, row, &scale);
    rope_row(row, a.rope, p, a.d, a.split_half);
    for (int j = threadIdx.x; j < a.d; j += blockDim.x) {
        a.kcache[(int64_t)slot * kvw + (int64_t)kh * a.d + j] = row[j];
        a.vcache[(int64_t)slot * kvw + (int64_t)kh * a.d + j] = a.kv[kvw + (int64_t)kh * a.d + j];
    }
}

// ------------------------------------------------------------------ fused row kernel
// grid heads + 1 + 4 kv_heads, 256 threads.  Blocks < heads: query h, RMSNorm
// with q_norm, RoPE at pos -> q_rot.  Block heads: the new latent row
// (RMSNorm with latent_norm) appended with its position and count 1.  The next
// 2 kv_heads blocks: the K rows of KV head kh (first kv_heads) or its V rows,
// [Wk; Wv] . latent with the latent normalized by the block itself (the same
// arithmetic as the appending block, so the same bits); the last 2 kv_heads
// blocks: the same for the row the previous step's compaction merged (its
// latent from the arena, at its position), when one is pending.  A K row then takes RMSNorm
// with k_norm and RoPE at the row's position; the rows go to the caches.
constexpr int kKvThreads = 256;

// RoPE of a row in LDS whose (cos, sin) for pair tid (tid < d/2 <= blockDim)
// the thread loaded beforehand (kernels.cl:30-44).
__device__ __forceinline__ void rope_row_pre(float *row, float c, float s, int d, int split_half) {
    const int half = d / 2, i = threadIdx.x;
    if (i < half) {
        const int j = split_half ? i : 2 * i, k = split_half ? i + half : 2 * i + 1;
        float u = row[j], v = row[k];
        rope_rotate(u, v, c, s);
        row[j] = u;
        row[k] = v;
    }
    __syncthreads();
}

// RMSNorm of x[0, width) (kernels.cl:19-28, the sum of squares reduced over
// the block) times gain into y (LDS); all threads return after y is written.
__device__ __forceinline__ void block_rms_row(const float *x, const float *gain, float eps, int width, float *y,
                                              float *red) {
    float v = 0.0f;
    for (int j = threadIdx.x; j < width; j += blockDim.x) {
        const float t = x[j];
        y[j] = t;
        v = fmaf(t, t, v);
    }
    const float sc = 1.0f / sqrtf(block_sum(v, red) / (float)width + eps);
    for (int j = threadIdx.x; j < width; j += blockDim.x) y[j] = y[j] * sc * (gain ? gain[j] : 1.0f);
    __syncthreads();
}

static_assert(kKvThreads == gemv::kGemvThreads, "the row kernel hosts GEMV workgroups");
constexpr int kFfnVec = 4;   // weight vectors per lane and row in one batch of the hosted gate/up rows

template <int DT>
__global__ void __launch_bounds__(kKvThreads) k_light_kv(LightArgs a) {
    constexpr int EB = DT == MR_F32 ? 4 : 2;   // bytes per weight element
    extern __shared__ __align__(16) float sm[];
    __shared__ float red[kKvThreads / kWave];
    const int nrow = a.heads + 1 + 4 * a.kv_heads;
    if ((int)blockIdx.x >= nrow) {   // the FFN branch's gate/up rows
        gemv::gemv_vec_block<DT, 1, kFfnVec, PRO_COPY, EPI_SWIGLU>(a.ffn, a.ffn_lpr, blockIdx.x - nrow, sm);
        return;
    }
    const int tid = threadIdx.x, d = a.d, kvw = a.kv_heads * d;
    const int b0 = (int)blockIdx.x - (a.heads + 1);    // cache-row blocks from 0
    const bool merged = b0 >= 2 * a.kv_heads;          // the pending merged row
    const int b = merged ? b0 - 2 * a.kv_heads : b0;
    const bool isk = b >= 0 && b < a.kv_heads;
    const int kh = isk ? b : b - a.kv_heads;
    // The weight loads depend on nothing this step computes: they go out
    // before the flag, position and state loads.
    BlockGemv<DT> gemv;
    if (b >= 0) gemv.issue((const char *)a.kv_w + ((int64_t)(isk ? 0 : kvw) + (int64_t)kh * d) * a.latent * EB, d,
                           a.latent);
    if (a.done && *a.done) return;
    const LightState st = *a.st;
    if (merged && !st.pending) return;
    const int pos = *a.pos;
    const int slot = merged ? st.merged_slot : (st.start + st.rows) % a.cap;
    const float *raw_latent = a.qlat + (int64_t)a.heads * d;
    // the rotation angles of this thread's pair at the row's position
    const bool pre = d / 2 <= kKvThreads;
    float rc = 1.0f, rsn = 0.0f;
    if (pre && tid < d / 2) {
        const float *cs = a.rope + ((int64_t)(merged ? st.merged_pos : pos) * (d / 2) + tid) * 2;
        rc = cs[0];
        rsn = cs[1];
    }
    if (b < 0) {
        if ((int)blockIdx.x < a.heads) {   // query blockIdx.x
            const int h = blockIdx.x;
            block_rms_row(a.qlat + (int64_t)h * d, a.q_gain, a.eps, d, sm, red);
            if (pre) rope_row_pre(sm, rc, rsn, d, a.split_half);
            else rope_row(sm, a.rope, pos, d, a.split_half);
            for (int j = tid; j < d; j += kKvThreads) a.q_rot[(int64_t)h * d + j] = sm[j];
            return;
        }
        block_rms_row(raw_latent, a.latent_gain, a.eps, a.latent, sm, red);   // the new latent row
        for (int j = tid; j < a.latent; j += kKvThreads) a.arena[(int64_t)slot * a.latent + j] = sm[j];
        if (tid == 0) {
            a.positions[slot] = (float)pos;
            a.counts[slot] = 1.0f;
        }
        return;
    }
    float *xs = sm, *ys = sm + ((a.latent + 3) & ~3);
    if (merged) {   // the merged latent, from this layer's arena (lat_new is shared by the layers)
        for (int j = tid; j < a.latent; j += kKvThreads) xs[j] = a.arena[(int64_t)slot * a.latent + j];
        __syncthreads();
    } else {
        block_rms_row(raw_latent, a.latent_gain, a.eps, a.latent, xs, red);
    }
    gemv.finish(xs, ys);
    __syncthreads();
    float *cache = (isk ? a.kcache : a.vcache) + (int64_t)slot * kvw + (int64_t)kh * d;
    if (isk) {   // RMSNorm with k_norm, RoPE at the row's position
        const int p = merged ? st.merged_pos : pos;
        float v = 0.0f;
        for (int j = tid; j < d; j += kKvThreads) v = fmaf(ys[j], ys[j], v);
        const float sc = 1.0f / sqrtf(block_sum(v, red) / (float)d + a.eps);
        for (int j = tid; j < d; j += kKvThreads) ys[j] = ys[j] * sc * (a.k_gain ? a.k_gain[j] : 1.0f);
        __syncthreads();
        if (pre) rope_row_pre(ys, rc, rsn, d, a.split_half);
        else rope_row(ys, a.rope, p, d, a.split_half);
    }
    for (int j = tid; j < d; j += kKvThreads) cache[j] = ys[j];
}

constexpr int kThreads = 256;

// grid heads, kThreads: attention of query head h over every row.
__global__ void __launch_bounds__(kThreads) k_light_attend(LightArgs a) {
    extern __shared__ float sh[];
    __shared__ float red[kThreads / 64];
    __shared__ float denom;
    if (a.done && *a.done) return;
    const int pos = *a.pos, d = a.d, tid = threadIdx.x;
    const LightState st = *a.st;
    const int n = st.rows + 1;   // with this step's row
    const int h = blockIdx.x, kh = h / (a.heads / a.kv_heads), kvw = a.kv_heads * d;
    const float earliest = (float)(pos - a.window + 1);
    float *qs = sh, *sc = sh + d;
    for (int j = tid; j < d; j += kThreads) qs[j] = a.q_rot[(int64_t)h * d + j];
    __syncthreads();
    const float root = sqrtf((float)d);
    for (int t = tid; t < n; t += kThreads) {   // kernels.cl:58-73, then latent_mask (86-91)
        const int slot = (st.start + t) % a.cap;
        const float *kr = a.kcache + (int64_t)slot * kvw + (int64_t)kh * d;
        float v = 0.0f;
        for (int j = 0; j < d; ++j) v += qs[j] * kr[j];
        v = v / root;
        if (t >= st.memory && a.positions[slot] < earliest) v = -INFINITY;
        sc[t] = v;
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int t = tid; t < n; t += kThreads) mx = fmaxf(mx, sc[t]);
    mx = block_max(mx, red);
    if (tid == 0) {   // kernels.cl:75-84
        float den = 0.0f;
        for (int t = 0; t < n; ++t) den += expf(sc[t] - mx);
        denom = den;
    }
    __syncthreads();
    for (int t = tid; t < n; t += kThreads) sc[t] = expf(sc[t] - mx) / denom;
    __syncthreads();
    for (int j = tid; j < d; j += kThreads) {   // kernels.cl:93-107
        float acc = 0.0f;
        for (int t = 0; t < n; ++t)
            acc += sc[t] * a.vcache[(int64_t)((st.start + t) % a.cap) * kvw + (int64_t)kh * d + j];
        a.out[(int64_t)h * d + j] = acc;
    }
}

// Compaction after this step's attention (model.py:168-188), by one workgroup.
__device__ __forceinline__ void compact_state(const LightArgs &a) {
    __shared__ LightState st;
    __shared__ int mode;   // 0 keep, 1 drop, 2 merge
    if (threadIdx.x == 0) {
        st = *a.st;
        const int n = st.rows + 1, overflow = max(0, n - a.window);
        st.skip_merged = 1;
        st.pending = 0;
        if (a.memory_slots == 0 && overflow > 0) {
            mode = 1;
            st.start = (st.start + overflow) % a.cap;
            st.rows = n - overflow;
            st.memory = 0;
        } else if (overflow > a.memory_slots) {
            mode = 2;
        } else {
            mode = 0;
            st.rows = n;
            st.memory = overflow;
        }
    }
    __syncthreads();
    if (mode == 2) {
        const int s0 = st.start, s1 = (st.start + 1) % a.cap;
        const float ca = a.counts[s0], cb = a.counts[s1];
        for (int j = threadIdx.x; j < a.latent; j += blockDim.x) {   // kernels.cl merge_rows
            const float v = (ca * a.arena[(int64_t)s0 * a.latent + j] + cb * a.arena[(int64_t)s1 * a.latent + j]) /
                            (ca + cb);
            a.arena[(int64_t)s1 * a.latent + j] = v;
            a.lat_new[j] = v;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            const float centre = (a.positions[s0] * ca + a.positions[s1] * cb) / (ca + cb);
            a.positions[s1] = rintf(centre);
            st.merged_pos = (int)rintf(centre);
            a.counts[s1] = ca + cb;
            st.start = s1;
            st.rows = st.rows;   // n - 1 = previous rows
            st.memory = a.memory_slots;
            st.skip_merged = 0;
            st.pending = 1;
            st.merged_slot = s1;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) *a.st = st;
}

// One workgroup: compaction after the single-workgroup attention.
__global__ void __launch_bounds__(64) k_light_compact(LightArgs a) {
    if (a.done && *a.done) return;
    compact_state(a);
}

// Rows per lane group and weight vectors per lane per batch of the down
// projection rows hosted below (one row per lane group: twice the
// workgroups of two, measured 3.7 % faster per step at 2048 x 5632).
constexpr int kDownRows = 1, kDownVec = 6;

// Split-key form of the same attention for head dims 32/64/128: workgroup
// (split s, head h) scores rows [64 s, 64 s + 64) of the memory with the
// latent mask (kernels.cl:86-91: non-memory rows older than the window) and
// writes its partial; a second kernel merges the splits of each head.
// grid (splits, heads + extra): the workgroups of the extra rows run the
// hosted down projection's GEMV blocks (workgroup (x, heads + e) is block
// e * splits + x) with weights of dtype DT.
template <int D, int DT>
__global__ void __launch_bounds__(split::kThreads) k_light_attend_part(LightArgs a) {
    if ((int)blockIdx.y >= a.heads) {
        const int b = ((int)blockIdx.y - a.heads) * (int)gridDim.x + (int)blockIdx.x;
        extern __shared__ float sm[];
        if (b < a.down_blocks)
            gemv::gemv_vec_block<DT, kDownRows, kDownVec, PRO_COPY, EPI_STORE>(a.down, a.down_lpr, b, sm);
        return;
    }
    if (a.done && *a.done) return;
    const LightState st = *a.st;
    const int n = st.rows + 1;                  // with this step's row
    const int t0 = blockIdx.x * kLightRows;
    const int h = blockIdx.y, kh = h / (a.heads / a.kv_heads), kvw = a.kv_heads * D;
    if (t0 >= n) {   // no rows in this split yet: an empty partial, so the merge needs no row count
        float *part = a.part + ((int64_t)h * gridDim.x + blockIdx.x) * (D + 2);
        for (int j = threadIdx.x; j < D + 2; j += split::kThreads) part[j] = j == 0 ? -INFINITY : 0.0f;
        return;
    }
    const float earliest = (float)(*a.pos - a.window + 1);
    const auto rows = [&](int t, const float **k, const float **v) {
        const int slot = (st.start + t) % a.cap;
        if (t >= st.memory && a.positions[slot] < earliest) return false;
        *k = a.kcache + (int64_t)slot * kvw + (int64_t)kh * D;
        *v = a.vcache + (int64_t)slot * kvw + (int64_t)kh * D;
        return true;
    };
    split::partial<D>(a.q_rot + (int64_t)h * D, t0, min(n, t0 + kLightRows), rows,
                      a.part + ((int64_t)h * gridDim.x + blockIdx.x) * (D + 2));
}

// grid heads + 1, split::kThreads: workgroup h < heads merges every split's
// partial of head h (empty ones included); the last workgroup compacts the
// memory beside them (its rows were all read by the split kernel before this
// launch, and the merges read only partials).
template <int D>
__global__ void __launch_bounds__(split::kThreads) k_light_attend_merge(LightArgs a, int splits) {
    if (a.done && *a.done) return;
    if ((int)blockIdx.x == a.heads) {
        compact_state(a);
        return;
    }
    split::merge<D>(a.part + (int64_t)blockIdx.x * splits * (D + 2), splits, -1, a.out + (int64_t)blockIdx.x * D);
}

__global__ void k_light_residual(float *hidden, const float *o, const float *f, const float *ag, const float *fg,
                                 float rs, int n, const int *done) {
    if (done && *done) return;
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    const float branch = (0.0f + ag[0] * o[j]) + fg[0] * f[j];
    hidden[j] = hidden[j] + rs * branch;
}

// k_light_residual over a chunk's rows: four values a thread, 16-byte loads
// and stores, the same operations per value (n a multiple of 4).
__global__ void k_light_residual4(float *hidden, const float *o, const float *f, const float *ag, const float *fg,
                                  float rs, int n4) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n4) return;
    const float a = ag[0], b = fg[0];
    const float4 ov = ((const float4 *)o)[j], fv = ((const float4 *)f)[j];
    float4 x = ((float4 *)hidden)[j];
    x.x = x.x + rs * ((0.0f + a * ov.x) + b * fv.x);
    x.y = x.y + rs * ((0.0f + a * ov.y) + b * fv.y);
    x.z = x.z + rs * ((0.0f + a * ov.z) + b * fv.z);
    x.w = x.w + rs * ((0.0f + a * ov.w) + b * fv.w);
    ((float4 *)hidden)[j] = x;
}

// ------------------------------------------------------------------ batched prefill
// one thread per latent column: the running logical row 0 through the chunk
// Logical row 0 through the chunk.  Every merge folds one original row
// (count 1) into row 0 and adds 1 to its count, so row 0 is the running mean
// of what it folded: with sum = count * row 0 a merge is sum += row, and row 0
// is sum / count wherever a step reads it (the value merge_rows gives step by
// step, up to rounding).  The chunk's steps go in segments of kRow0Seg: the
// merged rows are gathered by step (zeros where a step merges nothing), each
// segment's sum and merge count formed in parallel, the segments' starting
// states by one pass over them, and then every segment runs its steps from its
// starting state, in parallel.
constexpr int kRow0Seg = 128;

// merged[t] = the row step t's merge folds in, or zeros (one workgroup a step).
__global__ void __launch_bounds__(kWave) k_light_gather_merged(LightRowsArgs a) {
    const int t = blockIdx.x;
    float *dst = a.merged + (int64_t)t * a.latent;
    if (!(a.flags[t] & 2)) {
        for (int j = threadIdx.x; j < a.latent; j += kWave) dst[j] = 0.0f;
        return;
    }
    const int r = a.merge_row[t];
    const float *src = r >= a.p0 ? a.lat + (int64_t)(r - a.p0) * a.latent : a.arena + (int64_t)(r % a.cap) * a.latent;
    for (int j = threadIdx.x; j < a.latent; j += kWave) dst[j] = src[j];
}

// grid (segments, latent / 64), one wave: the segment's sum of merged rows
// (8 rows' loads in flight) and its merge count.
__global__ void __launch_bounds__(kWave) k_row0_segments(LightRowsArgs a, float *seg_sum, int *seg_cnt) {
    const int sg = blockIdx.x, lane = threadIdx.x, j = blockIdx.y * kWave + lane;
    const int t0 = sg * kRow0Seg, t1 = min(t0 + kRow0Seg, a.rows);
    const int jj = min(j, a.latent - 1);
    float acc = 0.0f;
    for (int t = t0; t < t1; t += 8) {
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = t + u < t1 ? a.merged[(int64_t)(t + u) * a.latent + jj] : 0.0f;
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += x[u];
    }
    if (j < a.latent) seg_sum[(int64_t)sg * a.latent + j] = acc;
    if (blockIdx.y == 0) {
        int c = 0;
        for (int t = t0 + lane; t < t1; t += kWave) c += (a.flags[t] & 2) ? 1 : 0;
        for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, kWave);
        if (lane == 0) seg_cnt[sg] = c;
    }
}

// grid latent / 64, one wave: segment starting sums (exclusive, in segment
// order, in place: each workgroup its own dims) and counts (into seg_start,
// by workgroup 0), row 0's count before the chunk's first merge
// (first_count[0]) and row 0 after the chunk.
__global__ void __launch_bounds__(kWave) k_row0_starts(LightRowsArgs a, float *seg_sum, const int *seg_cnt, int nseg,
                                                       float *first_count, int *seg_start) {
    const int lane = threadIdx.x, j = blockIdx.x * kWave + lane, jj = min(j, a.latent - 1);
    const float v0 = a.init_from_arena ? a.arena[(int64_t)a.init_slot * a.latent + jj] : a.lat[jj];
    float sum = 0.0f;
    int cnt = 0, first_seg = -1;
    for (int sg = 0; sg < nseg; ++sg) {
        const float x = seg_sum[(int64_t)sg * a.latent + jj];
        const int c = seg_cnt[sg];
        if (j < a.latent) seg_sum[(int64_t)sg * a.latent + j] = sum;
        if (blockIdx.x == 0 && lane == 0) seg_start[sg] = cnt;
        if (first_seg < 0 && c > 0) first_seg = sg;
        sum += x;
        cnt += c;
    }
    float c0 = 1.0f;
    if (first_seg >= 0)
        for (int t = first_seg * kRow0Seg;; ++t)
            if (a.flags[t] & 2) {
                c0 = a.merge_count[t];
                break;
            }
    if (blockIdx.x == 0 && lane == 0) first_count[0] = c0;
    if (j < a.latent) a.slot0_final[j] = cnt > 0 ? (c0 * v0 + sum) / (c0 + (float)cnt) : v0;
}

// grid (segments, latent / 64), one wave: the segment's steps from its
// starting state: a step that sees row 0 stores it, a merge adds its row
// (8 steps' records read ahead, no branches on them).
__global__ void __launch_bounds__(kWave) k_row0_steps(LightRowsArgs a, const float *seg_sum, const int *seg_cnt,
                                                      const float *first_count) {
    __shared__ __align__(16) int fl[kRow0Seg], ex[kRow0Seg];
    const int sg = blockIdx.x, lane = threadIdx.x, j = blockIdx.y * kWave + lane, jj = min(j, a.latent - 1);
    const bool on = j < a.latent;
    const int t0 = sg * kRow0Seg, nt = min(kRow0Seg, a.rows - t0);
    for (int i = lane; i < kRow0Seg; i += kWave) {
        fl[i] = i < nt ? a.flags[t0 + i] : 0;
        ex[i] = i < nt ? a.extra_index[t0 + i] : 0;
    }
    __syncthreads();
    const float v0 = a.init_from_arena ? a.arena[(int64_t)a.init_slot * a.latent + jj] : a.lat[jj];
    const float c0 = first_count[0];
    const int before = seg_cnt[sg];
    bool merged = before > 0;
    float sum = merged ? c0 * v0 + seg_sum[(int64_t)sg * a.latent + jj] : 0.0f;
    float count = c0 + (float)before;
    for (int i0 = 0; i0 < nt; i0 += 8) {
        int f[8], e[8];
        float x[8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int4 f4 = *(const int4 *)&fl[i0 + 4 * h], e4 = *(const int4 *)&ex[i0 + 4 * h];
            f[4 * h] = f4.x; f[4 * h + 1] = f4.y; f[4 * h + 2] = f4.z; f[4 * h + 3] = f4.w;
            e[4 * h] = e4.x; e[4 * h + 1] = e4.y; e[4 * h + 2] = e4.z; e[4 * h + 3] = e4.w;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = i0 + u < nt ? a.merged[(int64_t)(t0 + i0 + u) * a.latent + jj] : 0.0f;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if ((f[u] & 1) && on) a.slot0[(int64_t)e[u] * a.latent + j] = merged ? sum / count : v0;
            const bool m = (f[u] & 2) != 0;
            sum = m && !merged ? c0 * v0 : sum;
            merged = merged || m;
            sum += x[u];   // zeros where the step merges nothing
            count = m ? count + 1.0f : count;
        }
    }
}

// grid (rows, heads), 64 threads
__global__ void __launch_bounds__(64) k_light_extra(const float *qkv, int ld, const float *kv0, const int *extra_index,
                                                    float *ext, int heads, int kv_heads, int d) {
    const int t = blockIdx.x, h = blockIdx.y, kh = h / (heads / kv_heads), kvw = kv_heads * d;
    float *out = ext + ((int64_t)t * heads + h) * (d + 4);
    const int e = extra_index[t];
    if (e < 0) {
        for (int j = threadIdx.x; j < d; j += 64) out[4 + j] = 0.0f;
        if (threadIdx.x == 0) {
            out[0] = -INFINITY;
            out[1] = out[2] = out[3] = 0.0f;
        }
        return;
    }
    const float *q = qkv + (int64_t)t * ld + (int64_t)h * d, *k = kv0 + (int64_t)e * 2 * kvw + (int64_t)kh * d;
    float dot = 0.0f;
    for (int j = threadIdx.x; j < d; j += 64) dot = fmaf(q[j], k[j], dot);
    dot = wave_sum(dot);
    const float *v = k + kvw;
    for (int j = threadIdx.x; j < d; j += 64) out[4 + j] = v[j];
    if (threadIdx.x == 0) {
        out[0] = dot / sqrtf((float)d);
        out[1] = 1.0f;
        out[2] = out[3] = 0.0f;
    }
}

// grid rows stored, 256 threads
__global__ void __launch_bounds__(256) k_light_store_rows(LightRowsArgs a, int first) {
    const int r = first + blockIdx.x, slot = r % a.cap;
    const float *src = a.lat + (int64_t)(r - a.p0) * a.latent;
    for (int j = threadIdx.x; j < a.latent; j += 256) a.arena[(int64_t)slot * a.latent + j] = src[j];
    if (threadIdx.x == 0) {
        a.positions[slot] = (float)r;
        a.counts[slot] = 1.0f;
    }
}

__global__ void __launch_bounds__(256) k_light_finish(LightRowsArgs a, LightState *st, LightState fin, int write_slot0,
                                                      float slot0_position, float slot0_count) {
    if (write_slot0) {
        for (int j = threadIdx.x; j < a.latent; j += 256)
            a.arena[(int64_t)fin.start * a.latent + j] = a.slot0_final[j];
        if (threadIdx.x == 0) {
            a.positions[fin.start] = slot0_position;
            a.counts[fin.start] = slot0_count;
        }
    }
    if (threadIdx.x == 0) *st = fin;
}

}  // namespace

int launch_light_prep(hipStream_t s, const LightArgs &a) {
    k_light_prep<<<a.heads + 1, 64, (size_t)std::max(a.d, a.latent) * sizeof(float), s>>>(a);
    MR_LAUNCHED("enqueue latent prologue");
    return MR_OK;
}

int launch_light_store_kv(hipStream_t s, const LightArgs &a, bool merged) {
    k_light_store<<<a.kv_heads, 64, (size_t)a.d * sizeof(float), s>>>(a, merged ? 1 : 0);
    MR_LAUNCHED("enqueue latent key/value row");
    return MR_OK;
}

bool light_kv_fused(int dtype, int latent, int d) {
    const bool fits = dtype == MR_F32    ? block_gemv_fits<MR_F32>(latent)
                      : dtype == MR_BF16 ? block_gemv_fits<MR_BF16>(latent)
                      : dtype == MR_F16  ? block_gemv_fits<MR_F16>(latent)
                                         : false;
    return fits && d % 2 == 0;
}

bool light_down_in_attend(LightArgs &a, const GemvArgs &g, int dtype) {
    a.down_blocks = 0;
    const int e = dtype == MR_F32 ? 4 : 8, bytes = dtype == MR_F32 ? 4 : 2;
    if (!light_split_path(a.d, a.cap) || !a.part || g.k % e || (uintptr_t)g.w % 16 ||
        ((int64_t)g.k * bytes) % 16)
        return false;
    const int nvec = g.k / e;
    int lpr = 1;
    while (lpr * 2 <= nvec && lpr < kWave) lpr *= 2;
    a.down = g;
    a.down_dtype = dtype;
    a.down_lpr = lpr;
    a.down_blocks = ceil_div(g.n, gemv::kGemvWaves * (kWave / lpr) * kDownRows);
    return true;
}

bool light_ffn_in_row_kernel(LightArgs &a, const GemvArgs &g, int dtype) {
    a.ffn_blocks = 0;
    const int e = dtype == MR_F32 ? 4 : 8, bytes = dtype == MR_F32 ? 4 : 2;
    if (dtype != a.kv_dtype || g.k % e || (uintptr_t)g.w % 16 || (uintptr_t)g.w2 % 16 || ((int64_t)g.k * bytes) % 16)
        return false;
    const int nvec = g.k / e;
    int lpr = 1;
    while (lpr * 2 <= nvec && lpr < kWave) lpr *= 2;
    if (ceil_div(nvec, lpr) > kFfnVec) return false;   // one batch of kFfnVec vectors must cover a row
    a.ffn = g;
    a.ffn_lpr = lpr;
    a.ffn_blocks = ceil_div(g.n, gemv::kGemvWaves * (kWave / lpr));
    return true;
}

int launch_light_kv(hipStream_t s, const LightArgs &a) {
    MR_REQUIRE(light_kv_fused(a.kv_dtype, a.latent, a.d) && a.kv_w, "latent rows: unsupported projection geometry");
    const int grid = a.heads + 1 + 4 * a.kv_heads + a.ffn_blocks;
    size_t lds = (size_t)(((a.latent + 3) & ~3) + std::max(a.d, a.latent)) * sizeof(float);
    if (a.ffn_blocks) lds = std::max(lds, (size_t)gemv::gemv_lds_floats(a.ffn, PRO_COPY) * sizeof(float));
    if (a.kv_dtype == MR_BF16) k_light_kv<MR_BF16><<<grid, kKvThreads, lds, s>>>(a);
    else if (a.kv_dtype == MR_F16) k_light_kv<MR_F16><<<grid, kKvThreads, lds, s>>>(a);
    else k_light_kv<MR_F32><<<grid, kKvThreads, lds, s>>>(a);
    MR_LAUNCHED("enqueue latent rows");
    return MR_OK;
}

template <int D>
static void attend_part_launch(hipStream_t s, dim3 grid, size_t lds, const LightArgs &a) {
    if (a.down_blocks && a.down_dtype == MR_F32) k_light_attend_part<D, MR_F32><<<grid, split::kThreads, lds, s>>>(a);
    else if (a.down_blocks && a.down_dtype == MR_F16) k_light_attend_part<D, MR_F16><<<grid, split::kThreads, lds, s>>>(a);
    else k_light_attend_part<D, MR_BF16><<<grid, split::kThreads, lds, s>>>(a);
}

int launch_light_attend(hipStream_t s, const LightArgs &a) {
    if (light_split_path(a.d, a.cap) && a.part) {
        const int splits = light_splits(a.cap);
        const dim3 grid(splits, a.heads + ceil_div(a.down_blocks, splits));
        const size_t lds = a.down_blocks ? (size_t)gemv::gemv_lds_floats(a.down, PRO_COPY) * sizeof(float) : 0;
        MR_REQUIRE(lds <= 64 * 1024, "latent attention: hosted down projection exceeds shared memory");
        switch (a.d) {
            case 128:
                attend_part_launch<128>(s, grid, lds, a);
                MR_LAUNCHED("enqueue latent attention splits");
                k_light_attend_merge<128><<<a.heads + 1, split::kThreads, 0, s>>>(a, splits);
                break;
            case 64:
                attend_part_launch<64>(s, grid, lds, a);
                MR_LAUNCHED("enqueue latent attention splits");
                k_light_attend_merge<64><<<a.heads + 1, split::kThreads, 0, s>>>(a, splits);
                break;
            default:
                attend_part_launch<32>(s, grid, lds, a);
                MR_LAUNCHED("enqueue latent attention splits");
                k_light_attend_merge<32><<<a.heads + 1, split::kThreads, 0, s>>>(a, splits);
                break;
        }
        MR_LAUNCHED("enqueue latent attention merge and compaction");
        return MR_OK;
    }
    const size_t lds = (size_t)(a.d + a.cap) * sizeof(float);
    MR_REQUIRE(lds <= 64 * 1024, "latent attention: window and memory slots exceed shared memory");
    k_light_attend<<<a.heads, kThreads, lds, s>>>(a);
    MR_LAUNCHED("enqueue latent attention");
    k_light_compact<<<1, 64, 0, s>>>(a);
    MR_LAUNCHED("enqueue latent compaction");
    return MR_OK;
}

int launch_light_residual(hipStream_t s, float *hidden, const float *o, const float *f, const float *attention_gate,
                          const float *ffn_gate, float rs, int n, const int *done) {
    const bool vec = !done && n % 4 == 0 && (((uintptr_t)hidden | (uintptr_t)o | (uintptr_t)f) & 15) == 0;
    if (vec) k_light_residual4<<<ceil_div(n / 4, 256), 256, 0, s>>>(hidden, o, f, attention_gate, ffn_gate, rs, n / 4);
    else k_light_residual<<<ceil_div(n, 256), 256, 0, s>>>(hidden, o, f, attention_gate, ffn_gate, rs, n, done);
    MR_LAUNCHED("enqueue gated residual");
    return MR_OK;
}

int launch_light_slot0(hipStream_t s, const LightRowsArgs &a) {
    MR_REQUIRE(a.lat && a.arena && a.slot0 && a.slot0_final && a.flags && a.extra_index && a.merge_count &&
                   a.merge_row && a.merged && a.row0_ws && a.rows > 0 && a.latent > 0 && a.cap > 0,
               "latent rows: bad arguments");
    const int nseg = ceil_div(a.rows, kRow0Seg), slices = ceil_div(a.latent, kWave);
    float *seg_sum = a.row0_ws, *first_count = seg_sum + (size_t)nseg * a.latent;
    int *seg_cnt = (int *)(first_count + 4), *seg_start = seg_cnt + nseg;
    k_light_gather_merged<<<a.rows, kWave, 0, s>>>(a);
    MR_LAUNCHED("enqueue merged-row gather");
    k_row0_segments<<<dim3(nseg, slices), kWave, 0, s>>>(a, seg_sum, seg_cnt);
    MR_LAUNCHED("enqueue row 0 segment sums");
    k_row0_starts<<<slices, kWave, 0, s>>>(a, seg_sum, seg_cnt, nseg, first_count, seg_start);
    MR_LAUNCHED("enqueue row 0 segment starts");
    k_row0_steps<<<dim3(nseg, slices), kWave, 0, s>>>(a, seg_sum, seg_start, first_count);
    MR_LAUNCHED("enqueue row 0 steps");
    return MR_OK;
}

int launch_light_extra(hipStream_t s, const float *qkv, int ld, const float *kv0, const int *extra_index, float *ext,
                       int rows, int heads, int kv_heads, int d) {
    MR_REQUIRE(qkv && extra_index && ext && rows > 0 && kv_heads > 0 && heads % kv_heads == 0, "latent extra: bad arguments");
    k_light_extra<<<dim3(rows, heads), 64, 0, s>>>(qkv, ld, kv0, extra_index, ext, heads, kv_heads, d);
    MR_LAUNCHED("enqueue latent extra row");
    return MR_OK;
}

int launch_light_store_rows(hipStream_t s, const LightRowsArgs &a) {
    const int first = std::max(a.p0, a.p0 + a.rows - a.cap);
    k_light_store_rows<<<a.p0 + a.rows - first, 256, 0, s>>>(a, first);
    MR_LAUNCHED("enqueue latent rows");
    return MR_OK;
}

int launch_light_finish(hipStream_t s, const LightRowsArgs &a, LightState *st, const LightState &fin, int write_slot0,
                        float slot0_position, float slot0_count) {
    k_light_finish<<<1, 256, 0, s>>>(a, st, fin, write_slot0, slot0_position, slot0_count);
    MR_LAUNCHED("enqueue latent state");
    return MR_OK;
}

}  // namespace mr
