// Flag-in-data cells for activations exchanged between the workgroups of one
// persistent launch.
//
// A cell is 8 bytes: the float's bits in the low word and the epoch of the
// write in the high word, stored with one 64-bit agent-scope store, so a reader
// that sees the epoch it expects also sees the value written with it.  A
// consumer spins on exactly the cells it reads: there is no grid barrier and no
// separate flag, and a phase starts as soon as its own inputs exist.
//
// Epochs are position * stride + phase + 1, unique per write for the life of a
// sequence; the cells are cleared when the sequence is reset.  Every wait is
// bounded: a poll loop that runs past kSpinLimit sets the launch's error flag,
// and a set flag makes every other waiter give up, so all workgroups leave the
// kernel and the host reports a failed step.
#pragma once

#include "common.h"

namespace mr {
namespace ll {

typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));

constexpr unsigned kSpinLimit = 1u << 21;   // polls (>= ~1 s) before a wait is declared hung

__device__ __forceinline__ uint64_t cell(float v, unsigned ep) {
    return ((uint64_t)ep << 32) | (uint64_t)__float_as_uint(v);
}

__device__ __forceinline__ void put(uint64_t *p, float v, unsigned ep) {
    __hip_atomic_store(gmem(p), cell(v, ep), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t peek(const uint64_t *p) {
    return __hip_atomic_load(gmem(const_cast<uint64_t *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cells base[i], base[i+1] (i even, base 16-byte aligned) with one
// agent-coherent load (cache policy SC1); each 8-byte half is one cell as
// stored.  `base` must be the same for the whole wave (it becomes a buffer
// resource, which lives in scalar registers: a per-lane base would make the
// compiler issue the load once per distinct lane value); i varies per lane.
// Pairs at or past `limit` cells read as zero without touching memory (the
// buffer's bounds check), so lanes with nothing to read add no traffic.
__device__ __forceinline__ u64x2 peek2(const uint64_t *base, int i, int limit = 0x0fffffff) {
    __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, limit * 8, 0x00020000);
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, i * 8, 0, 16);
    u64x2 r;
    r.x = ((uint64_t)v.y << 32) | v.x;
    r.y = ((uint64_t)v.w << 32) | v.z;
    return r;
}

__device__ __forceinline__ int flag_load(const int *p) {
    return __hip_atomic_load(gmem(const_cast<int *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void flag_store(int *p, int v) {
    __hip_atomic_store(gmem(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-thread wait state.
struct Wait {
    int *err;
    unsigned polls;
    bool ok;
};

__device__ __forceinline__ Wait waiter(int *err) { return Wait{err, 0u, true}; }

// Pause between polls; false once the wait must stop (error or time limit).
__device__ __forceinline__ bool backoff(Wait &w) {
    if (!w.ok) return false;
    __builtin_amdgcn_s_sleep(2);
    ++w.polls;
    if ((w.polls & 255) == 0) {
        if (flag_load(w.err)) w.ok = false;
        else if (w.polls > kSpinLimit) {
            flag_store(w.err, 1);
            w.ok = false;
        }
    }
    return w.ok;
}

__device__ __forceinline__ float get(const uint64_t *p, unsigned ep, Wait &w) {
    uint64_t c = peek(p);
    while ((unsigned)(c >> 32) != ep && backoff(w)) c = peek(p);
    return __uint_as_float((unsigned)c);
}

__device__ __forceinline__ float2 get2(const uint64_t *base, int i, unsigned ep, Wait &w) {
    u64x2 c = peek2(base, i);
    while (((unsigned)(c.x >> 32) != ep || (unsigned)(c.y >> 32) != ep) && backoff(w)) c = peek2(base, i);
    return make_float2(__uint_as_float((unsigned)c.x), __uint_as_float((unsigned)c.y));
}

// Block-uniform result of the block's waits (all threads must call).
__device__ __forceinline__ bool all_ok(const Wait &w) { return !__syncthreads_or(!w.ok); }

// Read n cell pairs x[0..2n) into xs (FP32), lane `me` of `lanes` taking pairs
// me, me+lanes, ...: B pairs per lane in flight per round, and the whole batch
// is read again until every pair carries epoch ep.  Returns the lane's sum of
// squares of what it read (for an RMSNorm prologue).
template <int B>
__device__ __forceinline__ float read_pairs(const uint64_t *x, int n, unsigned ep, float *xs, int me, int lanes,
                                            Wait &w) {
    float ss = 0.0f;
    for (int base = me; base < n; base += lanes * B) {
        u64x2 c[B];
        bool ready;
        do {
#pragma unroll
            for (int i = 0; i < B; ++i) c[i] = peek2(x, 2 * (base + i * lanes), 2 * n);
            ready = true;
#pragma unroll
            for (int i = 0; i < B; ++i)
                ready &= base + i * lanes >= n ||
                         ((unsigned)(c[i].x >> 32) == ep && (unsigned)(c[i].y >> 32) == ep);
        } while (!ready && backoff(w));
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const int idx = base + i * lanes;
            if (idx < n) {
                const float a = __uint_as_float((unsigned)c[i].x), b = __uint_as_float((unsigned)c[i].y);
                xs[2 * idx] = a;
                xs[2 * idx + 1] = b;
                ss = fmaf(a, a, ss);
                ss = fmaf(b, b, ss);
            }
        }
    }
    return ss;
}

// Progress words: one 32-bit word per producer holds the epoch of the last
// phase whose outputs it has stored.  Epochs only grow within a sequence, so
// "word >= epoch" means the producer is done with that phase.  They are a
// cheap hint that the cells are there; the cells' own epochs stay the check.
__device__ __forceinline__ void mark(unsigned *p, unsigned ep) {
    __hip_atomic_store(gmem(p), ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned word(const unsigned *p) {
    return __hip_atomic_load(gmem(const_cast<unsigned *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until at least n - slack of words[0..n) reach ep.  Only the first wave
// of the caller polls (lane `me` < 64 takes words me, me+64, ...; 16 each in
// flight per round) and it pauses briefly between rounds (64-cycle pauses
// measured faster than longer ones; the step kernel spreads the workgroups'
// polls over several copies of its words).
__device__ __forceinline__ void wait_words(const unsigned *words, int n, unsigned ep, int me, int slack, Wait &w) {
    constexpr int B = 16;
    if (me >= kWave) return;
    bool done;
    do {
        int ready = 0;
        for (int base = me; base < n; base += kWave * B) {
#pragma unroll
            for (int i = 0; i < B; ++i) {
                const int idx = base + i * kWave;
                ready += idx < n && word(words + idx) >= ep;
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ready += __shfl_xor(ready, off);
        done = ready >= n - slack;
        if (!done) __builtin_amdgcn_s_sleep(1);
    } while (!done && backoff(w));
}

}  // namespace ll
}  // namespace mr
