// Internal helpers shared by the library's translation units (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "miracle_hip.h"

namespace mr {

// ---------------------------------------------------------------- errors
void set_error(const std::string &msg);
int fail(int code, const std::string &msg);

#define MR_HIP(expr, what)                                                                        \
    do {                                                                                          \
        hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess)                                                                     \
            return ::mr::fail(MR_ERR_HIP, std::string(what) + " failed (HIP error " +             \
                                              std::to_string((int)e_) + ": " + hipGetErrorString(e_) + ")"); \
    } while (0)

#define MR_REQUIRE(cond, msg)                                                                     \
    do {                                                                                          \
        if (!(cond)) return ::mr::fail(MR_ERR_INVALID, msg);                                     \
    } while (0)

#define MR_TRY(call)                                                                              \
    do {                                                                                          \
        int rc_ = (call);                                                                         \
        if (rc_ != MR_OK) return rc_;                                                             \
    } while (0)

// Launch-error check after a kernel launch.
#define MR_LAUNCHED(what) MR_HIP(hipGetLastError(), what)

}  // namespace mr

// The context: one device, one stream, a caching allocator.
struct mr_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    int64_t max_alloc = 0;
    bool fail_next = false;
    // size -> free device blocks (all blocks of one size class)
    std::unordered_map<size_t, std::vector<void *>> free_blocks;
    std::unordered_map<void *, size_t> live;   // block -> size class
    // The caller's reference plus one per live model; the stream and the
    // blocks are released when the last one goes (mr_ctx_destroy and
    // mr_model_destroy may then come in either order).
    int refs = 1;
    void *scratch = nullptr;   // this device's static attention scratch (device address)
};

namespace mr {

int ctx_alloc(mr_ctx *ctx, size_t bytes, void **ptr);
void ctx_release(mr_ctx *ctx, void *ptr);
void ctx_retain(mr_ctx *ctx);
void ctx_unref(mr_ctx *ctx);

// ---------------------------------------------------------------- device helpers
constexpr int kWave = 64;

// Global-memory view of a pointer.  Pointers that a kernel reads out of memory
// (rather than receives as arguments) have no known address space, and the
// compiler then emits FLAT accesses, which wait on the LDS counter too and so
// serialize prefetched loads; these casts keep them GLOBAL.
#define MR_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ const MR_GLOBAL T *gmem(const T *p) {
    return (const MR_GLOBAL T *)p;
}
template <typename T>
__device__ __forceinline__ MR_GLOBAL T *gmem(T *p) {
    return (MR_GLOBAL T *)p;
}

// 16-byte load of four floats from global memory.
__device__ __forceinline__ float4 load_f4(const float *p) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    f32x4 v = *gmem((const f32x4 *)p);
    return make_float4(v.x, v.y, v.z, v.w);
}

// 16-byte load of base[i .. i+4) that is coherent across the device's L2
// caches (cache policy SC1 = agent scope): for data another workgroup wrote
// during this kernel.  `base` must be the same for the whole wave (it becomes
// a buffer resource, which lives in scalar registers); i varies per lane.
__device__ __forceinline__ float4 load_f4_coherent(const float *base, int i) {
    __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7fffffff, 0x00020000);
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    f32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, i * 4, 0, 16);
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
    return (float)h;
}

// Lane exchanges within rows of 16 lanes (DPP, no LDS round trip).
// Controls: quad_perm(1,0,3,2) = 0xB1, quad_perm(2,3,0,1) = 0x4E,
// row_half_mirror = 0x141, row_mirror = 0x140.  Callers keep every lane of
// the wave active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Sum (max) over each row of 16 lanes; every lane of the row receives it.
__device__ __forceinline__ float row_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    return v;
}

__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return v;
}

// Sum over the 64 lanes of a wave; every lane receives the total.
__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ float wave_sum(float v) {
    v = row_sum(v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = row_max(v);
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// v of lane l combined with v of lane l ^ 16 (l ^ 32), in VALU lane swaps
// (v_permlane16/32_swap: each returns the two halves of a lane pair, so both
// lanes of a pair compute the same commutative sum or max).
__device__ __forceinline__ float xor16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum within aligned groups of `width` lanes (width a power of two <= 64);
// every lane of a group receives its group's sum.
__device__ __forceinline__ float group_sum(float v, int width) {
    if (width >= 16) {
        v = row_sum(v);
        if (width >= 32) v = xor16_sum(v);
        if (width == 64) v = xor32_sum(v);
        return v;
    }
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Block-wide sum for blockDim.x == nthreads (multiple of 64, <= 1024); uses `scratch`
// of at least nthreads/64 floats; all threads receive the total.
__device__ __forceinline__ float block_sum(float v, float *scratch) {
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < waves; ++w) t += scratch[w];
    return t;
}

__device__ __forceinline__ float block_max(float v, float *scratch) {
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    v = wave_max(v);
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int w = 0; w < waves; ++w) t = fmaxf(t, scratch[w]);
    return t;
}

// RoPE of one pair at an FP32 angle pos*freq (kernels.cl:38-43).  cos/sin are
// taken in double and rounded once, which is within half an ulp of the exact
// value for every angle the models reach.
__device__ __forceinline__ void rope_pair(float &u, float &v, float pos, float freq) {
    float a = pos * freq;
    double ad = (double)a;
    float c = (float)cos(ad), s = (float)sin(ad);
    float nu = u * c - v * s;
    float nv = u * s + v * c;
    u = nu;
    v = nv;
}

// Rotation of one pair by a tabulated (cos, sin) (kernels.cl:43).
__device__ __forceinline__ void rope_rotate(float &u, float &v, float c, float s) {
    float nu = u * c - v * s;
    float nv = u * s + v * c;
    u = nu;
    v = nv;
}

// Workgroup barrier that orders LDS accesses only: global loads still in
// flight (weights prefetched into registers) stay in flight across it, where
// __syncthreads would first wait for every one of them.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Element j of a weight row of the given storage dtype, widened to FP32.
template <int DT>
__device__ __forceinline__ float load_w(const void *w, int64_t i) {
    if constexpr (DT == MR_F32) return ((const float *)w)[i];
    else if constexpr (DT == MR_BF16) return bf16_to_f32(((const uint16_t *)w)[i]);
    else return f16_to_f32(((const uint16_t *)w)[i]);
}

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------- shared launches
// y[rows, n] = x[rows, k] . W[n, k]^T with FP32 accumulation; dispatches a GEMV
// (rows == 1) or a tiled GEMM.  Used by the op-level ABI and by the engine.
int launch_linear(hipStream_t s, const float *x, const void *w, int dtype, float *y, int rows, int n, int k);

}  // namespace mr
