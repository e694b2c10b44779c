// Devices, contexts, errors and device memory (reference: opencl.py:14-217).
#include <cstdio>
#include <cstring>
#include <string>

#include "attention.h"
#include "common.h"

namespace mr {

static thread_local std::string g_error;

void set_error(const std::string &msg) { g_error = msg; }

int fail(int code, const std::string &msg) {
    g_error = msg;
    return code;
}

// Size classes: 256 B granularity up to 1 MiB, then 64 KiB granularity.  Blocks
// are recycled within a context and returned to HIP when it is destroyed.
static size_t size_class(size_t bytes) {
    if (bytes == 0) bytes = 1;
    size_t g = bytes <= (1u << 20) ? 256 : (64u << 10);
    return (bytes + g - 1) / g * g;
}

int ctx_alloc(mr_ctx *ctx, size_t bytes, void **ptr) {
    size_t cls = size_class(bytes);
    auto it = ctx->free_blocks.find(cls);
    if (it != ctx->free_blocks.end() && !it->second.empty()) {
        *ptr = it->second.back();
        it->second.pop_back();
        ctx->live[*ptr] = cls;
        return MR_OK;
    }
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, cls);
    if (e != hipSuccess) {
        // Give cached blocks back and try once more.
        hipStreamSynchronize(ctx->stream);
        for (auto &kv : ctx->free_blocks)
            for (void *q : kv.second) hipFree(q);
        ctx->free_blocks.clear();
        (void)hipGetLastError();
        e = hipMalloc(&p, cls);
        if (e != hipSuccess)
            return fail(MR_ERR_NOMEM, "allocate " + std::to_string(bytes) + " bytes failed (HIP error " +
                                          std::to_string((int)e) + ": " + hipGetErrorString(e) + ")");
    }
    ctx->live[p] = cls;
    *ptr = p;
    return MR_OK;
}

void ctx_release(mr_ctx *ctx, void *ptr) {
    auto it = ctx->live.find(ptr);
    if (it == ctx->live.end()) return;
    ctx->free_blocks[it->second].push_back(ptr);
    ctx->live.erase(it);
}

void ctx_retain(mr_ctx *ctx) { ++ctx->refs; }

void ctx_unref(mr_ctx *ctx) {
    if (--ctx->refs > 0) return;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    for (auto &kv : ctx->free_blocks)
        for (void *p : kv.second) hipFree(p);
    for (auto &kv : ctx->live) hipFree(kv.first);
    hipStreamDestroy(ctx->stream);
    delete ctx;
}

}  // namespace mr

using namespace mr;

extern "C" {

const char *mr_last_error(void) { return g_error.c_str(); }

int mr_device_count(int *count) {
    MR_REQUIRE(count, "mr_device_count: null output");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice) {
        *count = 0;
        return MR_OK;
    }
    MR_HIP(e, "enumerate HIP devices");
    *count = n;
    return MR_OK;
}

int mr_device_get_info(int device, mr_device_info *out) {
    MR_REQUIRE(out, "mr_device_get_info: null output");
    hipDeviceProp_t p;
    MR_HIP(hipGetDeviceProperties(&p, device), "query device properties");
    std::memset(out, 0, sizeof(*out));
    // Some drivers leave the marketing name empty; name the device by its ISA then.
    if (p.name[0]) std::strncpy(out->name, p.name, sizeof(out->name) - 1);
    else std::snprintf(out->name, sizeof(out->name), "AMD GPU %.48s", p.gcnArchName);
    std::strncpy(out->arch, p.gcnArchName, sizeof(out->arch) - 1);
    out->memory_bytes = (int64_t)p.totalGlobalMem;
    // HIP has no per-allocation cap query; a single hipMalloc may use all free HBM.
    out->max_allocation_bytes = (int64_t)p.totalGlobalMem;
    out->compute_units = p.multiProcessorCount;
    out->pci_bus_id = p.pciBusID;
    out->clock_khz = p.clockRate;
    out->memory_clock_khz = p.memoryClockRate;
    out->memory_bus_width = p.memoryBusWidth;
    return MR_OK;
}

int mr_ctx_create(int device, mr_ctx **out) {
    MR_REQUIRE(out, "mr_ctx_create: null output");
    int n = 0;
    MR_TRY(mr_device_count(&n));
    if (device < 0 || device >= n)
        return fail(MR_ERR_INVALID, "No matching HIP GPU device " + std::to_string(device) + " (" +
                                        std::to_string(n) + " visible). No CPU fallback.");
    MR_HIP(hipSetDevice(device), "select device");
    hipDeviceProp_t p;
    MR_HIP(hipGetDeviceProperties(&p, device), "query device properties");
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(MR_ERR_INVALID, std::string("device ") + p.gcnArchName +
                                        " is not gfx950 (MI355X); this library carries gfx950 code only");
    void *scratch = nullptr;
    MR_TRY(static_scratch_address(device, &scratch));
    mr_ctx *ctx = new mr_ctx();
    ctx->device = device;
    ctx->scratch = scratch;
    ctx->max_alloc = (int64_t)p.totalGlobalMem;
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        MR_HIP(e, "create stream");
    }
    *out = ctx;
    return MR_OK;
}

int mr_ctx_destroy(mr_ctx *ctx) {
    if (!ctx) return MR_OK;
    ctx_unref(ctx);
    return MR_OK;
}

int mr_sync(mr_ctx *ctx) {
    MR_REQUIRE(ctx, "mr_sync: null context");
    MR_HIP(hipStreamSynchronize(ctx->stream), "finish queue");
    return MR_OK;
}

int mr_alloc(mr_ctx *ctx, size_t bytes, void **ptr) {
    MR_REQUIRE(ctx && ptr, "mr_alloc: null argument");
    if ((int64_t)bytes > ctx->max_alloc)
        return fail(MR_ERR_NOMEM, "Buffer needs " + std::to_string(bytes) + " bytes, above device memory " +
                                      std::to_string(ctx->max_alloc));
    return ctx_alloc(ctx, bytes, ptr);
}

int mr_free(mr_ctx *ctx, void *ptr) {
    MR_REQUIRE(ctx, "mr_free: null context");
    if (ptr) ctx_release(ctx, ptr);
    return MR_OK;
}

int mr_h2d(mr_ctx *ctx, void *dst, const void *src, size_t bytes) {
    MR_REQUIRE(ctx && (bytes == 0 || (dst && src)), "mr_h2d: null argument");
    if (!bytes) return MR_OK;
    MR_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "upload tensor");
    MR_HIP(hipStreamSynchronize(ctx->stream), "upload tensor");
    return MR_OK;
}

int mr_d2h(mr_ctx *ctx, void *dst, const void *src, size_t bytes) {
    MR_REQUIRE(ctx && (bytes == 0 || (dst && src)), "mr_d2h: null argument");
    if (!bytes) return MR_OK;
    MR_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "read tensor");
    MR_HIP(hipStreamSynchronize(ctx->stream), "read tensor");
    return MR_OK;
}

int mr_d2d(mr_ctx *ctx, void *dst, const void *src, size_t bytes) {
    MR_REQUIRE(ctx && (bytes == 0 || (dst && src)), "mr_d2d: null argument");
    if (!bytes) return MR_OK;
    MR_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream), "copy tensor");
    return MR_OK;
}

int mr_debug_fail_next(mr_ctx *ctx) {
    MR_REQUIRE(ctx, "mr_debug_fail_next: null context");
    ctx->fail_next = true;
    return MR_OK;
}

}  // extern "C"
