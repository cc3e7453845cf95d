// context.hip — library context, error reporting and device-memory plumbing of libtdgs.
#include <stdarg.h>
#include <stdio.h>

#include "internal.hpp"

namespace tdgs {

static thread_local char g_error[1024] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

int hip_fail(hipError_t e, const char* what, const char* file, int line) {
    set_error("HIP error %d (%s) in %s at %s:%d", (int)e, hipGetErrorString(e), what, file, line);
    return TDGS_ERR_HIP;
}

int read_counters(tdgs_ctx* ctx, hipStream_t stream, int count) {
    TDGS_HIP(hipMemcpyAsync(ctx->h_counters, ctx->d_counters, sizeof(int64_t) * count,
                            hipMemcpyDeviceToHost, stream));
    TDGS_HIP(hipStreamSynchronize(stream));
    return TDGS_OK;
}

}  // namespace tdgs

using namespace tdgs;

extern "C" {

int tdgs_abi_version(void) { return TDGS_ABI_VERSION; }

const char* tdgs_last_error(void) { return g_error; }

int tdgs_ctx_create(int device, tdgs_ctx** ctx_out) {
    TDGS_REQUIRE(ctx_out != nullptr, "null output");
    *ctx_out = nullptr;
    int count = 0;
    TDGS_HIP(hipGetDeviceCount(&count));
    TDGS_REQUIRE(device >= 0 && device < count, "device %d out of range (%d devices)", device, count);
    TDGS_HIP(hipSetDevice(device));
    tdgs_ctx* c = new tdgs_ctx();
    c->device = device;
    hipError_t e = hipMalloc((void**)&c->d_counters, sizeof(int64_t) * kCounters);
    if (e == hipSuccess) e = hipHostMalloc((void**)&c->h_counters, sizeof(int64_t) * kCounters);
    if (e == hipSuccess) e = hipMemset(c->d_counters, 0, sizeof(int64_t) * kCounters);
    if (e != hipSuccess) {
        if (c->d_counters) (void)hipFree(c->d_counters);
        if (c->h_counters) (void)hipHostFree(c->h_counters);
        delete c;
        return hip_fail(e, "tdgs_ctx_create", __FILE__, __LINE__);
    }
    *ctx_out = c;
    return TDGS_OK;
}

int tdgs_ctx_destroy(tdgs_ctx* ctx) {
    if (!ctx) return TDGS_OK;
    TDGS_HIP(hipDeviceSynchronize());
    TDGS_HIP(hipFree(ctx->d_counters));
    TDGS_HIP(hipHostFree(ctx->h_counters));
    delete ctx;
    return TDGS_OK;
}

int tdgs_malloc(void** ptr_out, size_t bytes) {
    TDGS_REQUIRE(ptr_out, "null output");
    TDGS_HIP(hipMalloc(ptr_out, bytes > 0 ? bytes : 1));
    return TDGS_OK;
}

int tdgs_free(void* ptr) {
    if (ptr) TDGS_HIP(hipFree(ptr));
    return TDGS_OK;
}

int tdgs_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    TDGS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
    return TDGS_OK;
}

int tdgs_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    TDGS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
    return TDGS_OK;
}

int tdgs_memset(void* dst, int value, size_t bytes, void* stream) {
    TDGS_HIP(hipMemsetAsync(dst, value, bytes, (hipStream_t)stream));
    return TDGS_OK;
}

int tdgs_stream_synchronize(void* stream) {
    TDGS_HIP(hipStreamSynchronize((hipStream_t)stream));
    return TDGS_OK;
}

}  // extern "C"
