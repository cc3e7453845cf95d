// context.hip — library context, error reporting and device-memory plumbing of libtdgs.
#include <stdarg.h>
#include <stdio.h>

#include <vector>

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

int read_counters(tdgs_ctx* ctx, hipStream_t stream) {
    TDGS_HIP(hipMemcpyAsync(ctx->h_counters, ctx->d_counters, sizeof(int64_t) * kCounters,
                            hipMemcpyDeviceToHost, stream));
    TDGS_HIP(hipStreamSynchronize(stream));
    const uint32_t flags = (uint32_t)ctx->h_counters[kErrSlot];
    if (flags != 0) {
        TDGS_HIP(hipMemsetAsync(ctx->d_counters + kErrSlot, 0, sizeof(int64_t), stream));
        TDGS_HIP(hipStreamSynchronize(stream));
        ctx->h_counters[kErrSlot] = 0;
        if (flags & kErrSortCounts)
            set_error("a radix sort on this context found counts that disagree with its keys; the sorted "
                      "lists of that call are incomplete (device flags 0x%x)", flags);
        else
            set_error("device error flags 0x%x raised on this context", flags);
        return TDGS_ERR_DEVICE;
    }
    return TDGS_OK;
}

// ---- stage profiler -------------------------------------------------------------------

namespace {
struct Profiler {
    bool on = false;
    int32_t max_records = 0;
    std::vector<hipEvent_t> events;   // pool, two per record
    std::vector<int> stages;          // stage of each started record
    int open[TDGS_STAGE_COUNT];       // index of the open record per stage, -1 if none
};
thread_local Profiler g_prof;
}  // namespace

void profile_mark(int stage, bool start, hipStream_t stream) {
    Profiler& p = g_prof;
    if (!p.on || stage < 0 || stage >= TDGS_STAGE_COUNT) return;
    if (start) {
        const size_t rec = p.stages.size();
        if ((int32_t)rec >= p.max_records) return;
        p.stages.push_back(stage);
        p.open[stage] = (int)rec;
        (void)hipEventRecord(p.events[2 * rec], stream);
    } else {
        const int rec = p.open[stage];
        if (rec < 0) return;
        p.open[stage] = -1;
        (void)hipEventRecord(p.events[2 * rec + 1], stream);
    }
}

}  // namespace tdgs

namespace tdgs {

// Makes `device` current for the scope and restores the caller's current device after it.
struct DeviceScope {
    int prev = -1;
    hipError_t err;
    explicit DeviceScope(int device) {
        err = hipGetDevice(&prev);
        if (err == hipSuccess) err = hipSetDevice(device);
    }
    ~DeviceScope() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

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
    DeviceScope scope(device);   // the caller's current device is left as it was
    TDGS_HIP(scope.err);
    tdgs_ctx* c = new tdgs_ctx();
    c->device = device;
    hipError_t e = hipMalloc((void**)&c->d_counters, sizeof(int64_t) * (kCounters + kMonitor));
    if (e == hipSuccess) e = hipHostMalloc((void**)&c->h_counters, sizeof(int64_t) * kCounters);
    if (e == hipSuccess) e = hipMemset(c->d_counters, 0, sizeof(int64_t) * (kCounters + kMonitor));
    if (e == hipSuccess)
        e = hipHostMalloc((void**)&c->h_monitor, sizeof(int64_t) * kMonitor, hipHostMallocCoherent | hipHostMallocMapped);
    if (e == hipSuccess) e = hipHostGetDevicePointer((void**)&c->h_monitor_dev, c->h_monitor, 0);
    if (e != hipSuccess) {
        if (c->d_counters) (void)hipFree(c->d_counters);
        if (c->h_counters) (void)hipHostFree(c->h_counters);
        if (c->h_monitor) (void)hipHostFree(c->h_monitor);
        delete c;
        return hip_fail(e, "tdgs_ctx_create", __FILE__, __LINE__);
    }
    for (int k = 0; k < kMonitor; ++k) c->h_monitor[k] = 0;
    *ctx_out = c;
    return TDGS_OK;
}

int tdgs_ctx_destroy(tdgs_ctx* ctx) {
    if (!ctx) return TDGS_OK;
    DeviceScope scope(ctx->device);   // wait for the context's device, not the caller's current one
    TDGS_HIP(scope.err);
    TDGS_HIP(hipDeviceSynchronize());
    TDGS_HIP(hipFree(ctx->d_counters));
    TDGS_HIP(hipHostFree(ctx->h_counters));
    TDGS_HIP(hipHostFree(ctx->h_monitor));
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

int tdgs_profile_begin(int32_t max_records) {
    TDGS_REQUIRE(max_records > 0, "max_records must be positive");
    Profiler& p = g_prof;
    while ((int32_t)p.events.size() < 2 * max_records) {
        hipEvent_t e;
        TDGS_HIP(hipEventCreate(&e));
        p.events.push_back(e);
    }
    p.max_records = max_records;
    p.stages.clear();
    for (int i = 0; i < TDGS_STAGE_COUNT; ++i) p.open[i] = -1;
    p.on = true;
    return TDGS_OK;
}

int tdgs_profile_end(double* ms_out, int64_t* executions_out) {
    Profiler& p = g_prof;
    TDGS_REQUIRE(p.on, "profiler not enabled");
    p.on = false;
    for (int i = 0; i < TDGS_STAGE_COUNT; ++i) {
        if (ms_out) ms_out[i] = 0.0;
        if (executions_out) executions_out[i] = 0;
    }
    for (size_t r = 0; r < p.stages.size(); ++r) {
        TDGS_HIP(hipEventSynchronize(p.events[2 * r + 1]));
        float ms = 0.0f;
        TDGS_HIP(hipEventElapsedTime(&ms, p.events[2 * r], p.events[2 * r + 1]));
        if (ms_out) ms_out[p.stages[r]] += ms;
        if (executions_out) executions_out[p.stages[r]] += 1;
    }
    p.stages.clear();
    return TDGS_OK;
}

int tdgs_stream_synchronize(void* stream) {
    TDGS_HIP(hipStreamSynchronize((hipStream_t)stream));
    return TDGS_OK;
}

int tdgs_stream_create(void** stream_out) {
    TDGS_REQUIRE(stream_out, "null output");
    *stream_out = nullptr;
    hipStream_t s;
    TDGS_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));   // default priority
    *stream_out = (void*)s;
    return TDGS_OK;
}

int tdgs_stream_destroy(void* stream) {
    TDGS_REQUIRE(stream, "null stream (the default stream is not destroyed)");
    TDGS_HIP(hipStreamDestroy((hipStream_t)stream));
    return TDGS_OK;
}

int tdgs_event_create(void** event_out) {
    TDGS_REQUIRE(event_out, "null output");
    *event_out = nullptr;
    hipEvent_t e;
    TDGS_HIP(hipEventCreate(&e));
    *event_out = (void*)e;
    return TDGS_OK;
}

int tdgs_event_destroy(void* event) {
    TDGS_REQUIRE(event, "null event");
    TDGS_HIP(hipEventDestroy((hipEvent_t)event));
    return TDGS_OK;
}

int tdgs_event_record(void* event, void* stream) {
    TDGS_REQUIRE(event, "null event");
    TDGS_HIP(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
    return TDGS_OK;
}

int tdgs_stream_wait_event(void* stream, void* event) {
    TDGS_REQUIRE(event, "null event");
    TDGS_HIP(hipStreamWaitEvent((hipStream_t)stream, (hipEvent_t)event, 0));
    return TDGS_OK;
}

int tdgs_event_synchronize(void* event) {
    TDGS_REQUIRE(event, "null event");
    TDGS_HIP(hipEventSynchronize((hipEvent_t)event));
    return TDGS_OK;
}

int tdgs_event_elapsed_ms(void* start, void* stop, float* ms_out) {
    TDGS_REQUIRE(start && stop && ms_out, "null arguments");
    TDGS_HIP(hipEventElapsedTime(ms_out, (hipEvent_t)start, (hipEvent_t)stop));
    return TDGS_OK;
}

int tdgs_host_malloc(void** ptr_out, size_t bytes) {
    TDGS_REQUIRE(ptr_out, "null output");
    *ptr_out = nullptr;
    TDGS_HIP(hipHostMalloc(ptr_out, bytes > 0 ? bytes : 1, hipHostMallocDefault));
    return TDGS_OK;
}

int tdgs_host_free(void* ptr) {
    if (ptr) TDGS_HIP(hipHostFree(ptr));
    return TDGS_OK;
}

int tdgs_ctx_check(tdgs_ctx* ctx, void* stream) {
    TDGS_REQUIRE(ctx, "null ctx");
    return read_counters(ctx, (hipStream_t)stream);
}

int tdgs_ctx_frame_monitor(tdgs_ctx* ctx, const int64_t** monitor_out) {
    TDGS_REQUIRE(ctx && monitor_out, "null arguments");
    *monitor_out = ctx->h_monitor;
    return TDGS_OK;
}

}  // extern "C"
