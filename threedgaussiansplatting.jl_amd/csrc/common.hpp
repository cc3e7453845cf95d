// common.hpp — error reporting, launch helpers and wave-level primitives shared by the
// gfx950 kernels of libtdgs.
#pragma once

#include <hip/hip_runtime.h>

#include <stddef.h>
#include <stdint.h>

#include "tdgs_math.hpp"

namespace tdgs {

// Last error message of the calling host thread (tdgs_last_error()).
void set_error(const char* fmt, ...);
int hip_fail(hipError_t e, const char* what, const char* file, int line);

#define TDGS_HIP(call)                                                              \
    do {                                                                            \
        hipError_t e_ = (call);                                                     \
        if (e_ != hipSuccess) return ::tdgs::hip_fail(e_, #call, __FILE__, __LINE__); \
    } while (0)

#define TDGS_LAUNCHED() TDGS_HIP(hipGetLastError())

#define TDGS_REQUIRE(cond, ...)               \
    do {                                      \
        if (!(cond)) {                        \
            ::tdgs::set_error(__VA_ARGS__);   \
            return TDGS_ERR_INVALID;          \
        }                                     \
    } while (0)

#define TDGS_TRY(expr)              \
    do {                            \
        int r_ = (expr);            \
        if (r_ != TDGS_OK) return r_; \
    } while (0)

constexpr int kWave = 64;

// Workgroups are dealt to the 8 XCDs in turn by linear id (workgroup i runs on XCD i mod 8),
// each XCD with its own L2.
constexpr int kXcds = 8;
// XCD-aware work order: the item (0-based) of workgroup i of a grid of n workgroups, XCD k
// taking the contiguous items k q .. k q + q - 1 (q = n / 8) in order, so that neighbouring
// items, which read much of the same data, meet in one L2. A bijection on the first 8 q ids;
// the remaining n mod 8 keep their own index.
__device__ __forceinline__ int xcd_band_item(int i, int n) {
    const int q = n / kXcds;
    return i < kXcds * q ? (i % kXcds) * q + i / kXcds : i;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t x, size_t a = 256) { return (x + a - 1) / a * a; }

// Bump allocator over a caller-provided scratch buffer.
struct Arena {
    char* base;
    size_t size;
    size_t used;
    Arena(void* p, size_t n) : base((char*)p), size(n), used(0) {}
    template <class T>
    T* take(int64_t count) {
        const size_t bytes = align_up((size_t)(count > 0 ? count : 1) * sizeof(T));
        if (used + bytes > size) return nullptr;
        T* p = (T*)(base + used);
        used += bytes;
        return p;
    }
};

// Counting-only twin of Arena: how many bytes a sequence of take() calls needs.
struct ArenaSize {
    size_t used = 0;
    template <class T>
    void take(int64_t count) { used += align_up((size_t)(count > 0 ? count : 1) * sizeof(T)); }
};

__device__ __forceinline__ uint64_t lanemask_lt() {
    return (1ull << __lane_id()) - 1ull;
}

// Wavefront vote straight from the lane mask (a scalar test, no vector compare).
__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// Device-wide scan over n int32 items produced by a functor, with int64 running sums
// (scan.hip). In(i) returns item i; Out(i, inclusive, item) consumes the result.
size_t scan_temp_bytes_internal(int64_t n);

}  // namespace tdgs
