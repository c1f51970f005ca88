// Host-side helpers shared by the library's translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

namespace yabt {

// Per-thread message of the last rejected call (yabt_last_error).
char* error_buffer();
constexpr size_t ERROR_LEN = 512;

inline int fail(int code, const char* msg) {
    snprintf(error_buffer(), ERROR_LEN, "%s", msg);
    return code;
}

inline int hip_fail(hipError_t e, const char* what) {
    snprintf(error_buffer(), ERROR_LEN, "%s: %s", what, hipGetErrorString(e));
    return -100;
}

inline int launch_status(const char* what) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_fail(e, what);
}

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

inline int launch_grid(int64_t work, int per_block, int cap) {
    int64_t g = (work + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int)g;
}

// Sequential carve of one workspace; with base == nullptr only sizes are summed.
struct Carve {
    char* base;
    size_t off;
    template <typename T>
    T* take(size_t count) {
        off = align_up(off, 256);
        T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
        off += count * sizeof(T);
        return p;
    }
};

}  // namespace yabt
