// Host-side helpers shared by the library's translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <chrono>

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

// A host spin on flags in mapped memory, which a kernel of the stream
// writes: stream_check() says when to ask the stream whether it failed or
// ended without writing them.  hipStreamQuery on a stream whose last kernel
// has no completion signal enqueues a marker behind it, and each marker held
// the next kernel ~5.7 us on the device; so the stream is asked only once the
// wait has lasted SPIN_CHECK_MS, which no healthy round takes.
constexpr int SPIN_CHECK_MS = 50;
struct SpinWait {
    std::chrono::steady_clock::time_point t0 = std::chrono::steady_clock::now();
    uint64_t spin = 0;
    bool stream_check() {
        if ((++spin & 1023) != 0) return false;
        const auto dt = std::chrono::steady_clock::now() - t0;
        return dt >= std::chrono::milliseconds(SPIN_CHECK_MS);
    }
};

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

inline int launch_grid(int64_t work, int per_block, int cap) {
    int64_t g = (work + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int)g;
}

// Pinned host buffers reused across calls.  hipHostMalloc / hipHostFree
// cost tens of microseconds and synchronise the device, which a tree of a
// millisecond cannot afford; a buffer is held by one call at a time, so
// concurrent calls (from several host threads) each get their own.  Buffers
// are kept per (device, flags) and never freed before the process ends.
int pinned_take(size_t bytes, unsigned flags, void** out, int* device);
void pinned_give(void* p, size_t bytes, unsigned flags, int device);

// Scoped hold of a pooled buffer; the holder's destructor returns it.
struct PinnedHold {
    void* p = nullptr;
    size_t bytes = 0;
    unsigned flags = 0;
    int device = 0;
    int take(size_t b, unsigned f) {
        bytes = b;
        flags = f;
        return pinned_take(b, f, &p, &device);
    }
    ~PinnedHold() {
        if (p) pinned_give(p, bytes, flags, device);
    }
};

// yabt_hist's work on a caller's workspace of yabt_hist_workspace_bytes()
// bytes (ops.hip); `who` names the entry point in error messages.
int hist_enqueue(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm, const float* grad,
                 const float* hess, int64_t n, int F, const uint32_t* rows, int64_t m, void* workspace, int64_t* out,
                 int32_t* out_shifts, hipStream_t stream, const char* who);

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
