// wzy_host.h -- host-side helpers of the library: error reporting, HIP checks, small utilities.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <string>

#include "../../include/wzy_kernels.h"

namespace wzy {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Fallible-call helpers: return a WZY_E* code from the enclosing function on failure.
#define WZY_HIP_TRY(expr)                                                                       \
    do {                                                                                        \
        hipError_t e_ = (expr);                                                                 \
        if (e_ != hipSuccess) {                                                                 \
            ::wzy::set_error("%s:%d: %s -> %s", __FILE__, __LINE__, #expr, hipGetErrorString(e_)); \
            return WZY_EHIP;                                                                    \
        }                                                                                       \
    } while (0)

#define WZY_REQUIRE(cond, ...)              \
    do {                                    \
        if (!(cond)) {                      \
            ::wzy::set_error(__VA_ARGS__);  \
            return WZY_EINVAL;              \
        }                                   \
    } while (0)

#define WZY_TRY(expr)              \
    do {                           \
        int r_ = (expr);           \
        if (r_ != WZY_OK) return r_; \
    } while (0)

// Check the launch that was just enqueued.
#define WZY_LAUNCH_CHECK() WZY_HIP_TRY(hipGetLastError())

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Bump allocator over a caller-provided workspace.
struct Arena {
    char* base;
    size_t cap, off = 0;
    Arena(void* b, size_t c) : base((char*) b), cap(c) {}
    template <class T>
    T* take(size_t n) {
        off = align_up(off, 256);
        T* p = (T*) (base + off);
        off += n * sizeof(T);
        return p;
    }
    bool ok() const { return off <= cap; }
};

}  // namespace wzy
