// runtime.hip -- device, memory and stream plumbing behind include/wzy_runtime.h.
#include <string.h>

#include "../../include/wzy_runtime.h"
#include "wzy_host.h"

using namespace wzy;

extern "C" int wzy_dev_count(int* n) {
    WZY_REQUIRE(n, "wzy_dev_count: null");
    *n = 0;
    const hipError_t e = hipGetDeviceCount(n);
    if (e != hipSuccess) { *n = 0; (void) hipGetLastError(); }
    return WZY_OK;
}
extern "C" int wzy_dev_set(int dev) {
    WZY_HIP_TRY(hipSetDevice(dev));
    return WZY_OK;
}
extern "C" int wzy_dev_name(int dev, char* buf, int buflen) {
    WZY_REQUIRE(buf && buflen > 0, "wzy_dev_name: bad buffer");
    hipDeviceProp_t p;
    WZY_HIP_TRY(hipGetDeviceProperties(&p, dev));
    strncpy(buf, p.gcnArchName, (size_t) buflen - 1);
    buf[buflen - 1] = 0;
    return WZY_OK;
}
extern "C" int wzy_mem_info(size_t* free_bytes, size_t* total_bytes) {
    WZY_REQUIRE(free_bytes && total_bytes, "wzy_mem_info: null");
    WZY_HIP_TRY(hipMemGetInfo(free_bytes, total_bytes));
    return WZY_OK;
}
extern "C" int wzy_dev_malloc(void** p, size_t bytes) {
    WZY_REQUIRE(p, "wzy_dev_malloc: null");
    *p = nullptr;
    if (bytes == 0) return WZY_OK;
    if (hipMalloc(p, bytes) != hipSuccess) {
        (void) hipGetLastError();
        *p = nullptr;
        set_error("wzy_dev_malloc: hipMalloc(%zu) failed", bytes);
        return WZY_ENOMEM;
    }
    return WZY_OK;
}
extern "C" int wzy_dev_free(void* p) {
    if (p) WZY_HIP_TRY(hipFree(p));
    return WZY_OK;
}
static int copy(void* dst, const void* src, size_t n, hipMemcpyKind k, void* stream) {
    if (n == 0) return WZY_OK;
    WZY_REQUIRE(dst && src, "memcpy: null pointer");
    if (stream) WZY_HIP_TRY(hipMemcpyAsync(dst, src, n, k, as_stream(stream)));
    else WZY_HIP_TRY(hipMemcpy(dst, src, n, k));
    return WZY_OK;
}
extern "C" int wzy_memcpy_h2d(void* dst, const void* src, size_t n, void* s) { return copy(dst, src, n, hipMemcpyHostToDevice, s); }
extern "C" int wzy_memcpy_d2h(void* dst, const void* src, size_t n, void* s) { return copy(dst, src, n, hipMemcpyDeviceToHost, s); }
extern "C" int wzy_memcpy_d2d(void* dst, const void* src, size_t n, void* s) { return copy(dst, src, n, hipMemcpyDeviceToDevice, s); }
extern "C" int wzy_memset(void* dst, int v, size_t n, void* stream) {
    if (n == 0) return WZY_OK;
    WZY_REQUIRE(dst, "wzy_memset: null pointer");
    if (stream) WZY_HIP_TRY(hipMemsetAsync(dst, v, n, as_stream(stream)));
    else WZY_HIP_TRY(hipMemset(dst, v, n));
    return WZY_OK;
}
extern "C" int wzy_stream_create(void** s) {
    WZY_REQUIRE(s, "wzy_stream_create: null");
    hipStream_t st;
    WZY_HIP_TRY(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    *s = st;
    return WZY_OK;
}
extern "C" int wzy_stream_destroy(void* s) {
    if (s) WZY_HIP_TRY(hipStreamDestroy(as_stream(s)));
    return WZY_OK;
}
extern "C" int wzy_stream_sync(void* s) {
    WZY_HIP_TRY(hipStreamSynchronize(as_stream(s)));
    return WZY_OK;
}
extern "C" int wzy_device_sync(void) {
    WZY_HIP_TRY(hipDeviceSynchronize());
    return WZY_OK;
}
extern "C" int wzy_host_malloc(void** p, size_t bytes) {
    WZY_REQUIRE(p, "wzy_host_malloc: null");
    WZY_HIP_TRY(hipHostMalloc(p, bytes, hipHostMallocDefault));
    return WZY_OK;
}
extern "C" int wzy_host_free(void* p) {
    if (p) WZY_HIP_TRY(hipHostFree(p));
    return WZY_OK;
}
