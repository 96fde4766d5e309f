/* wzy_runtime.h -- device / memory / stream plumbing of libwzy_amd.
 *
 * These entry points have no counterpart in the reference (its engine calls the CUDA runtime
 * directly).  They exist so that a host in any language can allocate device buffers, move data
 * and order work for the kernel and stage entry points without linking a second GPU runtime into
 * the process: a process must use exactly one HIP/HSA runtime, so callers such as the Python test
 * and benchmark harness use these instead of a framework's allocator.
 * All return WZY_OK or a negative WZY_E* code (see wzy_kernels.h).
 */
#ifndef WZY_RUNTIME_H
#define WZY_RUNTIME_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

int wzy_dev_count(int* n);
int wzy_dev_set(int dev);
int wzy_dev_name(int dev, char* buf, int buflen);     /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
int wzy_mem_info(size_t* free_bytes, size_t* total_bytes);
int wzy_dev_malloc(void** p, size_t bytes);
int wzy_dev_free(void* p);
/* host <-> device copies; stream NULL = synchronous on the null stream */
int wzy_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int wzy_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int wzy_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int wzy_memset(void* dst, int value, size_t bytes, void* stream);
int wzy_stream_create(void** stream);
int wzy_stream_destroy(void* stream);
int wzy_stream_sync(void* stream);
int wzy_device_sync(void);
/* pinned host memory (hipHostMalloc) for asynchronous copies */
int wzy_host_malloc(void** p, size_t bytes);
int wzy_host_free(void* p);

#ifdef __cplusplus
}
#endif
#endif /* WZY_RUNTIME_H */
