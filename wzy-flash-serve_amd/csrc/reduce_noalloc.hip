// reduce_noalloc.hip -- allocation-free variant of the vocabulary top-16 reduction, for callers that
// cannot call hipMalloc (code under HIP graph capture, tight serving loops, harnesses that forbid it).
//
// The reduction (row_topr_kernel, reduce.hip) needs a scratch of row arrival counters and per-chunk
// partial results.  Here that scratch is a file-scope device array of a fixed size, `scratch`.  Its
// host-side name is only a stand-in for the symbol: the device address is looked up once per device
// with hipGetSymbolAddress (each GPU holds its own copy) and only that address is ever passed to a
// kernel.  The counters start at zero (a fill kernel on the first call on a device) and every launch
// leaves them at zero again.  All calls on one device share the array, so calls that overlap in time
// on one device race.
#include <mutex>

#include "wzy_device.h"
#include "wzy_host.h"
#include "wzy_reduce.h"

using namespace wzy;

namespace {
constexpr int NA_MAX_T = WZY_MAX_W;          // rows per call
constexpr int NA_MAX_VOCAB = 262144;         // logits per row (the top-16 merge holds 128 chunks x 16)
constexpr int NA_MAX_DEVICES = 64;
// reduce_ws_bytes(NA_MAX_VOCAB, NA_MAX_T): 256 B of counters + 8 rows x 128 chunks x 16 x (4 + 4) B
constexpr size_t NA_SCRATCH_BYTES = 256 + (size_t) NA_MAX_T * (NA_MAX_VOCAB / 2048) * 16 * 8;   // 131,328
}  // namespace

static __device__ __align__(256) unsigned char scratch[NA_SCRATCH_BYTES];

__global__ void na_zero_words_kernel(unsigned* __restrict__ p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

static std::mutex na_mu;
static void* na_ptr[NA_MAX_DEVICES] = {nullptr};

// Device address of `scratch` on the current device; the first call on a device looks it up and
// enqueues the clear of the counter words on `st`.
static int na_scratch(hipStream_t st, void** out) {
    int dev = 0;
    WZY_HIP_TRY(hipGetDevice(&dev));
    WZY_REQUIRE(dev >= 0 && dev < NA_MAX_DEVICES, "wzy_row_top16_noalloc: device id %d out of range", dev);
    std::lock_guard<std::mutex> g(na_mu);
    if (!na_ptr[dev]) {
        void* p = nullptr;
        WZY_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        WZY_REQUIRE(p, "wzy_row_top16_noalloc: no device address for the scratch array");
        hipLaunchKernelGGL(na_zero_words_kernel, dim3(1), dim3(64), 0, st, (unsigned*) p, 64);
        WZY_LAUNCH_CHECK();
        na_ptr[dev] = p;
    }
    *out = na_ptr[dev];
    return WZY_OK;
}

extern "C" int wzy_row_top16_noalloc(const float* logits, int nvocab, int T, int* out_greedy, float* top_v,
                                     int* top_i, void* stream) {
    WZY_REQUIRE(logits, "wzy_row_top16_noalloc: null logits");
    WZY_REQUIRE(T >= 1 && T <= NA_MAX_T, "wzy_row_top16_noalloc: T = %d outside [1, %d]", T, NA_MAX_T);
    WZY_REQUIRE(nvocab >= 1 && nvocab <= NA_MAX_VOCAB,
                "wzy_row_top16_noalloc: nvocab = %d outside [1, %d] (the fixed scratch holds %zu bytes)", nvocab,
                NA_MAX_VOCAB, NA_SCRATCH_BYTES);
    WZY_REQUIRE(reduce_ws_bytes(nvocab, T) <= NA_SCRATCH_BYTES, "wzy_row_top16_noalloc: scratch too small");
    hipStream_t st = as_stream(stream);
    void* ws = nullptr;
    WZY_TRY(na_scratch(st, &ws));
    return launch_row_reduce(logits, nvocab, T, true, out_greedy, top_v, top_i, ws, st);
}
