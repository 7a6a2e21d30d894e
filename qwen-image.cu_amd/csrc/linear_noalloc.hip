// linear_noalloc.hip — qimg_linear for callers that cannot allocate device
// memory (code under graph capture, serving loops, harnesses that forbid
// hipMalloc): the quantized activations and their scales go to a static
// device array instead of caller scratch. The kernels are qimg_linear's.
//
// The array is part of the library's code object: each GPU the library runs
// on holds its own copy from the library's first use on that GPU until the
// process ends. In host code its name is only a host-side handle, never a
// device address: the device address of the current GPU's copy comes from
// hipGetSymbolAddress (once per device, on the first call there) and only
// that address is passed to kernels. Every call on one GPU shares the array
// and it keeps the last call's contents (each call writes every byte it
// reads before reading it, so nothing needs clearing); calls whose kernels
// can overlap on one GPU race.
#include <mutex>

#include "qimg_internal.h"

static __device__ __align__(256) uint8_t noalloc_scratch[QIMG_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDev = 64;
std::mutex g_mu;
void* g_ptr[kMaxDev] = {};

// Device address of the current GPU's copy of noalloc_scratch.
int scratch_ptr(const char* fn, void** out) {
    int dev = 0;
    int st = qimg::api_hip_status(hipGetDevice(&dev), fn);
    if (st) return st;
    if (dev < 0 || dev >= kMaxDev) return qimg::api_fail(QIMG_ERR_UNSUPPORTED, "%s: device %d out of range", fn, dev);
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_ptr[dev] == nullptr) {
        void* p = nullptr;
        st = qimg::api_hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch)), fn);
        if (st) return st;
        if (p == nullptr || (reinterpret_cast<uintptr_t>(p) & 255u) != 0)
            return qimg::api_fail(QIMG_ERR_HIP, "%s: no aligned device address for the static scratch", fn);
        g_ptr[dev] = p;
    }
    *out = g_ptr[dev];
    return QIMG_OK;
}

}  // namespace

extern "C" int qimg_linear_noalloc(const void* x, int x_dtype, int M, int K, const void* w_q, const float* w_scales,
                                   int N, int hbs, int mode, const uint16_t* bias_bf16, void* out, int out_dtype,
                                   int gelu, void* stream) {
    const char* fn = "qimg_linear_noalloc";
    int64_t need = 0;
    int st = qimg::check_linear(fn, x, x_dtype, M, K, w_q, w_scales, N, hbs, mode, out, out_dtype, &need);
    if (st || M == 0 || N == 0) return st;
    if (need > QIMG_NOALLOC_SCRATCH_BYTES)
        return qimg::api_fail(QIMG_ERR_SCRATCH,
                              "%s: M=%d rows of K=%d need %lld bytes of scratch, more than the library's static "
                              "%lld",
                              fn, M, K, static_cast<long long>(need),
                              static_cast<long long>(QIMG_NOALLOC_SCRATCH_BYTES));
    void* scratch = nullptr;
    st = scratch_ptr(fn, &scratch);
    if (st) return st;
    return qimg::run_linear(fn, x, x_dtype, M, K, w_q, w_scales, N, hbs, mode, bias_bf16, out, out_dtype, gelu,
                            scratch, static_cast<hipStream_t>(stream));
}
