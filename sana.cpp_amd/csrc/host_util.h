// Host-side helpers shared by the C ABI translation units (DiT and VAE):
// the thread-local last-error string behind sana_dit_last_error(), the error
// type the entry points translate into SANA_ERR_* codes, HIP error checks,
// and the context-owned device allocation.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <thread>
#include <vector>

#include "../../include/sana_dit.h"

namespace sana_host {

inline thread_local std::string g_last_error;

inline int set_err(int code, const char * fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

struct SanaError {
    int code;
    std::string msg;
};

[[noreturn]] inline void throw_err(int code, const std::string & m) { throw SanaError{code, m}; }

inline void hip_check(hipError_t e, const char * what) {
    if (e != hipSuccess) {
        throw_err(e == hipErrorOutOfMemory ? SANA_ERR_OUT_OF_MEMORY : SANA_ERR_HIP,
                  std::string(what) + ": " + hipGetErrorString(e));
    }
}

inline void launch_check(hipError_t e, const char * what) {
    if (e == hipErrorInvalidValue) throw_err(SANA_ERR_SHAPE, std::string(what) + ": shape not supported by kernel");
    hip_check(e, what);
}

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Largest finite fp16 value: the GEMM operands are fp16, so a weight outside
// [-65504, 65504] (or not finite) cannot be represented.  Magnitudes below
// fp16's smallest subnormal (2^-24) round to zero, like any rounding.
constexpr float kF16Max = 65504.0f;

// fp32 -> fp16 operand conversion that refuses a value fp16 cannot hold
// (SANA_ERR_FORMAT naming the tensor and the element).
inline _Float16 to_f16_checked(float v, const std::string & tensor, size_t i) {
    if (!(v <= kF16Max && v >= -kF16Max)) {  // NaN fails both comparisons
        char buf[96];
        snprintf(buf, sizeof(buf), "%g at element %zu", (double)v, i);
        throw_err(SANA_ERR_FORMAT, tensor + ": weight value " + buf + " is outside the fp16 operand range (|w| <= 65504)");
    }
    return (_Float16)v;
}

// Runs f(lo, hi) over contiguous ranges covering [0, n) on up to 16 host
// threads (one range per thread, none smaller than `grain`); f must not throw.
template <class F>
inline void host_parallel(size_t n, size_t grain, F f) {
    const size_t hw = std::max(1u, std::thread::hardware_concurrency());
    size_t nt = std::min<size_t>(std::min<size_t>(16, hw), (n + grain - 1) / std::max<size_t>(grain, 1));
    if (nt <= 1) {
        f((size_t)0, n);
        return;
    }
    const size_t per = (n + nt - 1) / nt;
    std::vector<std::thread> th;
    size_t t = 1;
    try {
        for (; t < nt; ++t) {
            const size_t lo = t * per, hi = std::min(n, lo + per);
            if (lo < hi) th.emplace_back(f, lo, hi);
        }
    } catch (...) {  // no thread to spare: range t and the ones after it run here
        for (; t < nt; ++t) {
            const size_t lo = t * per, hi = std::min(n, lo + per);
            if (lo < hi) f(lo, hi);
        }
    }
    f((size_t)0, std::min(n, per));
    for (auto & x : th) x.join();
}

// Lowest index recorded by concurrent ranges (SIZE_MAX when none).
inline void atomic_min(std::atomic<size_t> & a, size_t v) {
    size_t cur = a.load();
    while (v < cur && !a.compare_exchange_weak(cur, v)) {
    }
}

// IEEE fp16 bit patterns: refuse inf and NaN (exponent field all ones).
inline void check_f16_bits_finite(const uint16_t * h, size_t n, const std::string & tensor) {
    for (size_t i = 0; i < n; ++i)
        if ((h[i] & 0x7c00u) == 0x7c00u)
            throw_err(SANA_ERR_FORMAT, tensor + ": fp16 weight at element " + std::to_string(i) + " is not finite");
}

// Device allocation owned by the context.
struct DevMem {
    void * p = nullptr;
    size_t bytes = 0;
    DevMem() = default;
    DevMem(const DevMem &) = delete;
    DevMem & operator=(const DevMem &) = delete;
    ~DevMem() {
        if (p) (void)hipFree(p);
    }
    void ensure(size_t n, bool zero = true) {
        if (n <= bytes && p) return;
        if (p) hip_check(hipFree(p), "hipFree");
        p = nullptr;
        bytes = 0;
        hip_check(hipMalloc(&p, n ? n : 16), "hipMalloc");
        bytes = n;
        if (zero) {
            // A device memset may return before it completes, and work on a
            // non-blocking stream is not ordered after the null stream: wait
            // for the fill so every later launch sees the zeros.
            hip_check(hipMemset(p, 0, n), "hipMemset");
            hip_check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
        }
    }
    template <class T>
    T * as() const {
        return static_cast<T *>(p);
    }
};

// Host -> device copy that has landed when it returns: a pageable-source
// hipMemcpy may return once the data is staged, and a non-blocking stream is
// not ordered after the null stream's DMA.
inline void copy_to_device(void * dst, const void * src, size_t bytes, const char * what) {
    hip_check(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), what);
    hip_check(hipStreamSynchronize(nullptr), what);
}

// Runs f, translating SanaError, allocation failures and other exceptions into
// a SANA_ERR_* code with the message in g_last_error.
template <class F>
int guarded(F f) {
    try {
        f();
        return SANA_OK;
    } catch (const SanaError & e) {
        g_last_error = e.msg;
        return e.code;
    } catch (const std::bad_alloc &) {
        return set_err(SANA_ERR_OUT_OF_MEMORY, "host allocation failed");
    } catch (const std::exception & e) {
        return set_err(SANA_ERR_HIP, "%s", e.what());
    }
}

}  // namespace sana_host
