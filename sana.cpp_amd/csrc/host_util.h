// Host-side helpers shared by the C ABI translation units (DiT and VAE):
// the thread-local last-error string behind sana_dit_last_error(), the error
// type the entry points translate into SANA_ERR_* codes, HIP error checks,
// and the context-owned device allocation.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

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
