// Host-side helpers shared by the C-ABI entry points of libmq4: argument
// validation, the per-thread error message, and HIP error translation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "mq4.h"

namespace mq4 {

// Per-host-thread message of the last failing call.
std::string& last_error_ref();

inline int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    last_error_ref() = buf;
    return code;
}

inline int ok() {
    last_error_ref().clear();
    return MQ4_OK;
}

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Status of the kernels just enqueued (launch-configuration errors only;
// execution errors surface at the caller's next synchronization).
inline int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(MQ4_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

inline int check_format(const char* what, int group_size, int bits) {
    if (group_size != 64 || bits != 4)
        return fail(MQ4_ERR_UNSUPPORTED,
                    "%s: only group_size=64, bits=4 is implemented (got group_size=%d, bits=%d)",
                    what, group_size, bits);
    return MQ4_OK;
}

inline int check_k(const char* what, int64_t K) {
    if (K <= 0 || K % 64 != 0)
        return fail(MQ4_ERR_INVALID_ARG, "%s: K=%lld must be a positive multiple of 64", what,
                    (long long)K);
    return MQ4_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace mq4
