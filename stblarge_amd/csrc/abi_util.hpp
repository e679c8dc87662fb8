// Error reporting shared by every C-ABI entry point.
//
// Entry points with the reference's `void` signatures (stbl/kernels.h) cannot return a status, so
// every entry point records its last failure in a thread-local slot that stbl_amd_last_error()
// reads (and clears). Entry points of the v2 surface also return 0 or a negative hipError_t.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

namespace stbl {

struct LastError {
    int code;
    char msg[256];
};

LastError &last_error();

inline int abi_fail(hipError_t e, const char *fmt, ...) {
    LastError &le = last_error();
    le.code = (int)e;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(le.msg, sizeof le.msg, fmt, ap);
    va_end(ap);
    return -(int)e;
}

inline int abi_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return 0;
    return abi_fail(e, "%s: %s", what, hipGetErrorString(e));
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace stbl
