// Library-wide C-ABI helpers: the per-thread error slot and version query.
#include <string.h>

#include "abi_util.hpp"

namespace stbl {

LastError &last_error() {
    static thread_local LastError le = {0, {0}};
    return le;
}

}  // namespace stbl

extern "C" {

// Copies the calling thread's last recorded failure into buf (if given), clears it, and returns its
// hipError_t code (0 when nothing failed since the last call).
int stbl_amd_last_error(char *buf, int len) {
    stbl::LastError &le = stbl::last_error();
    const int code = le.code;
    if (buf && len > 0) {
        strncpy(buf, le.msg, (size_t)len - 1);
        buf[len - 1] = 0;
    }
    le.code = 0;
    le.msg[0] = 0;
    return code;
}

// The ABI version: raised whenever the signature or meaning of an exported function changes.
int stbl_amd_version(void) { return 2; }

}  // extern "C"
