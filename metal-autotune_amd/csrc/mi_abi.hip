// ABI bookkeeping: version, per-thread error messages, shared argument checks.
#include <stdarg.h>
#include <stdio.h>

#include "mi_common.h"

namespace {
thread_local char g_error[512] = "";
}

namespace mi {

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return code;
}

int launch_status(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(MI_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return MI_OK;
}

int check_quant(int64_t N, int64_t K, int group_size, int bits, int dtype) {
    if (!valid_dtype(dtype)) return fail(MI_ERR_UNSUPPORTED, "dtype code %d", dtype);
    if (bits != 4 && bits != 8)
        return fail(MI_ERR_UNSUPPORTED, "bits=%d; this build covers 4 and 8", bits);
    if (group_size != 32 && group_size != 64 && group_size != 128)
        return fail(MI_ERR_UNSUPPORTED, "group_size=%d; this build covers 32, 64, 128",
                    group_size);
    if (N < 0 || K <= 0 || K % group_size)
        return fail(MI_ERR_ARG, "K=%lld must be a positive multiple of group_size=%d",
                    (long long)K, group_size);
    return MI_OK;
}

}  // namespace mi

extern "C" int mi_abi_version(void) { return MI_ABI_VERSION; }

extern "C" const char *mi_last_error(void) { return g_error; }
