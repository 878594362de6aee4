// ABI bookkeeping of the reelcache HIP library: version, struct sizes and the last-error text.
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace rch {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* format, ...) {
    va_list args;
    va_start(args, format);
    vsnprintf(g_last_error, sizeof(g_last_error), format, args);
    va_end(args);
    return code;
}

int check_launch(const char* what) {
    const hipError_t status = hipGetLastError();
    if (status != hipSuccess) return fail(RCH_E_LAUNCH, "%s: %s", what, hipGetErrorString(status));
    return RCH_OK;
}

}  // namespace rch

extern "C" {

int rch_abi_version(void) { return RCH_ABI_VERSION; }
int rch_job_size(void) { return static_cast<int>(sizeof(rch_job)); }
int rch_pack_size(void) { return static_cast<int>(sizeof(rch_pack)); }
const char* rch_last_error(void) { return rch::g_last_error; }

}  // extern "C"
