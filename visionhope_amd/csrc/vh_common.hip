// Error reporting shared by every entry point of libvisionhope_hip.so.
#include "vh_common.h"

namespace vh {

namespace {
thread_local char g_last_error[512] = "";
}

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return set_error(VH_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(err));
    return VH_OK;
}

}  // namespace vh

extern "C" {

int vh_abi_version(void) { return VH_ABI_VERSION; }

const char* vh_last_error(void) { return vh::g_last_error; }

}  // extern "C"
