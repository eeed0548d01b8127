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

int check_srnl_consts(const vh_srnl_consts* k) {
    if (k == nullptr) return set_error(VH_ERR_ARG, "SRNL constants must not be null");
    if (!(k->min_retention >= 0.f && k->min_retention < 1.f))
        return set_error(VH_ERR_ARG, "MIN_RETENTION must be in [0, 1), got %g", (double)k->min_retention);
    if (!(k->injection_margin > 0.f && k->injection_margin < 1.f))
        return set_error(VH_ERR_ARG, "INJECTION_MARGIN must be in (0, 1), got %g", (double)k->injection_margin);
    if (!(k->step_scale > 0.f))
        return set_error(VH_ERR_ARG, "STEP_SCALE must be positive, got %g", (double)k->step_scale);
    // spectral_factor = 2 * SPECTRAL_MARGIN with SPECTRAL_MARGIN in (0, 1]
    if (k->spectral_clamp && !(k->spectral_factor > 0.f && k->spectral_factor <= 2.f))
        return set_error(VH_ERR_ARG, "SPECTRAL_MARGIN must be in (0, 1], got %g", 0.5 * (double)k->spectral_factor);
    return VH_OK;
}

}  // namespace vh

extern "C" {

int vh_abi_version(void) { return VH_ABI_VERSION; }

const char* vh_last_error(void) { return vh::g_last_error; }

}  // extern "C"
