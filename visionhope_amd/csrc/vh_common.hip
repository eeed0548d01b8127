// Error reporting shared by every entry point of libvisionhope_hip.so.
#include "vh_common.h"

#include <cstring>
#include <initializer_list>
#include <mutex>

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

// ---------------------------------------------------------------------------
// Dispatch overrides.  A fixed table of the names that may be overridden, each with a
// validator; values live in a mutex-guarded table and are copied out per lookup, so a
// lookup never sees a half-written value.
// ---------------------------------------------------------------------------
namespace {

bool is_uint(const char* v, long long lo, long long hi) {
    if (!v || !*v) return false;
    long long n = 0;
    for (const char* c = v; *c; ++c) {
        if (*c < '0' || *c > '9' || n > hi) return false;
        n = n * 10 + (*c - '0');
    }
    return n >= lo && n <= hi;
}
bool one_of(const char* v, std::initializer_list<const char*> options) {
    for (const char* o : options)
        if (std::strcmp(v, o) == 0) return true;
    return false;
}
bool scan_pack_ok(const char* v) {
    int l = 0, t = 0;
    char tail = 0;
    return std::sscanf(v, "%dx%d%c", &l, &t, &tail) == 2 && (l == 1 || l == 2 || l == 4) && (t == 2 || t == 4) &&
           l <= t;
}
bool pw_cfg_ok(const char* v) {
    int a = 0, b = 0, c = 0, d = 0;
    char tail = 0;
    if (v[0] == 'n') return one_of(v + 1, {"1", "2", "4"});
    if (v[0] == 'w') return one_of(v + 1, {"32", "64"});
    if (std::sscanf(v, "d%dx%do%d%c", &a, &b, &c, &tail) == 3) return a > 0 && b > 0 && c > 0;
    if (std::sscanf(v, "d%dx%do%dw%d%c", &a, &b, &c, &d, &tail) == 4) return a > 0 && b > 0 && c > 0 && (d == 2 || d == 4);
    if (std::sscanf(v, "t%dx%dk%do%d%c", &a, &b, &c, &d, &tail) == 4) return a > 0 && b > 0 && c > 0 && d > 0;
    return false;
}

bool fusion_tile_ok(const char* v) {
    int th = 0, tw = 0, hpb = 0;
    char tail = 0;
    return std::sscanf(v, "%dx%dx%d%c", &th, &tw, &hpb, &tail) == 3 && th >= 0 && th <= 4 && tw >= 0 && tw <= 4 &&
           hpb >= 1 && hpb <= 64;
}

struct OverrideSlot {
    const char* name;
    bool (*valid)(const char*);
    char value[32];
};

OverrideSlot g_overrides[] = {
    {"scan_ut", [](const char* v) { return one_of(v, {"0", "1"}); }, ""},
    {"scan_wide", [](const char* v) { return one_of(v, {"0", "1", "2", "4"}); }, ""},
    {"scan_tb", [](const char* v) { return one_of(v, {"1", "2"}); }, ""},
    {"scan_pack", scan_pack_ok, ""},
    {"scan_utw", [](const char* v) { return one_of(v, {"0", "1"}); }, ""},
    {"pw_cfg", pw_cfg_ok, ""},
    {"pw_resident", [](const char* v) { return one_of(v, {"0", "2"}); }, ""},
    {"dw_tile", [](const char* v) { return one_of(v, {"0", "1", "2"}); }, ""},   // off / by shape / everywhere
    {"dw_tile_cs", [](const char* v) { return one_of(v, {"8", "16", "32", "64"}); }, ""},
    {"dw_tile_p", [](const char* v) { return one_of(v, {"2", "7", "8"}); }, ""},
    {"dw_launch_bytes", [](const char* v) { return is_uint(v, 1, (1ll << 31) - 1); }, ""},
    {"ln_stage", [](const char* v) { return one_of(v, {"0", "1"}); }, ""},
    {"conv_band", [](const char* v) { return one_of(v, {"0", "1"}); }, ""},
    {"grn_spin_limit", [](const char* v) { return is_uint(v, 1, 1 << 20); }, ""},
    {"fusion_tile", fusion_tile_ok, ""},
    {"grn_pieces", [](const char* v) { return is_uint(v, 2, 64); }, ""},
    {"readout_tile", [](const char* v) { return one_of(v, {"8", "16"}); }, ""},
};
std::mutex g_override_mutex;

}  // namespace

Override::Override(const char* name) {
    value[0] = 0;
    std::lock_guard<std::mutex> lock(g_override_mutex);
    for (const OverrideSlot& s : g_overrides)
        if (std::strcmp(s.name, name) == 0) {
            std::memcpy(value, s.value, sizeof(value));
            return;
        }
}
int Override::as_int() const { return std::atoi(value); }
long long Override::as_i64() const { return std::atoll(value); }

}  // namespace vh

extern "C" {

int vh_set_dispatch_override(const char* name, const char* value) {
    using namespace vh;
    VH_REQUIRE(name != nullptr, VH_ERR_ARG, "dispatch override name must not be null");
    for (OverrideSlot& s : g_overrides) {
        if (std::strcmp(s.name, name) != 0) continue;
        const bool clear = value == nullptr || value[0] == 0;
        VH_REQUIRE(clear || (std::strlen(value) < sizeof(s.value) && s.valid(value)), VH_ERR_ARG,
                   "invalid value '%s' for dispatch override '%s'", value ? value : "", name);
        std::lock_guard<std::mutex> lock(g_override_mutex);
        if (clear) s.value[0] = 0;
        else std::snprintf(s.value, sizeof(s.value), "%s", value);
        return VH_OK;
    }
    return set_error(VH_ERR_ARG, "unknown dispatch override '%s'", name);
}

void vh_clear_dispatch_overrides(void) {
    std::lock_guard<std::mutex> lock(vh::g_override_mutex);
    for (vh::OverrideSlot& s : vh::g_overrides) s.value[0] = 0;
}

int vh_abi_version(void) { return VH_ABI_VERSION; }

const char* vh_last_error(void) { return vh::g_last_error; }

}  // extern "C"
