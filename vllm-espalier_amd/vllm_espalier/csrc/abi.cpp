// Host-side plumbing of the C ABI: per-thread error messages and launch checks.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../../include/espalier.h"

namespace esp_host {

static thread_local char g_error[512] = "";

const char* last_error() { return g_error; }

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_error[0] = '\0';
    return ESP_OK;
}

int launch_check(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ESP_ERR_HIP, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

}  // namespace esp_host

extern "C" const char* esp_last_error(void) { return esp_host::last_error(); }

extern "C" int esp_abi_version(void) { return 1; }
