// Library-level C-ABI entry points: error reporting, version and the device
// capability probe used by the Python host layer.

#include <cstdarg>

#include "kbn_common.h"

namespace kbn {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

}  // namespace kbn

extern "C" const char* kbn_last_error(void) { return kbn::g_last_error; }

extern "C" int kbn_abi_version(void) { return 1; }

// Writes the gcnArchName of `device` (e.g. "gfx950:sramecc+:xnack-") into buf.
extern "C" int kbn_device_arch(int device, char* buf, int len) {
    KBN_CHECK_ARG(buf && len > 0, "device_arch: null buffer");
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) {
        kbn::set_error("device_arch: hipGetDeviceProperties(%d) failed: %s", device, hipGetErrorString(e));
        return 2;
    }
    snprintf(buf, (size_t)len, "%s", prop.gcnArchName);
    return 0;
}
