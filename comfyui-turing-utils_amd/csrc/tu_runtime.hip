// Error reporting and device checks shared by every C entry point.
#include <cstdarg>
#include <cstring>

#include "tu_common.h"

namespace tu {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string &msg) { g_last_error = msg; }

int32_t fail(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return -1;
}

int32_t check_launch(const char *what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail("%s: launch failed: %s", what, hipGetErrorString(err));
    return 0;
}

int32_t require_gfx950() {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return fail("hipGetDevice failed: %s", hipGetErrorString(err));
    const int32_t ok = tu_device_supported(dev);
    if (ok < 0) return -1;
    if (ok == 0) return fail("device %d is not a gfx950 (MI355X-class) GPU", dev);
    return 0;
}

int32_t device_cus(int &cus) {
    static int cache[64];
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return fail("hipGetDevice failed: %s", hipGetErrorString(err));
    if (dev >= 0 && dev < 64 && cache[dev] > 0) {
        cus = cache[dev];
        return 0;
    }
    err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess || cus <= 0) return fail("hipDeviceGetAttribute(CU count) failed: %s", hipGetErrorString(err));
    if (dev >= 0 && dev < 64) cache[dev] = cus;
    return 0;
}

}  // namespace tu

extern "C" {

const char *tu_last_error(void) { return tu::g_last_error.c_str(); }

int32_t tu_abi_version(void) { return 13; }

int32_t tu_device_supported(int32_t device) {
    // The answer cannot change for a device during the process: cache it.
    static int cache[64];
    static bool filled[64];
    if (device >= 0 && device < 64 && filled[device]) return cache[device];
    hipDeviceProp_t prop;
    const hipError_t err = hipGetDeviceProperties(&prop, device);
    if (err != hipSuccess) {
        tu::fail("hipGetDeviceProperties(%d) failed: %s", device, hipGetErrorString(err));
        return -1;
    }
    const int ok = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
    if (device >= 0 && device < 64) {
        cache[device] = ok;
        filled[device] = true;
    }
    return ok;
}

}  // extern "C"
