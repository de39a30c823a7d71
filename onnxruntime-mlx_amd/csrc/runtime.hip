// Error state and device queries shared by every entry point of the kernel library.
#include <atomic>
#include <string>

#include "common.h"

namespace ortmi {

static thread_local std::string g_error;

void set_error(const std::string& msg) { g_error = msg; }

int fail(int code, const std::string& msg) {
    g_error = msg;
    return code;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ORTMI_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return ORTMI_OK;
}

// Compute-unit count of the current device, cached per device ordinal.
int device_cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
    const int slot = dev < 64 ? dev : 63;
    int n = cache[slot].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = 256;
    cache[slot].store(n, std::memory_order_relaxed);
    return n;
}

}  // namespace ortmi

extern "C" int ortmi_abi_version(void) { return ORTMI_ABI_VERSION; }

extern "C" const char* ortmi_last_error(void) { return ortmi::g_error.c_str(); }
