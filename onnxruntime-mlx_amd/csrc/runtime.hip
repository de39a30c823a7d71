// Error state and device queries shared by every entry point of the kernel library.
#include <atomic>
#include <cstring>
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

// A few small host-to-device copies as one launch: the bytes and destinations are
// the kernel's arguments. Byte stores: the copies are a few bytes each and the
// destinations have any alignment.
struct SmallCopies {
    uint8_t* dst[ORTMI_SMALL_COPIES];
    uint32_t end[ORTMI_SMALL_COPIES];  // cumulative byte count after copy k
    int n;
    uint8_t data[ORTMI_SMALL_COPY_BYTES];
};

__global__ __launch_bounds__(256) void small_copy_kernel(SmallCopies c) {
    const uint32_t total = c.end[c.n - 1];
    for (uint32_t i = threadIdx.x; i < total; i += blockDim.x) {
        int k = 0;
        while (i >= c.end[k]) ++k;  // i < total = end[n - 1]: stops at k <= n - 1
        c.dst[k][i - (k ? c.end[k - 1] : 0u)] = c.data[i];
    }
}

}  // namespace ortmi

extern "C" int ortmi_copy_small_h2d(int n, void* const* dst, const void* const* src,
                                    const size_t* bytes, void* stream) {
    using namespace ortmi;
    ORTMI_REQUIRE(n >= 0 && n <= ORTMI_SMALL_COPIES, "small copy: at most 16 copies");
    ORTMI_REQUIRE(n == 0 || (dst && src && bytes), "small copy: null argument");
    SmallCopies c{};
    uint32_t off = 0;
    for (int k = 0; k < n; ++k) {
        ORTMI_REQUIRE(bytes[k] <= (size_t)ORTMI_SMALL_COPY_BYTES - off,
                      "small copy: more than 1024 bytes in all");
        ORTMI_REQUIRE(bytes[k] == 0 || (dst[k] && src[k]), "small copy: null buffer");
        if (bytes[k]) std::memcpy(c.data + off, src[k], bytes[k]);
        off += (uint32_t)bytes[k];
        c.end[k] = off;
        c.dst[k] = static_cast<uint8_t*>(dst[k]);
    }
    c.n = n;
    if (off == 0) return ORTMI_OK;
    hipLaunchKernelGGL(small_copy_kernel, dim3(1), dim3(256), 0, as_stream(stream), c);
    return check_launch("small copy");
}

extern "C" int ortmi_abi_version(void) { return ORTMI_ABI_VERSION; }

extern "C" const char* ortmi_last_error(void) { return ortmi::g_error.c_str(); }
