// Status codes, the thread-local error text and the device check.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "../../include/tessera_hip.h"

namespace ts {

static thread_local char g_last[512] = "";

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last, sizeof g_last, fmt, ap);
    va_end(ap);
    return code;
}

int hip_status(hipError_t e, const char *what) {
    snprintf(g_last, sizeof g_last, "%s failed: %s (%d) %s", what, hipGetErrorName(e), (int)e,
             hipGetErrorString(e));
    return (int)e;
}

}  // namespace ts

extern "C" const char *tessera_hip_last_error(void) { return ts::g_last; }

extern "C" int tessera_hip_abi_version(void) { return TS_ABI_VERSION; }

extern "C" int tessera_hip_init(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return ts::hip_status(e, "hipGetDevice");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return ts::hip_status(e, "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return ts::fail(TS_ERR_ARCH, "device %d is %s; these kernels are built for gfx950 only", dev,
                        prop.gcnArchName);
    if (prop.warpSize != 64) return ts::fail(TS_ERR_ARCH, "wave size %d, expected 64", prop.warpSize);
    return TS_OK;
}
