// capi.hip -- status strings and device checks of the gsx C ABI.
#include <string.h>

#include "gsx_device.h"

extern "C" {

const char* gsx_strerror(int status) {
    switch (status) {
        case GSX_OK: return "ok";
        case GSX_ERR_INVALID: return "invalid argument (size, null pointer, alignment or shape)";
        case GSX_ERR_HIP: return "HIP runtime error";
        case GSX_ERR_WORKSPACE: return "workspace smaller than gsx_bin_workspace_bytes()";
        case GSX_ERR_TOO_LARGE: return "count exceeds the supported index range";
        case GSX_ERR_DEVICE:
            return "device-side check failed (a bounded wait in the chained scan expired)";
        default: return status > 0 ? "capacity too small (retry with the returned size)"
                                   : "unknown gsx status";
    }
}

int gsx_abi_version(void) { return GSX_ABI_VERSION; }

// Writes the current device's gcnArchName; returns 1 if it is gfx950 (the
// only target this library is built for), 0 if not, < 0 on error.
int gsx_device_check(char* name_out, int name_len) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return GSX_ERR_HIP;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return GSX_ERR_HIP;
    if (name_out && name_len > 0) {
        strncpy(name_out, prop.gcnArchName, (size_t)name_len - 1);
        name_out[name_len - 1] = '\0';
    }
    return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

}  // extern "C"
