// runtime.hip -- host-side helpers shared by the launchers.
#include "qk_common.h"

namespace rf {

// CU count of the current device, queried once per device and cached.  The
// query is a plain attribute read, so it is legal during stream capture.
int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

}  // namespace rf

// Library identification for loaders (the ctypes layer checks it).
extern "C" const char* rf_library_version() { return "rocmforge-cdna4 0.1 gfx950"; }
