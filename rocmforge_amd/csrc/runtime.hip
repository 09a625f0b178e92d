// runtime.hip -- host-side helpers shared by the launchers.
#include <stdlib.h>

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

int gemv_wg_per_cu(int dflt) {
    static int v = -1;
    if (v < 0) {
        const char* e = getenv("RF_GEMV_WG_PER_CU");
        int n = e ? atoi(e) : 0;
        v = (n >= 1 && n <= 16) ? n : 0;
    }
    return v ? v : dflt;
}

int gemv_rows_per_step(int dflt) {
    static int v = -1;
    if (v < 0) {
        const char* e = getenv("RF_GEMV_R");
        int n = e ? atoi(e) : 0;
        v = (n == 1 || n == 2 || n == 4) ? n : 0;
    }
    return v ? v : dflt;
}

int gemv_waves_per_wg(int dflt) {
    static int v = -1;
    if (v < 0) {
        const char* e = getenv("RF_GEMV_NW");
        int n = e ? atoi(e) : 0;
        v = (n == 4 || n == 8 || n == 16) ? n : 0;
    }
    return v ? v : dflt;
}

int gemv_q6_variant() {
    static int v = -1;
    if (v < 0) {
        const char* e = getenv("RF_Q6_V");
        v = e ? atoi(e) : 0;
    }
    return v;
}

int gemm_kernel_version() {
    static int v = -1;
    if (v < 0) {
        const char* e = getenv("RF_GEMM_V");
        const int n = e ? atoi(e) : 0;
        v = (n == 1 || n == 4 || n == 5 || n == 7) ? n : 0;
    }
    return v;
}

}  // namespace rf

// Library identification for loaders (the ctypes layer checks it).
extern "C" const char* rf_library_version() { return "rocmforge-cdna4 0.1 gfx950"; }
