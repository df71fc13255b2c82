// dq_runtime.hip - library version and device query.
#include "dq_common.h"

extern "C" int dq_version(void) { return 1; }

extern "C" int dq_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}
