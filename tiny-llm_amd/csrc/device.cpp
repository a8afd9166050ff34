// device.cpp -- facts about the current device that the launchers size their grids by.
#include "tq_common.h"

namespace tqhip {

int device_cu_count() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
            return 1;
        cus = n;
    }
    return cus;
}

}  // namespace tqhip
