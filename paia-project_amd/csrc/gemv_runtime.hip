// Process-wide device facts for grid sizing. Queried once (first launch) and cached; no allocation, no sync.
#include <hip/hip_runtime.h>

#include <atomic>

#include "gemv_kernel.h"
#include "paia_gemv.h"

namespace paia {

DeviceFacts device_facts()
{
    // cus is published last (release) and read first (acquire), so a reader that sees it also sees the LDS sizes
    static std::atomic<int> cus{0}, lds{0}, ldsb{0};
    DeviceFacts f;
    f.cus = cus.load(std::memory_order_acquire);
    f.lds_per_cu = lds.load(std::memory_order_relaxed);
    f.lds_per_block = ldsb.load(std::memory_order_relaxed);
    if (f.cus == 0) {
        int dev = 0, n = 0, l = 0, lb = 0;
        if (hipGetDevice(&dev) == hipSuccess) {
            if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
            if (hipDeviceGetAttribute(&l, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess) l = 0;
            if (hipDeviceGetAttribute(&lb, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) lb = 0;
        }
        f.cus = n > 0 ? n : 256;
        f.lds_per_cu = l > 0 ? l : 65536;
        f.lds_per_block = lb > 0 ? lb : 65536;
        lds.store(f.lds_per_cu, std::memory_order_relaxed);
        ldsb.store(f.lds_per_block, std::memory_order_relaxed);
        cus.store(f.cus, std::memory_order_release);
    }
    return f;
}

}  // namespace paia

extern "C" {

// Build identification (no reference counterpart): lets callers check which library they loaded.
const char* paia_gemv_build_info() { return "paia_gemv gfx950 HIP build (wave64, LDS-staged x, buffer-load streaming)"; }

}  // extern "C"
