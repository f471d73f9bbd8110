// Library lifecycle: the per-thread error slot and the device check.
#include <cstring>
#include <string>

#include "common.hpp"

namespace dtts {

int noalloc_scratch_address(const char *name, void **out);  // gemm.hip

static thread_local char g_error[1024] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

}  // namespace dtts

extern "C" const char *dtts_last_error(void) { return dtts::g_error; }

extern "C" int dtts_version(void) { return (1 << 16) | 0; }

extern "C" int dtts_init(void) {
    int dev = 0;
    DTTS_HIP_CHECK(hipGetDevice(&dev), "dtts_init: hipGetDevice");
    hipDeviceProp_t prop;
    DTTS_HIP_CHECK(hipGetDeviceProperties(&prop, dev), "dtts_init: hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        dtts::set_error("dtts_init: device %d is %s; this build holds gfx950 code only", dev,
                        prop.gcnArchName);
        return DTTS_ERR_UNSUPPORTED;
    }
    void *scratch = nullptr;  // the allocation-free projection's scratch on this device
    return dtts::noalloc_scratch_address("dtts_init", &scratch);
}
