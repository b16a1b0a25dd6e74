// Version and status strings of the libsynth_hip C ABI.
#include "synth_hip.h"

extern "C" uint32_t shp_abi_version(void) {
    return SHP_ABI_VERSION;
}

extern "C" const char * shp_status_string(shp_status_t status) {
    switch (status) {
        case SHP_OK:
            return "ok";
        case SHP_ERR_INVALID_ARG:
            return "invalid argument";
        case SHP_ERR_UNSUPPORTED:
            return "unsupported type, layout or mode";
        case SHP_ERR_BACKEND:
            return "HIP launch failure";
        default:
            return "unknown status";
    }
}
