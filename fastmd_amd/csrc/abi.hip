// ABI version and status strings of libfastmd_hip.so.
#include "common.h"

extern "C" {

int fmd_abi_version(void) { return FMD_ABI_VERSION; }

const char* fmd_error_string(int status) {
  switch (status) {
    case FMD_OK: return "success";
    case FMD_EINVAL: return "invalid argument (size or pointer no launch can honour)";
    case FMD_EUNSUPPORTED: return "configuration not supported by this build";
    case FMD_ETOOLARGE: return "size beyond the static scratch of an allocation-free entry point";
    default: return hipGetErrorString((hipError_t)status);
  }
}

}  // extern "C"
