// ABI utilities of libgdn_mi355x: version and status text.
#include "../../include/gdn_mi355x.h"

extern "C" int gdn_abi_version(void) { return GDN_ABI_VERSION; }

extern "C" const char* gdn_status_string(int status) {
  switch (status) {
    case GDN_OK: return "ok";
    case GDN_ERR_INVALID_ARGUMENT: return "invalid argument (null pointer, negative size or bad option)";
    case GDN_ERR_WORKSPACE_TOO_SMALL: return "workspace smaller than gdn_prefill_workspace_bytes()";
    case GDN_ERR_UNALIGNED: return "buffer misses its required alignment";
    case GDN_ERR_ALIASING: return "state and new_state must be different buffers";
    case GDN_ERR_TOO_LARGE: return "batch needs more workspace than the no-allocation scratch holds";
    default: return status > 0 ? "HIP launch error" : "unknown status";
  }
}
