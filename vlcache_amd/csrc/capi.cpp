// Status strings and ABI version of the C ABI declared in include/vlc_capi.h.
#include "common_host.h"

VLC_HOST_API int vlc_abi_version(void) { return VLC_ABI_VERSION; }

VLC_HOST_API const char* vlc_status_string(int status) {
  switch (status) {
    case VLC_OK: return "ok";
    case VLC_ERR_INVALID: return "invalid argument (null pointer, size, stride or alignment)";
    case VLC_ERR_UNSUPPORTED: return "unsupported shape";
    case VLC_ERR_WORKSPACE: return "workspace too small for the plan";
    case VLC_ERR_CAPACITY: return "plan buffer too small";
    case VLC_ERR_PLAN: return "plan does not match the call";
    case VLC_ERR_SCRATCH: return "call needs more than the library's fixed scratch (VLC_DECODE_NOALLOC_MAX_BYTES)";
    default: return status > 0 ? "HIP runtime error" : "unknown status";
  }
}
