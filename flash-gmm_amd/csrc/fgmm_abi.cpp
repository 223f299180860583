// Host-only parts of the C ABI: version and status strings.
#include "flashgmm.h"

extern "C" int fgmm_version(void) { return 1 * 10000 + 0 * 100 + 0; }

extern "C" const char* fgmm_strerror(int status) {
  switch (status) {
    case FGMM_OK: return "ok";
    case FGMM_ERR_INVALID_ARG: return "invalid argument (shape, stride, alignment or null pointer)";
    case FGMM_ERR_UNSUPPORTED: return "unsupported shape (outside the compiled range)";
    case FGMM_ERR_WORKSPACE: return "workspace smaller than the *_workspace_bytes() query";
    case FGMM_ERR_HIP: return "HIP runtime error or kernel launch failure";
    case FGMM_ERR_SOURCE: return "the host row source returned an error";
    case FGMM_ERR_SCRATCH: return "the call needs more workspace than the no-allocation entry point's scratch";
    default: return "unknown status";
  }
}
