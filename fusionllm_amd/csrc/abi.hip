// abi.hip — version and status-string entry points of libfusionmoe.so.
#include "fmoe_common.h"

extern "C" int fmoe_abi_version(void) { return FMOE_ABI_VERSION; }

extern "C" const char* fmoe_status_string(int status) {
  switch (status) {
    case FMOE_OK: return "ok";
    case FMOE_ERR_INVALID_ARG: return "invalid argument (null pointer or negative size)";
    case FMOE_ERR_SHAPE: return "unsupported shape (dim and inter must be multiples of 64, k <= min(E, 8))";
    case FMOE_ERR_ALIGN: return "pointer or leading dimension not 16-byte aligned";
    case FMOE_ERR_DTYPE: return "unknown dtype code";
    case FMOE_ERR_LAUNCH: return "kernel launch failed";
    case FMOE_ERR_WORKSPACE: return "workspace smaller than the size query returned";
    case FMOE_ERR_TOO_MANY_EXPERTS: return "number of experts outside 1..64";
    case FMOE_ERR_SCRATCH:
      return "workload larger than the static scratch of the allocation-free entry point "
             "(fmoe_dispatch_noalloc: fmoe_dispatch_workspace_bytes(T, E, k) must be <= 1 MiB); "
             "use fmoe_dispatch with a workspace";
    default: return "unknown status";
  }
}
