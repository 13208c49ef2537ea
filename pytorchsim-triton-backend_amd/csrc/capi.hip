// Library identity and status text for the C ABI declared in include/ptb_amd.h.
#include "ptb_common.h"

PTB_EXPORT int ptb_abi_version(void) { return PTB_ABI_VERSION; }

PTB_EXPORT const char* ptb_status_string(int status) {
  switch (status) {
    case PTB_OK: return "ok";
    case PTB_ERR_NULL: return "a required pointer is NULL";
    case PTB_ERR_SHAPE: return "bad shape";
    case PTB_ERR_ALIGN: return "pointer or row not aligned for 128-bit access";
    case PTB_ERR_DTYPE: return "unknown dtype or op code";
    case PTB_ERR_UNSUPPORTED: return "shape outside what the kernel implements";
    case PTB_ERR_GRID: return "grid past the hardware bound";
    case PTB_ERR_WORKSPACE: return "workspace too small";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}
