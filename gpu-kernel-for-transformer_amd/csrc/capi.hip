// Library-level C-ABI entry points: version and error strings.  The kernel
// entry points live beside their kernels (layernorm.hip, gemm.hip,
// attention.hip); every one of them is declared in include/xblock.h.
#include <hip/hip_runtime.h>

#include "../../include/xblock.h"

extern "C" int xb_abi_version(void) { return XB_ABI_VERSION; }

extern "C" const char* xb_strerror(int code) {
  switch (code) {
    case XB_OK: return "success";
    case XB_ERR_NULL_POINTER: return "xblock: a required pointer is NULL";
    case XB_ERR_BAD_SIZE: return "xblock: a size argument is negative, zero or too large";
    case XB_ERR_BAD_DTYPE: return "xblock: unsupported element type";
    case XB_ERR_UNSUPPORTED_SHAPE: return "xblock: unsupported shape (see include/xblock.h)";
    case XB_ERR_MISALIGNED: return "xblock: a pointer is not 16-byte aligned";
    case XB_ERR_BAD_EPILOGUE: return "xblock: unknown GEMM epilogue, mask mode or flag";
    case XB_ERR_WORKSPACE: return "xblock: workspace smaller than the call needs";
    case XB_ERR_WRONG_DEVICE: return "xblock: the stream does not belong to the current device";
    case XB_ERR_SCRATCH_TOO_SMALL:
      return "xblock: the call needs more than the static scratch (XB_DECODE_SCRATCH_BYTES); pass a workspace";
    default:
      if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
      return "xblock: unknown error";
  }
}
