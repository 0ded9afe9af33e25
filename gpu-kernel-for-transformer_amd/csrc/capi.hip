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
    case XB_ERR_BAD_VARIANT: return "xblock: kernel variant not built for this shape (see xb_select_*)";
    case XB_ERR_WRONG_DEVICE: return "xblock: the stream does not belong to the current device";
    case XB_ERR_SCRATCH_TOO_SMALL:
      return "xblock: the call needs more than the static scratch (XB_DECODE_SCRATCH_BYTES); pass a workspace";
    default:
      if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
      return "xblock: unknown error";
  }
}

extern "C" const char* xb_variant_name(int op, int variant) {
  switch (op) {
    case XB_OP_LINEAR:
      switch (variant) {
        case XB_LINEAR_DMA_256x256: return "mfma_gemm_dma_256x256";
        case XB_LINEAR_DMA_256x192: return "mfma_gemm_dma_256x192";
        case XB_LINEAR_DMA_128x256: return "mfma_gemm_dma_128x256";
        case XB_LINEAR_DMA_128x128: return "mfma_gemm_dma_128x128";
        case XB_LINEAR_NT_128x128: return "mfma_gemm_nt_128x128";
        case XB_LINEAR_NT_64x64: return "mfma_gemm_nt_64x64";
        default: return nullptr;
      }
    case XB_OP_ATTENTION:
      switch (variant) {
        case XB_ATTN_W4_Q16: return "flash_4wave_64q";
        case XB_ATTN_W4_Q32: return "flash_4wave_128q";
        case XB_ATTN_W4_Q64: return "flash_4wave_256q";
        case XB_ATTN_W8_Q16: return "flash_8wave_128q";
        case XB_ATTN_PINGPONG: return "flash_pingpong_8wave_512q";
        case XB_ATTN_PINGPONG_VT: return "flash_pingpong_vt_8wave_512q";
        default: return nullptr;
      }
    case XB_OP_FUSED_D128:
      switch (variant) {
        case XB_FUSED_PAIRS: return "fused_stack_1wg_8wave_pairs";
        case XB_FUSED_SPLIT: return "fused_stack_split_2wg";
        case XB_FUSED_HD128: return "fused_stack_1wg_8wave_hd128";
        default: return nullptr;
      }
    default:
      return nullptr;
  }
}
