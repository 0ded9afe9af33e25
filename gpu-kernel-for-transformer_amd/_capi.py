"""ctypes binding of ``libxblock.so`` (declared in include/xblock.h).

Loading never raises: `XBLOCK_AVAILABLE` / `XBLOCK_LOAD_ERROR` report whether
the library was found, mirroring the reference's import-safe availability
flags (triton_fused_norm.py:24-32).  Every call path, however, goes through
`lib()`, which raises RuntimeError when the library is missing, so the GPU path
can never run anything but the HIP kernels.

torch is imported before the library is opened: torch's bundled HIP runtime
(soname libamdhip64.so.7) is then already resident, and the library binds to
it instead of loading a second runtime into the process.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

import torch  # noqa: F401  (must precede the dlopen below; see module docstring)

LIBRARY_PATH = Path(
    os.environ.get("XBLOCK_LIBRARY", Path(__file__).resolve().parent / "libxblock.so")
)

# Constants mirrored from include/xblock.h.
XB_ABI_VERSION = 3
XB_F32 = 0
XB_F16 = 1
XB_EPI_BIAS = 0
XB_EPI_BIAS_GELU = 1
XB_PACK_PERMUTED = 0
XB_PACK_NATURAL = 1
XB_MASK_UPDATE = 1
XB_MASK_SUM = 2
XB_MASK_OUTPUT = 4
XB_SPLIT_SPINS_DEFAULT = -1
XB_SPLIT_FAULT_NO_PUBLISH = 1
XB_SPLIT_FAULT_FOREIGN_XCD = 2
XB_DECODE_SCRATCH_BYTES = 32 << 20
XB_VARIANT_AUTO = -1
XB_OP_LINEAR = 0
XB_OP_ATTENTION = 1
XB_OP_FUSED_D128 = 2
XB_FUSED_PAIRS = 0
XB_FUSED_SPLIT = 1
XB_FUSED_HD128 = 2
XB_LINEAR_DMA_256x256 = 0
XB_LINEAR_DMA_256x192 = 1
XB_LINEAR_DMA_128x256 = 2
XB_LINEAR_DMA_128x128 = 3
XB_LINEAR_NT_128x128 = 4
XB_LINEAR_NT_64x64 = 5
XB_ATTN_W4_Q16 = 0
XB_ATTN_W4_Q32 = 1
XB_ATTN_W4_Q64 = 2
XB_ATTN_W8_Q16 = 3
XB_ATTN_PINGPONG = 4
XB_ATTN_PINGPONG_VT = 5

EXPORTED_SYMBOLS = (
    "xb_abi_version",
    "xb_strerror",
    "xb_layernorm",
    "xb_residual_layernorm",
    "xb_residual_layernorm_masked",
    "xb_linear",
    "xb_linear_v",
    "xb_attention_causal",
    "xb_attention",
    "xb_attention_v",
    "xb_vt_row_stride",
    "xb_linear_qkv_vt",
    "xb_attention_causal_vt",
    "xb_select_linear",
    "xb_select_attention",
    "xb_select_fused_d128",
    "xb_variant_name",
    "xb_kv_cache_append",
    "xb_attention_kv_cache_workspace_bytes",
    "xb_attention_kv_cache",
    "xb_attention_kv_cache_noalloc",
    "xb_pack_linear_fragments",
    "xb_fused_forward_d128",
    "xb_fused_forward_d128_workspace_bytes",
    "xb_fused_forward_d128_ws",
)

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_SIGNATURES = {
    "xb_abi_version": (ctypes.c_int, []),
    "xb_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "xb_layernorm": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int, _i64, _i32, _f32, ctypes.c_int, _vp]),
    "xb_residual_layernorm": (
        ctypes.c_int,
        [_vp, _vp, ctypes.c_int, _vp, _vp, _vp, _vp, ctypes.c_int, _i64, _i32, _f32, ctypes.c_int, _vp],
    ),
    "xb_residual_layernorm_masked": (
        ctypes.c_int,
        [_vp, _vp, ctypes.c_int, _vp, _vp, _vp, _vp, ctypes.c_int, _i64, _i32, _f32, ctypes.c_int,
         _vp, ctypes.c_int, _vp],
    ),
    "xb_linear": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, ctypes.c_int, _vp]),
    "xb_attention_causal": (ctypes.c_int, [_vp, _vp, _i32, _i64, _i32, _i32, _f32, _vp]),
    "xb_attention": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i64, _i32, _i32, _f32, _i32, _vp]),
    "xb_linear_v": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, ctypes.c_int, ctypes.c_int, _vp]),
    "xb_attention_v": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i64, _i32, _i32, _f32, _i32, ctypes.c_int, _vp]),
    "xb_vt_row_stride": (_i64, [_i64]),
    "xb_linear_qkv_vt": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i32, _i32, _i32, ctypes.c_int, _vp]),
    "xb_attention_causal_vt": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i64, _i32, _i32, _f32, _vp]),
    "xb_select_linear": (ctypes.c_int, [_i64, _i32, _i32, ctypes.c_int]),
    "xb_select_attention": (ctypes.c_int, [_i32, _i64, _i32, _i32, _i32]),
    "xb_select_fused_d128": (ctypes.c_int, [_i64, _i32, _i32, _i32, _i32, _i32]),
    "xb_variant_name": (ctypes.c_char_p, [ctypes.c_int, ctypes.c_int]),
    "xb_kv_cache_append": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i64, _i32, _i32, _i64, _i64, _vp]),
    "xb_attention_kv_cache_workspace_bytes": (_i64, [_i32, _i64, _i32, _i32, _i64]),
    "xb_attention_kv_cache": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _i32, _i64, _i32, _i32, _i64, _i64, _f32, _vp, _i64, _vp],
    ),
    "xb_attention_kv_cache_noalloc": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _i32, _i64, _i32, _i32, _i64, _i64, _f32, _vp],
    ),
    "xb_pack_linear_fragments": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, _f32, _vp]),
    "xb_fused_forward_d128": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i64, _vp, _i32, _vp]),
    "xb_fused_forward_d128_workspace_bytes": (_i64, [_i64, _i32, _i32, _i32, _i32]),
    "xb_fused_forward_d128_ws": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i64, _vp, _i32, _vp, _i64, _i32, _i32, _vp],
    ),
}

_LIB: Optional[ctypes.CDLL] = None
XBLOCK_LOAD_ERROR: Optional[str] = None


def _load() -> Optional[ctypes.CDLL]:
    global XBLOCK_LOAD_ERROR
    if not LIBRARY_PATH.exists():
        XBLOCK_LOAD_ERROR = f"{LIBRARY_PATH} is not built (run __graft_entry__.build())"
        return None
    try:
        handle = ctypes.CDLL(str(LIBRARY_PATH))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = handle.xb_abi_version()
        if version != XB_ABI_VERSION:
            XBLOCK_LOAD_ERROR = f"ABI version {version} != expected {XB_ABI_VERSION}"
            return None
        return handle
    except (OSError, AttributeError) as error:
        XBLOCK_LOAD_ERROR = f"cannot load {LIBRARY_PATH}: {error}"
        return None


_LIB = _load()
XBLOCK_AVAILABLE = _LIB is not None


def reload() -> bool:
    """Re-open the library after a rebuild in this process; return availability."""
    global _LIB, XBLOCK_AVAILABLE, XBLOCK_LOAD_ERROR
    XBLOCK_LOAD_ERROR = None
    _LIB = _load()
    XBLOCK_AVAILABLE = _LIB is not None
    return XBLOCK_AVAILABLE


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError (no fallback) when it is missing."""
    if _LIB is None:
        raise RuntimeError(f"xblock HIP library unavailable: {XBLOCK_LOAD_ERROR}")
    return _LIB


def check(code: int, what: str) -> None:
    """Map a nonzero C-ABI return code to RuntimeError, as the reference's wrappers raise."""
    if code != 0:
        message = lib().xb_strerror(code).decode()
        raise RuntimeError(f"{what} failed with code {code}: {message}")


def gfx_arch(device: torch.device) -> str:
    props = torch.cuda.get_device_properties(device)
    return str(getattr(props, "gcnArchName", "")).split(":")[0]


def require_gfx950(tensor: torch.Tensor) -> None:
    """Raise unless `tensor` lives on a gfx950 (MI355X) GPU and the library is loaded."""
    lib()
    if tensor.device.type != "cuda":
        raise ValueError("the HIP kernels require GPU tensors (device 'cuda' on ROCm)")
    arch = gfx_arch(tensor.device)
    if arch != "gfx950":
        raise RuntimeError(f"the xblock kernels are built for gfx950, not {arch!r}")


def stream_handle(device: Optional[torch.device] = None) -> int:
    """hipStream_t of torch's current stream (torch.cuda is HIP on ROCm).

    For a device with an index (every GPU tensor's) the raw handle comes
    straight from torch's C API: building the Stream object that
    torch.cuda.current_stream returns cost several microseconds per launch.
    """
    if isinstance(device, torch.device) and device.index is not None:
        return torch._C._cuda_getCurrentRawStream(device.index)
    return torch.cuda.current_stream(device).cuda_stream
