"""ctypes binding of the gfx950 kernel library (include/claudemaxing_amd.h).

The library is loaded on first use, after torch (so it shares torch's HIP runtime and its
streams). A missing or mismatched library raises ImportError; a non-zero return code of an
entry point raises RuntimeError with the library's error string. There is no other code path:
the kernels either run on the GPU or the call fails.
"""

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libclaudemaxing_amd.so"
ABI_VERSION = 9

F32, F16, BF16, U8, I32, I64 = 0, 1, 2, 3, 4, 5
_DTYPE_CODES = {
    torch.float32: F32,
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.uint8: U8,
    torch.bool: U8,
    torch.int32: I32,
    torch.int64: I64,
}

_P, _I, _L, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float


class NF4Weight(ctypes.Structure):
    """cm_nf4_weight: one NF4 weight's device pointers and sizes."""

    _fields_ = [
        ("packed", ctypes.c_void_p),
        ("absmax", ctypes.c_void_p),
        ("nested", ctypes.c_int),
        ("code", ctypes.c_void_p),
        ("code2", ctypes.c_void_p),
        ("absmax2", ctypes.c_void_p),
        ("offset", ctypes.c_void_p),
        ("blocksize", ctypes.c_int),
        ("blocksize2", ctypes.c_int),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("scale_map", ctypes.c_void_p),
    ]


_PW = ctypes.POINTER(NF4Weight)
_PP = ctypes.POINTER(ctypes.c_void_p)
_PL = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); mirrors include/claudemaxing_amd.h
SIGNATURES = {
    "cm_abi_version": (_I, []),
    "cm_error_string": (ctypes.c_char_p, [_I]),
    "cm_nf4_dequant": (_I, [_P, _P, _I, _P, _P, _P, _P, _P, _I, _L, _I, _I, _P]),
    "cm_nf4_dequant_t": (_I, [_P, _P, _I, _P, _P, _P, _P, _P, _L, _L, _I, _I, _P]),
    "cm_gemm_f32_workspace_bytes": (_L, [_I, _I, _I, _I]),
    "cm_lora_weight_grads_workspace_bytes": (_L, [_L, _I, _I]),
    "cm_lora_weight_grads": (_I, [_P, _P, _P, _P, _P, _P, _I, _L, _I, _P, _L, _P]),
    "cm_gemm_f32": (_I, [_P, _L, _P, _L, _I, _P, _L, _P, _L, _I, _I, _I, _P, _P, _L, _P]),
    "cm_gemm_f32_kb": (_I, [_P, _L, _P, _L, _I, _P, _L, _P, _L, _I, _I, _I, _P, _P, _L, _P]),
    "cm_gemm_f32_add": (_I, [_P, _L, _P, _L, _I, _P, _L, _P, _L, _I, _I, _I, _P, _P, _P, _L,
                             _P]),
    "cm_rmsnorm_fwd": (_I, [_P, _I, _L, _P, _I, _P, _I, _P, _P, _P, _P, _I, _L, _I, _F, _P]),
    "cm_rmsnorm_bwd": (_I, [_P, _I, _P, _I, _P, _I, _P, _P, _I, _P, _P, _P, _I, _I, _L, _I, _P]),
    "cm_rmsnorm_bwd_partials": (_L, [_L]),
    "cm_rmsnorm_add_fwd": (_I, [_P, _P, _I, _L, _P, _I, _P, _P, _P, _P, _P, _P, _I, _L, _I, _F,
                                _P]),
    "cm_rmsnorm_bwd_res": (_I, [_P, _I, _P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _L,
                                _I, _P]),
    "cm_rope": (_I, [_P, _I, _L, _L, _L, _I, _P, _I, _P, _I, _L, _L, _L, _I, _P, _I, _P, _P, _I,
                     _L, _L, _I, _I, _I, _I, _P]),
    "cm_swiglu_fwd": (_I, [_P, _I, _P, _I, _P, _I, _L, _I, _P]),
    "cm_swiglu_bwd": (_I, [_P, _I, _P, _I, _P, _I, _P, _P, _L, _I, _I, _I, _P]),
    "cm_swiglu_fwd_rows": (_I, [_P, _I, _P, _I, _L, _P, _I, _L, _L, _L, _I, _P]),
    "cm_swiglu_bwd_rows": (_I, [_P, _I, _L, _P, _I, _P, _I, _L, _P, _P, _L, _L, _I, _I, _I, _P]),
    "cm_lora_pack": (_I, [_P, _I, _P, _P, _P, _L, _F, _P]),
    "cm_lora_unpack": (_I, [_P, _P, _P, _P, _P, _I, _L, _F, _P]),
    "cm_xent_rows": (_I, [_P, _I, _L, _P, _P, _P, _P, _L, _L, _I, _F, _P]),
    "cm_lmhead_ce": (_I, [_P, _L, _P, _L, _P, _L, _L, _I, _L, _P, _P, _P, _P, _F, _P, _L, _P]),
    "cm_lmhead_ce_workspace_bytes": (_L, [_L, _L, _I, _L]),
    "cm_lmhead_ce_plan": (_I, [_L, _L, _I, _L, _P, _P]),
    "cm_lmhead_ce_noalloc_plan": (_I, [_L, _L, _I, _L, _I, _P, _P]),
    "cm_lmhead_ce_noalloc": (_I, [_P, _L, _P, _L, _P, _L, _L, _I, _L, _P, _P, _P, _P, _F, _P]),
    "cm_attn_fwd": (_I, [_P, _I, _L, _L, _P, _I, _L, _L, _P, _I, _L, _L, _P, _L, _L, _I, _I, _I,
                         _F, _P, _P, _P, _L, _P]),
    "cm_attn_bwd": (_I, [_P, _I, _L, _L, _P, _I, _L, _L, _P, _I, _L, _L, _P, _P, _P, _P, _L, _L,
                         _I, _I, _I, _F, _P, _I, _P, _P, _I, _I, _P, _L, _P]),
    "cm_attn_fwd_rope": (_I, [_P, _I, _L, _L, _P, _I, _L, _L, _P, _I, _L, _L, _P, _P, _L, _P, _L,
                              _L, _I, _I, _I, _F, _P, _P, _P, _L, _P]),
    "cm_attn_bwd_rope": (_I, [_P, _I, _L, _L, _P, _I, _L, _L, _P, _I, _L, _L, _P, _P, _L, _P, _P,
                              _P, _P, _L, _L, _I, _I, _I, _F, _P, _I, _P, _I, _P, _I, _I, _P, _L,
                              _P]),
    "cm_attn_padded_tokens": (_L, [_P, _I]),
    "cm_attn_rows_bytes": (_L, []),
    "cm_attn_rows_image": (_L, [_P, _I, _P]),
    "cm_lora_fused_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _L, _I, _I, _I, _F, _F, _P]),
    "cm_lora_fused_bwd1": (_I, [_P, _P, _P, _P, _P, _L, _I, _I, _F, _P]),
    "cm_lora_fused_fwd_multi": (_I, [_P, _L, _I, _I, _F, _F, _I, _PP, _PP, _PP, _PP, _PP, _PP,
                                     _PP, _P, _P]),
    "cm_lora_fused_bwd1_multi": (_I, [_L, _I, _F, _I, _PP, _PP, _PP, _PP, _PP, _P, _P]),
    "cm_lora_fused_bwd2": (_I, [_P, _P, _P, _P, _P, _P, _P, _L, _I, _I, _F, _P]),
    "cm_attn_workspace_bytes": (_L, [_L, _I, _I, _I, _I]),
    "cm_nf4_linear_fwd": (_I, [_P, _L, _L, _PW, _I, _PP, _PP, _PL, _I, _P, _L, _P]),
    "cm_nf4_linear_bwd": (_I, [_PP, _PL, _L, _PW, _I, _P, _L, _I, _P, _L, _P]),
    "cm_nf4_linear_workspace_bytes": (_L, [_L, _PW, _I, _I]),
    "cm_probe_hbm": (_I, [_P, _P, _L, _I, _I, _P, _P]),
    "cm_probe_mfma_f16": (_I, [_P, _I, _I, _P, _P]),
    "cm_probe_mfma_f16_flops": (_L, [_I, _I]),
    "cm_probe_launch": (_I, [_I, _I, _P]),
    "cm_nf4_scale_map": (_I, [_PW, _P, _P]),
    "cm_nf4_dequant_group": (_I, [_PW, _I, _PP, _I, _P]),
}

_lock = threading.Lock()
_lib = None


def load():
    """The loaded library (ctypes.CDLL); ImportError if it is missing or its ABI differs."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build the gfx950 kernel library first "
                "(python -m claudemaxing_amd.build_lib)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                raise ImportError(f"{LIB_PATH} does not export {name}")
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.cm_abi_version()
        if version != ABI_VERSION:
            raise ImportError(f"{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


def call(name, *args):
    """Call entry point `name`; raise RuntimeError with the library's message on failure."""
    lib = load()
    code = getattr(lib, name)(*args)
    if code != 0:
        msg = lib.cm_error_string(code).decode()
        raise RuntimeError(f"{name} failed: {msg} (code {code})")


def dtype_code(dtype):
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}") from None


def ptr(t):
    """Device address of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


# torch's C accessor of the current stream's raw handle (what torch.cuda.current_stream(d)
# .cuda_stream returns, without building a Stream object: 0.07 us against 1.9 us per call on the
# MI355X box's host, and every launch asks for it); the public call where it is absent
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(device=None):
    """Handle of torch's current stream on `device`, for the stream argument."""
    if _RAW_STREAM is None:
        return torch.cuda.current_stream(device).cuda_stream
    if isinstance(device, torch.device):
        index = device.index
    elif device is None:
        index = None
    else:
        index = torch.device(device).index if isinstance(device, str) else int(device)
    if index is None:
        index = torch.cuda.current_device()
    return _RAW_STREAM(index)
