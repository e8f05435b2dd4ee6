"""ctypes binding of libwan_attn.so, the C ABI declared in include/wan_attn.h.

torch is imported first on purpose: the library is linked against the HIP
runtime by soname (libamdhip64.so.7), and the dynamic loader resolves that to
the copy torch has already loaded, so tensors, streams and kernels share one
runtime.  Loading fails loudly when the library has not been built; there is
no fallback path.
"""
import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see above)

LIB_NAME = "libwan_attn.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)


class WanTensor(ctypes.Structure):
    """struct wan_tensor: a [batch, token, head, 128] bf16 device view."""
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("batch_stride", ctypes.c_int64),
        ("token_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_L = ctypes.c_int64
_T = WanTensor

# name -> (restype, argtypes), one entry per function in include/wan_attn.h
SIGNATURES = {
    "wan_attn_last_error": (ctypes.c_char_p, []),
    "wan_attn_abi_version": (_I, []),
    "wan_attn_init": (_I, []),
    "wan_flash_self_attn": (_I, [_T, _T, _T, _T, _I, _I, _I, _I, _I, _F, _I, _P]),
    "wan_cross_attn": (_I, [_T, _T, _T, _T, _I, _I, _I, _I, _I, _F, _P, _P]),
    "wan_self_attn_fused_workspace": (_SZ, [_I, _I, _I]),
    "wan_self_attn_fused": (_I, [_T, _T, _T, _T, _I, _I, _I, _I, _P, _P, _F, _P, _P, _F, _P, _SZ, _P]),
    "wan_cross_attn_fused_workspace": (_SZ, [_I, _I, _I]),
    "wan_cross_attn_fused": (_I, [_T, _T, _T, _T, _I, _I, _I, _I, _I, _P, _F, _F, _P, _P, _SZ, _P]),
    "wan_cross_attn_fused_noalloc": (_I, [_T, _T, _T, _T, _I, _I, _I, _I, _I, _P, _F, _F, _P, _P]),
    "wan_rope": (_I, [_T, _P, _I, _I, _I, _I, _P, _P, _P]),
    "wan_rms_norm": (_I, [_T, _P, _I, _I, _I, _I, _P, _F, _P, _P, _P, _P]),
    "wan_rms_norm_qk": (_I, [_T, _T, _P, _I, _I, _I, _I, _P, _F, _P, _P, _P, _P]),
    "wan_flash_attn_qnorm": (_I, [_T, _T, _T, _T, _I, _I, _I, _I, _I, _P, _P, _P, _P, _F, _P, _P]),
    "wan_adaln": (_I, [_P, _P, _P, _P, _I, _I, _I, _P, _I, _I, _I, _I, _P, _P, _F, _P]),
    "wan_adaln_ex": (_I, [_P, _P, _P, _P, _I, _I, _I, _P, _I, _I, _P, _I, _I, _I, _P, _P, _F, _P]),
    "wan_qkv_proj_sumsq": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _L, _L, _L, _I, _P]),
    "wan_rms_norm_qk_sumsq": (_I, [_T, _P, _I, _I, _I, _I, _P, _F, _P, _P, _P, _P, _P]),
}

ABI_VERSION = 1

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library (loaded on first use). Raises if it is missing or stale."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python __graft_entry__.py build` "
                "(or wan2-ti2v-5b_amd/build.py) first")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.wan_attn_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI version {handle.wan_attn_abi_version()} != {ABI_VERSION}")
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().wan_attn_last_error().decode(errors="replace")


def check(fn_name: str, rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"{fn_name} failed (code {rc}): {last_error()}")


def tensor4(x: "torch.Tensor") -> WanTensor:
    """wan_tensor for a [B, L, H, 128] tensor (strides in elements)."""
    return WanTensor(x.data_ptr(), x.stride(0), x.stride(1), x.stride(2))
