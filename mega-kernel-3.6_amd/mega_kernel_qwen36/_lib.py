"""ctypes view of the C ABI (``include/mkq.h``) exported by ``libmkq.so``.

This is the binding a non-torch host would write (see the integration notes
for the equivalent C declarations).  Loading the library does not touch the
GPU; calling an entry point does.
"""

from __future__ import annotations

import ctypes
import pathlib
from typing import Optional

_HERE = pathlib.Path(__file__).resolve().parent
_LIB: Optional[ctypes.CDLL] = None

MKQ_OK = 0
MKQ_ERR_INVALID = 1
MKQ_ERR_UNSUPPORTED = 2
MKQ_ERR_HIP = 3

MKQ_DTYPE_F32 = 0
MKQ_DTYPE_F16 = 1
MKQ_DTYPE_BF16 = 2

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/mkq.h one to one.
SIGNATURES = {
    "mkq_last_error": (ctypes.c_char_p, []),
    "mkq_abi_version": (_i, []),
    "mkq_moe_decode_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "mkq_moe_decode": (
        _i,
        [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
         _i, _i, _i, _i, _i, _i, _f, _i, _vp, _sz, _vp],
    ),
    "mkq_moe_decode_status": (_i, [_vp, _sz, _i, ctypes.POINTER(_i), _vp]),
    "mkq_moe_decode_noalloc": (
        _i,
        [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
         _i, _i, _i, _i, _i, _i, _f, _i, _vp],
    ),
    "mkq_dense_ffn_decode_workspace_bytes": (_sz, [_i, _i, _i]),
    "mkq_dense_ffn_decode": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _i, _vp, _sz, _vp]),
    "mkq_full_attention_decode_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "mkq_full_attention_decode": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp, _sz, _vp]),
    "mkq_full_attention_decode_rope": (
        _i, [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp, _i, _vp, _sz, _vp]),
    "mkq_full_attention_decode_paged_append": (
        _i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _f, _vp, _sz, _vp]),
    "mkq_full_attention_decode_paged_append_rope": (
        _i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _f, _vp, _i, _vp, _sz, _vp]),
    "mkq_full_attention_decode_paged_rope": (
        _i, [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _f, _vp, _i, _vp, _sz, _vp]),
    "mkq_full_attention_decode_paged": (
        _i, [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _f, _vp, _sz, _vp]),
    "mkq_full_attention_decode_append": (
        _i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _vp, _i, _vp, _sz, _vp]),
    "mkq_linear_attention_decode": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp]),
    "mkq_gated_delta_decode": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "mkq_gated_delta_decode_qknorm": (
        _i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp]),
    "mkq_causal_conv1d_update": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "mkq_gated_rms_norm": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _f, _vp]),
    "mkq_linear_attention_step_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "mkq_linear_attention_step": (_i, [_i, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                       _f, _f, _vp, _sz, _vp]),
    "mkq_gemv": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "mkq_gemv_add": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "mkq_rms_norm_gemv": (_i, [_i, _vp, _vp, _f, _vp, _vp, _i, _i, _i, _vp]),
}


def library_path() -> pathlib.Path:
    return _HERE / "libmkq.so"


def load_library() -> ctypes.CDLL:
    """Load ``libmkq.so`` (once) and attach the argument types of every entry point."""
    global _LIB
    if _LIB is None:
        path = library_path()
        if not path.exists():
            raise RuntimeError(f"{path} is not built; run mega-kernel-3.6_amd/build.py")
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB


def check(rc: int, op: str) -> None:
    if rc != MKQ_OK:
        msg = load_library().mkq_last_error().decode(errors="replace")
        raise RuntimeError(f"{op} failed (status {rc}): {msg}")
