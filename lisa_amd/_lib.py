"""ctypes binding of liblisaq.so (the C ABI declared in include/lisaq.h).

The library is built in-tree by ``lisa_amd.build``.  Loading fails loudly when
it is missing: there is no CPU or PyTorch fallback for any op.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblisaq.so")

OK, EINVAL_SHAPE, EINVAL_DTYPE, EINVAL_LAYOUT, EUNSUPPORTED, EHIP, EWORKSPACE = range(7)
DTYPE_BF16, DTYPE_F32, DTYPE_F16 = 0, 1, 2

_STATUS_NAMES = {
    EINVAL_SHAPE: "EINVAL_SHAPE",
    EINVAL_DTYPE: "EINVAL_DTYPE",
    EINVAL_LAYOUT: "EINVAL_LAYOUT",
    EUNSUPPORTED: "EUNSUPPORTED",
    EHIP: "EHIP",
    EWORKSPACE: "EWORKSPACE",
}


class LisaqError(RuntimeError):
    """A non-zero lisaq_status; ``code`` is the status, the message comes from lisaq_last_error()."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{_STATUS_NAMES.get(code, code)}] {msg}")
        self.code = code


vp = ctypes.c_void_p
i64 = ctypes.c_int64
ci = ctypes.c_int
sz = ctypes.c_size_t
i64p = ctypes.POINTER(ctypes.c_int64)
cip = ctypes.POINTER(ctypes.c_int)

# name -> (restype, argtypes); must match include/lisaq.h
SIGNATURES = {
    "lisaq_version": (ci, []),
    "lisaq_last_error": (ctypes.c_char_p, []),
    "lisaq_set_path_override": (ci, [ctypes.c_char_p, ci]),
    "lisaq_read_stream": (ci, [vp, vp, sz, ci, vp]),
    "lisaq_timestamp": (ci, [vp, vp]),
    "lisaq_quantized_matmul": (ci, [vp, vp, vp, vp, vp, vp, i64, i64, i64, ci, ci, ci, vp, sz]),
    "lisaq_quantized_matmul_workspace": (sz, [i64, i64, i64, ci, ci]),
    "lisaq_quantized_matmul_noalloc": (ci, [vp, vp, vp, vp, vp, vp, i64, i64, i64, ci, ci, ci]),
    "lisaq_qmm_workspace": (sz, [i64, i64, i64, ci, ci]),
    "lisaq_quantized_matmul_serial_rows": (ci, [vp, vp, vp, vp, vp, vp, i64, i64, i64, ci, ci, ci, vp, sz]),
    "lisaq_qmv": (ci, [vp, vp, vp, vp, vp, vp, i64, i64, i64, ci, ci, vp, sz]),
    "lisaq_qmm": (ci, [vp, vp, vp, vp, vp, vp, i64, i64, i64, ci, ci, vp, sz]),
    "lisaq_dequantize": (ci, [vp, vp, vp, vp, vp, i64, i64, ci, ci]),
    "lisaq_quantize": (ci, [vp, vp, ci, vp, vp, vp, i64, i64, ci, ci]),
    "lisaq_qmv_addnorm": (ci, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, ctypes.c_float,
                               ci, ci, vp, sz]),
    "lisaq_moe_route": (ci, [vp, vp, i64, ci, ci, vp, vp]),
    "lisaq_moe_sort": (ci, [vp, vp, i64, ci, ci, vp, vp, vp, vp, vp]),
    "lisaq_gather_rows": (ci, [vp, vp, vp, vp, i64, i64]),
    "lisaq_gather_qmm": (ci, [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, ci, ci, ci, ci, vp, sz]),
    "lisaq_gather_qmm_workspace": (sz, [i64, i64, i64, ci, ci, ci]),
    "lisaq_swiglu": (ci, [vp, vp, vp, vp, i64]),
    "lisaq_gather_qmm_swiglu": (ci, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, ci, ci, ci, vp, sz]),
    "lisaq_gather_qmm_swiglu_workspace": (sz, [i64, i64, ci]),
    "lisaq_quantized_matmul_typed": (ci, [vp, vp, vp, vp, vp, vp, i64, i64, i64, ci, ci, ci, ci, vp, sz]),
    "lisaq_moe_decode_supported": (ci, [i64, i64, i64, ci, ci, ci, ci]),
    "lisaq_moe_combine": (ci, [vp, vp, vp, vp, vp, i64, ci, i64]),
    "lisaq_moe_forward": (ci, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                               i64, i64, i64, ci, ci, ci, ci, vp, vp, vp, sz]),
    "lisaq_moe_workspace": (sz, [i64, i64, i64, ci, ci, ci, ci]),
    "lisaq_detect_group_size": (ci, [i64, i64, ci]),
    "lisaq_qmv_batch_limit": (ci, [i64, i64]),
    "lisaq_check_layout": (ci, [i64, i64, i64, i64, i64, i64, ci, i64p, cip]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load liblisaq.so (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"liblisaq.so not found at {LIB_PATH}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` (no fallback exists)"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        raise LisaqError(rc, load().lisaq_last_error().decode(errors="replace"))


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


PATH_DEFAULT = -(2**31)


def set_path_override(name: str, value) -> None:
    """Force a dispatch path (test/diagnostic; see lisaq_set_path_override).
    ``value``: an int, a kernel letter string (first character used) or None
    for the dispatcher's own choice."""
    if value is None:
        v = PATH_DEFAULT
    elif isinstance(value, str):
        v = int(value) if value.lstrip("-").isdigit() and name != "LISAQ_QMV_KERNEL" else ord(value[0])
    else:
        v = int(value)
    check(load().lisaq_set_path_override(name.encode(), v))
