"""ctypes binding of ``libtree_attn.so`` (C ABI declared in include/tree_attn.h).

The library is loaded on first use.  ``torch`` is imported first so that the
library binds to the HIP runtime torch already loaded (both carry the soname
``libamdhip64.so.7``); stream handles from ``torch.cuda`` are then valid here.
There is no fallback: if the library is missing, every call raises.  The
environment variable ``TREE_ATTN_LIB`` selects another build of the library.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).with_name("libtree_attn.so")

TA_BF16, TA_FP16 = 0, 1
TA_SMALL, TA_LARGE64, TA_LARGE128, TA_LARGE256, TA_TAIL = 0, 1, 2, 3, 4
TA_NKINDS = 5
TA_ERR_ARG = 1001
TA_ERR_SCRATCH = 1004
NOALLOC_SCRATCH_BYTES = 32 << 20  # TA_NOALLOC_SCRATCH_BYTES
KIND_ROWS = {TA_LARGE64: 64, TA_LARGE128: 128, TA_LARGE256: 256}

_c_i32 = ctypes.c_int32
_c_ptr = ctypes.c_void_p

EXPORTS = ("ta_version", "ta_error_string", "ta_segment", "ta_merge", "ta_attention_matrix",
           "ta_attention_matrix_noalloc", "ta_tail_merge", "ta_segment_plan", "ta_merge_plan", "ta_decode_append", "ta_time_next_launch",
           "ta_read_stream")


class TaPlan(ctypes.Structure):
    """Mirror of ``struct ta_plan`` in include/tree_attn.h (same field order)."""
    _fields_ = [
        ("qids", _c_ptr), ("kstart", _c_ptr), ("qlen", _c_ptr), ("klen", _c_ptr),
        ("rowbase", _c_ptr), ("slots", _c_ptr), ("counts", _c_ptr),
        ("items", _c_ptr * TA_NKINDS), ("n_items", _c_i32 * TA_NKINDS), ("rest", _c_ptr),
        ("part", _c_ptr), ("lse", _c_ptr),
        ("njobs", _c_i32), ("maxr", _c_i32), ("maxs", _c_i32), ("nreq", _c_i32), ("nslot", _c_i32),
        ("hq", _c_i32), ("hk", _c_i32), ("d", _c_i32), ("dtype", _c_i32), ("n_rest", _c_i32),
        ("xtail", _c_ptr), ("xtail_stride", _c_i32), ("qbase", _c_ptr), ("slot_stride", _c_i32),
    ]


_lib = None
_lock = threading.Lock()


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and return the native library, with prototypes set."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        import torch  # noqa: F401  -- bind to torch's HIP runtime first
        target = Path(path) if path is not None else Path(os.environ.get("TREE_ATTN_LIB", LIB_PATH))
        if not target.exists():
            raise RuntimeError(
                f"tree_attn native library not found at {target}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` from the repository root")
        lib = ctypes.CDLL(str(target))
        lib.ta_version.restype = ctypes.c_char_p
        lib.ta_version.argtypes = []
        lib.ta_error_string.restype = ctypes.c_char_p
        lib.ta_error_string.argtypes = [ctypes.c_int]
        lib.ta_segment.restype = ctypes.c_int
        lib.ta_segment.argtypes = [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                   _c_ptr, _c_i32, _c_i32, _c_ptr, _c_ptr,
                                   _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_ptr]
        lib.ta_merge.restype = ctypes.c_int
        lib.ta_merge.argtypes = [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                 _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_ptr]
        lib.ta_attention_matrix.restype = ctypes.c_int
        lib.ta_attention_matrix.argtypes = [_c_ptr, _c_ptr, _c_ptr, _c_i32, ctypes.POINTER(TaPlan),
                                            _c_ptr, _c_ptr]
        lib.ta_attention_matrix_noalloc.restype = ctypes.c_int
        lib.ta_attention_matrix_noalloc.argtypes = [_c_ptr, _c_ptr, _c_ptr, _c_i32, ctypes.POINTER(TaPlan),
                                                    _c_ptr, _c_ptr]
        lib.ta_tail_merge.restype = ctypes.c_int
        lib.ta_tail_merge.argtypes = [_c_ptr, _c_ptr, _c_ptr, _c_i32, ctypes.POINTER(TaPlan), _c_ptr, _c_ptr]
        lib.ta_merge_plan.restype = ctypes.c_int
        lib.ta_merge_plan.argtypes = [ctypes.POINTER(TaPlan), _c_ptr, _c_ptr]
        lib.ta_segment_plan.restype = ctypes.c_int
        lib.ta_segment_plan.argtypes = [_c_ptr, _c_ptr, _c_ptr, _c_i32, ctypes.POINTER(TaPlan), _c_i32, _c_ptr]
        lib.ta_decode_append.restype = ctypes.c_int
        lib.ta_decode_append.argtypes = [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i32, _c_ptr, _c_ptr, _c_ptr,
                                         _c_ptr, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_ptr]
        lib.ta_time_next_launch.restype = ctypes.c_int
        lib.ta_time_next_launch.argtypes = [_c_ptr, _c_ptr]
        lib.ta_read_stream.restype = ctypes.c_int
        lib.ta_read_stream.argtypes = [_c_ptr, ctypes.c_int64, _c_ptr, _c_i32, _c_ptr]
        if path is None:
            _lib = lib
        return lib


def check(rc: int) -> None:
    """Raise ``RuntimeError`` for a non-zero return code of the library."""
    if rc:
        msg = load().ta_error_string(rc).decode()
        raise RuntimeError(f"tree_attn call failed ({rc}): {msg}")
