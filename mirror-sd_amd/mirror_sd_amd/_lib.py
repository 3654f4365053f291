"""ctypes binding of libdflash_hip.so (C ABI declared in include/dflash_hip.h).

The reference reaches its native draft back-end through PyO3 (`mirror_sd_ane`,
ane/src/lib.rs:6-16); this module is the equivalent thin binding.  Errors become
``ValueError`` for bad arguments / capacity (as wrapper.rs:397-406 and
ane_model.py:389-393, 620-624 raise) and ``RuntimeError`` otherwise
(wrapper.rs:204-209).  There is no fallback: if the library is missing, loading
raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libdflash_hip.so"
HERE = os.path.dirname(os.path.abspath(__file__))

DFL_OK, DFL_EINVAL, DFL_ERANGE, DFL_EHIP, DFL_ESTATE = 0, 1, 2, 3, 4

c_void_p = ctypes.c_void_p
c_int32 = ctypes.c_int32
c_int64 = ctypes.c_int64


class DflConfig(ctypes.Structure):
    _fields_ = [
        ("hidden", c_int32), ("n_heads", c_int32), ("n_kv_heads", c_int32),
        ("head_dim", c_int32), ("intermediate", c_int32), ("n_layers", c_int32),
        ("n_target_feat", c_int32), ("vocab", c_int32), ("max_block", c_int32),
        ("max_ctx", c_int32), ("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_double),
        ("max_seqs", c_int32),
    ]


PtrArray7 = c_void_p * 7

# name -> (restype, argtypes); every symbol declared in include/dflash_hip.h
SIGNATURES = {
    "dfl_create": (c_int32, [ctypes.POINTER(DflConfig), ctypes.POINTER(c_void_p)]),
    "dfl_destroy": (c_int32, [c_void_p]),
    "dfl_last_error": (ctypes.c_char_p, []),
    "dfl_quantize_w8": (c_int32, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p]),
    "dfl_load_layer_w8": (c_int32, [c_void_p, c_int32, PtrArray7, PtrArray7, c_void_p, c_void_p,
                                    c_void_p, c_void_p, c_void_p]),
    "dfl_load_fc": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p]),
    "dfl_load_head": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "dfl_ingest_context": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    "dfl_ingest_fused": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    "dfl_ingest_features": (c_int32, [c_void_p, ctypes.POINTER(c_void_p), c_int32,
                                      ctypes.c_int64, c_int32, c_void_p]),
    "dfl_concat_features": (c_int32, [ctypes.POINTER(c_void_p), c_int32, ctypes.c_int64,
                                      c_int32, c_int32, c_void_p, c_void_p]),
    "dfl_draft_block": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_void_p]),
    "dfl_draft_batch": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_int32, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_void_p]),
    "dfl_select_seq": (c_int32, [c_void_p, c_int32]),
    "dfl_set_num_layers": (c_int32, [c_void_p, c_int32]),
    "dfl_cache_trim": (c_int32, [c_void_p, c_int32]),
    "dfl_cache_commit": (c_int32, [c_void_p, c_int32]),
    "dfl_cache_reset": (c_int32, [c_void_p]),
    "dfl_cache_set_window": (c_int32, [c_void_p, c_int32, c_int32]),
    "dfl_cache_rows": (c_int32, [c_void_p, ctypes.POINTER(c_int32), c_int32,
                                 ctypes.POINTER(c_int32)]),
    "dfl_cache_set_offset": (c_int32, [c_void_p, c_int64]),
    "dfl_cache_state": (c_int32, [c_void_p, ctypes.POINTER(c_int32), ctypes.POINTER(c_int64)]),
    "dfl_cache_kv": (c_int32, [c_void_p, c_int32, ctypes.POINTER(c_void_p),
                               ctypes.POINTER(c_void_p), ctypes.POINTER(c_int32)]),
    "dfl_profile_enable": (c_int32, [c_void_p, c_int32]),
    "dfl_profile_read": (c_int32, [c_void_p, c_int32, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                   ctypes.POINTER(c_int64), ctypes.POINTER(c_int64),
                                   ctypes.POINTER(c_int32)]),
    "dfl_embed_block": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_int32, c_int32,
                                  c_int32, c_void_p, c_void_p]),
    "dfl_embed_block_noalloc": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_int32, c_void_p,
                                          c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                          c_void_p]),
    "dfl_device_errors": (c_int32, [c_void_p, ctypes.POINTER(c_int32), c_void_p]),
    "dfl_test_queue_timeout": (c_int32, [c_void_p, c_int32]),
    "dfl_set_sampling": (c_int32, [c_void_p, ctypes.c_float, ctypes.c_uint64]),
    "dfl_cache_assign": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_int32, c_void_p]),
    "dfl_set_rope_scaling": (c_int32, [c_void_p, c_int32, ctypes.c_double, ctypes.c_double,
                                       ctypes.c_double, c_int32]),
}

_lib = None
_lock = threading.Lock()


def lib_path() -> str:
    return os.environ.get("DFL_LIB", os.path.join(HERE, LIB_NAME))


def load():
    """Load the shared library once and attach argument/return types."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"{LIB_NAME} not found at {path}; build it with `python mirror-sd_amd/build.py` "
                "(there is no CPU fallback)")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


class DFlashError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class DFlashValueError(ValueError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


def check(rc: int, what: str):
    if rc == DFL_OK:
        return
    msg = load().dfl_last_error()
    msg = msg.decode("utf-8", "replace") if msg else ""
    text = f"{what} failed ({rc}): {msg}"
    if rc in (DFL_EINVAL, DFL_ERANGE):
        raise DFlashValueError(rc, text)
    raise DFlashError(rc, text)


def ptr(t) -> int:
    """Raw device pointer of a torch tensor (None -> NULL)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_handle(stream=None) -> int:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream
