"""ctypes binding of libgqa.so (declared in include/gqa.h).

The library is built in-tree by ``lara_amd.build`` (or ``__graft_entry__.build()``).
Loading never builds and never falls back: if the shared object is missing or cannot
be loaded, :func:`lib` raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, Structure, c_double, c_float, c_int32, c_int64, c_uint16, c_uint32, c_uint64, c_void_p
from pathlib import Path
from typing import Optional

LIB_PATH = Path(__file__).resolve().parent / "libgqa.so"

# Status codes (include/gqa.h); 0x01..0x12 match error_code_t of attn_pkg.sv:279-286.
GQA_OK = 0x00
GQA_ERR_BAD_CFG = 0x01
GQA_ERR_BUSY_START = 0x02
GQA_ERR_STREAM_LEN = 0x10
GQA_ERR_STREAM_DEST = 0x11
GQA_ERR_RESULT_LEN = 0x12
GQA_ERR_HIP = 0x20
GQA_ERR_OOM = 0x21
GQA_ERR_NO_DEVICE = 0x22
GQA_ERR_NULL = 0x23
GQA_ERR_RANGE = 0x24
GQA_ERR_TIMEOUT = 0x25
GQA_ERR_NO_TRANSACTION = 0x26
GQA_ERR_UNSUPPORTED = 0x27
GQA_ERR_SCRATCH = 0x28
GQA_NOALLOC_SCRATCH_BYTES = 16 << 20

GQA_STATUS_START_READY = 1 << 0
GQA_STATUS_BUSY = 1 << 1
GQA_STATUS_DONE = 1 << 2
GQA_STATUS_ERROR = 1 << 3

GQA_TIMER_APPEND = 0
GQA_TIMER_DECODE = 1
GQA_TIMER_COMBINE = 2
GQA_TIMER_PREFILL = 3
GQA_TIMER_NORM = 4
GQA_TIMER_PROJECTION = 5
GQA_TIMER_ROPE = 6
GQA_TIMER_COUNT = 7

GQA_OPT_DECODE_CHUNK = 1
GQA_OPT_PROFILE = 2
GQA_OPT_PREFILL_WGS = 3
GQA_OPT_NUMERICS = 4
GQA_OPT_DECODE_MERGE = 5
GQA_DECODE_MERGE_AUTO = 0
GQA_DECODE_MERGE_LAUNCH = 1
GQA_DECODE_MERGE_FUSED = 2
GQA_OPT_PREFILL_KERNEL = 6
GQA_OPT_LAYER = 7
GQA_MAX_LAYERS = 1024
GQA_PREFILL_KERNEL_AUTO = 0
GQA_PREFILL_KERNEL_SHARED = 1
GQA_PREFILL_KERNEL_ROWS = 2
GQA_PREFILL_KERNEL_PAIRED = 3
GQA_NUMERICS_EXACT = 0
GQA_NUMERICS_KV260 = 1


class GqaConfig(Structure):
    _fields_ = [
        ("batch", c_int32),
        ("n_q_heads", c_int32),
        ("n_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("max_seq_len", c_int32),
        ("max_q_len", c_int32),
        ("scale", c_float),
        ("device", c_int32),
    ]


class GqaError(RuntimeError):
    """A libgqa call returned a non-zero status."""

    def __init__(self, code: int, where: str, message: str) -> None:
        super().__init__(f"{where}: status 0x{code:02x} ({message})")
        self.code = code


_P16 = POINTER(c_uint16)
_P32 = POINTER(c_int32)
_PF = POINTER(c_float)
_CTX = c_void_p

# name -> argtypes; every function returns int (status)
_SIGNATURES = {
    "gqa_create": [POINTER(GqaConfig), POINTER(c_void_p)],
    "gqa_create_paged": [POINTER(GqaConfig), c_int32, c_int32, POINTER(c_void_p)],
    "gqa_create_paged_layers": [POINTER(GqaConfig), c_int32, c_int32, c_int32, POINTER(c_void_p)],
    "gqa_paged_layers": [_CTX, _P32, _P32],
    "gqa_destroy": [_CTX],
    "gqa_get_config": [_CTX, POINTER(GqaConfig)],
    "gqa_set_option": [_CTX, c_int32, c_int64],
    "gqa_device_count": [_P32],
    "gqa_load_kv": [_CTX, c_int32, c_int32, c_int32, _P16, _P16],
    "gqa_append_kv": [_CTX, _P16, _P16, _P32],
    "gqa_read_kv": [_CTX, c_int32, c_int32, c_int32, _P16, _P16],
    "gqa_decode": [_CTX, _P16, _P32, _P16, _PF],
    "gqa_decode_append": [_CTX, _P16, _P16, _P16, _P32, _P32, _P16, _PF],
    "gqa_prefill": [_CTX, c_int32, _P16, c_int32, c_int32, c_int32, c_int32, c_int32, _P16, _PF],
    "gqa_prefill_append": [_CTX, c_int32, _P16, _P16, _P16, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
                           _P16, _PF],
    "gqa_submit": [_CTX, c_int32, _P16, c_int32, c_int32, c_int32, c_int32, c_int32],
    "gqa_start": [_CTX],
    "gqa_status": [_CTX, POINTER(c_uint32)],
    "gqa_wait": [_CTX, c_int32],
    "gqa_read_output": [_CTX, _P16, c_int64],
    "gqa_read_perf": [_CTX, POINTER(c_uint64), POINTER(c_uint64), POINTER(c_uint64), POINTER(c_double)],
    "gqa_load_kv_device": [_CTX, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p],
    "gqa_append_kv_device": [_CTX, c_void_p, c_void_p, c_void_p, c_void_p],
    "gqa_decode_device": [_CTX, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    "gqa_decode_append_device": [_CTX, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                 c_void_p],
    "gqa_decode_append_noalloc": [POINTER(GqaConfig), c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    "gqa_prefill_device": [_CTX, c_int32, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_void_p,
                           c_void_p, c_void_p],
    "gqa_prefill_append_device": [_CTX, c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32,
                                  c_int32, c_int32, c_void_p, c_void_p, c_void_p],
    "gqa_cache_pointers": [_CTX, POINTER(c_void_p), POINTER(c_void_p), _P32],
    "gqa_paged_reserve": [_CTX, c_int32, c_int32],
    "gqa_paged_release": [_CTX, c_int32],
    "gqa_paged_evict_lru": [_CTX, c_int32, _P32, c_int32, _P32, c_int32, _P32],
    "gqa_paged_info": [_CTX, _P32, _P32, _P32, _P32],
    "gqa_paged_table": [_CTX, c_int32, _P32, c_int32],
    "gqa_submit_layer": [_CTX, c_int32, _P16, c_int32, c_int32, _P16, _P16, _P16, _P16, c_float, c_int32, c_int32,
                         c_int32, c_int32],
    "gqa_layer_qkv_device": [_CTX, c_int32, c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p,
                             c_float, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p],
    "gqa_layer_times": [_CTX, _PF, c_int32],
    "gqa_graph_capture_decode_append": [_CTX, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                        POINTER(c_void_p)],
    "gqa_graph_launch": [c_void_p, c_void_p],
    "gqa_graph_destroy": [c_void_p],
    "gqa_stream_read_device": [c_void_p, c_int64, c_int32, c_int32, c_void_p, c_void_p],
    "gqa_last_elapsed_us": [_CTX, _PF],
    "gqa_kernel_times": [_CTX, _PF, c_int32],
    "gqa_kernel_launch_counts": [_CTX, _P32, c_int32],
    "gqa_kernel_durations": [_CTX, c_int32, _PF, c_int32, _P32],
    "gqa_synchronize": [_CTX],
    "gqa_last_prefill_plan": [_CTX, _P32, _P32],
}

EXPORTED = tuple(_SIGNATURES) + ("gqa_status_string",)

_LIB: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load libgqa.so once; raise RuntimeError when it is not built or cannot load."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.is_file():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m lara_amd.build` (hipcc, gfx950). "
            "There is no CPU fallback for the attention engine."
        )
    handle = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = argtypes
        fn.restype = c_int32
    handle.gqa_status_string.argtypes = [c_int32]
    handle.gqa_status_string.restype = ctypes.c_char_p
    _LIB = handle
    return handle


def status_string(code: int) -> str:
    return lib().gqa_status_string(int(code)).decode("utf-8", "replace")


def check(code: int, where: str) -> None:
    if code != GQA_OK:
        raise GqaError(int(code), where, status_string(code))


def device_count() -> int:
    n = c_int32(0)
    check(lib().gqa_device_count(ctypes.byref(n)), "gqa_device_count")
    return int(n.value)


def as_u16_ptr(arr) -> "ctypes._Pointer":
    return arr.ctypes.data_as(_P16)


def as_i32_ptr(arr) -> "ctypes._Pointer":
    return arr.ctypes.data_as(_P32)


def as_f32_ptr(arr) -> "ctypes._Pointer":
    return arr.ctypes.data_as(_PF)
