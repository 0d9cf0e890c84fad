"""ctypes binding of oracle/librtl_exact.so, the C restatement of the KV260 bit-level
arithmetic (TEST INFRASTRUCTURE: only tests/ use it, as the oracle of the RTL-exact mode).

Build it with ``make -C oracle`` (``__graft_entry__.build()`` does).  The ROM tables come from
``lara_amd/data/*.hex`` (closed forms, pinned by SHA-256 to the board's ROM images).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "librtl_exact.so"
DATA = HERE.parent / "lara_amd" / "data"

# Mistakes the C library can plant on purpose (rtl_attention_planted), so tests can show that
# their word-level checks reject each one.
PLANT_P_RNE = 1             # P rounded to nearest even instead of truncated to its upper half
PLANT_SUM_REVERSED = 2      # a sub-block's row sum and PV sum taken from key 15 down
PLANT_FLAT_ACCUMULATE = 4   # O accumulated key by key instead of one delta per sub-block
PLANT_TILE_RESCALE = 8      # running max per 64-key tile instead of per 16-key sub-block
PLANT_EXACT_DIVIDE = 16     # O / l (IEEE) instead of O x R(l)
PLANT_QK_REVERSED = 32      # Q.K summed from the last dimension down
PLANT_FRAC_RNE = 64         # the exp table's interpolation fraction rounded to nearest instead of truncated
PLANTS = {"p_rne": PLANT_P_RNE, "sum_reversed": PLANT_SUM_REVERSED, "flat_accumulate": PLANT_FLAT_ACCUMULATE,
          "tile_rescale": PLANT_TILE_RESCALE, "exact_divide": PLANT_EXACT_DIVIDE, "qk_reversed": PLANT_QK_REVERSED,
          "frac_rne": PLANT_FRAC_RNE}

_U32 = ctypes.POINTER(ctypes.c_uint32)
_U16 = ctypes.POINTER(ctypes.c_uint16)
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            raise RuntimeError(f"{LIB_PATH} is not built; run `make -C oracle`")
        h = ctypes.CDLL(str(LIB_PATH))
        for name in ("rtl_fp32_add_n", "rtl_fp32_mul_n"):
            getattr(h, name).argtypes = [_U32, _U32, _U32, ctypes.c_int64]
        h.rtl_bf16_mul_n.argtypes = [_U16, _U16, _U32, ctypes.c_int64]
        h.rtl_exp_lookup_n.argtypes = [_U32, _U32, _U32, ctypes.c_int64]
        h.rtl_recip_lookup_n.argtypes = [_U32, _U32, _U32, ctypes.c_int64]
        h.rtl_attention.argtypes = [_U16, _U16, _U16, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint32, _U32, _U32, _U16,
                                    _U32, _U32]
        h.rtl_attention_planted.argtypes = h.rtl_attention.argtypes + [ctypes.c_int]
        _lib = h
    return _lib


def table(name: str) -> np.ndarray:
    return np.array([int(x, 16) for x in (DATA / name).read_text().split()], dtype=np.uint32)


def exp_lut() -> np.ndarray:
    return table("exp_lut.hex")


def recip_lut() -> np.ndarray:
    return table("recip_lut.hex")


def _p32(a):
    return a.ctypes.data_as(_U32)


def _p16(a):
    return a.ctypes.data_as(_U16)


def _binary(name, a, b, dtype=np.uint32):
    a = np.ascontiguousarray(a, dtype=dtype)
    b = np.ascontiguousarray(b, dtype=dtype)
    out = np.empty(a.shape, np.uint32)
    ptr = _p32 if dtype == np.uint32 else _p16
    getattr(lib(), name)(ptr(a), ptr(b), _p32(out), a.size)
    return out


def fp32_add(a, b):
    return _binary("rtl_fp32_add_n", a, b)


def fp32_mul(a, b):
    return _binary("rtl_fp32_mul_n", a, b)


def bf16_mul(a, b):
    return _binary("rtl_bf16_mul_n", a, b, np.uint16)


def exp_lookup(x):
    x = np.ascontiguousarray(x, dtype=np.uint32)
    out = np.empty(x.shape, np.uint32)
    lib().rtl_exp_lookup_n(_p32(x), _p32(exp_lut()), _p32(out), x.size)
    return out


def recip_lookup(x):
    x = np.ascontiguousarray(x, dtype=np.uint32)
    out = np.empty(x.shape, np.uint32)
    lib().rtl_recip_lookup_n(_p32(x), _p32(recip_lut()), _p32(out), x.size)
    return out


def attention(q, k, v, *, causal=True, q_pos_base=0, kv_pos_base=0, scale=None, plant=0):
    """One KV260 transaction: q [H_q, L, D], k/v [H_kv, L, D] bf16 words -> (out words, m bits, l bits).
    ``plant`` (PLANT_* flags) applies deliberate mistakes; 0 is the restatement itself."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    hq, L, d = q.shape
    hkv = k.shape[0]
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    scale_bits = int(np.float32(scale).view(np.uint32))
    out = np.empty_like(q)
    m = np.empty((hq, L), np.uint32)
    l = np.empty((hq, L), np.uint32)
    args = (_p16(q), _p16(k), _p16(v), hq, hkv, d, L, int(q_pos_base), int(kv_pos_base), int(bool(causal)), scale_bits,
            _p32(exp_lut()), _p32(recip_lut()), _p16(out), _p32(m), _p32(l))
    if plant:
        lib().rtl_attention_planted(*args, int(plant))
    else:
        lib().rtl_attention(*args)
    return out, m, l
