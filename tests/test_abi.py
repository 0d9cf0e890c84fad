"""The C-ABI library loads on a CPU-only host, exports every declared symbol, and rejects
bad arguments with the documented status codes before touching a device."""
import ctypes
import re
from pathlib import Path

import pytest

from lara_amd import _lib
from lara_amd import attn_driver as drv

HEADER = Path(__file__).resolve().parents[1] / "include" / "gqa.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(gqa_[a-z0-9_]+)\s*\(", text, flags=re.M)))


def test_header_declares_expected_set():
    names = declared_functions()
    assert len(names) >= 25
    assert sorted(_lib.EXPORTED) == names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_status_strings():
    assert _lib.status_string(_lib.GQA_OK) == "ok"
    for code in (0x01, 0x02, 0x10, 0x11, 0x12, 0x21, 0x22, 0x23, 0x24, 0x25, 0x26, 0x27, 0x28):
        assert _lib.status_string(code) not in ("", "unknown status")
    assert _lib.status_string(0x7F) == "unknown status"


def _cfg(**kw):
    base = dict(batch=1, n_q_heads=32, n_kv_heads=8, head_dim=128, max_seq_len=512, max_q_len=512, scale=0.0,
                device=0)
    base.update(kw)
    return _lib.GqaConfig(**base)


def test_create_rejects_bad_config_before_device():
    lib = _lib.lib()
    ctx = ctypes.c_void_p()
    assert lib.gqa_create(ctypes.byref(_cfg(n_q_heads=30)), ctypes.byref(ctx)) == _lib.GQA_ERR_BAD_CFG
    assert lib.gqa_create(ctypes.byref(_cfg(max_seq_len=0)), ctypes.byref(ctx)) == _lib.GQA_ERR_BAD_CFG
    # row counts are rounded up inside int32: lengths above 2^30 are refused, not wrapped
    assert lib.gqa_create(ctypes.byref(_cfg(max_seq_len=2**31 - 1)), ctypes.byref(ctx)) == _lib.GQA_ERR_BAD_CFG
    assert lib.gqa_create(ctypes.byref(_cfg(max_q_len=2**30 + 1)), ctypes.byref(ctx)) == _lib.GQA_ERR_BAD_CFG
    assert lib.gqa_create(ctypes.byref(_cfg(scale=-1.0)), ctypes.byref(ctx)) == _lib.GQA_ERR_BAD_CFG
    assert lib.gqa_create(ctypes.byref(_cfg(head_dim=96)), ctypes.byref(ctx)) == _lib.GQA_ERR_UNSUPPORTED
    assert lib.gqa_create(ctypes.byref(_cfg(n_q_heads=96, n_kv_heads=3)), ctypes.byref(ctx)) == _lib.GQA_ERR_UNSUPPORTED
    assert lib.gqa_create(None, ctypes.byref(ctx)) == _lib.GQA_ERR_NULL
    for n_layers in (0, _lib.GQA_MAX_LAYERS + 1):
        assert lib.gqa_create_paged_layers(ctypes.byref(_cfg()), 64, 8, n_layers, ctypes.byref(ctx)) == \
            _lib.GQA_ERR_BAD_CFG
    assert lib.gqa_create_paged_layers(ctypes.byref(_cfg()), 48, 8, 2, ctypes.byref(ctx)) == _lib.GQA_ERR_BAD_CFG
    assert not ctx.value
    with pytest.raises(ValueError):  # a multi-layer cache is a paged one
        drv.AttentionAccelerator(n_layers=2)


def test_null_context_is_rejected():
    lib = _lib.lib()
    assert lib.gqa_destroy(None) == _lib.GQA_ERR_NULL
    assert lib.gqa_decode(None, None, None, None, None) == _lib.GQA_ERR_NULL
    assert lib.gqa_start(None) == _lib.GQA_ERR_NULL
    assert lib.gqa_device_count(None) == _lib.GQA_ERR_NULL


def test_no_device_fails_loudly():
    if _lib.device_count() > 0:
        pytest.skip("a GPU is visible; the no-device path is exercised on CPU-only hosts")
    lib = _lib.lib()
    ctx = ctypes.c_void_p()
    assert lib.gqa_create(ctypes.byref(_cfg()), ctypes.byref(ctx)) == _lib.GQA_ERR_NO_DEVICE
    with pytest.raises(RuntimeError, match="no usable gfx950 device"):
        drv.AttentionAccelerator()
