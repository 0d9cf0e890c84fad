"""Drop-in host driver for the MI355X GQA attention engine.

This module keeps the public surface of the LARA KV260 driver ``sw/attn_driver.py``
(constants, bf16 helpers, ``TensorByteCounts``, ``RunProfile``, ``MockMMIO``,
``MockDMAChannel`` and ``AttentionAccelerator`` with every method and its error types),
so host code written against the board runs unchanged.  Behind it, the PYNQ overlay,
CSR block and AXI DMA are replaced by ``libgqa.so`` (``include/gqa.h``): K/V live in a
device-resident HBM cache, Q is staged once per transaction, and the attention runs as
hand-written HIP kernels for gfx950.  Beside the reference API it adds the decode-side
methods the board lacks: ``load_kv``, ``append_kv``, ``decode_step``, ``submit_query``,
``prefill_chunk``, ``read_output`` and ``read_kv``.

There is no CPU fallback: constructing an ``AttentionAccelerator`` without the built
library or without a gfx950 GPU raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import subprocess
import time
from dataclasses import asdict, dataclass
from datetime import datetime, timezone
from pathlib import Path
from typing import Any, Optional

import numpy as np

from . import _lib

HAS_PYNQ = False  # the board runtime is never used; kept for callers that test it

# CSR offsets, control and status bits (sw/attn_driver.py:33-57, attn_pkg.sv:248-277).
CSR_CTRL = 0x000
CSR_STATUS = 0x004
CSR_SEQ_LEN = 0x008
CSR_Q_POS_BASE = 0x00C
CSR_KV_POS_BASE = 0x010
CSR_CFG = 0x014
CSR_ERROR_CODE = 0x018
CSR_LOAD_REQ = 0x01C
CSR_STREAM_LEN = 0x028
CSR_STREAM_DEST = 0x02C
CSR_RESULT_LEN = 0x058
CSR_PERF_CYCLES = 0x100
CSR_PERF_MAC_CYCLES = 0x108
CSR_PERF_STALLS = 0x10C

CTRL_START = 1 << 0
CTRL_CLEAR_STATUS = 1 << 1
STATUS_START_READY = 1 << 0
STATUS_BUSY = 1 << 1
STATUS_DONE = 1 << 2
STATUS_ERROR = 1 << 3
STATUS_STREAM_ERROR = 1 << 4
STATUS_KV_LOAD_REQ = 1 << 5
STATUS_Q_LOAD_REQ = 1 << 6

DEST_K_CACHE = 0
DEST_V_CACHE = 1
DEST_Q_BUF = 2

# Default model contract (sw/attn_driver.py:63-78): Llama-3-8B GQA, seq_len <= 512.
HEAD_DIM = 128
TILE_Q = 32
N_Q_HEADS = 32
N_KV_HEADS = 8
GQA_GROUP_SIZE = N_Q_HEADS // N_KV_HEADS
MAX_SEQ_LEN = 512
ABSOLUTE_POSITION_LIMIT = 1 << 16
BF16_BYTES = 2
RMS_NORM_EPS = 1e-5  # RMSNorm epsilon of the Llama-3 layer (run_layer); the reference does not state one
PL_CLOCK_MHZ = 71.427856  # the board's signed-off PL clock; GPU timings use the device clock
DMA_LENGTH_WIDTH = 26
DMA_MAX_TRANSFER_BYTES = (1 << DMA_LENGTH_WIDTH) - 1
MAX_KV_HEAD_BYTES = MAX_SEQ_LEN * HEAD_DIM * BF16_BYTES
Q_TILE_BYTES = TILE_Q * HEAD_DIM * BF16_BYTES
MAX_OUTPUT_BYTES = N_Q_HEADS * MAX_SEQ_LEN * HEAD_DIM * BF16_BYTES

ERR_NONE = 0x00
ERR_BAD_CFG = 0x01
ERR_BUSY_START = 0x02
ERR_STREAM_LEN = 0x10
ERR_STREAM_DEST = 0x11
ERR_RESULT_LEN = 0x12

_CLOSED_MSG = "attention accelerator buffers have been released"


def fp32_to_bf16_u16(values: np.ndarray) -> np.ndarray:
    """Pack float values into bf16 upper-half words (sw/attn_driver.py:88-98).

    uint16 input is taken as bf16 words and passed through.  Packing matches the
    reference word for word: the round increment is added at bit 0 of the fp32 pattern
    before the low half is cleared, so the result is the truncated upper half except
    when the low 16 bits are 0xFFFF (then it carries into the upper half).
    """
    arr = np.asarray(values)
    if arr.dtype == np.uint16:
        return np.ascontiguousarray(arr)
    bits = np.ascontiguousarray(arr, dtype=np.float32).view(np.uint32)
    # The increment only changes the upper half when the low half is all ones.
    carry = (bits & np.uint32(0xFFFF)) == np.uint32(0xFFFF)
    upper = (bits >> np.uint32(16)) + carry.astype(np.uint32)
    return np.ascontiguousarray(upper.astype(np.uint16))


def bf16_u16_to_fp32(values: np.ndarray) -> np.ndarray:
    """bf16 words -> float32 (sw/attn_driver.py:101-103)."""
    words = np.asarray(values, dtype=np.uint16)
    return (words.astype(np.uint32) << np.uint32(16)).view(np.float32)


class MockMMIO:
    """Register model of the KV260 CSR block and its load-request sequence.

    Kept from the board driver (sw/attn_driver.py:106-182) for host code that exercises
    the board's request-service protocol without hardware.  For a transaction of
    ``seq_len`` rows it issues, per KV group, one K/V request followed by one Q request
    per (head, 32-row tile); LOAD_REQ packs them as in attn_axi_lite_slave.sv:235-244.
    The GPU engine does not use it.
    """

    def __init__(self) -> None:
        self.regs: dict[int, int] = {CSR_STATUS: STATUS_START_READY}
        self.trace: list[tuple[str, int, int]] = []
        self.requests: list[dict[str, int]] = []
        self.current: Optional[dict[str, int]] = None
        self.kv_stage = 0
        self.started = False

    def prepare(self, seq_len: int) -> None:
        n_tiles = -(-int(seq_len) // TILE_Q)
        self.requests = []
        for group in range(N_KV_HEADS):
            self.requests.append({"kind": 0, "group": group})
            self.requests.extend(
                {"kind": 1, "group": group, "head": head, "tile": tile, "bank": tile & 1}
                for head in range(GQA_GROUP_SIZE)
                for tile in range(n_tiles)
            )
        self.current = None
        self.kv_stage = 0
        self.started = False

    def _head(self) -> Optional[dict[str, int]]:
        if self.current is None and self.requests:
            self.current = self.requests[0]
        return self.current

    def _request_word(self) -> int:
        req = self._head()
        if req is None:
            return 0
        if req["kind"] == 0:
            return 0x1 | (req["group"] & 0x7) << 4
        return (0x2 | (req["bank"] & 0x1) << 2 | (req["group"] & 0x7) << 8 | (req["head"] & 0x3) << 12
                | (req["tile"] & 0xFF) << 16)

    def write(self, offset: int, value: int) -> None:
        value = int(value) & 0xFFFFFFFF
        self.trace.append(("write", offset, value))
        if offset != CSR_CTRL:
            self.regs[offset] = value
            return
        if value & CTRL_CLEAR_STATUS:
            self.regs[CSR_STATUS] = STATUS_START_READY
            self.regs[CSR_ERROR_CODE] = ERR_NONE
        if value & CTRL_START:
            self.started = True
            self.regs[CSR_STATUS] = STATUS_BUSY

    def read(self, offset: int) -> int:
        if offset == CSR_LOAD_REQ:
            value = self._request_word()
        elif offset == CSR_STATUS:
            if not self.started:
                value = STATUS_START_READY
            else:
                req = self._head()
                if req is None:
                    value = STATUS_DONE | STATUS_START_READY
                else:
                    value = STATUS_BUSY | (STATUS_KV_LOAD_REQ if req["kind"] == 0 else STATUS_Q_LOAD_REQ)
        else:
            value = self.regs.get(offset, 0)
        self.trace.append(("read", offset, value))
        return value

    def transfer_complete(self, dest: int) -> None:
        req = self.current
        if req is None:
            return
        if req["kind"] == 0:
            if self.kv_stage == 0 and dest == DEST_K_CACHE:
                self.kv_stage = 1
            elif self.kv_stage == 1 and dest == DEST_V_CACHE:
                self.requests.pop(0)
                self.current = None
                self.kv_stage = 0
        elif dest == DEST_Q_BUF:
            self.requests.pop(0)
            self.current = None


class MockDMAChannel:
    """Recording stand-in for a PYNQ DMA channel (sw/attn_driver.py:185-196)."""

    def __init__(self, name: str) -> None:
        self.name = name
        self.trace: list[tuple[str, str, int]] = []
        self.last_buffer: Optional[np.ndarray] = None

    def transfer(self, buf: np.ndarray) -> None:
        self.last_buffer = buf
        self.trace.append(("transfer", self.name, int(buf.nbytes)))

    def wait(self) -> None:
        self.trace.append(("wait", self.name, 0))


@dataclass(frozen=True)
class TensorByteCounts:
    q_bytes: int
    k_bytes: int
    v_bytes: int
    o_bytes: int


@dataclass
class RunProfile:
    """Per-transaction timing record; field names follow sw/attn_driver.py:207-247.

    On the GPU the ``pl_*`` cycle fields count device-clock ticks at ``clock_mhz``:
    total = copy-in to copy-out, mac = attention kernels, stall = output copy.
    """

    timestamp_utc: str
    git_commit: str
    bitstream_sha256: str | None
    clock_mhz: float
    seq_len: int
    causal: bool
    q_pos_base: int
    kv_pos_base: int
    host_rms_norm_ms: float = 0.0
    host_qkv_projection_ms: float = 0.0
    host_rope_ms: float = 0.0
    input_pack_ms: float = 0.0
    driver_setup_ms: float = 0.0
    request_service_ms: float = 0.0
    output_dma_setup_ms: float = 0.0
    output_dma_transfer_ms: float = 0.0
    attention_total_ms: float = 0.0
    layer_total_ms: float = 0.0
    kv_dma_setup_ms: float = 0.0
    kv_dma_transfer_ms: float = 0.0
    kv_dma_transfers: int = 0
    kv_dma_bytes: int = 0
    q_dma_setup_ms: float = 0.0
    q_dma_transfer_ms: float = 0.0
    q_dma_transfers: int = 0
    q_dma_bytes: int = 0
    output_dma_transfers: int = 0
    output_dma_bytes: int = 0
    pl_total_cycles: int = 0
    pl_mac_cycles: int = 0
    pl_stall_cycles: int = 0
    pl_core_active_cycles_excluding_stalls: int = 0
    pl_total_ms: float = 0.0
    pl_mac_ms: float = 0.0
    pl_stall_ms: float = 0.0
    pl_core_active_ms_excluding_stalls: float = 0.0
    backend: str = "hip-gfx950"

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)


class AttentionAccelerator:
    """GQA attention engine on one MI355X, with the KV260 driver's API.

    ``bitstream_path`` and ``overlay`` are accepted for compatibility; a bitstream path is
    only hashed into the run profile.  The keyword-only arguments size the engine; the
    defaults reproduce the board contract (32 Q / 8 KV heads, D = 128, L <= 512, one
    sequence).
    """

    def __init__(
        self,
        bitstream_path: str | None = None,
        overlay: Any | None = None,
        *,
        batch: int = 1,
        n_q_heads: int = N_Q_HEADS,
        n_kv_heads: int = N_KV_HEADS,
        head_dim: int = HEAD_DIM,
        max_seq_len: int = MAX_SEQ_LEN,
        max_q_len: int | None = None,
        scale: float | None = None,
        device: int = 0,
        position_limit: int = ABSOLUTE_POSITION_LIMIT,
        numerics: str = "exact",
        page_size: int | None = None,
        n_pages: int | None = None,
        n_layers: int | None = None,
    ) -> None:
        self._closed = True
        self._ctx = ctypes.c_void_p()
        self.bitstream_path = str(Path(bitstream_path).resolve()) if bitstream_path else None
        self.overlay = overlay
        self._git_hash = self._git_commit()
        self._bitstream_hash = self._bitstream_sha256()
        self.batch = int(batch)
        self.n_q_heads = int(n_q_heads)
        self.n_kv_heads = int(n_kv_heads)
        self.head_dim = int(head_dim)
        self.max_seq_len = int(max_seq_len)
        self.max_q_len = int(max_q_len if max_q_len is not None else max_seq_len)
        self.position_limit = int(position_limit)
        if self.n_kv_heads < 1 or self.n_q_heads % self.n_kv_heads:
            raise ValueError("n_q_heads must be a positive multiple of n_kv_heads")
        self.group_size = self.n_q_heads // self.n_kv_heads
        cfg = _lib.GqaConfig(self.batch, self.n_q_heads, self.n_kv_heads, self.head_dim, self.max_seq_len,
                             self.max_q_len, float(scale or 0.0), int(device))
        lib = _lib.lib()
        self.paged = page_size is not None
        if n_layers is not None and not self.paged:
            raise ValueError("a multi-layer cache is paged: give page_size with n_layers")
        self.n_layers = int(n_layers) if n_layers is not None else 1
        if self.paged:
            if n_pages is None:
                n_pages = self.batch * -(-self.max_seq_len // int(page_size))
            if n_layers is not None:
                rc = lib.gqa_create_paged_layers(ctypes.byref(cfg), int(page_size), int(n_pages), self.n_layers,
                                                 ctypes.byref(self._ctx))
            else:
                rc = lib.gqa_create_paged(ctypes.byref(cfg), int(page_size), int(n_pages), ctypes.byref(self._ctx))
        else:
            rc = lib.gqa_create(ctypes.byref(cfg), ctypes.byref(self._ctx))
        if rc != _lib.GQA_OK:
            raise RuntimeError(f"unable to create the GPU attention engine: {_lib.status_string(rc)} (0x{rc:02x})")
        got = _lib.GqaConfig()
        _lib.check(lib.gqa_get_config(self._ctx, ctypes.byref(got)), "gqa_get_config")
        self.scale = float(got.scale)
        self._lib = lib
        self.numerics = "exact"
        self._pl_clock_mhz = 0.0
        self._hw_ready = True
        self._closed = False
        self._regs: dict[int, int] = {CSR_STATUS: STATUS_START_READY}
        self._error_code = ERR_NONE
        self._pending: dict[str, int] | None = None
        self._txn_len = 0
        self.last_profile: RunProfile | None = None
        if numerics != "exact":
            try:
                self.set_numerics(numerics)
            except Exception:
                self.close()
                raise

    # ---- lifetime ---------------------------------------------------------------------
    @property
    def hw_ready(self) -> bool:
        return self._hw_ready and not self._closed

    @staticmethod
    def _git_commit() -> str:
        try:
            return subprocess.check_output(
                ["git", "rev-parse", "--short", "HEAD"],
                cwd=Path(__file__).resolve().parents[1],
                stderr=subprocess.DEVNULL,
                text=True,
            ).strip()
        except (OSError, subprocess.SubprocessError):
            return "unknown"

    def _bitstream_sha256(self) -> str | None:
        if self.bitstream_path is None:
            return None
        path = Path(self.bitstream_path)
        if not path.is_file():
            return None
        digest = hashlib.sha256()
        with path.open("rb") as stream:
            for chunk in iter(lambda: stream.read(1 << 20), b""):
                digest.update(chunk)
        return digest.hexdigest()

    def close(self) -> None:
        if self._closed:
            return
        self._lib.gqa_destroy(self._ctx)
        self._ctx = ctypes.c_void_p()
        self._closed = True

    def __del__(self) -> None:  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self) -> "AttentionAccelerator":
        self._ensure_open()
        return self

    def __exit__(self, exc_type: Any, exc: Any, traceback: Any) -> None:
        self.close()

    def _ensure_open(self) -> None:
        if self._closed:
            raise RuntimeError(_CLOSED_MSG)

    def _call(self, name: str, *args: Any) -> None:
        self._ensure_open()
        _lib.check(getattr(self._lib, name)(self._ctx, *args), name)

    def save_last_profile(self, path: str | Path) -> None:
        if self.last_profile is None:
            raise RuntimeError("no completed attention run is available")
        Path(path).write_text(json.dumps(self.last_profile.to_dict(), indent=2) + "\n", encoding="utf-8")

    def set_numerics(self, numerics: str) -> None:
        """Arithmetic of prefill / transactions: "exact" (fp32, exact exp and divide) or "kv260"
        (the deployed KV260 datapath bit for bit: LUT exp, bf16-truncated P, reciprocal-table
        normalisation, the board's sub-block order).  Decode steps require "exact"."""
        modes = {"exact": _lib.GQA_NUMERICS_EXACT, "kv260": _lib.GQA_NUMERICS_KV260}
        if numerics not in modes:
            raise ValueError(f"numerics must be one of {sorted(modes)}, got {numerics!r}")
        self._call("gqa_set_option", _lib.GQA_OPT_NUMERICS, modes[numerics])
        self.numerics = numerics

    # ---- size contract ------------------------------------------------------------------
    @staticmethod
    def _validate_seq_len(seq_len: int) -> None:
        if not 1 <= int(seq_len) <= MAX_SEQ_LEN:
            raise ValueError(f"seq_len must be in 1..{MAX_SEQ_LEN}, got {seq_len}")

    @classmethod
    def byte_counts(cls, seq_len: int) -> TensorByteCounts:
        """Q/K/V/O bytes of one board-contract transaction (sw/attn_driver.py:351-359)."""
        cls._validate_seq_len(seq_len)
        return TensorByteCounts(
            N_Q_HEADS * seq_len * HEAD_DIM * BF16_BYTES,
            N_KV_HEADS * seq_len * HEAD_DIM * BF16_BYTES,
            N_KV_HEADS * seq_len * HEAD_DIM * BF16_BYTES,
            N_Q_HEADS * seq_len * HEAD_DIM * BF16_BYTES,
        )

    def _check_len(self, seq_len: int) -> int:
        limit = min(self.max_seq_len, self.max_q_len)
        if not 1 <= int(seq_len) <= limit:
            raise ValueError(f"seq_len must be in 1..{limit}, got {seq_len}")
        return int(seq_len)

    def _check_positions(self, q_pos_base: int, kv_pos_base: int, q_len: int, kv_len: int) -> None:
        if (q_pos_base < 0 or kv_pos_base < 0 or q_pos_base + q_len > self.position_limit
                or kv_pos_base + kv_len > self.position_limit):
            raise ValueError("absolute position base + seq_len exceeds 16-bit range")

    # ---- CSR-level protocol ---------------------------------------------------------------
    def clear_status(self) -> None:
        self._ensure_open()
        self._error_code = ERR_NONE
        self._regs[CSR_ERROR_CODE] = ERR_NONE

    def configure(self, seq_len: int, *, q_pos_base: int = 0, kv_pos_base: int = 0, causal: bool = True) -> None:
        self._ensure_open()
        seq_len = self._check_len(seq_len)
        self._check_positions(q_pos_base, kv_pos_base, seq_len, seq_len)
        self._regs[CSR_SEQ_LEN] = seq_len
        self._regs[CSR_Q_POS_BASE] = int(q_pos_base)
        self._regs[CSR_KV_POS_BASE] = int(kv_pos_base)
        self._regs[CSR_CFG] = int(bool(causal))
        self._pending = {"q_len": seq_len, "kv_len": seq_len, "q_pos_base": int(q_pos_base),
                         "kv_pos_base": int(kv_pos_base), "causal": int(bool(causal))}

    def start(self) -> None:
        if not (self.status() & STATUS_START_READY):
            raise RuntimeError("accelerator is not ready to accept start")
        rc = self._lib.gqa_start(self._ctx)
        if rc == _lib.GQA_ERR_NO_TRANSACTION:
            raise RuntimeError("no transaction has been submitted (load K/V and submit the query first)")
        if rc == _lib.GQA_ERR_BUSY_START:
            self._error_code = ERR_BUSY_START
            raise RuntimeError("accelerator is not ready to accept start")
        _lib.check(rc, "gqa_start")

    def status(self) -> int:
        self._ensure_open()
        word = ctypes.c_uint32(0)
        rc = self._lib.gqa_status(self._ctx, ctypes.byref(word))
        value = int(word.value)
        if rc != _lib.GQA_OK:
            value |= STATUS_ERROR
            self._error_code = rc
        if self._error_code != ERR_NONE:
            value |= STATUS_ERROR
        return value

    def wait_done(self, q_heads: np.ndarray, k_heads: np.ndarray, v_heads: np.ndarray, seq_len: int,
                  timeout_ms: int | None = None) -> None:
        """Block until the running transaction completes (sw/attn_driver.py:442-456).

        Q/K/V were already placed in device memory before ``start()``; the arguments are
        kept for signature compatibility.  Raises ``RuntimeError`` on an error status and
        ``TimeoutError`` when ``timeout_ms`` expires.
        """
        self._ensure_open()
        status = self.status()
        if status & (STATUS_ERROR | STATUS_STREAM_ERROR):
            raise RuntimeError(f"accelerator error status=0x{status:08x}, code=0x{self._error_code:02x}")
        rc = self._lib.gqa_wait(self._ctx, -1 if timeout_ms is None else int(timeout_ms))
        if rc == _lib.GQA_ERR_TIMEOUT:
            raise TimeoutError("attention accelerator timed out while servicing load requests")
        if rc != _lib.GQA_OK:
            self._error_code = rc
            raise RuntimeError(f"accelerator error status=0x{self.status():08x}, code=0x{rc:02x}")

    def readback_o(self, seq_len: int, out_buf: np.ndarray | None = None) -> np.ndarray:
        """Copy of the transaction output as head-major bf16 words [H_q, seq_len, D]."""
        self._ensure_open()
        out = np.empty((self.n_q_heads, int(seq_len), self.head_dim), dtype=np.uint16)
        rc = self._lib.gqa_read_output(self._ctx, _lib.as_u16_ptr(out), ctypes.c_int64(out.size))
        if rc == _lib.GQA_ERR_RESULT_LEN:
            self._error_code = ERR_RESULT_LEN
        _lib.check(rc, "gqa_read_output")
        if out_buf is not None:
            flat = np.asarray(out_buf).reshape(-1).view(np.uint8)
            flat[: out.nbytes] = out.reshape(-1).view(np.uint8)
        return out

    def read_perf(self) -> dict[str, int]:
        self._ensure_open()
        total, kern, copy = ctypes.c_uint64(0), ctypes.c_uint64(0), ctypes.c_uint64(0)
        mhz = ctypes.c_double(0.0)
        _lib.check(self._lib.gqa_read_perf(self._ctx, ctypes.byref(total), ctypes.byref(kern), ctypes.byref(copy),
                                           ctypes.byref(mhz)), "gqa_read_perf")
        self._pl_clock_mhz = float(mhz.value)
        return {"cycles": int(total.value), "mac_cycles": int(kern.value), "stall_cycles": int(copy.value)}

    # ---- paged cache ------------------------------------------------------------------------
    def reserve(self, b: int, n_rows: int) -> None:
        """Map pages so rows 0..n_rows-1 of sequence ``b`` are backed (paged engines only).
        Raises ``MemoryError`` when the pool has too few free pages (nothing changes)."""
        self._ensure_open()
        rc = self._lib.gqa_paged_reserve(self._ctx, int(b), int(n_rows))
        if rc == _lib.GQA_ERR_OOM:
            raise MemoryError(f"page pool exhausted reserving {n_rows} rows for sequence {b}")
        _lib.check(rc, "gqa_paged_reserve")

    def release(self, b: int) -> None:
        """Return every page of sequence ``b`` to the pool."""
        self._call("gqa_paged_release", int(b))

    def evict_lru(self, n_free_pages: int, pinned=()) -> list[int]:
        """Release whole sequences, least recently used first and never those in ``pinned``,
        until ``n_free_pages`` pages are free; returns the evicted sequence indices.  Raises
        ``MemoryError`` (releasing nothing) when that is impossible."""
        self._ensure_open()
        pin = np.ascontiguousarray(np.asarray(list(pinned), dtype=np.int32))
        out = np.empty(self.batch, dtype=np.int32)
        n = ctypes.c_int32(0)
        rc = self._lib.gqa_paged_evict_lru(self._ctx, int(n_free_pages), _lib.as_i32_ptr(pin) if pin.size else None,
                                           int(pin.size), _lib.as_i32_ptr(out), int(out.size), ctypes.byref(n))
        if rc == _lib.GQA_ERR_OOM:
            raise MemoryError(f"cannot free {n_free_pages} pages without evicting a pinned sequence")
        _lib.check(rc, "gqa_paged_evict_lru")
        return [int(x) for x in out[: n.value]]

    def select_layer(self, layer: int) -> None:
        """Make ``layer`` the cache layer that every later call reads and writes (multi-layer
        paged engines; the block tables and the page pool are shared by all layers)."""
        if not 0 <= int(layer) < self.n_layers:
            raise ValueError(f"layer {layer} outside 0..{self.n_layers - 1}")
        self._call("gqa_set_option", _lib.GQA_OPT_LAYER, int(layer))

    @property
    def layer(self) -> int:
        """The active cache layer (0 on a single-layer engine)."""
        if not self.paged:
            return 0
        n, cur = ctypes.c_int32(0), ctypes.c_int32(0)
        self._call("gqa_paged_layers", ctypes.byref(n), ctypes.byref(cur))
        return int(cur.value)

    def last_prefill_plan(self) -> tuple[str, int]:
        """Decomposition ("rows", "shared", "paired"; "" before any prefill and after a kv260-numerics
        launch) and KV segment count of the engine's last prefill launch."""
        kernel, segs = ctypes.c_int32(0), ctypes.c_int32(0)
        self._call("gqa_last_prefill_plan", ctypes.byref(kernel), ctypes.byref(segs))
        names = {_lib.GQA_PREFILL_KERNEL_ROWS: "rows", _lib.GQA_PREFILL_KERNEL_SHARED: "shared",
                 _lib.GQA_PREFILL_KERNEL_PAIRED: "paired"}
        return names.get(int(kernel.value), ""), int(segs.value)

    def page_info(self) -> dict[str, int]:
        """Page size, pool size, free pages and block-table width of a paged engine."""
        vals = [ctypes.c_int32(0) for _ in range(4)]
        self._call("gqa_paged_info", *(ctypes.byref(v) for v in vals))
        return dict(zip(("page_size", "n_pages", "free_pages", "max_pages"), (int(v.value) for v in vals)))

    def page_table(self, b: int) -> np.ndarray:
        """Block table of sequence ``b``: page index per page-sized run of rows (-1 unmapped)."""
        width = self.page_info()["max_pages"]
        out = np.empty(width, dtype=np.int32)
        self._call("gqa_paged_table", int(b), _lib.as_i32_ptr(out), int(width))
        return out

    def _reserve_transaction(self, L: int) -> None:
        # A board transaction reloads the whole cache of its one sequence.
        if self.paged:
            self.reserve(0, L)

    # ---- data movement ----------------------------------------------------------------------
    def load_kv(self, k_heads: np.ndarray, v_heads: np.ndarray, *, b: int = 0, start_pos: int = 0) -> None:
        """Write K/V rows [H_kv, n, D] of sequence ``b`` at rows start_pos.. (bit-exact)."""
        self._ensure_open()
        k = fp32_to_bf16_u16(k_heads)
        v = fp32_to_bf16_u16(v_heads)
        if k.ndim != 3 or k.shape != v.shape or k.shape[0] != self.n_kv_heads or k.shape[2] != self.head_dim:
            raise ValueError(f"expected K/V of shape ({self.n_kv_heads}, n, {self.head_dim}); got {k.shape}, {v.shape}")
        if not 0 <= b < self.batch:
            raise ValueError(f"sequence index {b} outside 0..{self.batch - 1}")
        n = k.shape[1]
        if start_pos < 0 or start_pos + n > self.max_seq_len:
            raise ValueError(f"rows {start_pos}..{start_pos + n - 1} exceed the cache capacity {self.max_seq_len}")
        self._call("gqa_load_kv", int(b), int(start_pos), int(n), _lib.as_u16_ptr(k), _lib.as_u16_ptr(v))

    def _check_rows(self, k_rows, v_rows, positions):
        k = fp32_to_bf16_u16(k_rows)
        v = fp32_to_bf16_u16(v_rows)
        shape = (self.batch, self.n_kv_heads, self.head_dim)
        if k.shape != shape or v.shape != shape:
            raise ValueError(f"expected K/V rows of shape {shape}; got {k.shape}, {v.shape}")
        pos = np.ascontiguousarray(positions, dtype=np.int32).reshape(-1)
        if pos.shape != (self.batch,):
            raise ValueError(f"expected {self.batch} positions, got {pos.shape}")
        if np.any(pos < -1) or np.any(pos >= self.max_seq_len):
            raise ValueError(f"append position outside -1..{self.max_seq_len - 1}")
        return k, v, pos

    def append_kv(self, k_rows: np.ndarray, v_rows: np.ndarray, positions) -> None:
        """Append one K/V row per sequence: rows [B, H_kv, D] at ``positions[b]`` (-1 skips)."""
        self._ensure_open()
        k, v, pos = self._check_rows(k_rows, v_rows, positions)
        self._call("gqa_append_kv", _lib.as_u16_ptr(k), _lib.as_u16_ptr(v), _lib.as_i32_ptr(pos))

    def read_kv(self, b: int, start_pos: int, n: int) -> tuple[np.ndarray, np.ndarray]:
        """Copy rows start_pos..start_pos+n-1 of sequence ``b``: (K, V) as [H_kv, n, D] words."""
        self._ensure_open()
        k = np.empty((self.n_kv_heads, int(n), self.head_dim), dtype=np.uint16)
        v = np.empty_like(k)
        if not 0 <= b < self.batch:
            raise ValueError(f"sequence index {b} outside 0..{self.batch - 1}")
        if start_pos < 0 or n < 0 or start_pos + n > self.max_seq_len:
            raise ValueError("rows exceed the cache capacity")
        self._call("gqa_read_kv", int(b), int(start_pos), int(n), _lib.as_u16_ptr(k), _lib.as_u16_ptr(v))
        return k, v

    # ---- attention ----------------------------------------------------------------------------
    def decode_step(self, q: np.ndarray, ctx_lens, *, k_rows: np.ndarray | None = None,
                    v_rows: np.ndarray | None = None, positions=None, return_lse: bool = False):
        """One query row per sequence against rows 0..ctx_lens[b]-1 of the cache.

        q is [B, H_q, D] (bf16 words or floats); returns bf16 words [B, H_q, D], and with
        ``return_lse`` also the natural-log LSE [B, H_q] of the scaled scores.  With
        ``k_rows``/``v_rows`` [B, H_kv, D] and ``positions`` [B] the step first appends
        those rows (as ``append_kv``) in the same kernel launch, so the new token can be
        attended by the same call.
        """
        self._ensure_open()
        qw = fp32_to_bf16_u16(q)
        shape = (self.batch, self.n_q_heads, self.head_dim)
        if qw.shape != shape:
            raise ValueError(f"expected Q of shape {shape}; got {qw.shape}")
        lens = np.ascontiguousarray(ctx_lens, dtype=np.int32).reshape(-1)
        if lens.shape != (self.batch,):
            raise ValueError(f"expected {self.batch} context lengths, got {lens.shape}")
        if np.any(lens < 0) or np.any(lens > self.max_seq_len):
            raise ValueError(f"context length outside 0..{self.max_seq_len}")
        out = np.empty(shape, dtype=np.uint16)
        lse = np.empty(shape[:2], dtype=np.float32) if return_lse else None
        lse_ptr = _lib.as_f32_ptr(lse) if lse is not None else None
        if k_rows is None and v_rows is None and positions is None:
            self._call("gqa_decode", _lib.as_u16_ptr(qw), _lib.as_i32_ptr(lens), _lib.as_u16_ptr(out), lse_ptr)
        else:
            if k_rows is None or v_rows is None or positions is None:
                raise ValueError("k_rows, v_rows and positions must be given together")
            k, v, pos = self._check_rows(k_rows, v_rows, positions)
            self._call("gqa_decode_append", _lib.as_u16_ptr(qw), _lib.as_u16_ptr(k), _lib.as_u16_ptr(v),
                       _lib.as_i32_ptr(pos), _lib.as_i32_ptr(lens), _lib.as_u16_ptr(out), lse_ptr)
        return (out, lse) if return_lse else out

    def submit_query(self, q_heads: np.ndarray, *, b: int = 0, q_pos_base: int = 0, kv_len: int | None = None,
                     kv_pos_base: int = 0, causal: bool = True) -> None:
        """Stage Q [H_q, q_len, D] of sequence ``b`` for the next ``start()``."""
        self._ensure_open()
        qw = fp32_to_bf16_u16(q_heads)
        if qw.ndim != 3 or qw.shape[0] != self.n_q_heads or qw.shape[2] != self.head_dim:
            raise ValueError(f"expected Q of shape ({self.n_q_heads}, q_len, {self.head_dim}); got {qw.shape}")
        q_len = qw.shape[1]
        if not 1 <= q_len <= self.max_q_len:
            raise ValueError(f"q_len must be in 1..{self.max_q_len}, got {q_len}")
        kv_len = q_len if kv_len is None else int(kv_len)
        if not 0 <= kv_len <= self.max_seq_len:
            raise ValueError(f"kv_len must be in 0..{self.max_seq_len}, got {kv_len}")
        if not 0 <= b < self.batch:
            raise ValueError(f"sequence index {b} outside 0..{self.batch - 1}")
        self._check_positions(q_pos_base, kv_pos_base, q_len, kv_len)
        rc = self._lib.gqa_submit(self._ctx, int(b), _lib.as_u16_ptr(qw), int(q_len), int(q_pos_base), int(kv_len),
                                  int(kv_pos_base), int(bool(causal)))
        if rc == _lib.GQA_ERR_BUSY_START:
            raise RuntimeError("accelerator is not ready to accept start")
        _lib.check(rc, "gqa_submit")
        self._txn_len = q_len

    def read_output(self) -> np.ndarray:
        """Output of the last transaction, [H_q, q_len, D] bf16 words."""
        return self.readback_o(self._txn_len)

    def prefill_chunk(self, q_heads: np.ndarray, *, b: int = 0, q_pos_base: int = 0, kv_len: int | None = None,
                      kv_pos_base: int = 0, causal: bool = True, k_rows: np.ndarray | None = None,
                      v_rows: np.ndarray | None = None, return_lse: bool = False):
        """Attend a block of query rows [H_q, q_len, D] against cache rows 0..kv_len-1 (synchronous).

        With ``k_rows``/``v_rows`` [H_kv, n, D] the same launch first places those rows at cache
        rows kv_len-n .. kv_len-1 (the chunk's own keys of a chunked prefill), bit-exact.
        """
        self._ensure_open()
        qw = fp32_to_bf16_u16(q_heads)
        if qw.ndim != 3 or qw.shape[0] != self.n_q_heads or qw.shape[2] != self.head_dim:
            raise ValueError(f"expected Q of shape ({self.n_q_heads}, q_len, {self.head_dim}); got {qw.shape}")
        q_len = qw.shape[1]
        kv_len = q_pos_base + q_len if kv_len is None else int(kv_len)
        if not 1 <= q_len <= self.max_q_len or not 0 <= kv_len <= self.max_seq_len:
            raise ValueError("q_len or kv_len outside the configured capacity")
        if not 0 <= b < self.batch:
            raise ValueError(f"sequence index {b} outside 0..{self.batch - 1}")
        self._check_positions(q_pos_base, kv_pos_base, q_len, kv_len)
        out = np.empty_like(qw)
        lse = np.empty((self.n_q_heads, q_len), dtype=np.float32) if return_lse else None
        lse_ptr = _lib.as_f32_ptr(lse) if lse is not None else None
        if k_rows is None and v_rows is None:
            self._call("gqa_prefill", int(b), _lib.as_u16_ptr(qw), int(q_len), int(q_pos_base), int(kv_len),
                       int(kv_pos_base), int(bool(causal)), _lib.as_u16_ptr(out), lse_ptr)
        else:
            if k_rows is None or v_rows is None:
                raise ValueError("k_rows and v_rows must be given together")
            k = fp32_to_bf16_u16(k_rows)
            v = fp32_to_bf16_u16(v_rows)
            if k.ndim != 3 or k.shape != v.shape or k.shape[0] != self.n_kv_heads or k.shape[2] != self.head_dim:
                raise ValueError(f"expected K/V rows of shape ({self.n_kv_heads}, n, {self.head_dim}); got {k.shape}")
            n = k.shape[1]
            if not 1 <= n <= min(kv_len, self.max_q_len):
                raise ValueError(f"{n} new rows do not fit below kv_len {kv_len} (at most {self.max_q_len})")
            self._call("gqa_prefill_append", int(b), _lib.as_u16_ptr(qw), _lib.as_u16_ptr(k), _lib.as_u16_ptr(v),
                       int(n), int(q_len), int(q_pos_base), int(kv_len), int(kv_pos_base), int(bool(causal)),
                       _lib.as_u16_ptr(out), lse_ptr)
        return (out, lse) if return_lse else out

    def run_attention(
        self,
        q_heads: np.ndarray,
        k_heads: np.ndarray,
        v_heads: np.ndarray,
        *,
        seq_len: int | None = None,
        q_pos_base: int = 0,
        kv_pos_base: int = 0,
        causal: bool = True,
        timeout_ms: int | None = None,
    ) -> np.ndarray:
        """Run one full transaction; returns raw head-major bf16 words (sw/attn_driver.py:469-550)."""
        self._ensure_open()
        attention_start = time.perf_counter()
        L = int(seq_len if seq_len is not None else q_heads.shape[1])
        self._check_len(L)
        expected_q = (self.n_q_heads, L, self.head_dim)
        expected_kv = (self.n_kv_heads, L, self.head_dim)
        if q_heads.shape != expected_q or k_heads.shape != expected_kv or v_heads.shape != expected_kv:
            raise ValueError(f"expected Q={expected_q}, K/V={expected_kv}; got {q_heads.shape}, {k_heads.shape}, "
                             f"{v_heads.shape}")
        prof = RunProfile(
            timestamp_utc=datetime.now(timezone.utc).isoformat(),
            git_commit=self._git_hash,
            bitstream_sha256=self._bitstream_hash,
            clock_mhz=self._pl_clock_mhz,
            seq_len=L,
            causal=causal,
            q_pos_base=q_pos_base,
            kv_pos_base=kv_pos_base,
        )
        self.last_profile = prof

        t = time.perf_counter()
        q_u16 = fp32_to_bf16_u16(q_heads)
        k_u16 = fp32_to_bf16_u16(k_heads)
        v_u16 = fp32_to_bf16_u16(v_heads)
        prof.input_pack_ms = (time.perf_counter() - t) * 1000.0

        t = time.perf_counter()
        self.configure(L, q_pos_base=q_pos_base, kv_pos_base=kv_pos_base, causal=causal)
        self.clear_status()
        o_bytes = self.n_q_heads * L * self.head_dim * BF16_BYTES
        if o_bytes > DMA_MAX_TRANSFER_BYTES:
            raise ValueError(f"output DMA length {o_bytes} exceeds {DMA_LENGTH_WIDTH}-bit DMA limit")
        self._regs[CSR_RESULT_LEN] = o_bytes
        prof.driver_setup_ms = (time.perf_counter() - t) * 1000.0

        t = time.perf_counter()
        self._reserve_transaction(L)
        self.load_kv(k_u16, v_u16, b=0, start_pos=0)
        prof.kv_dma_transfer_ms = (time.perf_counter() - t) * 1000.0
        prof.kv_dma_transfers = 2
        prof.kv_dma_bytes = int(k_u16.nbytes + v_u16.nbytes)

        t = time.perf_counter()
        self.submit_query(q_u16, b=0, q_pos_base=q_pos_base, kv_len=L, kv_pos_base=kv_pos_base, causal=causal)
        prof.q_dma_transfer_ms = (time.perf_counter() - t) * 1000.0
        prof.q_dma_transfers = 1
        prof.q_dma_bytes = int(q_u16.nbytes)
        prof.output_dma_transfers = 1
        prof.output_dma_bytes = o_bytes

        self.start()
        t = time.perf_counter()
        self.wait_done(q_u16, k_u16, v_u16, L, timeout_ms=timeout_ms)
        prof.request_service_ms = (time.perf_counter() - t) * 1000.0

        t = time.perf_counter()
        result = self.readback_o(L)
        prof.output_dma_transfer_ms = (time.perf_counter() - t) * 1000.0
        perf = self.read_perf()
        prof.clock_mhz = self._pl_clock_mhz
        prof.pl_total_cycles = perf["cycles"]
        prof.pl_mac_cycles = perf["mac_cycles"]
        prof.pl_stall_cycles = perf["stall_cycles"]
        prof.pl_core_active_cycles_excluding_stalls = max(perf["cycles"] - perf["stall_cycles"], 0)
        per_ms = self._pl_clock_mhz * 1000.0 if self._pl_clock_mhz > 0 else 1.0
        prof.pl_total_ms = perf["cycles"] / per_ms
        prof.pl_mac_ms = perf["mac_cycles"] / per_ms
        prof.pl_stall_ms = perf["stall_cycles"] / per_ms
        prof.pl_core_active_ms_excluding_stalls = prof.pl_core_active_cycles_excluding_stalls / per_ms
        prof.attention_total_ms = (time.perf_counter() - attention_start) * 1000.0
        return result

    def run_layer(self, hidden_states: np.ndarray, wq: np.ndarray, wk: np.ndarray, wv: np.ndarray,
                  rms_weight: np.ndarray | None = None, *, q_pos_base: int = 0, kv_pos_base: int = 0,
                  causal: bool = True, timeout_ms: int | None = None, rms_eps: float = RMS_NORM_EPS,
                  rope: bool = True) -> np.ndarray:
        """RMSNorm + QKV projection + RoPE, then attention (sw/attn_driver.py:552-586).

        ``hidden_states`` is [L, hidden]; ``wq`` [H_q*D, hidden] and ``wk``/``wv`` [H_kv*D,
        hidden] (out x in: Q = x Wq^T, hw/rtl/ext/qkv_projection/qkv_projection.sv:7-8);
        ``rms_weight`` (gamma, [hidden]) or None for no normalisation.  All are packed to bf16
        words like the transaction inputs (uint16 passes through).  The reference runs these
        steps on the host through its ``host_attention`` module; here they run on the GPU
        (RMSNorm and RoPE kernels around a hipBLASLt bf16 GEMM with fp32 accumulation) and write
        Q and the cache directly.  ``rms_eps`` and ``rope`` extend the reference signature.
        Returns fp32 [L, H_q*D] (``bf16_u16_to_fp32(o).transpose(1, 0, 2).reshape(L, -1)``).
        The RunProfile fields host_rms_norm_ms / host_qkv_projection_ms / host_rope_ms hold
        the device time of the three stages.
        """
        self._ensure_open()
        layer_start = time.perf_counter()
        t = time.perf_counter()
        x = np.ascontiguousarray(fp32_to_bf16_u16(hidden_states))
        if x.ndim != 2:
            raise ValueError(f"hidden_states must be [L, hidden]; got shape {x.shape}")
        L, hidden = (int(n) for n in x.shape)
        self._check_len(L)
        self._check_positions(q_pos_base, kv_pos_base, L, L)
        nq, nkv = self.n_q_heads * self.head_dim, self.n_kv_heads * self.head_dim
        wq_u = np.ascontiguousarray(fp32_to_bf16_u16(wq))
        wk_u = np.ascontiguousarray(fp32_to_bf16_u16(wk))
        wv_u = np.ascontiguousarray(fp32_to_bf16_u16(wv))
        if wq_u.shape != (nq, hidden) or wk_u.shape != (nkv, hidden) or wv_u.shape != (nkv, hidden):
            raise ValueError(f"expected Wq ({nq}, {hidden}), Wk/Wv ({nkv}, {hidden}); got {wq_u.shape}, "
                             f"{wk_u.shape}, {wv_u.shape}")
        gamma = None
        if rms_weight is not None:
            gamma = np.ascontiguousarray(fp32_to_bf16_u16(rms_weight)).reshape(-1)
            if gamma.size != hidden:
                raise ValueError(f"rms_weight must have {hidden} elements; got {gamma.size}")
        if not (np.isfinite(rms_eps) and rms_eps >= 0):
            raise ValueError(f"rms_eps must be finite and >= 0; got {rms_eps}")
        pack_ms = (time.perf_counter() - t) * 1000.0

        prof = RunProfile(
            timestamp_utc=datetime.now(timezone.utc).isoformat(),
            git_commit=self._git_hash,
            bitstream_sha256=self._bitstream_hash,
            clock_mhz=self._pl_clock_mhz,
            seq_len=L,
            causal=causal,
            q_pos_base=q_pos_base,
            kv_pos_base=kv_pos_base,
        )
        self.last_profile = prof
        prof.input_pack_ms = pack_ms
        t = time.perf_counter()
        self.configure(L, q_pos_base=q_pos_base, kv_pos_base=kv_pos_base, causal=causal)
        self.clear_status()
        o_bytes = self.n_q_heads * L * self.head_dim * BF16_BYTES
        self._regs[CSR_RESULT_LEN] = o_bytes
        prof.driver_setup_ms = (time.perf_counter() - t) * 1000.0

        t = time.perf_counter()
        self._reserve_transaction(L)
        self._call("gqa_submit_layer", 0, _lib.as_u16_ptr(x), L, hidden, _lib.as_u16_ptr(wq_u),
                   _lib.as_u16_ptr(wk_u), _lib.as_u16_ptr(wv_u),
                   None if gamma is None else _lib.as_u16_ptr(gamma), float(rms_eps), int(q_pos_base),
                   int(kv_pos_base), int(bool(causal)), int(bool(rope)))
        prof.q_dma_transfer_ms = (time.perf_counter() - t) * 1000.0
        prof.q_dma_transfers = 1
        prof.q_dma_bytes = int(x.nbytes + wq_u.nbytes + wk_u.nbytes + wv_u.nbytes
                               + (0 if gamma is None else gamma.nbytes))
        prof.output_dma_transfers = 1
        prof.output_dma_bytes = o_bytes
        stage_us = (ctypes.c_float * 3)()
        self._call("gqa_layer_times", stage_us, 3)
        prof.host_rms_norm_ms, prof.host_qkv_projection_ms, prof.host_rope_ms = (v / 1000.0 for v in stage_us)

        attention_start = time.perf_counter()
        self.start()
        t = time.perf_counter()
        self.wait_done(None, None, None, L, timeout_ms=timeout_ms)
        prof.request_service_ms = (time.perf_counter() - t) * 1000.0
        t = time.perf_counter()
        words = self.readback_o(L)
        prof.output_dma_transfer_ms = (time.perf_counter() - t) * 1000.0
        perf = self.read_perf()
        prof.clock_mhz = self._pl_clock_mhz
        prof.pl_total_cycles = perf["cycles"]
        prof.pl_mac_cycles = perf["mac_cycles"]
        prof.pl_stall_cycles = perf["stall_cycles"]
        prof.pl_core_active_cycles_excluding_stalls = max(perf["cycles"] - perf["stall_cycles"], 0)
        per_ms = self._pl_clock_mhz * 1000.0 if self._pl_clock_mhz > 0 else 1.0
        prof.pl_total_ms = perf["cycles"] / per_ms
        prof.pl_mac_ms = perf["mac_cycles"] / per_ms
        prof.pl_stall_ms = perf["stall_cycles"] / per_ms
        prof.pl_core_active_ms_excluding_stalls = prof.pl_core_active_cycles_excluding_stalls / per_ms
        result = bf16_u16_to_fp32(words).transpose(1, 0, 2).reshape(L, nq)
        prof.attention_total_ms = (time.perf_counter() - attention_start) * 1000.0
        prof.layer_total_ms = (time.perf_counter() - layer_start) * 1000.0
        return result

    def layer_qkv_device(self, x_ptr: int, n_tokens: int, hidden: int, wq_ptr: int, wk_ptr: int, wv_ptr: int,
                         rms_weight_ptr: int | None, q_out_ptr: int, *, b: int = 0, q_pos_base: int = 0,
                         kv_pos_base: int = 0, kv_row0: int = 0, rms_eps: float = RMS_NORM_EPS, rope: bool = True,
                         stream: int | None = None) -> None:
        """Device-pointer layer input stage (``gqa_layer_qkv_device``): Q to ``q_out_ptr``
        ([H_q, n_tokens, D] bf16, 16-byte aligned), K/V into rows kv_row0.. of sequence ``b``;
        enqueued, not synchronised."""
        self._ensure_open()
        self._call("gqa_layer_qkv_device", int(b), ctypes.c_void_p(x_ptr), int(n_tokens), int(hidden),
                   ctypes.c_void_p(wq_ptr), ctypes.c_void_p(wk_ptr), ctypes.c_void_p(wv_ptr),
                   ctypes.c_void_p(rms_weight_ptr) if rms_weight_ptr else None, float(rms_eps), int(q_pos_base),
                   int(kv_pos_base), int(kv_row0), int(bool(rope)), ctypes.c_void_p(q_out_ptr),
                   ctypes.c_void_p(stream) if stream else None)

    def layer_stage_us(self) -> tuple[float, float, float]:
        """Device time (us) of the RMSNorm, projection and RoPE stages of the last ``run_layer``
        call (``layer_qkv_device`` calls made while profiling is on record in the kernel timers)."""
        self._ensure_open()
        out = (ctypes.c_float * 3)()
        self._call("gqa_layer_times", out, 3)
        return tuple(float(v) for v in out)


def _self_test() -> None:
    """Board-protocol self-test of the mock (sw/attn_driver.py:589-599), no GPU needed."""
    mmio = MockMMIO()
    send = MockDMAChannel("send")
    L = 16
    mmio.prepare(L)
    mmio.write(CSR_CTRL, CTRL_START)
    while True:
        st = mmio.read(CSR_STATUS)
        if st & STATUS_DONE:
            break
        req = mmio.read(CSR_LOAD_REQ)
        if req & 1:
            for dest in (DEST_K_CACHE, DEST_V_CACHE):
                send.transfer(np.zeros(L * HEAD_DIM, dtype=np.uint16))
                mmio.transfer_complete(dest)
        elif req & 2:
            send.transfer(np.zeros(TILE_Q * HEAD_DIM, dtype=np.uint16))
            mmio.transfer_complete(DEST_Q_BUF)
    n = len([x for x in send.trace if x[0] == "transfer"])
    assert n == N_KV_HEADS * 2 + N_KV_HEADS * GQA_GROUP_SIZE, n
    print("attn_driver request-service mock self-test PASSED")


if __name__ == "__main__":
    _self_test()
