"""Writes the KV260 ROM tables used by the RTL-exact numerics mode (exp_lut.hex, recip_lut.hex).

Closed forms (one lowercase hex word per line, as the board's ROM images):
  exp_lut[i]   = float32 bits of numpy.exp(numpy.linspace(-8, 0, 1024, dtype=float32)), i = 0..1023
                 (the interpolation table of hw/rtl/core/softmax_engine.sv:570-621)
  recip_lut[j] = round((2 / (1 + (j + 0.5) / 256) - 1) * 2**23), j = 0..255, 23-bit mantissas
                 (the normalisation table of hw/rtl/mem/output_buffer.sv:192-224)
numpy's float32 exp is implementation-dependent in the last bit, so the tables are generated
once and committed with their SHA-256 (TABLE_SHA256) rather than regenerated at build time.
Run from the repository root:  python lara_amd/data/make_luts.py
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
TABLE_SHA256 = {
    "exp_lut.hex": "0e756509a7ccf0f8b342df8eb609151f9d906bea278931b66cfe93d30eaaaf54",
    "recip_lut.hex": "17f2d5be90bf09b4849b1e8d637a38f55e56fee6c49d392f8d1bab252714dcc4",
}


def exp_table() -> np.ndarray:
    return np.exp(np.linspace(-8.0, 0.0, 1024, dtype=np.float32)).astype(np.float32).view(np.uint32)


def recip_table() -> np.ndarray:
    j = np.arange(256, dtype=np.float64)
    return np.round((2.0 / (1.0 + (j + 0.5) / 256.0) - 1.0) * 2.0 ** 23).astype(np.uint32)


def render(words, width: int) -> str:
    return "".join(f"{int(w):0{width}x}\n" for w in words)


def read_table(name: str) -> np.ndarray:
    return np.array([int(x, 16) for x in (HERE / name).read_text().split()], dtype=np.uint32)


def main() -> None:
    for name, words, width in (("exp_lut.hex", exp_table(), 8), ("recip_lut.hex", recip_table(), 6)):
        text = render(words, width)
        digest = hashlib.sha256(text.encode()).hexdigest()
        (HERE / name).write_text(text)
        status = "matches" if digest == TABLE_SHA256[name] else "DIFFERS FROM"
        print(f"wrote {name}: sha256 {digest} ({status} the recorded board ROM image)")


if __name__ == "__main__":
    main()
