"""Writes tests/golden/rope_tables.json: golden RoPE periods and sin/cos tables.

The reference holds no golden vectors for this path (its tests compute
their expectations at run time), so the fixtures come from an independent
restatement of rope::periods / rope::tables (engine/rope.rs:8-43): the f32
angle arithmetic is done with numpy float32 operations in the reference's
operand order, and sin/cos/pow are the platform libm's sinf/cosf/powf
called through ctypes (Rust's f32::sin/cos/powf call the same functions).
Neither the oracle nor the library is used here.

Grids: 2x3 and 4x4 (the reference's unit tests), 37x37 (518x518 at patch
14), 21x37 (518x294), 37x21 (the transpose), 16x16 (VGGT-Omega 256px at
patch 16) and 1x1.

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes
import ctypes.util
import hashlib
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GRIDS = [(2, 3), (4, 4), (37, 37), (21, 37), (37, 21), (16, 16), (1, 1)]

_libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
for _fn in ("sinf", "cosf"):
    getattr(_libm, _fn).restype = ctypes.c_float
    getattr(_libm, _fn).argtypes = [ctypes.c_float]
_libm.powf.restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]

F = np.float32


def periods() -> np.ndarray:
    # 100.0f32.powf(2.0 * i as f32 / 32.0)
    return np.array([_libm.powf(F(100.0), (F(2.0) * F(i)) / F(32.0)) for i in range(16)], F)


def tables(per: np.ndarray, h_p: int, w_p: int):
    side = F(max(h_p, w_p))
    tau = F(6.28318530717958647692)  # std::f32::consts::TAU

    def coord(n):
        i = np.arange(n, dtype=F)
        return (F(2.0) * ((i + F(0.5)) / side) - F(1.0)).astype(F)

    def angle_table(n):  # (n, 16) angles, each an f32 product then an f32 quotient
        c = coord(n)
        return ((tau * c)[:, None] / per[None, :]).astype(F)

    ah, aw = angle_table(h_p), angle_table(w_p)
    sinf = np.vectorize(lambda a: _libm.sinf(float(a)), otypes=[F])
    cosf = np.vectorize(lambda a: _libm.cosf(float(a)), otypes=[F])
    sh, ch, sw, cw = sinf(ah), cosf(ah), sinf(aw), cosf(aw)
    sin = np.empty((h_p, w_p, 64), F)
    cos = np.empty((h_p, w_p, 64), F)
    for half in (0, 32):
        sin[:, :, half:half + 16] = sh[:, None, :]
        cos[:, :, half:half + 16] = ch[:, None, :]
        sin[:, :, half + 16:half + 32] = sw[None, :, :]
        cos[:, :, half + 16:half + 32] = cw[None, :, :]
    return sin.reshape(h_p * w_p, 64), cos.reshape(h_p * w_p, 64)


def sample_rows(n: int) -> list[int]:
    return sorted({0, n // 2, n - 1, min(5, n - 1)})


def bits(a: np.ndarray) -> list[str]:
    return [f"{v:08x}" for v in np.ascontiguousarray(a, F).view(np.uint32).ravel()]


def main() -> None:
    per = periods()
    out = {"generator": "tests/golden/make_golden.py (numpy f32 + libm sinf/cosf/powf)",
           "periods_bits": bits(per), "grids": {}}
    for h_p, w_p in GRIDS:
        sin, cos = tables(per, h_p, w_p)
        rows = sample_rows(h_p * w_p)
        out["grids"][f"{h_p}x{w_p}"] = {
            "h_p": h_p, "w_p": w_p,
            "sin_sha256": hashlib.sha256(sin.tobytes()).hexdigest(),
            "cos_sha256": hashlib.sha256(cos.tobytes()).hexdigest(),
            "rows": {str(r): {"sin": bits(sin[r]), "cos": bits(cos[r])} for r in rows},
        }
    path = os.path.join(HERE, "rope_tables.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(path)


if __name__ == "__main__":
    main()
