"""Axial 2D RoPE tables (crates/headshot-server/src/engine/rope.rs:5-43).

Computed on the host in f32 by libheadshot_hip's ``hs_rope_periods`` /
``hs_rope_tables`` (bit-exact to the reference: same f32 operation order,
platform libm sinf/cosf/powf), once per session, then uploaded.
"""
from __future__ import annotations

import numpy as np

from . import _lib


def periods() -> np.ndarray:
    """``periods[i] = 100^(2i/32)``, i = 0..15 (engine/rope.rs:8-10)."""
    out = np.empty(16, np.float32)
    _lib.load().hs_rope_periods(out.ctypes.data)
    return out


def tables(periods16: np.ndarray, h_p: int, w_p: int) -> tuple[np.ndarray, np.ndarray]:
    """Sin/cos tables, each ``(h_p*w_p, 64)`` f32, patch rows h-outer/w-inner
    (engine/rope.rs:18-43)."""
    p16 = np.ascontiguousarray(periods16, dtype=np.float32)
    assert p16.shape == (16,), "periods must hold 16 values"
    n = h_p * w_p
    sin = np.empty((n, 64), np.float32)
    cos = np.empty((n, 64), np.float32)
    _lib.check(_lib.load().hs_rope_tables(p16.ctypes.data, h_p, w_p, sin.ctypes.data,
                                          cos.ctypes.data), "rope_tables")
    return sin, cos
