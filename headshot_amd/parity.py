"""Comparison metrics and pass/fail gates (crates/headshot-server/src/parity.rs).

``compare`` and ``Gate`` restate parity.rs:35-104 (NaN-proof: a NaN metric
always fails). ``assert_close`` is the reference tests' element predicate
``|a - e| <= tol + tol*|e|`` (tests/kernels.rs:35-43). ``f16_close`` is the
f16 gate for normalised outputs, ``|a - e| <= 2e-3 * max(1, |e|)``.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Metrics:
    max_abs_err: float
    mean_abs_err: float
    cosine_sim: float
    ref_scale: float

    def rel_max_err(self) -> float:
        return self.max_abs_err / max(self.ref_scale, np.finfo(np.float64).tiny)


def compare(ours, reference) -> Metrics:
    """parity.rs:35-60."""
    a = np.asarray(ours, np.float64).ravel()
    b = np.asarray(reference, np.float64).ravel()
    assert a.shape == b.shape, "length mismatch"
    assert a.size > 0
    d = np.abs(a - b)
    denom = max(np.sqrt((a * a).sum()) * np.sqrt((b * b).sum()), np.finfo(np.float64).tiny)
    return Metrics(float(d.max()), float(d.mean()), float((a * b).sum() / denom),
                   float(np.abs(b).max()))


@dataclass(frozen=True)
class Gate:
    """parity.rs:66-104."""
    rel_max: float | None
    min_cosine: float | None

    def check(self, name: str, m: Metrics) -> Metrics:
        if self.rel_max is not None:
            r = m.rel_max_err()
            if not (r <= self.rel_max):
                raise AssertionError(f"{name}: rel_max_err {r:.3e} !<= {self.rel_max:.3e} ({m})")
        if self.min_cosine is not None:
            if not (m.cosine_sim >= self.min_cosine):
                raise AssertionError(
                    f"{name}: cosine_sim {m.cosine_sim:.9f} !>= {self.min_cosine:.9f} ({m})")
        return m


Gate.F32_TIGHT = Gate(1e-4, 1.0 - 1e-6)   # parity.rs:74
Gate.F32_DEEP = Gate(0.5, 1.0 - 1e-4)     # parity.rs:81
Gate.F16_TRUNK = Gate(None, 0.999)        # parity.rs:83


def _worst(actual, expected, bound):
    err = np.abs(actual - expected)
    bad = ~(err <= bound)  # NaN fails
    if not bad.any():
        return None
    i = int(np.flatnonzero(bad.ravel())[0])
    return i, float(actual.ravel()[i]), float(expected.ravel()[i]), int(bad.sum())


def assert_close(actual, expected, tol: float, what: str) -> None:
    """tests/kernels.rs:35-43: ``|a - e| <= tol + tol*|e|`` element-wise."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    w = _worst(a, e, tol + tol * np.abs(e))
    if w is not None:
        i, av, ev, n = w
        raise AssertionError(f"{what}[{i}]: got {av}, want {ev} (tol {tol}); {n} elements off")


def f16_close(actual, expected, what: str, tol: float = 2e-3) -> None:
    """f16 gate: ``|a - e| <= tol * max(1, |e|)`` element-wise."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    w = _worst(a, e, tol * np.maximum(1.0, np.abs(e)))
    if w is not None:
        i, av, ev, n = w
        raise AssertionError(f"{what}[{i}]: got {av}, want {ev} (f16 tol {tol}); {n} elements off")


def assert_bit_exact(actual, expected, what: str) -> None:
    a = np.ascontiguousarray(actual)
    e = np.ascontiguousarray(expected)
    assert a.dtype == e.dtype and a.shape == e.shape, f"{what}: {a.dtype}{a.shape} vs {e.dtype}{e.shape}"
    ua = a.view(np.uint8).reshape(a.size, -1) if a.size else a.view(np.uint8)
    ue = e.view(np.uint8).reshape(e.size, -1) if e.size else e.view(np.uint8)
    if not np.array_equal(ua, ue):
        diff = np.flatnonzero((ua != ue).any(axis=-1))
        i = int(diff[0])
        raise AssertionError(f"{what}: {diff.size} elements differ; first [{i}] "
                             f"got {a.ravel()[i]!r}, want {e.ravel()[i]!r}")


def ulp_diff_f16(actual, expected) -> np.ndarray:
    """|ulp distance| between two float16 arrays (same sign assumed near 0)."""
    a = np.asarray(actual, np.float16).view(np.int16).astype(np.int32)
    e = np.asarray(expected, np.float16).view(np.int16).astype(np.int32)
    # map sign-magnitude to a monotonic integer line
    a = np.where(a < 0, -32768 - a, a)
    e = np.where(e < 0, -32768 - e, e)
    return np.abs(a - e)


# ---------------------------------------------------------------------------
# locally generated fixtures (parity.rs:106-176)

def fixtures_dir():
    """Where the locally generated fixtures live (converted weights in the
    directory itself, reference activation dumps under ``dumps/``):
    ``$HEADSHOT_FIXTURES_DIR``, else ``fixtures/`` at the repository root
    (parity.rs:106-112). Fixtures are derived from the gated checkpoint and
    are never committed."""
    import os
    from pathlib import Path

    env = os.environ.get("HEADSHOT_FIXTURES_DIR")
    return Path(env) if env else Path(__file__).resolve().parent.parent / "fixtures"


@dataclass(frozen=True)
class DumpMeta:
    """The ``headshot`` metadata a reference dump carries (parity.rs:114-125)."""
    scene: str
    variant: str
    device: str
    n_frames: int
    width: int
    height: int
    seed: int
    shapes: dict  # name -> shape list


class Dump:
    """A reference activation dump, one scene x one precision variant
    (``dump_{scene}_{variant}.safetensors``; parity.rs:127-176). Tensors are
    all f32."""

    def __init__(self, meta: DumpMeta, st):
        self.meta, self._st = meta, st

    @staticmethod
    def open(scene: str, variant: str) -> "Dump":
        return Dump.open_path(fixtures_dir() / "dumps" / f"dump_{scene}_{variant}.safetensors")

    @staticmethod
    def open_path(path) -> "Dump":
        import json

        from .weights import SafeTensorsFile, WeightsIoError

        try:
            st = SafeTensorsFile(path)
        except WeightsIoError as e:
            raise FileNotFoundError(f"{path}: {e} (generate with tools/dump_reference.py)") from None
        raw = (st.metadata or {}).get("headshot")
        if raw is None:
            raise ValueError(f"{path}: missing `headshot` metadata")
        m = json.loads(raw)
        meta = DumpMeta(str(m["scene"]), str(m["variant"]), str(m["device"]), int(m["n_frames"]),
                        int(m["width"]), int(m["height"]), int(m["seed"]),
                        {k: [int(d) for d in v] for k, v in m["shapes"].items()})
        return Dump(meta, st)

    def tensor(self, name: str):
        """(shape, f32 values) of one tensor; anything but f32 is an error."""
        if self._st.dtype(name) != "F32":
            raise ValueError(f"{name}: dump tensors must be f32, got {self._st.dtype(name)}")
        a = self._st.tensor(name)
        return list(a.shape), np.array(a, dtype=np.float32).ravel()

    def names(self) -> list:
        return self._st.names()
