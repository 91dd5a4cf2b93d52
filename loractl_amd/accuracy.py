"""Relative-accuracy gate — mirror of ``crates/loractl-core/src/accuracy.rs:43-131``.

``rel_deviation`` is the peak-normalized max deviation
``max|ours - ref| / max(peak|ref|, 1e-12)``, ``inf`` on a length mismatch,
empty input or any non-finite value. ``RelGate.apply`` accepts when the value
is finite, at most ``max(2*d_bar, floor)`` and at most ``ceil``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


def rel_deviation(ours, reference) -> float:
    a = np.asarray(ours, dtype=np.float64).reshape(-1)
    b = np.asarray(reference, dtype=np.float64).reshape(-1)
    if a.size == 0 or a.size != b.size:
        return math.inf
    if not (np.isfinite(a).all() and np.isfinite(b).all()):
        return math.inf
    peak = float(np.abs(b).max())
    return float(np.abs(a - b).max()) / max(peak, 1e-12)


def cosine(a, b) -> float:
    a = np.asarray(a, dtype=np.float64).reshape(-1)
    b = np.asarray(b, dtype=np.float64).reshape(-1)
    den = float(np.linalg.norm(a) * np.linalg.norm(b))
    return float(a @ b) / den if den > 0 else (1.0 if not a.any() and not b.any() else 0.0)


@dataclass(frozen=True)
class GateOutcome:
    d_ours: float
    band: float
    ceil: float
    finite: bool
    passed: bool

    def expect_pass(self, label: str):
        assert self.passed, (
            f"{label}: relative-accuracy gate FAILED — d_ours = {self.d_ours:e}, band = max(2·d_bar, floor) = "
            f"{self.band:e}, ceil = {self.ceil:e}, all-finite = {self.finite}"
        )


@dataclass(frozen=True)
class RelGate:
    d_bar: float
    floor: float
    ceil: float

    def apply(self, d_ours: float) -> GateOutcome:
        band = max(2.0 * self.d_bar, self.floor)
        finite = math.isfinite(d_ours)
        return GateOutcome(d_ours, band, self.ceil, finite, finite and d_ours <= band and d_ours <= self.ceil)
