"""Shared helpers for the tests: bf16 in numpy, seeded inputs, and oracle calls on numpy arrays."""
from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
F32, BF16 = 0, 1


def golden(name: str) -> dict:
    return json.loads((GOLDEN / name).read_text())


# ---- bf16 as uint16 bits -------------------------------------------------------------------

def to_bf16(x) -> np.ndarray:
    """float32 -> bf16 bits, round-to-nearest-even, NaN kept NaN (dtype.h:64-72)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def from_bf16(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    return from_bf16(to_bf16(x))


def randn_bf16(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    return to_bf16(rng.standard_normal(shape).astype(np.float32) * np.float32(std))


def ramp(shape, k: float) -> np.ndarray:
    """sin(i * k) over the flat index, in float32 (the reference tests' input pattern)."""
    n = int(np.prod(shape))
    return np.sin(np.arange(n, dtype=np.float64) * k).astype(np.float32).reshape(shape)


def addr(a) -> int | None:
    return None if a is None else a.ctypes.data


def empty_like_bf16(shape) -> np.ndarray:
    return np.zeros(shape, dtype=np.uint16)


# ---- comparison ----------------------------------------------------------------------------

def stats(got, want) -> dict:
    """max-abs, relative L2 and cosine similarity of got vs want (float arrays)."""
    g = np.asarray(got, dtype=np.float64).ravel()
    w = np.asarray(want, dtype=np.float64).ravel()
    diff = g - w
    nw = np.linalg.norm(w)
    cos = float(np.dot(g, w) / (np.linalg.norm(g) * nw)) if nw > 0 and np.linalg.norm(g) > 0 else 1.0
    return {"max_abs": float(np.max(np.abs(diff))) if diff.size else 0.0,
            "rel_l2": float(np.linalg.norm(diff) / nw) if nw > 0 else float(np.linalg.norm(diff)),
            "cosine": cos,
            "mismatch_frac": float(np.mean(g != w)) if g.size else 0.0}


TOLERANCE = json.loads((ROOT / "configs" / "tolerance.json").read_text()) \
    if (ROOT / "configs" / "tolerance.json").exists() else {}


def assert_within(got, want, op: str, where: str = "") -> dict:
    """Checks got against want with the per-op bf16 tolerance of configs/tolerance.json."""
    tol = TOLERANCE["ops"][op]
    s = stats(got, want)
    msg = f"{op} {where}: {s} vs tolerance {tol}"
    assert s["max_abs"] <= tol["max_abs"], msg
    assert s["rel_l2"] <= tol["rel_l2"], msg
    assert s["cosine"] >= tol["cosine"], msg
    return s
