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


# ---- the sampler through the oracle's (or the reference's) C entry points -------------------

# The pinned schedule's timesteps at 20 steps (/root/reference/tests/test_scheduler.cpp:21-22).
TIMESTEPS_20 = [999, 949, 899, 849, 799, 749, 699, 649, 599, 549,
                500, 450, 400, 350, 300, 250, 200, 150, 100, 50]


class HostSampler:
    """DPM-Solver++ 2M on host buffers: `prefix` "stock" (oracle/stock.cpp) or "ref" (the
    reference's own DPMSolverMultistep through oracle/ref_shim.cpp)."""

    def __init__(self, lib, prefix: str, steps: int | None = 20, **overrides):
        import burnisher_amd as bh
        import oracle
        self.lib, self.prefix = lib, prefix
        self.h = ctypes.c_void_p()
        self.cfg = bh.SchedConfig.pinned(**overrides)
        oracle.call(lib, f"{prefix}_sched_create", ctypes.byref(self.cfg), ctypes.byref(self.h))
        if steps is not None:
            self.set_timesteps(steps)

    def _call(self, name, *args):
        import oracle
        oracle.call(self.lib, f"{self.prefix}_{name}", self.h, *args)

    def set_timesteps(self, steps: int):
        self._call("sched_set_timesteps", steps)

    def steps(self) -> int:
        return getattr(self.lib, f"{self.prefix}_sched_steps")(self.h)

    def timestep(self, i: int) -> int:
        v = ctypes.c_int64()
        self._call("sched_timestep", i, ctypes.byref(v))
        return v.value

    def sigma(self, i: int) -> float:
        v = ctypes.c_double()
        self._call("sched_sigma", i, ctypes.byref(v))
        return v.value

    def coefficients(self, i: int):
        import burnisher_amd as bh
        c = bh.SchedCoefficients()
        self._call("sched_coefficients", i, ctypes.byref(c))
        return c

    def step(self, eps: np.ndarray, i: int, sample: np.ndarray, dtype: int):
        """In place on `sample` (float32 for F32, uint16 bf16 bits for BF16)."""
        assert eps.dtype == sample.dtype and eps.size == sample.size
        self._call("sched_step", addr(eps), i, addr(sample), sample.size, dtype)

    def reset(self):
        self._call("sched_reset")

    def close(self):
        if self.h:
            getattr(self.lib, f"{self.prefix}_sched_destroy")(self.h)
            self.h = ctypes.c_void_p()


COEFF_FIELDS = ("order", "sigma_s0", "sigma_t", "sigma_vp_s0", "sigma_vp_t", "alpha_t",
                "alpha_s0", "exp_neg_h", "r0")


def coeff_tuple(c) -> tuple:
    return tuple(getattr(c, f) for f in COEFF_FIELDS)
