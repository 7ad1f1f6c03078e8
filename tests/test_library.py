"""The C-ABI library on a host without a GPU: it loads, exports every entry point
include/burnisher_hip.h declares, reports its ABI, refuses bad arguments before touching a
device, and generates seeded inputs deterministically. Also: the product never reaches the
oracle."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import burnisher_amd as bh
from helpers import from_bf16

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> list[str]:
    text = (ROOT / "include" / "burnisher_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = bh.lib()
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert set(names) == set(bh.SIGNATURES), "Python signatures drift from the header"


def test_abi_and_build_info():
    lib = bh.lib()
    assert lib.bh_abi_version() == 1
    assert b"gfx950" in lib.bh_build_info()


def test_arguments_refused_before_any_device_work():
    lib = bh.lib()
    # null operands, negative shapes, bad enums: each refused with a sentence
    assert lib.bh_gemm(None, None, None, None, 4, 4, 4, 1, 0, 1, None) != 0
    assert b"null" in lib.bh_last_error()
    assert lib.bh_gemm(None, None, None, None, -1, 4, 4, 1, 0, 1, None) != 0
    assert b"negative" in lib.bh_last_error()
    assert lib.bh_norm(None, None, None, None, 4, 4, 1e-6, 1, 8, 4, 1, None) != 0
    assert b"GroupNorm has no RMS form" in lib.bh_last_error()
    assert lib.bh_conv2d(None, None, None, None, 1, 4, 8, 8, 4, 3, 0, 1, None) != 0
    assert b"same" in lib.bh_last_error()
    assert lib.bh_conv2d(None, None, None, None, 1, 4, 8, 8, 4, 3, 1, 0, None) != 0
    assert b"bf16 only" in lib.bh_last_error()
    assert lib.bh_chunk(None, None, None, 2, 4, 6, 9, -1, 1, None) != 0
    assert b"chunk" in lib.bh_last_error()
    # an odd timestep-embedding width is refused as the reference refuses it (weights.cpp:111)
    assert lib.bh_timestep_embedding(500.0, 7, 2, None, 1, None) != 0
    assert b"even dimension" in lib.bh_last_error()
    # an empty op is a no-op, not an error
    assert lib.bh_gemm(None, None, None, None, 0, 4, 4, 1, 0, 1, None) == 0
    assert lib.bh_last_error() == b""
    with pytest.raises(bh.BurnisherError):
        bh.call("bh_attention", None, None, None, None, 1, 1, 4, 0, 8, 0.0, None, None, 0, 1, None)
    # the launch profiler's sampling stride is at least one launch
    assert lib.bh_profile_sample(0) != 0
    assert b"at least 1" in lib.bh_last_error()
    assert lib.bh_profile_sample(1) == 0


def test_fill_normal_is_seeded_by_name_and_split_free():
    a = bh.fill_normal_bf16(100_001, "transformer_blocks.0.attn1.to_q.weight", 7, 0.02)
    b = bh.fill_normal_bf16(100_001, "transformer_blocks.0.attn1.to_q.weight", 7, 0.02)
    c = bh.fill_normal_bf16(100_001, "transformer_blocks.0.attn1.to_k.weight", 7, 0.02)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    # a prefix of a longer draw is the shorter draw: element i does not depend on n or threads
    big = bh.fill_normal_bf16(3_000_001, "x", 7, 1.0)
    small = bh.fill_normal_bf16(1001, "x", 7, 1.0)
    assert np.array_equal(big[:1000], small[:1000])
    f = from_bf16(big)
    assert abs(f.mean()) < 3e-3 and abs(f.std() - 1.0) < 3e-3
    g = from_bf16(a)
    assert abs(g.std() - 0.02) < 5e-4


def test_product_never_reaches_the_oracle():
    pkg = ROOT / "burnisher_amd"
    for p in list(pkg.rglob("*.py")) + list(pkg.rglob("*.cpp")) + list(pkg.rglob("*.hip")) + \
            list(pkg.rglob("*.h")):
        text = p.read_text()
        for pattern in (r"^\s*(import|from)\s+oracle\b", r"libstock|libref_stock",
                        r"\b(stock|ref)_[a-z_]+\s*\(", r"oracle/_(build|ref)"):
            assert not re.search(pattern, text, flags=re.M), f"{p} reaches the oracle ({pattern})"
