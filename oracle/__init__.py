"""oracle -- TEST INFRASTRUCTURE ONLY: ctypes access to the CPU parity checkers.

  stock()  oracle/_build/libstock.so, the restatement of the reference's `stock` ops, DiT
           graph and DPM-Solver++ sampler (oracle/stock.cpp). Built by `make -C oracle`.
  ref()    oracle/_ref/libref_stock.so, the reference's OWN stock path compiled from
           /root/reference (oracle/ref_shim.cpp + `make -C oracle ref`), or None where it was
           not built (it needs /root/reference at build time).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker -- never as the thing measured or shipped.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
STOCK_PATH = HERE / "_build" / "libstock.so"
REF_PATH = HERE / "_ref" / "libref_stock.so"
REFERENCE_ROOT = Path("/root/reference")

_V, _I, _I64, _F, _D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_double

_STOCK_SIGS = {
    "stock_last_error": ([], ctypes.c_char_p),
    "stock_gemm": ([_V, _V, _V, _V, _I64, _I64, _I64, _I, _I, _I, _I], _I),
    "stock_attention": ([_V, _V, _V, _V, _I64, _I64, _I64, _I64, _I64, _F, _V, _V, _I, _I, _I, _I], _I),
    "stock_norm": ([_V, _V, _V, _V, _I64, _I64, _F, _I, _I, _I], _I),
    "stock_modulate": ([_V, _V, _V, _V, _I64, _I64, _I64, _V, _V, _I], _I),
    "stock_activation": ([_V, _V, _I64, _I, _V, _I], _I),
    "stock_add": ([_V, _V, _V, _I64, _I64, _F, _I, _I], _I),
    "stock_chunk": ([_V, _V, _V, _I64, _I64, _I64, _I64, _I64, _I], _I),
    "stock_patch": ([_V, _V, _I64, _I64, _I64, _I64, _I, _I], _I),
    "stock_position_embedding": ([ctypes.POINTER(_D), _I, _I, _I, _D], _I),
    "stock_timestep_embedding": ([_D, _I, ctypes.POINTER(_F)], _I),
    "stock_dit_forward": ([_V, _V, _I64, _I64, _I64, _V, _D, _V, _V, _I, _V, _I, _I], _I),
    "stock_scale": ([_V, _V, _I64, _F, _I], _I),
    "stock_repeat": ([_V, _V, _I64, _I64, _I], _I),
    "stock_guidance": ([_V, _V, _I64, _I64, _I64, _F, _I], _I),
    "stock_sched_create": ([_V, ctypes.POINTER(_V)], _I),
    "stock_sched_destroy": ([_V], None),
    "stock_sched_set_timesteps": ([_V, _I], _I),
    "stock_sched_steps": ([_V], _I),
    "stock_sched_timestep": ([_V, _I, ctypes.POINTER(_I64)], _I),
    "stock_sched_sigma": ([_V, _I, ctypes.POINTER(_D)], _I),
    "stock_sched_coefficients": ([_V, _I, _V], _I),
    "stock_sched_step": ([_V, _V, _I, _V, _I64, _I], _I),
    "stock_sched_reset": ([_V], _I),
    "stock_conv2d": ([_V, _V, _V, _V, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I], _I),
    "stock_group_norm": ([_V, _V, _V, _V, _I64, _I64, _F, _I64, _I64, _I, _I], _I),
    "stock_upsample": ([_V, _V, _I64, _I64, _I64, _I64, _I64, _I], _I),
    "stock_transpose": ([_V, _V, _I64, _I64, _I64, _I, _I], _I),
    "stock_vae_forward": ([_V, _V, _V, _I64, _V, _I, _I], _I),
    "stock_t5_bucket": ([_I, _I, _I], _I),
    "stock_t5_forward": ([_V, _V, _V, _I64, _I64, _V, _I], _I),
}
_REF_SIGS = {
    "ref_last_error": ([], ctypes.c_char_p),
    "ref_gemm": ([_V, _V, _V, _V, _I64, _I64, _I64, _I, _I, _I], _I),
    "ref_attention": ([_V, _V, _V, _V, _I64, _I64, _I64, _I64, _I64, _F, _V, _V, _I, _I, _I], _I),
    "ref_norm": ([_V, _V, _V, _V, _I64, _I64, _F, _I, _I], _I),
    "ref_modulate": ([_V, _V, _V, _V, _I64, _I64, _I64, _V, _V, _I], _I),
    "ref_activation": ([_V, _V, _I64, _I, _V, _I], _I),
    "ref_add": ([_V, _V, _V, _I64, _I64, _F, _I, _I], _I),
    "ref_chunk": ([_V, _V, _V, _I64, _I64, _I64, _I64, _I64, _I, _I], _I),
    "ref_patch": ([_V, _V, _I64, _I64, _I64, _I64, _I, _I], _I),
    "ref_position_embedding": ([ctypes.POINTER(_D), _I, _I, _I, _D], _I),
    "ref_timestep_embedding": ([_D, _I, ctypes.POINTER(_F)], _I),
    "ref_dit_forward": ([_V, _V, _I64, _I64, _I64, _V, _D, _V, _V, _I, _V, _I], _I),
    "ref_scale": ([_V, _V, _I64, _F, _I], _I),
    "ref_repeat": ([_V, _V, _I64, _I64, _I], _I),
    "ref_guidance": ([_V, _V, _I64, _I64, _I64, _F, _I], _I),
    "ref_sched_create": ([_V, ctypes.POINTER(_V)], _I),
    "ref_sched_destroy": ([_V], None),
    "ref_sched_set_timesteps": ([_V, _I], _I),
    "ref_sched_steps": ([_V], _I),
    "ref_sched_timestep": ([_V, _I, ctypes.POINTER(_I64)], _I),
    "ref_sched_sigma": ([_V, _I, ctypes.POINTER(_D)], _I),
    "ref_sched_coefficients": ([_V, _I, _V], _I),
    "ref_sched_step": ([_V, _V, _I, _V, _I64, _I], _I),
    "ref_sched_reset": ([_V], _I),
    "ref_conv2d": ([_V, _V, _V, _V, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I], _I),
    "ref_group_norm": ([_V, _V, _V, _V, _I64, _I64, _F, _I64, _I64, _I], _I),
    "ref_upsample": ([_V, _V, _I64, _I64, _I64, _I64, _I64, _I], _I),
    "ref_transpose": ([_V, _V, _I64, _I64, _I64, _I, _I], _I),
    "ref_vae_forward": ([_V, _V, _V, _I64, _V], _I),
    "ref_t5_bucket": ([_I, _I, _I], _I),
    "ref_t5_forward": ([_V, _V, _V, _I64, _I64, _V], _I),
}

_stock = None
_ref = None


class OracleError(RuntimeError):
    pass


def _load(path: Path, sigs: dict) -> ctypes.CDLL:
    lib = ctypes.CDLL(str(path))
    for name, (args, ret) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = args, ret
    return lib


def build(reference: bool = True) -> None:
    """make -C oracle (and the `ref` and `registry` targets when /root/reference exists; the
    registry driver also needs the built burnisher_amd/lib/libburnisher_hip.so)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if reference and REFERENCE_ROOT.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)
        if (HERE.parent / "burnisher_amd" / "lib" / "libburnisher_hip.so").exists():
            subprocess.run(["make", "-s", "-C", str(HERE), "registry"], check=True)


REGISTRY_MAIN = HERE / "_ref" / "registry_main"


def registry_main() -> Path | None:
    """oracle/_ref/registry_main (the reference runtime with the hip-gfx950 registrations and the
    HIP device layer), or None where it was not built."""
    return REGISTRY_MAIN if REGISTRY_MAIN.exists() else None


def stock() -> ctypes.CDLL:
    global _stock
    if _stock is None:
        if not STOCK_PATH.exists():
            raise OracleError(f"{STOCK_PATH} is missing; run `make -C oracle`")
        _stock = _load(STOCK_PATH, _STOCK_SIGS)
    return _stock


def ref() -> ctypes.CDLL | None:
    global _ref
    if _ref is None and REF_PATH.exists():
        _ref = _load(REF_PATH, _REF_SIGS)
    return _ref


def call(lib: ctypes.CDLL, name: str, *args) -> None:
    if getattr(lib, name)(*args) != 0:
        err = (lib.stock_last_error() if hasattr(lib, "stock_last_error") else lib.ref_last_error())
        raise OracleError(f"{name}: {err.decode(errors='replace')}")
