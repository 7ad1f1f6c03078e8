"""burnisher_amd -- Python access to libburnisher_hip.so, the gfx950 dit-step library.

The library's C ABI (include/burnisher_hip.h) is the product boundary; this module only loads
it with ctypes and wraps each entry point so that a failing status raises `BurnisherError` with
the library's message. Device memory and streams come from PyTorch (tensors are passed by
`data_ptr()`); PyTorch computes nothing here.

If the library is missing this module raises on first use -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libburnisher_hip.so"

F32, BF16 = 0, 1
ST_F32, ST_BF16, ST_F16, ST_F8_E4M3 = 0, 1, 2, 3
ST_DTYPES = {ST_F32: "F32", ST_BF16: "BF16", ST_F16: "F16", ST_F8_E4M3: "F8_E4M3"}
EPI_NONE, EPI_GELU, EPI_SILU, EPI_GELU_GATED = 0, 1, 2, 3
DIT_FUSED, DIT_OPWISE = 0, 1
ROWS_JOINED, ROWS_SPLIT = 0, 1
(K_GEMM, K_GEMV, K_ATTN_SELF, K_ATTN_CROSS, K_NORM, K_ELEMENTWISE, K_GEMM_FF0, K_GEMM_FF2,
 K_GEMM_QKV) = range(9)
KERNEL_CLASSES = ["gemm", "gemv", "attention_self", "attention_cross", "norm", "elementwise",
                  "gemm_ff0", "gemm_ff2", "gemm_qkv"]


class BurnisherError(RuntimeError):
    pass


# ---- C structs (include/burnisher_hip.h) --------------------------------------------------

class GemmFused(ctypes.Structure):
    _fields_ = [("epilogue", ctypes.c_int), ("round_mid", ctypes.c_int),
                ("row_add", ctypes.c_void_p), ("row_add_period", ctypes.c_int64),
                ("residual", ctypes.c_void_p), ("gate", ctypes.c_void_p),
                ("gate_rows", ctypes.c_int64), ("ld_out", ctypes.c_int64)]


class DitConfig(ctypes.Structure):
    _fields_ = [("num_layers", ctypes.c_int), ("num_heads", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("patch_size", ctypes.c_int),
                ("in_channels", ctypes.c_int), ("out_channels", ctypes.c_int),
                ("caption_channels", ctypes.c_int), ("sample_size", ctypes.c_int),
                ("mlp_ratio", ctypes.c_double), ("eps", ctypes.c_double)]


BLOCK_FIELDS = ["scale_shift_table",
                "attn1_q_w", "attn1_q_b", "attn1_k_w", "attn1_k_b", "attn1_v_w", "attn1_v_b",
                "attn1_o_w", "attn1_o_b",
                "attn2_q_w", "attn2_q_b", "attn2_k_w", "attn2_k_b", "attn2_v_w", "attn2_v_b",
                "attn2_o_w", "attn2_o_b",
                "ff0_w", "ff0_b", "ff2_w", "ff2_b"]
TOP_FIELDS = ["pos_embed_w", "pos_embed_b", "t_emb1_w", "t_emb1_b", "t_emb2_w", "t_emb2_b",
              "adaln_w", "adaln_b", "cap1_w", "cap1_b", "cap2_w", "cap2_b", "out_table",
              "proj_out_w", "proj_out_b"]


class DitBlockWeights(ctypes.Structure):
    _fields_ = [(f, ctypes.c_void_p) for f in BLOCK_FIELDS]


class DitWeights(ctypes.Structure):
    _fields_ = [(f, ctypes.c_void_p) for f in TOP_FIELDS] + [
        ("blocks", ctypes.POINTER(DitBlockWeights))]


class SchedConfig(ctypes.Structure):
    _fields_ = [("num_train_timesteps", ctypes.c_int), ("beta_start", ctypes.c_double),
                ("beta_end", ctypes.c_double), ("beta_schedule", ctypes.c_char_p),
                ("solver_order", ctypes.c_int), ("algorithm_type", ctypes.c_char_p),
                ("solver_type", ctypes.c_char_p), ("prediction_type", ctypes.c_char_p),
                ("timestep_spacing", ctypes.c_char_p), ("lower_order_final", ctypes.c_int)]

    @classmethod
    def pinned(cls, **overrides) -> "SchedConfig":
        """The PixArt-Sigma configuration (scheduler.h:21-30), optionally changed field by field."""
        fields = dict(num_train_timesteps=1000, beta_start=0.0001, beta_end=0.02,
                      beta_schedule=b"linear", solver_order=2, algorithm_type=b"dpmsolver++",
                      solver_type=b"midpoint", prediction_type=b"epsilon",
                      timestep_spacing=b"linspace", lower_order_final=1)
        fields.update(overrides)
        return cls(**fields)


class ProbeResult(ctypes.Structure):
    _fields_ = [(f, ctypes.c_double) for f in (
        "mfma_tflops", "mfma_shader_mhz", "mfma_shader_mhz_min", "mfma_shader_mhz_max",
        "mfma_peak_at_clock_tflops", "copy_gbs", "max_clock_mhz", "wall_clock_mhz")] + \
        [("cus", ctypes.c_int)]

    def as_dict(self) -> dict:
        return {f: (round(getattr(self, f), 2) if f != "cus" else self.cus) for f, _ in self._fields_}


class SchedCoefficients(ctypes.Structure):
    _fields_ = [("order", ctypes.c_int)] + [
        (f, ctypes.c_double) for f in ("sigma_s0", "sigma_t", "sigma_vp_s0", "sigma_vp_t",
                                       "alpha_t", "alpha_s0", "exp_neg_h", "r0")]


# ---- loading -------------------------------------------------------------------------------

_lib = None

_V, _I, _I64, _F, _D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_double
SIGNATURES = {
    "bh_abi_version": ([], _I),
    "bh_build_info": ([], ctypes.c_char_p),
    "bh_last_error": ([], ctypes.c_char_p),
    "bh_init": ([_I], _I),
    "bh_set_operand_checks": ([_I], _I),
    "bh_synchronize": ([_V], _I),
    "bh_gemm": ([_V, _V, _V, _V, _I64, _I64, _I64, _I, _I, _I, _V], _I),
    "bh_gemm_fused_run": ([_V, _V, _V, _V, _I64, _I64, _I64, ctypes.POINTER(GemmFused), _V], _I),
    "bh_attention": ([_V, _V, _V, _V, _I64, _I64, _I64, _I64, _I64, _F, _V, _V, _I, _I, _V], _I),
    "bh_attention_noalloc": ([_V, _V, _V, _V, _I64, _I64, _I64, _I64, _I64, _F, _V, _V, _I, _I, _V], _I),
    "bh_attention_strided": ([_V, _I64, _V, _V, _I64, _V, _I64, _I64, _I64, _I64, _I64, _I64, _F,
                              _V, _I, _I, _V], _I),
    "bh_norm": ([_V, _V, _V, _V, _I64, _I64, _F, _I, _I64, _I64, _I, _V], _I),
    "bh_modulate": ([_V, _V, _V, _V, _I64, _I64, _I64, _V, _V, _I, _V], _I),
    "bh_activation": ([_V, _V, _I64, _I, _V, _I, _V], _I),
    "bh_add": ([_V, _V, _V, _I64, _I64, _F, _I, _I, _V], _I),
    "bh_chunk": ([_V, _V, _V, _I64, _I64, _I64, _I64, _I64, _I, _V], _I),
    "bh_patch": ([_V, _V, _I64, _I64, _I64, _I64, _I, _I, _V], _I),
    "bh_norm_modulate": ([_V, _V, _I64, _I64, _I64, _V, _I64, _I64, _V, _I64, _I64, _I64, _F, _V],
                         _I),
    "bh_dit_create": ([ctypes.POINTER(DitConfig), ctypes.POINTER(DitWeights), _I64, _I64, _I64, _I,
                       ctypes.POINTER(_V)], _I),
    "bh_dit_forward": ([_V, _V, _D, _V, _V, _I, _V, _V], _I),
    "bh_dit_workspace_bytes": ([_V], _I64),
    "bh_dit_position_table": ([_V, _V, _V], _I),
    "bh_dit_set_rows": ([_V, _I], _I),
    "bh_scale": ([_V, _V, _I64, _F, _I, _V], _I),
    "bh_timestep_embedding": ([_D, _I, _I64, _V, _I, _V], _I),
    "bh_probe_device": ([_V, _V, _I64, ctypes.POINTER(ProbeResult)], _I),
    "bh_dit_destroy": ([_V], None),
    "bh_profile_enable": ([_I], _I),
    "bh_profile_sample": ([_I], _I),
    "bh_profile_read": ([_I, ctypes.POINTER(_D), ctypes.POINTER(_I64), ctypes.POINTER(_D)], _I),
    "bh_fill_normal_bf16": ([_V, _I64, ctypes.c_uint64, ctypes.c_char_p, _F], _I),
    "bh_repeat": ([_V, _V, _I64, _I64, _I, _V], _I),
    "bh_guidance": ([_V, _V, _I64, _I64, _I64, _F, _I, _V], _I),
    "bh_sched_config_default": ([ctypes.POINTER(SchedConfig)], None),
    "bh_sched_create": ([ctypes.POINTER(SchedConfig), ctypes.POINTER(_V)], _I),
    "bh_sched_set_timesteps": ([_V, _I], _I),
    "bh_sched_steps": ([_V], _I),
    "bh_sched_timestep": ([_V, _I], _I64),
    "bh_sched_sigma": ([_V, _I], _D),
    "bh_sched_init_noise_sigma": ([_V], _D),
    "bh_sched_get_coefficients": ([_V, _I, ctypes.POINTER(SchedCoefficients)], _I),
    "bh_sched_reserve": ([_V, _I64, _I], _I),
    "bh_sched_step": ([_V, _V, _I, _V, _I64, _I, _V], _I),
    "bh_sched_reset": ([_V], _I),
    "bh_sched_destroy": ([_V], None),
    "bh_denoiser_create": ([_V, _V, _I, _F, ctypes.POINTER(_V)], _I),
    "bh_denoiser_run": ([_V, _V, _V, _V, _I, _I, _V], _I),
    "bh_denoiser_destroy": ([_V], None),
    "bh_checkpoint_open": ([ctypes.POINTER(ctypes.c_char_p), _I, ctypes.POINTER(_V)], _I),
    "bh_checkpoint_open_component": ([ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_V)], _I),
    "bh_checkpoint_close": ([_V], None),
    "bh_checkpoint_count": ([_V], _I64),
    "bh_checkpoint_entry": ([_V, _I64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_I),
                             ctypes.POINTER(_I), ctypes.POINTER(_I64), _I], _I),
    "bh_checkpoint_find": ([_V, ctypes.c_char_p, ctypes.POINTER(_I), ctypes.POINTER(_I),
                            ctypes.POINTER(_I64), _I], _I),
    "bh_checkpoint_read": ([_V, ctypes.c_char_p, _I, _V, _I64], _I),
    "bh_dit_weights_load": ([_V, ctypes.POINTER(DitConfig), _V, ctypes.POINTER(_V)], _I),
    "bh_dit_weights_view": ([_V], ctypes.POINTER(DitWeights)),
    "bh_dit_weights_bytes": ([_V], _I64),
    "bh_dit_weights_free": ([_V], None),
    "bh_vae_create": ([_V, _V, _I64, ctypes.POINTER(_V)], _I),
    "bh_vae_decode": ([_V, _V, _V, _V], _I),
    "bh_vae_workspace_bytes": ([_V], _I64),
    "bh_vae_destroy": ([_V], None),
    "bh_t5_relative_bucket": ([_I, _I, _I], _I),
    "bh_gather": ([_V, _V, _V, _I64, _I64, _I64, _I, _V], _I),
    "bh_t5_create": ([_V, _V, _I64, _I64, _V], _I),
    "bh_t5_encode": ([_V, _V, _V, _V], _I),
    "bh_t5_workspace_bytes": ([_V], _I64),
    "bh_t5_destroy": ([_V], None),
    "bh_t5_weights_load": ([_V, _V, _V, _V], _I),
    "bh_t5_weights_view": ([_V], _V),
    "bh_t5_weights_bytes": ([_V], _I64),
    "bh_t5_weights_free": ([_V], None),
    "bh_conv2d": ([_V, _V, _V, _V, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _V], _I),
    "bh_vae_weights_load": ([_V, _V, _V, ctypes.POINTER(_V)], _I),
    "bh_vae_weights_view": ([_V], _V),
    "bh_vae_weights_bytes": ([_V], _I64),
    "bh_vae_weights_free": ([_V], None),
    "bh_upsample": ([_V, _V, _I64, _I64, _I64, _I64, _I64, _I, _V], _I),
    "bh_transpose": ([_V, _V, _I64, _I64, _I64, _I, _I, _V], _I),
}


def lib() -> ctypes.CDLL:
    """The loaded library. Raises if it has not been built (python -m burnisher_amd.build)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise BurnisherError(
                f"{LIB_PATH} is missing: build it with `python -m burnisher_amd.build` "
                "(there is no CPU fallback for the hip-gfx950 path)")
        handle = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (args, ret) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = ret
        _lib = handle
    return _lib


def check(status: int, what: str = "") -> None:
    if status != 0:
        msg = lib().bh_last_error().decode(errors="replace")
        raise BurnisherError(f"{what}: {msg}" if what else msg)


def call(name: str, *args):
    """Calls entry point `name`; a nonzero status raises BurnisherError with its message."""
    status = getattr(lib(), name)(*args)
    check(status, name)


def ptr(t) -> int | None:
    """Device (or host) address of a torch tensor, None for None."""
    return None if t is None else t.data_ptr()


def stream_ptr(stream=None) -> int | None:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def fill_normal_bf16(n: int, name: str, seed: int, std: float):
    """n draws of N(0, std^2) as a uint16 numpy array of bf16 bits (host), keyed by name."""
    import numpy as np
    out = np.empty(n, dtype=np.uint16)
    call("bh_fill_normal_bf16", out.ctypes.data, n, seed, name.encode(), std)
    return out


# ---- checkpoints ---------------------------------------------------------------------------

class Checkpoint:
    """A safetensors checkpoint component, memory-mapped by the library (bh_checkpoint_*).

    Mirrors the reference's CheckpointWeights (src/models/weights.cpp:26-69): `has`, `shape`,
    `read` (host conversion to bf16 bits or fp32) and `require`, whose miss names near misses.
    """

    MAX_RANK = 8

    def __init__(self, handle: int):
        self._h = ctypes.c_void_p(handle)

    @classmethod
    def open(cls, *shards) -> "Checkpoint":
        paths = (ctypes.c_char_p * len(shards))(*[os.fsencode(str(p)) for p in shards])
        h = ctypes.c_void_p()
        call("bh_checkpoint_open", paths, len(shards), ctypes.byref(h))
        return cls(h.value)

    @classmethod
    def component(cls, directory, name: str) -> "Checkpoint":
        h = ctypes.c_void_p()
        call("bh_checkpoint_open_component", os.fsencode(str(directory)), name.encode(),
             ctypes.byref(h))
        return cls(h.value)

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise BurnisherError("checkpoint is closed")
        return self._h

    def close(self) -> None:
        if self._h is not None:
            lib().bh_checkpoint_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def entries(self) -> list[tuple[str, str, tuple]]:
        """(name, dtype name, shape) of every tensor, shard by shard, in name order."""
        out = []
        shape = (ctypes.c_int64 * self.MAX_RANK)()
        name, dt, rank = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int()
        for i in range(lib().bh_checkpoint_count(self.handle)):
            call("bh_checkpoint_entry", self.handle, i, ctypes.byref(name), ctypes.byref(dt),
                 ctypes.byref(rank), shape, self.MAX_RANK)
            out.append((name.value.decode(), ST_DTYPES[dt.value], tuple(shape[:rank.value])))
        return out

    def require(self, name: str) -> tuple[str, tuple]:
        """(dtype name, shape) of `name`; raises naming near misses when it is absent."""
        shape = (ctypes.c_int64 * self.MAX_RANK)()
        dt, rank = ctypes.c_int(), ctypes.c_int()
        call("bh_checkpoint_find", self.handle, name.encode(), ctypes.byref(dt),
             ctypes.byref(rank), shape, self.MAX_RANK)
        return ST_DTYPES[dt.value], tuple(shape[:rank.value])

    def has(self, name: str) -> bool:
        return lib().bh_checkpoint_find(self.handle, name.encode(), None, None, None, 0) == 0

    def read(self, name: str, dtype: int = BF16):
        """The tensor converted on the host: bf16 bits (uint16) or float32, in its shape."""
        import numpy as np
        _, shape = self.require(name)
        out = np.empty(shape, dtype=np.uint16 if dtype == BF16 else np.float32)
        call("bh_checkpoint_read", self.handle, name.encode(), dtype, out.ctypes.data, out.size)
        return out


class DitDeviceWeights:
    """The DiT's weights from a checkpoint, bf16 in one device arena (bh_dit_weights_load).

    `weights` is the DitWeights struct bh_dit_create takes; it stays valid until `free`."""

    def __init__(self, checkpoint: Checkpoint, cfg: DitConfig, stream=None):
        h = ctypes.c_void_p()
        call("bh_dit_weights_load", checkpoint.handle, ctypes.byref(cfg), stream, ctypes.byref(h))
        self._h = h
        self.weights = lib().bh_dit_weights_view(h).contents
        self.bytes = lib().bh_dit_weights_bytes(h)

    def free(self) -> None:
        if self._h is not None:
            lib().bh_dit_weights_free(self._h)
            self._h = None
            self.weights = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class T5DeviceWeights:
    """The T5 encoder's weights from a checkpoint's `text_encoder/` component, bf16 in one device
    arena (bh_t5_weights_load). `table` is the address of the bh_t5_weights bh_t5_create takes."""

    def __init__(self, checkpoint: Checkpoint, cfg, stream=None):
        h = ctypes.c_void_p()
        call("bh_t5_weights_load", checkpoint.handle, ctypes.byref(cfg), stream, ctypes.byref(h))
        self._h = h
        self.table = lib().bh_t5_weights_view(h)
        self.bytes = lib().bh_t5_weights_bytes(h)

    def free(self) -> None:
        if self._h is not None:
            lib().bh_t5_weights_free(self._h)
            self._h = None
            self.table = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class VaeDeviceWeights:
    """The VAE decoder's weights from a checkpoint's `vae/` component, bf16 in one device arena
    (bh_vae_weights_load). `table` is the address of the bh_vae_weights bh_vae_create takes."""

    def __init__(self, checkpoint: Checkpoint, cfg, stream=None):
        h = ctypes.c_void_p()
        call("bh_vae_weights_load", checkpoint.handle, ctypes.byref(cfg), stream, ctypes.byref(h))
        self._h = h
        self.table = lib().bh_vae_weights_view(h)
        self.bytes = lib().bh_vae_weights_bytes(h)

    def free(self) -> None:
        if self._h is not None:
            lib().bh_vae_weights_free(self._h)
            self._h = None
            self.table = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
