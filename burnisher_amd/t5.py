"""The T5 v1.1 encoder's configuration, weight table and seeded synthetic workload (t5-encode
stage).

Names and shapes follow the reference's declaration of the encoder's checkpoint tensors
(src/models/weights.cpp:226-244, the T5 part of declare_pixart_shapes): linear weights
[out, in], RMSNorm weights [d_model], the shared embedding [vocab_size, d_model] and the relative
attention bias [num_buckets, num_heads]. Synthetic weights are drawn per tensor name with
bh_fill_normal_bf16: projections N(0, 1/fan_in) except q, N(0, 1/(fan_in * d_kv)) (T5 does not
scale its scores; the 1/sqrt(d_kv) lives in q's initialisation), the embedding and the relative bias N(0, 1),
norm weights 1 + N(0, 0.1^2). Token ids are seeded integers in [2, vocab_size) closed by the
end-of-sequence id 1 and padded with id 0, as a tokenizer pads to the caption length.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import fill_normal_bf16
from .vae import VaeWeights as NamedWeights
from .vae import _from_bf16, _to_bf16

SEED = 20261203

# T5Config (models.h:94-103): T5 v1.1 XXL, the PixArt-Sigma text encoder; 32 relative buckets
# (weights.cpp:231-232).
T5_XXL = dict(num_layers=24, d_model=4096, d_ff=10240, d_kv=64, num_heads=64, vocab_size=32128,
              gated=1, num_buckets=32, eps=1e-6)


class T5Config(ctypes.Structure):
    _fields_ = [("num_layers", ctypes.c_int), ("d_model", ctypes.c_int), ("d_ff", ctypes.c_int),
                ("d_kv", ctypes.c_int), ("num_heads", ctypes.c_int), ("vocab_size", ctypes.c_int),
                ("gated", ctypes.c_int), ("num_buckets", ctypes.c_int), ("eps", ctypes.c_double)]


def config_struct(cfg: dict) -> T5Config:
    return T5Config(*(int(cfg[k]) for k in ("num_layers", "d_model", "d_ff", "d_kv", "num_heads",
                                            "vocab_size", "gated", "num_buckets")), float(cfg["eps"]))


def t5_tensors(cfg: dict) -> dict[str, tuple]:
    """Checkpoint name -> shape, in the reference's declaration order."""
    d, inner = cfg["d_model"], cfg["num_heads"] * cfg["d_kv"]
    out = {"shared.weight": (cfg["vocab_size"], d), "encoder.final_layer_norm.weight": (d,),
           "encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight":
               (cfg["num_buckets"], cfg["num_heads"])}
    for i in range(cfg["num_layers"]):
        b = f"encoder.block.{i}."
        out[b + "layer.0.layer_norm.weight"] = (d,)
        out[b + "layer.1.layer_norm.weight"] = (d,)
        for p in ("q", "k", "v"):
            out[b + f"layer.0.SelfAttention.{p}.weight"] = (inner, d)
        out[b + "layer.0.SelfAttention.o.weight"] = (d, inner)
        out[b + "layer.1.DenseReluDense.wi_0.weight"] = (cfg["d_ff"], d)
        if cfg["gated"]:
            out[b + "layer.1.DenseReluDense.wi_1.weight"] = (cfg["d_ff"], d)
        out[b + "layer.1.DenseReluDense.wo.weight"] = (d, cfg["d_ff"])
    return out


def synthetic_tensor(name: str, shape: tuple, seed: int, d_kv: int = 64) -> np.ndarray:
    n = int(np.prod(shape))
    if name.endswith("SelfAttention.q.weight"):   # T5 folds 1/sqrt(d_kv) into q's initialisation
        return fill_normal_bf16(n, name, seed, float(1.0 / np.sqrt(shape[1] * d_kv))).reshape(shape)
    if "layer_norm" in name:
        return _to_bf16(_from_bf16(fill_normal_bf16(n, name, seed, 0.1)) + np.float32(1.0)).reshape(shape)
    if name == "shared.weight" or "relative_attention_bias" in name:
        return fill_normal_bf16(n, name, seed, 1.0).reshape(shape)
    return fill_normal_bf16(n, name, seed, float(1.0 / np.sqrt(shape[1]))).reshape(shape)


def synthetic_ids(batch: int, seq: int, vocab: int, lengths, seed: int) -> np.ndarray:
    """fp32 [batch, seq]: row b holds lengths[b] tokens (the last is end-of-sequence id 1), then
    pad id 0."""
    rng = np.random.default_rng(seed)
    ids = np.zeros((batch, seq), np.float32)
    for b in range(batch):
        n = min(int(lengths[b]), seq)
        if n > 0:
            ids[b, :n - 1] = rng.integers(2, vocab, n - 1)
            ids[b, n - 1] = 1
    return ids


@dataclass
class T5Workload:
    """Host (numpy bf16 bits) weights and fp32 token ids of one encode."""
    cfg: dict
    batch: int
    seq: int
    weights: dict = field(default_factory=dict)
    ids: np.ndarray | None = None

    def table(self, tensors: dict | None = None):
        """(bh_t5_weights, keepalive) over numpy arrays (host) or torch tensors (device)."""
        src = self.weights if tensors is None else tensors
        names = list(src)
        arr_n = (ctypes.c_char_p * len(names))(*[n.encode() for n in names])

        def addr(a):
            return a.ctypes.data if isinstance(a, np.ndarray) else a.data_ptr()
        arr_t = (ctypes.c_void_p * len(names))(*[addr(src[n]) for n in names])
        w = NamedWeights(len(names), ctypes.cast(arr_n, ctypes.POINTER(ctypes.c_char_p)),
                         ctypes.cast(arr_t, ctypes.POINTER(ctypes.c_void_p)))
        return w, (arr_n, arr_t, src)

    def to_device(self, device="cuda") -> dict:
        import torch
        return {k: torch.from_numpy(np.ascontiguousarray(v).view(np.int16)).view(torch.bfloat16).to(device)
                for k, v in self.weights.items()}


def make_t5_workload(cfg: dict | None = None, *, batch: int = 2, seq: int = 300, lengths=None,
                     seed: int = SEED) -> T5Workload:
    cfg = dict(cfg or T5_XXL)
    wl = T5Workload(cfg=cfg, batch=batch, seq=seq)
    for name, shape in t5_tensors(cfg).items():
        wl.weights[name] = synthetic_tensor(name, shape, seed, cfg["d_kv"])
    if lengths is None:   # classifier-free guidance: the empty negative prompt, then a caption
        lengths = [1] + [max(2, (seq * 2) // 5)] * (batch - 1)
    wl.ids = synthetic_ids(batch, seq, cfg["vocab_size"], lengths, seed)
    return wl


def t5_encode_flops(cfg: dict, batch: int, seq: int) -> dict:
    """Algorithmic FLOP of one encode: 2 x MACs of every projection and 4 x S^2 x d_kv per head
    for attention (QK^T and PV). Norms, the gather, activations and adds are not counted."""
    m, d, f = batch * seq, cfg["d_model"], cfg["d_ff"]
    inner = cfg["num_heads"] * cfg["d_kv"]
    per = 2.0 * m * (4 * inner * d + (3 if cfg["gated"] else 2) * f * d)
    att = 4.0 * batch * cfg["num_heads"] * seq * seq * cfg["d_kv"]
    layers = cfg["num_layers"]
    return {"gemm": per * layers, "attention": att * layers, "total": (per + att) * layers}
