"""The VAE decoder's configuration, weight table and seeded synthetic workload (vae-decode stage).

Names and shapes follow the reference's declaration of the decoder's checkpoint tensors
(src/models/weights.cpp:284-320, the VAE part of declare_pixart_shapes): convolutions
[out, in, k, k], the mid-block attention's projections [out, in], norms [channels]. Synthetic
weights are drawn per tensor name with bh_fill_normal_bf16: convolution and projection weights
N(0, 1/fan_in) so activations stay O(1) through the up-blocks, biases N(0, 0.02^2), GroupNorm
weights 1 + N(0, 0.1^2) and biases N(0, 0.1^2); the latent is N(0, 1).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import BF16, fill_normal_bf16

SEED = 20261202

# VaeConfig (models.h:120-130): the SDXL VAE that PixArt-Sigma decodes with.
SDXL_VAE = dict(block_out_channels=(128, 256, 512, 512), layers_per_block=2, latent_channels=4,
                norm_num_groups=32, eps=1e-6)


class VaeConfig(ctypes.Structure):
    _fields_ = [("block_out_channels", ctypes.c_int * 8), ("num_blocks", ctypes.c_int),
                ("layers_per_block", ctypes.c_int), ("latent_channels", ctypes.c_int),
                ("norm_num_groups", ctypes.c_int), ("eps", ctypes.c_double)]


class VaeWeights(ctypes.Structure):
    _fields_ = [("count", ctypes.c_int), ("names", ctypes.POINTER(ctypes.c_char_p)),
                ("tensors", ctypes.POINTER(ctypes.c_void_p))]


def config_struct(cfg: dict) -> VaeConfig:
    c = VaeConfig()
    boc = list(cfg["block_out_channels"])
    for i, v in enumerate(boc):
        c.block_out_channels[i] = v
    c.num_blocks = len(boc)
    c.layers_per_block = cfg["layers_per_block"]
    c.latent_channels = cfg["latent_channels"]
    c.norm_num_groups = cfg["norm_num_groups"]
    c.eps = cfg["eps"]
    return c


def scale_factor(cfg: dict) -> int:
    return 1 << (len(cfg["block_out_channels"]) - 1)


def vae_tensors(cfg: dict) -> dict[str, tuple]:
    """Checkpoint name -> shape, in the reference's declaration order."""
    out: dict[str, tuple] = {}
    zc = cfg["latent_channels"]
    rev = list(reversed(cfg["block_out_channels"]))

    def conv(n, ci, co, k):
        out[n + ".weight"] = (co, ci, k, k)
        out[n + ".bias"] = (co,)

    def gn(n, ch):
        out[n + ".weight"] = (ch,)
        out[n + ".bias"] = (ch,)

    def res(n, ci, co):
        gn(n + ".norm1", ci)
        conv(n + ".conv1", ci, co, 3)
        gn(n + ".norm2", co)
        conv(n + ".conv2", co, co, 3)
        if ci != co:
            conv(n + ".conv_shortcut", ci, co, 1)

    conv("post_quant_conv", zc, zc, 1)
    conv("decoder.conv_in", zc, rev[0], 3)
    res("decoder.mid_block.resnets.0", rev[0], rev[0])
    res("decoder.mid_block.resnets.1", rev[0], rev[0])
    gn("decoder.mid_block.attentions.0.group_norm", rev[0])
    for p in ("to_q", "to_k", "to_v", "to_out.0"):
        out[f"decoder.mid_block.attentions.0.{p}.weight"] = (rev[0], rev[0])
        out[f"decoder.mid_block.attentions.0.{p}.bias"] = (rev[0],)
    prev = rev[0]
    for i, co in enumerate(rev):
        for j in range(cfg["layers_per_block"] + 1):
            res(f"decoder.up_blocks.{i}.resnets.{j}", prev if j == 0 else co, co)
        prev = co
        if i + 1 != len(rev):
            conv(f"decoder.up_blocks.{i}.upsamplers.0.conv", co, co, 3)
    gn("decoder.conv_norm_out", prev)
    conv("decoder.conv_out", prev, 3, 3)
    return out


def _to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def _from_bf16(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def synthetic_tensor(name: str, shape: tuple, seed: int) -> np.ndarray:
    n = int(np.prod(shape))
    if "norm" in name:   # GroupNorm affine: weight near 1, bias near 0
        std = 0.1
        base = fill_normal_bf16(n, name, seed, std)
        if name.endswith(".weight"):
            return _to_bf16(_from_bf16(base) + np.float32(1.0)).reshape(shape)
        return base.reshape(shape)
    if name.endswith(".bias"):
        return fill_normal_bf16(n, name, seed, 0.02).reshape(shape)
    fan_in = int(np.prod(shape[1:]))
    return fill_normal_bf16(n, name, seed, float(1.0 / np.sqrt(fan_in))).reshape(shape)


@dataclass
class VaeWorkload:
    """Host (numpy bf16 bits) weights and latent of one decode; batch 1, NCHW."""
    cfg: dict
    latent_hw: int
    weights: dict = field(default_factory=dict)
    latent: np.ndarray | None = None

    @property
    def image_hw(self) -> int:
        return self.latent_hw * scale_factor(self.cfg)

    def table(self, tensors: dict | None = None):
        """(VaeWeights, keepalive) over numpy arrays (host) or torch tensors (device)."""
        src = self.weights if tensors is None else tensors
        names = list(src)
        arr_n = (ctypes.c_char_p * len(names))(*[n.encode() for n in names])

        def addr(a):
            return a.ctypes.data if isinstance(a, np.ndarray) else a.data_ptr()
        arr_t = (ctypes.c_void_p * len(names))(*[addr(src[n]) for n in names])
        w = VaeWeights(len(names), ctypes.cast(arr_n, ctypes.POINTER(ctypes.c_char_p)),
                       ctypes.cast(arr_t, ctypes.POINTER(ctypes.c_void_p)))
        return w, (arr_n, arr_t, src)

    def to_device(self, device="cuda"):
        import torch

        def t(a):
            return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)
        return {k: t(v) for k, v in self.weights.items()}, t(self.latent)


def make_vae_workload(cfg: dict | None = None, *, latent_hw: int = 128, seed: int = SEED) -> VaeWorkload:
    cfg = dict(cfg or SDXL_VAE)
    wl = VaeWorkload(cfg=cfg, latent_hw=latent_hw)
    for name, shape in vae_tensors(cfg).items():
        wl.weights[name] = synthetic_tensor(name, shape, seed)
    wl.latent = fill_normal_bf16(cfg["latent_channels"] * latent_hw * latent_hw, "vae_latent", seed,
                                 1.0).reshape(1, cfg["latent_channels"], latent_hw, latent_hw)
    return wl


def vae_decode_flops(cfg: dict, latent_hw: int) -> dict:
    """Algorithmic FLOP of one decode: 2 x MACs of every convolution and projection, and
    4 x S^2 x C for the mid-block attention (QK^T and PV), as eval/burnscore/geometry.py counts
    attention. Norms, activations, adds and copies are not counted."""
    rev = list(reversed(cfg["block_out_channels"]))
    zc = cfg["latent_channels"]
    h = latent_hw
    conv = 0.0

    def c(ci, co, k, hh):
        return 2.0 * ci * co * k * k * hh * hh

    conv += c(zc, zc, 1, h) + c(zc, rev[0], 3, h)

    def res(ci, co, hh):
        return c(ci, co, 3, hh) + c(co, co, 3, hh) + (c(ci, co, 1, hh) if ci != co else 0.0)

    conv += 2 * res(rev[0], rev[0], h)
    s = h * h
    proj = 4 * 2.0 * s * rev[0] * rev[0]
    attn = 4.0 * s * s * rev[0]
    prev = rev[0]
    for i, co in enumerate(rev):
        for j in range(cfg["layers_per_block"] + 1):
            conv += res(prev if j == 0 else co, co, h)
        prev = co
        if i + 1 != len(rev):
            h *= 2
            conv += c(co, co, 3, h)
    conv += c(prev, 3, 3, h)
    return {"conv": conv, "attention_proj": proj, "attention": attn, "total": conv + proj + attn}
