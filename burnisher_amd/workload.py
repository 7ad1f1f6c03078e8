"""Synthetic dit-step workloads: the PixArt-Sigma DiT's weight table and inputs, seeded.

Weights are named and shaped as in the checkpoint (reference: src/models/weights.cpp:246-282) and
drawn N(0, 0.02^2) in bf16; the latent and caption are N(0, 1); timestep 500; the caption mask
keeps a prefix per batch row (row 0 a quarter of the caption, row 1 half of it), since under
classifier-free guidance the two rows have different lengths. Every tensor is drawn by
bh_fill_normal_bf16 keyed by its name, so the same workload is the same bytes in every process,
on every host, whatever the thread count.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import (BLOCK_FIELDS, BF16, TOP_FIELDS, DitBlockWeights, DitConfig, DitWeights,
               fill_normal_bf16)

SEED = 20260911
WEIGHT_STD = 0.02

# DiTConfig (models.h:105-118): the PixArt-Sigma 1024px transformer.
PIXART_SIGMA = dict(num_layers=28, num_heads=16, head_dim=72, patch_size=2, in_channels=4,
                    out_channels=8, caption_channels=4096, sample_size=128, mlp_ratio=4.0,
                    eps=1e-6)

# The BASELINE configs by resolution: latent side = resolution / 8 (the VAE factor).
RESOLUTIONS = {512: 64, 768: 96, 1024: 128, 1152: 144, 2048: 256}

# checkpoint name <- engine struct field
TOP_NAMES = {
    "pos_embed_w": "pos_embed.proj.weight", "pos_embed_b": "pos_embed.proj.bias",
    "t_emb1_w": "adaln_single.emb.timestep_embedder.linear_1.weight",
    "t_emb1_b": "adaln_single.emb.timestep_embedder.linear_1.bias",
    "t_emb2_w": "adaln_single.emb.timestep_embedder.linear_2.weight",
    "t_emb2_b": "adaln_single.emb.timestep_embedder.linear_2.bias",
    "adaln_w": "adaln_single.linear.weight", "adaln_b": "adaln_single.linear.bias",
    "cap1_w": "caption_projection.linear_1.weight", "cap1_b": "caption_projection.linear_1.bias",
    "cap2_w": "caption_projection.linear_2.weight", "cap2_b": "caption_projection.linear_2.bias",
    "out_table": "scale_shift_table", "proj_out_w": "proj_out.weight",
    "proj_out_b": "proj_out.bias",
}
BLOCK_NAMES = {
    "scale_shift_table": "scale_shift_table",
    "attn1_q_w": "attn1.to_q.weight", "attn1_q_b": "attn1.to_q.bias",
    "attn1_k_w": "attn1.to_k.weight", "attn1_k_b": "attn1.to_k.bias",
    "attn1_v_w": "attn1.to_v.weight", "attn1_v_b": "attn1.to_v.bias",
    "attn1_o_w": "attn1.to_out.0.weight", "attn1_o_b": "attn1.to_out.0.bias",
    "attn2_q_w": "attn2.to_q.weight", "attn2_q_b": "attn2.to_q.bias",
    "attn2_k_w": "attn2.to_k.weight", "attn2_k_b": "attn2.to_k.bias",
    "attn2_v_w": "attn2.to_v.weight", "attn2_v_b": "attn2.to_v.bias",
    "attn2_o_w": "attn2.to_out.0.weight", "attn2_o_b": "attn2.to_out.0.bias",
    "ff0_w": "ff.net.0.proj.weight", "ff0_b": "ff.net.0.proj.bias",
    "ff2_w": "ff.net.2.weight", "ff2_b": "ff.net.2.bias",
}


def d_model(cfg: dict) -> int:
    return cfg["num_heads"] * cfg["head_dim"]


def d_ff(cfg: dict) -> int:
    return int(d_model(cfg) * cfg["mlp_ratio"])


def top_shapes(cfg: dict) -> dict[str, tuple]:
    d, p = d_model(cfg), cfg["patch_size"]
    return {
        "pos_embed_w": (d, cfg["in_channels"], p, p), "pos_embed_b": (d,),
        "t_emb1_w": (d, 256), "t_emb1_b": (d,), "t_emb2_w": (d, d), "t_emb2_b": (d,),
        "adaln_w": (6 * d, d), "adaln_b": (6 * d,),
        "cap1_w": (d, cfg["caption_channels"]), "cap1_b": (d,),
        "cap2_w": (d, d), "cap2_b": (d,),
        "out_table": (2, d),
        "proj_out_w": (p * p * cfg["out_channels"], d), "proj_out_b": (p * p * cfg["out_channels"],),
    }


def block_shapes(cfg: dict) -> dict[str, tuple]:
    d, f = d_model(cfg), d_ff(cfg)
    s = {"scale_shift_table": (6, d)}
    for a in ("attn1", "attn2"):
        for p in ("q", "k", "v", "o"):
            s[f"{a}_{p}_w"] = (d, d)
            s[f"{a}_{p}_b"] = (d,)
    s.update({"ff0_w": (f, d), "ff0_b": (f,), "ff2_w": (d, f), "ff2_b": (d,)})
    return s


def config_struct(cfg: dict) -> DitConfig:
    return DitConfig(**{k: cfg[k] for k in (
        "num_layers", "num_heads", "head_dim", "patch_size", "in_channels", "out_channels",
        "caption_channels", "sample_size", "mlp_ratio", "eps")})


@dataclass
class DitWorkload:
    """Host (numpy, bf16 bits as uint16) weights and inputs of one dit-step."""
    cfg: dict
    batch: int
    latent_hw: int
    caption_len: int
    timestep: float
    top: dict = field(default_factory=dict)
    blocks: list = field(default_factory=list)
    latent: np.ndarray | None = None
    caption: np.ndarray | None = None
    mask: np.ndarray | None = None   # float32 [batch, caption_len]

    @property
    def tokens(self) -> int:
        g = self.latent_hw // self.cfg["patch_size"]
        return g * g

    def weight_struct(self, arrays_top: dict, arrays_blocks: list):
        """(DitWeights, keepalive) over any objects with an address: numpy arrays (host) or
        torch tensors (device)."""
        def addr(a):
            return a.ctypes.data if isinstance(a, np.ndarray) else a.data_ptr()
        blocks = (DitBlockWeights * len(arrays_blocks))()
        for i, blk in enumerate(arrays_blocks):
            for f in BLOCK_FIELDS:
                setattr(blocks[i], f, addr(blk[f]))
        w = DitWeights(**{f: addr(arrays_top[f]) for f in TOP_FIELDS})
        w.blocks = ctypes.cast(blocks, ctypes.POINTER(DitBlockWeights))
        return w, blocks

    def to_device(self, device="cuda"):
        """(top, blocks, latent, caption, mask) as torch tensors on `device` (bf16; mask fp32).

        Laid out as the checkpoint loader lays them (bh_dit_weights_load): each layer's
        self-attention Q, K, V weights in one allocation (and their biases in another), and every
        layer's cross-attention K, V weights in one allocation in layer order (biases likewise),
        so the fused engine reads its packed projections in place rather than copying them."""
        import torch

        def t(a):
            return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)
        top, blocks = self.weights_to_device(device)
        return (top, blocks, t(self.latent), t(self.caption),
                torch.from_numpy(self.mask).to(device))

    def weights_to_device(self, device="cuda"):
        """(top, blocks) of to_device: the weights alone, in the same packed layout."""
        import torch

        def t(a):
            return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)
        top = {k: t(v) for k, v in self.top.items()}
        packed = ("attn1_q", "attn1_k", "attn1_v", "attn2_k", "attn2_v")
        blocks = [{k: t(v) for k, v in b.items() if not k.startswith(packed)} for b in self.blocks]
        if self.blocks:
            kv_w = t(np.stack([np.stack([b["attn2_k_w"], b["attn2_v_w"]]) for b in self.blocks]))
            kv_b = t(np.stack([np.stack([b["attn2_k_b"], b["attn2_v_b"]]) for b in self.blocks]))
        for i, (src, blk) in enumerate(zip(self.blocks, blocks)):
            qkv_w = t(np.stack([src["attn1_q_w"], src["attn1_k_w"], src["attn1_v_w"]]))
            qkv_b = t(np.stack([src["attn1_q_b"], src["attn1_k_b"], src["attn1_v_b"]]))
            for j, p in enumerate("qkv"):
                blk[f"attn1_{p}_w"], blk[f"attn1_{p}_b"] = qkv_w[j], qkv_b[j]
            for j, p in enumerate("kv"):
                blk[f"attn2_{p}_w"], blk[f"attn2_{p}_b"] = kv_w[i, j], kv_b[i, j]
        return top, blocks


def prefix_mask(batch: int, caption_len: int) -> np.ndarray:
    """Row 0 keeps caption_len//4 tokens, row 1 caption_len//2 (each at least one); further rows
    alternate."""
    m = np.zeros((batch, caption_len), dtype=np.float32)
    for b in range(batch):
        keep = max(1, caption_len // 4 if b % 2 == 0 else caption_len // 2)
        m[b, :keep] = 1.0
    return m


def make_workload(cfg: dict | None = None, *, batch: int = 2, latent_hw: int = 128,
                  caption_len: int = 300, timestep: float = 500.0, seed: int = SEED,
                  layers: int | None = None) -> DitWorkload:
    cfg = dict(cfg or PIXART_SIGMA)
    if layers is not None:
        cfg["num_layers"] = layers
    w = DitWorkload(cfg, batch, latent_hw, caption_len, timestep)
    for f, shape in top_shapes(cfg).items():
        w.top[f] = fill_normal_bf16(int(np.prod(shape)), TOP_NAMES[f], seed, WEIGHT_STD).reshape(shape)
    for i in range(cfg["num_layers"]):
        blk = {}
        for f, shape in block_shapes(cfg).items():
            name = f"transformer_blocks.{i}.{BLOCK_NAMES[f]}"
            blk[f] = fill_normal_bf16(int(np.prod(shape)), name, seed, WEIGHT_STD).reshape(shape)
        w.blocks.append(blk)
    w.latent = fill_normal_bf16(batch * cfg["in_channels"] * latent_hw * latent_hw, "latent", seed,
                                1.0).reshape(batch, cfg["in_channels"], latent_hw, latent_hw)
    w.caption = fill_normal_bf16(batch * caption_len * cfg["caption_channels"], "caption", seed,
                                 1.0).reshape(batch, caption_len, cfg["caption_channels"])
    w.mask = prefix_mask(batch, caption_len)
    return w


# ---- algorithmic work (the reference's accounting, eval/burnscore/geometry.py:275-367) -------

def dit_step_flops(cfg: dict, *, batch: int, latent_hw: int, caption_len: int) -> dict:
    """FLOP of one dit-step by op family, restating the reference geometry: GEMMs 2mnk, attention
    4*B*H*Sq*Skv*dh, LayerNorm 5/element, modulation 2/element, gated residual 2/element,
    residual 1/element, GELU 9/element, position add 1/element, patch-embed conv
    2*grid^2*(cin*batch)*d*p^2. Reproduces 13,281,774,529,536 FLOP at 1024px and
    2,581,055,400,960 at 512px (eval/cells/BG-{1,2}/generation.json:49)."""
    L, H, dh = cfg["num_layers"], cfg["num_heads"], cfg["head_dim"]
    d, p = H * dh, cfg["patch_size"]
    cin, cout, cap = cfg["in_channels"], cfg["out_channels"], cfg["caption_channels"]
    dff = int(round(d * float(cfg["mlp_ratio"])))
    grid = latent_hw // p
    N = grid * grid
    M, Mc = batch * N, batch * caption_len
    g = lambda m, n, k: 2.0 * m * n * k
    gemm = (2.0 * grid * grid * (cin * batch) * d * p * p   # pos_embed conv, as the reference prices it
            + g(batch, d, 256) + g(batch, d, d) + g(batch, 6 * d, d)
            + g(Mc, d, cap) + g(Mc, d, d)
            + L * (4 * g(M, d, d) + g(M, d, d) + 2 * g(Mc, d, d) + g(M, d, d)
                   + g(M, dff, d) + g(M, d, dff))
            + g(M, p * p * cout, d))
    attn = L * (4.0 * batch * H * N * N * dh + 4.0 * batch * H * N * caption_len * dh)
    elem = (M * d                                   # position add
            + 9.0 * Mc * d                          # caption GELU
            + L * (5.0 * M * d + 2.0 * M * d + 2.0 * M * d    # norm1, modulate, gate residual
                   + 1.0 * M * d                    # attn2 residual
                   + 5.0 * M * d + 2.0 * M * d      # norm2, modulate
                   + 9.0 * M * dff + 2.0 * M * d)   # GELU, gate residual
            + 5.0 * M * d + 2.0 * M * d)            # norm_out, modulate
    return {"gemm": gemm, "attention": attn, "elementwise": elem, "total": gemm + attn + elem}
