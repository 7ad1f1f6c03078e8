"""Single stages from .npy inputs and a checkpoint directory: `dit-step` and `vae-decode`.

    python -m burnisher_amd.stage dit-step --weights DIR --latent L.npy --caption C.npy \\
        --mask M.npy --out O.npy [--timestep 500] [--layers N] [--warmup 1] [--plan fused]
    python -m burnisher_amd.stage vae-decode --weights DIR --latent L.npy --out O.npy [--warmup 1]

`vae-decode` mirrors the reference CLI's `decode` command (tools/burnisher_main.cpp:636-690): a
[1, 4, h, w] float32 latent (h == w here), the `vae/` component of the checkpoint, no division by
the scaling factor (that is the pipeline's, burnisher_main.cpp:661-663), output [1, 3, 8h, 8w].

Mirrors the reference CLI's `dit-step` command (tools/burnisher_main.cpp:694-747) for the
`hip-gfx950` implementation: the inputs are little-endian C-order float32 .npy files
(read_npy, burnisher_main.cpp:183-224, which refuses anything else), converted to bf16 with
round-to-nearest-even; the weights are the `transformer/` component of a safetensors checkpoint
(CheckpointWeights::component), converted to bf16 and uploaded once (bh_dit_weights_load);
`--layers` truncates the block stack; one untimed warm-up forward, then one timed forward
between two device synchronisations; the output is written as float32 .npy and the run is
reported as one `BURNISH_JSON:` line with the latency, the peak device memory, the effective
configuration and the output statistics (OutputStats::of, src/core/pipeline.cpp:9-24).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import sys
import time

import numpy as np

from . import (BF16, DIT_FUSED, DIT_OPWISE, BurnisherError, Checkpoint, DitDeviceWeights,
               T5DeviceWeights, VaeDeviceWeights, call, lib)
from .workload import PIXART_SIGMA, config_struct


def read_npy_f32(path: str) -> np.ndarray:
    """A little-endian C-order float32 .npy; any other dtype or order is refused, not converted
    (burnisher_main.cpp:195-202)."""
    arr = np.load(path, allow_pickle=False, mmap_mode="r")
    if arr.dtype != np.dtype("<f4"):
        raise BurnisherError(f"{path}: only little-endian fp32 is read (got {arr.dtype}); "
                             "converting silently would change the thing being compared")
    if arr.ndim > 1 and arr.flags.f_contiguous and not arr.flags.c_contiguous:
        raise BurnisherError(f"{path}: Fortran order is not read")
    return np.ascontiguousarray(arr)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bf16 bits with NaN kept NaN (the reference's f32_to_bf16,
    include/burnisher/dtype.h:64-72)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    return np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def output_stats(x: np.ndarray) -> dict:
    """Mean, population standard deviation (from E[x^2] - mean^2, floored at 0) and absolute
    maximum in float64 (OutputStats::of, pipeline.cpp:9-24)."""
    v = np.asarray(x, dtype=np.float64).ravel()
    if v.size == 0:
        return {"latent_mean": 0.0, "latent_std": 0.0, "latent_absmax": 0.0}
    mean = float(v.sum() / v.size)
    var = float((v * v).sum() / v.size - mean * mean)
    return {"latent_mean": mean, "latent_std": float(np.sqrt(max(0.0, var))),
            "latent_absmax": float(np.abs(v).max())}


def dit_step(weights: str, latent_path: str, caption_path: str, mask_path: str, out_path: str,
             timestep: float = 500.0, layers: int | None = None, warmup: int = 1,
             plan: str = "fused") -> dict:
    """Runs the stage; returns the BURNISH_JSON record (also written as one line to stdout by
    main)."""
    import torch

    cfg_d = dict(PIXART_SIGMA)
    if layers is not None:
        cfg_d["num_layers"] = int(layers)
    cfg = config_struct(cfg_d)
    latent = read_npy_f32(latent_path)
    caption = read_npy_f32(caption_path)
    mask = read_npy_f32(mask_path)
    if latent.ndim != 4 or latent.shape[1] != cfg.in_channels or latent.shape[2] != latent.shape[3]:
        raise BurnisherError(f"dit-step: latent must be [B, {cfg.in_channels}, H, H], got "
                             f"{list(latent.shape)}")
    batch, hw = latent.shape[0], latent.shape[2]
    if caption.ndim != 3 or caption.shape[0] != batch or caption.shape[2] != cfg.caption_channels:
        raise BurnisherError(f"dit-step: caption must be [{batch}, L, {cfg.caption_channels}], "
                             f"got {list(caption.shape)}")
    cap_len = caption.shape[1]
    if mask.size != batch * cap_len:   # pixart_dit.cpp:207-213
        raise BurnisherError(f"dit-step: caption_mask has {mask.size} elements, expected "
                             f"batch x caption_len = {batch * cap_len}")

    assert torch.cuda.is_available(), "the hip-gfx950 dit-step needs an MI355X"
    call("bh_init", 0)
    dev = "cuda"

    def upload(a: np.ndarray):
        bits = f32_to_bf16_bits(a)
        return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(dev)

    d_latent, d_caption, d_mask = upload(latent), upload(caption), upload(mask)
    out = torch.zeros((batch, cfg.out_channels, hw, hw), dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    with Checkpoint.component(weights, "transformer") as ck:
        dw = DitDeviceWeights(ck, cfg, stream)
    engine = ctypes.c_void_p()
    mode = {"fused": DIT_FUSED, "opwise": DIT_OPWISE}[plan]
    try:
        call("bh_dit_create", ctypes.byref(cfg), ctypes.byref(dw.weights), batch, hw, cap_len,
             mode, ctypes.byref(engine))

        def forward():
            call("bh_dit_forward", engine, d_latent.data_ptr(), float(timestep),
                 d_caption.data_ptr(), d_mask.data_ptr(), BF16, out.data_ptr(), stream)

        for _ in range(max(0, warmup)):
            forward()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        forward()
        torch.cuda.synchronize()
        secs = time.perf_counter() - t0
        host = bf16_bits_to_f32(out.cpu().view(torch.int16).numpy().view(np.uint16))
        # Device memory in use after the forward: the engine and the weights allocate everything
        # before the first forward and forward allocates nothing, so this is the run's peak.
        free, total = torch.cuda.mem_get_info()
        peak = int(total - free)
    finally:
        if engine.value:
            lib().bh_dit_destroy(engine)
        dw.free()
    np.save(out_path, host.astype("<f4"), allow_pickle=False)
    return {"metrics": {"latency_s": secs, "peak_vram_bytes": peak},
            "effective": {"stage": "dit-step", "dtype": "bf16", "impl": "hip-gfx950",
                          "weights": "checkpoint", "device": "cuda", "plan": plan,
                          "layers": cfg.num_layers},
            "output_stats": output_stats(host)}


def vae_decode(weights: str, latent_path: str, out_path: str, warmup: int = 1) -> dict:
    """Runs the vae-decode stage; returns the BURNISH_JSON record."""
    import torch

    from .vae import SDXL_VAE, config_struct as vae_config_struct, scale_factor

    cfg = vae_config_struct(SDXL_VAE)
    latent = read_npy_f32(latent_path)
    if latent.ndim != 4 or latent.shape[1] != cfg.latent_channels:
        raise BurnisherError(f"decode: expected [1, {cfg.latent_channels}, h, w], got {list(latent.shape)}")
    if latent.shape[0] != 1:   # vae_decoder.cpp:129-134
        raise BurnisherError("vae: batch 1 only -- classifier-free guidance is resolved into a "
                             "single latent before the decoder runs")
    if latent.shape[2] != latent.shape[3]:
        raise BurnisherError("vae-decode (hip-gfx950): square latents only")
    hw = latent.shape[2]
    side = hw * scale_factor(SDXL_VAE)
    assert torch.cuda.is_available(), "the hip-gfx950 vae-decode needs an MI355X"
    call("bh_init", 0)
    d_latent = torch.from_numpy(f32_to_bf16_bits(latent).view(np.int16)).view(torch.bfloat16).cuda()
    image = torch.zeros((1, 3, side, side), dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    with Checkpoint.component(weights, "vae") as ck:
        dw = VaeDeviceWeights(ck, cfg, stream)
    engine = ctypes.c_void_p()
    try:
        call("bh_vae_create", ctypes.byref(cfg), dw.table, hw, ctypes.byref(engine))
        for _ in range(max(0, warmup)):
            call("bh_vae_decode", engine, d_latent.data_ptr(), image.data_ptr(), stream)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        call("bh_vae_decode", engine, d_latent.data_ptr(), image.data_ptr(), stream)
        torch.cuda.synchronize()
        secs = time.perf_counter() - t0
        host = bf16_bits_to_f32(image.cpu().view(torch.int16).numpy().view(np.uint16))
        free, total = torch.cuda.mem_get_info()
        peak = int(total - free)
    finally:
        if engine.value:
            lib().bh_vae_destroy(engine)
        dw.free()
    np.save(out_path, host.astype("<f4"), allow_pickle=False)
    return {"metrics": {"latency_s": secs, "peak_vram_bytes": peak},
            "effective": {"stage": "vae-decode", "dtype": "bf16", "impl": "hip-gfx950",
                          "weights": "checkpoint", "device": "cuda"},
            "output_stats": output_stats(host)}


def t5_encode(weights: str, ids_path: str, out_path: str, warmup: int = 1,
              config: dict | None = None) -> dict:
    """Runs the t5-encode stage on token ids ([batch, seq] integers in a .npy, pad id 0); writes
    the encoder output [batch, seq, d_model] as fp32 and returns the BURNISH_JSON record."""
    import torch

    from .t5 import T5_XXL, config_struct as t5_config_struct

    spec = dict(T5_XXL, **(config or {}))
    cfg = t5_config_struct(spec)
    raw = np.load(ids_path, allow_pickle=False)
    if raw.ndim != 2:
        raise BurnisherError(f"t5-encode: expected ids [batch, seq], got {list(raw.shape)}")
    ids = np.ascontiguousarray(raw, dtype=np.float32)
    if not np.array_equal(ids, raw.astype(np.float64)):
        raise BurnisherError("t5-encode: token ids must be integers exactly representable in fp32")
    batch, seq = ids.shape
    assert torch.cuda.is_available(), "the hip-gfx950 t5-encode needs an MI355X"
    call("bh_init", 0)
    out = torch.zeros((batch, seq, spec["d_model"]), dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    with Checkpoint.component(weights, "text_encoder") as ck:
        dw = T5DeviceWeights(ck, cfg, stream)
    engine = ctypes.c_void_p()
    try:
        call("bh_t5_create", ctypes.byref(cfg), dw.table, batch, seq, ctypes.byref(engine))
        for _ in range(max(0, warmup)):
            call("bh_t5_encode", engine, ids.ctypes.data, out.data_ptr(), stream)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        call("bh_t5_encode", engine, ids.ctypes.data, out.data_ptr(), stream)
        torch.cuda.synchronize()
        secs = time.perf_counter() - t0
        host = bf16_bits_to_f32(out.cpu().view(torch.int16).numpy().view(np.uint16))
        free, total = torch.cuda.mem_get_info()
        peak = int(total - free)
    finally:
        if engine.value:
            lib().bh_t5_destroy(engine)
        dw.free()
    np.save(out_path, host.astype("<f4"), allow_pickle=False)
    return {"metrics": {"latency_s": secs, "peak_vram_bytes": peak},
            "effective": {"stage": "t5-encode", "dtype": "bf16", "impl": "hip-gfx950",
                          "weights": "checkpoint", "device": "cuda"},
            "output_stats": output_stats(host)}


def main(argv=None) -> int:
    p = argparse.ArgumentParser(prog="python -m burnisher_amd.stage")
    sub = p.add_subparsers(dest="stage", required=True)
    d = sub.add_parser("dit-step", help="one dit-step forward from .npy inputs")
    d.add_argument("--weights", required=True, help="checkpoint directory (holds transformer/)")
    d.add_argument("--latent", required=True)
    d.add_argument("--caption", required=True)
    d.add_argument("--mask", required=True)
    d.add_argument("--out", required=True)
    d.add_argument("--timestep", type=float, default=500.0)
    d.add_argument("--layers", type=int, default=None)
    d.add_argument("--warmup", type=int, default=1)
    d.add_argument("--plan", choices=["fused", "opwise"], default="fused")
    v = sub.add_parser("vae-decode", help="decode one latent to pixels")
    v.add_argument("--weights", required=True, help="checkpoint directory (holds vae/)")
    v.add_argument("--latent", required=True)
    v.add_argument("--out", required=True)
    v.add_argument("--warmup", type=int, default=1)
    t = sub.add_parser("t5-encode", help="encode token ids with the T5 encoder")
    t.add_argument("--weights", required=True, help="checkpoint directory (holds text_encoder/)")
    t.add_argument("--ids", required=True, help=".npy of [batch, seq] integer token ids, pad 0")
    t.add_argument("--out", required=True)
    t.add_argument("--warmup", type=int, default=1)
    t.add_argument("--config", default=None, help="JSON object of T5Config fields overriding XXL")
    a = p.parse_args(argv)
    try:
        if a.stage == "t5-encode":
            rec = t5_encode(a.weights, a.ids, a.out, a.warmup, json.loads(a.config) if a.config else None)
        elif a.stage == "vae-decode":
            rec = vae_decode(a.weights, a.latent, a.out, a.warmup)
        else:
            rec = dit_step(a.weights, a.latent, a.caption, a.mask, a.out, a.timestep, a.layers,
                           a.warmup, a.plan)
    except BurnisherError as e:   # burnisher_main.cpp:1035-1038: a sentence and exit 1
        print(f"!! {e}", file=sys.stderr)
        return 1
    print("BURNISH_JSON: " + json.dumps(rec))
    return 0


if __name__ == "__main__":
    sys.exit(main())
