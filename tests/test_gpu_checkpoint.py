"""Weights from a safetensors checkpoint on the device (bh_dit_weights_load) and the `dit-step`
stage (burnisher_amd/stage.py, the reference CLI's `dit-step`, tools/burnisher_main.cpp:694-747).

Checkpoints are written in F32, as the pinned PixArt-Sigma transformer is published
(configs/checkpoint-layout.json of the reference), with values that are not bf16 already, so the
load's rounding matters. The engine run on loaded weights must equal, byte for byte, the engine
run on weights rounded on the host and uploaded tensor by tensor; the stage's output must meet
the dit-step gate against the stock oracle's dit-step on the same rounded weights and inputs."""
from __future__ import annotations

import contextlib
import ctypes
import io
import json

import numpy as np
import pytest
from safetensors.numpy import save_file

import burnisher_amd as bh
from burnisher_amd import stage
from burnisher_amd.workload import (BLOCK_NAMES, PIXART_SIGMA, TOP_NAMES, DitWorkload, block_shapes,
                                    config_struct, prefix_mask, top_shapes)
from helpers import from_bf16, to_bf16
from test_gpu_dit import SMALL, Engine, check_step, oracle_forward

pytestmark = pytest.mark.gpu


def f32_tensors(cfg: dict, seed: int) -> dict[str, np.ndarray]:
    """Checkpoint name -> float32 N(0, 0.02^2) (not rounded to bf16)."""
    rng = np.random.default_rng(seed)
    out = {}
    for k, s in top_shapes(cfg).items():
        out[TOP_NAMES[k]] = (rng.standard_normal(s) * 0.02).astype(np.float32)
    for i in range(cfg["num_layers"]):
        for k, s in block_shapes(cfg).items():
            # the tables are O(1) in the published checkpoint; the rest like an initialisation
            std = 0.5 if k == "scale_shift_table" else 0.02
            out[f"transformer_blocks.{i}.{BLOCK_NAMES[k]}"] = (rng.standard_normal(s) * std).astype(np.float32)
    return out


def write_component(root, tensors: dict, shards: int = 2):
    """<root>/transformer/model-0000k-of-0000n.safetensors, tensors dealt over the shards."""
    d = root / "transformer"
    d.mkdir(parents=True)
    names = sorted(tensors)
    for k in range(shards):
        part = {n: tensors[n] for n in names[k::shards]}
        save_file(part, str(d / f"model-{k + 1:05d}-of-{shards:05d}.safetensors"),
                  metadata={"format": "pt"})
    return root


def workload_from(cfg, tensors, batch, hw, cap_len, seed) -> DitWorkload:
    """A DitWorkload whose bf16 weights are the checkpoint's, rounded on the host."""
    rng = np.random.default_rng(seed)
    wl = DitWorkload(cfg=cfg, batch=batch, latent_hw=hw, caption_len=cap_len, timestep=500.0)
    wl.top = {k: to_bf16(tensors[n]) for k, n in TOP_NAMES.items()}
    wl.blocks = [{k: to_bf16(tensors[f"transformer_blocks.{i}.{n}"]) for k, n in BLOCK_NAMES.items()}
                 for i in range(cfg["num_layers"])]
    wl.latent = to_bf16(rng.standard_normal((batch, cfg["in_channels"], hw, hw)).astype(np.float32))
    wl.caption = to_bf16(rng.standard_normal((batch, cap_len, cfg["caption_channels"])).astype(np.float32))
    wl.mask = prefix_mask(batch, cap_len)
    return wl


@pytest.mark.parametrize("flat_patch", [False, True], ids=["conv_layout", "flat_patch"])
def test_engine_on_loaded_weights_equals_host_rounded_upload(hip, tmp_path, flat_patch):
    cfg = dict(SMALL)
    tensors = f32_tensors(cfg, 11)
    if flat_patch:   # [out, in*kh*kw] holds the same bytes as [out, in, kh, kw]
        w = tensors["pos_embed.proj.weight"]
        tensors["pos_embed.proj.weight"] = w.reshape(w.shape[0], -1)
    write_component(tmp_path, tensors)
    wl = workload_from(cfg, tensors, batch=2, hw=8, cap_len=5, seed=12)
    ref_engine = Engine(wl, bh.DIT_FUSED)
    with bh.Checkpoint.component(tmp_path, "transformer") as ck:
        dw = bh.DitDeviceWeights(ck, config_struct(cfg))
    handle = ctypes.c_void_p()
    try:
        want = ref_engine.forward()
        assert dw.bytes >= 2 * sum(a.size for a in tensors.values())
        bh.call("bh_dit_create", ctypes.byref(ref_engine.cfg), ctypes.byref(dw.weights), wl.batch,
                wl.latent_hw, wl.caption_len, bh.DIT_FUSED, ctypes.byref(handle))
        # swap the engines' weights: same inputs and outputs, only the weight source differs
        ref_engine.close()
        ref_engine.handle = handle
        handle = ctypes.c_void_p()
        got = ref_engine.forward()
        assert np.array_equal(got, want), "engine on loaded weights differs from the host upload"
        check_step(got, oracle_forward(wl), "loaded weights vs oracle")
    finally:
        ref_engine.close()
        dw.free()


def test_loading_fewer_layers_than_the_checkpoint_holds(hip, tmp_path):
    cfg = dict(SMALL, num_layers=3)
    tensors = f32_tensors(cfg, 21)
    write_component(tmp_path, tensors, shards=1)
    one = dict(cfg, num_layers=1)
    wl = workload_from(one, tensors, batch=2, hw=8, cap_len=5, seed=22)
    with bh.Checkpoint.component(tmp_path, "transformer") as ck:
        dw = bh.DitDeviceWeights(ck, config_struct(one))
    e = Engine(wl, bh.DIT_FUSED)
    try:
        want = e.forward()
        e.close()
        bh.call("bh_dit_create", ctypes.byref(e.cfg), ctypes.byref(dw.weights), wl.batch,
                wl.latent_hw, wl.caption_len, bh.DIT_FUSED, ctypes.byref(e.handle))
        assert np.array_equal(e.forward(), want)
    finally:
        e.close()
        dw.free()


def test_dit_step_stage_matches_oracle(hip, tmp_path):
    # PixArt-Sigma widths (the stage's configuration), one block, a 256px latent, caption 120
    cfg = dict(PIXART_SIGMA, num_layers=1)
    tensors = f32_tensors(cfg, 31)
    write_component(tmp_path / "ckpt", tensors)
    wl = workload_from(cfg, tensors, batch=2, hw=32, cap_len=120, seed=32)
    paths = {k: str(tmp_path / f"{k}.npy") for k in ("latent", "caption", "mask", "out")}
    np.save(paths["latent"], from_bf16(wl.latent))
    np.save(paths["caption"], from_bf16(wl.caption))
    np.save(paths["mask"], wl.mask)
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        rc = stage.main(["dit-step", "--weights", str(tmp_path / "ckpt"), "--latent", paths["latent"],
                         "--caption", paths["caption"], "--mask", paths["mask"], "--out",
                         paths["out"], "--layers", "1"])
    assert rc == 0
    line, = [l for l in buf.getvalue().splitlines() if l.startswith("BURNISH_JSON: ")]
    rec = json.loads(line[len("BURNISH_JSON: "):])
    out = np.load(paths["out"])
    assert out.dtype == np.float32 and out.shape == (2, 8, 32, 32)
    assert rec["effective"]["stage"] == "dit-step" and rec["effective"]["impl"] == "hip-gfx950"
    assert rec["metrics"]["latency_s"] > 0
    assert rec["output_stats"] == stage.output_stats(out)
    check_step(to_bf16(out), oracle_forward(wl), "dit-step stage vs oracle")


def test_stage_refuses_what_the_reference_refuses(hip, tmp_path):
    bad = tmp_path / "f64.npy"
    np.save(bad, np.zeros((1, 4, 8, 8)))
    ok = tmp_path / "ok.npy"
    np.save(ok, np.zeros((1, 4, 8, 8), np.float32))
    with pytest.raises(bh.BurnisherError, match="little-endian fp32"):
        stage.read_npy_f32(str(bad))
    cap = tmp_path / "cap.npy"
    np.save(cap, np.zeros((1, 3, 4096), np.float32))
    mask = tmp_path / "mask.npy"
    np.save(mask, np.zeros((1, 4), np.float32))
    with pytest.raises(bh.BurnisherError, match="caption_mask has 4 elements"):
        stage.dit_step(str(tmp_path), str(ok), str(cap), str(mask), str(tmp_path / "o.npy"))
