"""The VAE decoder on the device against the stock oracle (oracle/stock.cpp, itself pinned
bit-for-bit to the reference's own code): the op-level entry points (bh_conv2d, GroupNorm through
bh_norm, bh_upsample, bh_transpose), the head_dim-512 attention, and the whole decoder engine
(bh_vae_create / bh_vae_decode) at the SDXL VAE's widths on small latents.

Gates (configs/tolerance.json): the implicit-GEMM convolution and the 1x1 GEMM take the GEMM
bound (fp32 summation order), the direct convolution, upsample and transpose are bit-identical,
GroupNorm takes the norm bound, the attention the attention bound, the decoder the vae_decode
bound."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from burnisher_amd.vae import SDXL_VAE, config_struct, make_vae_workload
from helpers import BF16, F32, TOLERANCE, addr, assert_within, from_bf16, randn_bf16, stats

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(11)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().view(torch.int16).numpy().view(np.uint16).copy()


def empty(shape):
    import torch
    return torch.zeros(shape, dtype=torch.bfloat16, device="cuda")


def call(name, *args):
    import burnisher_amd as bh
    bh.call(name, *args)


def st(name, *args):
    oracle.call(oracle.stock(), name, *args)


@pytest.mark.parametrize("shape", [(1, 128, 16, 16, 256, 3, 1), (1, 256, 8, 12, 128, 3, 1),
                                   (2, 64, 10, 10, 64, 3, 1), (1, 256, 8, 8, 128, 1, 0),
                                   (1, 4, 16, 16, 512, 3, 1), (1, 128, 16, 16, 3, 3, 1)],
                         ids=lambda s: "x".join(map(str, s)))
def test_conv2d_matches_oracle(hip, shape):
    B, ci, H, W, co, k, pad = shape
    x = randn_bf16(RNG, (B, ci, H, W))
    w = randn_bf16(RNG, (co, ci, k, k), float(1 / np.sqrt(ci * k * k)))
    b = randn_bf16(RNG, (co,), 0.1)
    want = np.zeros((B, co, H, W), np.uint16)
    st("stock_conv2d", addr(x), addr(w), addr(b), addr(want), B, ci, H, W, co, k, pad, BF16, 0)
    out = empty((B, co, H, W))
    dx, dw, db = dev(x), dev(w), dev(b)
    call("bh_conv2d", dx.data_ptr(), dw.data_ptr(), db.data_ptr(), out.data_ptr(), B, ci, H, W, co, k,
         pad, BF16, None)
    got = host(out)
    direct = not ((k == 3 and ci % 64 == 0 and co % 8 == 0) or k == 1)
    if direct:   # the reference's summation order: bit-identical
        assert np.array_equal(got, want), stats(from_bf16(got), from_bf16(want))
    else:
        assert_within(from_bf16(got), from_bf16(want), "gemm", f"conv {shape}")
    again = empty((B, co, H, W))
    call("bh_conv2d", dx.data_ptr(), dw.data_ptr(), db.data_ptr(), again.data_ptr(), B, ci, H, W, co,
         k, pad, BF16, None)
    assert np.array_equal(host(again), got), "not byte-identical across two calls"


@pytest.mark.parametrize("case", [(1, 128, 256, 32, True), (2, 512, 64, 32, True), (1, 64, 100, 32, False),
                                  (1, 256, 1024, 32, True)])
def test_group_norm_matches_oracle(hip, case):
    rows, C, S, G, affine = case
    x = randn_bf16(RNG, (rows, C * S), 2.0)
    w = randn_bf16(RNG, (C,), 0.3) if affine else None
    b = randn_bf16(RNG, (C,), 0.3) if affine else None
    want = np.zeros_like(x)
    st("stock_group_norm", addr(x), addr(w), addr(b), addr(want), rows, C * S, 1e-6, G, C, BF16, 0)
    out = empty((rows, C * S))
    dx = dev(x)   # device copies stay referenced until the read-back below
    dw = dev(w) if affine else None
    db = dev(b) if affine else None
    call("bh_norm", dx.data_ptr(), dw.data_ptr() if affine else None, db.data_ptr() if affine else None,
         out.data_ptr(), rows, C * S, 1e-6, 0, G, C, BF16, None)
    assert_within(from_bf16(host(out)), from_bf16(want), "norm", f"groupnorm {case}")


def test_upsample_and_transpose_match_oracle(hip):
    x = randn_bf16(RNG, (2, 5, 6, 7))
    want = np.zeros((2, 5, 12, 14), np.uint16)
    st("stock_upsample", addr(x), addr(want), 2, 5, 6, 7, 2, BF16)
    out = empty((2, 5, 12, 14))
    dx = dev(x)
    call("bh_upsample", dx.data_ptr(), out.data_ptr(), 2, 5, 6, 7, 2, BF16, None)
    assert np.array_equal(host(out), want)
    t = randn_bf16(RNG, (3, 37, 70))
    for to_cf, shape_in, shape_out in ((0, (3, 37, 70), (3, 70, 37)), (1, (3, 70, 37), (3, 37, 70))):
        src = t if to_cf == 0 else t.transpose(0, 2, 1).copy()
        want = np.zeros(shape_out, np.uint16)
        st("stock_transpose", addr(src), addr(want), 3, 37, 70, to_cf, BF16)
        out = empty(shape_out)
        dsrc = dev(src)
        call("bh_transpose", dsrc.data_ptr(), out.data_ptr(), 3, 37, 70, to_cf, BF16, None)
        assert np.array_equal(host(out), want)


@pytest.mark.parametrize("S", [64, 100, 333])
def test_attention_head_dim_512_matches_oracle(hip, S):
    q, k, v = (randn_bf16(RNG, (1, S, 1, 512)) for _ in range(3))
    want = np.zeros_like(q)
    st("stock_attention", addr(q), addr(k), addr(v), addr(want), 1, 1, S, S, 512, 0.0, None, None, F32,
       BF16, 0, 0)
    out = empty((1, S, 1, 512))
    dq, dk, dv = dev(q), dev(k), dev(v)   # referenced until the read-back
    call("bh_attention", dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), 1, 1,
         S, S, 512, 0.0, None, None, F32, BF16, None)
    assert_within(from_bf16(host(out)), from_bf16(want), "attention", f"head_dim 512 S={S}")


def decode(wl):
    import burnisher_amd as bh
    tensors, latent = wl.to_device()
    cfg = config_struct(wl.cfg)
    w, keep = wl.table(tensors)
    h = ctypes.c_void_p()
    bh.call("bh_vae_create", ctypes.byref(cfg), ctypes.byref(w), wl.latent_hw, ctypes.byref(h))
    try:
        out = empty((1, 3, wl.image_hw, wl.image_hw))
        # a host operand is refused before any launch
        host_latent = np.zeros(latent.numel(), np.uint16)
        assert bh.lib().bh_vae_decode(h, host_latent.ctypes.data, out.data_ptr(), None) != 0
        assert b"HOST" in bh.lib().bh_last_error()
        bh.call("bh_vae_decode", h, latent.data_ptr(), out.data_ptr(), None)
        first = host(out)
        bh.call("bh_vae_decode", h, latent.data_ptr(), out.data_ptr(), None)
        assert np.array_equal(host(out), first), "decode is not byte-identical across two calls"
        return first
    finally:
        bh.lib().bh_vae_destroy(h)


def oracle_decode(wl):
    cfg = config_struct(wl.cfg)
    w, keep = wl.table()
    out = np.zeros((1, 3, wl.image_hw, wl.image_hw), np.uint16)
    st("stock_vae_forward", ctypes.byref(cfg), ctypes.byref(w), addr(wl.latent), wl.latent_hw, addr(out),
       0, -1)
    return out


def check_decode(got, want, where):
    tol = TOLERANCE["vae_decode"]
    s = stats(from_bf16(got), from_bf16(want))
    print(f"vae-decode parity {where}: {s}")
    assert np.all(np.isfinite(from_bf16(got))), where
    assert s["rel_l2"] <= tol["rel_l2"] and s["cosine"] >= tol["cosine"], f"{where}: {s} vs {tol}"


@pytest.mark.parametrize("cfg,latent_hw", [(SDXL_VAE, 8),
                                           (dict(SDXL_VAE, block_out_channels=(64, 128, 128, 128),
                                                 layers_per_block=1), 6)],
                         ids=["sdxl_widths_8", "narrow_6"])
def test_vae_decoder_matches_oracle(hip, cfg, latent_hw):
    wl = make_vae_workload(cfg, latent_hw=latent_hw, seed=5)
    check_decode(decode(wl), oracle_decode(wl), f"{cfg['block_out_channels']} latent {latent_hw}")


def test_vae_create_refuses_bad_configurations(hip):
    import burnisher_amd as bh
    wl = make_vae_workload(dict(SDXL_VAE, block_out_channels=(12, 24, 24, 24), norm_num_groups=4,
                                layers_per_block=0), latent_hw=2)
    tensors, _ = wl.to_device()
    w, keep = wl.table(tensors)
    h = ctypes.c_void_p()
    cfg = config_struct(wl.cfg)
    assert bh.lib().bh_vae_create(ctypes.byref(cfg), ctypes.byref(w), 2, ctypes.byref(h)) != 0
    assert b"groups" in bh.lib().bh_last_error() or b"64" in bh.lib().bh_last_error()
    wl2 = make_vae_workload(SDXL_VAE, latent_hw=2)
    tensors2, _ = wl2.to_device()
    del tensors2["decoder.conv_out.bias"]
    w2, keep2 = wl2.table(tensors2)
    assert bh.lib().bh_vae_create(ctypes.byref(config_struct(SDXL_VAE)), ctypes.byref(w2), 2,
                                  ctypes.byref(h)) != 0
    assert b"missing" in bh.lib().bh_last_error()


def test_vae_weights_from_a_checkpoint_and_the_decode_stage(hip, tmp_path):
    """The `vae/` component of an F32 checkpoint (as the pinned one is published): loaded weights
    give the same bytes as weights rounded on the host, and the stage meets the decoder gate."""
    import contextlib
    import io
    import json

    import burnisher_amd as bh
    from burnisher_amd import stage
    from burnisher_amd.vae import vae_tensors
    from safetensors.numpy import save_file

    rng = np.random.default_rng(21)
    f32 = {}
    for name, shape in vae_tensors(SDXL_VAE).items():
        std = 0.1 if "norm" in name else (0.02 if name.endswith(".bias") else 1 / np.sqrt(np.prod(shape[1:])))
        v = (rng.standard_normal(shape) * std).astype(np.float32)
        if "norm" in name and name.endswith(".weight"):
            v += 1.0
        f32[name] = v
    d = tmp_path / "ckpt" / "vae"
    d.mkdir(parents=True)
    save_file(f32, str(d / "diffusion_pytorch_model.safetensors"))
    wl = make_vae_workload(SDXL_VAE, latent_hw=4, seed=22)
    from helpers import to_bf16
    wl.weights = {n: to_bf16(a) for n, a in f32.items()}
    want = oracle_decode(wl)
    # the stage, end to end
    lat = tmp_path / "latent.npy"
    np.save(lat, from_bf16(wl.latent))
    out = tmp_path / "image.npy"
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        assert stage.main(["vae-decode", "--weights", str(tmp_path / "ckpt"), "--latent", str(lat),
                           "--out", str(out)]) == 0
    rec = json.loads(buf.getvalue().split("BURNISH_JSON: ")[1])
    img = np.load(out)
    assert img.shape == (1, 3, 32, 32) and rec["effective"]["stage"] == "vae-decode"
    assert rec["output_stats"] == stage.output_stats(img)
    check_decode(to_bf16(img), want, "vae-decode stage")
    # loaded weights == host-rounded upload, byte for byte
    assert np.array_equal(to_bf16(img), decode(wl))
