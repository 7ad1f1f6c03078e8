"""The stock oracle's VAE decoder (oracle/stock.cpp: conv2d, GroupNorm, upsample, transpose and
the vae_decoder.cpp graph), pinned three ways:
  - bit-for-bit against the reference's own stock code compiled into oracle/_ref (ops_cpu.cpp,
    vae_decoder.cpp, weights.cpp's declaration of the decoder's shapes);
  - closed forms a plausible mistake fails: an identity convolution, a one-hot tap that shifts
    the image (a transposed kernel or a wrong padding side moves it the wrong way), GroupNorm
    moments per group, nearest-neighbour replication;
  - float64 numpy brute force on tiny shapes.
The weight table's names and shapes are pinned to the published checkpoint layout
(tests/golden/vae_decoder_layout.json, from the reference's configs/checkpoint-layout.json)."""
from __future__ import annotations

import ctypes
import json

import numpy as np
import pytest

import oracle
from burnisher_amd.vae import SDXL_VAE, config_struct, make_vae_workload, vae_tensors
from helpers import BF16, F32, GOLDEN, addr, from_bf16, randn_bf16, to_bf16

RNG = np.random.default_rng(7)


def st(name, *args):
    oracle.call(oracle.stock(), name, *args)


def conv_np(x, w, b, pad):
    """float64 NCHW conv, stride 1."""
    B, ci, H, W = x.shape
    co, _, k, _ = w.shape
    xp = np.pad(x, ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    Ho, Wo = H + 2 * pad - k + 1, W + 2 * pad - k + 1
    out = np.zeros((B, co, Ho, Wo))
    for ky in range(k):
        for kx in range(k):
            patch = xp[:, :, ky:ky + Ho, kx:kx + Wo]
            out += np.einsum("bchw,oc->bohw", patch, w[:, :, ky, kx])
    return out + (0 if b is None else b[None, :, None, None])


def test_decoder_weight_table_is_the_published_layout():
    g = json.loads((GOLDEN / "vae_decoder_layout.json").read_text())["tensors"]
    mine = vae_tensors(SDXL_VAE)
    assert list(mine) != [] and set(mine) == set(g)
    assert all(tuple(g[k]["shape"]) == v for k, v in mine.items())


@pytest.mark.parametrize("dt", [BF16, F32])
@pytest.mark.parametrize("shape", [(1, 3, 7, 9, 5, 3, 1), (2, 8, 6, 6, 4, 1, 0), (1, 4, 5, 5, 16, 3, 1),
                                   (1, 16, 4, 4, 3, 3, 1)])
def test_conv2d_matches_reference_bit_for_bit(ref, dt, shape):
    B, ci, H, W, co, k, pad = shape
    x = RNG.standard_normal((B, ci, H, W)).astype(np.float32)
    w = (RNG.standard_normal((co, ci, k, k)) * 0.3).astype(np.float32)
    b = (RNG.standard_normal(co) * 0.1).astype(np.float32)
    if dt == BF16:
        x, w, b = to_bf16(x), to_bf16(w), to_bf16(b)
    Ho, Wo = H + 2 * pad - k + 1, W + 2 * pad - k + 1
    got = np.zeros((B, co, Ho, Wo), x.dtype)
    want = np.zeros_like(got)
    st("stock_conv2d", addr(x), addr(w), addr(b), addr(got), B, ci, H, W, co, k, pad, dt, 3)
    oracle.call(ref, "ref_conv2d", addr(x), addr(w), addr(b), addr(want), B, ci, H, W, co, k, pad, dt)
    assert np.array_equal(got, want)
    xf, wf, bf = (from_bf16(a) if dt == BF16 else a for a in (x, w, b))
    g = from_bf16(got) if dt == BF16 else got
    np.testing.assert_allclose(g, conv_np(xf.astype(np.float64), wf.astype(np.float64), bf, pad),
                               rtol=1e-2 if dt == BF16 else 1e-5, atol=1e-2 if dt == BF16 else 1e-5)


def test_conv2d_closed_forms():
    x = randn_bf16(RNG, (1, 5, 6, 7))
    ident = np.zeros((5, 5, 3, 3), np.float32)
    for c in range(5):
        ident[c, c, 1, 1] = 1.0
    out = np.zeros_like(x)
    st("stock_conv2d", addr(x), addr(to_bf16(ident)), None, addr(out), 1, 5, 6, 7, 5, 3, 1, BF16, 2)
    assert np.array_equal(out, x)                                   # identity
    shift = np.zeros((1, 1, 3, 3), np.float32)
    shift[0, 0, 0, 2] = 1.0                                         # tap (ky=0, kx=2): in[y-1, x+1]
    one = x[:, :1]
    out1 = np.zeros_like(one)
    st("stock_conv2d", addr(np.ascontiguousarray(one)), addr(to_bf16(shift)), None, addr(out1), 1, 1, 6,
       7, 1, 3, 1, BF16, 1)
    want = np.zeros_like(one)
    want[0, 0, 1:, :-1] = one[0, 0, :-1, 1:]
    assert np.array_equal(out1, want)


@pytest.mark.parametrize("dt", [BF16, F32])
@pytest.mark.parametrize("shape", [(1, 32, 16, 32), (2, 64, 9, 32), (1, 16, 25, 8)])
def test_group_norm_matches_reference_and_moments(ref, dt, shape):
    B, C, S, G = shape
    x = (RNG.standard_normal((B, C * S)) * 3 + 1).astype(np.float32)
    w = (1 + RNG.standard_normal(C) * 0.1).astype(np.float32)
    b = (RNG.standard_normal(C) * 0.1).astype(np.float32)
    if dt == BF16:
        x, w, b = to_bf16(x), to_bf16(w), to_bf16(b)
    got, want = np.zeros_like(x), np.zeros_like(x)
    st("stock_group_norm", addr(x), addr(w), addr(b), addr(got), B, C * S, 1e-6, G, C, dt, 3)
    oracle.call(ref, "ref_group_norm", addr(x), addr(w), addr(b), addr(want), B, C * S, 1e-6, G, C, dt)
    assert np.array_equal(got, want)
    # without the affine, every group has mean 0 and variance 1 (float64 brute force)
    plain = np.zeros_like(x)
    st("stock_group_norm", addr(x), None, None, addr(plain), B, C * S, 1e-6, G, C, dt, 2)
    pf = (from_bf16(plain) if dt == BF16 else plain).reshape(B, G, -1).astype(np.float64)
    xf = (from_bf16(x) if dt == BF16 else x).reshape(B, G, -1).astype(np.float64)
    expect = (xf - xf.mean(-1, keepdims=True)) / np.sqrt(xf.var(-1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(pf, expect, atol=2e-2 if dt == BF16 else 1e-5)


def test_group_norm_refuses_what_the_reference_refuses():
    x = np.zeros(30, np.uint16)
    with pytest.raises(oracle.OracleError, match="not divisible"):
        st("stock_group_norm", addr(x), None, None, addr(x), 1, 30, 1e-6, 4, 6, BF16, 1)


def test_upsample_and_transpose(ref):
    x = randn_bf16(RNG, (2, 3, 4, 5))
    up, upr = np.zeros((2, 3, 8, 10), np.uint16), np.zeros((2, 3, 8, 10), np.uint16)
    st("stock_upsample", addr(x), addr(up), 2, 3, 4, 5, 2, BF16)
    oracle.call(ref, "ref_upsample", addr(x), addr(upr), 2, 3, 4, 5, 2, BF16)
    assert np.array_equal(up, upr)
    assert np.array_equal(up, x.repeat(2, axis=2).repeat(2, axis=3))
    t = randn_bf16(RNG, (2, 6, 35))
    sf, sfr = np.zeros((2, 35, 6), np.uint16), np.zeros((2, 35, 6), np.uint16)
    st("stock_transpose", addr(t), addr(sf), 2, 6, 35, 0, BF16)
    oracle.call(ref, "ref_transpose", addr(t), addr(sfr), 2, 6, 35, 0, BF16)
    assert np.array_equal(sf, sfr) and np.array_equal(sf, t.transpose(0, 2, 1))
    back = np.zeros_like(t)
    st("stock_transpose", addr(sf), addr(back), 2, 6, 35, 1, BF16)
    assert np.array_equal(back, t)


SMALL_VAE = dict(block_out_channels=(16, 32, 32, 32), layers_per_block=1, latent_channels=4,
                 norm_num_groups=8, eps=1e-6)


def vae_out(lib, fn, wl, *extra):
    cfg = config_struct(wl.cfg)
    w, keep = wl.table()
    out = np.zeros((1, 3, wl.image_hw, wl.image_hw), np.uint16)
    oracle.call(lib, fn, ctypes.byref(cfg), ctypes.byref(w), addr(wl.latent), wl.latent_hw, addr(out),
                *extra)
    return out


def test_vae_decoder_matches_reference_bit_for_bit(ref):
    wl = make_vae_workload(SMALL_VAE, latent_hw=4, seed=3)
    got = vae_out(oracle.stock(), "stock_vae_forward", wl, 4, -1)
    want = vae_out(ref, "ref_vae_forward", wl)
    assert np.array_equal(got, want)
    f = from_bf16(got)
    assert np.all(np.isfinite(f)) and f.std() > 1e-3
    # the result does not depend on the thread count
    assert np.array_equal(got, vae_out(oracle.stock(), "stock_vae_forward", wl, 1, -1))
