"""The oracle's DiT graph (stock_dit_forward) pinned at a small config: bit-for-bit against the
reference's own PixArtDiT::forward on stock (oracle/_ref), plus the reference's graph invariants
(tests/test_models.cpp:274-348) and thread-count invariance."""
import numpy as np
import pytest

import oracle
from burnisher_amd.workload import config_struct, make_workload
from helpers import BF16, F32, addr, from_bf16

SMALL = dict(num_layers=2, num_heads=4, head_dim=8, patch_size=2, in_channels=4, out_channels=8,
             caption_channels=32, sample_size=8, mlp_ratio=4.0, eps=1e-6)


def run(lib, fn, wl, *, threads=2, timestep=None, caption=None, mask=None, layers=-1):
    cfg = config_struct(wl.cfg)
    w, keep = wl.weight_struct(wl.top, wl.blocks)
    cap = wl.caption if caption is None else caption
    m = wl.mask if mask is None else mask
    out = np.zeros((wl.batch, wl.cfg["out_channels"], wl.latent_hw, wl.latent_hw), np.uint16)
    t = wl.timestep if timestep is None else timestep
    import ctypes
    args = [ctypes.byref(cfg), ctypes.byref(w), wl.batch, wl.latent_hw, wl.caption_len,
            addr(wl.latent), t, addr(cap), addr(m), F32, addr(out)]
    if fn == "stock_dit_forward":
        oracle.call(lib, fn, *args, threads, layers)
    else:
        oracle.call(lib, fn, *args, layers)
    return out


@pytest.fixture(scope="module")
def small():
    return make_workload(SMALL, batch=2, latent_hw=8, caption_len=5)


def test_dit_matches_reference_bit_for_bit(stock, ref, small):
    a = run(stock, "stock_dit_forward", small)
    b = run(ref, "ref_dit_forward", small)
    assert np.array_equal(a, b)
    assert np.all(np.isfinite(from_bf16(a)))


def test_dit_matches_reference_at_dit_head_dim(stock, ref):
    # head_dim 72 and a caption longer than the attention block, one block deep
    cfg = dict(SMALL, num_heads=2, head_dim=72, num_layers=1, caption_channels=64)
    wl = make_workload(cfg, batch=2, latent_hw=8, caption_len=70)
    assert np.array_equal(run(stock, "stock_dit_forward", wl), run(ref, "ref_dit_forward", wl))


def test_dit_invariants(stock, small):
    a = run(stock, "stock_dit_forward", small)
    assert np.array_equal(a, run(stock, "stock_dit_forward", small))       # reproduces itself
    assert np.array_equal(a, run(stock, "stock_dit_forward", small, threads=1))
    assert np.array_equal(a, run(stock, "stock_dit_forward", small, threads=7))
    fa = from_bf16(a)
    # the timestep reaches the output
    assert np.max(np.abs(fa - from_bf16(run(stock, "stock_dit_forward", small, timestep=100.0)))) > 1e-6
    # so does the caption
    cap2 = small.caption.copy()
    cap2.view(np.uint16)[:] = np.roll(cap2.ravel(), 7).reshape(cap2.shape)
    assert np.max(np.abs(fa - from_bf16(run(stock, "stock_dit_forward", small, caption=cap2)))) > 1e-6
    # masked caption positions do not reach the output
    cap3 = small.caption.copy()
    for b in range(small.batch):
        keep = int(small.mask[b].sum())
        cap3[b, keep:, :] = 0x42C6   # 99.0 in bf16
    assert np.array_equal(a, run(stock, "stock_dit_forward", small, caption=cap3))
    # and the mask is not ignored
    ones = np.ones_like(small.mask)
    assert np.max(np.abs(fa - from_bf16(run(stock, "stock_dit_forward", small, mask=ones)))) > 1e-6


def test_dit_layer_truncation(stock, small):
    one = run(stock, "stock_dit_forward", small, layers=1)
    two = run(stock, "stock_dit_forward", small, layers=2)
    assert not np.array_equal(one, two)
