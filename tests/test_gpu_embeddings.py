"""The DiT's two embedding tables as the device path computes them, pinned bit for bit to the stock
oracle and to the reference's own known-answer vectors:

- the timestep embedding (`sinusoidal_timestep_embedding`, /root/reference/src/models/weights.cpp:
  107-121; golden /root/reference/tests/test_models.cpp:186-200), computed on the device in fp64
  by bh_timestep_embedding, the kernel the engine runs every step;
- the 2-D position table (`dit_position_embedding`, pixart_dit.cpp:53-105; golden
  test_models.cpp:141-185) that bh_dit_create builds, read back from the engine itself.

A swapped sin/cos half, a wrong frequency ladder, a transposed mesh or an interpolation scale
other than 2 each changes many stored bf16 values, so each fails here directly rather than
hiding inside the whole-step gate."""
import ctypes

import numpy as np
import pytest

import oracle
from burnisher_amd.workload import PIXART_SIGMA, config_struct, make_workload
from helpers import BF16, F32, from_bf16, golden, to_bf16

pytestmark = pytest.mark.gpu


def device_timestep(t, dim, batch, dtype):
    import torch
    import burnisher_amd as bh
    out = torch.zeros(batch, dim, device="cuda",
                      dtype=torch.float32 if dtype == F32 else torch.bfloat16)
    bh.call("bh_timestep_embedding", float(t), dim, batch, out.data_ptr(), dtype, None)
    torch.cuda.synchronize()
    if dtype == F32:
        return out.cpu().numpy()
    return out.cpu().view(torch.int16).numpy().view(np.uint16)


def stock_timestep(stock, t, dim):
    out = np.zeros(dim, np.float32)
    oracle.call(stock, "stock_timestep_embedding", float(t), dim,
                out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return out


def test_timestep_embedding_golden(hip):
    g = golden("reference_vectors.json")["timestep_embedding"]
    got = device_timestep(g["t"], g["dim"], 1, F32)[0]
    np.testing.assert_allclose(got, np.array(g["values"], np.float32), rtol=0, atol=g["tolerance"])
    # cos first: at t = 0 the first half is 1, the second 0
    z = device_timestep(0.0, 8, 1, F32)[0]
    assert np.array_equal(z, np.array([1, 1, 1, 1, 0, 0, 0, 0], np.float32))


def test_timestep_embedding_equals_oracle_every_training_timestep(hip, stock):
    # Every timestep the 1000-step schedule can hand the model, plus fractional ones: fp32 output
    # equal to the oracle's (glibc fp64 cos/sin/exp/log, then one rounding to float), and the
    # bf16 the engine stores equal to that float rounded once more.
    ts = list(range(0, 1000)) + [0.5, 37.25, 499.999, 1e-3, 1234.5]
    for t in ts:
        want = stock_timestep(stock, t, 256)
        got32 = device_timestep(t, 256, 2, F32)
        assert np.array_equal(got32[0], want) and np.array_equal(got32[1], want), f"t={t}"
        got16 = device_timestep(t, 256, 2, BF16)
        assert np.array_equal(got16[1], to_bf16(want)), f"t={t} (bf16)"


def test_timestep_embedding_refuses_odd_dim(hip):
    import torch
    import burnisher_amd as bh
    out = torch.zeros(2, 8, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(bh.BurnisherError, match="even dimension"):
        bh.call("bh_timestep_embedding", 500.0, 7, 2, out.data_ptr(), BF16, None)
    host = np.zeros(16, np.uint16)
    with pytest.raises(bh.BurnisherError, match="HOST"):
        bh.call("bh_timestep_embedding", 500.0, 8, 2, host.ctypes.data, BF16, None)


def engine_position_table(cfg, latent_hw):
    """The table an engine built for (cfg, latent_hw) holds, as bf16 bits [grid*grid, d]."""
    import torch
    import burnisher_amd as bh
    wl = make_workload(cfg, batch=1, latent_hw=latent_hw, caption_len=8, layers=1)
    top, blocks, *_ = wl.to_device()
    c = config_struct(wl.cfg)
    w, keep = wl.weight_struct(top, blocks)
    h = ctypes.c_void_p()
    bh.call("bh_dit_create", ctypes.byref(c), ctypes.byref(w), 1, latent_hw, 8, bh.DIT_FUSED,
            ctypes.byref(h))
    try:
        grid = latent_hw // cfg["patch_size"]
        d = cfg["num_heads"] * cfg["head_dim"]
        out = torch.zeros(grid * grid, d, device="cuda", dtype=torch.bfloat16)
        bh.call("bh_dit_position_table", h, out.data_ptr(), None)
        torch.cuda.synchronize()
        return out.cpu().view(torch.int16).numpy().view(np.uint16)
    finally:
        bh.lib().bh_dit_destroy(h)


def stock_position_table(stock, d, grid, base):
    out = np.zeros(grid * grid * d, np.float64)
    oracle.call(stock, "stock_position_embedding", out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                d, grid, base, 2.0)
    # the reference stores it through Tensor::set: double -> float -> bf16 (pixart_dit.cpp:102-103)
    return to_bf16(out.astype(np.float32)).reshape(grid * grid, d)


def test_position_table_golden(hip):
    # dim 8, grid 4, base 4 (test_models.cpp:141-185): an engine with hidden 1 x 8, patch 2,
    # sample_size 8 (base 4) over an 8x8 latent (grid 4).
    g = golden("reference_vectors.json")["position_embedding"]
    cfg = dict(num_layers=1, num_heads=1, head_dim=8, patch_size=2, in_channels=4, out_channels=8,
               caption_channels=16, sample_size=8, mlp_ratio=4.0, eps=1e-6)
    got = engine_position_table(cfg, 8)
    want = to_bf16(np.array(g["values"], np.float64).astype(np.float32)).reshape(16, 8)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("latent_hw", [32, 64, 128, 256], ids=["256px", "512px", "1024px", "2048px"])
def test_position_table_equals_oracle(hip, stock, latent_hw):
    cfg = PIXART_SIGMA
    grid = latent_hw // cfg["patch_size"]
    got = engine_position_table(cfg, latent_hw)
    want = stock_position_table(stock, 1152, grid, cfg["sample_size"] // cfg["patch_size"])
    assert np.array_equal(got, want), f"grid {grid}: {np.sum(got != want)} values differ"
    # sanity on the layout: row 0 is position (0, 0): sin 0 = 0 then cos 0 = 1 in each half
    f = from_bf16(got[0])
    assert np.all(f[:288] == 0) and np.all(f[288:576] == 1) and np.all(f[576:864] == 0)
