"""The T5 encoder on the device against the stock oracle (oracle/stock.cpp, itself pinned
bit-for-bit to the reference's own code): the embedding gather (bit-identical), attention with
the relative-position bias and key mask (attention gate), and the whole encoder engine
(bh_t5_create / bh_t5_encode) on small configurations and at T5-XXL widths (t5_encode gate)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import burnisher_amd as bh
import oracle
from burnisher_amd.t5 import T5_XXL, config_struct, make_t5_workload
from helpers import BF16, F32, TOLERANCE, addr, assert_within, from_bf16, randn_bf16, stats

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(13)
SMALL = dict(num_layers=2, d_model=64, d_ff=96, d_kv=16, num_heads=4, vocab_size=100, gated=1,
             num_buckets=32, eps=1e-6)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().view(torch.int16).numpy().view(np.uint16).copy()


@pytest.mark.parametrize("cols", [64, 37])
def test_gather_bit_identical(hip, cols):
    import torch
    table = randn_bf16(RNG, (50, cols))
    ids = np.array([3, 0, 49, 7.9, 3, -0.5, 50, 1e9, np.nan], np.float32)
    dt, di = dev(table), torch.from_numpy(ids).cuda()
    out = torch.zeros((len(ids), cols), dtype=torch.bfloat16, device="cuda")
    bh.call("bh_gather", dt.data_ptr(), di.data_ptr(), out.data_ptr(), len(ids), cols, 50, BF16, None)
    got = host(out)
    for r, f in enumerate(ids):
        if np.isfinite(f) and -1 < f < 50:
            assert np.array_equal(got[r], table[int(f)]), r
        else:
            assert np.all(np.isnan(from_bf16(got[r]))), f"row {r} (id {f}) should be NaN"
    t32 = RNG.standard_normal((50, cols)).astype(np.float32)
    o32 = torch.zeros((4, cols), dtype=torch.float32, device="cuda")
    ids32 = torch.tensor([1, 2, 3, 49], dtype=torch.float32, device="cuda")
    d32 = torch.from_numpy(t32).cuda()
    bh.call("bh_gather", d32.data_ptr(), ids32.data_ptr(), o32.data_ptr(), 4, cols, 50, F32, None)
    assert np.array_equal(o32.cpu().numpy(), t32[[1, 2, 3, 49]])


@pytest.mark.parametrize("shape", [(2, 4, 37, 64), (2, 8, 300, 64), (1, 3, 70, 16)],
                         ids=lambda s: "x".join(map(str, s)))
def test_attention_with_relative_bias_and_mask(hip, shape):
    import torch
    B, H, S, D = shape
    q, k, v = (randn_bf16(RNG, (B, S, H, D)) for _ in range(3))
    bias = randn_bf16(RNG, (H, S, S), 2.0)
    mask = np.ones((B, S), np.uint16) * 0x3F80
    mask[0, S // 3:] = 0
    want = np.zeros_like(q)
    oracle.call(oracle.stock(), "stock_attention", addr(q), addr(k), addr(v), addr(want), B, H, S, S, D,
                1.0, addr(bias), addr(mask), BF16, BF16, 0, 0)
    out = torch.zeros((B, S, H, D), dtype=torch.bfloat16, device="cuda")
    dq, dk, dv, db, dm = dev(q), dev(k), dev(v), dev(bias), dev(mask)
    bh.call("bh_attention", dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), B, H, S, S, D,
            1.0, db.data_ptr(), dm.data_ptr(), BF16, BF16, None)
    assert_within(from_bf16(host(out)), from_bf16(want), "attention", f"biased {shape}")


def stock_encode(wl):
    cfg = config_struct(wl.cfg)
    w, keep = wl.table()
    out = np.zeros((wl.batch, wl.seq, wl.cfg["d_model"]), np.uint16)
    oracle.call(oracle.stock(), "stock_t5_forward", ctypes.byref(cfg), ctypes.byref(w),
                wl.ids.ctypes.data, wl.batch, wl.seq, out.ctypes.data, 0)
    return out


def device_encode(wl):
    import torch
    tensors = wl.to_device()
    cfg = config_struct(wl.cfg)
    w, keep = wl.table(tensors)
    h = ctypes.c_void_p()
    bh.call("bh_t5_create", ctypes.byref(cfg), ctypes.byref(w), wl.batch, wl.seq, ctypes.byref(h))
    try:
        out = torch.zeros((wl.batch, wl.seq, wl.cfg["d_model"]), dtype=torch.bfloat16, device="cuda")
        host_out = np.zeros((wl.batch, wl.seq, wl.cfg["d_model"]), np.uint16)
        assert bh.lib().bh_t5_encode(h, wl.ids.ctypes.data, host_out.ctypes.data, None) != 0
        assert b"HOST" in bh.lib().bh_last_error()
        bh.call("bh_t5_encode", h, wl.ids.ctypes.data, out.data_ptr(), None)
        first = host(out)
        bh.call("bh_t5_encode", h, wl.ids.ctypes.data, out.data_ptr(), None)
        assert np.array_equal(host(out), first), "encode is not byte-identical across two calls"
        bad = wl.ids.copy()
        bad[0, 0] = wl.cfg["vocab_size"]
        assert bh.lib().bh_t5_encode(h, bad.ctypes.data, out.data_ptr(), None) != 0
        assert b"vocabulary" in bh.lib().bh_last_error()
        assert np.array_equal(host(out), first), "a refused call touched the output"
        return first
    finally:
        bh.lib().bh_t5_destroy(h)


def check(got, want, where):
    tol = TOLERANCE["t5_encode"]
    s = stats(from_bf16(got), from_bf16(want))
    print(f"t5-encode parity {where}: {s}")
    assert np.all(np.isfinite(from_bf16(got))), where
    assert s["rel_l2"] <= tol["rel_l2"] and s["cosine"] >= tol["cosine"] and s["max_abs"] <= tol["max_abs"], \
        f"{where}: {s} vs {tol}"


@pytest.mark.parametrize("cfg,batch,seq,lengths", [
    (SMALL, 2, 9, [3, 9]),
    (dict(SMALL, gated=0, num_layers=1), 2, 9, [9, 5]),
    (dict(SMALL, d_model=256, d_ff=640, d_kv=64, num_heads=4, vocab_size=1000, num_layers=3), 2, 77, [1, 40]),
    (dict(T5_XXL, num_layers=1), 2, 48, [1, 30]),
], ids=["small", "plain_gelu", "mid", "xxl_widths_1layer"])
def test_encoder_matches_oracle(hip, cfg, batch, seq, lengths):
    wl = make_t5_workload(cfg, batch=batch, seq=seq, lengths=lengths, seed=9)
    check(device_encode(wl), stock_encode(wl), f"{cfg['d_model']}x{cfg['num_layers']} B{batch} S{seq}")


def test_t5_weights_from_a_sharded_checkpoint_and_the_encode_stage(hip, tmp_path):
    """The `text_encoder/` component split over two F32 shards with an index (as T5 XXL is
    published): loaded weights give the same bytes as weights rounded on the host, and the
    t5-encode stage meets the encoder gate."""
    import contextlib
    import io
    import json

    from burnisher_amd import stage
    from burnisher_amd.t5 import t5_tensors
    from helpers import to_bf16
    from safetensors.numpy import save_file

    cfg = dict(SMALL, num_layers=2)
    rng = np.random.default_rng(31)
    f32 = {}
    for name, shape in t5_tensors(cfg).items():
        std = 0.1 if "layer_norm" in name else (1.0 if name == "shared.weight" or "relative" in name
                                                else 1 / np.sqrt(shape[1]))
        v = (rng.standard_normal(shape) * std).astype(np.float32)
        if "layer_norm" in name:
            v += 1.0
        f32[name] = v
    d = tmp_path / "ckpt" / "text_encoder"
    d.mkdir(parents=True)
    names = list(f32)
    halves = [names[: len(names) // 2], names[len(names) // 2:]]
    weight_map = {}
    for i, part in enumerate(halves):
        fn = f"model-0000{i + 1}-of-00002.safetensors"
        save_file({n: f32[n] for n in part}, str(d / fn))
        weight_map.update({n: fn for n in part})
    (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    wl = make_t5_workload(cfg, batch=2, seq=9, lengths=[3, 9], seed=32)
    wl.weights = {n: to_bf16(a) for n, a in f32.items()}
    want = stock_encode(wl)
    ids = tmp_path / "ids.npy"
    np.save(ids, wl.ids.astype(np.int64))
    out = tmp_path / "caption.npy"
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        assert stage.main(["t5-encode", "--weights", str(tmp_path / "ckpt"), "--ids", str(ids), "--out",
                           str(out), "--config", json.dumps(cfg)]) == 0
    rec = json.loads(buf.getvalue().split("BURNISH_JSON: ")[1])
    got = np.load(out)
    assert got.shape == (2, 9, cfg["d_model"]) and rec["effective"]["stage"] == "t5-encode"
    check(to_bf16(got), want, "t5-encode stage")
    assert np.array_equal(to_bf16(got), device_encode(wl))
    # a missing tensor is refused before anything is allocated
    bad = tmp_path / "bad" / "text_encoder"
    bad.mkdir(parents=True)
    save_file({n: f32[n] for n in names if n != "encoder.final_layer_norm.weight"}, str(bad / "model.safetensors"))
    with contextlib.redirect_stdout(io.StringIO()):
        assert stage.main(["t5-encode", "--weights", str(tmp_path / "bad"), "--ids", str(ids), "--out",
                           str(out), "--config", json.dumps(cfg)]) == 1
