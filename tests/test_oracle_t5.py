"""The stock oracle's T5 encoder (oracle/stock.cpp: the relative-position bucket and the
t5_encoder.cpp graph), and the product's host-side bucket function, pinned:
  - the bucket against the reference's own known-answer table (tests/test_models.cpp:208-229,
    probes straddling the sign split, max_exact and the saturation at max_distance), and
    exhaustively against the reference's own function compiled into oracle/_ref;
  - the whole encoder bit-for-bit against the reference's own stock code (t5_encoder.cpp,
    ops_cpu.cpp, weights.cpp's declaration of the encoder's shapes) in oracle/_ref;
  - properties a plausible mistake fails: buckets are monotone in distance within each side,
    keys after the query use the upper half; padding only enters through the key mask."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import burnisher_amd as bh
import oracle
from burnisher_amd.t5 import config_struct, make_t5_workload, t5_tensors

# tests/test_models.cpp:208-229: (relative position, bucket) at 32 buckets, max_distance 128.
KNOWN_BUCKETS = [(-300, 15), (-129, 15), (-128, 15), (-127, 15), (-64, 14), (-16, 10), (-9, 8),
                 (-8, 8), (-7, 7), (-1, 1), (0, 0), (1, 17), (7, 23), (8, 24), (9, 24), (16, 26),
                 (64, 30), (127, 31), (128, 31), (129, 31), (300, 31)]

SMALL = dict(num_layers=2, d_model=64, d_ff=96, d_kv=16, num_heads=4, vocab_size=100, gated=1,
             num_buckets=32, eps=1e-6)


def stock_bucket(rp, nb, md):
    return oracle.stock().stock_t5_bucket(rp, nb, md)


def test_bucket_known_answers():
    lib = bh.lib()
    for rp, want in KNOWN_BUCKETS:
        assert stock_bucket(rp, 32, 128) == want, rp
        assert lib.bh_t5_relative_bucket(rp, 32, 128) == want, rp
    ref = oracle.ref()
    if ref is not None:
        for rp, want in KNOWN_BUCKETS:
            assert ref.ref_t5_bucket(rp, 32, 128) == want, rp


def test_bucket_exhaustive_and_monotone():
    lib = bh.lib()
    ref = oracle.ref()
    for nb in (8, 16, 32, 64):
        for md in (20, 128, 512):
            got = [stock_bucket(rp, nb, md) for rp in range(-700, 701)]
            assert got == [lib.bh_t5_relative_bucket(rp, nb, md) for rp in range(-700, 701)], (nb, md)
            if ref is not None:
                assert got == [ref.ref_t5_bucket(rp, nb, md) for rp in range(-700, 701)], (nb, md)
            half = nb // 2
            left, right = got[:700][::-1], got[701:]          # |rp| = 1, 2, ... on each side
            assert got[700] == 0
            assert all(0 <= b < half for b in left) and all(half <= b < nb for b in right)
            assert all(a <= b for a, b in zip(left, left[1:])) and all(a <= b for a, b in zip(right, right[1:]))
            assert left[: half // 2 - 1] == list(range(1, half // 2))   # exact distances
            assert left[-1] == half - 1 and right[-1] == nb - 1          # saturation


def run_stock(wl, threads=0):
    cfg = config_struct(wl.cfg)
    w, keep = wl.table()
    out = np.zeros((wl.batch, wl.seq, wl.cfg["d_model"]), np.uint16)
    oracle.call(oracle.stock(), "stock_t5_forward", ctypes.byref(cfg), ctypes.byref(w),
                wl.ids.ctypes.data, wl.batch, wl.seq, out.ctypes.data, threads)
    return out


@pytest.mark.parametrize("cfg,lengths", [(SMALL, [3, 9]), (dict(SMALL, gated=0, num_layers=1), [9, 5]),
                                         (dict(SMALL, d_kv=8, num_heads=8), [1, 7])],
                         ids=["gated", "plain_gelu", "eight_heads"])
def test_encoder_matches_reference_bit_for_bit(cfg, lengths):
    ref = oracle.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built (no /root/reference here)")
    wl = make_t5_workload(cfg, batch=2, seq=9, lengths=lengths, seed=3)
    got = run_stock(wl, threads=3)
    c = config_struct(wl.cfg)
    w, keep = wl.table()
    want = np.zeros_like(got)
    oracle.call(ref, "ref_t5_forward", ctypes.byref(c), ctypes.byref(w), wl.ids.ctypes.data, 2, 9,
                want.ctypes.data)
    assert np.array_equal(got, want)
    assert np.array_equal(run_stock(wl, threads=1), got), "thread count changed the result"


def test_encoder_properties():
    wl = make_t5_workload(SMALL, batch=2, seq=9, lengths=[4, 9], seed=4)
    base = run_stock(wl)
    # a pad id is masked out as a key: row 0's real positions ignore everything past its padding,
    # so giving row 0 a different padded tail (still pads) is impossible -- instead make the
    # padded positions real tokens and check the real positions move
    alt = make_t5_workload(SMALL, batch=2, seq=9, lengths=[4, 9], seed=4)
    alt.ids[0, 4:] = 5
    moved = run_stock(alt)
    assert not np.array_equal(moved[0, :4], base[0, :4]), "padding keys are not masked"
    assert np.array_equal(moved[1], base[1]), "batch rows leak into each other"
    # the relative bias reaches the scores: zeroing it changes the output
    zb = make_t5_workload(SMALL, batch=2, seq=9, lengths=[4, 9], seed=4)
    name = "encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight"
    zb.weights[name] = np.zeros_like(zb.weights[name])
    assert not np.array_equal(run_stock(zb), base)
    # an id outside the vocabulary is refused (t5_encoder.cpp:146-156)
    bad = make_t5_workload(SMALL, batch=2, seq=9, lengths=[4, 9], seed=4)
    bad.ids[1, 2] = SMALL["vocab_size"]
    with pytest.raises(RuntimeError, match="vocabulary"):
        run_stock(bad)


def test_table_matches_the_declaration():
    names = list(t5_tensors(SMALL))
    assert names[:3] == ["shared.weight", "encoder.final_layer_norm.weight",
                         "encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight"]
    assert len(names) == 3 + 2 * 9
    assert len(t5_tensors(dict(SMALL, gated=0))) == 3 + 2 * 8


def test_create_refuses_before_any_device_work():
    lib = bh.lib()
    wl = make_t5_workload(dict(SMALL, num_layers=1), batch=1, seq=4, lengths=[4])
    w, keep = wl.table()
    h = ctypes.c_void_p()
    cfg = config_struct(dict(SMALL, num_layers=1, d_kv=200))
    assert lib.bh_t5_create(ctypes.byref(cfg), ctypes.byref(w), 1, 4, ctypes.byref(h)) != 0
    assert b"d_kv" in lib.bh_last_error()
    cfg = config_struct(dict(SMALL, num_layers=2))   # the table holds one layer only
    assert lib.bh_t5_create(ctypes.byref(cfg), ctypes.byref(w), 1, 4, ctypes.byref(h)) != 0
    assert b"missing" in lib.bh_last_error() and b"encoder.block.1." in lib.bh_last_error()
    assert lib.bh_gather(None, None, None, -1, 4, 4, 1, None) != 0
