"""The oracle (oracle/stock.cpp) pinned before it is trusted as the parity checker.

Four independent anchors, so that a plausible slip (a dropped term, a swapped operand, a wrong
index) fails at least one of them:
  1. the reference's own known-answer vectors and closed forms (tests/golden/reference_vectors.json,
     from /root/reference/tests/test_models.cpp and test_ops.cpp);
  2. the reference's invariants (head-last slicing, mask invariance, streaming == materialized,
     rows sum to one, LayerNorm mean 0 / variance 1, patch orderings by formula);
  3. float64 numpy brute force on tiny shapes (an independent textbook implementation);
  4. bit-for-bit agreement with the reference's OWN stock code compiled into oracle/_ref
     (skipped where that library was not built).
Plus the property the CPU baseline relies on: results do not depend on the thread count.
"""
import ctypes

import numpy as np
import pytest

import oracle
from helpers import (BF16, F32, addr, from_bf16, golden, ramp, randn_bf16, round_bf16, to_bf16)

RNG = np.random.default_rng(1234)


def stock_call(lib, name, *args):
    oracle.call(lib, name, *args)


# ---- 1. known answers ---------------------------------------------------------------------

def test_bf16_rounding_known_answers():
    g = golden("reference_vectors.json")["bf16"]
    for v in g["exact"]:
        assert from_bf16(to_bf16(np.float32(v)))[()] == v
    tie = g["tie_to_even"]
    assert from_bf16(to_bf16(np.float32(tie["input"])))[()] == tie["expect"]
    assert np.isnan(from_bf16(to_bf16(np.float32(np.nan))))
    assert np.isinf(from_bf16(to_bf16(np.float32(np.inf))))


@pytest.mark.parametrize("transposed", [False, True])
def test_gemm_known_answer(stock, transposed):
    g = golden("reference_vectors.json")["gemm"]
    a = np.array(g["a"], dtype=np.float32)
    b = np.array(g["b_nk"] if transposed else g["b_kn"], dtype=np.float32)
    out = np.zeros((2, 2), dtype=np.float32)
    stock_call(stock, "stock_gemm", addr(a), addr(b), None, addr(out), 2, 2, 3, int(transposed), 0, F32, 1)
    for idx, want in g["out"].items():
        assert abs(out.ravel()[int(idx)] - want) <= g["tolerance"]


def test_position_embedding_golden(stock):
    g = golden("reference_vectors.json")["position_embedding"]
    out = np.zeros(len(g["values"]), dtype=np.float64)
    stock_call(stock, "stock_position_embedding", out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
               g["dim"], g["grid"], g["base"], g["interpolation_scale"])
    assert np.max(np.abs(out - np.array(g["values"]))) < g["tolerance"]


def test_timestep_embedding_golden(stock):
    g = golden("reference_vectors.json")["timestep_embedding"]
    out = np.zeros(g["dim"], dtype=np.float32)
    stock_call(stock, "stock_timestep_embedding", g["t"], g["dim"],
               out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    assert np.max(np.abs(out - np.array(g["values"]))) < g["tolerance"]
    # cos first: at t = 0 the first half is 1 and the second half 0
    stock_call(stock, "stock_timestep_embedding", 0.0, 8, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    assert np.allclose(out[:4], 1.0) and np.allclose(out[4:], 0.0)
    with pytest.raises(oracle.OracleError):
        stock_call(stock, "stock_timestep_embedding", 0.0, 7, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))


# ---- 2. invariants ------------------------------------------------------------------------

def attention(stock, q, k, v, B, H, S, KV, D, mask=None, bias=None, materialized=False, dt=F32,
              scale=0.0):
    out = np.zeros((B, S, H, D), dtype=np.float32 if dt == F32 else np.uint16)
    stock_call(stock, "stock_attention", addr(q), addr(k), addr(v), addr(out), B, H, S, KV, D, scale,
               addr(bias), addr(mask), F32, dt, int(materialized), 2)
    return out


def test_streaming_equals_materialized(stock):
    B, H, S, M, D = 2, 3, 7, 5, 4
    q, k, v = ramp((B, S, H, D), 0.31), ramp((B, M, H, D), 0.17), ramp((B, M, H, D), 0.53)
    a = attention(stock, q, k, v, B, H, S, M, D)
    b = attention(stock, q, k, v, B, H, S, M, D, materialized=True)
    assert np.max(np.abs(a - b)) < 1e-5


def test_softmax_rows_sum_to_one_and_bias_moves_mass(stock):
    S, D = 4, 2
    q, k = ramp((1, S, 1, D), 0.7), ramp((1, S, 1, D), 0.3)
    v = np.zeros((1, S, 1, D), dtype=np.float32)
    v[0, :, 0, 0] = 1.0
    v[0, :, 0, 1] = np.arange(S)
    out = attention(stock, q, k, v, 1, 1, S, S, D)
    assert np.allclose(out[0, :, 0, 0], 1.0, atol=1e-5)
    bias = np.zeros((1, S, S), dtype=np.float32)
    bias[0, :, 0] = 50.0
    biased = attention(stock, q, k, v, 1, 1, S, S, D, bias=bias)
    assert np.max(np.abs(out - biased)) > 1e-6
    assert np.allclose(biased[0, :, 0, 1], 0.0, atol=1e-4)


def test_head_last_layout(stock):
    B, H, S, D = 2, 3, 5, 4
    q, k, v = ramp((B, S, H, D), 0.29), ramp((B, S, H, D), 0.13), ramp((B, S, H, D), 0.41)
    multi = attention(stock, q, k, v, B, H, S, S, D)
    for b in range(B):
        for h in range(H):
            sq, sk, sv = (np.ascontiguousarray(t[b:b + 1, :, h:h + 1, :]) for t in (q, k, v))
            single = attention(stock, sq, sk, sv, 1, 1, S, S, D)
            assert np.allclose(multi[b, :, h, :], single[0, :, 0, :], atol=1e-5)


def test_key_mask(stock):
    B, H, S, KV, D = 2, 2, 3, 4, 2
    q, k = ramp((B, S, H, D), 0.7), ramp((B, KV, H, D), 0.3)
    v = np.arange(B * KV * H * D, dtype=np.float32).reshape(B, KV, H, D)
    keep = [3, 2]
    mask = np.array([[1.0 if j < keep[b] else 0.0 for j in range(KV)] for b in range(B)], dtype=np.float32)
    out = attention(stock, q, k, v, B, H, S, KV, D, mask=mask)
    v2 = v.copy()
    for b in range(B):
        v2[b, keep[b]:] = 1234.0
    out2 = attention(stock, q, k, v2, B, H, S, KV, D, mask=mask)
    assert np.max(np.abs(out - out2)) < 1e-4
    outm = attention(stock, q, k, v, B, H, S, KV, D, mask=mask, materialized=True)
    assert np.max(np.abs(out - outm)) < 1e-5
    # all keys masked: every score is -1e9, so the row is the plain average of V (finite)
    none = np.zeros((B, KV), dtype=np.float32)
    outn = attention(stock, q, k, v, B, H, S, KV, D, mask=none)
    assert np.all(np.isfinite(outn))
    assert np.allclose(outn, np.broadcast_to(v.mean(axis=1, keepdims=True), (B, S, H, D)), atol=1e-3)


def test_layernorm_moments_and_rms(stock):
    x = np.array([[1, 2, 3, 4]], dtype=np.float32)
    out = np.zeros_like(x)
    stock_call(stock, "stock_norm", addr(x), None, None, addr(out), 1, 4, 1e-6, 0, F32, 1)
    assert abs(out.mean()) < 1e-5 and abs((out ** 2).mean() - 1.0) < 1e-4
    r = np.zeros_like(x)
    stock_call(stock, "stock_norm", addr(x), None, None, addr(r), 1, 4, 1e-6, 1, F32, 1)
    assert abs(r.mean()) > 0.1


def test_modulate_closed_form(stock):
    B, T, C = 2, 3, 2
    x, res = ramp((B, T, C), 0.4), ramp((B, T, C), 0.8)
    scale = np.full((B, C), 0.5, np.float32)
    shift = np.full((B, C), -0.25, np.float32)
    gate = np.full((B, C), 2.0, np.float32)
    out = np.zeros_like(x)
    stock_call(stock, "stock_modulate", addr(x), addr(scale), addr(shift), addr(out), B, T, C, None, None, F32)
    assert np.allclose(out, x * 1.5 - 0.25, atol=1e-5)
    gated = np.zeros_like(x)
    stock_call(stock, "stock_modulate", addr(x), addr(scale), addr(shift), addr(gated), B, T, C,
               addr(res), addr(gate), F32)
    assert np.allclose(gated, (x * 1.5 - 0.25) * 2.0 + res, atol=1e-5)


def test_patch_orderings_by_formula(stock):
    # inverse (unpatchify): channel varies FASTEST within a token -- (ky, kx, c)
    C, P, G = 3, 2, 4
    tokens = np.arange(G * G * C * P * P, dtype=np.float32).reshape(1, G * G, C * P * P)
    img = np.zeros((1, C, G * P, G * P), dtype=np.float32)
    stock_call(stock, "stock_patch", addr(tokens), addr(img), 1, C, G, P, 1, F32)
    for ty in range(G):
        for tx in range(G):
            for ky in range(P):
                for kx in range(P):
                    for c in range(C):
                        assert img[0, c, ty * P + ky, tx * P + kx] == tokens[0, ty * G + tx, (ky * P + kx) * C + c]
    # forward (patchify): (c, ky, kx), column fastest -- a conv weight's layout
    C, P, G = 2, 2, 2
    im = np.arange(C * (G * P) ** 2, dtype=np.float32).reshape(1, C, G * P, G * P)
    tok = np.zeros((1, G * G, C * P * P), dtype=np.float32)
    stock_call(stock, "stock_patch", addr(im), addr(tok), 1, C, G, P, 0, F32)
    for ty in range(G):
        for tx in range(G):
            for c in range(C):
                for ky in range(P):
                    for kx in range(P):
                        assert tok[0, ty * G + tx, (c * P + ky) * P + kx] == im[0, c, ty * P + ky, tx * P + kx]


# ---- 3. float64 brute force ---------------------------------------------------------------

def np_gelu(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


@pytest.mark.parametrize("epi", [0, 1, 2])
def test_gemm_vs_float64(stock, epi):
    M, N, K = 13, 11, 37
    a, b, bias = randn_bf16(RNG, (M, K)), randn_bf16(RNG, (N, K), 0.1), randn_bf16(RNG, (N,), 0.1)
    out = np.zeros((M, N), dtype=np.uint16)
    stock_call(stock, "stock_gemm", addr(a), addr(b), addr(bias), addr(out), M, N, K, 1, epi, BF16, 3)
    acc = from_bf16(a).astype(np.float64) @ from_bf16(b).astype(np.float64).T + from_bf16(bias)
    want = {0: acc, 1: np_gelu(acc), 2: acc / (1.0 + np.exp(-acc))}[epi]
    got = from_bf16(out)
    # one bf16 rounding of the output plus fp32 accumulation error
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -8 + 1e-5)


def test_attention_vs_float64(stock):
    B, H, S, KV, D = 2, 3, 9, 6, 8
    q, k, v = (randn_bf16(RNG, s) for s in ((B, S, H, D), (B, KV, H, D), (B, KV, H, D)))
    mask = np.ones((B, KV), dtype=np.float32)
    mask[1, 4:] = 0.0
    out = attention(stock, q, k, v, B, H, S, KV, D, mask=mask, dt=BF16)
    qf, kf, vf = (from_bf16(t).astype(np.float64) for t in (q, k, v))
    s = np.einsum("bshd,bkhd->bhsk", qf, kf) / np.sqrt(D)
    s = np.where(mask[:, None, None, :] == 0, -1e9, s)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    want = np.einsum("bhsk,bkhd->bshd", p, vf)
    assert np.all(np.abs(from_bf16(out) - want) <= np.abs(want) * 2.0 ** -8 + 1e-5)


def test_layernorm_vs_float64(stock):
    rows, cols = 7, 1152
    x = randn_bf16(RNG, (rows, cols), 3.0)
    out = np.zeros_like(x)
    stock_call(stock, "stock_norm", addr(x), None, None, addr(out), rows, cols, 1e-6, 0, BF16, 2)
    xf = from_bf16(x).astype(np.float64)
    want = (xf - xf.mean(1, keepdims=True)) / np.sqrt(xf.var(1, keepdims=True) + 1e-6)
    assert np.all(np.abs(from_bf16(out) - want) <= np.abs(want) * 2.0 ** -8 + 1e-6)


# ---- 4. bit-for-bit against the reference's own stock code --------------------------------

def test_ops_match_reference_bit_for_bit(stock, ref):
    # gemm, both layouts and every DiT epilogue
    M, N, K = 9, 13, 40
    a, b, bias = randn_bf16(RNG, (M, K)), randn_bf16(RNG, (N, K), 0.05), randn_bf16(RNG, (N,), 0.1)
    for bt in (0, 1):
        for epi in (0, 1, 2):
            o1, o2 = np.zeros((M, N), np.uint16), np.zeros((M, N), np.uint16)
            stock_call(stock, "stock_gemm", addr(a), addr(b), addr(bias), addr(o1), M, N, K, bt, epi, BF16, 4)
            oracle.call(ref, "ref_gemm", addr(a), addr(b), addr(bias), addr(o2), M, N, K, bt, epi, BF16)
            assert np.array_equal(o1, o2), (bt, epi)
    # attention with mask and bias, bf16 and fp32, streaming and materialized
    B, H, S, KV, D = 2, 3, 7, 5, 4
    for dt in (F32, BF16):
        cvt = (lambda t: t) if dt == F32 else to_bf16
        q, k, v = cvt(ramp((B, S, H, D), 0.31)), cvt(ramp((B, KV, H, D), 0.17)), cvt(ramp((B, KV, H, D), 0.53))
        bias = cvt(ramp((H, S, KV), 0.07))
        mask = np.array([[1, 1, 1, 0, 0], [1, 0, 0, 0, 0]], dtype=np.float32)
        for mat in (0, 1):
            shape, typ = (B, S, H, D), (np.float32 if dt == F32 else np.uint16)
            o1, o2 = np.zeros(shape, typ), np.zeros(shape, typ)
            stock_call(stock, "stock_attention", addr(q), addr(k), addr(v), addr(o1), B, H, S, KV, D, 1.0,
                       addr(bias), addr(mask), F32, dt, mat, 3)
            oracle.call(ref, "ref_attention", addr(q), addr(k), addr(v), addr(o2), B, H, S, KV, D, 1.0,
                        addr(bias), addr(mask), F32, dt, mat)
            assert np.array_equal(o1, o2), (dt, mat)
    # norm, modulate, activation, add, chunk, patch
    x = randn_bf16(RNG, (6, 1152), 2.0)
    o1, o2 = np.zeros_like(x), np.zeros_like(x)
    stock_call(stock, "stock_norm", addr(x), None, None, addr(o1), 6, 1152, 1e-6, 0, BF16, 2)
    oracle.call(ref, "ref_norm", addr(x), None, None, addr(o2), 6, 1152, 1e-6, 0, BF16)
    assert np.array_equal(o1, o2)
    Bm, T, C = 2, 5, 24
    xm, res = randn_bf16(RNG, (Bm, T, C)), randn_bf16(RNG, (Bm, T, C))
    sc, sh, gt = (randn_bf16(RNG, (Bm, C), 0.3) for _ in range(3))
    for r, g in ((None, None), (res, gt)):
        o1, o2 = np.zeros_like(xm), np.zeros_like(xm)
        stock_call(stock, "stock_modulate", addr(xm), addr(sc), addr(sh), addr(o1), Bm, T, C, addr(r), addr(g), BF16)
        oracle.call(ref, "ref_modulate", addr(xm), addr(sc), addr(sh), addr(o2), Bm, T, C, addr(r), addr(g), BF16)
        assert np.array_equal(o1, o2)
    for kind in (1, 2):
        o1, o2 = np.zeros_like(xm), np.zeros_like(xm)
        stock_call(stock, "stock_activation", addr(xm), addr(o1), xm.size, kind, None, BF16)
        oracle.call(ref, "ref_activation", addr(xm), addr(o2), xm.size, kind, None, BF16)
        assert np.array_equal(o1, o2)
    for bcast in (0, 1):
        bb = randn_bf16(RNG, (T * C,) if bcast else (Bm, T * C))
        o1, o2 = np.zeros((Bm, T * C), np.uint16), np.zeros((Bm, T * C), np.uint16)
        aa = xm.reshape(Bm, T * C)
        stock_call(stock, "stock_add", addr(aa), addr(bb), addr(o1), Bm, T * C, 1.0, bcast, BF16)
        oracle.call(ref, "ref_add", addr(aa), addr(bb), addr(o2), Bm, T * C, 1.0, bcast, BF16)
        assert np.array_equal(o1, o2)
    mod, table = randn_bf16(RNG, (2, 6 * C)), randn_bf16(RNG, (6, C))
    for chunk, trow in ((0, 0), (4, 4), (2, -1)):
        o1, o2 = np.zeros((2, C), np.uint16), np.zeros((2, C), np.uint16)
        stock_call(stock, "stock_chunk", addr(mod), addr(table), addr(o1), 2, C, 6, chunk, trow, BF16)
        oracle.call(ref, "ref_chunk", addr(mod), addr(table), addr(o2), 2, C, 6, chunk, trow, 6, BF16)
        assert np.array_equal(o1, o2)
    img = randn_bf16(RNG, (2, 4, 8, 8))
    o1, o2 = np.zeros((2, 16, 16), np.uint16), np.zeros((2, 16, 16), np.uint16)
    stock_call(stock, "stock_patch", addr(img), addr(o1), 2, 4, 4, 2, 0, BF16)
    oracle.call(ref, "ref_patch", addr(img), addr(o2), 2, 4, 4, 2, 0, BF16)
    assert np.array_equal(o1, o2)
    i1, i2 = np.zeros((2, 4, 8, 8), np.uint16), np.zeros((2, 4, 8, 8), np.uint16)
    stock_call(stock, "stock_patch", addr(o1), addr(i1), 2, 4, 4, 2, 1, BF16)
    oracle.call(ref, "ref_patch", addr(o1), addr(i2), 2, 4, 4, 2, 1, BF16)
    assert np.array_equal(i1, i2)


def test_embeddings_match_reference(stock, ref):
    for dim, grid, base in ((1152, 8, 64), (64, 16, 4)):
        a = np.zeros(grid * grid * dim, np.float64)
        b = np.zeros_like(a)
        P = ctypes.POINTER(ctypes.c_double)
        stock_call(stock, "stock_position_embedding", a.ctypes.data_as(P), dim, grid, base, 2.0)
        oracle.call(ref, "ref_position_embedding", b.ctypes.data_as(P), dim, grid, base, 2.0)
        assert np.array_equal(a, b)
    a, b = np.zeros(256, np.float32), np.zeros(256, np.float32)
    P = ctypes.POINTER(ctypes.c_float)
    stock_call(stock, "stock_timestep_embedding", 500.0, 256, a.ctypes.data_as(P))
    oracle.call(ref, "ref_timestep_embedding", 500.0, 256, b.ctypes.data_as(P))
    assert np.array_equal(a, b)


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_stock_scale_matches_reference(stock, ref, dtype):
    # ScaleArgs (ops_cpu.cpp:351-353): one multiply, one rounding; equal to the reference bit for bit
    # and, being a single IEEE multiply, to numpy's float32 product rounded the same way.
    x = ramp((4099,), 0.37) * np.float32(3.0)
    xin = x if dtype == F32 else to_bf16(x)
    o1 = np.zeros_like(xin)
    o2 = np.zeros_like(xin)
    oracle.call(stock, "stock_scale", addr(xin), addr(o1), xin.size, 0.18215, dtype)
    oracle.call(ref, "ref_scale", addr(xin), addr(o2), xin.size, 0.18215, dtype)
    assert np.array_equal(o1, o2)
    xf = xin if dtype == F32 else from_bf16(xin)
    want = (xf * np.float32(0.18215)).astype(np.float32)
    assert np.array_equal(o1, want if dtype == F32 else to_bf16(want))
