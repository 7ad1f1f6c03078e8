"""Each hip-gfx950 op against the stock oracle on identical seeded inputs, through the C ABI.

Modelled on the reference's device-vs-oracle tests (/root/reference/tests/test_cuda_ops.cpp):
odd small shapes that catch stride and layout slips, the DiT's own shapes, masks that keep
different key counts per batch row (one keeps a single key), and a byte-identical second call.
Tolerances are configs/tolerance.json's per-op bf16 gates.
"""
import numpy as np
import pytest

import oracle
from helpers import (BF16, F32, addr, assert_within, from_bf16, ramp, randn_bf16, stats, to_bf16)

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(20260911)


# Device copies made inline as call arguments (`P(dev(x))`) would be freed -- and their memory
# handed to the next copy by the caching allocator -- before the asynchronous kernel reads them.
# They are kept here until the next synchronising read-back.
_LIVE = []


def dev(a):
    import torch
    if a is None:
        return None
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).cuda()
    else:
        t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    _LIVE.append(t)
    return t


def host(t, like):
    import torch
    torch.cuda.synchronize()
    _LIVE.clear()
    if t.dtype == torch.bfloat16:
        return t.cpu().view(torch.int16).numpy().view(np.uint16).reshape(like.shape)
    return t.cpu().numpy().reshape(like.shape)


def empty(shape, bf16=True):
    import torch
    return torch.zeros(shape, dtype=torch.bfloat16 if bf16 else torch.float32, device="cuda")


def P(t):
    return None if t is None else t.data_ptr()


def call(name, *args):
    import burnisher_amd as bh
    bh.call(name, *args)


def st(name, *args):
    oracle.call(oracle.stock(), name, *args)


# ---- gemm ---------------------------------------------------------------------------------

GEMM_SHAPES = [(13, 11, 40), (37, 150, 64), (2, 6912, 1152), (5, 1152, 256), (600, 1152, 4096),
               (1024, 1152, 1152), (512, 3456, 1152), (512, 4608, 1152), (256, 1152, 4608),
               (1024, 32, 1152), (2048, 1152, 16), (300, 200, 72),
               # the MFMA kernel with ragged M and N tiles, and k-tile counts of 1, 2 and 5
               (37, 152, 128), (777, 296, 320), (300, 1152, 64),
               # more tiles than CUs: the persistent loop, whole and ragged tile grids
               (3072, 3456, 128), (4100, 2312, 64),
               # tile heights: 128 rows (96 tiles of 256 rows would fill 96 CUs), 64 rows, 192 rows
               # (the 768px N = 1152 shape: 144 tiles of 256 rows against 192 of 192), and 192
               # rows with ragged M and N
               (2048, 1728, 256), (1000, 1160, 192), (4608, 1152, 1152), (4500, 1160, 192)]


@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("epi", [0, 1, 2])
def test_gemm_matches_oracle(hip, shape, epi):
    M, N, K = shape
    a, b, bias = randn_bf16(RNG, (M, K)), randn_bf16(RNG, (N, K), 0.02), randn_bf16(RNG, (N,), 0.02)
    want = np.zeros((M, N), np.uint16)
    st("stock_gemm", addr(a), addr(b), addr(bias), addr(want), M, N, K, 1, epi, BF16, 0)
    da, db, dbias = dev(a), dev(b), dev(bias)
    got, again = empty((M, N)), empty((M, N))
    call("bh_gemm", P(da), P(db), P(dbias), P(got), M, N, K, 1, epi, BF16, None)
    call("bh_gemm", P(da), P(db), P(dbias), P(again), M, N, K, 1, epi, BF16, None)
    g = host(got, want)
    assert_within(from_bf16(g), from_bf16(want), "gemm", f"{shape} epi={epi}")
    assert np.array_equal(g, host(again, want)), "not byte-identical across two calls"


@pytest.mark.parametrize("act", [0, 1], ids=["plain", "gelu"])
def test_gemm_tile_heights_agree(hip, act):
    # The tile height is chosen per launch from M and N (on 256 CUs: 64 rows at M = 2048, 128 at
    # 4096, 192 at 4608 and 256 at 8192 for N = 1152); every height sums an output's k-tiles in the
    # same order with the same MFMAs, so the rows a shorter launch shares with a taller one are
    # bit-identical.
    M, N, K = 8192, 1152, 1152
    a, b, bias = randn_bf16(RNG, (M, K)), randn_bf16(RNG, (N, K), 0.02), randn_bf16(RNG, (N,), 0.02)
    da, db, dbias = dev(a), dev(b), dev(bias)
    full = empty((M, N))
    call("bh_gemm", P(da), P(db), P(dbias), P(full), M, N, K, 1, act, BF16, None)
    want = host(full, np.zeros((M, N), np.uint16))
    for rows in (2048, 4096, 4608, 4500):
        part = empty((rows, N))
        call("bh_gemm", P(da), P(db), P(dbias), P(part), rows, N, K, 1, act, BF16, None)
        assert np.array_equal(host(part, want[:rows]), want[:rows]), f"{rows} rows differ from {M}"


def test_gemm_tile_heights_agree_gated_residual(hip):
    # The same for the gated-residual store (x + gate[row / tokens] * bf16(A . B^T + bias), in
    # place), the epilogue of the out-projection and ff2: 4608 rows run 192-row tiles, 8192 rows
    # 256-row tiles, 2048 rows 64-row tiles.
    import burnisher_amd as bh
    import ctypes
    M, N, K, tokens = 8192, 1152, 1152, 256
    a, b, bias = randn_bf16(RNG, (M, K)), randn_bf16(RNG, (N, K), 0.02), randn_bf16(RNG, (N,), 0.02)
    x, gate = randn_bf16(RNG, (M, N)), randn_bf16(RNG, (M // tokens, N), 0.5)
    da, db, dbias, dgate = dev(a), dev(b), dev(bias), dev(gate)
    results = {}
    for rows in (M, 4608, 2048):
        dx = dev(x[:rows])
        f = bh.GemmFused(epilogue=0, round_mid=1, residual=P(dx), gate=P(dgate), gate_rows=tokens, ld_out=N)
        call("bh_gemm_fused_run", P(da), P(db), P(dbias), P(dx), rows, N, K, ctypes.byref(f), None)
        results[rows] = host(dx, x[:rows])
    for rows in (4608, 2048):
        assert np.array_equal(results[rows], results[M][:rows]), f"{rows} rows differ from {M}"


def test_gemm_unaligned_k_and_plain_layouts(hip):
    # K % 8 != 0, B as [K, N], and fp32: the reference-order kernel, bit-exact with the oracle
    M, N, K = 9, 7, 13
    a, b, bias = randn_bf16(RNG, (M, K)), randn_bf16(RNG, (N, K), 0.3), randn_bf16(RNG, (N,), 0.1)
    for bt in (1, 0):
        want = np.zeros((M, N), np.uint16)
        st("stock_gemm", addr(a), addr(b), addr(bias), addr(want), M, N, K, bt, 1, BF16, 1)
        got = empty((M, N))
        call("bh_gemm", P(dev(a)), P(dev(b)), P(dev(bias)), P(got), M, N, K, bt, 1, BF16, None)
        assert np.array_equal(host(got, want), want)
    af, bf = from_bf16(a), from_bf16(b)
    want = np.zeros((M, N), np.float32)
    st("stock_gemm", addr(af), addr(bf), None, addr(want), M, N, K, 1, 0, F32, 1)
    got = empty((M, N), bf16=False)
    call("bh_gemm", P(dev(af)), P(dev(bf)), None, P(got), M, N, K, 1, 0, F32, None)
    assert np.array_equal(host(got, want), want)


def test_gemm_fused_epilogues(hip):
    import burnisher_amd as bh
    import ctypes
    B, N_tok, d, K = 2, 300, 1152, 1152
    M = B * N_tok
    a, w, bias = randn_bf16(RNG, (M, K)), randn_bf16(RNG, (d, K), 0.02), randn_bf16(RNG, (d,), 0.02)
    x, gate = randn_bf16(RNG, (M, d)), randn_bf16(RNG, (B, d), 0.5)
    pos = randn_bf16(RNG, (N_tok, d))
    zero = np.zeros((B, d), np.uint16)
    proj = np.zeros((M, d), np.uint16)
    st("stock_gemm", addr(a), addr(w), addr(bias), addr(proj), M, d, K, 1, 0, BF16, 0)
    # gated residual: x + gate * proj, through modulate with zero scale/shift (pixart_dit.cpp:249)
    want = x.copy()
    st("stock_modulate", addr(proj), addr(zero), addr(zero), addr(want), B, N_tok, d, addr(want), addr(gate), BF16)
    # residual add (pixart_dit.cpp:268) and broadcast position add (pixart_dit.cpp:149)
    want_add = x.copy()
    st("stock_add", addr(want_add), addr(proj), addr(want_add), M, d, 1.0, 0, BF16)
    want_pos = np.zeros_like(proj)
    st("stock_add", addr(proj), addr(pos), addr(want_pos), B, N_tok * d, 1.0, 1, BF16)

    dx, dgate, dpos = dev(x), dev(gate), dev(pos)
    da, dw, db = dev(a), dev(w), dev(bias)
    f = bh.GemmFused(epilogue=0, round_mid=1, residual=P(dx), gate=P(dgate), gate_rows=N_tok, ld_out=d)
    call("bh_gemm_fused_run", P(da), P(dw), P(db), P(dx), M, d, K, ctypes.byref(f), None)
    s1 = assert_within(from_bf16(host(dx, want)), from_bf16(want), "gemm_fused", "gated residual")
    dx2 = dev(x)
    f = bh.GemmFused(epilogue=0, round_mid=1, residual=P(dx2), ld_out=d)
    call("bh_gemm_fused_run", P(da), P(dw), P(db), P(dx2), M, d, K, ctypes.byref(f), None)
    assert_within(from_bf16(host(dx2, want_add)), from_bf16(want_add), "gemm_fused", "residual add")
    out = empty((M, d))
    f = bh.GemmFused(epilogue=0, round_mid=1, row_add=P(dpos), row_add_period=N_tok, ld_out=d)
    call("bh_gemm_fused_run", P(da), P(dw), P(db), P(out), M, d, K, ctypes.byref(f), None)
    assert_within(from_bf16(host(out, want_pos)), from_bf16(want_pos), "gemm_fused", "row add")
    assert s1["mismatch_frac"] < 0.01


@pytest.mark.parametrize("B,N_tok", [(2, 1024), (7, 143)], ids=["whole_bands", "ragged_band"])
def test_gemm_small_k_fused_epilogues(hip, B, N_tok):
    # K = 16, the patch embedding's in_channels * patch^2: the register-weight kernel. Whole bands
    # of rows take the path that issues every load of the band before its first store (plain and
    # row-add stores); M = 1001 leaves a ragged last band, which walks its rows one at a time, as
    # do the residual epilogues.
    import burnisher_amd as bh
    import ctypes
    d, K = 1152, 16
    M = B * N_tok
    a, w, bias = randn_bf16(RNG, (M, K)), randn_bf16(RNG, (d, K), 0.02), randn_bf16(RNG, (d,), 0.02)
    x, gate, pos = randn_bf16(RNG, (M, d)), randn_bf16(RNG, (B, d), 0.5), randn_bf16(RNG, (N_tok, d))
    zero = np.zeros((B, d), np.uint16)
    proj = np.zeros((M, d), np.uint16)
    st("stock_gemm", addr(a), addr(w), addr(bias), addr(proj), M, d, K, 1, 0, BF16, 0)
    want_pos = np.zeros_like(proj)
    st("stock_add", addr(proj), addr(pos), addr(want_pos), B, N_tok * d, 1.0, 1, BF16)
    want_gated = x.copy()
    st("stock_modulate", addr(proj), addr(zero), addr(zero), addr(want_gated), B, N_tok, d,
       addr(want_gated), addr(gate), BF16)
    da, dw, db, dpos, dgate = dev(a), dev(w), dev(bias), dev(pos), dev(gate)
    out = empty((M, d))
    f = bh.GemmFused(epilogue=0, round_mid=1, row_add=P(dpos), row_add_period=N_tok, ld_out=d)
    call("bh_gemm_fused_run", P(da), P(dw), P(db), P(out), M, d, K, ctypes.byref(f), None)
    assert_within(from_bf16(host(out, want_pos)), from_bf16(want_pos), "gemm_fused", f"row add M={M}")
    plain = empty((M, d))
    call("bh_gemm", P(da), P(dw), P(db), P(plain), M, d, K, 1, 0, BF16, None)
    assert_within(from_bf16(host(plain, proj)), from_bf16(proj), "gemm", f"plain M={M}")
    dx = dev(x)
    f = bh.GemmFused(epilogue=0, round_mid=1, residual=P(dx), gate=P(dgate), gate_rows=N_tok, ld_out=d)
    call("bh_gemm_fused_run", P(da), P(dw), P(db), P(dx), M, d, K, ctypes.byref(f), None)
    assert_within(from_bf16(host(dx, want_gated)), from_bf16(want_gated), "gemm_fused", f"gated M={M}")


def test_gemm_split_k_epilogues(hip):
    # A long-K GEMM with few output tiles (the 512px ff2 shape at 300 tokens per row: 24 tiles of
    # 256 x 144, 72 k-tiles) runs as K slices whose fp32 partials are summed in slice order by the
    # epilogue kernel: gated residual, residual and GELU store against the oracle, byte-identical
    # across calls, and a larger then a smaller call through the library's partial buffer.
    import burnisher_amd as bh
    import ctypes
    B, N_tok, d, K = 2, 300, 1152, 4608
    M = B * N_tok
    a, w, bias = randn_bf16(RNG, (M, K)), randn_bf16(RNG, (d, K), 0.02), randn_bf16(RNG, (d,), 0.02)
    x, gate = randn_bf16(RNG, (M, d)), randn_bf16(RNG, (B, d), 0.5)
    zero = np.zeros((B, d), np.uint16)
    proj = np.zeros((M, d), np.uint16)
    st("stock_gemm", addr(a), addr(w), addr(bias), addr(proj), M, d, K, 1, 0, BF16, 0)
    want_gated = x.copy()
    st("stock_modulate", addr(proj), addr(zero), addr(zero), addr(want_gated), B, N_tok, d,
       addr(want_gated), addr(gate), BF16)
    want_add = x.copy()
    st("stock_add", addr(want_add), addr(proj), addr(want_add), M, d, 1.0, 0, BF16)
    da, dw, db, dgate = dev(a), dev(w), dev(bias), dev(gate)
    for rep in range(2):
        print(f"split-K gated / residual, call {rep}", flush=True)
        dx = dev(x)
        f = bh.GemmFused(epilogue=0, round_mid=1, residual=P(dx), gate=P(dgate), gate_rows=N_tok, ld_out=d)
        call("bh_gemm_fused_run", P(da), P(dw), P(db), P(dx), M, d, K, ctypes.byref(f), None)
        g = host(dx, want_gated)
        assert_within(from_bf16(g), from_bf16(want_gated), "gemm_fused", f"split-K gated residual {rep}")
        if rep == 0:
            first = g
        else:
            assert np.array_equal(g, first), "split-K gated residual not byte-identical"
        dx2 = dev(x)
        f = bh.GemmFused(epilogue=0, round_mid=1, residual=P(dx2), ld_out=d)
        call("bh_gemm_fused_run", P(da), P(dw), P(db), P(dx2), M, d, K, ctypes.byref(f), None)
        assert_within(from_bf16(host(dx2, want_add)), from_bf16(want_add), "gemm_fused",
                      f"split-K residual {rep}")
    # GELU store, then a smaller long-K call (one row block) through the same partial buffer
    for m in (M, 40):
        want = np.zeros((m, d), np.uint16)
        st("stock_gemm", addr(a[:m]), addr(w), addr(bias), addr(want), m, d, K, 1, 1, BF16, 0)
        got = empty((m, d))
        call("bh_gemm", P(dev(a[:m])), P(dw), P(db), P(got), m, d, K, 1, 1, BF16, None)
        assert_within(from_bf16(host(got, want)), from_bf16(want), "gemm", f"split-K GELU M={m}")


# ---- attention ----------------------------------------------------------------------------

def attention_case(B, S, KV, H, D, mask=None, scale=0.0, strided=False, inputs=None):
    if inputs is None:
        q, k, v = (randn_bf16(RNG, s) for s in ((B, S, H, D), (B, KV, H, D), (B, KV, H, D)))
    else:
        q, k, v = inputs
    want = np.zeros((B, S, H, D), np.uint16)
    st("stock_attention", addr(q), addr(k), addr(v), addr(want), B, H, S, KV, D, scale, None,
       addr(mask), F32, BF16, 0, 0)
    dmask = dev(mask)
    got, again = empty((B, S, H, D)), empty((B, S, H, D))
    if strided:
        import torch
        d = H * D
        # Q, K, V as column blocks of one [B*S, 3d] tensor (the fused QKV projection layout)
        assert S == KV
        fused = torch.cat([dev(q).reshape(B * S, d), dev(k).reshape(B * S, d), dev(v).reshape(B * S, d)], 1).contiguous()
        for out in (got, again):
            call("bh_attention_strided", fused.data_ptr(), 3 * d, fused.data_ptr() + 2 * d,
                 fused.data_ptr() + 4 * d, 3 * d, P(out), d, B, H, S, KV, D, scale, P(dmask), F32, BF16, None)
    else:
        dq, dk, dv = dev(q), dev(k), dev(v)
        for out in (got, again):
            call("bh_attention", P(dq), P(dk), P(dv), P(out), B, H, S, KV, D, scale, None, P(dmask),
                 F32, BF16, None)
    g = host(got, want)
    assert np.array_equal(g, host(again, want)), "attention is not byte-identical across two calls"
    return g, want


@pytest.mark.parametrize("case", [
    (2, 7, 5, 3, 4), (2, 9, 9, 2, 6), (2, 64, 64, 2, 72), (2, 64, 20, 2, 72), (1, 300, 300, 2, 64),
    (2, 257, 100, 3, 72), (2, 1024, 1024, 16, 72), (2, 1024, 300, 16, 72), (1, 130, 70, 1, 128),
    (1, 40, 33, 2, 16)], ids=lambda c: "B{}S{}K{}H{}D{}".format(*c))
def test_attention_matches_oracle(hip, case):
    B, S, KV, H, D = case
    mask = None
    if KV != S:
        mask = np.zeros((B, KV), np.float32)
        mask[0, :max(1, KV // 4)] = 1.0
        if B > 1:
            mask[1, :1] = 1.0   # one row keeps a single key
    g, want = attention_case(B, S, KV, H, D, mask=mask)
    assert_within(from_bf16(g), from_bf16(want), "attention", str(case))


def test_attention_masks(hip):
    B, S, KV, H, D = 2, 128, 300, 4, 72
    # non-prefix mask, a fully masked 64-key block in the middle, and an all-masked row
    mask = np.ones((B, KV), np.float32)
    mask[0, 64:128] = 0.0
    mask[0, 200:260:3] = 0.0
    mask[1, :] = 0.0
    g, want = attention_case(B, S, KV, H, D, mask=mask)
    assert_within(from_bf16(g), from_bf16(want), "attention", "masks")
    # the all-masked row is the plain mean of V, not NaN
    assert np.all(np.isfinite(from_bf16(g)))


def test_attention_key_splits_masked(hip):
    # 16 workgroups of 512 queries over 16 key blocks: the head_dim-72 kernel splits the keys 8
    # ways (two blocks each) and combines the fp32 partials. Row 0 has live keys in the first split
    # only, row 1 none at all (the plain mean of V over every split), row 2 a hole covering whole
    # splits in the middle and a ragged last block.
    B, S, KV, H, D = 3, 600, 1000, 4, 72
    mask = np.zeros((B, KV), np.float32)
    mask[0, :40] = 1.0
    mask[2, :] = 1.0
    mask[2, 200:700] = 0.0
    mask[2, 990:] = 0.0
    g, want = attention_case(B, S, KV, H, D, mask=mask)
    assert_within(from_bf16(g), from_bf16(want), "attention", "key splits, masked")
    assert np.all(np.isfinite(from_bf16(g)))
    # unmasked, with a key count that is not a multiple of the 64-key block
    g, want = attention_case(1, 1000, 1000, 4, D)
    assert_within(from_bf16(g), from_bf16(want), "attention", "key splits, ragged")


def test_attention_ragged_last_round_masked(hip):
    # 16 heads x 17 query blocks = 272 workgroups of 512 queries on 256 CUs: query blocks 0-15
    # run whole and block 16 (508 queries) splits its 136 key blocks 8 ways. Masked: a key count
    # that is not a multiple of 64 and holes, one of them covering whole splits.
    B, S, KV, H, D = 1, 8700, 8699, 16, 72
    mask = np.ones((B, KV), np.float32)
    mask[0, 1000:3000] = 0.0
    mask[0, 5000:8000:7] = 0.0
    g, want = attention_case(B, S, KV, H, D, mask=mask)
    assert_within(from_bf16(g), from_bf16(want), "attention", "ragged last round, masked")
    lo = 16 * 512   # the split query block on its own
    assert_within(from_bf16(g[:, lo:]), from_bf16(want[:, lo:]), "attention", "the split query block")


def test_launch_profiler_sampling(hip):
    import ctypes
    # bh_profile_sample(3) brackets launches 0, 3 and 6 of seven; every launch after sample(1)
    B, S, H, D = 1, 256, 2, 72
    q, k, v = (dev(randn_bf16(RNG, (B, S, H, D))) for _ in range(3))
    out = empty((B, S, H, D))
    ms, n, work = ctypes.c_double(), ctypes.c_int64(), ctypes.c_double()
    for every, want in ((3, 3), (1, 7)):
        call("bh_profile_sample", every)
        call("bh_profile_enable", 1 << 2)   # BH_K_ATTN_SELF
        for _ in range(7):
            call("bh_attention", P(q), P(k), P(v), P(out), B, H, S, S, D, 0.0, None, None, F32, BF16, None)
        call("bh_profile_read", 2, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(work))
        call("bh_profile_enable", 0)
        assert n.value == want, (every, n.value)
        assert ms.value > 0 and work.value == want * 4.0 * B * H * S * S * D
    call("bh_profile_sample", 1)


def test_attention_masked_values_do_not_leak(hip):
    B, S, KV, H, D = 2, 64, 150, 2, 72
    q, k, v = (randn_bf16(RNG, s) for s in ((B, S, H, D), (B, KV, H, D), (B, KV, H, D)))
    mask = np.zeros((B, KV), np.float32)
    mask[0, :37] = 1.0
    mask[1, :75] = 1.0
    g1, _ = attention_case(B, S, KV, H, D, mask=mask, inputs=(q, k, v))
    v2 = v.copy()
    v2[0, 37:] = to_bf16(np.float32(1234.0))
    v2[1, 75:] = to_bf16(np.float32(-77.0))
    g2, _ = attention_case(B, S, KV, H, D, mask=mask, inputs=(q, k, v2))
    assert np.array_equal(g1, g2)


def test_attention_strided_qkv(hip):
    g, want = attention_case(2, 512, 512, 16, 72, strided=True)
    assert_within(from_bf16(g), from_bf16(want), "attention", "strided")


def test_attention_reference_order_path(hip):
    # fp32, and an additive bias: the reference-order kernel
    B, S, KV, H, D = 2, 7, 5, 3, 4
    q, k, v = ramp((B, S, H, D), 0.31), ramp((B, KV, H, D), 0.17), ramp((B, KV, H, D), 0.53)
    bias = ramp((H, S, KV), 0.07)
    mask = np.array([[1, 1, 1, 0, 0], [1, 0, 0, 0, 0]], np.float32)
    want = np.zeros((B, S, H, D), np.float32)
    st("stock_attention", addr(q), addr(k), addr(v), addr(want), B, H, S, KV, D, 1.0, addr(bias),
       addr(mask), F32, F32, 0, 1)
    got = empty((B, S, H, D), bf16=False)
    call("bh_attention", P(dev(q)), P(dev(k)), P(dev(v)), P(got), B, H, S, KV, D, 1.0, P(dev(bias)),
         P(dev(mask)), F32, F32, None)
    # reference tolerance for fp32 device kernels (test_cuda_ops.cpp:50)
    assert np.max(np.abs(host(got, want) - want)) < 2e-5


# ---- norm and the fused norm + modulate ---------------------------------------------------

@pytest.mark.parametrize("rows,cols", [(37, 1152), (8, 100), (3, 4608), (1, 8)])
def test_norm_matches_oracle(hip, rows, cols):
    x = randn_bf16(RNG, (rows, cols), 2.0)
    x[0, :] = to_bf16(np.float32(3.0) + ramp((cols,), 0.01))  # a nearly constant row
    for rms in (0, 1):
        want = np.zeros_like(x)
        st("stock_norm", addr(x), None, None, addr(want), rows, cols, 1e-6, rms, BF16, 1)
        got = empty((rows, cols))
        call("bh_norm", P(dev(x)), None, None, P(got), rows, cols, 1e-6, rms, 0, 0, BF16, None)
        s = assert_within(from_bf16(host(got, want)), from_bf16(want), "norm", f"{rows}x{cols} rms={rms}")
        assert s["mismatch_frac"] <= 1e-4, s


def test_norm_affine_and_unsupported_groupnorm_refused(hip):
    import burnisher_amd as bh
    rows, cols = 5, 64
    x, w, b = randn_bf16(RNG, (rows, cols)), randn_bf16(RNG, (cols,)), randn_bf16(RNG, (cols,))
    want = np.zeros_like(x)
    st("stock_norm", addr(x), addr(w), addr(b), addr(want), rows, cols, 1e-6, 0, BF16, 1)
    got = empty((rows, cols))
    call("bh_norm", P(dev(x)), P(dev(w)), P(dev(b)), P(got), rows, cols, 1e-6, 0, 0, 0, BF16, None)
    assert np.array_equal(host(got, want), want)
    # the lane-dense kernel (1152 channels) with weight and bias, LayerNorm and RMSNorm
    x2, w2, b2 = randn_bf16(RNG, (9, 1152), 1.5), randn_bf16(RNG, (1152,)), randn_bf16(RNG, (1152,))
    for rms in (0, 1):
        want = np.zeros_like(x2)
        st("stock_norm", addr(x2), addr(w2), addr(b2), addr(want), 9, 1152, 1e-6, rms, BF16, 1)
        got = empty((9, 1152))
        call("bh_norm", P(dev(x2)), P(dev(w2)), P(dev(b2)), P(got), 9, 1152, 1e-6, rms, 0, 0, BF16, None)
        s = assert_within(from_bf16(host(got, want)), from_bf16(want), "norm", f"affine 9x1152 rms={rms}")
        assert s["mismatch_frac"] <= 1e-4, s
    # GroupNorm runs where its channel split fits the kernel (tests/test_gpu_vae.py); 4 channels
    # do not (channels % 8 != 0) and are refused with a sentence, not run approximately
    with pytest.raises(bh.BurnisherError, match="groupnorm"):
        call("bh_norm", P(dev(x)), None, None, P(got), 1, rows * cols, 1e-6, 0, 4, 4, BF16, None)


@pytest.mark.parametrize("tokens", [1024, 77])
def test_norm_modulate_matches_oracle_sequence(hip, tokens):
    B, C = 2, 1152
    x = randn_bf16(RNG, (B * tokens, C), 1.5)
    mod, table = randn_bf16(RNG, (B, 6 * C), 0.5), randn_bf16(RNG, (6, C), 0.5)
    normed, shift, scale, want = (np.zeros(s, np.uint16) for s in ((B * tokens, C), (B, C), (B, C), (B * tokens, C)))
    # the reference block's op sequence, pixart_dit.cpp:226-231 (chunks 3/4: the MLP half)
    st("stock_norm", addr(x), None, None, addr(normed), B * tokens, C, 1e-6, 0, BF16, 0)
    st("stock_chunk", addr(mod), addr(table), addr(shift), B, C, 6, 3, 3, BF16)
    st("stock_chunk", addr(mod), addr(table), addr(scale), B, C, 6, 4, 4, BF16)
    st("stock_modulate", addr(normed), addr(scale), addr(shift), addr(want), B, tokens, C, None, None, BF16)
    got = empty((B * tokens, C))
    call("bh_norm_modulate", P(dev(x)), P(dev(mod)), 6, 3, 4, P(dev(table)), 3, 4, P(got), B, tokens, C,
         1e-6, None)
    s = assert_within(from_bf16(host(got, want)), from_bf16(want), "norm_modulate", str(tokens))
    assert s["mismatch_frac"] <= 1e-4, s


# ---- elementwise --------------------------------------------------------------------------

@pytest.mark.parametrize("C", [1152, 12])
def test_modulate_matches_oracle(hip, C):
    B, T = 2, 33
    x, res = randn_bf16(RNG, (B, T, C)), randn_bf16(RNG, (B, T, C))
    sc, sh, gt = (randn_bf16(RNG, (B, C), 0.3) for _ in range(3))
    for r, g in ((None, None), (res, gt)):
        want = np.zeros_like(x)
        st("stock_modulate", addr(x), addr(sc), addr(sh), addr(want), B, T, C, addr(r), addr(g), BF16)
        got = empty((B, T, C))
        call("bh_modulate", P(dev(x)), P(dev(sc)), P(dev(sh)), P(got), B, T, C, P(dev(r)), P(dev(g)), BF16, None)
        assert np.array_equal(host(got, want), want)
    # in place on the residual, as the graph calls it (pixart_dit.cpp:249)
    zero = np.zeros((B, C), np.uint16)
    want = res.copy()
    st("stock_modulate", addr(x), addr(zero), addr(zero), addr(want), B, T, C, addr(want), addr(gt), BF16)
    dres = dev(res)
    call("bh_modulate", P(dev(x)), P(dev(zero)), P(dev(zero)), P(dres), B, T, C, P(dres), P(dev(gt)), BF16, None)
    assert np.array_equal(host(dres, want), want)


def test_add_chunk_activation_patch(hip):
    B, T, C = 2, 40, 1152
    a, b, row = randn_bf16(RNG, (B, T * C)), randn_bf16(RNG, (B, T * C)), randn_bf16(RNG, (T * C,))
    for bb, bc in ((b, 0), (row, 1)):
        want = np.zeros_like(a)
        st("stock_add", addr(a), addr(bb), addr(want), B, T * C, 1.0, bc, BF16)
        got = empty((B, T * C))
        call("bh_add", P(dev(a)), P(dev(bb)), P(got), B, T * C, 1.0, bc, BF16, None)
        assert np.array_equal(host(got, want), want)
        # in place on a (the graph's residual add), with a scale
        want = np.zeros_like(a)
        st("stock_add", addr(a), addr(bb), addr(want), B, T * C, -0.5, bc, BF16)
        da = dev(a)
        call("bh_add", P(da), P(dev(bb)), P(da), B, T * C, -0.5, bc, BF16, None)
        assert np.array_equal(host(da, want), want)
    # rows that are not whole 16-byte vectors take the element-wise kernel
    a3, b3 = randn_bf16(RNG, (3, 36)), randn_bf16(RNG, (36,))
    want = np.zeros_like(a3)
    st("stock_add", addr(a3), addr(b3), addr(want), 3, 36, 1.0, 1, BF16)
    got = empty((3, 36))
    call("bh_add", P(dev(a3)), P(dev(b3)), P(got), 3, 36, 1.0, 1, BF16, None)
    assert np.array_equal(host(got, want), want)
    mod, table, emb, out_table = (randn_bf16(RNG, s) for s in ((B, 6 * C), (6, C), (B, C), (2, C)))
    for m, t, chunks, chunk, trow in ((mod, table, 6, 2, 2), (mod, table, 6, 5, -1), (emb, out_table, 1, 0, 1)):
        want = np.zeros((B, C), np.uint16)
        st("stock_chunk", addr(m), addr(t), addr(want), B, C, chunks, chunk, trow, BF16)
        got = empty((B, C))
        call("bh_chunk", P(dev(m)), P(dev(t)), P(got), B, C, chunks, chunk, trow, BF16, None)
        assert np.array_equal(host(got, want), want)
    x = randn_bf16(RNG, (B, C), 3.0)
    for kind in (1, 2):
        want = np.zeros_like(x)
        st("stock_activation", addr(x), addr(want), x.size, kind, None, BF16)
        got = empty((B, C))
        call("bh_activation", P(dev(x)), P(got), x.size, kind, None, BF16, None)
        assert_within(from_bf16(host(got, want)), from_bf16(want), "activation", f"kind={kind}")
    img = randn_bf16(RNG, (2, 4, 32, 32))
    want = np.zeros((2, 256, 16), np.uint16)
    st("stock_patch", addr(img), addr(want), 2, 4, 16, 2, 0, BF16)
    got = empty((2, 256, 16))
    call("bh_patch", P(dev(img)), P(got), 2, 4, 16, 2, 0, BF16, None)
    assert np.array_equal(host(got, want), want)
    tok = randn_bf16(RNG, (2, 256, 32))
    want = np.zeros((2, 8, 32, 32), np.uint16)
    st("stock_patch", addr(tok), addr(want), 2, 8, 16, 2, 1, BF16)
    got = empty((2, 8, 32, 32))
    call("bh_patch", P(dev(tok)), P(got), 2, 8, 16, 2, 1, BF16, None)
    assert np.array_equal(host(got, want), want)


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_scale_matches_oracle(hip, dtype):
    x = ramp((5003,), 0.29) * np.float32(4.0)
    xin = x if dtype == F32 else to_bf16(x)
    want = np.zeros_like(xin)
    st("stock_scale", addr(xin), addr(want), xin.size, 0.18215, dtype)
    got = empty(xin.shape, bf16=dtype == BF16)
    call("bh_scale", P(dev(xin)), P(got), xin.size, 0.18215, dtype, None)
    assert np.array_equal(host(got, want), want)
    # in place
    d = dev(xin)
    call("bh_scale", P(d), P(d), xin.size, 0.18215, dtype, None)
    assert np.array_equal(host(d, want), want)


def test_host_operands_refused_by_every_op(hip):
    # Each op's entry point refuses a host operand with an error before any launch
    # (the reference's require_device, ops_cuda.cu:79-88).
    import burnisher_amd as bh
    lib = bh.lib()
    h = np.zeros(4096, np.uint16)
    d = empty((4096,))
    H, D = h.ctypes.data, P(d)
    cases = {
        "conv2d": lambda: lib.bh_conv2d(H, D, None, D, 1, 4, 4, 4, 4, 3, 1, BF16, None),
        "conv2d out": lambda: lib.bh_conv2d(D, D, None, H, 1, 4, 4, 4, 4, 3, 1, BF16, None),
        "upsample": lambda: lib.bh_upsample(H, D, 1, 4, 4, 4, 2, BF16, None),
        "transpose": lambda: lib.bh_transpose(D, H, 1, 4, 16, 0, BF16, None),
        "repeat": lambda: lib.bh_repeat(H, D, 2, 16, BF16, None),
        "guidance": lambda: lib.bh_guidance(D, H, 8, 4, 16, 4.5, BF16, None),
        "scale": lambda: lib.bh_scale(H, D, 16, 2.0, BF16, None),
        "timestep": lambda: lib.bh_timestep_embedding(1.0, 8, 1, H, BF16, None),
        "modulate": lambda: lib.bh_modulate(D, D, H, D, 1, 4, 4, None, None, BF16, None),
    }
    for name, fn in cases.items():
        assert fn() != 0, name
        assert b"HOST" in lib.bh_last_error(), (name, lib.bh_last_error())


def test_contract_errors(hip):
    import burnisher_amd as bh
    host_a = np.zeros((4, 8), np.uint16)
    d = empty((4, 8))
    with pytest.raises(bh.BurnisherError, match="HOST pointer|not memory"):
        call("bh_gemm", host_a.ctypes.data, P(d), None, P(d), 4, 4, 8, 1, 0, BF16, None)
    with pytest.raises(bh.BurnisherError, match="GeluGated"):
        call("bh_gemm", P(d), P(d), None, P(d), 4, 4, 8, 1, 3, BF16, None)
    with pytest.raises(bh.BurnisherError, match="dtype"):
        call("bh_add", P(d), P(d), P(d), 4, 8, 1.0, 0, 7, None)
