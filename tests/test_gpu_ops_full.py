"""Each hot op at the exact 1024px dit-step shapes against the stock oracle.

The whole-step gate at full depth cannot see one wrong tile or one wrong head (the summation-order
noise of 28 blocks is as large), so the GEMMs and both attentions are also checked one by one at
the shapes the 1024px step runs: M = 2 x 4096 token rows, hidden 1152, MLP 4608, 16 heads of 72,
4096 image keys and a 300-token caption with per-row prefix masks (75 and 150 live keys). Every
output element is compared, and the attention additionally per (batch, head), so a single wrong
head fails its own gate. Reference: /root/reference/tests/test_cuda_ops.cpp:104-139 (the device
ops against stock at DiT shapes).
"""
import ctypes

import numpy as np
import pytest

import oracle
from helpers import BF16, F32, addr, assert_within, from_bf16, randn_bf16, stats, TOLERANCE

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(20261202)
M, D, DFF, H, DH, S, CAP = 8192, 1152, 4608, 16, 72, 4096, 300


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def back(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def st(name, *args):
    oracle.call(oracle.stock(), name, *args)


@pytest.mark.parametrize("n,k,epi", [(D, D, 0), (3 * D, D, 0), (DFF, D, 1)],
                         ids=["out_proj_1152x1152", "qkv_3456x1152", "ff0_4608x1152_gelu"])
def test_gemm_1024px_shapes(hip, n, k, epi):
    import burnisher_amd as bh
    import torch
    a, b, bias = randn_bf16(RNG, (M, k)), randn_bf16(RNG, (n, k), 0.02), randn_bf16(RNG, (n,), 0.02)
    want = np.zeros((M, n), np.uint16)
    st("stock_gemm", addr(a), addr(b), addr(bias), addr(want), M, n, k, 1, epi, BF16, 0)
    da, db, dbias = dev(a), dev(b), dev(bias)
    out = torch.zeros((M, n), dtype=torch.bfloat16, device="cuda")
    print(f"bh_gemm {M}x{n}x{k} epi={epi}", flush=True)
    bh.call("bh_gemm", da.data_ptr(), db.data_ptr(), dbias.data_ptr(), out.data_ptr(), M, n, k, 1, epi,
            BF16, None)
    s = assert_within(from_bf16(back(out)), from_bf16(want), "gemm", f"{M}x{n}x{k} epi={epi}")
    print(s)


@pytest.mark.parametrize("k,gated", [(DFF, True), (D, False)], ids=["ff2_gated_1152x4608", "cross_out_residual_1152x1152"])
def test_gemm_1024px_residual_epilogues(hip, k, gated):
    # ff2's gated residual x + gate * (h W^T + b) and the cross-attention out-projection's
    # residual add, fused into the GEMM epilogue, against the oracle's separate GEMM + modulate
    # (pixart_dit.cpp:249-283)
    import burnisher_amd as bh
    import torch
    B, N_tok = 2, S
    a, w, bias = randn_bf16(RNG, (M, k)), randn_bf16(RNG, (D, k), 0.02), randn_bf16(RNG, (D,), 0.02)
    x, gate = randn_bf16(RNG, (M, D)), randn_bf16(RNG, (B, D), 0.5)
    proj = np.zeros((M, D), np.uint16)
    st("stock_gemm", addr(a), addr(w), addr(bias), addr(proj), M, D, k, 1, 0, BF16, 0)
    want = x.copy()
    if gated:
        zero = np.zeros((B, D), np.uint16)
        st("stock_modulate", addr(proj), addr(zero), addr(zero), addr(want), B, N_tok, D, addr(want),
           addr(gate), BF16)
    else:
        st("stock_add", addr(want), addr(proj), addr(want), M, D, 1.0, 0, BF16)
    da, dw, db, dx, dg = dev(a), dev(w), dev(bias), dev(x), dev(gate)
    if gated:
        f = bh.GemmFused(epilogue=0, round_mid=1, residual=dx.data_ptr(), gate=dg.data_ptr(), gate_rows=N_tok, ld_out=D)
    else:
        f = bh.GemmFused(epilogue=0, round_mid=1, residual=dx.data_ptr(), ld_out=D)
    print(f"bh_gemm_fused_run {M}x{D}x{k} gated={gated}", flush=True)
    bh.call("bh_gemm_fused_run", da.data_ptr(), dw.data_ptr(), db.data_ptr(), dx.data_ptr(), M, D, k,
            ctypes.byref(f), None)
    s = assert_within(from_bf16(back(dx)), from_bf16(want), "gemm_fused", f"{M}x{D}x{k} gated={gated}")
    print(s)


def per_head_worst(got, want, B, Sq):
    """The worst (batch, head) slice's figures: one wrong head cannot hide behind the others."""
    g = from_bf16(got).reshape(B, Sq, H, DH)
    w = from_bf16(want).reshape(B, Sq, H, DH)
    worst = None
    for b in range(B):
        for h in range(H):
            s = stats(g[b, :, h], w[b, :, h])
            if worst is None or s["rel_l2"] > worst[1]["rel_l2"]:
                worst = ((b, h), s)
    return worst


@pytest.mark.parametrize("cross", [False, True], ids=["self_2x16x4096x4096", "cross_2x16x4096x300_masked"])
def test_attention_1024px_shapes(hip, cross):
    import burnisher_amd as bh
    import torch
    B = 2
    kv = CAP if cross else S
    q = randn_bf16(RNG, (B, S, H, DH))
    k = randn_bf16(RNG, (B, kv, H, DH))
    v = randn_bf16(RNG, (B, kv, H, DH))
    mask = None
    if cross:
        mask = np.zeros((B, kv), np.float32)
        mask[0, :75] = 1.0
        mask[1, :150] = 1.0
    want = np.zeros((B, S, H, DH), np.uint16)
    st("stock_attention", addr(q), addr(k), addr(v), addr(want), B, H, S, kv, DH, 0.0, None,
       addr(mask), F32, BF16, 0, 0)
    dq, dk, dv = dev(q), dev(k), dev(v)
    dm = None if mask is None else torch.from_numpy(mask).cuda()
    out = torch.zeros((B, S, H, DH), dtype=torch.bfloat16, device="cuda")
    print(f"bh_attention B{B} H{H} {S}x{kv} d{DH} cross={cross}", flush=True)
    bh.call("bh_attention", dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), B, H, S, kv, DH,
            0.0, None, None if dm is None else dm.data_ptr(), F32, BF16, None)
    got = back(out)
    s = assert_within(from_bf16(got), from_bf16(want), "attention", f"{S}x{kv} cross={cross}")
    (b, h), ws = per_head_worst(got, want, B, S)
    tol = TOLERANCE["ops"]["attention"]
    print(s, "worst head", (b, h), ws)
    assert ws["max_abs"] <= tol["max_abs"] and ws["rel_l2"] <= tol["rel_l2"] and ws["cosine"] >= tol["cosine"], \
        f"head {(b, h)}: {ws} vs {tol}"


def test_attention_1152px_self_ragged_round(hip):
    # The held-out 1152px self-attention: 2 x 16 heads x 11 query blocks = 352 workgroups on the
    # 256 CUs. Query blocks 0-7 of every head run whole, blocks 8-10 (the last one 64 queries)
    # split their 81 key blocks two ways and are combined: every path of that plan is held to
    # the gate, per head too.
    import burnisher_amd as bh
    import torch
    B, S2 = 2, 5184
    q = randn_bf16(RNG, (B, S2, H, DH))
    k = randn_bf16(RNG, (B, S2, H, DH))
    v = randn_bf16(RNG, (B, S2, H, DH))
    want = np.zeros((B, S2, H, DH), np.uint16)
    st("stock_attention", addr(q), addr(k), addr(v), addr(want), B, H, S2, S2, DH, 0.0, None,
       None, F32, BF16, 0, 0)
    dq, dk, dv = dev(q), dev(k), dev(v)   # held: a freed operand's memory could be reused
    out = torch.zeros((B, S2, H, DH), dtype=torch.bfloat16, device="cuda")
    print(f"bh_attention B{B} H{H} {S2}x{S2} d{DH}", flush=True)
    bh.call("bh_attention", dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), B, H,
            S2, S2, DH, 0.0, None, None, F32, BF16, None)
    got = back(out)
    s = assert_within(from_bf16(got), from_bf16(want), "attention", f"{S2}x{S2}")
    (b, h), ws = per_head_worst(got, want, B, S2)
    tol = TOLERANCE["ops"]["attention"]
    print(s, "worst head", (b, h), ws)
    assert ws["max_abs"] <= tol["max_abs"] and ws["rel_l2"] <= tol["rel_l2"] and ws["cosine"] >= tol["cosine"], \
        f"head {(b, h)}: {ws} vs {tol}"
    # the split query rows and the whole ones, each against the oracle on its own
    for lo, hi in ((0, 8 * 512), (8 * 512, S2)):
        assert_within(from_bf16(got[:, lo:hi]), from_bf16(want[:, lo:hi]), "attention", f"queries {lo}..{hi - 1}")
