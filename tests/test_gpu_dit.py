"""The dit-step engine (bh_dit_create / bh_dit_forward) against the stock oracle's dit-step on
the same seeded weights and inputs, and the reference's graph invariants on the device
(/root/reference/tests/test_models.cpp:274-348)."""
import ctypes
import os

import numpy as np
import pytest

import oracle
from burnisher_amd.workload import PIXART_SIGMA, config_struct, make_workload
from helpers import F32, TOLERANCE, addr, from_bf16, stats

pytestmark = pytest.mark.gpu

SMALL = dict(num_layers=2, num_heads=4, head_dim=8, patch_size=2, in_channels=4, out_channels=8,
             caption_channels=32, sample_size=8, mlp_ratio=4.0, eps=1e-6)
# head_dim 72 with an odd head count: the width (216) is no multiple of 144, so the projections
# do not write V^T and the attention op transposes V into the engine's own buffer.
ODD72 = dict(num_layers=2, num_heads=3, head_dim=72, patch_size=2, in_channels=4, out_channels=8,
             caption_channels=64, sample_size=16, mlp_ratio=4.0, eps=1e-6)


class Engine:
    """A device copy of a workload plus one engine over it."""

    def __init__(self, wl, mode):
        import torch
        import burnisher_amd as bh
        self.wl = wl
        self.top, self.blocks, self.latent, self.caption, self.mask = wl.to_device()
        self.cfg = config_struct(wl.cfg)
        self.w, self._keep = wl.weight_struct(self.top, self.blocks)
        self.handle = ctypes.c_void_p()
        bh.call("bh_dit_create", ctypes.byref(self.cfg), ctypes.byref(self.w), wl.batch, wl.latent_hw,
                wl.caption_len, mode, ctypes.byref(self.handle))
        self.out = torch.zeros((wl.batch, wl.cfg["out_channels"], wl.latent_hw, wl.latent_hw),
                               dtype=torch.bfloat16, device="cuda")

    def forward(self, timestep=None, caption=None, mask=None):
        import torch
        import burnisher_amd as bh
        cap = self.caption if caption is None else caption
        m = self.mask if mask is None else mask
        t = self.wl.timestep if timestep is None else timestep
        bh.call("bh_dit_forward", self.handle, self.latent.data_ptr(), t, cap.data_ptr(), m.data_ptr(),
                F32, self.out.data_ptr(), None)
        torch.cuda.synchronize()
        return self.out.cpu().view(torch.int16).numpy().view(np.uint16).copy()

    def close(self):
        import burnisher_amd as bh
        if self.handle:
            bh.lib().bh_dit_destroy(self.handle)
            self.handle = ctypes.c_void_p()


# The oracle runs on the host's share of cores (16 per GPU on the GPU boxes), whatever the
# machine reports; its result does not depend on the thread count.
THREADS = min(16, os.cpu_count() or 1)


def oracle_forward(wl, layers=-1):
    cfg = config_struct(wl.cfg)
    w, keep = wl.weight_struct(wl.top, wl.blocks)
    out = np.zeros((wl.batch, wl.cfg["out_channels"], wl.latent_hw, wl.latent_hw), np.uint16)
    oracle.call(oracle.stock(), "stock_dit_forward", ctypes.byref(cfg), ctypes.byref(w), wl.batch,
                wl.latent_hw, wl.caption_len, addr(wl.latent), wl.timestep, addr(wl.caption),
                addr(wl.mask), F32, addr(out), THREADS, layers)
    return out


def check_step(got, want, where, gate="dit_step"):
    tol = TOLERANCE[gate]
    s = stats(from_bf16(got), from_bf16(want))
    print(f"dit-step parity {where}: {s}")
    assert np.all(np.isfinite(from_bf16(got))), where
    assert s["max_abs"] <= tol["max_abs"] and s["rel_l2"] <= tol["rel_l2"] and \
        s["cosine"] >= tol["cosine"], f"{where}: {s} vs {tol}"
    return s


@pytest.mark.parametrize("mode", [0, 1], ids=["fused", "opwise"])
def test_small_config_matches_oracle(hip, mode):
    wl = make_workload(SMALL, batch=2, latent_hw=8, caption_len=5)
    e = Engine(wl, mode)
    try:
        got = e.forward()
        check_step(got, oracle_forward(wl), f"small mode={mode}")
        assert np.array_equal(got, e.forward()), "not byte-identical across two forwards"
    finally:
        e.close()


@pytest.mark.parametrize("mode", [0, 1], ids=["fused", "opwise"])
def test_odd_heads_head_dim72_matches_oracle(hip, mode):
    wl = make_workload(ODD72, batch=2, latent_hw=16, caption_len=20)
    e = Engine(wl, mode)
    try:
        check_step(e.forward(), oracle_forward(wl), f"odd72 mode={mode}", gate="dit_block")
    finally:
        e.close()


def test_packed_and_scattered_weights_agree(hip):
    # The fused engine reads Q/K/V and the caption K/V in place when the caller's weights are laid
    # out packed (the checkpoint loader's and the workload's layout) and copies them otherwise:
    # both give the same bytes, and the packed engine holds no copy (3 + 2 d x d per layer less).
    import torch
    import burnisher_amd as bh
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=32, caption_len=120, layers=3)
    packed = Engine(wl, 0)
    scattered = Engine(wl, 0)
    try:
        scattered.close()
        scattered.blocks = [{k: v.clone() for k, v in b.items()} for b in packed.blocks]   # one allocation each
        scattered.w, scattered._keep = wl.weight_struct(scattered.top, scattered.blocks)
        scattered.handle = ctypes.c_void_p()
        bh.call("bh_dit_create", ctypes.byref(scattered.cfg), ctypes.byref(scattered.w), wl.batch,
                wl.latent_hw, wl.caption_len, 0, ctypes.byref(scattered.handle))
        assert np.array_equal(packed.forward(), scattered.forward())
        d = 1152
        saved = bh.lib().bh_dit_workspace_bytes(scattered.handle) - bh.lib().bh_dit_workspace_bytes(packed.handle)
        assert saved == 3 * (5 * d * d + 5 * d) * 2, saved
    finally:
        packed.close()
        scattered.close()


def test_fused_cross_attention_equals_opwise_plan_1024px(hip):
    # At 1024px the fused plan runs each block's cross-attention Q projection and attention as one
    # kernel (cross_fused.hip); it must equal the op-by-op plan's GEMM + attention bit for bit:
    # with the workload's prefix masks (2 and 3 live key blocks of 5), with every key live (5
    # blocks: two resident chunks per head) and with every key masked (the uniform average).
    import torch
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=128, caption_len=300, layers=2)
    a, b = Engine(wl, 0), Engine(wl, 1)
    try:
        for name, mask in (("prefix", None), ("all live", torch.ones_like(a.mask)),
                           ("all masked", torch.zeros_like(a.mask))):
            print(f"cross-attention mask: {name}", flush=True)
            assert np.array_equal(a.forward(mask=mask), b.forward(mask=mask)), name
    finally:
        a.close()
        b.close()


def test_row_schedules_are_bit_identical_1024px(hip):
    # The joined schedule runs the fused cross-attention kernel over both rows; each row of the
    # split schedule is too few tiles for it and runs the GEMM and the attention kernel.
    import burnisher_amd as bh
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=128, caption_len=300, layers=2)
    e = Engine(wl, 0)
    try:
        joined = e.forward()
        bh.call("bh_dit_set_rows", e.handle, bh.ROWS_SPLIT)
        assert np.array_equal(e.forward(), joined)
    finally:
        e.close()


@pytest.mark.parametrize("hw,layers", [(64, 2), (96, 1)], ids=["512px", "768px"])
def test_fused_plan_equals_opwise_plan(hip, hw, layers):
    # Fusion moves no rounding point, so the two plans agree bit for bit (at 768px the fused QKV
    # projection runs 256-row tiles and the separate Q, K and V projections 192-row ones).
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=hw, caption_len=300, layers=layers)
    a, b = Engine(wl, 0), Engine(wl, 1)
    try:
        assert np.array_equal(a.forward(), b.forward())
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("cfg,batch,hw,cap,layers", [
    (PIXART_SIGMA, 2, 64, 300, 2),   # the CFG pair at 512px: one row per stream, head_dim 72
    (SMALL, 3, 8, 5, None),          # groups of two rows and one, the generic attention
    (ODD72, 2, 16, 20, None),        # head_dim 72, V transposed per row group by the attention op
    (PIXART_SIGMA, 2, 144, 128, 1),  # 1152px: the self-attention's last-round query blocks split
], ids=["512px_b2", "small_b3", "odd72_b2", "1152px_b2"])
def test_row_schedules_are_bit_identical(hip, cfg, batch, hw, cap, layers):
    # Rows never mix, so running the two row groups on two streams changes no bit of the output,
    # forward after forward.
    import burnisher_amd as bh
    wl = make_workload(cfg, batch=batch, latent_hw=hw, caption_len=cap, layers=layers)
    e = Engine(wl, 0)
    try:
        joined = e.forward()
        bh.call("bh_dit_set_rows", e.handle, bh.ROWS_SPLIT)
        print(f"split rows, batch {batch}", flush=True)
        for rep in range(2):
            assert np.array_equal(e.forward(), joined), f"split rows, forward {rep}"
        # the caption is read per row group too: a new mask reaches the output under the split
        import torch
        bh.call("bh_dit_set_rows", e.handle, bh.ROWS_JOINED)
        want = e.forward(mask=torch.ones_like(e.mask))
        bh.call("bh_dit_set_rows", e.handle, bh.ROWS_SPLIT)
        assert np.array_equal(e.forward(mask=torch.ones_like(e.mask)), want)
    finally:
        e.close()


def test_row_schedule_refusals(hip):
    import burnisher_amd as bh
    wl = make_workload(SMALL, batch=2, latent_hw=8, caption_len=5)
    fused, opwise = Engine(wl, 0), Engine(wl, 1)
    try:
        with pytest.raises(bh.BurnisherError, match="unknown row schedule"):
            bh.call("bh_dit_set_rows", fused.handle, 2)
        with pytest.raises(bh.BurnisherError, match="op-by-op"):
            bh.call("bh_dit_set_rows", opwise.handle, bh.ROWS_SPLIT)
        bh.call("bh_dit_set_rows", opwise.handle, bh.ROWS_JOINED)
    finally:
        fused.close()
        opwise.close()


def test_two_blocks_512px_matches_oracle(hip):
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=64, caption_len=300, layers=2)
    e = Engine(wl, 0)
    try:
        check_step(e.forward(), oracle_forward(wl), "512px, 2 blocks")
    finally:
        e.close()


def test_one_block_1024px_matches_oracle(hip):
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=128, caption_len=300, layers=1)
    e = Engine(wl, 0)
    try:
        check_step(e.forward(), oracle_forward(wl), "1024px, 1 block", "dit_block")
    finally:
        e.close()


def test_full_depth_512px_matches_oracle(hip):
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=64, caption_len=300)
    e = Engine(wl, 0)
    try:
        check_step(e.forward(), oracle_forward(wl), "512px, 28 blocks")
    finally:
        e.close()


def test_config0_one_block_512px_batch1_caption120(hip):
    # one block, 512px (1024 tokens), batch 1, a 120-token caption.
    wl = make_workload(PIXART_SIGMA, batch=1, latent_hw=64, caption_len=120, layers=1)
    for mode in (0, 1):
        e = Engine(wl, mode)
        try:
            check_step(e.forward(), oracle_forward(wl), f"512px B=1 caption 120, 1 block, mode={mode}",
                       "dit_block")
        finally:
            e.close()


def test_full_depth_1024px_matches_oracle(hip):
    # The headline configuration at full depth against the oracle.
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=128, caption_len=300)
    e = Engine(wl, 0)
    try:
        got = e.forward()
    finally:
        e.close()
    check_step(got, oracle_forward(wl), "1024px, 28 blocks")


def test_one_block_2048px_matches_oracle(hip):
    # BASELINE configs[4]'s shape (16384 image tokens, the long-sequence case), one block.
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=256, caption_len=300, layers=1)
    e = Engine(wl, 0)
    try:
        got = e.forward()
    finally:
        e.close()
    check_step(got, oracle_forward(wl), "2048px, 1 block", "dit_block")


# The reference scores every cell on a resolution and caption length held out from tuning
# (768 or 1152 px, caption 128 or 300: /root/reference/configs/axes.json:10-24,
# eval/bench.py:221-224). 1152px has 2 x 5184 = 10368 token rows, no multiple of the GEMMs'
# 256-row tile, and a 5184-key self-attention whose last 512-query block is ragged.
@pytest.mark.parametrize("hw,cap", [(96, 128), (96, 300), (144, 128), (144, 300)],
                         ids=["768px_cap128", "768px_cap300", "1152px_cap128", "1152px_cap300"])
def test_held_out_shapes_one_block_match_oracle(hip, hw, cap):
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=hw, caption_len=cap, layers=1)
    for mode in (0, 1):
        e = Engine(wl, mode)
        try:
            got = e.forward()
        finally:
            e.close()
        check_step(got, oracle_forward(wl), f"{hw * 8}px caption {cap}, 1 block, mode={mode}", "dit_block")


def test_full_depth_768px_matches_oracle(hip):
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=96, caption_len=300)
    e = Engine(wl, 0)
    try:
        got = e.forward()
    finally:
        e.close()
    check_step(got, oracle_forward(wl), "768px, 28 blocks")


def test_full_depth_1152px_invariants(hip):
    # The held-out 1152px shape at full depth: finite, varied, replayable, timestep- and
    # caption-sensitive, blind to masked caption positions, and the two plans bit-equal.
    import torch
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=144, caption_len=128)
    e = Engine(wl, 0)
    try:
        a = e.forward()
        fa = from_bf16(a)
        assert np.all(np.isfinite(fa)) and fa.std() > 1e-3
        assert np.array_equal(a, e.forward())
        assert np.max(np.abs(fa - from_bf16(e.forward(timestep=100.0)))) > 1e-3
        cap = e.caption.clone()
        for b in range(wl.batch):
            keep = int(wl.mask[b].sum())
            cap[b, keep:, :] = 99.0
        assert np.array_equal(a, e.forward(caption=cap))
        assert np.max(np.abs(fa - from_bf16(e.forward(mask=torch.ones_like(e.mask))))) > 1e-3
    finally:
        e.close()
    o = Engine(wl, 1)
    try:
        assert np.array_equal(a, o.forward()), "fused and op-by-op plans differ at 1152px"
    finally:
        o.close()


def test_full_depth_2048px_invariants(hip):
    # configs[4] at full depth: finite, varied, replayable, timestep- and caption-sensitive, and
    # blind to masked caption positions. (The oracle's full 2048px step is ~100 TFLOP of host
    # work; one block is checked against it above.)
    import torch
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=256, caption_len=300)
    e = Engine(wl, 0)
    try:
        a = e.forward()
        fa = from_bf16(a)
        assert np.all(np.isfinite(fa)) and fa.std() > 1e-3
        assert np.array_equal(a, e.forward())
        assert np.max(np.abs(fa - from_bf16(e.forward(timestep=100.0)))) > 1e-3
        cap = e.caption.clone()
        for b in range(wl.batch):
            keep = int(wl.mask[b].sum())
            cap[b, keep:, :] = 99.0
        assert np.array_equal(a, e.forward(caption=cap))
        assert np.max(np.abs(fa - from_bf16(e.forward(mask=torch.ones_like(e.mask))))) > 1e-3
    finally:
        e.close()


def test_full_depth_1024px_invariants(hip):
    wl = make_workload(PIXART_SIGMA, batch=2, latent_hw=128, caption_len=300)
    e = Engine(wl, 0)
    try:
        a = e.forward()
        fa = from_bf16(a)
        assert np.all(np.isfinite(fa)) and fa.std() > 1e-3
        assert np.array_equal(a, e.forward())
        assert np.max(np.abs(fa - from_bf16(e.forward(timestep=100.0)))) > 1e-3
        # masked caption positions do not reach the output
        import torch
        cap = e.caption.clone()
        for b in range(wl.batch):
            keep = int(wl.mask[b].sum())
            cap[b, keep:, :] = 99.0
        assert np.array_equal(a, e.forward(caption=cap))
        assert np.max(np.abs(fa - from_bf16(e.forward(mask=torch.ones_like(e.mask))))) > 1e-3
    finally:
        e.close()


def test_forward_refuses_host_operands(hip):
    import burnisher_amd as bh
    wl = make_workload(SMALL, batch=2, latent_hw=8, caption_len=5)
    e = Engine(wl, 0)
    try:
        host_latent = np.zeros(wl.latent.size, np.uint16)
        lib = bh.lib()
        assert lib.bh_dit_forward(e.handle, host_latent.ctypes.data, 500.0, e.caption.data_ptr(),
                                  e.mask.data_ptr(), F32, e.out.data_ptr(), None) != 0
        assert b"HOST" in lib.bh_last_error() and b"latent" in lib.bh_last_error()
        host_out = np.zeros(e.out.numel(), np.uint16)
        assert lib.bh_dit_forward(e.handle, e.latent.data_ptr(), 500.0, e.caption.data_ptr(),
                                  e.mask.data_ptr(), F32, host_out.ctypes.data, None) != 0
        assert b"out" in lib.bh_last_error()
        # host weights are refused at create
        cfg = config_struct(wl.cfg)
        w, keep = wl.weight_struct(wl.top, wl.blocks)
        h = ctypes.c_void_p()
        assert lib.bh_dit_create(ctypes.byref(cfg), ctypes.byref(w), 2, 8, 5, 0, ctypes.byref(h)) != 0
        assert b"HOST" in lib.bh_last_error()
    finally:
        e.close()


def test_engine_rejects_bad_geometry(hip):
    import burnisher_amd as bh
    wl = make_workload(SMALL, batch=2, latent_hw=8, caption_len=5)
    top, blocks, *_ = wl.to_device()
    cfg = config_struct(wl.cfg)
    w, keep = wl.weight_struct(top, blocks)
    h = ctypes.c_void_p()
    with pytest.raises(bh.BurnisherError, match="divisible"):
        bh.call("bh_dit_create", ctypes.byref(cfg), ctypes.byref(w), 2, 9, 5, 0, ctypes.byref(h))
    w.t_emb1_w = None
    with pytest.raises(bh.BurnisherError, match="null"):
        bh.call("bh_dit_create", ctypes.byref(cfg), ctypes.byref(w), 2, 8, 5, 0, ctypes.byref(h))
