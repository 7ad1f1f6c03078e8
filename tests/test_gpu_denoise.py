"""The denoise loop on the device: bh_repeat, bh_guidance and bh_sched_step against the oracle
(bit for bit: all three are exact restatements of the reference's double arithmetic), the
golden trajectories of /root/reference/tests/test_scheduler.cpp:111-137 through the device
sampler, and bh_denoiser_run -- eager and as a replayed HIP graph -- against the reference's own
loop structure (pipeline.cpp:110-131: repeat, DiT forward, guidance, then the sampler on host
copies), built here from the same engine plus the oracle's guidance and sampler."""
import ctypes

import numpy as np
import pytest

import burnisher_amd as bh
import oracle
from burnisher_amd.workload import make_workload
from helpers import BF16, F32, HostSampler, addr, to_bf16
from test_gpu_dit import SMALL, Engine

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16 if a.dtype == np.uint16
                                                          else a.dtype)).cuda()


def host(t, like):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy().view(like.dtype).reshape(like.shape)


def enc(dtype):
    return (lambda v: np.asarray(v, np.float32)) if dtype == F32 else to_bf16


def same_bits(got, want) -> bool:
    """Bit-identical, except that a NaN matches any NaN: the host and the GPU produce NaNs of
    different sign and payload (a schedule without lower_order_final divides by h = inf on its
    last step, in the reference as here)."""
    def nan(a):
        if a.dtype == np.uint16:
            return (a & 0x7FFF) > 0x7F80
        return np.isnan(a)
    gn, wn = nan(got), nan(want)
    if not np.array_equal(gn, wn):
        return False
    g = got.view(np.uint16 if got.dtype == np.uint16 else np.uint32)
    w = want.view(np.uint16 if want.dtype == np.uint16 else np.uint32)
    return bool(np.array_equal(g[~gn], w[~wn]))


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("outer,inner", [(1, 1), (2, 7), (3, 5), (2, 4 * 64 * 64), (2, 16384 + 3)])
def test_repeat_matches_oracle(hip, stock, dtype, outer, inner):
    print(f"repeat dtype={dtype} outer={outer} inner={inner}", flush=True)
    x = enc(dtype)(np.random.default_rng(inner).standard_normal(inner))
    want = np.zeros(outer * inner, x.dtype)
    oracle.call(stock, "stock_repeat", addr(x), addr(want), outer, inner, dtype)
    dx, dy = dev(x), dev(np.zeros_like(want))
    bh.call("bh_repeat", dx.data_ptr(), dy.data_ptr(), outer, inner, dtype, None)
    assert np.array_equal(host(dy, want), want)


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("scale", [0.0, 1.0, 4.5, -2.25])
def test_guidance_matches_oracle(hip, stock, dtype, scale):
    oc, ch, sp = 8, 4, 32 * 32 + 5
    print(f"guidance dtype={dtype} scale={scale}", flush=True)
    pred = enc(dtype)(np.random.default_rng(5).standard_normal(2 * oc * sp) * 2)
    want = np.zeros(ch * sp, pred.dtype)
    oracle.call(stock, "stock_guidance", addr(pred), addr(want), oc, ch, sp, scale, dtype)
    dp, do = dev(pred), dev(np.zeros_like(want))
    bh.call("bh_guidance", dp.data_ptr(), do.data_ptr(), oc, ch, sp, scale, dtype, None)
    assert np.array_equal(host(do, want), want)


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_guidance_matches_oracle_at_bf16_ties(hip, stock, dtype):
    # 4M outputs at an irregular scale: the fp64 combine is inexact in float, so a few dozen
    # floats land exactly on a bf16 tie, where one fused f64 -> bf16 rounding and the reference's
    # two roundings (f64 -> f32 -> bf16) disagree.
    oc, ch, sp = 8, 4, 1024 * 1024
    pred = enc(dtype)(np.random.default_rng(11).standard_normal(2 * oc * sp) * 2)
    want = np.zeros(ch * sp, pred.dtype)
    oracle.call(stock, "stock_guidance", addr(pred), addr(want), oc, ch, sp, 4.1, dtype)
    dp, do = dev(pred), dev(np.zeros_like(want))
    bh.call("bh_guidance", dp.data_ptr(), do.data_ptr(), oc, ch, sp, 4.1, dtype, None)
    got = host(do, want)
    assert np.array_equal(got, want), f"{np.sum(got != want)} of {want.size} differ"


class DeviceSampler:
    def __init__(self, steps, **overrides):
        self.h = ctypes.c_void_p()
        self.cfg = bh.SchedConfig.pinned(**overrides)
        bh.call("bh_sched_create", ctypes.byref(self.cfg), ctypes.byref(self.h))
        bh.call("bh_sched_set_timesteps", self.h, steps)

    def step(self, eps_dev, i, sample_dev, n, dtype):
        bh.call("bh_sched_step", self.h, eps_dev.data_ptr(), i, sample_dev.data_ptr(), n, dtype,
                None)

    def close(self):
        if self.h:
            bh.lib().bh_sched_destroy(self.h)
            self.h = ctypes.c_void_p()


def run_both(dtype, n, steps, seed, overrides=None, check_each=True):
    """The device sampler and the oracle over the same inputs; returns the final samples."""
    overrides = overrides or {}
    import oracle as o
    rng = np.random.default_rng(seed)
    e_ = enc(dtype)
    x = e_(rng.standard_normal(n))
    ref = HostSampler(o.stock(), "stock", steps=steps, **overrides)
    d = DeviceSampler(steps, **overrides)
    try:
        dx = dev(x)
        for i in range(steps):
            e = e_(rng.standard_normal(n))
            ref.step(e, i, x, dtype)
            d.step(dev(e), i, dx, n, dtype)
            if check_each or i == steps - 1:
                assert same_bits(host(dx, x), x), f"step {i} of {steps}"
    finally:
        d.close()
        ref.close()
    return x


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("steps,overrides", [
    (20, {}), (1, {}), (2, {}), (20, dict(lower_order_final=0)), (8, dict(solver_order=1)),
    (8, dict(solver_order=3)),
])
def test_sched_step_matches_oracle(hip, dtype, steps, overrides):
    print(f"sched dtype={dtype} steps={steps} {overrides}", flush=True)
    run_both(dtype, 4 * 128 * 128 + 7, steps, seed=steps, overrides=overrides)


def test_sched_golden_trajectory_on_device(hip):
    """test_scheduler.cpp:111-137 through the device sampler."""
    import math
    d = DeviceSampler(20)
    try:
        x = dev(np.array([math.sin(j * 0.7) for j in range(4)], np.float32))
        golden = {0: [-0.636623, 0.446139, 1.087361, 1.016999],
                  1: [-1.606111, 0.176379, 1.302189, 1.331266],
                  10: [-52.355724, -10.762326, 18.087229, 24.356478],
                  19: [-147.538956, -29.536594, 52.469440, 70.689590]}
        for i in range(20):
            e = np.array([math.cos(j * 0.3 + i * 0.11) for j in range(4)], np.float32)
            d.step(dev(e), i, x, 4, F32)
            if i in golden:
                got = host(x, np.zeros(4, np.float32))
                for j, w in enumerate(golden[i]):
                    assert abs(got[j] - w) <= 1e-3 * max(1.0, abs(w)), (i, j, got[j], w)
    finally:
        d.close()


def test_sched_reset_and_reuse(hip):
    """A reset forgets the history: the next step is first order, as on a fresh sampler."""
    import oracle as o
    n = 1000
    rng = np.random.default_rng(9)
    x = to_bf16(rng.standard_normal(n))
    e = to_bf16(rng.standard_normal(n))
    d = DeviceSampler(10)
    ref = HostSampler(o.stock(), "stock", steps=10)
    try:
        dx = dev(x)
        for i in range(3):
            ref.step(e, i, x, BF16)
            d.step(dev(e), i, dx, n, BF16)
        bh.call("bh_sched_reset", d.h)
        ref.reset()
        for i in range(3, 6):
            ref.step(e, i, x, BF16)
            d.step(dev(e), i, dx, n, BF16)
        assert np.array_equal(host(dx, x), x)
    finally:
        d.close()
        ref.close()


# ---- the whole loop -------------------------------------------------------------------------


def reference_loop(engine, latent0, steps, scale, caption=None):
    """pipeline.cpp:110-131 as the reference runs it: repeat -> DiT forward -> guidance on the
    device engine's output, then the sampler on host copies (here the oracle's guidance and
    sampler, which the tests above pin to the device ops bit for bit)."""
    import torch
    import oracle as o
    wl = engine.wl
    C, hw = wl.cfg["in_channels"], wl.latent_hw
    oc = wl.cfg["out_channels"]
    sampler = HostSampler(o.stock(), "stock", steps=steps)
    lat = latent0.copy()
    try:
        for i in range(steps):
            batched = np.tile(lat, (2, 1, 1, 1))
            engine.latent.view(torch.int16).copy_(torch.from_numpy(batched.view(np.int16)).cuda())
            pred = engine.forward(timestep=float(sampler.timestep(i)), caption=caption)
            eps = np.zeros((C, hw * hw), np.uint16)
            o.call(o.stock(), "stock_guidance", addr(pred), addr(eps), oc, C, hw * hw, scale, BF16)
            flat = lat.reshape(-1)
            sampler.step(eps.reshape(-1), i, flat, BF16)
            lat = flat.reshape(lat.shape)
    finally:
        sampler.close()
    return lat


class Denoiser:
    def __init__(self, engine, steps, scale, guided=True):
        self.sched = DeviceSampler(steps)
        self.h = ctypes.c_void_p()
        bh.call("bh_denoiser_create", engine.handle, self.sched.h, int(guided), scale,
                ctypes.byref(self.h))
        self.engine = engine

    def run(self, latent_dev, graph, caption=None, mask=None):
        e = self.engine
        bh.call("bh_denoiser_run", self.h, latent_dev.data_ptr(),
                (e.caption if caption is None else caption).data_ptr(),
                (e.mask if mask is None else mask).data_ptr(), F32, int(graph), None)

    def close(self):
        if self.h:
            bh.lib().bh_denoiser_destroy(self.h)
            self.h = ctypes.c_void_p()
        self.sched.close()


def small_engine():
    wl = make_workload(SMALL, batch=2, latent_hw=8, caption_len=5)
    return Engine(wl, 0)


def test_denoiser_matches_reference_loop(hip):
    print("denoiser eager vs reference loop, small config, 6 steps", flush=True)
    e = small_engine()
    d = Denoiser(e, 6, 4.5)
    try:
        C, hw = SMALL["in_channels"], e.wl.latent_hw
        latent0 = to_bf16(np.random.default_rng(1).standard_normal((1, C, hw, hw)))
        want = reference_loop(e, latent0, 6, 4.5)
        lat = dev(latent0)
        d.run(lat, graph=False)
        assert np.array_equal(host(lat, latent0), want)
    finally:
        d.close()
        e.close()


def test_denoiser_recomputes_a_new_caption(hip):
    """Steps after the first reuse the caption branch of step 0; a new caption (or new caption
    contents) in the next run is projected afresh."""
    import torch
    print("denoiser with two captions, small config", flush=True)
    e = small_engine()
    d = Denoiser(e, 4, 3.0)
    try:
        C, hw = SMALL["in_channels"], e.wl.latent_hw
        latent0 = to_bf16(np.random.default_rng(4).standard_normal((1, C, hw, hw)))
        other = to_bf16(np.random.default_rng(5).standard_normal(tuple(e.caption.shape)))
        cap2 = torch.from_numpy(other.view(np.int16)).cuda()
        lat = dev(latent0)
        d.run(lat, graph=False)
        lat2 = dev(latent0)
        d.run(lat2, graph=False, caption=cap2)
        assert np.array_equal(host(lat2, latent0), reference_loop(e, latent0, 4, 3.0, caption=cap2))
        # Same pointer, new contents, through the graph.
        g = dev(latent0)
        d.run(g, graph=True)
        assert np.array_equal(host(g, latent0), host(lat, latent0))
        e.caption.view(torch.int16).copy_(cap2)
        g.copy_(torch.from_numpy(latent0.view(np.int16)).cuda())
        d.run(g, graph=True)
        assert np.array_equal(host(g, latent0), host(lat2, latent0))
    finally:
        d.close()
        e.close()


def test_denoiser_graph_replays_equal_eager(hip):
    """The captured loop, replayed several times with eager work in between, gives the eager
    loop's latent bit for bit every time; a new binding or schedule is captured afresh."""
    import torch
    print("denoiser graph vs eager, small config", flush=True)
    e = small_engine()
    d = Denoiser(e, 5, 4.5)
    try:
        C, hw = SMALL["in_channels"], e.wl.latent_hw
        rng = np.random.default_rng(2)
        starts = [to_bf16(rng.standard_normal((1, C, hw, hw))) for _ in range(3)]
        eager = []
        for s in starts:
            lat = dev(s)
            d.run(lat, graph=False)
            eager.append(host(lat, s))
        g = dev(starts[0])
        for rep in range(3):
            for k, s in enumerate(starts):
                g.copy_(torch.from_numpy(s.view(np.int16)).cuda())
                d.run(g, graph=True)
                assert np.array_equal(host(g, s), eager[k]), (rep, k)
                # Eager work between replays.
                other = dev(starts[(k + 1) % 3])
                d.run(other, graph=False)
                assert np.array_equal(host(other, s), eager[(k + 1) % 3])
        # A new schedule invalidates the capture.
        bh.call("bh_sched_set_timesteps", d.sched.h, 3)
        lat = dev(starts[0])
        d.run(lat, graph=False)
        want3 = host(lat, starts[0])
        g.copy_(torch.from_numpy(starts[0].view(np.int16)).cuda())
        d.run(g, graph=True)
        assert np.array_equal(host(g, starts[0]), want3)
    finally:
        d.close()
        e.close()


def test_denoiser_graph_with_row_split(hip):
    """With the CFG rows on two streams, the loop captures the second stream through the engine's
    fork/join events: eager and replayed runs equal the single-stream loop bit for bit."""
    import torch
    print("denoiser graph vs eager with split rows, small config", flush=True)
    e = small_engine()
    d = Denoiser(e, 4, 4.5)
    try:
        C, hw = SMALL["in_channels"], e.wl.latent_hw
        rng = np.random.default_rng(7)
        starts = [to_bf16(rng.standard_normal((1, C, hw, hw))) for _ in range(2)]
        want = []
        for s in starts:
            lat = dev(s)
            d.run(lat, graph=False)
            want.append(host(lat, s))
        g = dev(starts[0])
        d.run(g, graph=True)   # captured with the rows joined
        bh.call("bh_dit_set_rows", e.handle, bh.ROWS_SPLIT)
        lat = dev(starts[0])
        d.run(lat, graph=False)
        assert np.array_equal(host(lat, starts[0]), want[0])
        for rep in range(3):   # a new schedule is captured afresh, then replayed
            for k, s in enumerate(starts):
                g.copy_(torch.from_numpy(s.view(np.int16)).cuda())
                d.run(g, graph=True)
                assert np.array_equal(host(g, s), want[k]), (rep, k)
                other = dev(starts[1 - k])
                d.run(other, graph=False)
                assert np.array_equal(host(other, s), want[1 - k]), (rep, k)
    finally:
        d.close()
        e.close()


def test_denoiser_rejects_mismatched_batch(hip):
    e = small_engine()
    s = DeviceSampler(4)
    try:
        h = ctypes.c_void_p()
        assert bh.lib().bh_denoiser_create(e.handle, s.h, 0, 1.0, ctypes.byref(h)) != 0
        assert b"negative prompt" in bh.lib().bh_last_error()
    finally:
        s.close()
        e.close()
