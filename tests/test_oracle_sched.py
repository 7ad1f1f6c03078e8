"""The denoise loop's oracle -- DPM-Solver++ 2M, repeat and guidance in oracle/stock.cpp -- pinned
against the reference's own known answers and against mathematics that fixes the sampler
independently of any implementation; then the product library's host-side schedule (which needs
no GPU) against the pinned oracle.

Known answers: /root/reference/tests/test_scheduler.cpp (timesteps, orders, the final step's
coefficients, and golden trajectories taken from diffusers' DPMSolverMultistepScheduler at the
pinned configuration). Mathematics: with a model that returns the true noise of a fixed clean
sample, the DPM-Solver++ update is exact -- every step lands on alpha_t*x0 + sigma_t*noise, and
the last on x0 itself -- which fails for any mix-up of the Karras and variance-preserving sigmas,
a wrong sign, a missing term or a step-index slip. Where oracle/_ref exists (the reference's own
dpm_solver.cpp and ops_cpu.cpp compiled here), the oracle must also match it bit for bit.
"""
import ctypes
import math

import numpy as np
import pytest

import burnisher_amd as bh
import oracle
from helpers import BF16, F32, TIMESTEPS_20, HostSampler, addr, coeff_tuple, from_bf16, to_bf16

# ---- the oracle against the reference's known answers -----------------------------------------


def test_timesteps_and_sigmas(stock):
    s = HostSampler(stock, "stock")
    assert s.steps() == 20
    assert [s.timestep(i) for i in range(20)] == TIMESTEPS_20
    sig = [s.sigma(i) for i in range(21)]
    assert all(sig[i] < sig[i - 1] for i in range(1, 20))
    assert sig[20] == 0.0 and sig[0] > 1.0
    # sigma at t=999 of the linear 1e-4..0.02 schedule: prod(1 - beta) = 4.036e-5, so
    # sqrt((1 - acp)/acp) = 157.4 (the value the reference's comments quote as "157").
    assert abs(sig[0] - 157.4) < 0.1
    with pytest.raises(oracle.OracleError):
        s.timestep(20)


def test_orders_and_finiteness(stock):
    """test_scheduler.cpp:36-52: first and last steps first order, the rest second order."""
    s = HostSampler(stock, "stock")
    sample = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    eps = np.array([0.0, 0.1, 0.2, 0.3], np.float32)
    orders = []
    for i in range(20):
        orders.append(s.coefficients(i).order)
        s.step(eps, i, sample, F32)
    assert orders[0] == 1 and orders[-1] == 1
    assert all(o == 2 for o in orders[1:-1])
    assert np.all(np.isfinite(sample))


def test_final_step_reduces_to_x0(stock):
    """test_scheduler.cpp:54-64: exp(-h) is exactly 0 on the last step and alpha_t is 1."""
    s = HostSampler(stock, "stock")
    c = s.coefficients(19)
    assert c.sigma_t == 0.0 and c.exp_neg_h == 0.0
    assert abs(c.alpha_t - 1.0) < 1e-12


# test_scheduler.cpp:111-116, from diffusers' DPMSolverMultistepScheduler.
GOLDEN = {0: [-0.636623, 0.446139, 1.087361, 1.016999],
          1: [-1.606111, 0.176379, 1.302189, 1.331266],
          10: [-52.355724, -10.762326, 18.087229, 24.356478],
          19: [-147.538956, -29.536594, 52.469440, 70.689590]}


def golden_run(step_fn):
    """The golden protocol (test_scheduler.cpp:117-137): x[j] = sin(0.7 j), eps[j] at step i is
    cos(0.3 j + 0.11 i), 20 steps in fp32. Returns the sample after each step."""
    x = np.array([math.sin(j * 0.7) for j in range(4)], np.float32)
    out = []
    for i in range(20):
        e = np.array([math.cos(j * 0.3 + i * 0.11) for j in range(4)], np.float32)
        x = step_fn(e, i, x)
        out.append(x.copy())
    return out


def check_golden(traj):
    for i, want in GOLDEN.items():
        for j in range(4):
            got = float(traj[i][j])
            assert abs(got - want[j]) <= 1e-3 * max(1.0, abs(want[j])), (i, j, got, want[j])


def test_golden_trajectory(stock):
    s = HostSampler(stock, "stock")

    def step(e, i, x):
        s.step(e, i, x, F32)
        return x
    check_golden(golden_run(step))


def test_single_step_and_refusals(stock):
    """test_scheduler.cpp:77-97: one step is first order, zero steps and other samplers refused."""
    s = HostSampler(stock, "stock", steps=1)
    assert s.steps() == 1 and s.coefficients(0).order == 1
    with pytest.raises(oracle.OracleError):
        s.set_timesteps(0)
    for bad in (dict(algorithm_type=b"dpmsolver"), dict(solver_type=b"heun"),
                dict(prediction_type=b"v_prediction"), dict(beta_schedule=b"cosine")):
        with pytest.raises(oracle.OracleError):
            HostSampler(stock, "stock", steps=None, **bad)
    with pytest.raises(oracle.OracleError):
        HostSampler(stock, "stock", timestep_spacing=b"leading")


def test_determinism(stock):
    def run():
        s = HostSampler(stock, "stock", steps=8)
        x = np.sin(np.arange(6) * np.float32(0.7)).astype(np.float32)
        e = np.cos(np.arange(6) * np.float32(0.3)).astype(np.float32)
        for i in range(8):
            s.step(e, i, x, F32)
        return x
    assert np.array_equal(run(), run())


# ---- the oracle against mathematics ---------------------------------------------------------


@pytest.mark.parametrize("steps", [1, 2, 5, 20, 50])
def test_exact_model_lands_on_the_noising_path(stock, steps):
    """With eps the true noise of a fixed x0, the DPM-Solver++ update is exact for both orders:
    x_{i+1} = alpha(t_{i+1}) x0 + sigma_vp(t_{i+1}) noise, and the final sample is x0."""
    rng = np.random.default_rng(7)
    x0 = rng.standard_normal(512)
    noise = rng.standard_normal(512)
    s = HostSampler(stock, "stock", steps=steps)

    def vp(k):
        r = math.sqrt(k * k + 1.0)
        return 1.0 / r, k / r
    a0, sv0 = vp(s.sigma(0))
    x = (a0 * x0 + sv0 * noise).astype(np.float32)
    e = noise.astype(np.float32)
    for i in range(steps):
        s.step(e, i, x, F32)
        a, sv = vp(s.sigma(i + 1))
        want = a * x0 + sv * noise
        assert np.max(np.abs(x - want)) < 2e-5 * (1 + np.max(np.abs(want))), (steps, i)
    assert np.max(np.abs(x - x0)) < 2e-5 * (1 + np.max(np.abs(x0)))


def test_coefficient_identities(stock):
    """exp(-h) is the Karras ratio; alpha^2 + sigma_vp^2 = 1; r0 = h0/h from log sigmas."""
    s = HostSampler(stock, "stock", steps=20)
    sample = np.zeros(4, np.float32)
    for i in range(19):
        c = s.coefficients(i)
        assert abs(c.alpha_t ** 2 + c.sigma_vp_t ** 2 - 1.0) < 1e-12
        assert abs(c.sigma_vp_s0 / c.alpha_s0 - c.sigma_s0) < 1e-9 * c.sigma_s0
        assert c.exp_neg_h == c.sigma_t / c.sigma_s0
        if c.order == 2:
            h = math.log(s.sigma(i) / s.sigma(i + 1))
            h0 = math.log(s.sigma(i - 1) / s.sigma(i))
            assert abs(c.r0 - h0 / h) < 1e-12
        s.step(sample, i, sample.copy(), F32)


def test_repeat_and_guidance_closed_forms(stock):
    rng = np.random.default_rng(3)
    x = to_bf16(rng.standard_normal(37))
    out = np.zeros(3 * 37, np.uint16)
    oracle.call(stock, "stock_repeat", addr(x), addr(out), 3, 37, BF16)
    assert np.array_equal(out.reshape(3, 37), np.tile(x, (3, 1)))
    oc, ch, sp = 8, 4, 33
    pred = to_bf16(rng.standard_normal((2, oc, sp)) * 2)
    got = np.zeros((ch, sp), np.uint16)
    for scale, want in ((0.0, pred[0, :ch]), (1.0, pred[1, :ch])):
        oracle.call(stock, "stock_guidance", addr(pred), addr(got), oc, ch, sp, scale, BF16)
        assert np.array_equal(got, want), scale
    # Any other scale: u + s(c - u) in double, rounded to float, then to bf16.
    u = from_bf16(pred[0, :ch]).astype(np.float64)
    c = from_bf16(pred[1, :ch]).astype(np.float64)
    oracle.call(stock, "stock_guidance", addr(pred), addr(got), oc, ch, sp, 4.5, BF16)
    assert np.array_equal(got, to_bf16((u + 4.5 * (c - u)).astype(np.float32)))


# ---- the oracle against the reference's own code (oracle/_ref) ------------------------------


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("steps,overrides", [
    (20, {}), (1, {}), (2, {}), (3, {}), (25, {}),
    (20, dict(lower_order_final=0)), (10, dict(solver_order=1)), (10, dict(solver_order=3)),
    (15, dict(beta_schedule=b"scaled_linear", beta_start=0.00085, beta_end=0.012)),
])
def test_stock_sampler_matches_reference(stock, ref, dtype, steps, overrides):
    rng = np.random.default_rng(steps + 100 * dtype)
    a = HostSampler(stock, "stock", steps=steps, **overrides)
    b = HostSampler(ref, "ref", steps=steps, **overrides)
    for i in range(steps + 1):
        assert a.sigma(i) == b.sigma(i)
    n = 1000
    enc = (lambda v: v.astype(np.float32)) if dtype == F32 else to_bf16
    xa = enc(rng.standard_normal(n))
    xb = xa.copy()
    for i in range(steps):
        assert a.timestep(i) == b.timestep(i)
        assert coeff_tuple(a.coefficients(i)) == coeff_tuple(b.coefficients(i)), i
        e = enc(rng.standard_normal(n))
        a.step(e, i, xa, dtype)
        b.step(e, i, xb, dtype)
        assert np.array_equal(xa, xb), f"step {i}"
    a.reset()
    b.reset()
    assert a.coefficients(0).order == b.coefficients(0).order == 1


def test_stock_timesteps_match_reference_for_every_count(stock, ref):
    for steps in range(1, 60):
        a = HostSampler(stock, "stock", steps=steps)
        b = HostSampler(ref, "ref", steps=steps)
        assert [a.timestep(i) for i in range(steps)] == [b.timestep(i) for i in range(steps)]
        assert [a.sigma(i) for i in range(steps + 1)] == [b.sigma(i) for i in range(steps + 1)]


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_stock_repeat_guidance_match_reference(stock, ref, dtype):
    rng = np.random.default_rng(11)
    enc = (lambda v: v.astype(np.float32)) if dtype == F32 else to_bf16
    x = enc(rng.standard_normal(4 * 9))
    o1 = np.zeros(2 * x.size, x.dtype)
    o2 = o1.copy()
    oracle.call(stock, "stock_repeat", addr(x), addr(o1), 2, x.size, dtype)
    oracle.call(ref, "ref_repeat", addr(x), addr(o2), 2, x.size, dtype)
    assert np.array_equal(o1, o2)
    oc, ch, sp = 8, 4, 50
    pred = enc(rng.standard_normal(2 * oc * sp) * 3)
    for scale in (0.0, 1.0, 4.5, -1.25, 7.0):
        g1 = np.zeros(ch * sp, x.dtype)
        g2 = g1.copy()
        oracle.call(stock, "stock_guidance", addr(pred), addr(g1), oc, ch, sp, scale, dtype)
        oracle.call(ref, "ref_guidance", addr(pred), addr(g2), oc, ch, sp, scale, dtype)
        assert np.array_equal(g1, g2), scale


# ---- the product's host-side schedule (no GPU needed) ---------------------------------------


class DeviceSampler:
    """bh_sched_* of the product library: schedule and coefficients are host computations."""

    def __init__(self, steps=20, **overrides):
        self.lib = bh.lib()
        self.h = ctypes.c_void_p()
        self.cfg = bh.SchedConfig.pinned(**overrides)
        bh.call("bh_sched_create", ctypes.byref(self.cfg), ctypes.byref(self.h))
        if steps is not None:
            bh.call("bh_sched_set_timesteps", self.h, steps)

    def coefficients(self, i):
        c = bh.SchedCoefficients()
        bh.call("bh_sched_get_coefficients", self.h, i, ctypes.byref(c))
        return c

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.bh_sched_destroy(self.h)


def test_library_default_config_is_the_pinned_one():
    c = bh.SchedConfig()
    bh.lib().bh_sched_config_default(ctypes.byref(c))
    p = bh.SchedConfig.pinned()
    for name, _ in bh.SchedConfig._fields_:
        assert getattr(c, name) == getattr(p, name), name


@pytest.mark.parametrize("steps,overrides", [
    (20, {}), (1, {}), (7, {}), (50, {}), (1000, {}),
    (15, dict(beta_schedule=b"scaled_linear", beta_start=0.00085, beta_end=0.012)),
])
def test_library_schedule_matches_oracle(stock, steps, overrides):
    d = DeviceSampler(steps, **overrides)
    o = HostSampler(stock, "stock", steps=steps, **overrides)
    lib = bh.lib()
    assert lib.bh_sched_steps(d.h) == steps
    assert [lib.bh_sched_timestep(d.h, i) for i in range(steps)] == \
        [o.timestep(i) for i in range(steps)]
    assert [lib.bh_sched_sigma(d.h, i) for i in range(steps + 1)] == \
        [o.sigma(i) for i in range(steps + 1)]
    for i in range(steps):  # fresh history: every step's coefficients at order 1
        assert coeff_tuple(d.coefficients(i)) == coeff_tuple(o.coefficients(i)), i
    assert lib.bh_sched_init_noise_sigma(d.h) == 1.0
    assert lib.bh_sched_timestep(d.h, steps) == -1 and b"range" in lib.bh_last_error()
    assert math.isnan(lib.bh_sched_sigma(d.h, steps + 1))


def test_library_refusals():
    lib = bh.lib()
    for bad in (dict(algorithm_type=b"dpmsolver"), dict(solver_type=b"heun"),
                dict(prediction_type=b"v_prediction"), dict(beta_schedule=b"cosine"),
                dict(solver_order=0)):
        with pytest.raises(bh.BurnisherError):
            DeviceSampler(None, **bad)
    with pytest.raises(bh.BurnisherError, match="linspace"):
        DeviceSampler(20, timestep_spacing=b"trailing")
    d = DeviceSampler(20)
    with pytest.raises(bh.BurnisherError, match="at least one step"):
        bh.call("bh_sched_set_timesteps", d.h, 0)
    with pytest.raises(bh.BurnisherError, match="range"):
        d.coefficients(20)
    # Size-zero ops succeed without touching the device; a bad dtype is refused.
    assert lib.bh_repeat(None, None, 0, 5, BF16, None) == 0
    assert lib.bh_guidance(None, None, 8, 4, 0, 1.0, BF16, None) == 0
    assert lib.bh_repeat(None, None, 2, 5, 7, None) != 0 and b"dtype" in lib.bh_last_error()
    assert lib.bh_guidance(None, None, 4, 8, 5, 1.0, BF16, None) != 0
    assert lib.bh_denoiser_create(None, None, 1, 4.5, ctypes.byref(ctypes.c_void_p())) != 0
