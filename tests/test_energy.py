"""Energy measurement (crispybits_kernels.energy): the reference's trapezoid integration
(quantization/crispybits_quant/energy.py:50-93) and the steady-state accumulator method,
on synthetic samplers whose true energy is known; the AMD-SMI sampler on the GPU."""
import time

import pytest

from crispybits_kernels import energy as E


class ConstantPower(E.PowerSampler):
    def __init__(self, watts):
        self.watts = watts

    def read_watts(self):
        return self.watts


class SteppedCounter(E.PowerSampler):
    """An accumulator that, like MI355X's, advances only every ``period`` seconds."""
    def __init__(self, watts, period):
        self.watts, self.period, self.t0 = watts, period, time.perf_counter()

    def read_energy(self):
        t = time.perf_counter() - self.t0
        tq = (t // self.period) * self.period
        return self.watts * tq, tq


def test_integrate_constant_power():
    m = E.integrate_energy(lambda: time.sleep(0.2), ConstantPower(100.0), hz=200)
    assert m.seconds == pytest.approx(0.2, abs=0.05)
    assert m.joules == pytest.approx(100.0 * m.seconds, rel=1e-9)
    assert m.mean_watts == pytest.approx(100.0) and m.samples >= 3


def test_steady_energy_with_a_coarse_counter():
    m = E.steady_energy(lambda: time.sleep(0.002), SteppedCounter(250.0, 0.1), seconds=0.8, settle=0.15)
    assert m.mean_watts == pytest.approx(250.0, rel=1e-6)
    assert m.joules == pytest.approx(250.0 * 0.8 / m.samples, rel=0.1)
    assert m.seconds >= 0.2


def test_steady_energy_needs_two_updates():
    with pytest.raises(RuntimeError, match="did not advance twice"):
        E.steady_energy(lambda: time.sleep(0.002), SteppedCounter(250.0, 10.0), seconds=0.2, settle=0.05)


@pytest.mark.gpu
def test_amdsmi_sampler_reads_the_gpu():
    import torch
    try:
        s = E.AMDSMIPowerSampler(0)
    except RuntimeError as e:
        pytest.skip(f"AMD-SMI unavailable on this box: {e}")
    try:
        w = s.read_watts()
        assert 10.0 < w < 3000.0
        x = torch.randn(4096, 4096, device="cuda", dtype=torch.float16)
        m = E.steady_energy(lambda: x @ x, s, seconds=3.0, synchronize=torch.cuda.synchronize)
        assert 50.0 < m.mean_watts < 3000.0 and m.joules > 0 and m.samples > 10
    finally:
        s.close()


class RampPower(E.PowerSampler):
    """Power rising linearly in time: the trapezoid rule with interpolated edges is exact."""
    def __init__(self, w0, slope):
        self.w0, self.slope, self.t0 = w0, slope, time.perf_counter()

    def read_watts(self):
        return self.w0 + self.slope * (time.perf_counter() - self.t0)


def test_integrate_linear_ramp_exactly():
    s = RampPower(50.0, 400.0)
    start = time.perf_counter() - s.t0
    m = E.integrate_energy(lambda: time.sleep(0.25), s, hz=100)
    end = time.perf_counter() - s.t0
    L = m.seconds

    def ramp(a):                              # energy of the ramp over [a, a + L]
        return 50.0 * L + 200.0 * ((a + L) ** 2 - a ** 2)

    # the window [t0, t0 + L] lies inside [start, end]; the energy grows with t0
    assert ramp(start) * (1 - 1e-6) <= m.joules <= ramp(end - L) * (1 + 1e-6)
    assert m.samples >= 10
