"""GPU energy measurement on MI355X through AMD-SMI.

The reference measures energy per request with a ``PowerSampler`` (NVML or a Jetson sysfs
node) whose ``read_watts`` a background thread samples and ``integrate_energy`` integrates
with trapezoids (quantization/crispybits_quant/energy.py:12-93).  This module keeps that
interface -- ``EnergyMeasurement``, ``PowerSampler.read_watts``, ``integrate_energy(fn,
sampler, hz, synchronize)`` -- and adds the sampler for AMD GPUs:

* ``AMDSMIPowerSampler.read_watts`` is the socket power AMD-SMI reports (W);
* ``AMDSMIPowerSampler.read_energy`` is the GPU's hardware energy accumulator (J, with the
  accumulator's own timestamp).  On MI355X that counter advances about once a second, so
  ``steady_energy`` measures a workload by running it back to back for a few seconds and
  dividing the accumulated energy between two counter updates that both fall inside the
  busy window by the time between them: the mean power of the steady state, exact up to the
  counter resolution, which a 50 Hz sample of a slowly refreshed power reading is not.
"""
from __future__ import annotations

from dataclasses import dataclass
from threading import Event, Thread
from time import perf_counter, sleep
from typing import Callable, List, Optional, Tuple


@dataclass
class EnergyMeasurement:
    joules: float
    seconds: float
    samples: int
    mean_watts: float


class PowerSampler:
    def read_watts(self) -> float:
        raise NotImplementedError

    def read_energy(self) -> Tuple[float, float]:
        """(joules accumulated so far, time of the last accumulator update in seconds)."""
        raise NotImplementedError


def _torch_pci_bus(device_index: int) -> Optional[int]:
    try:
        import torch
        return int(torch.cuda.get_device_properties(device_index).pci_bus_id)
    except Exception:               # no torch / no GPU / older torch: fall back to the index
        return None


class AMDSMIPowerSampler(PowerSampler):
    """Socket power and the energy accumulator of one GPU via the ``amdsmi`` package.
    ``device_index`` is the HIP device; the AMD-SMI handle is matched by PCI bus number
    (AMD-SMI enumerates every GPU the node exposes, HIP only the visible ones)."""

    def __init__(self, device_index: int = 0):
        try:
            import amdsmi
        except ImportError as e:
            raise RuntimeError("the amdsmi package (ROCm) is needed for AMD GPU power measurement") from e
        self.smi = amdsmi
        try:
            amdsmi.amdsmi_init(amdsmi.AmdSmiInitFlags.INIT_AMD_GPUS)
            handles = amdsmi.amdsmi_get_processor_handles()
        except Exception as e:      # the library's own exception types: no driver, no permission
            raise RuntimeError(f"AMD-SMI initialisation failed: {e}") from e
        if not handles:
            raise RuntimeError("AMD-SMI sees no GPU")
        bus = _torch_pci_bus(device_index)
        self.handle = None
        if bus is not None:
            for h in handles:
                bdf = amdsmi.amdsmi_get_gpu_device_bdf(h)          # "dddd:bb:dd.f"
                if int(bdf.split(":")[1], 16) == bus:
                    self.handle = h
                    break
        if self.handle is None:
            if device_index >= len(handles):
                raise RuntimeError(f"AMD-SMI has {len(handles)} GPU(s), no device {device_index}")
            self.handle = handles[device_index]

    def read_watts(self) -> float:
        info = self.smi.amdsmi_get_power_info(self.handle)
        for key in ("current_socket_power", "average_socket_power", "socket_power"):
            v = info.get(key)
            if isinstance(v, (int, float)) and v > 0:
                return float(v)
        raise RuntimeError(f"AMD-SMI reports no socket power: {info}")

    def read_energy(self) -> Tuple[float, float]:
        e = self.smi.amdsmi_get_energy_count(self.handle)
        return e["energy_accumulator"] * e["counter_resolution"] * 1e-6, e["timestamp"] * 1e-9

    def close(self):
        self.smi.amdsmi_shut_down()


class _PowerTrace:
    """Power readings taken every ``period`` seconds on a daemon thread, one before the
    window opens and one after it closes, so the window's edges can be interpolated."""

    def __init__(self, sampler: PowerSampler, period: float):
        self.sampler, self.period = sampler, period
        self.t: List[float] = []
        self.w: List[float] = []
        self._stop = Event()
        self._thread = Thread(target=self._run, daemon=True)

    def _read(self):
        w = self.sampler.read_watts()
        self.t.append(perf_counter())
        self.w.append(w)

    def _run(self):
        while not self._stop.wait(self.period):
            self._read()

    def __enter__(self):
        self._read()
        self._thread.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        self._thread.join()
        self._read()
        return False

    def energy(self, t0: float, t1: float) -> float:
        """Trapezoid integral of the readings over [t0, t1], the edge powers interpolated
        between the readings around them (held at the nearest reading beyond the ends)."""
        import numpy as np
        t, w = np.asarray(self.t), np.asarray(self.w)
        inside = (t > t0) & (t < t1)
        ts = np.concatenate(([t0], t[inside], [t1]))
        ws = np.concatenate(([np.interp(t0, t, w)], w[inside], [np.interp(t1, t, w)]))
        return float(np.trapezoid(ws, ts))


def integrate_energy(fn: Callable[[], None], sampler: PowerSampler, hz: float = 50.0,
                     synchronize: Optional[Callable[[], None]] = None) -> EnergyMeasurement:
    """Energy of one call of ``fn`` from its power readings at ``hz`` (the reference's
    integrate_energy interface, quantization/crispybits_quant/energy.py:50-93): the window
    runs from after a first ``synchronize`` to after the last one; the readings inside it,
    plus the powers at its two edges interpolated from the readings around them, are
    integrated with the trapezoid rule.  ``samples`` counts the readings inside the window."""
    if synchronize:
        synchronize()
    with _PowerTrace(sampler, 1.0 / hz) as trace:
        t0 = perf_counter()
        fn()
        if synchronize:
            synchronize()
        t1 = perf_counter()
    joules = trace.energy(t0, t1)
    inside = sum(1 for t in trace.t if t0 < t < t1)
    return EnergyMeasurement(joules, t1 - t0, inside + 2, joules / max(t1 - t0, 1e-12))


def steady_energy(step: Callable[[], None], sampler: PowerSampler, seconds: float = 4.0, settle: float = 1.1,
                  synchronize: Optional[Callable[[], None]] = None, poll: float = 0.02) -> EnergyMeasurement:
    """Mean power and energy per call of ``step`` in steady state, from the energy accumulator.

    ``step`` is enqueued back to back for ``seconds`` (the device stays busy: the host blocks
    when the queue is full) while a thread polls ``read_energy``.  The window runs from the
    first accumulator update seen at least ``settle`` seconds after the start (so it happened
    after the start) to the last update seen before the final synchronize; its energy over
    its duration is the mean power.  ``joules`` is the energy of one step (mean power times the
    wall time per step), ``samples`` the number of steps, ``seconds`` the counter window."""
    stop = Event()
    reads: List[Tuple[float, float, float]] = []              # (host time, joules, counter time)

    def worker():
        while not stop.is_set():
            j, ts = sampler.read_energy()
            reads.append((perf_counter(), j, ts))
            sleep(poll)

    if synchronize:
        synchronize()
    th = Thread(target=worker, daemon=True)
    t0 = perf_counter()
    th.start()
    steps = 0
    while perf_counter() - t0 < seconds:
        step()
        steps += 1
    t_enq = perf_counter()
    if synchronize:
        synchronize()
    t1 = perf_counter()
    stop.set()
    th.join()
    inside = [r for r in reads if t0 + settle <= r[0] <= min(t_enq, t1)]
    updates = []
    for r in inside:
        if not updates or r[2] != updates[-1][2]:
            updates.append(r)
    if len(updates) < 2:
        raise RuntimeError(f"the energy counter did not advance twice in the busy window "
                           f"({len(updates)} updates in {t1 - t0:.2f} s); run longer")
    (_, ja, ta), (_, jb, tb) = updates[0], updates[-1]
    watts = (jb - ja) / (tb - ta)
    per_step = (t1 - t0) / steps
    return EnergyMeasurement(watts * per_step, tb - ta, steps, watts)
