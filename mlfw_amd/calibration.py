"""Calibration observers on the device, behind the reference's interface.

Mirrors src/compiler/analysis/calibration.ts: a ValueObserver keeps the
running min / max / count of one float value and, when a histogram is
enabled, a HistogramCollector; a CalibrationCollector holds one observer per value and
hands out a CalibrationResult whose get_quant_params() turns the observed
range into static activation quantization parameters (minmax, percentile
0.999 or KL entropy).

The state of every observer lives in device memory (libq8hip.so,
q8_observer_*): update() enqueues four kernels on torch's current stream and
never synchronises; reading min / max / the histogram back synchronises.
Threshold and parameter selection run on the host inside the library
(q8_hist_percentile, q8_hist_entropy, q8_calib_params), as the reference
runs them on the CPU.

Values are keyed by any hashable (the reference keys them by graph Value;
this module has no graph IR, so callers name them).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib as L

MODES = {"minmax": L.Q8_CALIB_MINMAX, "percentile": L.Q8_CALIB_PERCENTILE,
         "entropy": L.Q8_CALIB_ENTROPY}
SCHEMES = {"per_tensor_symmetric": L.Q8_SCHEME_PER_TENSOR_SYMMETRIC,
           "per_tensor_asymmetric": L.Q8_SCHEME_PER_TENSOR_ASYMMETRIC,
           "per_channel": L.Q8_SCHEME_PER_CHANNEL}
DEFAULT_BINS = 2048     # enableHistogram(numBins = 2048), calibration.ts:36


def _stream() -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


@dataclass
class HistogramCollector:
    """A read-back HistogramCollector (calibration.ts:41-56): bins, range,
    total count.  The thresholds are computed by the library."""
    num_bins: int
    bins: np.ndarray
    range_min: float
    range_max: float
    initialized: bool
    total_count: float
    _summary: np.ndarray

    def compute_percentile_threshold(self, percentile: float) -> float:
        """computePercentileThreshold (calibration.ts:130-141)."""
        t = C.c_double()
        L.call("q8_hist_percentile", _dptr(self._summary), _dptr(self.bins), float(percentile),
               C.byref(t))
        return t.value

    def compute_entropy_threshold(self, num_quant_bins: int) -> float:
        """computeEntropyThreshold (calibration.ts:143-187)."""
        t = C.c_double()
        L.call("q8_hist_entropy", _dptr(self._summary), _dptr(self.bins), int(num_quant_bins),
               C.byref(t))
        return t.value


class ValueObserver:
    """ValueObserver (calibration.ts:11-39) with its state in device memory."""

    def __init__(self, device: torch.device | str | None = None):
        self.device = torch.device(device) if device is not None else \
            torch.device("cuda", torch.cuda.current_device())
        self._num_bins = 1
        self._hist = False
        self._state = None
        self._reset()

    def _reset(self) -> None:
        n = C.c_size_t()
        L.call("q8_observer_state_bytes", self._num_bins, C.byref(n))
        # int64 storage keeps the buffer 8-byte aligned (torch's allocator
        # aligns far more, but the dtype states the requirement)
        self._state = torch.empty((n.value + 7) // 8, dtype=torch.int64, device=self.device)
        with torch.cuda.device(self.device):
            L.call("q8_observer_reset", C.c_void_p(self._state.data_ptr()), self._num_bins,
                   int(self._hist), _stream())

    def enable_histogram(self, num_bins: int = DEFAULT_BINS) -> None:
        """enableHistogram (calibration.ts:36-38).  The device observer starts
        the histogram together with min / max, so this is allowed only before
        the first update (the reference's CalibrationCollector enables it right after
        construction)."""
        if self.count:
            raise ValueError("enable_histogram: the observer has already seen data")
        if not 1 <= num_bins <= L.Q8_OBS_MAX_BINS:
            raise ValueError(f"enable_histogram: num_bins must be in [1, {L.Q8_OBS_MAX_BINS}]")
        self._num_bins = int(num_bins)
        self._hist = True
        self._reset()

    def update(self, data: torch.Tensor) -> None:
        """update(data) (calibration.ts:24-34) on a float32 device tensor."""
        if not isinstance(data, torch.Tensor) or data.dtype != torch.float32:
            raise TypeError("ValueObserver.update: data must be a float32 tensor")
        if data.device != self.device:
            raise ValueError(f"ValueObserver.update: data is on {data.device}, "
                             f"the observer on {self.device}")
        data = data.contiguous()
        with torch.cuda.device(self.device):
            L.call("q8_observer_update", C.c_void_p(self._state.data_ptr()),
                   C.c_void_p(data.data_ptr()), data.numel(), _stream())

    def read(self, with_bins: bool = True):
        """Synchronise and return (summary[9], bins or None)."""
        summary = np.zeros(L.Q8_OBS_SUMMARY, np.float64)
        bins = np.zeros(self._num_bins, np.float64) if (with_bins and self._hist) else None
        with torch.cuda.device(self.device):
            L.call("q8_observer_read", C.c_void_p(self._state.data_ptr()), _dptr(summary),
                   _dptr(bins) if bins is not None else None, _stream())
        return summary, bins

    @property
    def min(self) -> float:
        return float(self.read(False)[0][0])

    @property
    def max(self) -> float:
        return float(self.read(False)[0][1])

    @property
    def count(self) -> float:
        return float(self.read(False)[0][2])

    @property
    def histogram(self) -> HistogramCollector | None:
        if not self._hist:
            return None
        s, b = self.read(True)
        return HistogramCollector(int(s[8]), b, float(s[5]), float(s[6]), bool(s[4]),
                                  float(s[7]), s)


class CalibrationResult:
    """CalibrationResult (calibration.ts:231-279)."""

    def __init__(self, observers: dict, mode: str):
        self._observers = observers
        self._mode = mode

    def get_range(self, value):
        """getRange: {'min', 'max'} or None when nothing was observed."""
        obs = self._observers.get(value)
        if obs is None:
            return None
        s, _ = obs.read(False)
        if s[2] == 0:
            return None
        return {"min": float(s[0]), "max": float(s[1])}

    def get_quant_params(self, value, scheme: str = "per_tensor_symmetric", dtype: str = "i8"):
        """getQuantParams (calibration.ts:246-268) -> {'scale', 'zero_point',
        'scheme', 'dtype'} or None."""
        if scheme not in SCHEMES:
            raise ValueError(f"get_quant_params: unknown scheme {scheme!r}")
        if dtype not in ("i8", "ui8"):
            raise ValueError(f"get_quant_params: dtype must be 'i8' or 'ui8' (got {dtype!r})")
        obs = self._observers.get(value)
        if obs is None:
            return None
        s, b = obs.read(self._mode != "minmax")
        scale, zp, ok = C.c_double(), C.c_double(), C.c_int()
        L.call("q8_calib_params", _dptr(s), _dptr(b) if b is not None else None,
               MODES[self._mode], SCHEMES[scheme], int(dtype == "ui8"), C.byref(scale),
               C.byref(zp), C.byref(ok))
        if not ok.value:
            return None
        return {"scale": scale.value, "zero_point": zp.value, "scheme": scheme, "dtype": dtype}

    def has_data(self, value) -> bool:
        obs = self._observers.get(value)
        return obs is not None and obs.count > 0

    def values(self):
        return iter(self._observers.keys())


class CalibrationCollector:
    """CalibrationCollector (calibration.ts:188-229): one observer per float value;
    histograms for the 'entropy' and 'percentile' modes."""

    def __init__(self, mode: str = "minmax", device: torch.device | str | None = None):
        if mode not in MODES:
            raise ValueError(f"CalibrationCollector: unknown mode {mode!r}")
        self.mode = mode
        self.device = device
        self.observers: dict = {}

    def attach(self, values) -> None:
        """attach(func): creates an observer for every named float value."""
        for v in values:
            obs = ValueObserver(self.device)
            if self.mode in ("entropy", "percentile"):
                obs.enable_histogram()
            self.observers[v] = obs

    def observe(self, value, data: torch.Tensor) -> None:
        obs = self.observers.get(value)
        if obs is not None:
            obs.update(data)

    def get_result(self) -> CalibrationResult:
        return CalibrationResult(self.observers, self.mode)
