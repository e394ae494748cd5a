"""Calibration observers (src/compiler/analysis/calibration.ts).

CPU part:
  * the oracle's ValueObserver / HistogramCollector is pinned by the
    reference's own known answers (tests/compiler/analysis/calibration.test.js),
    by bins worked out by hand for small batches (first-batch range, range
    expansion with re-bucketing by centres, NaN / empty batches), by a closed
    form of the 0.999 percentile, and by an independent brute force of the
    KL threshold (numpy add.reduceat + scipy.special.rel_entr);
  * the library's host-side scale selection (q8_hist_percentile,
    q8_hist_entropy, q8_calib_params) must equal the oracle on read-back
    states; fromRange is pinned by closed forms.
GPU part (marked gpu): the device observer (q8_observer_*) against the oracle
on batch sequences, bit for bit (min / max up to the sign of zero).
"""
import ctypes as C
import math
import zlib

import numpy as np
import pytest

from mlfw_amd import _lib as L


def f32(*v):
    return np.array(v, np.float32)


def summary_of(o, num_bins, histogram=True):
    """The q8_observer_read summary layout built from an oracle observer."""
    st = o.state
    return np.array([st["min"], st["max"], st["count"], float(histogram), st["initialized"],
                     st["range_min"], st["range_max"], st["total_count"], num_bins], np.float64)


# ------------------------------------------------------------ oracle pinning

def test_reference_known_answers(oracle):
    # calibration.test.js:5-16 -- expansion does not double count
    o = oracle.Observer(16)
    o.update(f32(0, 1, 2, 3))
    assert o.state["total_count"] == 4
    o.update(f32(0, 1, 100, 2))
    st = o.state
    assert st["total_count"] == 8 and st["bins"].sum() == 8
    # calibration.test.js:18-26 -- in-range batches count once
    o = oracle.Observer(8)
    o.update(f32(0, 10))
    o.update(f32(1, 2, 3))
    st = o.state
    assert st["total_count"] == 5 and st["bins"].sum() == 5


def test_bins_by_hand(oracle):
    o = oracle.Observer(16)
    o.update(f32(0, 1, 2, 3))
    # range [0,3], scale 16/3: 0->0, 1->5, 2->10, 3->min(15, 16)
    exp = np.zeros(16)
    exp[[0, 5, 10, 15]] = 1
    st = o.state
    assert (st["range_min"], st["range_max"]) == (0.0, 3.0)
    assert np.array_equal(st["bins"], exp)
    o.update(f32(0, 1, 100, 2))
    # new range [0,100], scale 0.16; old centres 0.09375, 1.03125, 1.96875,
    # 2.90625 all land in bin 0; the batch: 0,1,2 -> bin 0, 100 -> bin 15
    exp = np.zeros(16)
    exp[0], exp[15] = 7, 1
    st = o.state
    assert (st["range_min"], st["range_max"]) == (0.0, 100.0)
    assert np.array_equal(st["bins"], exp)
    assert (st["min"], st["max"], st["count"]) == (0.0, 100.0, 8)


def test_constant_nan_and_empty_batches(oracle):
    # a constant first batch gets range [c, c+1]
    o = oracle.Observer(4)
    o.update(f32(2, 2, 2))
    st = o.state
    assert (st["range_min"], st["range_max"]) == (2.0, 3.0)
    assert np.array_equal(st["bins"], [3, 0, 0, 0])
    # NaN counts, is never binned and never moves min / max or the range
    o.update(f32(np.nan, 2.5, np.nan))
    st = o.state
    assert np.array_equal(st["bins"], [3, 0, 1, 0])
    assert (st["count"], st["total_count"], st["min"], st["max"]) == (6, 6, 2.0, 2.5)
    # an empty or all-NaN FIRST batch leaves an inverted range: the
    # histogram never bins again (range <= 0), the observer still counts
    for first in (f32(), f32(np.nan, np.nan)):
        o = oracle.Observer(4)
        o.update(first)
        o.update(f32(1, 2))
        st = o.state
        assert st["initialized"] == 1 and st["range_min"] == math.inf and st["range_max"] == -math.inf
        assert st["bins"].sum() == 0 and st["total_count"] == 0
        assert st["count"] == first.size + 2 and (st["min"], st["max"]) == (1.0, 2.0)


def test_no_histogram_observer(oracle):
    o = oracle.Observer(8, histogram=False)
    o.update(f32(-3, 1, 7))
    st = o.state
    assert (st["min"], st["max"], st["count"], st["initialized"]) == (-3.0, 7.0, 3, 0)
    assert st["bins"].sum() == 0
    assert o.params("percentile") == o.params("minmax") == (7.0 / 127.0, 0.0)
    assert oracle.Observer(8).params("minmax") is None          # getRange -> null


def test_percentile_closed_form(oracle):
    # values 0..2047 over range [0, 2047]: bin(v) = floor(v * 2048/2047) = v
    # for v < 2047 and 2047 -> 2047, one value per bin.  cum(i) = i + 1 >=
    # 0.999 * 2048 = 2045.952 first at i = 2045 -> threshold 2046 * 2047/2048
    o = oracle.Observer(2048)
    o.update(np.arange(2048, dtype=np.float32))
    assert np.array_equal(o.state["bins"], np.ones(2048))
    assert o.percentile(0.999) == 2046 * (2047 / 2048)
    assert o.percentile(1.0) == 2048 * (2047 / 2048)
    assert o.percentile(0.0) == 1 * (2047 / 2048)


def entropy_brute(bins, total, lo, hi, nq):
    """computeEntropyThreshold restated with numpy reduceat + scipy rel_entr."""
    from scipy.special import rel_entr
    nb = bins.size
    ref = bins / total
    best_t, best = nb, math.inf
    for t in range(nq, nb + 1):
        edges = np.floor(np.arange(nq + 1) * (t / nq)).astype(np.int64)
        edges = np.minimum(edges, t)
        starts = edges[:-1]
        counts = edges[1:] - starts
        keep = counts > 0
        sums = np.add.reduceat(ref[:t], starts[keep]) if keep.any() else np.zeros(0)
        q = np.zeros(t)
        for a, c, sm in zip(starts[keep], counts[keep], sums):
            q[a:a + c] = sm / c
        m = (ref[:t] > 0) & (q > 0)
        kl = float(np.sum(rel_entr(ref[:t][m], q[m])))
        if kl < best:
            best, best_t = kl, t
    return lo + best_t * ((hi - lo) / nb), best_t


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_entropy_brute_force(oracle, seed):
    rng = np.random.default_rng(seed)
    nb, nq = 96, 15
    o = oracle.Observer(nb)
    x = rng.standard_normal(4000).astype(np.float32)
    x[:5] *= 8                                    # a long tail worth clipping
    o.update(x)
    st = o.state
    thr, best_t = entropy_brute(st["bins"], st["total_count"], st["range_min"], st["range_max"], nq)
    assert nq <= best_t <= nb
    assert o.entropy(nq) == pytest.approx(thr, rel=0, abs=1e-12)


def test_entropy_exact_fit_picks_first_threshold(oracle):
    # all mass in the first nq bins: t = nq reproduces the histogram exactly
    # (KL 0) and a later t can only tie, so the threshold is lo + nq * w
    nb, nq = 64, 8
    o = oracle.Observer(nb)
    o.update(np.concatenate([np.arange(8, dtype=np.float32) + 0.5, f32(64.0)]))
    st = o.state
    w = (st["range_max"] - st["range_min"]) / nb
    assert st["bins"][:8].sum() == 8 and st["bins"][63] == 1
    thr = o.entropy(nq)
    # with the outlier in bin 63 no t < 64 sees it, so KL = 0 from t = nq on
    assert thr == st["range_min"] + nq * w


def test_from_range_closed_forms(oracle):
    o = oracle.Observer(8, histogram=False)
    o.update(f32(-1, 3))
    assert o.params("minmax", "per_tensor_symmetric") == (3 / 127, 0.0)
    s, z = o.params("minmax", "per_tensor_asymmetric")
    assert s == 4 / 255 and z == -64.0                 # round(-128 + 63.75)
    assert o.params("minmax", "per_channel") == (s, z)  # fromRange's non-symmetric branch
    s, z = o.params("minmax", "per_tensor_asymmetric", unsigned=True)
    assert s == 4 / 255 and z == 64.0                  # round(0 + 63.75)
    zero = oracle.Observer(8, histogram=False)
    zero.update(f32(0, 0))
    assert zero.params("minmax") == (1e-10, 0.0)       # absMax / bound || 1e-10


# ------------------------------------------- library host side vs the oracle

@pytest.fixture(scope="module")
def lib():
    L.load()
    return L


def lib_params(summary, bins, mode, scheme, unsigned=False):
    s, z, ok = C.c_double(), C.c_double(), C.c_int()
    L.call("q8_calib_params", summary.ctypes.data_as(C.c_void_p),
           None if bins is None else bins.ctypes.data_as(C.c_void_p),
           mode, scheme, int(unsigned), C.byref(s), C.byref(z), C.byref(ok))
    return (s.value, z.value) if ok.value else None


SCHEME_IDS = {"per_tensor_symmetric": 0, "per_tensor_asymmetric": 1, "per_channel": 2}
MODE_IDS = {"minmax": 0, "percentile": 1, "entropy": 2}


@pytest.mark.parametrize("seed", [0, 1])
def test_library_host_scale_selection_matches_oracle(oracle, lib, seed):
    rng = np.random.default_rng(seed)
    nb = 512
    o = oracle.Observer(nb)
    for k in range(4):
        x = (rng.standard_normal(3000) * (1 + k)).astype(np.float32)
        x[rng.integers(0, x.size, 3)] *= 20
        o.update(x)
    st = o.state
    summ = summary_of(o, nb)
    bins = st["bins"].copy()
    t = C.c_double()
    L.call("q8_hist_percentile", summ.ctypes.data_as(C.c_void_p), bins.ctypes.data_as(C.c_void_p),
           0.999, C.byref(t))
    assert t.value == o.percentile(0.999)
    for nq in (255, 256):
        L.call("q8_hist_entropy", summ.ctypes.data_as(C.c_void_p),
               bins.ctypes.data_as(C.c_void_p), nq, C.byref(t))
        assert t.value == o.entropy(nq)
    for mode in MODE_IDS:
        for scheme in SCHEME_IDS:
            for u in (False, True):
                assert same_params(lib_params(summ, bins, MODE_IDS[mode], SCHEME_IDS[scheme], u),
                                   o.params(mode, scheme, u)), (mode, scheme, u)


def test_library_calib_params_edge_cases(lib):
    empty = np.array([math.inf, -math.inf, 0, 1, 0, 0, 0, 0, 16], np.float64)
    assert lib_params(empty, np.zeros(16), 1, 0) is None           # nothing observed
    # minmax never needs the bins
    s = np.array([-2.0, 1.0, 5, 0, 0, 0, 0, 0, 1], np.float64)
    assert lib_params(s, None, 0, 0) == (2 / 127, 0.0)
    # percentile on an observer without histogram falls back to min / max
    assert lib_params(s, None, 1, 0) == (2 / 127, 0.0)
    # percentile with a histogram but no bins is refused
    sh = s.copy()
    sh[3] = 1
    rc = L.load().q8_calib_params(sh.ctypes.data_as(C.c_void_p), None, 1, 0, 0,
                                  C.byref(C.c_double()), C.byref(C.c_double()),
                                  C.byref(C.c_int()))
    assert rc == L.Q8_ERR_INVALID
    rc = L.load().q8_calib_params(s.ctypes.data_as(C.c_void_p), None, 7, 0, 0,
                                  C.byref(C.c_double()), C.byref(C.c_double()),
                                  C.byref(C.c_int()))
    assert rc == L.Q8_ERR_INVALID
    n = C.c_size_t()
    assert L.load().q8_observer_state_bytes(0, C.byref(n)) == L.Q8_ERR_INVALID
    assert L.load().q8_observer_state_bytes(L.Q8_OBS_MAX_BINS + 1, C.byref(n)) == L.Q8_ERR_INVALID
    L.call("q8_observer_state_bytes", 2048, C.byref(n))
    assert n.value == 128 + 16 * 2048
    assert L.load().q8_observer_reset(None, 16, 1, None) == L.Q8_ERR_INVALID
    assert L.load().q8_observer_update(C.c_void_p(0x1000), None, 5, None) == L.Q8_ERR_INVALID


# ---------------------------------------------------------- device observer

def batches_for(case, rng):
    if case == "normal_growing":
        return [(rng.standard_normal(n) * (1 + i)).astype(np.float32)
                for i, n in enumerate([5000, 70000, 3, 300001])]
    if case == "expansions_each_side":
        return [f32(0, 1, 2, 3), f32(0, 1, 100, 2), f32(-50, 7), f32(-1e3, 1e3, 0.5),
                rng.uniform(-1e3, 1e3, 100003).astype(np.float32)]
    if case == "nan_and_empty":
        b = rng.standard_normal(9999).astype(np.float32)
        b[::7] = np.nan
        return [f32(), f32(np.nan), b, f32(), (b * 3).astype(np.float32)]
    if case == "constant_first":
        return [np.full(1000, 2.5, np.float32), rng.standard_normal(4096).astype(np.float32)]
    if case == "outliers":
        x = rng.standard_normal(1 << 20).astype(np.float32)
        x[rng.integers(0, x.size, 100)] *= 50
        return [x, x[::3].copy(), -x[:77777]]
    if case == "infinite":
        return [f32(1, 2, np.inf), f32(-np.inf, 0.5), rng.standard_normal(1000).astype(np.float32)]
    raise KeyError(case)


CASES = ["normal_growing", "expansions_each_side", "nan_and_empty", "constant_first", "outliers",
         "infinite"]


def same_params(a, b):
    """(scale, zero_point) pairs equal as numbers, NaN equal to NaN."""
    if a is None or b is None:
        return a is b
    return all(x == y or (math.isnan(x) and math.isnan(y)) for x, y in zip(a, b))


def assert_same_state(dev_sum, dev_bins, o, nb, hist):
    st = o.state
    # min / max equal as numbers (the sign of a zero may differ), NaN-free
    assert dev_sum[0] == st["min"] and dev_sum[1] == st["max"], (dev_sum[:2], st["min"], st["max"])
    assert dev_sum[2] == st["count"]
    assert dev_sum[3] == float(hist) and dev_sum[8] == nb
    assert dev_sum[4] == st["initialized"]
    for k, key in ((5, "range_min"), (6, "range_max")):
        a, b = dev_sum[k], st[key]
        assert (a == b) or (math.isnan(a) and math.isnan(b)), (key, a, b)
    assert dev_sum[7] == st["total_count"]
    if hist:
        bad = np.nonzero(dev_bins != st["bins"])[0]
        assert bad.size == 0, f"{bad.size} bins differ, first {bad[:5]}: " \
                              f"{dev_bins[bad[:5]]} vs {st['bins'][bad[:5]]}"


@pytest.mark.gpu
@pytest.mark.parametrize("nb", [2048, 1, 8192, 100])
@pytest.mark.parametrize("case", CASES)
def test_device_observer_matches_oracle(oracle, case, nb):
    import torch
    from mlfw_amd.calibration import ValueObserver
    print(f"[calib] case={case} nb={nb}", flush=True)
    rng = np.random.default_rng(zlib.crc32(case.encode()))
    obs = ValueObserver("cuda:0")
    obs.enable_histogram(nb)
    o = oracle.Observer(nb)
    for b in batches_for(case, rng):
        obs.update(torch.from_numpy(b).to("cuda:0"))
        o.update(b)
        s, bins = obs.read()
        assert_same_state(s, bins, o, nb, True)
    # scale selection through the read-back state
    s, bins = obs.read()
    for mode in MODE_IDS:
        for scheme in SCHEME_IDS:
            assert same_params(lib_params(s, bins, MODE_IDS[mode], SCHEME_IDS[scheme]),
                               o.params(mode, scheme)), (mode, scheme)


@pytest.mark.gpu
def test_device_observer_without_histogram_and_collector(oracle):
    import torch
    from mlfw_amd.calibration import CalibrationCollector, ValueObserver
    rng = np.random.default_rng(7)
    obs = ValueObserver("cuda:0")
    o = oracle.Observer(1, histogram=False)
    for n in (1, 17, 1 << 18):
        x = rng.standard_normal(n).astype(np.float32)
        obs.update(torch.from_numpy(x).to("cuda:0"))
        o.update(x)
    s, bins = obs.read()
    assert bins is None
    assert_same_state(s, None, o, 1, False)
    assert obs.histogram is None
    # the collector interface (calibration.ts:188-279)
    for mode in ("minmax", "percentile", "entropy"):
        col = CalibrationCollector(mode, "cuda:0")
        col.attach(["x", "h"])
        ref = oracle.Observer(2048, histogram=mode != "minmax")
        for i in range(3):
            x = (rng.standard_normal(50000) * (i + 1)).astype(np.float32)
            col.observe("x", torch.from_numpy(x).to("cuda:0"))
            col.observe("unknown", torch.from_numpy(x).to("cuda:0"))   # ignored
            ref.update(x)
        res = col.get_result()
        assert res.has_data("x") and not res.has_data("h")
        assert res.get_range("h") is None and res.get_quant_params("h") is None
        r = res.get_range("x")
        assert (r["min"], r["max"]) == (ref.state["min"], ref.state["max"])
        for scheme in SCHEME_IDS:
            for dt in ("i8", "ui8"):
                p = res.get_quant_params("x", scheme, dt)
                assert (p["scale"], p["zero_point"]) == ref.params(mode, scheme, dt == "ui8")
        if mode != "minmax":
            h = col.observers["x"].histogram
            assert h.compute_percentile_threshold(0.999) == ref.percentile(0.999)
            assert h.compute_entropy_threshold(255) == ref.entropy(255)
