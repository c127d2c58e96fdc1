"""The sampler's correctly rounded binary32 math (gemma4.pas_amd/csrc/
g4s_crmath.h) built for the host: checked against 60-digit mpmath on random
and constructed hard inputs, and against long double on a strided sweep of
all binary32 inputs (the full sweep is tests/native/crmath_sweep.cpp with
stride 1; it found 0 disagreements)."""
import ctypes
import os
from fractions import Fraction

import numpy as np
import pytest

mp = pytest.importorskip("mpmath")
mp.mp.dps = 60
F32 = np.float32
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def cr():
    path = os.path.join(HERE, "native", "build", "libcrmath_host.so")
    if not os.path.exists(path):
        import subprocess
        subprocess.run(["make", "-s", "-C", os.path.join(HERE, "native")], check=True)
    L = ctypes.CDLL(path)
    d, f = ctypes.c_double, ctypes.c_float
    L.t_exp_cr32.restype = f
    L.t_exp_cr32.argtypes = [d, d]
    L.t_exp_diff_cr32.restype = f
    L.t_exp_diff_cr32.argtypes = [f, f]
    L.t_softcap_topk_cr32.restype = f
    L.t_softcap_topk_cr32.argtypes = [f, f]
    L.t_softcap_full_cr32.restype = f
    L.t_softcap_full_cr32.argtypes = [f, f, f]
    L.t_mul_u_p_cr32.restype = f
    L.t_mul_u_p_cr32.argtypes = [d, f]
    L.t_round_dd_f32.restype = f
    L.t_round_dd_f32.argtypes = [d, d]
    L.t_exp_fast_d.restype = d
    L.t_exp_fast_d.argtypes = [d]
    L.t_tanh_fast_d.restype = d
    L.t_tanh_fast_d.argtypes = [d]
    return L


def rn32(v):
    """Correctly rounded binary32 of an mpf (ties to even), with overflow."""
    if v >= mp.mpf(2) ** 128 - mp.mpf(2) ** 103:
        return F32(np.inf)
    if v <= -(mp.mpf(2) ** 128 - mp.mpf(2) ** 103):
        return F32(-np.inf)
    with np.errstate(over="ignore"):
        f = F32(float(v))
    best = None
    for c in (np.nextafter(f, F32(-np.inf)), f, np.nextafter(f, F32(np.inf))):
        if not np.isfinite(c):
            continue
        dist = abs(mp.mpf(float(c)) - v)
        key = (dist, int(np.array(c, F32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return F32(best[1])


def test_fast_paths_within_error_budget(cr):
    rng = np.random.default_rng(1)
    worst_e = worst_t = 0
    for x in rng.uniform(-104, 89, 3000):
        t = mp.exp(mp.mpf(x))
        worst_e = max(worst_e, abs((mp.mpf(cr.t_exp_fast_d(x)) - t) / t))
    for w in np.concatenate([rng.uniform(-0.6, 0.6, 1500), rng.uniform(-25, 25, 1500)]):
        t = mp.tanh(mp.mpf(w))
        if t != 0:
            worst_t = max(worst_t, abs((mp.mpf(cr.t_tanh_fast_d(w)) - t) / t))
    assert worst_e < mp.mpf(2) ** -51  # accept test assumes 2^-50
    assert worst_t < mp.mpf(2) ** -50  # accept test assumes 2^-49 after the cap product


def test_exp_random(cr):
    rng = np.random.default_rng(2)
    for x in np.concatenate([rng.uniform(-104, 89, 2000), rng.uniform(-1e-3, 1e-3, 200)]):
        assert cr.t_exp_cr32(x, 0.0) == rn32(mp.exp(mp.mpf(x))), x


def test_exp_of_binary32_difference(cr):
    rng = np.random.default_rng(3)
    a = rng.normal(0, 10, 1500).astype(F32)
    b = (rng.normal(0, 10, 1500).astype(F32) * F32(1e-9) + a.max()).astype(F32)
    b[:500] = rng.normal(0, 10, 500).astype(F32)
    for ai, bi in zip(a, b):
        exact = mp.exp(mp.mpf(float(ai)) - mp.mpf(float(bi)))
        assert cr.t_exp_diff_cr32(ai, bi) == rn32(exact)


def test_exp_constructed_hard_cases(cr):
    """x = RN64(ln(midpoint)): e^x lies within ~2^-53 of a binary32 midpoint,
    so the binary64 fast path cannot decide and the double-double path must."""
    rng = np.random.default_rng(4)
    hard = 0
    for _ in range(400):
        f = F32(rng.uniform(1e-30, 1e30) ** rng.choice([1, -1]) if rng.random() < 0.5
                else rng.uniform(0.01, 1.0))
        if not np.isfinite(f) or f <= 0:
            continue
        g = np.nextafter(f, F32(np.inf))
        mid = (mp.mpf(float(f)) + mp.mpf(float(g))) / 2
        x = float(mp.log(mid))
        y = cr.t_exp_fast_d(x)
        low = int(np.array(y).view(np.uint64)) & 0x1FFFFFFF
        hard += abs(low - 0x10000000) <= 8
        assert cr.t_exp_cr32(x, 0.0) == rn32(mp.exp(mp.mpf(x))), x
    assert hard > 50  # the fallback really was exercised


def test_exp_edges(cr):
    assert cr.t_exp_cr32(0.0, 0.0) == 1.0
    assert cr.t_exp_cr32(-200.0, 0.0) == 0.0
    assert cr.t_exp_cr32(100.0, 0.0) == np.inf
    assert np.isnan(cr.t_exp_cr32(float("nan"), 0.0))
    # subnormal results round on the 2^-149 grid
    for x in (-88.0, -95.5, -100.0, -103.2, -103.9):
        assert cr.t_exp_cr32(x, 0.0) == rn32(mp.exp(mp.mpf(x)))


def test_exp_try_path_agrees(cr):
    """exp_cr32_try (the branch-free binary64 route the row tables use) gives
    exp_cr32's value whenever it settles an input, and refuses the inputs
    whose result lies too close to a binary32 midpoint (those take the
    double-double route): random differences over the whole range, results
    down to the subnormals, the special cases and constructed hard cases."""
    rng = np.random.default_rng(11)
    n = 200000
    a = np.concatenate([rng.normal(0, 10, n // 2), rng.uniform(-120, 95, n // 2)]).astype(F32)
    b = np.concatenate([rng.normal(0, 10, n // 2), np.zeros(n // 2)]).astype(F32)
    out_t = np.zeros(n, F32)
    out_r = np.zeros(n, F32)
    ok = np.zeros(n, np.int32)
    cr.t_exp_diff_try_bulk.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_long]
    cr.t_exp_diff_try_bulk(a.ctypes.data, b.ctypes.data, out_t.ctypes.data, out_r.ctypes.data,
                           ok.ctypes.data, n)
    settled = ok.astype(bool)
    assert settled.mean() > 0.999
    assert np.array_equal(out_t[settled].view(np.uint32), out_r[settled].view(np.uint32))
    assert (out_r[settled] == 0).any() and (out_r[settled] < np.finfo(F32).tiny).any()
    cr.t_exp_cr32_try.argtypes = [ctypes.c_double, ctypes.c_double, ctypes.POINTER(ctypes.c_float)]
    r = ctypes.c_float()
    for x, want in ((float("nan"), None), (100.0, np.inf), (-200.0, 0.0), (0.0, 1.0)):
        assert cr.t_exp_cr32_try(x, 0.0, ctypes.byref(r)) == 1
        assert (np.isnan(r.value) if want is None else r.value == want)
    refused = 0
    for _ in range(300):
        f = F32(rng.uniform(0.01, 1.0))
        g = np.nextafter(f, F32(np.inf))
        x = float(mp.log((mp.mpf(float(f)) + mp.mpf(float(g))) / 2))
        if cr.t_exp_cr32_try(x, 0.0, ctypes.byref(r)):
            assert r.value == cr.t_exp_cr32(x, 0.0)
        else:
            refused += 1
    assert refused > 30


def test_softcap_random_and_hard(cr):
    rng = np.random.default_rng(5)
    inv = F32(1.0) / F32(30.0)
    xs = np.concatenate([rng.normal(0, 12, 1500), rng.normal(0, 0.01, 200),
                         rng.uniform(-400, 400, 200)]).astype(F32)
    for x in xs:
        a = mp.mpf(float(x))
        assert cr.t_softcap_topk_cr32(x, 30.0) == rn32(30 * mp.tanh(a / 30)), x
        assert cr.t_softcap_full_cr32(x, inv, 30.0) == rn32(mp.tanh(a * mp.mpf(float(inv))) * 30), x
    for cap in (1.0, 5.5, 50.0):
        for x in rng.normal(0, cap, 200).astype(F32):
            a = mp.mpf(float(x))
            assert cr.t_softcap_topk_cr32(x, cap) == rn32(cap * mp.tanh(a / cap))
    assert cr.t_softcap_topk_cr32(np.inf, 30.0) == 30.0
    assert cr.t_softcap_topk_cr32(-np.inf, 30.0) == -30.0


def test_mul_u_p_exact(cr):
    rng = np.random.default_rng(6)
    for _ in range(3000):
        u = float(rng.integers(0, 2**32)) / 2**32
        p = F32(rng.choice([0.8, 0.9, 0.95, 0.99, 1.0, rng.random()]))
        exact = Fraction(u) * Fraction(float(p))
        assert cr.t_mul_u_p_cr32(u, p) == rn32(mp.mpf(exact.numerator) / exact.denominator)


def test_round_dd_midpoints(cr):
    one = 1.0
    mid = 1.0 + 2.0 ** -24  # midpoint of 1 and 1+2^-23
    assert cr.t_round_dd_f32(mid, 0.0) == F32(1.0)  # tie -> even
    assert cr.t_round_dd_f32(mid, 1e-30) == np.nextafter(F32(1.0), F32(2.0))
    assert cr.t_round_dd_f32(mid, -1e-30) == F32(1.0)
    mid3 = 1.0 + 3 * 2.0 ** -24  # midpoint of 1+2^-23 and 1+2^-22 (even is the upper)
    assert cr.t_round_dd_f32(mid3, 0.0) == F32(1.0 + 2 ** -22)
    assert cr.t_round_dd_f32(mid3, -1e-30) == F32(1.0 + 2 ** -23)
    big = 2.0 ** 128 - 2.0 ** 103
    assert cr.t_round_dd_f32(big, -1.0) == np.finfo(F32).max
    assert cr.t_round_dd_f32(big, 1.0) == np.inf
    assert cr.t_round_dd_f32(one, 0.0) == F32(1.0)


def test_strided_sweep_vs_long_double():
    path = os.path.join(HERE, "native", "build", "libcrmath_sweep.so")
    L = ctypes.CDLL(path)
    L.crmath_sweep.restype = ctypes.c_long
    L.crmath_sweep.argtypes = [ctypes.c_int, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint,
                               ctypes.c_int, ctypes.POINTER(ctypes.c_uint), ctypes.c_long,
                               ctypes.POINTER(ctypes.c_long)]
    for fn in (0, 1, 2):
        bad = (ctypes.c_uint * 64)()
        slow = ctypes.c_long()
        n = L.crmath_sweep(fn, 0, 0x7F800000, 211, 8, bad, 64, ctypes.byref(slow))
        assert n == 0, (fn, list(bad[:n]))
