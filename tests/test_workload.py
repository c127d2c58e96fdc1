"""Host workload generators: determinism and the distributions the five
benchmark configurations ask for."""
import numpy as np

from gemma4_sampler import workload as wl

V = wl.V_GEMMA4


def test_peaky_row_shape_and_spikes():
    r = wl.host_peaky_rows(1, 0, 2, V)
    assert r.shape == (2, V) and r.dtype == np.float32
    r2 = wl.host_peaky_rows(1, 0, 2, V, threads=1)
    assert np.array_equal(r.view(np.uint32), r2.view(np.uint32)), "deterministic"
    base = np.sort(r[0])[:-16]
    assert abs(base.mean()) < 0.05 and abs(base.std() - 3.0) < 0.05
    assert abs(np.mean(np.abs(base) < 3.0) - 0.6827) < 0.01
    # 16 indices raised by U(6,12): the top of the row sits well above the
    # N(0, 9) bulk's expected maximum (~13.6 for 262144 draws)
    assert np.sort(r[0])[-16:].mean() > 11.0
    assert not np.array_equal(r[0], r[1])


def test_greedy_rows_have_planted_max_copies():
    rows = wl.host_peaky_rows(3, 99, 1, V, greedy_every=100)
    m = rows[0].max()
    assert 3 <= np.sum(rows[0] == m) <= 5
    plain = wl.host_peaky_rows(3, 98, 1, V, greedy_every=100)
    assert np.sum(plain[0] == plain[0].max()) == 1


def test_flat_bf16_and_params():
    b = wl.host_flat_bf16_rows(2, 0, 1, 65536)
    x = (b.astype(np.uint32) << 16).view(np.float32)
    assert abs(x.std() - 0.5) < 0.01
    t, k, p = wl.host_mixed_params(5, 0, 4096)
    assert t.min() >= 0.3 and t.max() <= 1.5
    assert set(k.tolist()) == {1, 20, 64, 256}
    assert set(p.tolist()) == {float(np.float32(v)) for v in (0.8, 0.9, 0.95, 1.0)}
    u = wl.host_row_u(5, 0, 10000)
    assert u.min() >= 0 and u.max() < 1
    assert np.all((u * 2.0**32) == np.floor(u * 2.0**32)), "u on the 2^-32 grid"


def test_q4_weights_and_hidden():
    w = wl.host_q4_weights(7, 8, 256)
    assert w.size == 8 * 8 * 18
    blocks = w.reshape(-1, 18)
    scales = (blocks[:, 0].astype(np.uint16) | (blocks[:, 1].astype(np.uint16) << 8)).view(np.float16)
    assert scales.min() >= 0.0009 and scales.max() <= 0.0201
    h = wl.host_hidden(7, 4, 2560)
    assert abs(h.std() - 1.0) < 0.05
