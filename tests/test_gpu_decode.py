"""GPU parity of the decode-sized top-k launch (batches of up to 8 rows with
TopK <= 256, csrc/g4s_decode.hip) against the CPU oracle through the C ABI:
token ids, survivor index sets, probabilities (bit-exact; the stated
tolerance is 1e-6 relative), LSum and the greedy id.  The launch's merge is
exact only when every wave list is complete below the K-th key, or made
complete by re-reading the waves whose lists reach it, so rows are built to
reach each of its branches: no ties, lowest-index ties, heap-layout ties,
waves holding more than four of the top K (re-read), more such waves than
the merge re-reads (heap replay), rows with fewer valid logits than K, and
K = 1 with planted copies of the maximum.  A batch of more than 8 rows takes
the chunked launch (g4s_topk.hip); both launches must agree on every output.
"""
import numpy as np
import pytest

from gemma4_sampler import hip, native, workload as wl
from test_gpu_topk import _params, check_rows

pytestmark = pytest.mark.gpu
F32 = np.float32
V = wl.V_GEMMA4
CAP = wl.SOFTCAP_GEMMA4


def _sample(s, rows, t, k, p, u, dtype=native.DTYPE_F32, stride=None, check=True):
    B = len(rows)
    d = hip.Buffer.from_array(rows)
    outs = native.DeviceOutputs(B, 64)
    rc, ids = s.sample(d, B, _params(t, k, p), u, dtype=dtype, outputs=outs.struct,
                       row_stride=stride if stride is not None else rows.shape[1], check=check)
    return rc, ids, outs.read()


@pytest.mark.parametrize("vocab", [2, 3, 7, 100, 1000, 4097, 40000])
def test_decode_small_vocab_ties(orc, vocab):
    """Dense integer ties, masked logits and every K regime up to 64, eight
    rows per call (the decode-sized launch)."""
    rng = np.random.default_rng(1000 + vocab)
    B = 8
    s = native.Sampler(vocab, max_batch=B, softcap=CAP)
    stride = (vocab + 3) // 4 * 4
    for rep in range(3):
        rows = np.empty((B, vocab), F32)
        for r in range(B):
            kind = (r + rep) % 4
            if kind == 0:
                rows[r] = rng.normal(0, 3, vocab)
            elif kind == 1:
                rows[r] = rng.integers(0, 6, vocab)
            elif kind == 2:
                rows[r] = rng.integers(0, 3, vocab)
                rows[r][rng.random(vocab) < 0.3] = -np.inf
            else:
                rows[r] = np.sort(rng.integers(0, 50, vocab)).astype(F32)
        k = np.array([rng.choice([1, 2, 5, 20, 64]) for _ in range(B)], np.int32)
        k = np.clip(k, 1, vocab - 1)
        t = rng.choice([0.0, 0.7, 1.0, 1.3], B).astype(F32)
        p = rng.choice([0.0, 0.5, 0.95, 1.0], B).astype(F32)
        u = np.floor(rng.random(B) * 2**32) / 2**32
        padded = np.full((B, stride), 1e30, F32)  # past `vocab`: values that would win
        padded[:, :vocab] = rows
        rc, ids, o = _sample(s, padded, t, k, p, u, stride=stride, check=False)
        empty = [r for r in range(B) if not np.any(rows[r] > F32(-1e30))]
        assert rc == (native.G4S_ERR_EMPTY_ROW if empty else 0), s.last_error()
        for r in empty:
            assert ids[r] == -1 and (o["flags"][r] & native.FLAG_EMPTY)
        keep = [r for r in range(B) if r not in empty]
        sub = {key: (val[keep] if hasattr(val, "__len__") else val) for key, val in o.items()}
        check_rows(orc, rows[keep], t[keep], k[keep], p[keep], u[keep], ids[keep], sub,
                   label=f"V={vocab} rep {rep}")
    s.close()


def _full_size_rows(rng):
    rows = np.empty((8, V), F32)
    rows[0] = 0.0                                   # all equal
    rows[1] = rng.integers(0, 2, V)                 # 0/1 with ten late 2s
    rows[1][rng.choice(V, 10, replace=False)] = 2.0
    rows[2] = rng.integers(0, 2, V)
    rows[2][V - 5:] = 3.0
    rows[3] = wl.host_peaky_rows(20261202, 0, 1, V)[0]
    # six of the top entries in one wave of 256 logits (its list holds four)
    rows[4] = rng.normal(0, 1, V).astype(F32)
    rows[4][4096 + np.arange(0, 12, 2)] = np.arange(20, 26, dtype=F32)
    # the maximum planted three more times (K = 1 keeps the first copy)
    rows[5] = wl.host_peaky_rows(20261202, 1, 1, V)[0]
    m = rows[5].max()
    rows[5][rng.choice(V, 3, replace=False)] = m
    # fewer than K logits above -1e30
    rows[6] = -np.inf
    rows[6][rng.choice(V, 40, replace=False)] = rng.normal(0, 1, 40)
    # tied at the K-th value with every larger key first in index order
    # (one per wave, so every wave list is complete below it)
    rows[7] = rng.normal(0, 1, V).astype(F32)
    rows[7][np.arange(10) * 300] = 9.0
    rows[7][3000 + np.arange(30) * 997] = 5.0
    return rows


def test_decode_full_size_regimes(orc):
    rng = np.random.default_rng(91)
    rows = _full_size_rows(rng)
    t = np.array([0.7, 1.0, 0.5, 0.7, 1.0, 0.0, 0.9, 0.8], F32)
    k = np.array([64, 64, 20, 64, 64, 1, 64, 20], np.int32)
    p = np.array([0.95, 0.9, 0.8, 0.95, 0.99, 0.95, 0.9, 0.97], F32)
    u = np.array([0.5, 0.25, 0.125, 0.75, 0.875, 0.0, 0.3, 0.6])
    s = native.Sampler(V, max_batch=9, softcap=CAP)
    rc, ids, o = _sample(s, rows, t, k, p, u)
    assert rc == 0, s.last_error()
    check_rows(orc, rows, t, k, p, u, ids, o, label="decode regimes")
    assert o["flags"][5] & native.FLAG_TIE_LOWEST
    assert o["flags"][7] & native.FLAG_TIE_LOWEST
    for r in (0, 1, 2):  # every wave list incomplete below the K-th key
        assert o["flags"][r] & native.FLAG_HEAP_REPLAY, (r, hex(o["flags"][r]))
    # row 4: one wave holds six of the top K -- re-read, no replay
    for r in (3, 4, 6):
        assert not (o["flags"][r] & (native.FLAG_HEAP_REPLAY | native.FLAG_TIE_LOWEST)), r
    s.close()


def test_decode_and_chunked_launches_agree(orc):
    """The same eight rows once as a batch of eight (the decode-sized launch)
    and once at the head of a batch of 65 (the chunked launch): every output
    equal (flags may name a different resolution of the same ties)."""
    rng = np.random.default_rng(92)
    rows = _full_size_rows(rng)
    t = np.array([0.7, 1.0, 0.5, 0.7, 1.0, 0.0, 0.9, 0.8], F32)
    k = np.array([64, 64, 20, 64, 64, 1, 64, 20], np.int32)
    p = np.array([0.95, 0.9, 0.8, 0.95, 0.99, 0.95, 0.9, 0.97], F32)
    u = np.array([0.5, 0.25, 0.125, 0.75, 0.875, 0.0, 0.3, 0.6])
    s = native.Sampler(V, max_batch=65, softcap=CAP)
    _, ids8, o8 = _sample(s, rows, t, k, p, u)
    n = 65
    rep = np.arange(n) % 8
    _, ids9, o9 = _sample(s, rows[rep], t[rep], k[rep], p[rep], u[rep])
    assert np.array_equal(ids8, ids9[:8])
    for key in ("count", "argmax"):
        assert np.array_equal(o8[key], o9[key][:8]), key
    assert np.array_equal(o8["lsum"].view(np.uint32), o9["lsum"][:8].view(np.uint32))
    assert np.array_equal(ids9[8:], ids9[rep[8:]])
    for r in range(8):
        n = int(o8["count"][r])
        assert np.array_equal(o8["indices"][r][:n], o9["indices"][r][:n]), r
        assert np.array_equal(o8["probs"][r][:n].view(np.uint32),
                              o9["probs"][r][:n].view(np.uint32)), r
    s.close()


def test_decode_bf16_rows(orc):
    B = 8
    s = native.Sampler(V, max_batch=B, softcap=CAP)
    b = wl.host_flat_bf16_rows(20261203, 0, B, V)
    rows = (b.astype(np.uint32) << 16).view(F32)
    k = np.array([1, 20, 64, 2, 1, 20, 64, 5], np.int32)
    t = np.array([1.0, 1.0, 0.7, 0.0, 1.0, 1.3, 1.0, 0.5], F32)
    p = np.full(B, 0.99, F32)
    u = wl.host_row_u(20261203, 0, B)
    rc, ids, o = _sample(s, b, t, k, p, u, dtype=native.DTYPE_BF16)
    assert rc == 0, s.last_error()
    check_rows(orc, rows, t, k, p, u, ids, o, label="decode bf16")
    s.close()


def test_decode_stream_rows(orc):
    """200 decode rows of the benchmark's stream (every 10th greedy with
    planted copies of its maximum), one row per call."""
    n = 200
    rows = wl.host_peaky_rows(20261204, 0, n, V, greedy_every=10)
    u = wl.host_row_u(20261204, 0, n)
    s = native.Sampler(V, max_batch=1, softcap=CAP)
    d = hip.Buffer.from_array(rows)
    got = np.empty(n, np.int32)
    for r in range(n):
        kk = 1 if r % 10 == 9 else 64
        got[r] = s.DoSample(d.offset(r * V * 4), float(u[r]),
                            native.TSamplingParams.make(0.7, kk, 0.95))
    for r in range(n):
        kk = 1 if r % 10 == 9 else 64
        want, _, _, _ = orc.do_sample(rows[r], 0.7, kk, 0.95, float(u[r]), softcap=CAP,
                                      want_probs=False)
        assert got[r] == want, (r, got[r], want)
    s.close()


def _wide_wave_rows(rng, n):
    """N(0, 1) rows with groups of large values planted inside single waves
    of 256 logits (the lists hold four per wave): row r plants r % 4 + 1
    groups of 5-12 values above 6, so the K-th largest key of K >= 20 lies
    among them or below."""
    rows = rng.normal(0, 1, (n, V)).astype(F32)
    for r in range(n):
        for _ in range(r % 4 + 1):
            w = int(rng.integers(0, V // 256))
            m = int(rng.integers(5, 13))
            pos = w * 256 + rng.choice(256, m, replace=False)
            rows[r, pos] = rng.uniform(6, 9, m).astype(F32)
    return rows


@pytest.mark.parametrize("B", [4, 8])
def test_decode_large_k_and_rereads(orc, B):
    """K up to 256: peaky rows, and rows whose large values crowd single
    waves so that the merge re-reads them; every output against the
    oracle."""
    rng = np.random.default_rng(93 + B)
    half = B // 2
    rows = np.concatenate([wl.host_peaky_rows(20261206, 0, B - half, V),
                           _wide_wave_rows(rng, half)])
    t, k, p = wl.host_mixed_params(20261206, 0, B)
    k = np.array([(1, 20, 64, 256, 200, 130)[r % 6] for r in range(B)], np.int32)
    u = wl.host_row_u(20261206, 0, B)
    s = native.Sampler(V, max_batch=B, softcap=CAP)
    d = hip.Buffer.from_array(rows)
    outs = native.DeviceOutputs(B, 256)
    rc, ids = s.sample(d, B, _params(t, k, p), u, outputs=outs.struct)
    assert rc == 0, s.last_error()
    o = outs.read()
    check_rows(orc, rows, t, k, p, u, ids, o, label=f"B={B} large K")
    assert not np.any(o["flags"] & native.FLAG_HEAP_REPLAY), o["flags"]
    s.close()


def test_mixed_benchmark_batch(orc):
    """The mixed-settings benchmark batch (64 peaky rows, K in {1, 20, 64,
    256}, launched with k_bound 256: the chunked launch) through the
    stream-ordered entry point: ids against the oracle's."""
    B = 64
    rows = wl.host_peaky_rows(20261207, 0, B, V)
    t, k, p = wl.host_mixed_params(20261207, 0, B)
    u = wl.host_row_u(20261207, 0, B)
    s = native.Sampler(V, max_batch=B, softcap=CAP)
    d = hip.Buffer.from_array(rows)
    parr = native.params_array(_params(t, k, p))
    dp = hip.Buffer(16 * B)
    hip.check(hip.lib().hipMemcpy(dp.ptr, parr, 16 * B, hip.H2D))
    du = hip.Buffer.from_array(np.asarray(u, np.float64))
    di = hip.Buffer(4 * B)
    s.sample_async(d, B, dp, du, 256, 0, di)
    hip.synchronize()
    ids = di.download(np.int32)
    want = orc.sample_batch(rows, 0, V, V, (t, k, p), u, softcap=CAP, threads=16)
    assert np.array_equal(ids, want), (np.nonzero(ids != want), ids, want)
    s.close()
