"""GPU parity of the top-k path (0 < TopK < V) against the CPU oracle, through
the C ABI.  Token ids, survivor index sets, probabilities, LSum and the greedy
id must all equal the oracle's bit for bit (the stated tolerance for
probabilities is 1e-6 relative; exact equality is asserted).  Draws whose
threshold lies within 1e-6 of a running-sum boundary are counted and printed.
"""
import numpy as np
import pytest

from gemma4_sampler import hip, native, workload as wl

pytestmark = pytest.mark.gpu
F32 = np.float32
V = wl.V_GEMMA4
CAP = wl.SOFTCAP_GEMMA4
SEED = 20261201


def _params(t, k, p):
    return [native.TSamplingParams.make(float(a), int(b), float(c)) for a, b, c in zip(t, k, p)]


def check_rows(orc, rows, t, k, p, u, got_ids, outs, softcap=CAP, label=""):
    """Compare every row with the oracle; returns the number of boundary draws."""
    boundary = 0
    for r in range(len(rows)):
        tok, det, idx, probs = orc.do_sample(rows[r], t[r], k[r], p[r], u[r], softcap=softcap)
        ctx = f"{label} row {r} (T={t[r]}, K={k[r]}, P={p[r]}, u={u[r]!r})"
        assert got_ids[r] == tok, f"{ctx}: gpu id {got_ids[r]} != oracle {tok}"
        if outs is not None:
            n = det["count"]
            assert outs["count"][r] == n, ctx
            assert np.array_equal(outs["indices"][r][:n], idx), ctx
            gp = outs["probs"][r][:n]
            rel = np.max(np.abs(gp.astype(np.float64) - probs) / np.maximum(probs, 1e-45)) if n else 0
            assert rel <= 1e-6, f"{ctx}: prob rel diff {rel}"
            assert np.array_equal(gp.view(np.uint32), probs.view(np.uint32)), f"{ctx}: probs not bit-exact"
            assert outs["lsum"][r] == det["lsum"], ctx
            assert outs["argmax"][r] == idx[det["argmax_pos"]], ctx
        if det["drew"] and det["reached"]:
            th = det["threshold"]
            d = min(th - det["cum_prev"] if det["chosen_pos"] > 0 else np.inf, det["cum_at"] - th)
            boundary += d < 1e-6
    return boundary


@pytest.fixture(scope="module")
def big():
    s = native.Sampler(V, max_batch=64, softcap=CAP)
    yield s
    s.close()


def test_generators_match_host():
    n = 3
    d = hip.Buffer(n * V * 4)
    wl.dev_peaky_rows(d, SEED, 98, n, V, greedy_every=100)
    hip.synchronize()
    host = wl.host_peaky_rows(SEED, 98, n, V, greedy_every=100)
    dev = d.download(np.float32).reshape(n, V)
    assert np.array_equal(dev.view(np.uint32), host.view(np.uint32))
    b = hip.Buffer(2 * V * 2)
    wl.dev_flat_bf16_rows(b, SEED, 0, 2, V)
    hip.synchronize()
    assert np.array_equal(b.download(np.uint16).reshape(2, V), wl.host_flat_bf16_rows(SEED, 0, 2, V))
    w = hip.Buffer(64 * 80 * 18)
    wl.dev_q4_weights(w, SEED, 64, 2560)
    h = hip.Buffer(4 * 2560 * 4)
    wl.dev_hidden(h, SEED, 4, 2560)
    hip.synchronize()
    assert np.array_equal(w.download(np.uint8), wl.host_q4_weights(SEED, 64, 2560))
    assert np.array_equal(h.download(np.float32).reshape(4, 2560).view(np.uint32),
                          wl.host_hidden(SEED, 4, 2560).view(np.uint32))


def test_peaky_row_single(big, orc):
    """One peaky row, T=0.7 K=64 P=0.95 (the CPU-reference configuration)."""
    row = wl.host_peaky_rows(SEED, 0, 1, V)
    u = wl.host_row_u(SEED, 0, 1)
    d = hip.Buffer.from_array(row)
    outs = native.DeviceOutputs(1, 64)
    _, ids = big.sample(d, 1, [native.TSamplingParams.make(0.7, 64, 0.95)], u,
                        outputs=outs.struct)
    o = outs.read()
    check_rows(orc, row, [0.7], [64], [0.95], u, ids, o, label="peaky")
    assert o["flags"][0] & native.FLAG_TOPK_PATH and o["count"][0] == 64


def test_decode_rows_back_to_back(big, orc):
    """300 peaky rows one at a time (B=1), every 100th greedy with planted ties."""
    n = 300
    rows = wl.host_peaky_rows(SEED, 0, n, V, greedy_every=wl.GREEDY_EVERY)
    u = wl.host_row_u(SEED, 0, n)
    t, k, p = wl.peaky_params(range(n))
    d = hip.Buffer.from_array(rows)
    ids = np.empty(n, np.int32)
    for r in range(n):
        _, one = big.sample(d.offset(r * V * 4), 1, _params(t[r:r + 1], k[r:r + 1], p[r:r + 1]),
                            u[r:r + 1])
        ids[r] = one[0]
    nb = check_rows(orc, rows, t, k, p, u, ids, None, label="decode")
    for r in range(wl.GREEDY_EVERY - 1, n, wl.GREEDY_EVERY):
        m = rows[r].max()
        assert ids[r] == int(np.flatnonzero(rows[r] == m)[0]), "lowest index among planted maxima"
    print(f"decode rows: {n}, boundary draws (|u*P - cum| < 1e-6): {nb}")


def test_mixed_batch(big, orc):
    """B=64 peaky rows with per-row T ~ U(0.3,1.5), K in {1,20,64,256}, P in {.8,.9,.95,1}."""
    B = 64
    rows = wl.host_peaky_rows(SEED + 1, 0, B, V)
    t, k, p = wl.host_mixed_params(SEED + 1, 0, B)
    u = wl.host_row_u(SEED + 1, 0, B)
    d = hip.Buffer.from_array(rows)
    outs = native.DeviceOutputs(B, 256)
    _, ids = big.sample(d, B, _params(t, k, p), u, outputs=outs.struct)
    nb = check_rows(orc, rows, t, k, p, u, ids, outs.read(), label="mixed")
    print(f"mixed batch: boundary draws {nb}")


@pytest.mark.parametrize("B", [16, 40, 65, 80])
def test_batch_launch_modes(big, orc, B):
    """K <= 64 batches of the chunked launch on both sides of its merge-launch
    split: 16 rows of 32 chunk workgroups fit the device at once (one launch,
    last-workgroup merges); 40, 65 and 80 rows do not (a chunk launch, then a
    merge launch)."""
    rows = wl.host_peaky_rows(SEED + 7, 0, B, V)
    ks = [1, 7, 33, 64]
    k = np.array([ks[r % 4] for r in range(B)], np.int32)
    t = np.array([(0.0, 0.7, 1.0, 1.3)[(r // 4) % 4] for r in range(B)], F32)
    p = np.array([(0.9, 0.95, 1.0)[r % 3] for r in range(B)], F32)
    u = wl.host_row_u(SEED + 7, 0, B)
    d = hip.Buffer.from_array(rows)
    outs = native.DeviceOutputs(B, 64)
    s = big if B <= 64 else native.Sampler(V, max_batch=B, softcap=CAP)  # big holds 64 rows
    _, ids = s.sample(d, B, _params(t, k, p), u, outputs=outs.struct)
    check_rows(orc, rows, t, k, p, u, ids, outs.read(), label=f"B={B}")
    if s is not big:
        s.close()


@pytest.mark.parametrize("dtype,vocab,B", [(native.DTYPE_F32, 100000, 72),
                                           (native.DTYPE_BF16, V, 40)])
def test_chunked_two_launch_large_k(orc, dtype, vocab, B):
    """Batches whose K bound lies in 65..256 and whose chunk workgroups do not
    fit the device at once take a chunk launch and then a merge launch of the
    1024 x 32 shape: fp32 rows of a vocabulary that ends in a partial chunk,
    and bf16 rows.  Rows 0 and 1 are massively tied (all equal; 0/1 with a
    few 2s), so their chunks hold more candidates than slots and take the
    exact per-chunk select; the others are ordinary rows with K in
    {1, 20, 64, 256}."""
    rng = np.random.default_rng(vocab + B)
    if dtype == native.DTYPE_F32:
        rows = wl.host_peaky_rows(SEED + 11, 0, B, vocab)
    else:
        rows = (wl.host_flat_bf16_rows(SEED + 11, 0, B, vocab).astype(np.uint32) << 16).view(F32)
    rows[0] = 0.25
    rows[1] = rng.integers(0, 2, vocab)
    rows[1][rng.choice(vocab, 7, replace=False)] = 2.0
    ks = [256, 200, 1, 20, 64, 256]
    k = np.array([ks[r] if r < 2 else ks[2 + r % 4] for r in range(B)], np.int32)
    t = np.array([(0.7, 1.0, 1.3)[r % 3] for r in range(B)], F32)
    p = np.array([(0.9, 0.95, 1.0)[r % 3] for r in range(B)], F32)
    u = wl.host_row_u(SEED + 11, 0, B)
    host = rows if dtype == native.DTYPE_F32 else (rows.view(np.uint32) >> 16).astype(np.uint16)
    d = hip.Buffer.from_array(np.ascontiguousarray(host))
    s = native.Sampler(vocab, max_batch=B, softcap=CAP)
    outs = native.DeviceOutputs(B, 256)
    _, ids = s.sample(d, B, _params(t, k, p), u, dtype=dtype, outputs=outs.struct)
    o = outs.read()
    check_rows(orc, rows, t, k, p, u, ids, o, label=f"two launches dtype={dtype}")
    assert o["flags"][0] & native.FLAG_TIE_LOWEST
    s.close()


def test_async_matches_sync(big, orc):
    B = 16
    rows = wl.host_peaky_rows(SEED + 2, 0, B, V)
    t, k, p = wl.host_mixed_params(SEED + 2, 0, B)
    u = wl.host_row_u(SEED + 2, 0, B)
    d = hip.Buffer.from_array(rows)
    parr = native.params_array(_params(t, k, p))
    dp = hip.Buffer(16 * B)
    hip.check(hip.lib().hipMemcpy(dp.ptr, parr, 16 * B, hip.H2D))
    du = hip.Buffer.from_array(u)
    di = hip.Buffer(4 * B)
    big.sample_async(d, B, dp, du, int(k.max()), 0, di)
    hip.synchronize()
    _, ids = big.sample(d, B, _params(t, k, p), u)
    assert np.array_equal(di.download(np.int32), ids)
    check_rows(orc, rows, t, k, p, u, ids, None, label="async")


@pytest.mark.parametrize("vocab", [2, 3, 7, 100, 1000, 5000, 40000])
def test_small_vocab_random(orc, vocab):
    """Integer-valued rows (dense ties), masked logits, every K regime incl. V-1."""
    rng = np.random.default_rng(vocab)
    B = 24
    s = native.Sampler(vocab, max_batch=B, softcap=CAP)
    rows = np.empty((B, vocab), F32)
    for r in range(B):
        kind = r % 4
        if kind == 0:
            rows[r] = rng.normal(0, 3, vocab)
        elif kind == 1:
            rows[r] = rng.integers(0, 6, vocab)
        elif kind == 2:
            rows[r] = rng.integers(0, 3, vocab)
            rows[r][rng.random(vocab) < 0.3] = -np.inf
        else:
            rows[r] = np.sort(rng.integers(0, 50, vocab)).astype(F32)
    k = np.array([rng.choice([1, 2, min(5, vocab - 1), min(64, vocab - 1), vocab - 1,
                              min(1024, vocab - 1)]) for _ in range(B)], np.int32)
    k = np.clip(k, 1, min(vocab - 1, native.max_top_k()))
    t = rng.choice([0.0, 0.7, 1.0, 1.3], B).astype(F32)
    p = rng.choice([0.0, 0.5, 0.95, 1.0], B).astype(F32)
    u = np.floor(rng.random(B) * 2**32) / 2**32
    # rows padded to a 16-byte stride; the padding holds values that would win
    # every selection if the kernel read past `vocab`
    stride = (vocab + 3) // 4 * 4
    padded = np.full((B, stride), 1e30, F32)
    padded[:, :vocab] = rows
    d = hip.Buffer.from_array(padded)
    cap = int(k.max())
    outs = native.DeviceOutputs(B, cap)
    rc, ids = s.sample(d, B, _params(t, k, p), u, row_stride=stride, outputs=outs.struct,
                       check=False)
    o = outs.read()
    empty = [r for r in range(B) if not np.any(rows[r] > F32(-1e30))]
    if empty:
        assert rc == native.G4S_ERR_EMPTY_ROW
        for r in empty:
            assert ids[r] == -1 and (o["flags"][r] & native.FLAG_EMPTY)
    else:
        assert rc == 0, s.last_error()
    keep = [r for r in range(B) if r not in empty]
    sub = {key: (val[keep] if hasattr(val, "__len__") else val) for key, val in o.items()}
    check_rows(orc, rows[keep], t[keep], k[keep], p[keep], u[keep], ids[keep], sub,
               label=f"V={vocab}")
    s.close()


def test_heap_tie_counterexample(orc):
    s = native.Sampler(4, max_batch=1, softcap=CAP)
    row = np.array([1, 1, 4, 2], F32)
    d = hip.Buffer.from_array(row)
    outs = native.DeviceOutputs(1, 3)
    _, ids = s.sample(d, 1, [native.TSamplingParams.make(0.7, 3, 0.95)], [0.25],
                      outputs=outs.struct)
    o = outs.read()
    assert list(o["indices"][0]) == [1, 2, 3]
    assert o["flags"][0] & native.FLAG_HEAP_REPLAY
    check_rows(orc, row[None], [0.7], [3], [0.95], [0.25], ids, o)
    s.close()


def test_full_size_tie_regimes(big, orc):
    """Full-size rows whose K-th value is massively tied: all-equal rows
    (chunked launch: exact per-chunk select, lowest-index rule; decode-sized
    launch: every wave list incomplete, heap replay), 0/1 rows with late 2s
    (heap replay), and bf16-valued rows -- as a batch of 4 (the decode-sized
    launch) and at the head of a batch of 65 (the chunked launch)."""
    rng = np.random.default_rng(77)
    rows = np.zeros((4, V), F32)
    rows[1] = rng.integers(0, 2, V)
    rows[1][rng.choice(V, 10, replace=False)] = 2.0
    rows[2] = (rng.normal(0, 0.5, V).astype(F32).view(np.uint32) & 0xFFFF0000).view(F32)
    rows[3] = rng.integers(0, 2, V)
    rows[3][V - 5:] = 3.0
    t = np.array([0.7, 1.0, 1.0, 0.5], F32)
    k = np.array([64, 64, 256, 20], np.int32)
    p = np.array([0.95, 0.9, 0.99, 0.8], F32)
    u = np.array([0.5, 0.25, 0.75, 0.125])
    d = hip.Buffer.from_array(rows)
    outs = native.DeviceOutputs(4, 256)
    _, ids = big.sample(d, 4, _params(t, k, p), u, outputs=outs.struct)
    o = outs.read()
    check_rows(orc, rows, t, k, p, u, ids, o, label="ties")
    assert o["flags"][0] & native.FLAG_HEAP_REPLAY
    assert o["flags"][3] & native.FLAG_HEAP_REPLAY
    n = 65
    rep = np.arange(n) % 4
    s = native.Sampler(V, max_batch=n, softcap=CAP)
    d65 = hip.Buffer.from_array(rows[rep])
    outs = native.DeviceOutputs(n, 256)
    _, ids65 = s.sample(d65, n, _params(t[rep], k[rep], p[rep]), u[rep], outputs=outs.struct)
    o = outs.read()
    assert np.array_equal(ids65, ids[rep]), (ids65, ids)
    sub = {key: (val[:4] if hasattr(val, "__len__") else val) for key, val in o.items()}
    check_rows(orc, rows, t, k, p, u, ids65[:4], sub, label="ties (chunked)")
    assert o["flags"][0] & native.FLAG_TIE_LOWEST
    assert o["flags"][3] & native.FLAG_HEAP_REPLAY
    s.close()


def test_bf16_logits_topk(orc):
    B = 8
    s = native.Sampler(V, max_batch=B, softcap=CAP)
    b = wl.host_flat_bf16_rows(SEED + 3, 0, B, V)
    rows = (b.astype(np.uint32) << 16).view(F32)
    k = np.array([1, 20, 64, 256, 1, 20, 64, 256], np.int32)
    t = np.full(B, 1.0, F32)
    p = np.full(B, 0.99, F32)
    u = wl.host_row_u(SEED + 3, 0, B)
    d = hip.Buffer.from_array(b)
    outs = native.DeviceOutputs(B, 256)
    _, ids = s.sample(d, B, _params(t, k, p), u, dtype=native.DTYPE_BF16, outputs=outs.struct)
    check_rows(orc, rows, t, k, p, u, ids, outs.read(), label="bf16")
    s.close()


def test_argument_errors_on_device(big):
    d = hip.Buffer.from_array(np.zeros(V, F32))
    # TopK above g4s_max_top_k() takes the wide path: all-equal logits keep
    # the first 2000 indices (lowest-index tie rule), each p = fl32(1/2000);
    # u=0.5 picks the first index whose binary32 running sum reaches 0.5
    rc, ids = big.sample(d, 1, [native.TSamplingParams.make(1.0, 2000, 1.0)], [0.5], check=False)
    p, c, want = F32(1.0) / F32(2000.0), F32(0.0), -1
    for i in range(2000):
        c = F32(c + p)
        if c >= F32(0.5):
            want = i
            break
    assert rc == native.G4S_OK and ids[0] == want, (rc, ids, want, big.last_error())
    di = hip.Buffer(4)
    rc = native.load().g4s_sample_async(big.h, d.addr, native.DTYPE_F32, V, 1, d.addr, d.addr,
                                        V, 0, di.addr, None)
    assert rc == native.G4S_ERR_INVALID_ARGUMENT and "k_bound" in big.last_error()
    rc, _ = big.sample(d, 1, [native.TSamplingParams.make(1.0, 5, 0.9)], [1.0], check=False)
    assert rc == native.G4S_ERR_INVALID_ARGUMENT
    rc, _ = big.sample(d.offset(4), 1, [native.TSamplingParams.make(1.0, 5, 0.9)], [0.5],
                       check=False)
    assert rc == native.G4S_ERR_INVALID_ARGUMENT and "aligned" in big.last_error()
    rc, _ = big.sample(d, 65, [native.TSamplingParams.make(1.0, 5, 0.9)] * 65, [0.5] * 65,
                       check=False)
    assert rc == native.G4S_ERR_INVALID_ARGUMENT


def _heap_select(x, K, right_if_le=False):
    """The reference's min-heap pass (Model.pas:2632-2676), used here only to
    show that a planted row tells the child-tie rule apart: right_if_le=True
    swaps the strict `<` of :2653-2654 for `<=`.  The oracle, pinned by hand
    traces, stays the checker."""
    hv = [F32(-1e30)] * K
    hi = [-1] * K
    xs = np.asarray(x, F32)
    cand = np.nonzero(xs > F32(-1e30))[0]
    for i in cand:
        v = xs[i]
        if v <= hv[0]:
            continue
        p = 0
        while True:
            c = 2 * p + 1
            if c >= K:
                break
            if c + 1 < K and ((hv[c + 1] <= hv[c]) if right_if_le else (hv[c + 1] < hv[c])):
                c += 1
            if hv[c] >= v:
                break
            hv[p], hi[p] = hv[c], hi[c]
            p = c
        hv[p], hi[p] = v, int(i)
    return sorted(i for i in hi if i >= 0)


def test_heap_child_tie_full_size(big, orc):
    """Full-size rows where the surviving tied copies depend on the heap's
    child-tie rule (Model.pas:2653-2654): the 0,0,0,1,1 pattern (K=4) on an
    excluded (-1e30) background and on a random background, and a wide row
    (K=1500 > g4s_max_top_k) with 1000 ones and 1000 zeros scattered over a
    random background.  Every row is checked to give a different survivor
    set under `<=`, so a kernel using the wrong rule fails."""
    rng = np.random.default_rng(2653)
    rows = np.empty((3, V), F32)
    rows[0] = F32(-1e30)
    pos = np.sort(rng.choice(V, 5, replace=False))
    rows[0][pos] = [0, 0, 0, 1, 1]
    for attempt in range(50):
        bg = (F32(-20) - np.abs(rng.normal(0, 1, V))).astype(F32)
        pos1 = np.sort(rng.choice(V, 5, replace=False))
        bg[pos1] = [0, 0, 0, 1, 1]
        if _heap_select(bg, 4) != _heap_select(bg, 4, right_if_le=True):
            break
    rows[1] = bg
    for attempt in range(50):
        bg = (F32(-20) - np.abs(rng.normal(0, 1, V))).astype(F32)
        pl = rng.choice(V, 2000, replace=False)
        bg[pl[:1000]] = 1.0
        bg[pl[1000:]] = 0.0
        if _heap_select(bg, 1500) != _heap_select(bg, 1500, right_if_le=True):
            break
    rows[2] = bg
    k = np.array([4, 4, 1500], np.int32)
    t = np.array([0.7, 1.0, 1.0], F32)
    p = np.array([0.95, 0.9, 0.99], F32)
    u = np.array([0.3, 0.6, 0.45])
    want_sets = [_heap_select(rows[r], int(k[r])) for r in range(3)]
    for r in range(3):
        assert want_sets[r] != _heap_select(rows[r], int(k[r]), right_if_le=True), \
            f"row {r} does not tell the child-tie rules apart"
        assert list(orc.select_topk_indices(rows[r], int(k[r]))) == want_sets[r], r
    s = native.Sampler(V, max_batch=3, softcap=CAP)
    d = hip.Buffer.from_array(rows)
    outs = native.DeviceOutputs(3, 1500)
    _, ids = s.sample(d, 3, _params(t, k, p), u, outputs=outs.struct)
    o = outs.read()
    check_rows(orc, rows, t, k, p, u, ids, o, label="child-tie")
    for r in range(3):
        assert list(o["indices"][r][:o["count"][r]]) == want_sets[r], r
        assert o["flags"][r] & native.FLAG_HEAP_REPLAY, (r, hex(o["flags"][r]))
    assert o["flags"][2] & native.FLAG_WIDE_K
    s.close()


def test_async_rejects_rows_whose_path_is_not_enqueued(big):
    """g4s_sample_async with full_rows = 0 leaves no full-vocabulary row
    with an earlier call's id, and k_bound = 0 none of the top-k rows: such
    rows get id -1 and G4S_FLAG_ERROR plus the path they would have taken."""
    rows = wl.host_peaky_rows(SEED, 0, 2, V)
    d = hip.Buffer.from_array(rows)
    for k_bound, full_rows, ks, bad, path in ((64, 0, [64, 0], 1, native.FLAG_FULL_PATH),
                                              (0, 1, [0, 5], 1, native.FLAG_TOPK_PATH)):
        parr = native.params_array(_params([0.7, 0.7], ks, [0.95, 0.95]))
        dp = hip.Buffer(16 * 2)
        hip.check(hip.lib().hipMemcpy(dp.ptr, parr, 32, hip.H2D))
        du = hip.Buffer.from_array(np.array([0.5, 0.5]))
        di = hip.Buffer.from_array(np.array([12345, 12345], np.int32))
        outs = native.DeviceOutputs(2, 1)
        big.sample_async(d, 2, dp, du, k_bound, full_rows, di, outputs=outs.struct)
        hip.synchronize()
        ids, fl = di.download(np.int32), outs.read()["flags"]
        assert ids[bad] == -1 and fl[bad] & native.FLAG_ERROR and fl[bad] & path, (ids, fl)
        assert ids[1 - bad] != 12345 and not (fl[1 - bad] & native.FLAG_ERROR), (ids, fl)
