"""GPU parity of the streaming pipeline of full bf16 rows (vocabulary a
multiple of 1024) in its rare regimes, against the CPU oracle through the C
ABI: codes outside the per-row table of e (infinities, codes far below the
row's largest |x|, with and without one shared value), rows whose set of
codes with e == 1 reaches below the table, masked rows, +inf maxima, and the
probabilities of every code.

The reference path is CpuLogitSoftcap + DoSampleTopP + CpuSoftmaxF32
(src/Gemma4.Layers.pas:300-316, src/Gemma4.Model.pas:2691-2737,
src/Gemma4.Tensors.pas:638-673).  Ids, LSum, the greedy id and the
probabilities must equal the oracle's bit for bit.
"""
import numpy as np
import pytest

from gemma4_sampler import hip, native, workload as wl

pytestmark = pytest.mark.gpu
F32 = np.float32
V = wl.V_GEMMA4
CAP = wl.SOFTCAP_GEMMA4


def _b16(x):
    """Round-to-nearest-even bf16 codes of float32 values (NaN-free input)."""
    b = np.asarray(x, F32).view(np.uint32).astype(np.uint64)
    r = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def _widen(codes):
    return (codes.astype(np.uint32) << 16).view(F32)


def _run(orc, codes, t, k, p, u, softcap, probs):
    B = codes.shape[0]
    s = native.Sampler(V, max_batch=B, softcap=softcap)
    d = hip.Buffer.from_array(np.ascontiguousarray(codes))
    params = [native.TSamplingParams.make(float(a), int(b), float(c)) for a, b, c in zip(t, k, p)]
    outs = native.DeviceOutputs(B, V if probs else 1)
    _, ids = s.sample(d, B, params, u, outputs=outs.struct, dtype=native.DTYPE_BF16)
    o = outs.read()
    rows = _widen(codes)
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(8) as ex:
        refs = list(ex.map(lambda r: orc.do_sample(rows[r], t[r], k[r], p[r], u[r], softcap=softcap,
                                                   want_probs=probs), range(B)))
    for r in range(B):
        tok, det, _, pr = refs[r]
        ctx = f"row {r} (T={t[r]}, K={k[r]}, P={p[r]}, u={u[r]!r}, cap={softcap})"
        assert ids[r] == tok, f"{ctx}: gpu id {ids[r]} != oracle {tok}"
        assert o["flags"][r] & native.FLAG_FULL_PATH, ctx
        assert o["lsum"][r].view(np.uint32) == np.float32(det["lsum"]).view(np.uint32), \
            f"{ctx}: lsum {o['lsum'][r]!r} != {det['lsum']!r}"
        assert o["argmax"][r] == det["argmax_pos"], f"{ctx}: argmax {o['argmax'][r]} != {det['argmax_pos']}"
        if probs:
            assert np.array_equal(o["probs"][r].view(np.uint32), pr.view(np.uint32)), f"{ctx}: probs"
    s.close()


def _settings(rng, B):
    t = rng.choice([1.0, 0.7, 1.3], B).astype(F32)
    k = rng.choice([0, -1, V], B).astype(np.int32)
    p = rng.choice([0.9, 0.99, 1.0], B).astype(F32)
    u = np.floor(rng.random(B) * 2**32) / 2**32
    return t, k, p, u


@pytest.mark.parametrize("softcap", [CAP, 0.0])
@pytest.mark.parametrize("probs", [False, True])
def test_tiny_codes_and_zeros(orc, softcap, probs):
    """N(0, 0.5^2) rows with planted +-0, subnormal and far-below codes (below
    the table's 32 binades of |x|): they share one e, so the streaming passes
    take it from the row's constants."""
    rng = np.random.default_rng(11 + int(softcap) + 2 * probs)
    B = 4
    codes = _b16(rng.normal(0, 0.5, (B, V)))
    for r in range(B):
        pos = rng.choice(V, 600, replace=False)
        codes[r, pos[:100]] = 0x0000
        codes[r, pos[100:200]] = 0x8000
        codes[r, pos[200:300]] = rng.integers(1, 0x80, 100)            # +subnormals
        codes[r, pos[300:400]] = 0x8000 | rng.integers(1, 0x80, 100)   # -subnormals
        codes[r, pos[400:600]] = _b16(rng.choice([1e-20, -3e-25, 2e-30, -1e-33], 200))
    _run(orc, codes, *_settings(rng, B), softcap, probs)


@pytest.mark.parametrize("softcap", [CAP, 0.0])
def test_masked_rows(orc, softcap):
    """Rows with -inf at 5 % and 50 % of the positions (masked logits): the
    table follows the largest finite |x|, -inf takes e(-inf)."""
    rng = np.random.default_rng(21 + int(softcap))
    B = 4
    codes = _b16(rng.normal(0, 0.5, (B, V)))
    for r in range(B):
        frac = 0.05 if r % 2 == 0 else 0.5
        codes[r, rng.random(V) < frac] = 0xFF80
    _run(orc, codes, *_settings(rng, B), softcap, probs=(softcap > 0))


def test_plus_inf_maxima(orc):
    """+inf logits under the softcap (y = cap): e(+inf) == 1, the argmax is the
    first +inf, which lies outside the table."""
    rng = np.random.default_rng(31)
    B = 3
    codes = _b16(rng.normal(0, 2.0, (B, V)))
    for r in range(B):
        codes[r, rng.choice(V, 3 + r, replace=False)] = 0x7F80
    t, k, p, u = _settings(rng, B)
    t[:] = 1.0
    _run(orc, codes, t, k, p, u, CAP, probs=True)


def test_all_tiny_rows(orc):
    """Every logit within 1e-30 of 0: every e rounds to 1 near the maximum,
    and the codes with e == 1 reach the bottom of the table (every chunk is
    searched for the argmax); T <= 0 rows take the greedy id."""
    rng = np.random.default_rng(41)
    B = 4
    codes = _b16(rng.normal(0, 1e-31, (B, V)))
    t, k, p, u = _settings(rng, B)
    t[0] = 0.0
    _run(orc, codes, t, k, p, u, CAP, probs=True)


def test_below_table_codes_that_differ(orc):
    """A row whose largest |x| is far larger than the rest (-1e6 among
    N(0, 0.01^2)): codes below the table's binades have different e, so the
    chunks holding them are left to the chains' exact re-evaluation."""
    rng = np.random.default_rng(51)
    B = 2
    codes = _b16(rng.normal(0, 0.01, (B, V)))
    codes[:, 12345] = _b16(np.float32(-1e6))
    t, k, p, u = _settings(rng, B)
    _run(orc, codes, t, k, p, u, CAP, probs=False)


def _rn32(fr):
    """The binary32 nearest to a positive rational (ties to even), exactly."""
    from fractions import Fraction
    f = np.float32(float(fr))
    lo = f if Fraction(float(f)) <= fr else np.nextafter(f, F32(0))
    hi = np.nextafter(lo, F32(np.inf))
    dl, dh = fr - Fraction(float(lo)), Fraction(float(hi)) - fr
    if dl != dh:
        return lo if dl < dh else hi
    return lo if (int(lo.view(np.uint32)) & 1) == 0 else hi


def _u_for(thr, top_p):
    """A double u with RN32(u * TopP) == thr (the draw's threshold,
    Model.pas:2726, the product correctly rounded)."""
    from fractions import Fraction
    u = float(Fraction(float(thr)) / Fraction(float(top_p)))
    for _ in range(64):
        got = _rn32(Fraction(u) * Fraction(float(top_p)))
        if got == thr:
            return u
        u = float(np.nextafter(u, np.inf if got < thr else -np.inf))
    raise AssertionError(f"no u gives thr {thr!r}")


def _half_unit_ties(p):
    """Indices i whose step S = RN32(S + p[i]) of the left-to-right binary32
    running sum is a tie (S + p[i] exactly halfway between two binary32
    values), and the running sums.  The exact S + p[i] fits a double here."""
    s = np.add.accumulate(p, dtype=F32)
    prev = np.concatenate([[0.0], s[:-1].astype(np.float64)])
    a = prev + p.astype(np.float64)
    m, e = np.frexp(a)                    # a = m * 2^e, 0.5 <= m < 1
    q = np.ldexp(a, 25 - e.astype(np.int64))  # units of half the binary32 spacing there
    tie = (q == np.floor(q)) & (np.mod(q, 2.0) == 1.0) & (p > 0)
    return np.nonzero(tie)[0], s


def test_draw_targets_after_half_unit_ties(orc):
    """Draws whose threshold is the exact running sum a few lanes after a step
    that rounds a half-unit tie (Model.pas:2727-2735).  Past chunk 0 the
    chunk holding the target is staged for the draw chain and the tie sits in
    a lane before the target's, so it enters through that chunk's lane maps;
    in chunk 0 it enters through the draw's walk of chunk 0.  A lane map that
    rounded the tie as if the sum's parity did not matter would leave the
    running sum one unit off at the target, and the first index that reaches
    thr would move.  Rows of N(0, 0.5^2) logits are drawn until 12 have such
    a tie past chunk 0 (they are rare there: a few rows in ten) and 4 more in
    chunk 0; the expected ids come from the oracle's p and the binary32
    running sum, and must also be the oracle's own."""
    rng = np.random.default_rng(61)
    B = 16
    picked, targets = [], []
    for _ in range(400):
        if len(picked) == B:
            break
        need_past0 = len(picked) < 12
        c = _b16(rng.normal(0, 0.5, V))
        _, det, idx, pr = orc.do_sample(_widen(c), 1.0, 0, 0.99, 0.5, softcap=CAP, want_probs=True)
        assert det["count"] == V and np.array_equal(idx, np.arange(V))
        ties, s = _half_unit_ties(pr)
        ok = ties[(ties % 1024 < 1024 - 48) & ((ties >= 1024) if need_past0 else (ties < 1024))]
        if ok.size == 0:
            continue
        i = int(ok[0])
        thr = s[i + 40]
        if not 0 < thr < F32(0.99):
            continue
        picked.append(c)
        targets.append((i, thr, int(np.argmax(s >= thr))))
    assert len(picked) == B, f"only {len(picked)} rows with a usable tie"
    codes = np.stack(picked)
    rows = _widen(codes)
    t = np.full(B, 1.0, F32)
    k = np.zeros(B, np.int32)
    p = np.full(B, 0.99, F32)
    u = np.array([_u_for(thr, p[r]) for r, (_, thr, _) in enumerate(targets)])
    for r, (i, thr, first) in enumerate(targets):
        tok, _, _, _ = orc.do_sample(rows[r], 1.0, 0, 0.99, u[r], softcap=CAP, want_probs=False)
        assert tok == first, f"row {r}: oracle {tok}, running sum says {first} (tie at {i})"
    _run(orc, codes, t, k, p, u, CAP, probs=False)


def _target_u(orc, row, t, p, pos):
    """u that makes the draw of a full row land exactly on index `pos` (the
    threshold is the exact running sum there) and that index."""
    _, _, _, pr = orc.do_sample(row, t, 0, p, 0.5, softcap=CAP, want_probs=True)
    s = np.add.accumulate(pr, dtype=F32)
    thr = s[pos]
    u = _u_for(thr, F32(p))
    return u, int(np.argmax(s >= thr))


def test_row_state_between_calls(orc):
    """The pipeline's per-row words are accumulated (row maxima, the
    smallest key with e == 1 and the argmax by atomics) or handed from
    kernel to kernel (the draw's exact sum and hit in chunk 0, the staged
    chunk counts), and the draw chain resets them for the next call after
    reading its own.  One handle samples four calls in a row through the
    same row slots, each slot chosen so that a word left over from the
    previous call, or read after its reset, changes the result:
      slot 0: maximum 12 early (greedy) -> maximum 2.5 late (draw; a stale
              row maximum or argmax) -> maximum 6 late behind early 3.0s
              (greedy; a stale smallest key with e == 1 picks a 3.0);
      slot 1: draw inside chunk 0 -> draw in a late chunk (a stale hit)
              -> inside chunk 0 -> late chunk;
      slot 2: top-k row -> full draw -> (not in the call) -> greedy with the
              argmax early;
      slot 3: draw late with |x| up to 40 -> P = 0 (the chains' early exit)
              -> (not in the call) -> draw inside chunk 0 (the running sum of
              chunk 0 read before its reset).
    Ids, LSum and the greedy id of every full row equal the oracle's."""
    rng = np.random.default_rng(73)
    s = native.Sampler(V, max_batch=4, softcap=CAP)

    def base():
        return rng.normal(0, 0.5, V).astype(F32)

    calls = []
    # call 1
    r0 = base(); r0[3] = 12.0; r0[rng.integers(1000, V)] = -40.0
    r1 = base()
    r2 = base()
    r3 = base(); r3[rng.choice(V, 8, replace=False)] = -40.0
    calls.append([(r0, 0.0, 0, 0.95, None), (r1, 1.0, 0, 0.99, 300),
                  (r2, 0.7, 64, 0.95, "u"), (r3, 1.0, 0, 0.99, 200000)])
    # call 2
    r0 = base(); r0[250000] = 2.5
    r1 = base()
    r2 = base()
    r3 = base()
    calls.append([(r0, 1.0, 0, 0.99, 150000), (r1, 1.0, 0, 0.99, 180000),
                  (r2, 1.0, 0, 0.99, 90000), (r3, 1.0, 0, 0.0, None)])
    # call 3 (two rows)
    r0 = base(); r0[rng.choice(1000, 10, replace=False)] = 3.0; r0[200000] = 6.0
    r1 = base()
    calls.append([(r0, 0.0, 0, 0.95, None), (r1, 1.0, 0, 0.99, 700)])
    # call 4
    r0 = base()
    r1 = base()
    r2 = base(); r2[10] = 4.0
    r3 = base()
    calls.append([(r0, 1.0, 0, 0.99, 100000), (r1, 1.0, 0, 0.99, 240000),
                  (r2, 0.0, 0, 0.95, None), (r3, 1.0, 0, 0.99, 500)])

    for ci, call in enumerate(calls):
        B = len(call)
        codes = np.stack([_b16(c[0]) for c in call])
        rows = _widen(codes)
        t = np.array([c[1] for c in call], F32)
        k = np.array([c[2] for c in call], np.int32)
        p = np.array([c[3] for c in call], F32)
        u = np.empty(B)
        for r, c in enumerate(call):
            if c[4] is None:
                u[r] = 0.5
            elif c[4] == "u":
                u[r] = 0.375
            else:
                u[r], _ = _target_u(orc, rows[r], float(t[r]), float(p[r]), c[4])
        d = hip.Buffer.from_array(np.ascontiguousarray(codes))
        params = [native.TSamplingParams.make(float(a), int(b), float(q))
                  for a, b, q in zip(t, k, p)]
        outs = native.DeviceOutputs(B, 1)
        rc, ids = s.sample(d, B, params, u, outputs=outs.struct, dtype=native.DTYPE_BF16)
        assert rc == 0, s.last_error()
        o = outs.read()
        for r in range(B):
            tok, det, _, _ = orc.do_sample(rows[r], t[r], k[r], p[r], u[r], softcap=CAP,
                                           want_probs=False)
            ctx = f"call {ci + 1} slot {r} (T={t[r]}, K={k[r]}, P={p[r]}, u={u[r]!r})"
            assert ids[r] == tok, f"{ctx}: gpu id {ids[r]} != oracle {tok}"
            if k[r] <= 0:
                assert o["flags"][r] & native.FLAG_FULL_PATH, ctx
                assert o["lsum"][r].view(np.uint32) == np.float32(det["lsum"]).view(np.uint32), \
                    f"{ctx}: lsum {o['lsum'][r]!r} != {det['lsum']!r}"
                assert o["argmax"][r] == det["argmax_pos"], \
                    f"{ctx}: argmax {o['argmax'][r]} != {det['argmax_pos']}"
            c = call[r]
            if isinstance(c[4], int) and p[r] > 0:  # the draw lands in the chunk aimed at
                assert ids[r] // 1024 == c[4] // 1024, f"{ctx}: id {ids[r]}, aimed at {c[4]}"
        d.free()
    s.close()
