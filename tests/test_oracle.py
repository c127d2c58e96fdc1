"""Pins the CPU oracle (oracle/g4s_oracle.cpp) against closed forms,
invariants, brute force and hand-traced heap cases, so that a plausible
restatement mistake (a dropped term, a flipped comparison, a wrong index)
fails here.  The reference ships no sampler tests or golden vectors."""
import itertools

import numpy as np
import pytest

F32 = np.float32


def test_semantics_switch(orc):
    assert orc.load().orc_semantics().decode() == "Extended=x87-80bit"
    assert orc.load(double=True).orc_semantics().decode() == "Extended=binary64"


# --------------------------------------------------------------- a6 top-k
def test_heap_tie_counterexample(orc):
    # Hand trace of Model.pas:2632-2664 on [1,1,4,2], K=3: index 0 is evicted.
    assert list(orc.select_topk_indices([1, 1, 4, 2], 3)) == [1, 2, 3]


def test_heap_hand_traces(orc):
    # [5,5,5] K=2: third 5 is rejected (v <= root) -> first two survive
    assert list(orc.select_topk_indices([5, 5, 5], 2)) == [0, 1]
    # [1,2,2,3] K=2: 1 in, 2 in (root 1), 2@2 replaces root 1, 3 replaces root (2@1 or 2@2)
    # heap after 2@2: [(2,2),(2,1)]? trace: init[-e,-e]; 1@0 -> child=1: -e<1 -> heap[0]=-e,pos=1 ->
    # [(-e),(1,0)]; 2@1 root -e: child 1 (1,0) >= 2? no -> heap[0]=(1,0), pos=1 -> [(1,0),(2,1)];
    # 2@2: root 1 < 2: child 1 (2,1) >= 2 -> break -> heap[0]=(2,2) -> [(2,2),(2,1)];
    # 3@3: root 2 < 3: child (2,1) >= 3? no -> heap[0]=(2,1), pos 1 -> [(2,1),(3,3)]
    assert list(orc.select_topk_indices([1, 2, 2, 3], 2)) == [1, 3]


def _brute_multiset(x, k):
    v = np.array(x, F32)
    valid = v[v > F32(-1e30)]
    return sorted(valid.tolist(), reverse=True)[:k]


@pytest.mark.parametrize("seed", range(6))
def test_topk_multiset_and_order(orc, seed):
    rng = np.random.default_rng(seed)
    for _ in range(60):
        V = int(rng.integers(1, 300))
        alphabet = rng.integers(2, 40)
        x = rng.integers(0, alphabet, V).astype(F32) - alphabet / 2
        if rng.random() < 0.3:
            x[rng.random(V) < 0.2] = -np.inf
        K = int(rng.integers(1, V + 2))
        idx = orc.select_topk_indices(x, K)
        assert list(idx) == sorted(idx), "ascending by index"
        assert len(set(idx.tolist())) == len(idx)
        assert sorted(x[idx].tolist(), reverse=True) == _brute_multiset(x, K)


def test_k1_is_first_argmax(orc):
    rng = np.random.default_rng(7)
    for _ in range(200):
        x = rng.integers(0, 5, int(rng.integers(1, 50))).astype(F32)
        assert list(orc.select_topk_indices(x, 1)) == [int(np.argmax(x))]


def test_exhaustive_tiny(orc):
    # all rows over {0,1,2} of length <= 6, all K: multiset + ascending + K=1 rule
    for V in range(1, 7):
        for row in itertools.product([0.0, 1.0, 2.0], repeat=V):
            x = np.array(row, F32)
            for K in range(1, V + 1):
                idx = orc.select_topk_indices(x, K)
                assert sorted(x[idx].tolist(), reverse=True) == _brute_multiset(x, K)
                assert list(idx) == sorted(idx)
            assert list(orc.select_topk_indices(x, 1)) == [int(np.argmax(x))]


def test_minus_1e30_never_selected(orc):
    x = np.array([-1e30, -1e30, -3e38, 0.5], F32)
    assert list(orc.select_topk_indices(x, 3)) == [3]
    assert list(orc.select_topk_indices(np.array([-1e30], F32), 1)) == []


# --------------------------------------------------------------- a9 softcap
def test_softcap_closed_forms(orc):
    assert orc.softcap_topk(0.0) == 0.0
    assert orc.logit_softcap([0.0])[0] == 0.0
    for x in (0.3, 2.0, 17.0, 29.0, 100.0):
        assert orc.softcap_topk(-x) == -orc.softcap_topk(x)
    assert orc.softcap_topk(1e6) == F32(30.0)
    assert orc.logit_softcap([1e6])[0] == F32(30.0)
    xs = np.linspace(-80, 80, 4001, dtype=F32)
    ys = np.array([orc.softcap_topk(x) for x in xs])
    assert np.all(np.diff(ys) >= 0), "monotone"


def test_softcap_forms_are_correctly_rounded(orc):
    mp = pytest.importorskip("mpmath")
    mp.mp.dps = 50
    rng = np.random.default_rng(3)
    inv = F32(1.0) / F32(30.0)
    for x in rng.normal(0, 12, 300).astype(F32):
        a = mp.mpf(float(x))
        exact_topk = 30 * mp.tanh(a / 30)
        exact_full = mp.tanh(a * mp.mpf(float(inv))) * 30
        assert orc.softcap_topk(x) == _rn32(exact_topk)
        assert orc.logit_softcap([x])[0] == _rn32(exact_full)


def _rn32(v):
    import mpmath as mp
    f = F32(float(v))
    cands = [f, np.nextafter(f, F32(np.inf)), np.nextafter(f, F32(-np.inf))]
    return min(cands, key=lambda c: abs(mp.mpf(float(c)) - v))


# --------------------------------------------------------------- a8 softmax
def test_softmax_sequential_sum(orc):
    rng = np.random.default_rng(11)
    x = rng.normal(0, 2, 5000).astype(F32)
    p, lsum = orc.softmax_f32(x)
    m = x.max()
    e = np.array([orc.exp_diff(v, m) for v in x], F32)
    assert lsum == np.cumsum(e, dtype=F32)[-1], "left-to-right binary32 sum"
    inv = F32(1.0) / lsum
    assert np.array_equal(p, e * inv), "reciprocal multiply, not division"
    assert abs(float(lsum) - float(np.sum(e.astype(np.float64)))) < 1e-3 * float(lsum)


def test_seqsum_literal(orc):
    rng = np.random.default_rng(12)
    a = rng.random(100000).astype(F32)
    s, first = orc.seqsum(a, F32(1000.5))
    c = np.cumsum(a, dtype=F32)
    assert s == c[-1]
    assert first == int(np.argmax(c >= F32(1000.5)))


# --------------------------------------------------- a5/a7 DoSample tail
def test_equal_logits_uniform(orc):
    x = np.zeros(1000, F32)
    tok, det, idx, probs = orc.do_sample(x, 0.7, 8, 0.95, 0.0)
    assert list(idx) == list(range(8))  # K-th value tied everywhere: heap keeps indices 0..7
    assert np.all(probs == F32(1.0) / F32(8.0))


def test_u_zero_picks_first_survivor(orc):
    rng = np.random.default_rng(5)
    x = rng.normal(0, 3, 4096).astype(F32)
    for k in (5, 64, 0):
        tok, det, idx, probs = orc.do_sample(x, 0.7, k, 0.95, 0.0)
        assert tok == int(idx[0]) and det["chosen_pos"] == 0


def test_threshold_above_total_falls_back_to_argmax(orc):
    x = np.array([0.0, 3.0, 1.0, 3.0], F32)
    # P huge => u*P beyond the final running sum
    tok, det, idx, probs = orc.do_sample(x, 1.0, 3, 1e30, 0.5)
    assert det["reached"] == 0 and tok == int(idx[det["argmax_pos"]])
    assert tok == 1  # first maximum of p


def test_temperature_nonpositive_is_greedy(orc):
    rng = np.random.default_rng(6)
    x = rng.normal(0, 3, 2048).astype(F32)
    for T in (0.0, -1.0):
        for k in (10, 0):
            tok, det, idx, probs = orc.do_sample(x, T, k, 0.95, 0.9)
            assert det["drew"] == 0
            assert tok == int(np.argmax(x))


def test_temperature_one_is_unscaled(orc):
    rng = np.random.default_rng(8)
    x = rng.normal(0, 3, 1024).astype(F32)
    _, _, idx1, p1 = orc.do_sample(x, 1.0, 16, 0.9, 0.3, softcap=0.0)
    e = np.array([orc.exp_diff(v, x[idx1].max()) for v in x[idx1]], F32)
    lsum = np.cumsum(e, dtype=F32)[-1]
    assert np.array_equal(p1, e / lsum)


def test_topp_nonpositive_picks_first(orc):
    rng = np.random.default_rng(9)
    x = rng.normal(0, 3, 1024).astype(F32)
    tok, det, idx, _ = orc.do_sample(x, 0.8, 32, 0.0, 0.77)
    assert det["chosen_pos"] == 0


def test_position_monotone_in_u(orc):
    rng = np.random.default_rng(10)
    x = rng.normal(0, 1, 2048).astype(F32)
    for k in (64, 0):
        last = -1
        for u in np.linspace(0, 0.999, 40):
            _, det, _, _ = orc.do_sample(x, 1.3, k, 0.9, u)
            assert det["chosen_pos"] >= last
            last = det["chosen_pos"]


def test_full_path_matches_pieces(orc):
    rng = np.random.default_rng(13)
    x = rng.normal(0, 1, 3000).astype(F32)
    T, P, u = 0.8, 0.9, 0.37
    s = orc.logit_softcap(x)
    inv = F32(1.0) / F32(T)
    s = s * inv
    p, lsum = orc.softmax_f32(s)
    t = F32(np.float64(u) * np.float64(F32(P)))
    c = np.cumsum(p, dtype=F32)
    want = int(np.argmax(c >= t))
    tok, det, idx, probs = orc.do_sample(x, T, 0, P, u)
    assert tok == want and np.array_equal(probs, p) and det["lsum"] == lsum


# ----------------------------------------------------- conversions / Q4_0
def test_bf16_widening_exhaustive(orc):
    # every non-NaN bf16 pattern (ctypes' float return quiets signalling NaNs)
    bits = np.arange(65536, dtype=np.uint32)
    not_nan = ((bits >> 7) & 0xFF) != 0xFF
    not_nan |= (bits & 0x7F) == 0
    want = (bits << 16).view(F32)
    got = np.array([orc.bf16_to_f32(b) for b in bits[not_nan]], F32)
    assert np.array_equal(got.view(np.uint32), want[not_nan].view(np.uint32))


def test_f16_normals_match_ieee_and_denormal_quirk(orc):
    for b in list(range(0x0400, 0x7C00, 97)) + [0x3C00, 0xBC00, 0x7BFF]:
        assert orc.f16_to_f32(b) == np.array([b], np.uint16).view(np.float16).astype(F32)[0]
    # Types.pas:459-463 raises the exponent while normalising a denormal:
    # 0x0001 decodes to 2^-4, not 2^-24 (restated as written)
    assert orc.f16_to_f32(0x0001) == F32(0.0625)
    assert orc.f16_from_f32(F32(1.0)) == 0x3C00
    assert orc.f16_from_f32(F32(1e-6)) == 0  # flush to zero


def test_q4_roundtrip(orc):
    rng = np.random.default_rng(14)
    x = rng.normal(0, 1, 32 * 50).astype(F32)
    q = orc.f32_to_q4(x)
    for b in range(50):
        blk = q[b * 18:(b + 1) * 18]
        d = orc.dequant_q4_block(blk)
        scale = orc.f16_to_f32(int(blk[0]) | (int(blk[1]) << 8))
        assert np.all(np.abs(d - x[b * 32:(b + 1) * 32]) <= scale * 1.5 + 1e-6)


def test_matvec_q4_one_hot_and_ones(orc):
    rng = np.random.default_rng(15)
    rows, cols = 16, 128
    w = rng.integers(0, 256, rows * (cols // 32) * 18).astype(np.uint8)
    for r in range(rows):
        for b in range(cols // 32):  # plausible fp16 scales
            off = (r * (cols // 32) + b) * 18
            s = orc.f16_from_f32(F32(rng.uniform(0.001, 0.02)))
            w[off], w[off + 1] = s & 0xFF, s >> 8
    deq = np.concatenate([orc.dequant_q4_block(w[i * 18:(i + 1) * 18])
                          for i in range(rows * cols // 32)]).reshape(rows, cols)
    for c in (0, 1, 31, 32, 77, 127):
        h = np.zeros(cols, F32)
        h[c] = 1.0
        assert np.array_equal(orc.matvec_q4(w, h, rows, cols), deq[:, c])
    ones = np.ones(cols, F32)
    got = orc.matvec_q4(w, ones, rows, cols)
    want = np.array([np.cumsum(deq[r], dtype=F32)[-1] for r in range(rows)], F32)
    assert np.array_equal(got, want)


# ------------------------------------------- pins written out by hand
def test_heap_child_tie_rule(orc):
    # Hand trace of Model.pas:2632-2664 on [0,0,0,1,1], K=4.  The sift-down
    # takes the right child only when it is strictly smaller
    # (LHeapVal[LChild+1] < LHeapVal[LChild], :2653-2654):
    #   after 0@0, 0@1, 0@2 the heap is [-1e30, (0,1), (0,2), (0,0)];
    #   1@3: children (0,1), (0,2) tie -> left: heap [(0,1), (0,0), (0,2), (1,3)];
    #   1@4: children (0,0), (0,2) tie -> left, then (1,3) >= 1 stops:
    #        heap [(0,0), (1,4), (0,2), (1,3)]  -> indices {0,2,3,4}.
    # Under `<=` the right child would be taken and the result is {0,1,3,4}.
    assert list(orc.select_topk_indices([0, 0, 0, 1, 1], 4)) == [0, 2, 3, 4]
    # [2,2,2,2,3,3] K=5: after the four 2s the heap is
    # [-1e30, (2,2), (2,3), (2,0), (2,1)]; 3@4 walks the left children (2,2),
    # (2,0): [(2,2), (2,0), (2,3), (3,4), (2,1)]; 3@5 goes left to (2,0),
    # then right to the strictly smaller (2,1): [(2,0), (2,1), (2,3), (3,4),
    # (3,5)] -> {0,1,3,4,5}.  Under `<=` the same row gives {1,2,3,4,5}.
    assert list(orc.select_topk_indices([2, 2, 2, 2, 3, 3], 5)) == [0, 1, 3, 4, 5]


# Q4_0 block = fp16 scale (little-endian) + 16 bytes; byte j holds element 2j
# in its low nibble and element 2j+1 in its high nibble, value = nibble - 8
# (Types.pas:139-142, Quant.pas:209-239, Tensors.pas:581-593).
_HAND_BLOCK = bytes([0x00, 0x3C,                      # scale 1.0
                     0x9A, 0x0F, 0xF0] + [0x88] * 13)
_HAND_VALUES = [2.0, 1.0, 7.0, -8.0, -8.0, 7.0] + [0.0] * 26


def test_q4_dequant_hand_built_blocks(orc):
    blk = np.frombuffer(_HAND_BLOCK, np.uint8)
    assert list(orc.dequant_q4_block(blk)) == _HAND_VALUES
    half = np.frombuffer(bytes([0x00, 0x38]) + _HAND_BLOCK[2:], np.uint8)   # scale 0.5
    assert list(orc.dequant_q4_block(half)) == [v * 0.5 for v in _HAND_VALUES]
    neg = np.frombuffer(bytes([0x00, 0xB8]) + _HAND_BLOCK[2:], np.uint8)    # scale -0.5
    assert list(orc.dequant_q4_block(neg)) == [v * -0.5 + 0.0 for v in _HAND_VALUES]


def test_q4_quantize_bankers_round_and_interleave(orc):
    # max |x| = 7 -> scale = 7/7 = 1 exactly, 1/scale = 1: Round(x) applies to
    # x itself, and Delphi's Round sends exact halves to the even integer
    x1 = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 6.5, 7.0, -7.0, 4.5, -3.5, 5.5, -5.5, 0.0, 1.0,
          -6.5, 0.25, 0.75, -4.5, 2.0, -2.0, 3.0, -3.0, 4.0, -4.0, 5.0, -5.0, 6.0, -6.0, 0.4, -0.6]
    # q = 0 2 2 0 -2 -2 4 6 7 -7 4 -4 6 -6 0 1 -6 0 1 -4 2 -2 3 -3 4 -4 5 -5 6 -6 0 -1
    want1 = [0x00, 0x3C, 0xA8, 0x8A, 0x66, 0xEC, 0x1F, 0x4C, 0x2E, 0x98,
             0x82, 0x49, 0x6A, 0x5B, 0x4C, 0x3D, 0x2E, 0x78]
    # max |x| = 3.5 -> scale 0.5 (fp16 0x3800), 1/scale = 2: 0.25 -> Round(0.5) = 0,
    # 0.75 -> Round(1.5) = 2, -0.75 -> -2, 1.25 -> Round(2.5) = 2, -1.25 -> -2
    x2 = [3.5, 0.25, 0.75, -0.75, 1.25, -1.25] + [0.0] * 26
    want2 = [0x00, 0x38, 0x8F, 0x6A, 0x6A] + [0x88] * 13
    q = orc.f32_to_q4(np.array(x1 + x2, F32))
    assert list(q[:18]) == want1
    assert list(q[18:36]) == want2


def test_matvec_q4_hand_values(orc):
    cols = 32
    w = np.frombuffer(_HAND_BLOCK + bytes([0x00, 0x3C, 0x99, 0x79] + [0x88] * 14), np.uint8)
    # row 0: 2*1 + 1*10 + 7*100 - 8*1000 - 8*0.5 + 7*0.25 = -7290.25
    h = np.zeros(cols, F32)
    h[:6] = [1, 10, 100, 1000, 0.5, 0.25]
    assert orc.matvec_q4(w, h, 2, cols)[0] == F32(-7290.25)
    # row 1 (q = 1, 1, 1, -1) with h = (2^24, 1, 1, 2^24): the left-to-right
    # binary32 sum is ((2^24 + 1) + 1) - 2^24 = 0 (each +1 is a tie that
    # rounds to the even 2^24); a pairwise sum would give 1, a reversed one 2
    h = np.zeros(cols, F32)
    h[:4] = [2.0 ** 24, 1.0, 1.0, 2.0 ** 24]
    assert orc.matvec_q4(w, h, 2, cols)[1] == F32(0.0)


def _f32_from_bits(b):
    return np.array([b], np.uint32).view(F32)[0]


def test_bf16_from_single_truncates(orc):
    """TBFloat16.FromSingle (Types.pas:426-434) truncates.  Values chosen so
    that round-to-nearest(-even) gives another code: 0x3F80FFFF lies just
    below 0x3F81 and 0x3F818000 is a tie whose even neighbour is 0x3F82."""
    for bits, want in ((0x3F80FFFF, 0x3F80), (0xBF80FFFF, 0xBF80), (0x3F818000, 0x3F81),
                       (0x7F7FFFFF, 0x7F7F), (0x00000001, 0x0000), (0x80000000, 0x8000)):
        assert orc.f32_to_bf16(_f32_from_bits(bits)) == want, hex(bits)
    # every non-NaN bf16 value converts back to its own code
    codes = np.arange(65536, dtype=np.uint32)
    ok = (((codes >> 7) & 0xFF) != 0xFF) | ((codes & 0x7F) == 0)
    for c in codes[ok][::7]:
        assert orc.f32_to_bf16(orc.bf16_to_f32(int(c))) == c
    # truncation toward zero: the code's value has x's sign, is no larger in
    # magnitude than x, and the next code up in magnitude is larger than x
    rng = np.random.default_rng(31)
    xs = rng.normal(0, 1, 2000).astype(F32) * F32(2.0) ** rng.integers(-60, 60, 2000).astype(F32)
    for x in xs:
        b = orc.f32_to_bf16(x)
        w = orc.bf16_to_f32(b)
        up = orc.bf16_to_f32(b + 1)
        assert np.signbit(w) == np.signbit(x) and abs(w) <= abs(x) < abs(up), (x, hex(b))


def test_f16_from_single_truncates(orc):
    """TFloat16.FromSingle (Types.pas:483-501): truncation, results below the
    smallest normal flushed to a signed zero, overflow to infinity.  Each
    value below rounds to a different code under round-to-nearest."""
    h = F32(2.0) ** -11  # half a unit of f16 at 1.0
    for x, want in ((F32(1) + h + F32(2.0) ** -23, 0x3C00),  # just above a half-unit
                    (F32(1) + 2 * h - F32(2.0) ** -23, 0x3C00),  # just below the next code
                    (F32(-1) - h - F32(2.0) ** -23, 0xBC00),
                    (F32(65535.0), 0x7BFF),  # round-to-nearest would overflow
                    (F32(65536.0), 0x7C00),
                    (F32(2.0) ** -14, 0x0400),  # smallest normal
                    (F32(2.0) ** -14 * F32(1 - 2.0 ** -24), 0x0000),  # just below: flushed
                    (-F32(2.0) ** -15, 0x8000)):
        assert orc.f16_from_f32(x) == want, (x, want)
    # every normal f16 code converts back to itself (the decode is pinned to
    # IEEE half for normals above)
    for c in list(range(0x0400, 0x7C00, 13)) + list(range(0x8400, 0xFC00, 29)):
        assert orc.f16_from_f32(orc.f16_to_f32(c)) == c, hex(c)
    # truncation toward zero against numpy's IEEE half decode
    rng = np.random.default_rng(32)
    xs = (rng.uniform(-1, 1, 2000) * 2.0 ** rng.integers(-13, 15, 2000)).astype(F32)
    for x in xs:
        c = orc.f16_from_f32(x)
        if (c & 0x7C00) == 0:
            continue
        dec = np.array([c], np.uint16).view(np.float16).astype(F32)[0]
        nxt = np.array([c + 1], np.uint16).view(np.float16).astype(F32)[0]
        assert np.signbit(dec) == np.signbit(x) and abs(dec) <= abs(x) < abs(nxt), (x, hex(c))
