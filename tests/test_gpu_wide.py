"""GPU parity of the wide top-k path (g4s_max_top_k() < TopK < V) against the
CPU oracle, through the C ABI.

DoSelectTopKIndices keeps the K largest logits by a min-heap whose layout
decides which copies of a tied K-th value survive
(src/Gemma4.Model.pas:2615-2689); the tail softcaps, scales, softmaxes with a
left-to-right binary32 LSum and a division, and draws by a left-to-right
running sum (Model.pas:2765-2826).  Token ids, the survivor index set (in
ascending order), every probability, LSum and the greedy id must equal the
oracle's bit for bit (the stated tolerance for probabilities, 1e-6 relative,
is met with equality).  The rows below force both tie rules: the lowest-index
rule and the exact heap replay.
"""
import numpy as np
import pytest

from gemma4_sampler import hip, native, workload as wl

pytestmark = pytest.mark.gpu
F32 = np.float32
V = wl.V_GEMMA4
CAP = wl.SOFTCAP_GEMMA4
KMAX = 1024


def _params(t, k, p):
    return [native.TSamplingParams.make(float(a), int(b), float(c)) for a, b, c in zip(t, k, p)]


def _widen(b16):
    return (np.asarray(b16, np.uint16).astype(np.uint32) << 16).view(F32)


def check(orc, rows, t, k, p, u, ids, o, softcap, label, capacity=None):
    """Every row against the oracle; returns the flags seen."""
    seen = 0
    for r in range(len(rows)):
        tok, det, idx, probs = orc.do_sample(rows[r], t[r], k[r], p[r], u[r], softcap=softcap)
        ctx = f"{label} row {r} (T={t[r]}, K={k[r]}, P={p[r]}, u={u[r]!r}, cap={softcap})"
        assert ids[r] == tok, f"{ctx}: gpu id {ids[r]} != oracle {tok}"
        if o is None:
            continue
        n = det["count"]
        assert o["count"][r] == n, f"{ctx}: count {o['count'][r]} != {n}"
        m = n if capacity is None else min(n, capacity)
        assert np.array_equal(o["indices"][r][:m], idx[:m]), f"{ctx}: survivor indices"
        assert np.array_equal(o["probs"][r][:m].view(np.uint32), probs[:m].view(np.uint32)), \
            f"{ctx}: probs"
        assert o["lsum"][r:r + 1].view(np.uint32)[0] == np.float32(det["lsum"]).view(np.uint32), \
            f"{ctx}: lsum"
        assert o["argmax"][r] == idx[det["argmax_pos"]], f"{ctx}: argmax"
        assert o["flags"][r] & native.FLAG_TOPK_PATH, ctx
        if k[r] > KMAX:
            assert o["flags"][r] & native.FLAG_WIDE_K, ctx
        seen |= int(o["flags"][r])
    return seen


def _run(orc, rows, t, k, p, u, softcap, dtype, label, capacity=None):
    B, vocab = rows.shape
    esize = 4 if dtype == "f32" else 2
    stride = (vocab * esize + 15) // 16 * 16 // esize
    if dtype == "f32":
        dev = np.full((B, stride), -1e30, F32)
        dev[:, :vocab] = rows
        host = rows
    else:
        b16 = (rows.view(np.uint32) >> 16).astype(np.uint16)
        dev = np.full((B, stride), 0xFF80, np.uint16)  # -inf padding
        dev[:, :vocab] = b16
        host = _widen(b16)
    s = native.Sampler(vocab, max_batch=B, softcap=softcap)
    d = hip.Buffer.from_array(dev)
    cap = vocab if capacity is None else capacity
    outs = native.DeviceOutputs(B, cap)
    _, ids = s.sample(d, B, _params(t, k, p), u, row_stride=stride, outputs=outs.struct,
                      dtype=native.DTYPE_F32 if dtype == "f32" else native.DTYPE_BF16)
    seen = check(orc, host, t, k, p, u, ids, outs.read(), softcap, label, capacity)
    s.close()
    return seen


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("vocab", [1100, 3000, 20000])
def test_wide_small_vocab(orc, vocab, dtype):
    """Random rows, integer rows (heavy ties at the K-th value), masked rows;
    T <= 0 / 1 / other, P in [0, 1], u at 0 and near 1, softcap on and off."""
    rng = np.random.default_rng(vocab * 3 + (dtype == "bf16"))
    B = 12
    rows = np.empty((B, vocab), F32)
    for r in range(B):
        kind = r % 4
        if kind == 0:
            rows[r] = rng.normal(0, 3, vocab)
        elif kind == 1:
            rows[r] = rng.integers(-3, 4, vocab)
        elif kind == 2:
            rows[r] = rng.normal(0, 0.5, vocab)
            rows[r][rng.random(vocab) < 0.5] = -np.inf
        else:
            rows[r] = rng.integers(0, 2, vocab) * 4.0
    k = rng.integers(KMAX + 1, vocab, B).astype(np.int32)
    k[1] = vocab - 1
    t = rng.choice([0.0, 0.7, 1.0, 1.3], B).astype(F32)
    p = rng.choice([0.0, 0.5, 0.95, 1.0], B).astype(F32)
    u = np.floor(rng.random(B) * 2**32) / 2**32
    u[0] = 0.0
    u[2] = 1.0 - 2**-32
    seen = 0
    for softcap in (CAP, 0.0):
        seen |= _run(orc, rows, t, k, p, u, softcap, dtype, f"V={vocab} {dtype}")
    print(f"V={vocab} {dtype}: flags seen {seen:#x}")


def test_wide_tie_rules_both_exercised(orc):
    """Rows built so that the K-th value is tied: one where every larger
    value comes first (lowest-index rule), one where larger values follow
    the tied copies (heap replay)."""
    vocab = 5000
    K = 2000
    low = np.zeros(vocab, F32)
    low[:1500] = 5.0                      # all larger values first
    low[1500:] = 1.0                      # then 3500 copies of the K-th value
    heap = np.ones(vocab, F32)            # copies of the K-th value first ...
    heap[3000:4500] = 5.0                 # ... then the larger values
    rows = np.stack([low, heap, low, heap])
    t = np.array([1.0, 1.0, 0.7, 0.0], F32)
    k = np.full(4, K, np.int32)
    p = np.array([0.9, 0.9, 1.0, 0.9], F32)
    u = np.array([0.3, 0.6, 0.99, 0.5])
    seen = 0
    for dtype in ("f32", "bf16"):
        seen |= _run(orc, rows, t, k, p, u, CAP, dtype, f"ties {dtype}")
    assert seen & native.FLAG_TIE_LOWEST
    assert seen & native.FLAG_HEAP_REPLAY


def test_wide_capacity_below_count(orc):
    vocab = 4000
    rng = np.random.default_rng(11)
    rows = rng.normal(0, 2, (3, vocab)).astype(F32)
    t = np.array([0.8, 1.0, 1.2], F32)
    k = np.array([1500, 3999, 2048], np.int32)
    p = np.array([0.95, 0.9, 1.0], F32)
    u = np.array([0.1, 0.5, 0.9])
    _run(orc, rows, t, k, p, u, CAP, "f32", "capacity", capacity=1200)


def test_wide_full_size_rows(orc):
    """V=262144: K = V-1 on flat bf16 rows and K = 100000 on peaky fp32 rows."""
    B = 4
    b16 = wl.host_flat_bf16_rows(9001, 0, B, V)
    rows = _widen(b16)
    t = np.array([1.0, 0.7, 1.0, 0.0], F32)
    k = np.array([V - 1, V - 1, 5000, V - 1], np.int32)
    p = np.array([0.99, 0.95, 0.9, 0.9], F32)
    u = wl.host_row_u(9001, 0, B)
    s = native.Sampler(V, max_batch=B, softcap=CAP)
    d = hip.Buffer.from_array(b16)
    outs = native.DeviceOutputs(B, V)
    _, ids = s.sample(d, B, _params(t, k, p), u, dtype=native.DTYPE_BF16, outputs=outs.struct)
    check(orc, rows, t, k, p, u, ids, outs.read(), CAP, "flat bf16 wide")
    d.free()
    rows = wl.host_peaky_rows(9002, 0, 2, V)
    d = hip.Buffer.from_array(rows)
    t2, k2, p2 = np.array([0.7, 1.3], F32), np.array([100000, 2000], np.int32), \
        np.array([0.95, 0.8], F32)
    u2 = wl.host_row_u(9002, 0, 2)
    _, ids = s.sample(d, 2, _params(t2, k2, p2), u2)
    check(orc, rows, t2, k2, p2, u2, ids, None, CAP, "peaky fp32 wide")
    s.close()


def test_wide_mixed_with_topk_and_full_rows_async(orc):
    """One batch with top-k, wide and full rows, through the stream-ordered
    entry point (k_bound above g4s_max_top_k() adds the wide launches) and
    through the synchronous one."""
    B = 6
    b16 = wl.host_flat_bf16_rows(9003, 0, B, V)
    rows = _widen(b16)
    k = np.array([64, 3000, 0, V - 1, 1, 100000], np.int32)
    t = np.array([0.7, 1.0, 1.0, 0.9, 0.7, 1.1], F32)
    p = np.array([0.95, 0.9, 0.99, 0.95, 0.9, 0.8], F32)
    u = wl.host_row_u(9003, 0, B)
    s = native.Sampler(V, max_batch=B, softcap=CAP)
    d = hip.Buffer.from_array(b16)
    parr = native.params_array(_params(t, k, p))
    dp = hip.Buffer(16 * B)
    hip.check(hip.lib().hipMemcpy(dp.ptr, parr, 16 * B, hip.H2D))
    du = hip.Buffer.from_array(u)
    di = hip.Buffer(4 * B)
    s.sample_async(d, B, dp, du, int(V - 1), 1, di, dtype=native.DTYPE_BF16)
    hip.synchronize()
    got = di.download(np.int32)
    _, ids = s.sample(d, B, _params(t, k, p), u, dtype=native.DTYPE_BF16)
    assert np.array_equal(got, ids)
    check(orc, rows, t, k, p, u, ids, None, CAP, "mixed wide")
    s.close()
