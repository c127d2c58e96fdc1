"""GPU parity of the full-vocabulary path (TopK <= 0 or TopK >= V) against the
CPU oracle, through the C ABI.

The reference softcaps every logit, softmaxes over the whole vocabulary with
a left-to-right binary32 LSum, and draws by a left-to-right binary32 running
sum (src/Gemma4.Model.pas:2691-2737,2756-2763; src/Gemma4.Tensors.pas:638-673;
src/Gemma4.Layers.pas:300-316).  Token ids, LSum, the greedy id and (where
requested) every probability must equal the oracle's bit for bit; the stated
tolerance for probabilities is 1e-6 relative and exact equality is asserted.
Draws whose threshold lies within 1e-6 of a running-sum boundary are counted
and printed.
"""
import numpy as np
import pytest

from gemma4_sampler import hip, native, workload as wl

pytestmark = pytest.mark.gpu
F32 = np.float32
V = wl.V_GEMMA4
CAP = wl.SOFTCAP_GEMMA4
SEED = 4100


def _params(t, k, p):
    return [native.TSamplingParams.make(float(a), int(b), float(c)) for a, b, c in zip(t, k, p)]


def _widen(b16):
    return (np.asarray(b16, np.uint16).astype(np.uint32) << 16).view(F32)


def check(orc, rows, t, k, p, u, ids, o, softcap, label, probs=False, threads=1):
    boundary = 0

    def ref(r):
        return orc.do_sample(rows[r], t[r], k[r], p[r], u[r], softcap=softcap, want_probs=probs)

    if threads > 1:
        # the oracle call releases the GIL (ctypes), so rows run in parallel
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(threads) as ex:
            refs = list(ex.map(ref, range(len(rows))))
    else:
        refs = None
    for r in range(len(rows)):
        tok, det, _, pr = refs[r] if refs is not None else ref(r)
        ctx = f"{label} row {r} (T={t[r]}, K={k[r]}, P={p[r]}, u={u[r]!r}, cap={softcap})"
        assert ids[r] == tok, f"{ctx}: gpu id {ids[r]} != oracle {tok}"
        if o is not None:
            assert o["flags"][r] & native.FLAG_FULL_PATH, ctx
            assert o["lsum"][r].view(np.uint32) == np.float32(det["lsum"]).view(np.uint32), \
                f"{ctx}: lsum {o['lsum'][r]!r} != {det['lsum']!r}"
            assert o["argmax"][r] == det["argmax_pos"], ctx
            assert o["count"][r] == rows.shape[1], ctx
            if probs:
                n = rows.shape[1]
                gp = o["probs"][r][:n]
                assert np.array_equal(gp.view(np.uint32), pr.view(np.uint32)), f"{ctx}: probs"
                assert np.array_equal(o["indices"][r][:n], np.arange(n)), ctx
        if det["drew"] and det["reached"]:
            th = det["threshold"]
            d = min(th - det["cum_prev"] if det["chosen_pos"] > 0 else np.inf, det["cum_at"] - th)
            boundary += d < 1e-6
    return boundary


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("vocab", [2, 3, 7, 100, 1000, 5000, 16385, 40000])
def test_small_vocab_random(orc, vocab, dtype):
    """Every regime: dense ties, masked logits, T <= 0 / = 1 / other, P in
    [0, 1], softcap on and off, K <= 0 and K >= V, rows spanning chunks."""
    rng = np.random.default_rng(vocab * 7 + (dtype == "bf16"))
    B = 16
    rows = np.empty((B, vocab), F32)
    for r in range(B):
        kind = r % 4
        if kind == 0:
            rows[r] = rng.normal(0, 3, vocab)
        elif kind == 1:
            rows[r] = rng.integers(-3, 4, vocab)
        elif kind == 2:
            rows[r] = rng.normal(0, 0.5, vocab)
            rows[r][rng.random(vocab) < 0.2] = -np.inf
        else:
            rows[r] = rng.normal(0, 20, vocab)
    if dtype == "bf16":
        b16 = (rows.view(np.uint32) >> 16).astype(np.uint16)
        rows = _widen(b16)
    k = rng.choice([0, -1, vocab, vocab + 5], B).astype(np.int32)
    t = rng.choice([0.0, 0.7, 1.0, 1.3, -1.0], B).astype(F32)
    p = rng.choice([0.0, 0.5, 0.99, 1.0], B).astype(F32)
    u = np.floor(rng.random(B) * 2**32) / 2**32
    u[0] = 0.0
    u[1] = 1.0 - 2**-32
    esize = 4 if dtype == "f32" else 2
    stride = (vocab * esize + 15) // 16 * 16 // esize
    for softcap in (CAP, 0.0):
        s = native.Sampler(vocab, max_batch=B, softcap=softcap)
        if dtype == "f32":
            dev = np.full((B, stride), 1e30, F32)
            dev[:, :vocab] = rows
        else:
            dev = np.full((B, stride), 0x7F00, np.uint16)
            dev[:, :vocab] = b16
        d = hip.Buffer.from_array(dev)
        outs = native.DeviceOutputs(B, vocab)
        _, ids = s.sample(d, B, _params(t, k, p), u, row_stride=stride, outputs=outs.struct,
                          dtype=native.DTYPE_F32 if dtype == "f32" else native.DTYPE_BF16)
        check(orc, rows, t, k, p, u, ids, outs.read(), softcap, f"V={vocab} {dtype}",
              probs=True)
        s.close()


def test_flat_bf16_rows_full_size(orc):
    """The flat worst case: B=8 bf16 N(0, 0.5^2) rows, T=1, TopK disabled,
    P=0.99 -- the nucleus holds tens of thousands of tokens."""
    B = 8
    b16 = wl.host_flat_bf16_rows(SEED, 0, B, V)
    rows = _widen(b16)
    t, k, p = wl.flat_params(B)
    u = wl.host_row_u(SEED, 0, B)
    s = native.Sampler(V, max_batch=B, softcap=CAP)
    d = hip.Buffer.from_array(b16)
    outs = native.DeviceOutputs(B, 1)
    _, ids = s.sample(d, B, _params(t, k, p), u, dtype=native.DTYPE_BF16, outputs=outs.struct)
    nb = check(orc, rows, t, k, p, u, ids, outs.read(), CAP, "flat")
    print(f"flat bf16 rows: {B}, boundary draws (|u*P - cum| < 1e-6): {nb}")
    s.close()


def test_flat_bf16_probabilities_full_size(orc):
    """Every normalised probability of a full-size row equals the oracle's."""
    b16 = wl.host_flat_bf16_rows(SEED + 1, 0, 2, V)
    rows = _widen(b16)
    t = np.array([1.0, 0.8], F32)
    k = np.array([0, V], np.int32)
    p = np.array([0.99, 0.9], F32)
    u = wl.host_row_u(SEED + 1, 0, 2)
    s = native.Sampler(V, max_batch=2, softcap=CAP)
    d = hip.Buffer.from_array(b16)
    outs = native.DeviceOutputs(2, V)
    _, ids = s.sample(d, 2, _params(t, k, p), u, dtype=native.DTYPE_BF16, outputs=outs.struct)
    check(orc, rows, t, k, p, u, ids, outs.read(), CAP, "flat-probs", probs=True)
    s.close()


def test_peaky_fp32_full_path(orc):
    """fp32 logits through the full path (no table: every e evaluated)."""
    B = 3
    rows = wl.host_peaky_rows(SEED + 2, 0, B, V)
    t = np.array([0.7, 1.0, 0.0], F32)
    k = np.array([0, -5, V], np.int32)
    p = np.array([0.95, 0.5, 0.9], F32)
    u = wl.host_row_u(SEED + 2, 0, B)
    s = native.Sampler(V, max_batch=B, softcap=CAP)
    d = hip.Buffer.from_array(rows)
    outs = native.DeviceOutputs(B, 1)
    _, ids = s.sample(d, B, _params(t, k, p), u, outputs=outs.struct)
    check(orc, rows, t, k, p, u, ids, outs.read(), CAP, "peaky-full")
    s.close()


def test_mixed_topk_and_full_rows(orc):
    """One batch with top-k and full-vocabulary rows side by side."""
    B = 8
    b16 = wl.host_flat_bf16_rows(SEED + 3, 0, B, V)
    rows = _widen(b16)
    k = np.array([0, 64, 1, 0, 256, -1, 20, V], np.int32)
    t = np.array([1.0, 0.7, 0.7, 0.5, 1.2, 1.0, 0.9, 1.0], F32)
    p = np.array([0.99, 0.95, 0.95, 0.8, 1.0, 0.9, 0.9, 0.99], F32)
    u = wl.host_row_u(SEED + 3, 0, B)
    s = native.Sampler(V, max_batch=B, softcap=CAP)
    d = hip.Buffer.from_array(b16)
    _, ids = s.sample(d, B, _params(t, k, p), u, dtype=native.DTYPE_BF16)
    check(orc, rows, t, k, p, u, ids, None, CAP, "mixed")
    s.close()


def test_async_full_matches_sync(orc):
    B = 4
    b16 = wl.host_flat_bf16_rows(SEED + 4, 0, B, V)
    t, k, p = wl.flat_params(B)
    u = wl.host_row_u(SEED + 4, 0, B)
    s = native.Sampler(V, max_batch=B, softcap=CAP)
    d = hip.Buffer.from_array(b16)
    parr = native.params_array(_params(t, k, p))
    dp = hip.Buffer(16 * B)
    hip.check(hip.lib().hipMemcpy(dp.ptr, parr, 16 * B, hip.H2D))
    du = hip.Buffer.from_array(u)
    di = hip.Buffer(4 * B)
    s.sample_async(d, B, dp, du, 0, 1, di, dtype=native.DTYPE_BF16)
    hip.synchronize()
    _, ids = s.sample(d, B, _params(t, k, p), u, dtype=native.DTYPE_BF16)
    assert np.array_equal(di.download(np.int32), ids)
    check(orc, _widen(b16), t, k, p, u, ids, None, CAP, "async-full")
    s.close()


@pytest.mark.parametrize("B", [128, 256])
def test_flat_bf16_large_batches(orc, B):
    """The flat worst case at the batch sizes whose streaming passes take 2
    (B=128) and 4 (B=256) vocabulary chunks per wave: every id, LSum and
    greedy id against the oracle, and at B=256 every probability of every row
    (capacity >= V).  Boundary draws are counted and printed."""
    b16 = wl.host_flat_bf16_rows(SEED + 10 + B, 0, B, V)
    rows = _widen(b16)
    t, k, p = wl.flat_params(B)
    u = wl.host_row_u(SEED + 10 + B, 0, B)
    s = native.Sampler(V, max_batch=B, softcap=CAP)
    d = hip.Buffer.from_array(b16)
    cap = V if B == 256 else 1
    outs = native.DeviceOutputs(B, cap)
    _, ids = s.sample(d, B, _params(t, k, p), u, dtype=native.DTYPE_BF16, outputs=outs.struct)
    o = outs.read()
    del outs
    nb = check(orc, rows, t, k, p, u, ids, o, CAP, f"flat B={B}", probs=(cap == V), threads=16)
    print(f"flat bf16 B={B}: {B} rows bit-exact, boundary draws (|u*P - cum| < 1e-6): {nb}")
    s.close()
