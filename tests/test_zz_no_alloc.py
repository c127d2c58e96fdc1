"""g4s_sample_topk_noalloc -- the handle-free top-k entry point whose
workspace is a fixed device array -- against g4s_sample_async, the entry
point it is a variant of, through the C ABI: two calls in a row, the second
with a smaller input, every id and every optional output bit for bit, and
the ids against the oracle.  Size limits are rejected with a clear error."""
import numpy as np
import pytest

from gemma4_sampler import hip, native, workload as wl

pytestmark = pytest.mark.gpu
F32 = np.float32
V = wl.V_GEMMA4
CAP = wl.SOFTCAP_GEMMA4


def _dev_params(t, k, p):
    parr = native.params_array([native.TSamplingParams.make(float(a), int(b), float(c))
                                for a, b, c in zip(t, k, p)])
    dp = hip.Buffer(16 * len(t))
    hip.check(hip.lib().hipMemcpy(dp.ptr, parr, 16 * len(t), hip.H2D))
    return dp


def _both(d, B, dtype, t, k, p, u, k_bound, capacity):
    dp = _dev_params(t, k, p)
    du = hip.Buffer.from_array(np.asarray(u, np.float64))
    # the existing entry point, on its own handle
    s = native.Sampler(V, max_batch=B, softcap=CAP)
    di_a = hip.Buffer.from_array(np.full(B, 777, np.int32))
    out_a = native.DeviceOutputs(B, capacity)
    s.sample_async(d, B, dp, du, k_bound, 0, di_a, dtype=dtype, outputs=out_a.struct)
    hip.synchronize()
    s.close()
    # the allocation-free one
    di_n = hip.Buffer.from_array(np.full(B, 999, np.int32))
    out_n = native.DeviceOutputs(B, capacity)
    native.sample_topk_noalloc(d, B, dp, du, k_bound, di_n, V, dtype=dtype, softcap=CAP,
                               outputs=out_n.struct)
    hip.synchronize()
    return (di_a.download(np.int32), out_a.read()), (di_n.download(np.int32), out_n.read())


def _same(a, n, label):
    ids_a, oa = a
    ids_n, on = n
    assert np.array_equal(ids_a, ids_n), f"{label}: ids {ids_a} vs {ids_n}"
    assert np.array_equal(oa["flags"], on["flags"]), f"{label}: flags"
    for r in range(len(ids_a)):
        if oa["flags"][r] & native.FLAG_ERROR:
            continue  # a rejected row has only its id and flags written
        ctx = f"{label} row {r}"
        assert oa["count"][r] == on["count"][r] and oa["argmax"][r] == on["argmax"][r], ctx
        assert oa["lsum"][r:r + 1].view(np.uint32) == on["lsum"][r:r + 1].view(np.uint32), ctx
        c = min(int(oa["count"][r]), oa["indices"].shape[1])
        assert np.array_equal(oa["indices"][r][:c], on["indices"][r][:c]), ctx
        assert np.array_equal(oa["probs"][r][:c].view(np.uint32),
                              on["probs"][r][:c].view(np.uint32)), ctx


def test_noalloc_matches_async_two_calls(orc):
    # call 1: 24 fp32 decode-like rows, K in {1, 20, 64, 256}, one full row
    # (K = 0) and one row above k_bound, both rejected by either entry point
    B1 = 24
    rows1 = wl.host_peaky_rows(9001, 0, B1, V, greedy_every=5)
    t1, k1, p1 = wl.host_mixed_params(9001, 0, B1)
    k1 = k1.copy()
    k1[5] = 0
    k1[7] = 300
    u1 = wl.host_row_u(9001, 0, B1)
    d1 = hip.Buffer.from_array(rows1)
    a, n = _both(d1, B1, native.DTYPE_F32, t1, k1, p1, u1, 256, 256)
    _same(a, n, "call 1")
    ids = n[0]
    for r in range(B1):
        if r in (5, 7):
            assert ids[r] == -1 and n[1]["flags"][r] & native.FLAG_ERROR
            continue
        tok, _, _, _ = orc.do_sample(rows1[r], t1[r], k1[r], p1[r], u1[r], softcap=CAP,
                                     want_probs=False)
        assert ids[r] == tok, f"call 1 row {r}: {ids[r]} != oracle {tok}"
    # call 2: a smaller input -- 3 bf16 rows, k_bound 64
    B2 = 3
    b16 = wl.host_flat_bf16_rows(9002, 0, B2, V)
    rows2 = (b16.astype(np.uint32) << 16).view(F32)
    t2 = np.array([0.7, 1.0, 0.0], F32)
    k2 = np.array([64, 1, 20], np.int32)
    p2 = np.array([0.95, 0.9, 0.8], F32)
    u2 = wl.host_row_u(9002, 0, B2)
    d2 = hip.Buffer.from_array(b16)
    a, n = _both(d2, B2, native.DTYPE_BF16, t2, k2, p2, u2, 64, 64)
    _same(a, n, "call 2")
    for r in range(B2):
        tok, _, _, _ = orc.do_sample(rows2[r], t2[r], k2[r], p2[r], u2[r], softcap=CAP,
                                     want_probs=False)
        assert n[0][r] == tok, f"call 2 row {r}"


def test_noalloc_rejects_sizes_beyond_its_array():
    d = hip.Buffer.from_array(np.zeros(V, F32))
    dp = _dev_params([1.0], [5], [0.9])
    du = hip.Buffer.from_array(np.array([0.5]))
    di = hip.Buffer(4 * 64)
    L = native.load()
    rc = native.sample_topk_noalloc(d, native.NOALLOC_MAX_ROWS + 1, dp, du, 64, di, 1024,
                                    check=False)
    assert rc == native.G4S_ERR_INVALID_ARGUMENT
    assert "G4S_NOALLOC_MAX_ROWS" in L.g4s_last_error(None).decode()
    rc = native.sample_topk_noalloc(d, 1, dp, du, native.max_top_k() + 1, di, V, check=False)
    assert rc == native.G4S_ERR_INVALID_ARGUMENT and "k_bound" in L.g4s_last_error(None).decode()
    rc = native.sample_topk_noalloc(d.offset(4), 1, dp, du, 64, di, V, check=False)
    assert rc == native.G4S_ERR_INVALID_ARGUMENT and "aligned" in L.g4s_last_error(None).decode()
