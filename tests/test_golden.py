"""Golden fixtures (tests/golden/*.json, written by tests/golden/make_golden.py).

CPU tests: the oracle still reproduces every fixture, and the fixtures agree
with what the reference's algorithm fixes independently of any rounding
(survivors are the K largest in ascending index order, K=1 and T<=0 pick the
first maximum, u=0 picks the first survivor, the draw position is monotone
in u).  GPU tests: the HIP path through the C ABI reproduces every fixture
bit for bit (token, LSum, argmax, survivor indices, probabilities).
"""
import hashlib
import json
import os
from collections import defaultdict

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
F32 = np.float32


def _load(name):
    with open(os.path.join(HERE, name)) as f:
        return json.load(f)


SMALL = _load("small.json")["cases"]
LARGE = _load("large.json")


def _row(c):
    return np.asarray(c["logits"], np.uint32).view(F32)


def _digest(idx, probs):
    h = hashlib.sha256()
    h.update(np.asarray(idx, np.int32).tobytes())
    h.update(np.asarray(probs, F32).tobytes())
    return h.hexdigest()


def test_oracle_reproduces_small_fixtures(orc):
    for c in SMALL:
        tok, det, idx, probs = orc.do_sample(_row(c), c["t"], c["k"], c["p"], c["u"],
                                             softcap=c["softcap"])
        assert tok == c["token"], c["label"]
        assert int(F32(det["lsum"]).view(np.uint32)) == c["lsum"], c["label"]
        assert list(idx) == c["indices"], c["label"]
        assert [int(b) for b in probs.view(np.uint32)] == c["probs"], c["label"]


def test_fixtures_obey_rounding_free_facts():
    """Facts of src/Gemma4.Model.pas:2615-2827 that no rounding can change."""
    for c in SMALL:
        x = _row(c)
        V, k = x.size, c["k"]
        full = k <= 0 or k >= V
        idx = c["indices"]
        assert idx == sorted(idx), c["label"]
        if not full:
            assert len(idx) == k
            kth = np.sort(x)[::-1][k - 1]
            assert all(x[i] >= kth for i in idx), c["label"]
            assert sum(x > kth) <= k, c["label"]
        else:
            assert idx == list(range(V)), c["label"]
        first_max = int(np.argmax(x))
        if k == 1 or c["t"] <= 0:
            assert c["token"] == first_max, c["label"]
        if c["u"] == 0.0 and c["t"] > 0 and c["p"] > 0:
            assert c["token"] == idx[0], c["label"]
    # the u sweep on one row is monotone in u
    sweep = [c for c in SMALL if c["label"].startswith("u")]
    sweep.sort(key=lambda c: c["u"])
    toks = [c["token"] for c in sweep]
    assert toks == sorted(toks)


def test_oracle_reproduces_large_fixtures(orc):
    from gemma4_sampler import workload as wl
    V = wl.V_GEMMA4
    d = LARGE["decode"]
    n = 40
    rows = wl.host_peaky_rows(d["seed"], 0, n, V, greedy_every=wl.GREEDY_EVERY)
    t, k, p = wl.peaky_params(range(n))
    u = wl.host_row_u(d["seed"], 0, n)
    ids = orc.sample_batch(rows, 0, V, V, (t, k, p), u, softcap=30.0, threads=8)
    assert list(ids) == d["ids"][:n]
    _, _, idx, probs = orc.do_sample(rows[0], t[0], k[0], p[0], u[0], softcap=30.0)
    assert _digest(idx, probs) == d["row0_sha256"]


def _pad_rows(rows):
    """Rows padded to a 16-byte stride with -1e30 (never a candidate)."""
    B, V = rows.shape
    stride = (V + 3) // 4 * 4
    out = np.full((B, stride), -1e30, F32)
    out[:, :V] = rows
    return out, stride


@pytest.mark.gpu
def test_gpu_small_fixtures():
    from gemma4_sampler import hip, native
    groups = defaultdict(list)
    for c in SMALL:
        groups[(len(c["logits"]), c["softcap"])].append(c)
    for (V, cap), cases in groups.items():
        rows, stride = _pad_rows(np.stack([_row(c) for c in cases]))
        B = len(cases)
        s = native.Sampler(V, max_batch=B, softcap=cap)
        d = hip.Buffer.from_array(rows)
        outs = native.DeviceOutputs(B, V)
        params = [native.TSamplingParams.make(c["t"], c["k"], c["p"]) for c in cases]
        _, ids = s.sample(d, B, params, [c["u"] for c in cases], row_stride=stride,
                          outputs=outs.struct)
        o = outs.read()
        for r, c in enumerate(cases):
            ctx = f"{c['label']} (V={V}, cap={cap})"
            n = c["count"]
            assert ids[r] == c["token"], ctx
            assert int(o["lsum"][r:r + 1].view(np.uint32)[0]) == c["lsum"], ctx
            assert o["count"][r] == n, ctx
            assert list(o["indices"][r][:n]) == c["indices"], ctx
            assert [int(b) for b in o["probs"][r][:n].view(np.uint32)] == c["probs"], ctx
            assert o["argmax"][r] == c["indices"][c["argmax_pos"]], ctx
        s.close()


@pytest.mark.gpu
def test_gpu_large_fixtures():
    from gemma4_sampler import hip, native, workload as wl
    V = wl.V_GEMMA4
    d = LARGE["decode"]
    n = d["rows"]
    s = native.Sampler(V, max_batch=64, softcap=30.0)
    buf = hip.Buffer(V * 4)
    t, k, p = wl.peaky_params(range(n))
    u = wl.host_row_u(d["seed"], 0, n)
    outs = native.DeviceOutputs(1, 64)
    for r in range(n):
        wl.dev_peaky_rows(buf, d["seed"], r, 1, V, greedy_every=wl.GREEDY_EVERY)
        hip.synchronize()
        _, ids = s.sample(buf, 1, [native.TSamplingParams.make(t[r], k[r], p[r])], [u[r]],
                          outputs=outs.struct if r == 0 else None)
        assert ids[0] == d["ids"][r], f"decode row {r}"
        if r == 0:
            o = outs.read()
            m = o["count"][0]
            assert m == d["row0_count"]
            assert _digest(o["indices"][0][:m], o["probs"][0][:m]) == d["row0_sha256"]
    buf.free()

    m = LARGE["mixed"]
    B = m["rows"]
    buf = hip.Buffer(B * V * 4)
    wl.dev_peaky_rows(buf, m["seed"], 0, B, V)
    hip.synchronize()
    t, k, p = wl.host_mixed_params(m["seed"], 0, B)
    params = [native.TSamplingParams.make(a, b, c) for a, b, c in zip(t, k, p)]
    _, ids = s.sample(buf, B, params, wl.host_row_u(m["seed"], 0, B))
    assert list(ids) == m["ids"]
    buf.free()
    s.close()

    f = LARGE["flat_bf16"]
    B = f["rows"]
    s = native.Sampler(V, max_batch=B, softcap=30.0)
    buf = hip.Buffer(B * V * 2)
    wl.dev_flat_bf16_rows(buf, f["seed"], 0, B, V)
    hip.synchronize()
    t, k, p = wl.flat_params(B)
    params = [native.TSamplingParams.make(a, b, c) for a, b, c in zip(t, k, p)]
    outs = native.DeviceOutputs(B, V)
    _, ids = s.sample(buf, B, params, wl.host_row_u(f["seed"], 0, B), dtype=native.DTYPE_BF16,
                      outputs=outs.struct)
    assert list(ids) == f["ids"]
    o = outs.read()
    assert int(o["lsum"][0:1].view(np.uint32)[0]) == f["row0_lsum"]
    assert _digest(o["indices"][0][:V], o["probs"][0][:V]) == f["row0_sha256"]
    buf.free()
    s.close()
