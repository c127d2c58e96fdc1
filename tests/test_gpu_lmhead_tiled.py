"""GPU parity of the Q4_0 weight upload from a VPK archive, the TILED64
layout, the LM head on it (g4s_lmhead_q4_0_tiled) and the LM head fused with
the sampler (g4s_lmhead_sample_q4_0), through the C ABI.

- Upload (TWeightStore.LoadTensor + the engine's staged upload,
  src/Gemma4.Tensors.pas:477-506, src/Gemma4.Model.pas:494-640): the ROWS
  layout must hold the archive's bytes unchanged; TILED64 must equal a
  numpy restatement of the layout, with every fp16 scale widened by the
  oracle's TFloat16.ToSingle (src/Gemma4.Types.pas:438-481).
- LM head: logits bit-exact against the oracle's CpuMatVecQ4
  (src/Gemma4.Tensors.pas:546-598).
- Fused LM head + sample: ids, LSum, greedy id, survivor indices and
  probabilities equal to the oracle's DoSample on the oracle's logits, and
  to g4s_sample_ex on the same logits, including rows whose ties force the
  exact candidate path and heap replay.
"""
import numpy as np
import pytest

from gemma4_sampler import hip, native, workload as wl

import vpkfix

pytestmark = pytest.mark.gpu
F32 = np.float32
D = wl.HIDDEN_GEMMA4
V = wl.V_GEMMA4
EMBED = "model.language_model.embed_tokens.weight"

_F16 = None


def _f16_table(orc):
    global _F16
    if _F16 is None:
        _F16 = np.array([orc.f16_to_f32(v) for v in range(65536)], F32)
    return _F16


def _tiled_ref(orc, w_rows, rows, cols):
    """numpy restatement of TILED64 from ROWS bytes."""
    nblk = cols // 32
    groups = (rows + 63) // 64
    blocks = np.frombuffer(w_rows, np.uint8).reshape(rows, nblk, 18)
    scale = _f16_table(orc)[blocks[:, :, 0].astype(np.uint32) | (blocks[:, :, 1].astype(np.uint32) << 8)]
    sc = np.zeros((groups * 64, nblk), F32)
    sc[:rows] = scale
    q = np.full((groups * 64, nblk, 16), 0x88, np.uint8)
    q[:rows] = blocks[:, :, 2:]
    out = np.empty((groups, nblk, 1280), np.uint8)
    out[:, :, :256] = sc.reshape(groups, 64, nblk).transpose(0, 2, 1).copy().view(np.uint8).reshape(
        groups, nblk, 256)
    out[:, :, 256:] = q.reshape(groups, 64, nblk, 16).transpose(0, 2, 1, 3).reshape(groups, nblk, 1024)
    return out.reshape(-1)


def _params(t, k, p):
    return [native.TSamplingParams.make(float(a), int(b), float(c)) for a, b, c in zip(t, k, p)]


def _archive(tmp_path, rows, cols, seed):
    w = wl.host_q4_weights(seed, rows, cols)
    data, _ = vpkfix.weights_archive([
        ("model.language_model.norm.weight", "F32", [cols], np.ones(cols, F32).tobytes()),
        (EMBED, "Q4_0", [rows, cols], w.tobytes()),
    ])
    path = tmp_path / "gemma.vpk"
    path.write_bytes(data)
    return str(path), w


@pytest.mark.parametrize("rows, cols", [(700, 160), (4096 + 64 * 300 + 5, D)])
def test_upload_rows_and_tiled(orc, tmp_path, rows, cols):
    path, w = _archive(tmp_path, rows, cols, 31 + rows)
    st = native.WeightStore()
    assert st.Open(path), st.LastError()
    nrows = native.q4_0_device_bytes(rows, cols, native.Q4_LAYOUT_ROWS)
    ntile = native.q4_0_device_bytes(rows, cols, native.Q4_LAYOUT_TILED64)
    d_rows, d_tile = hip.Buffer(nrows), hip.Buffer(ntile)
    st.UploadQ4_0(EMBED, native.Q4_LAYOUT_ROWS, d_rows, nrows)
    st.UploadQ4_0(EMBED, native.Q4_LAYOUT_TILED64, d_tile, ntile)
    assert np.array_equal(d_rows.download(np.uint8), w)
    want = _tiled_ref(orc, w.tobytes(), rows, cols)
    got = d_tile.download(np.uint8)
    assert np.array_equal(got, want), f"{np.sum(got != want)} tiled bytes differ"
    # the device-side repack of the ROWS upload gives the same bytes
    d_rep = hip.Buffer(ntile)
    native.q4_0_repack(d_rows, rows, cols, d_rep)
    hip.synchronize()
    assert np.array_equal(d_rep.download(np.uint8), want)
    st.Close()


def _tiled_lmhead(s, w, rows, cols, hidden):
    ntile = native.q4_0_device_bytes(rows, cols, native.Q4_LAYOUT_TILED64)
    d_rows = hip.Buffer.from_array(w)
    d_tile = hip.Buffer(ntile)
    native.q4_0_repack(d_rows, rows, cols, d_tile)
    B = hidden.shape[0]
    dh = hip.Buffer.from_array(np.ascontiguousarray(hidden, F32))
    dl = hip.Buffer(4 * B * rows)
    s.lmhead_q4_0_tiled(d_tile, rows, cols, dh, B, dl, rows)
    hip.synchronize()
    return dl.download(F32).reshape(B, rows)


@pytest.mark.parametrize("batch", [1, 5, 32, 33, 70])
def test_tiled_lmhead_bit_exact(orc, batch):
    """Rows not a multiple of 64 and batches that leave a tile partly empty
    or need several passes over the weights."""
    rows, cols = 700, D
    w = wl.host_q4_weights(91, rows, cols)
    hidden = wl.host_hidden(92 + batch, batch, cols)
    s = native.Sampler(V, max_batch=1, softcap=30.0)
    got = _tiled_lmhead(s, w, rows, cols, hidden)
    want = orc.matvec_q4_batch(w, hidden, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{np.sum(got != want)} logits differ"
    s.close()


def test_tiled_lmhead_scale_edge_cases(orc):
    """Zero, subnormal (the engine's own widening), largest and negative fp16
    scales; tiny and large hidden values; one block per row."""
    rows, cols = 130, 32
    rng = np.random.default_rng(7)
    w = wl.host_q4_weights(93, rows, cols).reshape(rows, 18)
    specials = [0x0000, 0x8000, 0x0001, 0x0200, 0x03FF, 0x8155, 0x0400, 0x7BFF, 0xFBFF, 0x3C00]
    for i in range(rows):
        if i % 2 == 0:
            v = specials[(i // 2) % len(specials)]
            w[i, 0], w[i, 1] = v & 0xFF, v >> 8
    w = w.reshape(-1)
    hidden = rng.normal(0, 1, (3, cols)).astype(F32)
    hidden[1] *= 1e-20
    hidden[2] *= 1e3
    s = native.Sampler(V, max_batch=1, softcap=30.0)
    got = _tiled_lmhead(s, w, rows, cols, hidden)
    want = orc.matvec_q4_batch(w, hidden, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    s.close()


def _fused_check(orc, vocab, w, hidden, t, k, p, u, label, capacity=None):
    """Fused call against the oracle on its own logits and against
    g4s_sample_ex on the written logits."""
    B = hidden.shape[0]
    cols = hidden.shape[1]
    ntile = native.q4_0_device_bytes(vocab, cols, native.Q4_LAYOUT_TILED64)
    d_rows = hip.Buffer.from_array(w)
    d_tile = hip.Buffer(ntile)
    native.q4_0_repack(d_rows, vocab, cols, d_tile)
    s = native.Sampler(vocab, max_batch=B, softcap=30.0)
    dh = hip.Buffer.from_array(np.ascontiguousarray(hidden, F32))
    dl = hip.Buffer(4 * B * vocab)
    cap = capacity or 256
    outs = native.DeviceOutputs(B, cap)
    _, ids = s.lmhead_sample_q4_0(d_tile, cols, dh, B, dl, _params(t, k, p), u,
                                  outputs=outs.struct)
    o = outs.read()
    logits = dl.download(F32).reshape(B, vocab)
    want_logits = orc.matvec_q4_batch(w, hidden, vocab, cols, threads=16)
    assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32)), label
    outs2 = native.DeviceOutputs(B, cap)
    _, ids2 = s.sample(dl, B, _params(t, k, p), u, outputs=outs2.struct)
    o2 = outs2.read()
    assert np.array_equal(ids, ids2), (label, ids, ids2)
    for r in range(B):
        tok, det, idx, pr = orc.do_sample(want_logits[r], t[r], k[r], p[r], u[r], softcap=30.0,
                                          want_probs=True)
        ctx = f"{label} row {r} (T={t[r]}, K={k[r]}, P={p[r]}, u={u[r]!r})"
        assert ids[r] == tok, f"{ctx}: fused id {ids[r]} != oracle {tok}"
        assert o["lsum"][r].view(np.uint32) == np.float32(det["lsum"]).view(np.uint32), ctx
        assert o["argmax"][r] == o2["argmax"][r], ctx
        if 0 < k[r] < vocab:
            n = o["count"][r]
            assert n == len(idx) and n == o2["count"][r], ctx
            if n <= cap:
                assert np.array_equal(o["indices"][r][:n], idx), ctx
                assert np.array_equal(o["probs"][r][:n].view(np.uint32), pr.view(np.uint32)), ctx
    s.close()
    return o


@pytest.mark.parametrize("vocab", [1000, 20000])
def test_fused_lmhead_sample(orc, vocab):
    """Mixed rows: top-k (K = 1, 20, 64, 256, 1000), a full-vocabulary row and
    a wide row (K > g4s_max_top_k) in one call; T <= 0 rows; u at 0 and
    1 - 2^-32."""
    B = 12
    cols = 256
    w = wl.host_q4_weights(101 + vocab, vocab, cols)
    hidden = wl.host_hidden(102 + vocab, B, cols)
    rng = np.random.default_rng(vocab)
    k = np.array([1, 20, 64, 256, 64, 1000, 0, 64, 1, 1100, 20, 64], np.int32)
    k = np.minimum(k, vocab - 1)
    t = np.array([0.7, 1.0, 0.7, 1.3, 0.0, 0.9, 1.0, -1.0, 0.7, 1.0, 0.5, 0.7], F32)
    p = np.array([0.95, 0.9, 0.95, 1.0, 0.95, 0.8, 0.99, 0.95, 0.95, 0.9, 0.0, 0.95], F32)
    u = np.floor(rng.random(B) * 2 ** 32) / 2 ** 32
    u[0], u[1] = 0.0, 1.0 - 2 ** -32
    _fused_check(orc, vocab, w, hidden, t, k, p, u, f"fused V={vocab}", capacity=1100)


def test_fused_heavy_ties(orc):
    """Zero hidden vectors (every logit 0: the candidate groups hold far more
    keys than the slots, so the exact path and the heap replay decide) next
    to rows whose hidden vector is one-hot (a few hundred tied logits)."""
    vocab, cols, B = 9000, 64, 6
    w = wl.host_q4_weights(111, vocab, cols)
    hidden = np.zeros((B, cols), F32)
    hidden[2, 5] = 1.0
    hidden[3, 0] = 0.5
    hidden[4] = wl.host_hidden(112, 1, cols)[0]
    k = np.array([64, 1, 20, 256, 64, 1000], np.int32)
    t = np.array([0.7, 0.7, 1.0, 0.7, 0.7, 1.0], F32)
    p = np.array([0.95, 0.95, 0.9, 0.95, 0.95, 1.0], F32)
    u = wl.host_row_u(113, 0, B)
    o = _fused_check(orc, vocab, w, hidden, t, k, p, u, "ties", capacity=1000)
    assert o["flags"][0] & native.FLAG_CHUNK_EXACT, hex(o["flags"][0])


def test_fused_full_size_matches_unfused(orc):
    """The LM head + sampler workload (32 hidden vectors, 262144 x 2560
    weights, T=0.7, K=64, P=0.95, every 100th-style greedy row at K=1): the
    tiled logits equal g4s_lmhead_q4_0's (pinned to the oracle at this size
    elsewhere) and the fused ids equal g4s_sample_ex's on them."""
    B, rows, cols = 32, V, D
    nblocks = rows * (cols // 32)
    d_rows = hip.Buffer(nblocks * 18)
    wl.dev_q4_weights(d_rows, 80, rows, cols)
    hidden = wl.host_hidden(81, B, cols)
    dh = hip.Buffer.from_array(hidden)
    s = native.Sampler(V, max_batch=B, softcap=30.0)
    d_old = hip.Buffer(4 * B * rows)
    s.lmhead_q4_0(d_rows, rows, cols, dh, B, d_old, rows)
    ntile = native.q4_0_device_bytes(rows, cols, native.Q4_LAYOUT_TILED64)
    d_tile = hip.Buffer(ntile)
    native.q4_0_repack(d_rows, rows, cols, d_tile)
    del d_rows
    d_new = hip.Buffer(4 * B * rows)
    k = np.full(B, 64, np.int32)
    k[::8] = 1
    params = _params(np.full(B, 0.7, F32), k, np.full(B, 0.95, F32))
    u = wl.host_row_u(82, 0, B)
    _, ids = s.lmhead_sample_q4_0(d_tile, cols, dh, B, d_new, params, u)
    old = d_old.download(F32)
    new = d_new.download(F32)
    assert np.array_equal(old.view(np.uint32), new.view(np.uint32)), \
        f"{np.sum(old != new)} logits differ between the LM heads"
    _, ids2 = s.sample(d_new, B, params, u)
    assert np.array_equal(ids, ids2), (ids, ids2)
    want = orc.sample_batch(new.reshape(B, rows), 0, V, V,
                            (np.full(B, 0.7, F32), k, np.full(B, 0.95, F32)), u,
                            softcap=30.0, threads=16)
    assert np.array_equal(ids, want), (ids, want)
    s.close()


def test_vpk_to_sample_end_to_end(orc, tmp_path):
    """Archive -> TILED64 upload -> fused LM head + sample, against the
    oracle's CpuMatVecQ4 + DoSample on the archive's bytes."""
    vocab, cols, B = 5000, D, 4
    path, w = _archive(tmp_path, vocab, cols, 121)
    st = native.WeightStore()
    assert st.Open(path), st.LastError()
    ntile = native.q4_0_device_bytes(vocab, cols, native.Q4_LAYOUT_TILED64)
    d_tile = hip.Buffer(ntile)
    st.UploadQ4_0(EMBED, native.Q4_LAYOUT_TILED64, d_tile, ntile)
    hidden = wl.host_hidden(122, B, cols)
    s = native.Sampler(vocab, max_batch=B, softcap=30.0)
    dh = hip.Buffer.from_array(hidden)
    dl = hip.Buffer(4 * B * vocab)
    t, k, p = np.full(B, 0.7, F32), np.array([64, 1, 64, 20], np.int32), np.full(B, 0.95, F32)
    u = wl.host_row_u(123, 0, B)
    _, ids = s.lmhead_sample_q4_0(d_tile, cols, dh, B, dl, _params(t, k, p), u)
    logits = orc.matvec_q4_batch(np.frombuffer(st.GetRawBytes(EMBED), np.uint8), hidden, vocab,
                                 cols, threads=16)
    for r in range(B):
        tok, _, _, _ = orc.do_sample(logits[r], t[r], k[r], p[r], u[r], softcap=30.0,
                                     want_probs=False)
        assert ids[r] == tok, (r, ids[r], tok)
    st.Close()
    s.close()


def _no_logits_check(orc, s, d_tile, w, hidden, t, k, p, u, label, capacity=256):
    """The fused call without logits against the oracle's CpuMatVecQ4 +
    DoSample: ids, LSum, greedy id, survivor indices and probabilities."""
    B, cols = hidden.shape
    vocab = s.vocab
    dh = hip.Buffer.from_array(np.ascontiguousarray(hidden, F32))
    outs = native.DeviceOutputs(B, capacity)
    rc, ids = s.lmhead_sample_q4_0(d_tile, cols, dh, B, None, _params(t, k, p), u,
                                   outputs=outs.struct)
    assert rc == 0, s.last_error()
    o = outs.read()
    logits = orc.matvec_q4_batch(w, hidden, vocab, cols, threads=16)
    for r in range(B):
        tok, det, idx, pr = orc.do_sample(logits[r], t[r], k[r], p[r], u[r], softcap=30.0,
                                          want_probs=True)
        ctx = f"{label} row {r} (T={t[r]}, K={k[r]}, P={p[r]}, u={u[r]!r})"
        assert ids[r] == tok, f"{ctx}: id {ids[r]} != oracle {tok}"
        assert o["lsum"][r].view(np.uint32) == np.float32(det["lsum"]).view(np.uint32), ctx
        assert o["argmax"][r] == idx[det["argmax_pos"]], ctx  # a survivor position there
        n = o["count"][r]
        assert n == len(idx), ctx
        assert np.array_equal(o["indices"][r][:n], idx), ctx
        assert np.array_equal(o["probs"][r][:n].view(np.uint32), pr.view(np.uint32)), ctx
    return o


def test_fused_no_logits_full_size(orc):
    """The LM head + sampler workload (32 hidden vectors, 262144 x 2560
    weights, T=0.7, K=64 with every 8th row K=1, P=0.95) without logits:
    candidate groups give their maxima or are recomputed (about one group in
    two rows holds two keys of the top K), bit-exact with the oracle."""
    B, rows, cols = 32, V, D
    w = wl.host_q4_weights(80, rows, cols, threads=16)
    ntile = native.q4_0_device_bytes(rows, cols, native.Q4_LAYOUT_TILED64)
    d_rows = hip.Buffer.from_array(w)
    d_tile = hip.Buffer(ntile)
    native.q4_0_repack(d_rows, rows, cols, d_tile)
    hip.synchronize()
    d_rows.free()
    hidden = wl.host_hidden(81, B, cols)
    s = native.Sampler(V, max_batch=B, softcap=30.0)
    k = np.full(B, 64, np.int32)
    k[::8] = 1
    t = np.full(B, 0.7, F32)
    p = np.full(B, 0.95, F32)
    u = wl.host_row_u(82, 0, B)
    o = _no_logits_check(orc, s, d_tile, w, hidden, t, k, p, u, "full size", capacity=64)
    assert not np.any(o["flags"] & native.FLAG_ROW_RECOMPUTED), o["flags"]
    s.close()


def test_fused_no_logits_ties(orc):
    """Without logits: zero hidden vectors (every logit 0; the row is
    recomputed whole and sampled again), one-hot vectors (hundreds of tied
    logits), groups whose first two rows have the same weights (every group
    maximum tied inside its group: recompute jobs that decide ties by index),
    and plain rows; K from 1 to 1000."""
    vocab, cols, B = 9000, 64, 8
    w = wl.host_q4_weights(131, vocab, cols).reshape(vocab, cols // 32 * 18)
    w[1::64] = w[0::64][: w[1::64].shape[0]]
    w = w.reshape(-1)
    ntile = native.q4_0_device_bytes(vocab, cols, native.Q4_LAYOUT_TILED64)
    d_rows = hip.Buffer.from_array(w)
    d_tile = hip.Buffer(ntile)
    native.q4_0_repack(d_rows, vocab, cols, d_tile)
    hip.synchronize()
    hidden = wl.host_hidden(132, B, cols)
    hidden[0] = 0.0
    hidden[1] = 0.0
    hidden[2] = 0.0
    hidden[2, 5] = 1.0
    hidden[3] = 0.0
    hidden[3, 0] = 0.5
    k = np.array([64, 1, 20, 256, 64, 1000, 5, 64], np.int32)
    t = np.array([0.7, 0.7, 1.0, 0.7, 0.7, 1.0, 0.0, 1.3], F32)
    p = np.array([0.95, 0.95, 0.9, 0.95, 0.95, 1.0, 0.95, 0.99], F32)
    u = wl.host_row_u(133, 0, B)
    s = native.Sampler(vocab, max_batch=B, softcap=30.0)
    o = _no_logits_check(orc, s, d_tile, w, hidden, t, k, p, u, "ties", capacity=1000)
    assert o["flags"][0] & native.FLAG_ROW_RECOMPUTED, hex(o["flags"][0])
    # the same call with the logits written gives the same outputs
    dh = hip.Buffer.from_array(hidden)
    dl = hip.Buffer(4 * B * vocab)
    outs = native.DeviceOutputs(B, 1000)
    _, ids2 = s.lmhead_sample_q4_0(d_tile, cols, dh, B, dl, _params(t, k, p), u,
                                   outputs=outs.struct)
    o2 = outs.read()
    for key in ("count", "argmax"):
        assert np.array_equal(o[key], o2[key]), key
    assert np.array_equal(o["lsum"].view(np.uint32), o2["lsum"].view(np.uint32))
    s.close()


def test_fused_no_logits_rejects_full_rows(orc):
    vocab, cols = 1000, 64
    w = wl.host_q4_weights(141, vocab, cols)
    ntile = native.q4_0_device_bytes(vocab, cols, native.Q4_LAYOUT_TILED64)
    d_rows = hip.Buffer.from_array(w)
    d_tile = hip.Buffer(ntile)
    native.q4_0_repack(d_rows, vocab, cols, d_tile)
    hip.synchronize()
    s = native.Sampler(vocab, max_batch=2, softcap=30.0)
    dh = hip.Buffer.from_array(wl.host_hidden(142, 2, cols))
    for kk in (0, vocab, 2000):
        params = _params([0.7, 0.7], [64, kk], [0.95, 0.95])
        rc, _ = s.lmhead_sample_q4_0(d_tile, cols, dh, 2, None, params, [0.5, 0.5], check=False)
        assert rc == native.G4S_ERR_INVALID_ARGUMENT, (kk, rc, s.last_error())
    s.close()
