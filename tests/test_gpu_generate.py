"""GPU parity of the batched decode loop (g4s_generate, TModel.Generate for
several sequences, src/Gemma4.Model.pas:2829-2938) and of the embedding
lookup (g4s_embed_q4_0, DoEmbeddingLookup, :2047-2080), through the C ABI.

The caller's forward pass is a one-token model built from the tied Q4_0
table alone: the embedding of the fed token, scaled by fl32(sqrt(hidden)),
times the same table (the LM head).  The oracle runs the same model on the
CPU (oracle.embed_q4 + CpuMatVecQ4) under its restatement of Generate, with
the same per-sequence random streams; every sequence's tokens and the order
of its random draws must match.
"""
import ctypes

import numpy as np
import pytest

from gemma4_sampler import hip, native, workload as wl

pytestmark = pytest.mark.gpu
F32 = np.float32
V, COLS = 4096, 256
SCALE = F32(np.sqrt(2560.0))


def _table():
    w = wl.host_q4_weights(131, V, COLS).reshape(V, COLS // 32, 18).copy()
    # row 50 (an EOS id) := 2 x row 7: the model's greedy successor of 7 is EOS
    w[50] = w[7]
    for k in range(COLS // 32):
        h = int(w[7, k, 0]) | (int(w[7, k, 1]) << 8)
        h2 = h + (1 << 10) if (h & 0x7C00) not in (0, 0x7C00) and (h & 0x7C00) < 0x7800 else h
        w[50, k, 0], w[50, k, 1] = h2 & 0xFF, h2 >> 8
    return w.reshape(-1)


def test_embedding_lookup_bit_exact(orc):
    w = _table()
    s = native.Sampler(V, max_batch=4, softcap=30.0)
    toks = np.array([0, 7, V - 1, 50, -1, V], np.int32)
    dw, dt = hip.Buffer.from_array(w), hip.Buffer.from_array(toks)
    dh = hip.Buffer(4 * len(toks) * COLS)
    s.embed_q4_0(dw, V, COLS, dt, len(toks), SCALE, dh)
    hip.synchronize()
    got = dh.download(F32).reshape(len(toks), COLS)
    for i, t in enumerate(toks):
        want = orc.embed_q4(w, int(t), COLS, SCALE) if 0 <= t < V else np.zeros(COLS, F32)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), (i, t)
    s.close()


@pytest.mark.parametrize("max_tokens", [0, 1, 8])
def test_generate_matches_oracle(orc, max_tokens):
    w = _table()
    B = 6
    params = [(0.0, 64, 0.95), (0.7, 64, 0.95), (1.0, 0, 0.99), (1.3, 20, 0.9),
              (0.7, 1, 0.95), (0.9, V, 0.8)]
    prompts = np.array([7, 11, 12, 13, 14, 15], np.int32)
    stop_after = {3: 3}

    s = native.Sampler(V, max_batch=B, softcap=30.0)
    dw = hip.Buffer.from_array(w)
    ntile = native.q4_0_device_bytes(V, COLS, native.Q4_LAYOUT_TILED64)
    dtile = hip.Buffer(ntile)
    native.q4_0_repack(dw, V, COLS, dtile)
    dtok = hip.Buffer(4 * B)
    dh = hip.Buffer(4 * B * COLS)
    dl = hip.Buffer(4 * B * V)
    fed = []

    def gpu_forward(tokens):
        fed.append(list(tokens))
        dtok.upload(np.ascontiguousarray(tokens, np.int32))
        s.embed_q4_0(dw, V, COLS, dtok, B, SCALE, dh)
        s.lmhead_q4_0_tiled(dtile, V, COLS, dh, B, dl, V)
        return True

    def cpu_forward(tokens):
        rows = np.zeros((B, V), F32)
        hid = np.stack([orc.embed_q4(w, t, COLS, SCALE) if t >= 0 else np.zeros(COLS, F32)
                        for t in tokens])
        live = [b for b in range(B) if tokens[b] >= 0]
        if live:
            rows[live] = orc.matvec_q4_batch(w, hid[live], V, COLS)
        return rows

    def streams():
        gens = [orc.lcg_uniforms(1000 + b) for b in range(B)]
        log = []

        def rnd(b):
            log.append(b)
            return next(gens[b])
        return rnd, log

    def stopper():
        seen = {}

        def on_token(b, t):
            seen[b] = seen.get(b, 0) + 1
            return not (b in stop_after and seen[b] >= stop_after[b])
        return on_token

    # prompt logits, then the loop
    gpu_forward(prompts)
    first = dl.download(F32).reshape(B, V)
    assert np.array_equal(first.view(np.uint32), cpu_forward(list(prompts)).view(np.uint32))
    g_rnd, g_log = streams()
    got = s.Generate(dl, B, [native.TSamplingParams.make(*p) for p in params], max_tokens,
                     gpu_forward, g_rnd, stopper())
    c_rnd, c_log = streams()
    want = orc.generate(first, params, max_tokens, cpu_forward, c_rnd, stopper(), softcap=30.0)
    for b in range(B):
        assert list(got[b]) == want[b], f"sequence {b} {params[b]}: gpu {list(got[b])} != {want[b]}"
    assert g_log == c_log, "random draws differ in order or number"
    if max_tokens >= 1:
        assert list(got[0]) == [50]  # 7 -> 50, an EOS id
    if max_tokens == 8:
        assert len(got[3]) == 3      # the callback's stop
        # once a sequence is done the forward sees -1 in its place
        done_at = [len(x) for x in want]
        for step, toks in enumerate(fed[1:], start=1):
            for b in range(B):
                if toks[b] >= 0:
                    assert step <= done_at[b]
    s.close()


def test_generate_forward_failure_is_reported():
    s = native.Sampler(V, max_batch=2, softcap=30.0)
    dl = hip.Buffer.from_array(np.zeros((2, V), F32))
    with pytest.raises(native.SamplerError) as ei:
        s.Generate(dl, 2, native.TSamplingParams.make(0.0, 64, 0.95), 4,
                   lambda toks: False, lambda b: 0.5)
    assert ei.value.code == native.G4S_ERR_ABORTED
    s.close()
