"""GPU parity of g4s_sample_graph, the handle-owned hipGraph launch of the
stream-ordered sample, against the CPU oracle through the C ABI.

A decode loop keeps its buffers and rewrites them every step, so the graph
captured on the first call is replayed with new logits, parameters and
uniforms: every replay's ids (and device outputs) must equal the oracle's.
Eager work runs on the same stream between replays (graph nodes have given
wrong results on replays after the first when a capture recorded memory
fills, so each replay is checked on its own).  A second argument set (a
mixed batch with full-vocabulary rows, bf16) gets its own graph; both stay
cached and are replayed alternately.
"""
import numpy as np
import pytest

from gemma4_sampler import hip, native, workload as wl
from test_gpu_topk import check_rows

pytestmark = pytest.mark.gpu
F32 = np.float32
V = wl.V_GEMMA4
CAP = wl.SOFTCAP_GEMMA4
SEED = 20261205


def _pbuf(params):
    return hip.Buffer.from_array(np.frombuffer(bytes(native.params_array(params)), np.uint8))


@pytest.fixture(scope="module")
def rig():
    st = hip.Stream(nonblocking=True)
    s = native.Sampler(V, max_batch=8, softcap=CAP, stream=st)
    yield st, s
    s.close()
    st.destroy()


def test_graph_decode_stream_replays(orc, rig):
    st, s = rig
    n = 24
    rows = wl.host_peaky_rows(SEED, 0, n, V, greedy_every=6)
    u = wl.host_row_u(SEED, 0, n)
    d_row = hip.Buffer(V * 4)
    d_par = hip.Buffer(16)
    d_u = hip.Buffer(8)
    d_id = hip.Buffer(4)
    d_other = hip.Buffer.from_array(rows[0])
    d_oid = hip.Buffer(4)
    outs = native.DeviceOutputs(1, 64)
    for r in range(n):
        k = 1 if r % 6 == 5 else 64
        p = native.TSamplingParams.make(0.7, k, 0.95)
        st.synchronize()
        d_row.upload(rows[r])
        d_par.upload(np.frombuffer(bytes(native.params_array([p])), np.uint8))
        d_u.upload(np.array([u[r]], np.float64))
        s.sample_graph(d_row, 1, d_par, d_u, 64, 0, d_id, outputs=outs.struct)
        # eager work on the same stream between replays
        s.sample_async(d_other, 1, d_par, d_u, 64, 0, d_oid)
        st.synchronize()
        got = int(d_id.download(np.int32)[0])
        check_rows(orc, rows[r:r + 1], [0.7], [k], [0.95], [u[r]], [got], outs.read(),
                   label=f"graph replay {r}")


def test_graph_two_argument_sets(orc, rig):
    """A B=1 fp32 graph and a B=6 bf16 graph with full-vocabulary rows (the
    softmax launches) replayed alternately, three rounds each."""
    st, s = rig
    B = 6
    d1 = hip.Buffer(V * 4)
    p1 = hip.Buffer(16)
    u1 = hip.Buffer(8)
    i1 = hip.Buffer(4)
    d6 = hip.Buffer(B * V * 2)
    p6 = hip.Buffer(16 * B)
    u6 = hip.Buffer(8 * B)
    i6 = hip.Buffer(4 * B)
    k6 = np.array([0, 20, 64, 0, 1, 5], np.int32)
    t6 = np.array([1.0, 0.7, 1.3, 0.9, 0.0, 1.0], F32)
    q6 = np.array([0.99, 0.9, 0.95, 0.8, 0.95, 1.0], F32)
    for rnd in range(3):
        row = wl.host_peaky_rows(SEED + 1, rnd, 1, V)
        b = wl.host_flat_bf16_rows(SEED + 2, rnd * B, B, V)
        uu1 = wl.host_row_u(SEED + 1, rnd, 1)
        uu6 = wl.host_row_u(SEED + 2, rnd * B, B)
        st.synchronize()
        d1.upload(row)
        p1.upload(np.frombuffer(bytes(native.params_array(
            [native.TSamplingParams.make(0.7, 64, 0.95)])), np.uint8))
        u1.upload(np.asarray(uu1, np.float64))
        d6.upload(b)
        p6.upload(np.frombuffer(bytes(native.params_array(
            [native.TSamplingParams.make(float(t), int(k), float(q))
             for t, k, q in zip(t6, k6, q6)])), np.uint8))
        u6.upload(np.asarray(uu6, np.float64))
        s.sample_graph(d1, 1, p1, u1, 64, 0, i1)
        s.sample_graph(d6, B, p6, u6, 64, 1, i6, dtype=native.DTYPE_BF16)
        st.synchronize()
        got1 = i1.download(np.int32)
        got6 = i6.download(np.int32)
        check_rows(orc, row, [0.7], [64], [0.95], uu1, got1, None, label=f"B=1 round {rnd}")
        rows6 = (b.astype(np.uint32) << 16).view(F32)
        check_rows(orc, rows6, t6, k6, q6, uu6, got6, None, label=f"B=6 bf16 round {rnd}")


def test_graph_needs_a_stream(orc):
    s = native.Sampler(V, max_batch=1, softcap=CAP)  # the null stream
    d = hip.Buffer(V * 4)
    p = _pbuf([native.TSamplingParams.make(0.7, 64, 0.95)])
    u = hip.Buffer.from_array(np.array([0.5]))
    i = hip.Buffer(4)
    with pytest.raises(native.SamplerError) as e:
        s.sample_graph(d, 1, p, u, 64, 0, i)
    assert e.value.code == native.G4S_ERR_UNSUPPORTED
    s.close()
