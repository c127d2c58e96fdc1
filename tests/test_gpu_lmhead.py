"""GPU parity of the Q4_0 LM head (g4s_lmhead_q4_0) against the oracle's
CpuMatVecQ4 restatement (src/Gemma4.Tensors.pas:546-598), and of the
LM head + sampler workload (B=32 hidden vectors, 262144 x 2560 weights, the
decode-stream sampling settings) through the C ABI.

Logits must equal the oracle's bit for bit: the kernel evaluates every
term in the reference's order with one binary32 fma, which is what the
reference's Extended-precision step rounds to for these magnitudes.  The
sampled ids are then the sampler's, compared against the oracle sampler on
the same logits.
"""
import numpy as np
import pytest

from gemma4_sampler import hip, native, workload as wl

pytestmark = pytest.mark.gpu
F32 = np.float32
D = wl.HIDDEN_GEMMA4
V = wl.V_GEMMA4


def _lmhead(s, w_host_or_buf, rows, cols, hidden):
    B = hidden.shape[0]
    dw = w_host_or_buf if isinstance(w_host_or_buf, hip.Buffer) else \
        hip.Buffer.from_array(w_host_or_buf)
    dh = hip.Buffer.from_array(np.ascontiguousarray(hidden, F32))
    dl = hip.Buffer(4 * B * rows)
    s.lmhead_q4_0(dw, rows, cols, dh, B, dl, rows)
    hip.synchronize()
    return dl.download(F32).reshape(B, rows)


@pytest.mark.parametrize("batch", [1, 5, 32, 40])
def test_lmhead_small_bit_exact(orc, batch):
    rows, cols = 700, D
    w = wl.host_q4_weights(77, rows, cols)
    hidden = wl.host_hidden(78 + batch, batch, cols)
    s = native.Sampler(V, max_batch=1, softcap=30.0)
    got = _lmhead(s, w, rows, cols, hidden)
    want = orc.matvec_q4_batch(w, hidden, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{np.sum(got != want)} logits differ"
    s.close()


def test_lmhead_odd_block_count_and_unaligned_hidden(orc):
    """An odd number of Q4_0 blocks per row (the kernel stages hidden values
    two blocks at a time, so the last group is half empty) and a hidden
    matrix that starts 4 bytes past a 16-byte boundary (staged with scalar
    loads instead of 16-byte ones)."""
    rows, cols, B = 300, 5 * 32, 3
    w = wl.host_q4_weights(81, rows, cols)
    hidden = wl.host_hidden(82, B, cols)
    s = native.Sampler(V, max_batch=1, softcap=30.0)
    dw = hip.Buffer.from_array(w)
    dh = hip.Buffer(4 * (B * cols + 1))
    dh.upload(np.ascontiguousarray(hidden, F32), offset=4)
    dl = hip.Buffer(4 * B * rows)
    s.lmhead_q4_0(dw, rows, cols, dh.offset(4), B, dl, rows)
    hip.synchronize()
    got = dl.download(F32).reshape(B, rows)
    want = orc.matvec_q4_batch(w, hidden, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{np.sum(got != want)} logits differ"
    s.close()


def test_lmhead_scale_edge_cases(orc):
    """fp16 scales that are zero, subnormal (the reference's own decoding of
    them, Types.pas:452-466), the largest finite, and negative; tiny and
    large hidden values."""
    rows, cols = 64, 256
    rng = np.random.default_rng(5)
    w = wl.host_q4_weights(79, rows, cols).reshape(rows * cols // 32, 18)
    specials = [0x0000, 0x8000, 0x0001, 0x0200, 0x03FF, 0x8155, 0x0400, 0x7BFF, 0xFBFF, 0x3C00]
    for i in range(w.shape[0]):
        if i % 3 == 0:
            v = specials[(i // 3) % len(specials)]
            w[i, 0], w[i, 1] = v & 0xFF, v >> 8
    w = w.reshape(-1)
    hidden = rng.normal(0, 1, (3, cols)).astype(F32)
    hidden[1] *= 1e-20
    hidden[2] *= 1e3
    s = native.Sampler(V, max_batch=1, softcap=30.0)
    got = _lmhead(s, w, rows, cols, hidden)
    want = orc.matvec_q4_batch(w, hidden, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    s.close()


def test_lmhead_hand_built_blocks():
    """Hand-built Q4_0 blocks with written-out expected logits: byte j holds
    element 2j in its low nibble and 2j+1 in its high nibble (Tensors.pas:
    581-593), and the row sum runs left to right in binary32."""
    cols = 32
    w = np.frombuffer(bytes([0x00, 0x3C, 0x9A, 0x0F, 0xF0] + [0x88] * 13) +
                      bytes([0x00, 0x3C, 0x99, 0x79] + [0x88] * 14), np.uint8)
    h = np.zeros((2, cols), F32)
    h[0, :6] = [1, 10, 100, 1000, 0.5, 0.25]     # row 0 weights 2, 1, 7, -8, -8, 7
    h[1, :4] = [2.0 ** 24, 1.0, 1.0, 2.0 ** 24]   # row 1 weights 1, 1, 1, -1
    s = native.Sampler(V, max_batch=1, softcap=30.0)
    got = _lmhead(s, w, 2, cols, h)
    # 2 + 10 + 700 - 8000 - 4 + 1.75; ((2^24 + 1) + 1) - 2^24 = 0 left to right
    assert got[0, 0] == F32(-7290.25) and got[1, 1] == F32(0.0), got
    s.close()


def test_lmhead_plus_sampler_full_size(orc):
    """The full LM head + sampler workload: 32 hidden vectors ~ N(0,1),
    262144 x 2560 Q4_0 weights (generated on the device and, bit-identically,
    on the host), T=0.7, K=64, P=0.95.  Every one of the 32 x 262144 logits
    is checked against the oracle's CpuMatVecQ4, and every sampled id against
    the oracle's DoSample applied to the oracle's own logits (end to end)."""
    B, rows, cols = 32, V, D
    nblocks = rows * (cols // 32)
    dw = hip.Buffer(nblocks * 18)
    wl.dev_q4_weights(dw, 80, rows, cols)
    hidden = wl.host_hidden(81, B, cols)
    s = native.Sampler(V, max_batch=B, softcap=30.0)
    logits = _lmhead(s, dw, rows, cols, hidden)
    w_host = wl.host_q4_weights(80, rows, cols, threads=16)
    want = orc.matvec_q4_batch(w_host, hidden, rows, cols, threads=16)
    del w_host
    nbad = int(np.sum(logits.view(np.uint32) != want.view(np.uint32)))
    assert nbad == 0, f"{nbad} of {B * rows} logits differ from CpuMatVecQ4"
    # sampling on the device-resident logits
    dl = hip.Buffer.from_array(logits)
    t = np.full(B, 0.7, F32)
    k = np.full(B, 64, np.int32)
    p = np.full(B, 0.95, F32)
    u = wl.host_row_u(82, 0, B)
    _, ids = s.sample(dl, B, [native.TSamplingParams.make(0.7, 64, 0.95)] * B, u)
    want_ids = orc.sample_batch(want, 0, V, V, (t, k, p), u, softcap=30.0, threads=16)
    assert np.array_equal(ids, want_ids), (ids, want_ids)
    print(f"LM head + sampler: {B * rows} logits and {B} ids bit-exact end to end")
    s.close()
