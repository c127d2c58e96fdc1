"""The oracle's decode loop (oracle.generate, TModel.Generate restated,
src/Gemma4.Model.pas:2887-2928) on hand-built logits whose outcomes are
written out, and the embedding lookup against a hand-dequantised row.  CPU
only."""
import numpy as np

F32 = np.float32
V = 300


def _onehot(token, v=V):
    row = np.full(v, -5.0, F32)
    row[token] = 5.0
    return row


def _chain_forward(nxt, calls):
    """forward(tokens): greedy successor table `nxt` (token -> next token)."""
    def forward(tokens):
        calls.append(list(tokens))
        return np.stack([_onehot(nxt.get(t, 7)) if t >= 0 else np.zeros(V, F32) for t in tokens])
    return forward


def test_eos_maximum_callback_and_extra_step(orc):
    greedy = (0.0, 64, 0.95)
    first = np.stack([_onehot(3), _onehot(50), _onehot(9), _onehot(9)])
    nxt = {3: 4, 4: 106, 9: 9, 7: 7}
    calls = []
    stop_after = {3: 2}  # sequence 3 stops itself after its second token
    seen = {}

    def on_token(b, t):
        seen[b] = seen.get(b, 0) + 1
        return not (b in stop_after and seen[b] >= stop_after[b])

    out = orc.generate(first, [greedy] * 4, 5, _chain_forward(nxt, calls), lambda b: 0.5,
                       on_token=on_token)
    # 3 -> 4 -> 106 (EOS kept); 50 is EOS at once; 9 repeats up to the
    # maximum; sequence 3 (9 -> 9 ...) stops after its second token by callback
    assert out == [[3, 4, 106], [50], [9, 9, 9, 9, 9], [9, 9]]
    assert sum(1 for c in calls if c[3] >= 0) == 1  # no step after the callback's stop
    # sequence 2 appends its 5th token and still takes the step the
    # reference takes (Forward + DoSample, :2919-2923) before the loop ends
    steps_of_2 = sum(1 for c in calls if c[2] >= 0)
    assert steps_of_2 == 5
    # forward sees -1 for sequences that are done
    assert calls[-1] == [-1, -1, 9, -1]


def test_zero_and_one_token_budgets_consume_randomness_like_generate(orc):
    drawn = []

    def rnd(b):
        drawn.append(b)
        return 0.25

    sampled = (0.7, 64, 0.95)
    first = np.stack([_onehot(12), _onehot(13)])
    calls = []
    assert orc.generate(first, [sampled] * 2, 0, _chain_forward({}, calls), rnd) == [[], []]
    assert drawn == [0, 1] and calls == []  # the first DoSample still draws (:2889)
    drawn.clear()
    out = orc.generate(first, [sampled] * 2, 1, _chain_forward({}, calls), rnd)
    assert out == [[12], [13]]
    # one token each, then the reference's last Forward + DoSample: a second draw each
    assert drawn == [0, 1, 0, 1] and len(calls) == 1


def test_embedding_lookup_by_hand(orc):
    """Row 1 of a 2-row table: scale 1.0 (fp16 0x3C00), nibbles 0..15 in
    order, times fl32(sqrt(2560))."""
    cols = 32
    row0 = bytes([0x00, 0x3C] + [0x88] * 16)
    nib = bytes((2 * j) | ((2 * j + 1) << 4) for j in range(8)) + \
        bytes((2 * j - 16) | ((2 * j + 1 - 16) << 4) for j in range(8, 16))
    row1 = bytes([0x00, 0x3C]) + nib
    w = np.frombuffer(row0 + row1, np.uint8)
    sc = F32(np.sqrt(2560.0))
    got = orc.embed_q4(w, 1, cols, sc)
    want = (np.array([(j % 16) - 8 for j in range(32)], F32) * sc).astype(F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
