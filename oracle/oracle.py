"""ctypes wrapper of the CPU oracle (oracle/g4s_oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product path.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "build", "liboracle.so")
LIB_D = os.path.join(HERE, "build", "liboracle_d.so")


class Params(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int32),
                ("top_p", ctypes.c_float), ("repetition_penalty", ctypes.c_float)]


class Detail(ctypes.Structure):
    _fields_ = [("path", ctypes.c_int32), ("count", ctypes.c_int32),
                ("argmax_pos", ctypes.c_int32), ("chosen_pos", ctypes.c_int32),
                ("drew", ctypes.c_int32), ("reached", ctypes.c_int32),
                ("lsum", ctypes.c_float), ("threshold", ctypes.c_float),
                ("cum_prev", ctypes.c_float), ("cum_at", ctypes.c_float),
                ("max_val", ctypes.c_float), ("token", ctypes.c_int32)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


def build():
    subprocess.run(["make", "-s", "-C", HERE, "all", "double"], check=True)


_libs = {}


def load(double=False):
    path = LIB_D if double else LIB
    if path not in _libs:
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
        L.orc_semantics.restype = ctypes.c_char_p
        L.orc_bf16_to_f32.restype = f32
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = f32
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_from_f32.restype = ctypes.c_uint16
        L.orc_f16_from_f32.argtypes = [f32]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [f32]
        L.orc_logit_softcap.argtypes = [vp, i32, f32]
        L.orc_softcap_topk.restype = f32
        L.orc_softcap_topk.argtypes = [f32, f32]
        L.orc_exp_diff.restype = f32
        L.orc_exp_diff.argtypes = [f32, f32]
        L.orc_softmax_f32.restype = f32
        L.orc_softmax_f32.argtypes = [vp, i32]
        L.orc_select_topk_indices.restype = i32
        L.orc_select_topk_indices.argtypes = [vp, i32, i32, vp]
        L.orc_sample_topp.restype = i32
        L.orc_sample_topp.argtypes = [vp, i32, f32, f32, ctypes.c_double, vp]
        L.orc_do_sample.restype = i32
        L.orc_do_sample.argtypes = [vp, i32, f32, vp, ctypes.c_double, vp, vp, i32, vp]
        L.orc_sample_batch.restype = i32
        L.orc_sample_batch.argtypes = [vp, i32, i32, i64, i32, vp, vp, f32, vp, i32]
        L.orc_dequant_q4_block.argtypes = [vp, vp]
        L.orc_f32_to_q4_buffer.restype = ctypes.c_uint64
        L.orc_f32_to_q4_buffer.argtypes = [vp, vp, ctypes.c_uint64]
        L.orc_matvec_q4.argtypes = [vp, vp, vp, i32, i32, i32, i32]
        L.orc_matvec_q4_batch.argtypes = [vp, vp, vp, i32, i32, i32, i32]
        L.orc_seqsum_f32.restype = f32
        L.orc_seqsum_f32.argtypes = [vp, i64, f32, ctypes.POINTER(i64)]
        _libs[path] = L
    return _libs[path]


def _vp(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def select_topk_indices(logits, k, double=False):
    x = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.empty(max(k, 1), np.int32)
    n = load(double).orc_select_topk_indices(_vp(x), x.size, int(k), _vp(out))
    return out[:n].copy()


def do_sample(logits, temperature, top_k, top_p, u, softcap=30.0, want_probs=True, double=False):
    """DoSample on one fp32 row.  Returns (token, detail dict, indices, probs)."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    V = x.size
    p = Params(float(temperature), int(top_k), float(top_p), 1.0)
    full = top_k <= 0 or top_k >= V
    cap = V if full else max(int(top_k), 1)
    idx = np.empty(cap, np.int32) if want_probs else None
    probs = np.empty(cap, np.float32) if want_probs else None
    d = Detail()
    tok = load(double).orc_do_sample(_vp(x), V, float(softcap), ctypes.byref(p), float(u),
                                     _vp(idx) if want_probs else None,
                                     _vp(probs) if want_probs else None,
                                     cap if want_probs else 0, ctypes.byref(d))
    det = d.as_dict()
    if want_probs:
        n = det["count"]
        idx, probs = idx[:n].copy(), probs[:n].copy()
    return tok, det, idx, probs


def sample_batch(logits, dtype, vocab, row_stride, params, u, softcap=30.0, threads=1):
    """orc_sample_batch: params = (t, k, p) arrays; returns ids."""
    t, k, pp = params
    B = len(t)
    parr = (Params * B)()
    for i in range(B):
        parr[i] = Params(float(t[i]), int(k[i]), float(pp[i]), 1.0)
    uu = np.ascontiguousarray(u, np.float64)
    ids = np.empty(B, np.int32)
    x = np.ascontiguousarray(logits)
    load().orc_sample_batch(_vp(x), int(dtype), int(vocab), int(row_stride), B, parr, _vp(uu),
                            float(softcap), _vp(ids), int(threads))
    return ids


def softcap_topk(x, cap=30.0):
    return np.float32(load().orc_softcap_topk(float(x), float(cap)))


def logit_softcap(x, cap=30.0):
    a = np.array(x, np.float32).copy()
    load().orc_logit_softcap(_vp(a), a.size, float(cap))
    return a


def softmax_f32(x):
    a = np.array(x, np.float32).copy()
    lsum = load().orc_softmax_f32(_vp(a), a.size)
    return a, np.float32(lsum)


def exp_diff(a, b):
    return np.float32(load().orc_exp_diff(float(a), float(b)))


def seqsum(a, threshold=np.inf):
    x = np.ascontiguousarray(a, np.float32)
    first = ctypes.c_int64()
    s = load().orc_seqsum_f32(_vp(x), x.size, float(threshold), ctypes.byref(first))
    return np.float32(s), first.value


def bf16_to_f32(v):
    return np.float32(load().orc_bf16_to_f32(int(v)))


def f16_to_f32(v):
    return np.float32(load().orc_f16_to_f32(int(v)))


def f16_from_f32(x):
    return load().orc_f16_from_f32(float(x))


def f32_to_bf16(x):
    return load().orc_f32_to_bf16(float(x))


def dequant_q4_block(block18):
    b = np.ascontiguousarray(block18, np.uint8)
    out = np.empty(32, np.float32)
    load().orc_dequant_q4_block(_vp(b), _vp(out))
    return out


def f32_to_q4(src):
    s = np.ascontiguousarray(src, np.float32)
    out = np.empty((s.size // 32) * 18, np.uint8)
    load().orc_f32_to_q4_buffer(_vp(s), _vp(out), s.size)
    return out


def matvec_q4(matrix, vec, rows, cols, row0=0, nrows=None):
    m = np.ascontiguousarray(matrix, np.uint8)
    v = np.ascontiguousarray(vec, np.float32)
    dst = np.zeros(rows, np.float32)
    load().orc_matvec_q4(_vp(m), _vp(v), _vp(dst), rows, cols, row0,
                         rows - row0 if nrows is None else nrows)
    return dst


def matvec_q4_batch(matrix, vecs, rows, cols, threads=8):
    m = np.ascontiguousarray(matrix, np.uint8)
    v = np.ascontiguousarray(vecs, np.float32)
    B = v.shape[0]
    dst = np.zeros((B, rows), np.float32)
    load().orc_matvec_q4_batch(_vp(m), _vp(v), _vp(dst), rows, cols, B, threads)
    return dst


# --------------------------------------------------------------------------
# Decode loop (TModel.Generate) and its embedding lookup

EOS_TOKENS = (1, 106, 50)  # CEosTokenId1..3 / IsEosToken, src/Gemma4.Types.pas:65-67,554-559


def embed_q4(matrix, token, cols, scale):
    """DoEmbeddingLookup for a Q4_0 table (src/Gemma4.Model.pas:2047-2080):
    Q4ToF32Buffer of row `token` (DequantQ4Block per block, Quant.pas:209-239)
    then CpuScaleF32 by `scale` (Tensors.pas:626-636), in binary32."""
    nblk = cols // 32
    m = np.ascontiguousarray(matrix, np.uint8)
    row = m[token * nblk * 18:(token + 1) * nblk * 18].reshape(nblk, 18)
    out = np.concatenate([dequant_q4_block(row[k]) for k in range(nblk)])
    return (out * np.float32(scale)).astype(np.float32)


def generate(first_logits, params, max_tokens, forward, random, on_token=None, softcap=30.0):
    """TModel.Generate (src/Gemma4.Model.pas:2887-2928) for each sequence b of
    a batch, restated step by step: LTokenId := DoSample (:2889); while
    LI < AMaxTokens (:2904): append (:2906), stop on IsEosToken (:2908-2909)
    or a False callback (:2911-2916), Forward (:2919), DoSample (:2923),
    Inc(LI) (:2926).  Sequences advance together; forward(tokens) gets -1 for
    sequences that take no step and returns the next logits rows; random(b)
    stands in for System.Random, called as DoSample would (only T > 0).
    Returns the token lists."""
    B = len(params)

    def sample(rows, b):
        t, k, p = params[b]
        u = random(b) if t > 0 else 0.0
        tok, _, _, _ = do_sample(rows[b], t, k, p, u, softcap=softcap, want_probs=False)
        return tok

    cur = [sample(first_logits, b) for b in range(B)]
    out = [[] for _ in range(B)]
    live = [True] * B
    while True:
        step = [-1] * B
        for b in range(B):
            if not live[b]:
                continue
            if len(out[b]) >= max_tokens:
                live[b] = False
                continue
            out[b].append(cur[b])
            if cur[b] in EOS_TOKENS or (on_token is not None and not on_token(b, cur[b])):
                live[b] = False
                continue
            step[b] = cur[b]
        if all(t < 0 for t in step):
            return out
        rows = forward(step)
        for b in range(B):
            if step[b] >= 0:
                cur[b] = sample(rows, b)


def lcg_uniforms(seed):
    """A multiplicative-congruential stream of uniforms in [0, 1) with 2^-32
    granularity (x := x * 134775813 + 1 mod 2^32, u = x / 2^32), the shape of
    the engine's System.Random draws; test input only."""
    x = seed & 0xFFFFFFFF
    while True:
        x = (x * 134775813 + 1) & 0xFFFFFFFF
        yield x / 4294967296.0
