"""Synthetic workloads of the sampler's five benchmark configurations
(libg4s_workload.so, built from workload/g4w.hip).  Host and device
generators produce bit-identical data."""
import ctypes
import os

import numpy as np

from . import hip

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libg4s_workload.so")

V_GEMMA4 = 262144       # CVocabSize, src/Gemma4.Types.pas:43
HIDDEN_GEMMA4 = 2560    # CHiddenSize, src/Gemma4.Types.pas:36
SOFTCAP_GEMMA4 = 30.0   # CLogitSoftcap, src/Gemma4.Types.pas:49
GREEDY_EVERY = 100

_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is missing: build the package first")
        L = ctypes.CDLL(LIB_PATH)
        u64, i64, i32, vp = ctypes.c_uint64, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p
        L.g4w_host_peaky_rows.argtypes = [u64, i64, i64, i32, i64, vp, i32, i32]
        L.g4w_host_flat_bf16_rows.argtypes = [u64, i64, i64, i32, i64, vp, i32]
        L.g4w_host_row_u.argtypes = [u64, i64, i64, vp]
        L.g4w_host_mixed_params.argtypes = [u64, i64, i64, vp, vp, vp]
        L.g4w_host_hidden.argtypes = [u64, i32, i32, vp]
        L.g4w_host_q4_weights.argtypes = [u64, i64, i64, vp, i32]
        L.g4w_dev_peaky_rows.argtypes = [u64, i64, i64, i32, i64, vp, i32, vp]
        L.g4w_dev_flat_bf16_rows.argtypes = [u64, i64, i64, i32, i64, vp, vp]
        L.g4w_dev_q4_weights.argtypes = [u64, i64, i64, vp, vp]
        L.g4w_dev_hidden.argtypes = [u64, i32, i32, vp, vp]
        _lib = L
    return _lib


def _vp(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def host_peaky_rows(seed, row0, nrows, vocab=V_GEMMA4, greedy_every=0, threads=8):
    out = np.empty((nrows, vocab), dtype=np.float32)
    load().g4w_host_peaky_rows(seed, row0, nrows, vocab, vocab, _vp(out), greedy_every, threads)
    return out


def host_flat_bf16_rows(seed, row0, nrows, vocab=V_GEMMA4, threads=8):
    out = np.empty((nrows, vocab), dtype=np.uint16)
    load().g4w_host_flat_bf16_rows(seed, row0, nrows, vocab, vocab, _vp(out), threads)
    return out


def host_row_u(seed, row0, nrows):
    out = np.empty(nrows, dtype=np.float64)
    load().g4w_host_row_u(seed, row0, nrows, _vp(out))
    return out


def host_mixed_params(seed, row0, nrows):
    t = np.empty(nrows, np.float32)
    k = np.empty(nrows, np.int32)
    p = np.empty(nrows, np.float32)
    load().g4w_host_mixed_params(seed, row0, nrows, _vp(t), _vp(k), _vp(p))
    return t, k, p


def host_hidden(seed, batch, cols=HIDDEN_GEMMA4):
    out = np.empty((batch, cols), np.float32)
    load().g4w_host_hidden(seed, batch, cols, _vp(out))
    return out


def host_q4_weights(seed, rows, cols=HIDDEN_GEMMA4, block0=0, threads=8):
    nblocks = rows * (cols // 32)
    out = np.empty(nblocks * 18, np.uint8)
    load().g4w_host_q4_weights(seed, block0, nblocks, _vp(out), threads)
    return out


def dev_peaky_rows(buf, seed, row0, nrows, vocab=V_GEMMA4, stride=None, greedy_every=0,
                   stream=None):
    rc = load().g4w_dev_peaky_rows(seed, row0, nrows, vocab, vocab if stride is None else stride,
                                   buf.ptr, greedy_every,
                                   stream.handle if stream is not None else None)
    hip.check(rc, "g4w_dev_peaky_rows")


def dev_flat_bf16_rows(buf, seed, row0, nrows, vocab=V_GEMMA4, stride=None, stream=None):
    rc = load().g4w_dev_flat_bf16_rows(seed, row0, nrows, vocab,
                                       vocab if stride is None else stride, buf.ptr,
                                       stream.handle if stream is not None else None)
    hip.check(rc, "g4w_dev_flat_bf16_rows")


def dev_q4_weights(buf, seed, rows, cols=HIDDEN_GEMMA4, stream=None):
    rc = load().g4w_dev_q4_weights(seed, 0, rows * (cols // 32), buf.ptr,
                                   stream.handle if stream is not None else None)
    hip.check(rc, "g4w_dev_q4_weights")


def dev_hidden(buf, seed, batch, cols=HIDDEN_GEMMA4, stream=None):
    rc = load().g4w_dev_hidden(seed, batch, cols, buf.ptr,
                               stream.handle if stream is not None else None)
    hip.check(rc, "g4w_dev_hidden")


# --- per-configuration sampling parameters ----------------------------------

def peaky_params(rows, greedy_every=GREEDY_EVERY):
    """T=0.7, TopK=64, TopP=0.95; every `greedy_every`-th row is greedy (TopK=1)."""
    t = np.full(len(rows), 0.7, np.float32)
    k = np.array([1 if greedy_every and (r % greedy_every) == greedy_every - 1 else 64
                  for r in rows], np.int32)
    p = np.full(len(rows), 0.95, np.float32)
    return t, k, p


def flat_params(n):
    """T=1.0, TopK disabled (0 -> full-vocabulary path), TopP=0.99."""
    return (np.full(n, 1.0, np.float32), np.zeros(n, np.int32), np.full(n, 0.99, np.float32))
