"""ctypes binding of libgemma4_sampler.so (include/gemma4_sampler.h).

The names mirror the reference's sampling surface: TSamplingParams
(src/Gemma4.Model.pas:70-76, SetDefaults :346-352), the TInference setters
SetTemperature / SetTopK / SetTopP (src/Gemma4.Inference.pas:2186-2199) and
DoSample (src/Gemma4.Model.pas:2739-2827), so tests read like the engine's
own call sites.  There is no fallback: if the library is missing, loading
raises.
"""
import ctypes
import os

import numpy as np

from . import hip

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libgemma4_sampler.so")

G4S_OK = 0
G4S_ERR_INVALID_ARGUMENT = -1
G4S_ERR_UNSUPPORTED = -2
G4S_ERR_NO_DEVICE = -3
G4S_ERR_OUT_OF_MEMORY = -4
G4S_ERR_HIP = -5
G4S_ERR_EMPTY_ROW = -6
G4S_ERR_IO = -7
G4S_ERR_FORMAT = -8
G4S_ERR_NOT_FOUND = -9
G4S_ERR_ABORTED = -10

EOS_TOKENS = (1, 106, 50)  # IsEosToken, src/Gemma4.Types.pas:65-67,554-559

# TDtypeKind (src/Gemma4.Types.pas:94-100)
WDTYPE_UNKNOWN, WDTYPE_BF16, WDTYPE_F16, WDTYPE_F32, WDTYPE_Q4_0 = range(5)
Q4_LAYOUT_ROWS = 0
Q4_LAYOUT_TILED64 = 1
MAX_DIMS = 8

DTYPE_F32 = 0
DTYPE_BF16 = 1

FLAG_TOPK_PATH = 0x1
FLAG_FULL_PATH = 0x2
FLAG_DREW = 0x4
FLAG_REACHED = 0x8
FLAG_TIE_LOWEST = 0x10
FLAG_HEAP_REPLAY = 0x20
FLAG_CHUNK_EXACT = 0x40
FLAG_WIDE_MERGE = 0x80
FLAG_WIDE_K = 0x100
FLAG_ROW_RECOMPUTED = 0x200
FLAG_EMPTY = 0x40000000
FLAG_ERROR = 0x80000000

EXPORTS = ("g4s_version", "g4s_params_set_defaults", "g4s_max_top_k", "g4s_create",
           "g4s_destroy", "g4s_last_error", "g4s_sample", "g4s_sample_ex", "g4s_sample_async",
           "g4s_sample_graph",
           "g4s_sample_topk_noalloc", "g4s_lmhead_q4_0", "g4s_lmhead_q4_0_tiled",
           "g4s_lmhead_sample_q4_0", "g4s_store_open", "g4s_store_close", "g4s_store_last_error",
           "g4s_store_tensor_count", "g4s_store_tensor_info", "g4s_store_find_tensor",
           "g4s_store_raw_pointer", "g4s_store_verify", "g4s_q4_0_device_bytes",
           "g4s_store_upload_q4_0", "g4s_q4_0_repack", "g4s_embed_q4_0", "g4s_generate")

FORWARD_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32),
                              ctypes.c_int32)
RANDOM_FN = ctypes.CFUNCTYPE(ctypes.c_double, ctypes.c_void_p, ctypes.c_int32)
TOKEN_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32)


class TSamplingParams(ctypes.Structure):
    """g4s_params == TSamplingParams (Model.pas:70-76)."""
    _fields_ = [("Temperature", ctypes.c_float), ("TopK", ctypes.c_int32),
                ("TopP", ctypes.c_float), ("RepetitionPenalty", ctypes.c_float)]

    def SetDefaults(self):
        load().g4s_params_set_defaults(ctypes.byref(self))
        return self

    @classmethod
    def make(cls, temperature, top_k, top_p):
        return cls(float(temperature), int(top_k), float(top_p), 1.0)


class Outputs(ctypes.Structure):
    _fields_ = [("count", ctypes.c_void_p), ("indices", ctypes.c_void_p),
                ("probs", ctypes.c_void_p), ("capacity", ctypes.c_int32),
                ("argmax", ctypes.c_void_p), ("lsum", ctypes.c_void_p),
                ("flags", ctypes.c_void_p)]


class TensorInfo(ctypes.Structure):
    """g4s_tensor_info == TTensorInfo (src/Gemma4.Types.pas:119-129) minus the name."""
    _fields_ = [("SourceDtype", ctypes.c_int32), ("OutputDtype", ctypes.c_int32),
                ("Offset", ctypes.c_uint64), ("DataSize", ctypes.c_uint64),
                ("ndim", ctypes.c_int32), ("shape_", ctypes.c_int32 * MAX_DIMS)]

    @property
    def Shape(self):
        return tuple(self.shape_[i] for i in range(self.ndim))


class SamplerError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"g4s error {code}: {msg}")
        self.code = code


_lib = None


def load():
    """Load libgemma4_sampler.so from the package's lib/ (built in-tree)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: run `python -c 'import __graft_entry__ as g; g.build()'`")
        L = ctypes.CDLL(LIB_PATH)
        L.g4s_version.restype = ctypes.c_char_p
        L.g4s_last_error.restype = ctypes.c_char_p
        L.g4s_last_error.argtypes = [ctypes.c_void_p]
        L.g4s_max_top_k.restype = ctypes.c_int32
        L.g4s_create.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int32, ctypes.c_int32,
                                 ctypes.c_float, ctypes.c_void_p]
        L.g4s_destroy.argtypes = [ctypes.c_void_p]
        L.g4s_sample.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                                 ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.g4s_sample_ex.argtypes = L.g4s_sample.argtypes + [ctypes.c_void_p]
        L.g4s_sample_async.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
                                       ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p,
                                       ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                       ctypes.c_void_p, ctypes.c_void_p]
        L.g4s_sample_graph.argtypes = L.g4s_sample_async.argtypes
        L.g4s_lmhead_q4_0.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
                                      ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
                                      ctypes.c_void_p, ctypes.c_int64]
        L.g4s_lmhead_q4_0_tiled.argtypes = L.g4s_lmhead_q4_0.argtypes
        L.g4s_lmhead_sample_q4_0.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
                                             ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p,
                                             ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                             ctypes.c_void_p, ctypes.c_void_p]
        L.g4s_store_open.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p,
                                     ctypes.c_char_p, ctypes.c_char_p]
        L.g4s_store_close.argtypes = [ctypes.c_void_p]
        L.g4s_store_last_error.restype = ctypes.c_char_p
        L.g4s_store_last_error.argtypes = [ctypes.c_void_p]
        L.g4s_store_tensor_count.restype = ctypes.c_int32
        L.g4s_store_tensor_count.argtypes = [ctypes.c_void_p]
        L.g4s_store_tensor_info.argtypes = [ctypes.c_void_p, ctypes.c_int32,
                                            ctypes.POINTER(TensorInfo), ctypes.c_char_p,
                                            ctypes.c_int32]
        L.g4s_store_find_tensor.argtypes = [ctypes.c_void_p, ctypes.c_char_p,
                                            ctypes.POINTER(TensorInfo)]
        L.g4s_store_raw_pointer.restype = ctypes.c_void_p
        L.g4s_store_raw_pointer.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
        L.g4s_store_verify.argtypes = [ctypes.c_void_p]
        L.g4s_q4_0_device_bytes.restype = ctypes.c_int64
        L.g4s_q4_0_device_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
        L.g4s_store_upload_q4_0.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int32,
                                            ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]
        L.g4s_q4_0_repack.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                      ctypes.c_void_p, ctypes.c_void_p]
        L.g4s_embed_q4_0.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
                                     ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
                                     ctypes.c_float, ctypes.c_void_p]
        L.g4s_generate.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
                                   ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, FORWARD_FN,
                                   RANDOM_FN, TOKEN_FN, ctypes.c_void_p, ctypes.c_void_p,
                                   ctypes.c_void_p]
        L.g4s_sample_topk_noalloc.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                              ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p,
                                              ctypes.c_void_p, ctypes.c_int32, ctypes.c_float,
                                              ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        _lib = L
    return _lib


NOALLOC_MAX_ROWS = 32
NOALLOC_SCRATCH_BYTES = 8602880


def sample_topk_noalloc(d_logits, batch, d_params, d_u, k_bound, d_ids, vocab,
                        dtype=DTYPE_F32, row_stride=None, softcap=30.0, outputs=None,
                        stream=None, check=True):
    """g4s_sample_topk_noalloc: the handle-free top-k path whose workspace is
    a fixed device array; returns the status (raises unless check=False)."""
    L = load()
    stride = vocab if row_stride is None else int(row_stride)
    rc = L.g4s_sample_topk_noalloc(_ptr(d_logits), int(dtype), int(vocab), stride, int(batch),
                                   _ptr(d_params), _ptr(d_u), int(k_bound), float(softcap),
                                   _ptr(d_ids),
                                   ctypes.byref(outputs) if outputs is not None else None,
                                   stream.handle if stream is not None else None)
    if check and rc != G4S_OK:
        raise SamplerError(rc, L.g4s_last_error(None).decode())
    return rc


def version():
    return load().g4s_version().decode()


def max_top_k():
    return load().g4s_max_top_k()


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, hip.Buffer):
        return x.ptr
    if isinstance(x, int):
        return ctypes.c_void_p(x)
    return x


def params_array(params):
    arr = (TSamplingParams * len(params))()
    for i, p in enumerate(params):
        arr[i] = p
    return arr


class Sampler:
    """One g4s_sampler handle: the device-side replacement of TModel.DoSample."""

    def __init__(self, vocab, max_batch=1, softcap=30.0, stream=None):
        L = load()
        h = ctypes.c_void_p()
        rc = L.g4s_create(ctypes.byref(h), int(vocab), int(max_batch), float(softcap),
                          stream.handle if stream is not None else None)
        if rc != G4S_OK:
            raise SamplerError(rc, L.g4s_last_error(None).decode())
        self.h = h
        self.vocab = int(vocab)
        self.max_batch = int(max_batch)
        self.softcap = float(softcap)
        self.params = TSamplingParams().SetDefaults()  # TInference.FSamplingParams

    # TInference sampling surface (Inference.pas:2186-2199)
    def SetTemperature(self, value):
        self.params.Temperature = float(value)

    def SetTopK(self, value):
        self.params.TopK = int(value)

    def SetTopP(self, value):
        self.params.TopP = float(value)

    @property
    def SamplingParams(self):
        return self.params

    def last_error(self):
        return load().g4s_last_error(self.h).decode()

    def _check(self, rc):
        if rc != G4S_OK:
            raise SamplerError(rc, self.last_error())

    def sample(self, d_logits, batch, params, u, dtype=DTYPE_F32, row_stride=None, outputs=None,
               check=True):
        """Synchronous g4s_sample(_ex); returns (status, ids ndarray)."""
        L = load()
        if isinstance(params, TSamplingParams):
            params = [params] * batch
        parr = params_array(params)
        uarr = np.ascontiguousarray(np.asarray(u, dtype=np.float64).reshape(-1))
        assert uarr.size == batch
        ids = np.full(batch, -7, dtype=np.int32)
        stride = self.vocab if row_stride is None else int(row_stride)
        rc = L.g4s_sample_ex(self.h, _ptr(d_logits), int(dtype), stride, int(batch), parr,
                             uarr.ctypes.data_as(ctypes.c_void_p),
                             ids.ctypes.data_as(ctypes.c_void_p),
                             ctypes.byref(outputs) if outputs is not None else None)
        if check:
            self._check(rc)
        return rc, ids

    def DoSample(self, d_logits, u, params=None, dtype=DTYPE_F32):
        """Model.pas:2739: one row, this handle's SamplingParams unless given."""
        _, ids = self.sample(d_logits, 1, [params or self.params], [u], dtype=dtype)
        return int(ids[0])

    def sample_async(self, d_logits, batch, d_params, d_u, k_bound, full_rows, d_ids,
                     dtype=DTYPE_F32, row_stride=None, outputs=None):
        L = load()
        stride = self.vocab if row_stride is None else int(row_stride)
        rc = L.g4s_sample_async(self.h, _ptr(d_logits), int(dtype), stride, int(batch),
                                _ptr(d_params), _ptr(d_u), int(k_bound), int(full_rows),
                                _ptr(d_ids), ctypes.byref(outputs) if outputs is not None else None)
        self._check(rc)

    def sample_graph(self, d_logits, batch, d_params, d_u, k_bound, full_rows, d_ids,
                     dtype=DTYPE_F32, row_stride=None, outputs=None):
        """g4s_sample_graph: sample_async replayed from a graph this handle owns."""
        L = load()
        stride = self.vocab if row_stride is None else int(row_stride)
        rc = L.g4s_sample_graph(self.h, _ptr(d_logits), int(dtype), stride, int(batch),
                                _ptr(d_params), _ptr(d_u), int(k_bound), int(full_rows),
                                _ptr(d_ids), ctypes.byref(outputs) if outputs is not None else None)
        self._check(rc)

    def lmhead_q4_0(self, d_weights, rows, cols, d_hidden, batch, d_logits, logits_stride=None):
        L = load()
        rc = L.g4s_lmhead_q4_0(self.h, _ptr(d_weights), int(rows), int(cols), _ptr(d_hidden),
                               int(batch), _ptr(d_logits),
                               int(rows if logits_stride is None else logits_stride))
        self._check(rc)

    def lmhead_q4_0_tiled(self, d_tiles, rows, cols, d_hidden, batch, d_logits,
                          logits_stride=None):
        L = load()
        rc = L.g4s_lmhead_q4_0_tiled(self.h, _ptr(d_tiles), int(rows), int(cols), _ptr(d_hidden),
                                     int(batch), _ptr(d_logits),
                                     int(rows if logits_stride is None else logits_stride))
        self._check(rc)

    def lmhead_sample_q4_0(self, d_tiles, cols, d_hidden, batch, d_logits, params, u,
                           logits_stride=None, outputs=None, check=True):
        """g4s_lmhead_sample_q4_0: LM head + sample; returns (status, ids).
        d_logits None: no logits are written (top-k rows only)."""
        L = load()
        if isinstance(params, TSamplingParams):
            params = [params] * batch
        parr = params_array(params)
        uarr = np.ascontiguousarray(np.asarray(u, dtype=np.float64).reshape(-1))
        assert uarr.size == batch
        ids = np.full(batch, -7, dtype=np.int32)
        stride = self.vocab if logits_stride is None else int(logits_stride)
        rc = L.g4s_lmhead_sample_q4_0(self.h, _ptr(d_tiles), int(cols), _ptr(d_hidden),
                                      int(batch), _ptr(d_logits), stride, parr,
                                      uarr.ctypes.data_as(ctypes.c_void_p),
                                      ids.ctypes.data_as(ctypes.c_void_p),
                                      ctypes.byref(outputs) if outputs is not None else None)
        if check:
            self._check(rc)
        return rc, ids

    def embed_q4_0(self, d_weights, rows, cols, d_tokens, batch, scale, d_hidden):
        """DoEmbeddingLookup of a ROWS-layout Q4_0 table (Model.pas:2047-2080)."""
        rc = load().g4s_embed_q4_0(self.h, _ptr(d_weights), int(rows), int(cols), _ptr(d_tokens),
                                   int(batch), float(scale), _ptr(d_hidden))
        self._check(rc)

    def Generate(self, d_logits, batch, params, max_tokens, forward, random, on_token=None,
                 dtype=DTYPE_F32, row_stride=None):
        """g4s_generate: TModel.Generate for `batch` sequences.  forward(tokens
        ndarray) -> bool (True = ok), random(seq) -> float, on_token(seq, token)
        -> bool (False = stop).  Returns a list of token arrays."""
        L = load()
        if isinstance(params, TSamplingParams):
            params = [params] * batch
        parr = params_array(params)
        mt = max(int(max_tokens), 0)
        toks = np.zeros(max(batch * mt, 1), np.int32)
        lens = np.zeros(batch, np.int32)
        errors = []

        def fwd(_, tp, n):
            try:
                return 0 if forward(np.ctypeslib.as_array(tp, (n,)).copy()) else 1
            except Exception as e:  # noqa: BLE001 -- reported after the loop
                errors.append(e)
                return 1

        def rnd(_, seq):
            try:
                return float(random(int(seq)))
            except Exception as e:  # noqa: BLE001
                errors.append(e)
                return -1.0

        def tok(_, seq, t):
            try:
                return 1 if on_token(int(seq), int(t)) else 0
            except Exception as e:  # noqa: BLE001
                errors.append(e)
                return 0

        cf, cr = FORWARD_FN(fwd), RANDOM_FN(rnd)
        ct = TOKEN_FN(tok) if on_token is not None else ctypes.cast(None, TOKEN_FN)
        stride = self.vocab if row_stride is None else int(row_stride)
        rc = L.g4s_generate(self.h, int(batch), parr, int(max_tokens), _ptr(d_logits), int(dtype),
                            stride, cf, cr, ct, None, toks.ctypes.data_as(ctypes.c_void_p),
                            lens.ctypes.data_as(ctypes.c_void_p))
        if errors:
            raise errors[0]
        self._check(rc)
        return [toks[b * mt:b * mt + lens[b]].copy() for b in range(batch)]

    def close(self):
        if self.h is not None and self.h.value:
            load().g4s_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceOutputs:
    """Device buffers for g4s_outputs plus host readback."""

    def __init__(self, batch, capacity):
        self.batch, self.capacity = batch, capacity
        self.count = hip.Buffer(4 * batch)
        self.indices = hip.Buffer(4 * batch * capacity)
        self.probs = hip.Buffer(4 * batch * capacity)
        self.argmax = hip.Buffer(4 * batch)
        self.lsum = hip.Buffer(4 * batch)
        self.flags = hip.Buffer(4 * batch)
        self.struct = Outputs(self.count.addr, self.indices.addr, self.probs.addr, capacity,
                              self.argmax.addr, self.lsum.addr, self.flags.addr)

    def read(self):
        return dict(count=self.count.download(np.int32),
                    indices=self.indices.download(np.int32).reshape(self.batch, self.capacity),
                    probs=self.probs.download(np.float32).reshape(self.batch, self.capacity),
                    argmax=self.argmax.download(np.int32),
                    lsum=self.lsum.download(np.float32),
                    flags=self.flags.download(np.uint32))


def q4_0_device_bytes(rows, cols, layout):
    return int(load().g4s_q4_0_device_bytes(int(rows), int(cols), int(layout)))


def q4_0_repack(d_rows, rows, cols, d_tiled, stream=None):
    """g4s_q4_0_repack: ROWS -> TILED64 on the device (stream-ordered)."""
    L = load()
    rc = L.g4s_q4_0_repack(_ptr(d_rows), int(rows), int(cols), _ptr(d_tiled),
                           stream.handle if stream is not None else None)
    if rc != G4S_OK:
        raise SamplerError(rc, L.g4s_store_last_error(None).decode())


class WeightStore:
    """TWeightStore (src/Gemma4.Tensors.pas:321-516) over the C ABI:
    Open / Close / FindTensor / TensorCount / GetTensorInfo / GetRawPointer,
    plus the Q4_0 upload into device memory."""

    def __init__(self):
        self.h = None

    def Open(self, vpk_path, manifest_path=None, weights_path=None):
        """Returns True on success; LastError() says why not (the engine's
        Boolean-plus-errors convention)."""
        L = load()
        self.Close()
        h = ctypes.c_void_p()
        enc = lambda x: None if x is None else str(x).encode()
        rc = L.g4s_store_open(ctypes.byref(h), enc(vpk_path), enc(manifest_path),
                              enc(weights_path))
        self._open_rc = rc
        self._open_err = "" if rc == G4S_OK else L.g4s_store_last_error(None).decode()
        if rc == G4S_OK:
            self.h = h
        return rc == G4S_OK

    def IsOpen(self):
        return self.h is not None

    def LastError(self):
        if self.h is None:
            return getattr(self, "_open_err", "")
        return load().g4s_store_last_error(self.h).decode()

    def Close(self):
        if self.h is not None:
            load().g4s_store_close(self.h)
        self.h = None

    def TensorCount(self):
        return int(load().g4s_store_tensor_count(self.h)) if self.h is not None else 0

    def GetTensorInfo(self, index):
        info = TensorInfo()
        name = ctypes.create_string_buffer(1024)
        rc = load().g4s_store_tensor_info(self.h, int(index), ctypes.byref(info), name, 1024)
        if rc != G4S_OK:
            raise SamplerError(rc, self.LastError())
        return name.value.decode(), info

    def FindTensor(self, name):
        """(found, TensorInfo) as TWeightStore.FindTensor's Boolean + out."""
        info = TensorInfo()
        rc = load().g4s_store_find_tensor(self.h, name.encode(), ctypes.byref(info))
        return rc == G4S_OK, info

    def GetRawBytes(self, name):
        """The tensor's bytes in the mapped archive (GetRawPointer + DataSize)."""
        ok, info = self.FindTensor(name)
        if not ok:
            raise SamplerError(G4S_ERR_NOT_FOUND, self.LastError())
        p = load().g4s_store_raw_pointer(self.h, name.encode())
        if not p:
            raise SamplerError(G4S_ERR_FORMAT, self.LastError())
        return ctypes.string_at(p, info.DataSize)

    def Verify(self):
        rc = load().g4s_store_verify(self.h)
        return rc == G4S_OK

    def UploadQ4_0(self, name, layout, d_dst, dst_bytes, stream=None):
        L = load()
        rc = L.g4s_store_upload_q4_0(self.h, name.encode(), int(layout), _ptr(d_dst),
                                     int(dst_bytes), stream.handle if stream is not None else None)
        if rc != G4S_OK:
            raise SamplerError(rc, self.LastError())

    def __del__(self):
        try:
            self.Close()
        except Exception:
            pass
