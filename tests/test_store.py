"""The weight store (g4s_store_*, TWeightStore over TVFS) on the host: archive
and manifest parsing, lookups and every error path of TVFS.Open /
TWeightStore.Open (src/vendor/StdApp/StdApp.VFS.pas:243-363,
src/Gemma4.Tensors.pas:321-516), on archives written by tests/vpkfix.py.
No GPU: nothing here reaches a HIP call.
"""
import ctypes
import json
import os
import zlib

import numpy as np
import pytest

from gemma4_sampler import native, workload as wl

import vpkfix

EMBED = "model.language_model.embed_tokens.weight"


def _q4(rows, cols, seed=5):
    return wl.host_q4_weights(seed, rows, cols).tobytes()


def _write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


@pytest.fixture
def model_vpk(tmp_path):
    rows, cols = 96, 64
    norm = np.arange(cols, dtype=np.float32).tobytes()
    data, entries = vpkfix.weights_archive([
        ("model.language_model.norm.weight", "F32", [cols], norm),
        (EMBED, "Q4_0", [rows, cols], _q4(rows, cols)),
    ])
    return _write(tmp_path, "model.vpk", data), entries


def test_open_lists_the_manifest(model_vpk):
    path, entries = model_vpk
    st = native.WeightStore()
    assert st.Open(path), st.LastError()
    assert st.TensorCount() == 2
    for i, e in enumerate(entries):
        name, info = st.GetTensorInfo(i)
        assert name == e["name"]
        assert info.Offset == e["offset"] and info.DataSize == e["size"]
        assert info.Shape == tuple(e["shape"])
    ok, info = st.FindTensor(EMBED)
    assert ok and info.OutputDtype == native.WDTYPE_Q4_0 and info.SourceDtype == native.WDTYPE_BF16
    assert st.GetRawBytes(EMBED) == _q4(96, 64)
    assert st.GetRawBytes("model.language_model.norm.weight") == \
        np.arange(64, dtype=np.float32).tobytes()
    assert st.Verify()
    ok, _ = st.FindTensor("nope")
    assert not ok and "Tensor not found: nope" in st.LastError()
    st.Close()
    assert not st.IsOpen()


def test_record_layout_by_hand(tmp_path):
    """One entry written byte by byte from the packed records' field sizes
    (header 4+4+4+8+32, entry 520+8+8+4+4), independently of vpkfix."""
    man = json.dumps({"tensors": [{"name": "t", "source_dtype": "F32", "output_dtype": "F32",
                                   "offset": 0, "size": 4, "shape": [1]}]}).encode()
    w = np.float32(1.5).tobytes()
    files = [("e4b/manifest.json", man), ("e4b/weights.bin", w)]
    raw = bytearray(b"VPK0" + (1).to_bytes(4, "little") + (2).to_bytes(4, "little"))
    start = 52 + 2 * 544
    raw += start.to_bytes(8, "little") + bytes(32)
    off = start
    for p, b in files:
        path = p.encode("utf-16-le").ljust(520, b"\0")
        raw += path + off.to_bytes(8, "little") + len(b).to_bytes(8, "little")
        raw += (zlib.crc32(b) & 0xFFFFFFFF).to_bytes(4, "little") + bytes(4)
        off += len(b)
    raw += man + w
    assert bytes(raw) == vpkfix.pack(files)
    st = native.WeightStore()
    assert st.Open(_write(tmp_path, "h.vpk", bytes(raw))), st.LastError()
    assert st.GetRawBytes("t") == w and st.Verify()


def test_extension_is_forced_to_vpk(model_vpk, tmp_path):
    """TVFS.Open applies TPath.ChangeExtension(name, 'vpk')."""
    path, _ = model_vpk
    st = native.WeightStore()
    assert st.Open(path[:-4] + ".bin"), st.LastError()
    assert st.Open(path[:-4]), st.LastError()
    st.Close()


def test_paths_are_normalised(model_vpk):
    path, _ = model_vpk
    st = native.WeightStore()
    assert st.Open(path, "E4B\\MANIFEST.JSON", "e4b/Weights.BIN"), st.LastError()
    assert st.TensorCount() == 2


@pytest.mark.parametrize("case, code, text", [
    ("missing", native.G4S_ERR_IO, "Failed to open VPK"),
    ("short", native.G4S_ERR_FORMAT, "truncated"),
    ("magic", native.G4S_ERR_FORMAT, "Invalid VPK magic"),
    ("version", native.G4S_ERR_FORMAT, "Unsupported VPK version: 2"),
    ("directory", native.G4S_ERR_FORMAT, "truncated"),
    ("no_manifest", native.G4S_ERR_NOT_FOUND, "Manifest not found in VPK"),
    ("no_weights", native.G4S_ERR_NOT_FOUND, "Weights file not found in VPK"),
    ("bad_json", native.G4S_ERR_FORMAT, "Failed to parse manifest JSON"),
    ("no_tensors", native.G4S_ERR_FORMAT, "Missing tensors array in manifest"),
    ("empty", native.G4S_ERR_FORMAT, "Manifest lists no tensors"),
    ("beyond", native.G4S_ERR_FORMAT, "beyond the archive"),
])
def test_open_errors(tmp_path, case, code, text):
    man = vpkfix.manifest([{"name": "t", "source_dtype": "F32", "output_dtype": "F32",
                            "offset": 0, "size": 4, "shape": [1]}])
    w = bytes(4)
    good = [("E4B/manifest.json", man), ("E4B/weights.bin", w)]
    data = {
        "short": b"VPK0\x01\x00",
        "magic": vpkfix.pack(good, magic=b"VPK1"),
        "version": vpkfix.pack(good, version=2),
        "directory": vpkfix.pack(good, count=5),
        "no_manifest": vpkfix.pack(good[1:]),
        "no_weights": vpkfix.pack(good[:1]),
        "bad_json": vpkfix.pack([("E4B/manifest.json", b'{"tensors": [}')] + good[1:]),
        "no_tensors": vpkfix.pack([("E4B/manifest.json", b'{"tensor": []}')] + good[1:]),
        "empty": vpkfix.pack([("E4B/manifest.json", b'{"tensors": []}')] + good[1:]),
        "beyond": vpkfix.pack(good, offset_shift={"E4B/weights.bin": 100}),
    }.get(case)
    path = str(tmp_path / "absent.vpk") if data is None else _write(tmp_path, "m.vpk", data)
    L = native.load()
    h = ctypes.c_void_p(1234)
    rc = L.g4s_store_open(ctypes.byref(h), path.encode(), None, None)
    assert rc == code and not h.value
    assert text in L.g4s_store_last_error(None).decode()


def test_manifest_field_defaults_and_duplicates(tmp_path):
    """TJSON accessors with defaults (AsString(''), AsUInt64(0), AsInt32(0)),
    case-sensitive dtype names (DtypeKindFromString, Types.pas:505-517) and
    AddOrSetValue: a repeated name resolves to its last entry."""
    man = json.dumps({"tensors": [
        {"name": "a", "output_dtype": "q4_0", "offset": 8, "size": 4, "shape": [2, 3]},
        {"name": "b", "source_dtype": 7, "output_dtype": "F16", "offset": -1, "size": 1.5},
        {"name": "a", "source_dtype": "BF16", "output_dtype": "Q4_0", "offset": 0, "size": 4,
         "shape": []},
        {"name": "café \\ud83d", "output_dtype": "F32", "size": 4},
    ]}).encode()
    data = vpkfix.pack([("E4B/manifest.json", man), ("E4B/weights.bin", bytes(16))])
    st = native.WeightStore()
    assert st.Open(_write(tmp_path, "d.vpk", data)), st.LastError()
    assert st.TensorCount() == 4
    n0, i0 = st.GetTensorInfo(0)
    assert n0 == "a" and i0.OutputDtype == native.WDTYPE_UNKNOWN and i0.Shape == (2, 3)
    _, i1 = st.GetTensorInfo(1)
    assert i1.SourceDtype == native.WDTYPE_UNKNOWN and i1.OutputDtype == native.WDTYPE_F16
    assert i1.Offset == 0 and i1.DataSize == 0 and i1.Shape == ()
    ok, ia = st.FindTensor("a")
    assert ok and ia.OutputDtype == native.WDTYPE_Q4_0 and ia.Offset == 0 and ia.Shape == ()
    n3, _ = st.GetTensorInfo(3)
    assert n3 == "café \\ud83d"


def test_unicode_entry_paths(tmp_path):
    """Entry paths are UTF-16 in the directory; non-ASCII paths are found
    when asked for exactly as stored."""
    man = vpkfix.manifest([{"name": "t", "source_dtype": "F32", "output_dtype": "F32",
                            "offset": 0, "size": 4, "shape": [1]}])
    data = vpkfix.pack([("münchen/manifest.json", man), ("münchen/w\U0001F600.bin",
                                                               bytes(4))])
    st = native.WeightStore()
    assert st.Open(_write(tmp_path, "u.vpk", data), "münchen/manifest.json",
                   "münchen/w\U0001F600.bin"), st.LastError()


def test_checksum_mismatch_is_reported(tmp_path):
    man = vpkfix.manifest([{"name": "t", "source_dtype": "F32", "output_dtype": "F32",
                            "offset": 0, "size": 4, "shape": [1]}])
    data = vpkfix.pack([("E4B/manifest.json", man), ("E4B/weights.bin", bytes(4))],
                       bad_crc=("E4B/weights.bin",))
    st = native.WeightStore()
    assert st.Open(_write(tmp_path, "c.vpk", data))  # TVFS.Open does not check CRCs
    assert not st.Verify() and "CRC-32 of e4b/weights.bin" in st.LastError()


def test_tensor_beyond_weights_entry(tmp_path):
    man = vpkfix.manifest([{"name": "t", "source_dtype": "F32", "output_dtype": "F32",
                            "offset": 2, "size": 4, "shape": [1]}])
    data = vpkfix.pack([("E4B/manifest.json", man), ("E4B/weights.bin", bytes(4))])
    st = native.WeightStore()
    assert st.Open(_write(tmp_path, "b.vpk", data))
    with pytest.raises(native.SamplerError, match="beyond the weights entry"):
        st.GetRawBytes("t")


def test_device_bytes():
    assert native.q4_0_device_bytes(262144, 2560, native.Q4_LAYOUT_ROWS) == 377487360
    assert native.q4_0_device_bytes(262144, 2560, native.Q4_LAYOUT_TILED64) == 4096 * 80 * 1280
    assert native.q4_0_device_bytes(65, 64, native.Q4_LAYOUT_TILED64) == 2 * 2 * 1280
    assert native.q4_0_device_bytes(10, 48, native.Q4_LAYOUT_ROWS) == -1
    assert native.q4_0_device_bytes(10, 64, 7) == -1


@pytest.mark.parametrize("case, text", [
    ("not_q4", "is not Q4_0"),
    ("shape", r"a Q4_0 matrix \[rows, cols\]"),
    ("size", r"a \[4, 64\] Q4_0 matrix has 144"),
    ("layout", "layout 9 is unknown"),
    ("small", "the layout needs"),
    ("align", "not 16-byte aligned"),
    ("missing", "Tensor not found"),
])
def test_upload_argument_errors(tmp_path, case, text):
    """Upload checks that fail before any device work."""
    q = _q4(4, 64)
    data, _ = vpkfix.weights_archive([
        ("f", "F32", [4], bytes(16)),
        ("bad_shape", "Q4_0", [4, 48], q),
        ("bad_size", "Q4_0", [4, 64], q[:-18]),
        ("w", "Q4_0", [4, 64], q),
    ])
    st = native.WeightStore()
    assert st.Open(_write(tmp_path, "e.vpk", data)), st.LastError()
    name, layout, ptr, nbytes = {
        "not_q4": ("f", 0, 4096, 1 << 20),
        "shape": ("bad_shape", 0, 4096, 1 << 20),
        "size": ("bad_size", 0, 4096, 1 << 20),
        "layout": ("w", 9, 4096, 1 << 20),
        "small": ("w", 1, 4096, 100),
        "align": ("w", 0, 4104, 1 << 20),
        "missing": ("zz", 0, 4096, 1 << 20),
    }[case]
    with pytest.raises(native.SamplerError, match=text):
        st.UploadQ4_0(name, layout, ptr, nbytes)
