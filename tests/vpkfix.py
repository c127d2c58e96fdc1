"""Writer of small VPK archives for the weight-store tests.

It follows the layout the engine's packer produces: TVFS.Pack
(src/vendor/StdApp/StdApp.VFS.pas:460-640) writes a 52-byte header (magic
"VPK0", version 1, entry count, data start, 32 reserved bytes), then one
544-byte record per file (path as 260 UTF-16 code units, normalised to
lower case with '/', then offset, size, CRC-32 and flags), then the files'
bytes back to back; TPacker (src/Gemma4.Packer.pas:339-395) writes
weights.bin and a manifest.json whose "tensors" array lists name,
source_dtype, output_dtype, offset, size and shape per tensor.  The knobs
below break one rule at a time for the error-path tests.
"""
import json
import struct
import zlib

HEADER = struct.Struct("<4sIIQ32s")
ENTRY_TAIL = struct.Struct("<QQII")
PATH_UNITS = 260
ENTRY_BYTES = PATH_UNITS * 2 + ENTRY_TAIL.size
assert HEADER.size == 52 and ENTRY_BYTES == 544


def entry_path_bytes(path):
    units = path.encode("utf-16-le")
    assert len(units) // 2 <= PATH_UNITS
    return units + b"\0" * (PATH_UNITS * 2 - len(units))


def pack(files, magic=b"VPK0", version=1, count=None, bad_crc=(), truncate=None,
         offset_shift=None, normalise=True):
    """bytes of an archive holding `files` (list of (path, bytes)).
    bad_crc: paths whose stored CRC is off by one; offset_shift: {path: n}
    moves an entry's recorded offset; truncate: cut the archive to n bytes."""
    n = len(files)
    data_start = HEADER.size + n * ENTRY_BYTES
    out = bytearray(HEADER.pack(magic, version, n if count is None else count, data_start,
                                b"\0" * 32))
    off = data_start
    recs = []
    for path, blob in files:
        p = path.replace("\\", "/").lower() if normalise else path
        crc = zlib.crc32(blob) & 0xFFFFFFFF
        if path in bad_crc:
            crc ^= 1
        o = off + (offset_shift or {}).get(path, 0)
        recs.append(entry_path_bytes(p) + ENTRY_TAIL.pack(o, len(blob), crc, 0))
        off += len(blob)
    for r in recs:
        out += r
    for _, blob in files:
        out += blob
    if truncate is not None:
        out = out[:truncate]
    return bytes(out)


def manifest(tensors):
    """manifest.json text for tensors given as dicts (name, source_dtype,
    output_dtype, offset, size, shape) -- the packer's field names."""
    return json.dumps({"tensors": tensors}, indent=2).encode()


def weights_archive(tensors, extra_files=(), manifest_path="E4B/manifest.json",
                    weights_path="E4B/weights.bin", **kw):
    """A model archive: tensors as (name, output_dtype, shape, bytes), stored
    back to back in weights.bin with their manifest entries."""
    blob = bytearray()
    entries = []
    for name, dtype, shape, data in tensors:
        entries.append({"name": name, "source_dtype": "BF16" if dtype == "Q4_0" else dtype,
                        "output_dtype": dtype, "offset": len(blob), "size": len(data),
                        "shape": list(shape)})
        blob += data
    files = [(manifest_path, manifest(entries)), (weights_path, bytes(blob))] + list(extra_files)
    return pack(files, **kw), entries
