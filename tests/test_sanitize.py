"""Host AddressSanitizer / UndefinedBehaviorSanitizer run on the CPU: the
oracle on rows of every regime, every entry point's argument checks, and the
weight store on well-formed, malformed and randomly damaged VPK archives
(`tests/native/sanitize_check.cpp`, built by `make -C tests/native
sanitize`).  A sanitizer report aborts the driver, so the test passes only
when every access stays in bounds and no undefined operation runs."""
import json
import os
import random
import subprocess

import numpy as np
import pytest

from gemma4_sampler import workload as wl

import vpkfix

HERE = os.path.dirname(os.path.abspath(__file__))
NATIVE = os.path.join(HERE, "native")
DRIVER = os.path.join(NATIVE, "build", "sanitize", "sanitize_check")


def _archives(tmp_path):
    """Paths of archives: good ones, each rule of the format broken, and
    manifests with random damage."""
    rng = random.Random(7)
    q = wl.host_q4_weights(3, 64, 64).tobytes()
    good, _ = vpkfix.weights_archive([
        ("model.language_model.norm.weight", "F32", [64], np.ones(64, np.float32).tobytes()),
        ("model.language_model.embed_tokens.weight", "Q4_0", [64, 64], q),
        ("odd_shape", "Q4_0", [3, 48], q[:3 * 2 * 18]),
        ("beyond", "Q4_0", [64, 64], q),
    ])
    man = json.dumps({"tensors": [
        {"name": "a", "source_dtype": "BF16", "output_dtype": "Q4_0", "offset": 0,
         "size": len(q), "shape": [64, 64]},
        {"name": "far", "output_dtype": "F32", "offset": 2 ** 40, "size": 16, "shape": [4]},
        {"name": "huge", "output_dtype": "F32", "offset": 0, "size": 2 ** 63, "shape": [4]},
        {"name": "neg", "output_dtype": "F32", "offset": -5, "size": 4, "shape": [-1, 1e30]},
        {"name": "deep", "shape": [[[[1]]]], "size": "7"},
    ]}).encode()
    blobs = {
        "good": good,
        "odd_records": vpkfix.pack([("E4B/manifest.json", man), ("E4B/weights.bin", q)]),
        "truncated_header": good[:30],
        "truncated_dir": good[:52 + 544],
        "truncated_data": good[:-100],
        "bad_magic": vpkfix.pack([("E4B/manifest.json", man)], magic=b"XXXX"),
        "count_huge": vpkfix.pack([("E4B/manifest.json", man)], count=0xFFFFFFFF),
        "offset_beyond": vpkfix.pack([("E4B/manifest.json", man), ("E4B/weights.bin", q)],
                                     offset_shift={"E4B/weights.bin": 1 << 40}),
        "nested": vpkfix.pack([("E4B/manifest.json", b"[" * 5000 + b"]" * 5000),
                               ("E4B/weights.bin", q)]),
        "empty_json": vpkfix.pack([("E4B/manifest.json", b""), ("E4B/weights.bin", q)]),
        "escapes": vpkfix.pack([("E4B/manifest.json",
                                 b'{"tensors":[{"name":"\\ud83d\\ude00\\u0000\\ud800x\\"",'
                                 b'"offset":1e400,"size":0.5,"shape":[1,2,3,4,5,6,7,8]}]}'),
                                ("E4B/weights.bin", q)]),
        "too_many_dims": vpkfix.pack([("E4B/manifest.json",
                                       b'{"tensors":[{"name":"t","shape":[1,2,3,4,5,6,7,8,9]}]}'),
                                      ("E4B/weights.bin", q)]),
        "no_nul_path": vpkfix.pack([("x" * 260, man), ("E4B/weights.bin", q)]),
    }
    # random damage to a good manifest: cut, flipped bytes, inserted brackets
    text = man.decode()
    for i in range(40):
        t = list(text)
        kind = i % 4
        if kind == 0:
            t = t[:rng.randrange(len(t))]
        elif kind == 1:
            for _ in range(5):
                t[rng.randrange(len(t))] = chr(rng.randrange(32, 127))
        elif kind == 2:
            pos = rng.randrange(len(t))
            t[pos:pos] = list(rng.choice(["[", "{", "\"", "\\", "\\u12", "-", "1e", ",]"]))
        else:
            t = list(text.replace("\"size\": ", "\"size\": -" if i % 8 == 3 else "\"size\": 9"))
        blobs[f"damaged_{i}"] = vpkfix.pack([("E4B/manifest.json", "".join(t).encode("utf-8",
                                                                                   "replace")),
                                             ("E4B/weights.bin", q)])
    paths = []
    for name, data in blobs.items():
        p = tmp_path / f"{name}.vpk"
        p.write_bytes(data)
        paths.append(str(p))
    return paths


def test_host_code_under_asan_and_ubsan(tmp_path):
    r = subprocess.run(["make", "-C", NATIVE, "sanitize", "-j8"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    env = dict(os.environ)
    # the HIP runtime keeps process-lifetime allocations: leak reports off,
    # every other report fatal
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    r = subprocess.run([DRIVER] + _archives(tmp_path), capture_output=True, text=True, env=env,
                       timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-5000:]
    assert "clean" in r.stdout
