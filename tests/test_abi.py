"""The C ABI library loads on the CPU and exports every function that
include/gemma4_sampler.h declares; host-side argument handling."""
import ctypes
import os
import re

import pytest

from gemma4_sampler import hip, native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            src = open(os.path.join(ROOT, "include", fn)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            names |= set(re.findall(r"\b(g4s_[a-z0-9_]+)\s*\(", src))
    return names


def test_exports_every_declared_symbol():
    L = native.load()
    decl = declared_functions()
    assert decl == set(native.EXPORTS)
    for name in decl:
        assert hasattr(L, name), name


def test_version_defaults_limits():
    assert native.version().startswith("gemma4_sampler")
    p = native.TSamplingParams().SetDefaults()
    assert (p.Temperature, p.TopK, round(p.TopP, 6), p.RepetitionPenalty) == (1.0, 64, 0.95, 1.0)
    assert native.max_top_k() == 1024


@pytest.mark.skipif(hip.device_count() > 0, reason="checks the no-device error path")
def test_create_without_device_reports_no_device():
    with pytest.raises(native.SamplerError) as e:
        native.Sampler(262144, 1)
    assert e.value.code == native.G4S_ERR_NO_DEVICE


def test_create_argument_errors():
    L = native.load()
    h = ctypes.c_void_p()
    assert L.g4s_create(None, 10, 1, 30.0, None) == native.G4S_ERR_INVALID_ARGUMENT
    assert L.g4s_create(ctypes.byref(h), 1, 1, 30.0, None) == native.G4S_ERR_INVALID_ARGUMENT
    assert b"vocab" in L.g4s_last_error(None)
    assert L.g4s_create(ctypes.byref(h), 100, 0, 30.0, None) == native.G4S_ERR_INVALID_ARGUMENT
    assert L.g4s_create(ctypes.byref(h), 100, 1, float("nan"), None) == \
        native.G4S_ERR_INVALID_ARGUMENT
    assert L.g4s_destroy(None) == 0
    assert L.g4s_sample(None, None, 0, 0, 1, None, None, None) == \
        native.G4S_ERR_INVALID_ARGUMENT
