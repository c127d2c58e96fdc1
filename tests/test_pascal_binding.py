"""The Pascal binding unit (gemma4.pas_amd/pascal/Gemma4.Sampler.pas) against
the C header (include/gemma4_sampler.h) and the built library, on the CPU.

No Pascal compiler exists in this image, so the unit is checked by reading
it: every `external` declaration must name an export of the header with the
same number, order and C types of arguments (a Pascal value parameter of a
pointer type is the C pointer; `const`, `var` and `out` parameters are
refused, since how a compiler passes them is not the C ABI), the records must
have the C structs' fields in order, and every constant must equal the
header's.  Then every export is called through ctypes with argument types
derived from the Pascal declaration, on paths that need no GPU.
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
UNIT = os.path.join(ROOT, "gemma4.pas_amd", "pascal", "Gemma4.Sampler.pas")
HEADER = os.path.join(ROOT, "include", "gemma4_sampler.h")

# Pascal type -> canonical C type
PAS2C = {
    "Integer": "int32_t", "Int64": "int64_t", "Single": "float", "Double": "double",
    "Cardinal": "uint32_t", "Pointer": "void*", "PAnsiChar": "char*",
    "PG4SSampler": "g4s_sampler*", "PPG4SSampler": "g4s_sampler**",
    "PG4SParams": "g4s_params*", "PG4SOutputs": "g4s_outputs*", "PDouble": "double*",
    "PInteger": "int32_t*", "PSingle": "float*", "PCardinal": "uint32_t*",
    "UInt64": "uint64_t", "PG4SStore": "g4s_store*", "PPG4SStore": "g4s_store**",
    "PG4STensorInfo": "g4s_tensor_info*", "TG4SForwardFn": "g4s_forward_fn",
    "TG4SRandomFn": "g4s_random_fn", "TG4STokenFn": "g4s_token_fn",
}
# canonical C type -> ctypes type
C2CT = {
    "int32_t": ctypes.c_int32, "int64_t": ctypes.c_int64, "float": ctypes.c_float,
    "double": ctypes.c_double, "uint32_t": ctypes.c_uint32, "char*": ctypes.c_char_p,
    "uint64_t": ctypes.c_uint64, None: None,
}


def _strip_pascal_comments(s):
    s = re.sub(r"\{.*?\}", "", s, flags=re.S)
    s = re.sub(r"\(\*.*?\*\)", "", s, flags=re.S)
    return re.sub(r"//[^\n]*", "", s)


def _strip_c_comments(s):
    s = re.sub(r"/\*.*?\*/", "", s, flags=re.S)
    return re.sub(r"//[^\n]*", "", s)


def _canon_c(t):
    t = t.replace("const", " ")
    t = re.sub(r"\s*\*\s*", "*", t)
    t = re.sub(r"\s+", " ", t).strip()
    return "int32_t" if t == "int" else t  # C int is 32 bits on LP64 Linux


def pascal_externals():
    src = _strip_pascal_comments(open(UNIT).read())
    decls = {}
    pat = re.compile(r"\b(function|procedure)\s+(g4s_\w+)\s*\((.*?)\)\s*(?::\s*(\w+))?\s*;"
                     r"\s*cdecl\s*;\s*external\s+CG4SLib\s*;", re.S)
    for kind, name, args, ret in pat.findall(src):
        params = []
        for group in [g.strip() for g in args.split(";") if g.strip()]:
            assert not re.match(r"(const|var|out)\b", group), \
                f"{name}: parameter '{group}' is not passed by value"
            names, typ = group.split(":")
            for _ in names.split(","):
                params.append(PAS2C[typ.strip()])
        decls[name] = (PAS2C[ret] if kind == "function" else "void", params)
    return decls


def header_prototypes():
    src = _strip_c_comments(open(HEADER).read())
    protos = {}
    for ret, name, args in re.findall(r"([A-Za-z_][\w \*]*?)\s*\b(g4s_\w+)\s*\(([^)]*)\)\s*;",
                                      src):
        params = []
        if args.strip() not in ("", "void"):
            for a in args.split(","):
                a = a.strip()
                m = re.match(r"(.*?)(\w+)$", a)
                params.append(_canon_c(m.group(1)))
        protos[name] = (_canon_c(ret), params)
    return protos


def c_struct_fields(name):
    src = _strip_c_comments(open(HEADER).read())
    body = re.search(r"typedef struct %s \{(.*?)\}" % name, src, re.S).group(1)
    return [(_canon_c(m.group(1)) + (f"[{m.group(3)}]" if m.group(3) else ""), m.group(2))
            for m in re.finditer(r"([\w \*]+?)\s*\b(\w+)\s*(?:\[(\w+)\])?\s*;", body)]


def pascal_record_fields(name):
    src = _strip_pascal_comments(open(UNIT).read())
    body = re.search(r"\b%s\s*=\s*record(.*?)\bend;" % name, src, re.S).group(1)
    out = []
    for line in [x.strip() for x in body.split(";") if x.strip()]:
        fname, typ = [x.strip() for x in line.split(":", 1)]
        arr = re.match(r"array\s*\[\s*0\s*\.\.\s*(\w+)\s*-\s*1\s*\]\s*of\s+(\w+)", typ)
        if arr:
            out.append((PAS2C[arr.group(2)] + "[" + arr.group(1) + "]", fname))
        else:
            out.append((PAS2C[typ], fname))
    return out


def test_every_external_matches_the_header():
    pas, hdr = pascal_externals(), header_prototypes()
    assert set(pas) == set(hdr), (set(pas) ^ set(hdr))
    for name in hdr:
        assert pas[name] == hdr[name], f"{name}: Pascal {pas[name]} vs C {hdr[name]}"


@pytest.mark.parametrize("c_name,p_name", [("g4s_params", "TG4SParams"),
                                            ("g4s_outputs", "TG4SOutputs"),
                                            ("g4s_tensor_info", "TG4STensorInfo")])
def test_records_match_the_structs(c_name, p_name):
    c = c_struct_fields(c_name)
    p = pascal_record_fields(p_name)
    assert [t for t, _ in p] == [t for t, _ in c], (p, c)
    # same field names up to case and underscores
    assert [n.lower() for _, n in p] == [n.replace("_", "").lower() for _, n in c]


def test_constants_match_the_header():
    hsrc = _strip_c_comments(open(HEADER).read())
    want = {m.group(1): int(m.group(2), 0)
            for m in re.finditer(r"#define\s+(G4S_\w+)\s+(0x[0-9a-fA-F]+|\d+)u?", hsrc)}
    for m in re.finditer(r"\b(G4S_\w+)\s*=\s*(-?\d+)", hsrc):
        want[m.group(1)] = int(m.group(2))
    psrc = _strip_pascal_comments(open(UNIT).read())
    got = {}
    for m in re.finditer(r"\b(G4S_\w+)\s*=\s*(-?\$?[0-9A-Fa-f]+)\s*;", psrc):
        v = m.group(2)
        got[m.group(1)] = int(v.replace("$", "0x"), 0) if "$" in v else int(v)
    assert set(got) == set(want), set(got) ^ set(want)
    for k in want:
        assert got[k] == want[k], k


@pytest.fixture(scope="module")
def lib():
    from gemma4_sampler import native
    return ctypes.CDLL(native.LIB_PATH)


def _bind(lib, decls, name):
    ret, params = decls[name]
    f = getattr(lib, name)
    f.restype = C2CT.get(ret) if ret != "void" else None
    f.argtypes = [C2CT[p] if p in C2CT else ctypes.c_void_p for p in params]
    return f


def test_call_every_export_with_the_declared_shapes(lib):
    """No GPU here: create reports G4S_ERR_NO_DEVICE, the sampling and LM-head
    entry points reject a nil handle with G4S_ERR_INVALID_ARGUMENT, and the
    pure host exports answer."""
    d = pascal_externals()
    f = {n: _bind(lib, d, n) for n in d}
    assert f["g4s_version"]().decode().startswith("gemma4_sampler")
    assert f["g4s_max_top_k"]() == 1024

    class Params(ctypes.Structure):
        _fields_ = [("Temperature", ctypes.c_float), ("TopK", ctypes.c_int32),
                    ("TopP", ctypes.c_float), ("RepetitionPenalty", ctypes.c_float)]
    p = Params(0.0, 0, 0.0, 0.0)
    f["g4s_params_set_defaults"](ctypes.addressof(p))
    assert (p.Temperature, p.TopK, round(p.TopP, 6), p.RepetitionPenalty) == (1.0, 64, 0.95, 1.0)

    h = ctypes.c_void_p(0)
    rc = f["g4s_create"](ctypes.addressof(h), 262144, 1, 30.0, None)
    assert rc in (-3, 0)  # NO_DEVICE here; OK where a GPU is visible
    if rc != 0:
        assert h.value is None
        assert len(f["g4s_last_error"](None)) > 0
    u = ctypes.c_double(0.5)
    ids = ctypes.c_int32(-7)
    assert f["g4s_sample"](None, None, 0, 262144, 1, ctypes.addressof(p), ctypes.addressof(u),
                           ctypes.addressof(ids)) == -1
    assert f["g4s_sample_ex"](None, None, 0, 262144, 1, ctypes.addressof(p),
                              ctypes.addressof(u), ctypes.addressof(ids), None) == -1
    assert f["g4s_sample_async"](None, None, 0, 262144, 1, None, None, 64, 0, None, None) == -1
    assert f["g4s_lmhead_q4_0"](None, None, 262144, 2560, None, 1, None, 262144) == -1
    assert f["g4s_lmhead_q4_0_tiled"](None, None, 262144, 2560, None, 1, None, 262144) == -1
    assert f["g4s_lmhead_sample_q4_0"](None, None, 2560, None, 1, None, 262144,
                                       ctypes.addressof(p), ctypes.addressof(u),
                                       ctypes.addressof(ids), None) == -1
    assert f["g4s_last_error"](None).decode() == "sampler is NULL"
    # weight store: nil handles are refused, the pure host exports answer
    st = ctypes.c_void_p(7)
    assert f["g4s_store_open"](ctypes.addressof(st), b"/nonexistent/x.vpk", None, None) == -7
    assert st.value is None and b"Failed to open VPK" in f["g4s_store_last_error"](None)
    assert f["g4s_store_close"](None) == 0
    assert f["g4s_store_tensor_count"](None) == 0
    assert f["g4s_store_tensor_info"](None, 0, None, None, 0) == -1
    assert f["g4s_store_find_tensor"](None, b"x", None) == -1
    assert f["g4s_store_raw_pointer"](None, b"x") is None
    assert f["g4s_store_verify"](None) == -1
    assert f["g4s_store_upload_q4_0"](None, b"x", 0, None, 0, None) == -1
    assert f["g4s_q4_0_device_bytes"](64, 64, 0) == 64 * 2 * 18
    assert f["g4s_q4_0_repack"](None, 64, 64, None, None) == -1
    assert f["g4s_embed_q4_0"](None, None, 64, 64, None, 1, 1.0, None) == -1
    assert f["g4s_generate"](None, 1, None, 4, None, 0, 64, None, None, None, None, None,
                             None) == -1
    if rc == 0:
        assert f["g4s_destroy"](h) == 0
    assert f["g4s_destroy"](None) == 0


# --------------------------------------------------------------------------
# TGpuSampler.Sample and the engine-side integration (model_integration.py)
# --------------------------------------------------------------------------

def _method_body(src, header_regex):
    """Text between `begin` and the matching final `end;` of one method."""
    m = re.search(header_regex + r".*?\bbegin\b(.*?)\nend;", src, re.S)
    assert m, header_regex
    return m.group(1)


def test_sample_draws_random_only_when_the_row_draws():
    """DoSample calls Random only when Temperature > 0 (Model.pas:2723-2726 on
    the full path, :2811-2813 on the top-k path): the shim that takes its
    place must consume the RTL stream the same way, or every later T > 0
    token of the process is drawn from a shifted stream."""
    src = _strip_pascal_comments(open(UNIT).read())
    body = _method_body(src, r"function TGpuSampler\.Sample\(")
    flat = re.sub(r"\s+", " ", body)
    assert len(re.findall(r"\bRandom\b", flat)) == 1, flat
    assert re.search(r"if AParams\^\.Temperature > 0\.0 then LU := Random else LU := 0\.0;",
                     flat), flat
    # the only use of u is the library call, after the guard
    assert flat.index("Random") < flat.index("g4s_sample(")


def _integration():
    import importlib.util
    p = os.path.join(ROOT, "gemma4.pas_amd", "pascal", "model_integration.py")
    spec = importlib.util.spec_from_file_location("model_integration", p)
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def test_integration_do_sample_calls_only_the_gpu_sampler():
    mi = _integration()
    body = mi.DO_SAMPLE.split("procedure TModel.SetDeviceLogits")[0]
    code = _strip_pascal_comments(body)
    calls = re.findall(r"\b([A-Za-z_][\w\.]*)\s*\(", code)
    # GetErrors().Add reports missing logits; PG4SParams is a type cast
    assert [c for c in calls if c not in ("TModel.DoSample", "GetErrors", "Add",
                                          "PG4SParams")] == ["FSampler.Sample"], calls
    for banned in ("Random", "FLogits", "DoSelectTopKIndices", "DoSampleTopP", "CpuSoftmaxF32",
                   "CpuLogitSoftcap", "Exp", "Tanh"):
        assert not re.search(r"\b%s\b" % banned, code), banned


REF_MODEL = "/root/reference/src/Gemma4.Model.pas"


@pytest.mark.skipif(not os.path.exists(REF_MODEL), reason="the engine's Model.pas is not here")
def test_integration_applies_to_the_engine_model():
    mi = _integration()
    src = open(REF_MODEL, encoding="utf-8-sig").read().replace("\r\n", "\n")
    out = mi.apply(src)
    code = _strip_pascal_comments(out)
    # the logits never come back to the host
    assert "DownloadFromBuffer(FGpuLogits" not in code
    assert "Exit(Copy(FLogits))" not in code
    # DoSample: one call into the GPU sampler, no CPU sampling left in it
    body = _method_body(code, r"function TModel\.DoSample\(const AParams: TSamplingParams\)")
    assert "FSampler.Sample(FDevLogits, G4S_DTYPE_F32, PG4SParams(@AParams), Result)" in body
    for banned in ("Random", "FLogits", "DoSelectTopKIndices", "DoSampleTopP", "Exp("):
        assert banned not in body, banned
    # Generate: a failed sample ends the loop before its id is added
    gen = _method_body(code, r"function TModel\.Generate\(")
    flat = re.sub(r"\s+", " ", gen)
    assert flat.count("LResult.Add(LTokenId);") == 1
    assert "while LI < AMaxTokens do begin if LTokenId < 0 then Break; LResult.Add(LTokenId);" \
        in flat, flat[:400]
    # the sampler lives with the GPU buffers
    alloc = _method_body(code, r"function TModel\.DoAllocateResidentGpuBuffers\(\)")
    assert re.search(r"FSampler := TGpuSampler\.Create\(\);\s*FSampler\.SetErrors\(GetErrors\(\)\);"
                     r"\s*if not FSampler\.Open\(FConfig\.VocabSize, 1, "
                     r"FConfig\.FinalLogitSoftcapping\) then\s*Exit;", alloc)
    free = _method_body(code, r"procedure TModel\.DoFreeGpuBuffers\(\)")
    assert re.match(r"\s*FreeAndNil\(FSampler\);", free)
    assert re.search(r"\bGemma4\.Compute,\s*Gemma4\.Sampler;", code)
    assert re.search(r"FSampler: TGpuSampler;\s*FDevLogits: Pointer;", code)
    # every anchor is consumed: a second application finds nothing to edit
    with pytest.raises(mi.IntegrationError):
        mi.apply(out)


def test_integration_refuses_a_file_it_does_not_know():
    mi = _integration()
    with pytest.raises(mi.IntegrationError, match="uses"):
        mi.apply("unit Gemma4.Model;\ninterface\nimplementation\nend.\n")
