"""The sampler's integration into the engine's src/Gemma4.Model.pas, as code.

`apply(text)` takes the text of the engine's Gemma4.Model.pas and returns it
with the GPU sampler wired in (the unit Gemma4.Sampler.pas beside this file
must be on the engine's unit path):

  uses        Gemma4.Sampler joins the interface uses clause;
  fields      TModel gains FSampler (TGpuSampler) and FDevLogits (the HIP
              address of the logits row), and a public SetDeviceLogits;
  lifetime    the sampler is opened in DoAllocateResidentGpuBuffers next to
              the logits buffer (one workspace for the model's life, nothing
              allocated per token) and freed first thing in
              DoFreeGpuBuffers;
  readback    the per-token logits download of DoForwardGpu
              (Model.pas:1379-1387) and the one after the last prefill chunk
              (Model.pas:1889-1891) are removed: the logits stay on the GPU;
  Forward     the GPU path returns nil instead of Copy(FLogits)
              (Model.pas:2571): its callers in Generate discard the result;
  DoSample    the body (Model.pas:2739-2827) becomes one TGpuSampler.Sample
              call on FDevLogits (Random is drawn inside it, only when
              Temperature > 0, as the reference draws it);
  Generate    `if LTokenId < 0 then Break;` before `LResult.Add(LTokenId)`
              (Model.pas:2907), so a failed sample (-1, SM02 in GetErrors())
              ends generation instead of feeding Forward(-1).

Each edit is anchored on a pattern that must match the engine's file exactly
once; a file that differs from the one these anchors were written against
raises IntegrationError naming the edit, rather than being half-edited.
The replacement texts are this integration's own code.  FDevLogits is set by
the host program through SetDeviceLogits once it has imported the logits
buffer into HIP ("Getting the logits into HIP memory");
until then DoSample fails with SM02 and Generate stops.

    python model_integration.py path/to/src/Gemma4.Model.pas -o Gemma4.Model.pas
"""
import argparse
import re
import sys


class IntegrationError(RuntimeError):
    pass


class Edit:
    """Replace the single match of `pattern` (re.S) by `repl` (a template in
    which \\g<name> refers to the pattern's groups)."""

    def __init__(self, name, pattern, repl):
        self.name = name
        self.pattern = re.compile(pattern, re.S)
        self.repl = repl

    def apply(self, text):
        hits = list(self.pattern.finditer(text))
        if len(hits) != 1:
            raise IntegrationError(f"edit '{self.name}': anchor matched {len(hits)} times "
                                   f"(expected exactly once)")
        return self.pattern.sub(self.repl, text, count=1)


DO_SAMPLE = """function TModel.DoSample(const AParams: TSamplingParams): Integer;
begin
  // GPU sampler on the device-resident logits row (libgemma4_sampler.so):
  // top-k or full-vocabulary path, softcap, temperature, softmax and the
  // draw as the former CPU body did them; System.Random is drawn inside
  // TGpuSampler.Sample only when AParams.Temperature > 0.  -1 on failure,
  // with SM02 in GetErrors(); Generate stops on it.
  Result := -1;
  if FDevLogits = nil then
  begin
    GetErrors().Add(esError, CSM_ERR_SAMPLE,
      'No device logits: call SetDeviceLogits before Generate', []);
    Exit;
  end;
  if not FSampler.Sample(FDevLogits, G4S_DTYPE_F32, PG4SParams(@AParams), Result) then
    Result := -1;
end;

procedure TModel.SetDeviceLogits(const ADevLogits: Pointer);
begin
  FDevLogits := ADevLogits;
end;

"""

EDITS = [
    Edit("uses",
         r"(?P<head>\n  Gemma4\.Vulkan,\n  Gemma4\.Compute);",
         "\\g<head>,\n  Gemma4.Sampler;"),
    Edit("fields",
         r"(?P<line>\n    FLogits: TArray<Single>;[^\n]*)",
         "\\g<line>\n"
         "    FSampler: TGpuSampler;         // the GPU sampler (libgemma4_sampler.so)\n"
         "    FDevLogits: Pointer;           // HIP address of the logits row (SetDeviceLogits)"),
    Edit("setter declaration",
         r"(?P<line>\n    function Forward\(const ATokenId: Integer\): TArray<Single>;)",
         "\\g<line>\n"
         "    // HIP address of the logits buffer FGpuLogits, imported by the host;\n"
         "    // DoSample reads the logits there\n"
         "    procedure SetDeviceLogits(const ADevLogits: Pointer);"),
    Edit("open sampler",
         r"(?P<head>function TModel\.DoAllocateResidentGpuBuffers\(\): Boolean;.*?"
         r"\n  if not LOk then Exit;\n)",
         "\\g<head>"
         "\n"
         "  // the GPU sampler beside the logits buffer: its whole workspace is\n"
         "  // allocated here, once, never per token\n"
         "  FreeAndNil(FSampler);\n"
         "  FSampler := TGpuSampler.Create();\n"
         "  FSampler.SetErrors(GetErrors());\n"
         "  if not FSampler.Open(FConfig.VocabSize, 1, FConfig.FinalLogitSoftcapping) then\n"
         "    Exit;                                  // SM01 is in GetErrors()\n"),
    Edit("free sampler",
         r"(?P<head>procedure TModel\.DoFreeGpuBuffers\(\);\s*var\s*LI: Integer;\s*begin\n)",
         "\\g<head>"
         "  FreeAndNil(FSampler);                    // before any early exit below\n"
         "  FDevLogits := nil;\n"),
    Edit("decode readback",
         r"\n  // --- Phase: download \(logits readback\) ---\n.*?"
         r"DownloadFromBuffer\(FGpuLogits, @FLogits\[0\],.*?"
         r"FProfDownloadMs := FProfDownloadMs \+ LSw\.Elapsed\.TotalMilliseconds;\n",
         "\n  // the logits stay on the GPU: DoSample reads them at FDevLogits\n"),
    Edit("prefill readback",
         r"\n  if AIsLast then\n    FComputeKernels\.Device\.DownloadFromBuffer\(FGpuLogits, "
         r"@FLogits\[0\],\n[^\n]*\n",
         "\n  // the last chunk's logits stay on the GPU for DoSample\n"),
    Edit("forward result",
         r"(?P<call>\n    DoForwardGpu\(ATokenId\);)\n    Exit\(Copy\(FLogits\)\);",
         "\\g<call>\n    Exit(nil);                             // the logits stay on the GPU"),
    Edit("do sample",
         r"function TModel\.DoSample\(const AParams: TSamplingParams\): Integer;\n.*?"
         r"\nend;\n\n(?=function TModel\.Generate\()",
         DO_SAMPLE.replace("\\", "\\\\")),
    Edit("generate guard",
         r"(?P<ind>\n      )LResult\.Add\(LTokenId\);",
         "\\g<ind>if LTokenId < 0 then"
         "\\g<ind>  Break;                               // the sampler failed: see GetErrors()"
         "\\g<ind>LResult.Add(LTokenId);"),
]


def apply(text):
    """The engine's Gemma4.Model.pas text with every edit applied, in order."""
    for e in EDITS:
        text = e.apply(text)
    return text


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("model_pas", help="the engine's src/Gemma4.Model.pas")
    ap.add_argument("-o", "--output", help="where to write the edited unit (default: stdout)")
    a = ap.parse_args(argv)
    with open(a.model_pas, "rb") as f:
        raw = f.read()
    bom = raw.startswith(b"\xef\xbb\xbf")
    src = raw.decode("utf-8-sig")
    crlf = "\r\n" in src
    out = apply(src.replace("\r\n", "\n"))
    if crlf:
        out = out.replace("\n", "\r\n")
    if a.output:
        with open(a.output, "w", encoding="utf-8-sig" if bom else "utf-8", newline="") as f:
            f.write(out)
    else:
        sys.stdout.write(out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
