{===============================================================================
  Gemma4.Sampler - binding of libgemma4_sampler.so, the MI355X (gfx950) token
  sampler, for the Gemma4.pas engine (Delphi Linux64, or FPC in Delphi mode).

  The library replaces TModel.DoSample and its helpers
  (src/Gemma4.Model.pas:2615-2827, src/Gemma4.Tensors.pas:638-673,
  src/Gemma4.Layers.pas:300-316) on logits that stay in GPU memory.  Every
  external below is one export of include/gemma4_sampler.h, with the same
  argument order and the same C types: arrays and out-values are typed
  pointers (PG4SParams, PDouble, PInteger, ...), passed by value, so nothing
  depends on how a compiler passes `const` or `var` records.

  TGpuSampler wraps one handle the way the engine wraps its GPU objects: a
  failing call adds an esError entry to GetErrors() with a unit code
  CSM_ERR_* and the library's message (StdApp.Base.pas TErrors.Add), and
  returns False.
===============================================================================}

unit Gemma4.Sampler;

{$IFDEF FPC}{$MODE DELPHI}{$ENDIF}

interface

uses
  SysUtils,
  StdApp.Base;

const
  CG4SLib = 'libgemma4_sampler.so';

  CSM_ERR_CREATE = 'SM01';
  CSM_ERR_SAMPLE = 'SM02';
  CSM_ERR_LMHEAD = 'SM03';
  CSM_ERR_STORE = 'SM04';

  G4S_ABI_VERSION = 1;

  // g4s_status
  G4S_OK = 0;
  G4S_ERR_INVALID_ARGUMENT = -1;
  G4S_ERR_UNSUPPORTED = -2;
  G4S_ERR_NO_DEVICE = -3;
  G4S_ERR_OUT_OF_MEMORY = -4;
  G4S_ERR_HIP = -5;
  G4S_ERR_EMPTY_ROW = -6;
  G4S_ERR_IO = -7;
  G4S_ERR_FORMAT = -8;
  G4S_ERR_NOT_FOUND = -9;
  G4S_ERR_ABORTED = -10;

  // IsEosToken (src/Gemma4.Types.pas:65-67)
  G4S_EOS_TOKEN_1 = 1;
  G4S_EOS_TOKEN_2 = 106;
  G4S_EOS_TOKEN_3 = 50;

  // g4s_dtype
  G4S_DTYPE_F32 = 0;
  G4S_DTYPE_BF16 = 1;

  // per-row flags (TG4SOutputs.Flags)
  G4S_FLAG_TOPK_PATH = $1;
  G4S_FLAG_FULL_PATH = $2;
  G4S_FLAG_DREW = $4;
  G4S_FLAG_REACHED = $8;
  G4S_FLAG_TIE_LOWEST = $10;
  G4S_FLAG_HEAP_REPLAY = $20;
  G4S_FLAG_CHUNK_EXACT = $40;
  G4S_FLAG_WIDE_MERGE = $80;
  G4S_FLAG_WIDE_K = $100;
  G4S_FLAG_ROW_RECOMPUTED = $200;
  G4S_FLAG_EMPTY = $40000000;
  G4S_FLAG_ERROR = $80000000;

  // g4s_wdtype: TDtypeKind (src/Gemma4.Types.pas:94-100), same order
  G4S_WDTYPE_UNKNOWN = 0;
  G4S_WDTYPE_BF16 = 1;
  G4S_WDTYPE_F16 = 2;
  G4S_WDTYPE_F32 = 3;
  G4S_WDTYPE_Q4_0 = 4;
  G4S_MAX_DIMS = 8;

  // device layouts of a Q4_0 matrix
  G4S_Q4_LAYOUT_ROWS = 0;
  G4S_Q4_LAYOUT_TILED64 = 1;

  // g4s_sample_topk_noalloc: rows per call and bytes of its device array
  G4S_NOALLOC_MAX_ROWS = 32;
  G4S_NOALLOC_SCRATCH_BYTES = 8602880;

type
  { PG4SSampler }
  // opaque g4s_sampler*
  PG4SSampler = Pointer;
  PPG4SSampler = ^PG4SSampler;

  { TG4SParams }
  // g4s_params: the field order, types and meaning of TSamplingParams
  // (src/Gemma4.Model.pas:70-76), so @AParams of the engine's record is a
  // valid PG4SParams.
  TG4SParams = record
    Temperature: Single;
    TopK: Integer;
    TopP: Single;
    RepetitionPenalty: Single;
  end;
  PG4SParams = ^TG4SParams;

  { TG4SOutputs }
  // g4s_outputs: optional per-row outputs; every pointer is GPU memory and
  // may be nil
  TG4SOutputs = record
    Count: PInteger;
    Indices: PInteger;
    Probs: PSingle;
    Capacity: Integer;
    Argmax: PInteger;
    LSum: PSingle;
    Flags: PCardinal;
  end;
  PG4SOutputs = ^TG4SOutputs;

  { PG4SStore }
  // opaque g4s_store*
  PG4SStore = Pointer;
  PPG4SStore = ^PG4SStore;

  { TG4STensorInfo }
  // g4s_tensor_info: TTensorInfo (src/Gemma4.Types.pas:119-129) without the
  // name, with the shape in a fixed array
  TG4STensorInfo = record
    SourceDtype: Integer;
    OutputDtype: Integer;
    Offset: UInt64;
    Size: UInt64;
    NDim: Integer;
    Shape: array[0..G4S_MAX_DIMS - 1] of Integer;
  end;
  PG4STensorInfo = ^TG4STensorInfo;

  // g4s_generate callbacks (cdecl): the caller's Forward, System.Random per
  // sequence, and Generate's ACallback per sequence
  TG4SForwardFn = function(AUser: Pointer; ATokens: PInteger; ABatch: Integer): Integer; cdecl;
  TG4SRandomFn = function(AUser: Pointer; ASeq: Integer): Double; cdecl;
  TG4STokenFn = function(AUser: Pointer; ASeq: Integer; AToken: Integer): Integer; cdecl;

function g4s_version(): PAnsiChar; cdecl; external CG4SLib;
procedure g4s_params_set_defaults(AParams: PG4SParams); cdecl; external CG4SLib;
function g4s_max_top_k(): Integer; cdecl; external CG4SLib;
function g4s_create(AOut: PPG4SSampler; AVocab: Integer; AMaxBatch: Integer;
  ASoftcap: Single; AHipStream: Pointer): Integer; cdecl; external CG4SLib;
function g4s_destroy(ASampler: PG4SSampler): Integer; cdecl; external CG4SLib;
function g4s_last_error(ASampler: PG4SSampler): PAnsiChar; cdecl; external CG4SLib;
function g4s_sample(ASampler: PG4SSampler; ADevLogits: Pointer; ADType: Integer;
  ARowStride: Int64; ABatch: Integer; AParams: PG4SParams; AU: PDouble;
  AIds: PInteger): Integer; cdecl; external CG4SLib;
function g4s_sample_ex(ASampler: PG4SSampler; ADevLogits: Pointer; ADType: Integer;
  ARowStride: Int64; ABatch: Integer; AParams: PG4SParams; AU: PDouble;
  AIds: PInteger; AOutputs: PG4SOutputs): Integer; cdecl; external CG4SLib;
function g4s_sample_async(ASampler: PG4SSampler; ADevLogits: Pointer; ADType: Integer;
  ARowStride: Int64; ABatch: Integer; ADevParams: PG4SParams; ADevU: PDouble;
  AKBound: Integer; AFullRows: Integer; ADevIds: PInteger;
  AOutputs: PG4SOutputs): Integer; cdecl; external CG4SLib;
function g4s_sample_graph(ASampler: PG4SSampler; ADevLogits: Pointer; ADType: Integer;
  ARowStride: Int64; ABatch: Integer; ADevParams: PG4SParams; ADevU: PDouble;
  AKBound: Integer; AFullRows: Integer; ADevIds: PInteger;
  AOutputs: PG4SOutputs): Integer; cdecl; external CG4SLib;
// no counterpart in the engine: for callers that cannot allocate GPU memory
// (graph capture, serving loops); no handle, errors via g4s_last_error(nil)
function g4s_sample_topk_noalloc(ADevLogits: Pointer; ADType: Integer; AVocab: Integer;
  ARowStride: Int64; ABatch: Integer; ADevParams: PG4SParams; ADevU: PDouble;
  AKBound: Integer; ASoftcap: Single; ADevIds: PInteger; AOutputs: PG4SOutputs;
  AHipStream: Pointer): Integer; cdecl; external CG4SLib;
function g4s_lmhead_q4_0(ASampler: PG4SSampler; ADevWeights: Pointer; ARows: Integer;
  ACols: Integer; ADevHidden: PSingle; ABatch: Integer; ADevLogits: PSingle;
  ALogitsStride: Int64): Integer; cdecl; external CG4SLib;
function g4s_lmhead_q4_0_tiled(ASampler: PG4SSampler; ADevTiles: Pointer; ARows: Integer;
  ACols: Integer; ADevHidden: PSingle; ABatch: Integer; ADevLogits: PSingle;
  ALogitsStride: Int64): Integer; cdecl; external CG4SLib;
function g4s_lmhead_sample_q4_0(ASampler: PG4SSampler; ADevTiles: Pointer; ACols: Integer;
  ADevHidden: PSingle; ABatch: Integer; ADevLogits: PSingle; ALogitsStride: Int64;
  AParams: PG4SParams; AU: PDouble; AIds: PInteger;
  AOutputs: PG4SOutputs): Integer; cdecl; external CG4SLib;
function g4s_embed_q4_0(ASampler: PG4SSampler; ADevWeights: Pointer; ARows: Integer;
  ACols: Integer; ADevTokens: PInteger; ABatch: Integer; AScale: Single;
  ADevHidden: PSingle): Integer; cdecl; external CG4SLib;
function g4s_generate(ASampler: PG4SSampler; ABatch: Integer; AParams: PG4SParams;
  AMaxTokens: Integer; ADevLogits: Pointer; ADType: Integer; ARowStride: Int64;
  AForward: TG4SForwardFn; ARandom: TG4SRandomFn; AOnToken: TG4STokenFn; AUser: Pointer;
  ATokens: PInteger; ALengths: PInteger): Integer; cdecl; external CG4SLib;
function g4s_store_open(AOut: PPG4SStore; AVpkPath: PAnsiChar; AManifestPath: PAnsiChar;
  AWeightsPath: PAnsiChar): Integer; cdecl; external CG4SLib;
function g4s_store_close(AStore: PG4SStore): Integer; cdecl; external CG4SLib;
function g4s_store_last_error(AStore: PG4SStore): PAnsiChar; cdecl; external CG4SLib;
function g4s_store_tensor_count(AStore: PG4SStore): Integer; cdecl; external CG4SLib;
function g4s_store_tensor_info(AStore: PG4SStore; AIndex: Integer; AInfo: PG4STensorInfo;
  AName: PAnsiChar; ANameCapacity: Integer): Integer; cdecl; external CG4SLib;
function g4s_store_find_tensor(AStore: PG4SStore; AName: PAnsiChar;
  AInfo: PG4STensorInfo): Integer; cdecl; external CG4SLib;
function g4s_store_raw_pointer(AStore: PG4SStore; AName: PAnsiChar): Pointer; cdecl;
  external CG4SLib;
function g4s_store_verify(AStore: PG4SStore): Integer; cdecl; external CG4SLib;
function g4s_q4_0_device_bytes(ARows: Integer; ACols: Integer; ALayout: Integer): Int64; cdecl;
  external CG4SLib;
function g4s_store_upload_q4_0(AStore: PG4SStore; AName: PAnsiChar; ALayout: Integer;
  ADevDst: Pointer; ADstBytes: UInt64; AHipStream: Pointer): Integer; cdecl; external CG4SLib;
function g4s_q4_0_repack(ADevRows: Pointer; ARows: Integer; ACols: Integer;
  ADevTiled: Pointer; AHipStream: Pointer): Integer; cdecl; external CG4SLib;

type
  { TGpuSampler }
  // One sampler handle of a model: opened next to the GPU logits buffer
  // (Model.pas:791-792) and closed with it (Model.pas:701-702).
  TGpuSampler = class(TBaseObject)
  private
    FHandle: PG4SSampler;
    FVocab: Integer;
    FMaxBatch: Integer;
    function Fail(const ACode: string; const AStatus: Integer): Boolean;
  public
    destructor Destroy(); override;

    // g4s_create: the whole workspace is allocated here, never per call
    function Open(const AVocab: Integer; const AMaxBatch: Integer;
      const ASoftcap: Single; const AHipStream: Pointer = nil): Boolean;
    procedure Close();

    // DoSample on one GPU-resident logits row: u is the engine's Random, as
    // at Model.pas:2726,2813, drawn only when AParams^.Temperature > 0 (a
    // greedy row consumes no Random, as in the reference).  False (and
    // ATokenId = -1) on failure.
    function Sample(const ADevLogits: Pointer; const ADType: Integer;
      const AParams: PG4SParams; out ATokenId: Integer): Boolean;

    // ABatch rows at ADevLogits + i*ARowStride elements; AParams, AU and
    // AIds point at ABatch host entries each.  AU[i] is read only for rows
    // with Temperature > 0: a caller reproducing the reference fills it
    // with Random for those rows alone, in row order, and leaves the greedy
    // rows' entries unread (any value in [0, 1)).
    function SampleBatch(const ADevLogits: Pointer; const ADType: Integer;
      const ARowStride: Int64; const ABatch: Integer; const AParams: PG4SParams;
      const AU: PDouble; const AIds: PInteger): Boolean;

    // Q4_0 LM head straight into the buffer the sampler reads
    function LmHeadQ4_0(const ADevWeights: Pointer; const ARows: Integer;
      const ACols: Integer; const ADevHidden: PSingle; const ABatch: Integer;
      const ADevLogits: PSingle; const ALogitsStride: Int64): Boolean;

    // The tied LM head (TILED64 weights from TGpuWeightStore.UploadQ4_0)
    // fused with the sampler: Forward's last projection + DoSample for
    // ABatch hidden vectors (Model.pas:1285-1300,2739-2827); ADevLogits = nil
    // writes no logits (top-k rows with 0 < TopK <= g4s_max_top_k only)
    function LmHeadSampleQ4_0(const ADevTiles: Pointer; const ACols: Integer;
      const ADevHidden: PSingle; const ABatch: Integer; const ADevLogits: PSingle;
      const AParams: PG4SParams; const AU: PDouble; const AIds: PInteger): Boolean;

    function LastError(): string;

    property Handle: PG4SSampler read FHandle;
    property Vocab: Integer read FVocab;
    property MaxBatch: Integer read FMaxBatch;
  end;

  { TGpuWeightStore }
  // TWeightStore (src/Gemma4.Tensors.pas:321-516) on the library: the VPK
  // archive's manifest and the GPU upload of a Q4_0 tensor.
  TGpuWeightStore = class(TBaseObject)
  private
    FHandle: PG4SStore;
    function Fail(const AStatus: Integer): Boolean;
  public
    destructor Destroy(); override;
    // AManifestPath / AWeightsPath empty: the engine's E4B/ paths
    function Open(const AVpkPath: string; const AManifestPath: string = '';
      const AWeightsPath: string = ''): Boolean;
    procedure Close();
    function IsOpen(): Boolean;
    function TensorCount(): Integer;
    function FindTensor(const AName: string; out AInfo: TG4STensorInfo): Boolean;
    // into ADevDst (ADstBytes >= g4s_q4_0_device_bytes(rows, cols, ALayout))
    function UploadQ4_0(const AName: string; const ALayout: Integer;
      const ADevDst: Pointer; const ADstBytes: UInt64;
      const AHipStream: Pointer = nil): Boolean;
    function LastError(): string;
  end;

implementation

{ TGpuSampler }

destructor TGpuSampler.Destroy();
begin
  Close();
  inherited;
end;

function TGpuSampler.LastError(): string;
begin
  Result := string(AnsiString(g4s_last_error(FHandle)));
end;

function TGpuSampler.Fail(const ACode: string; const AStatus: Integer): Boolean;
begin
  GetErrors().Add(esError, ACode, 'Sampler status %d: %s', [AStatus, LastError()]);
  Result := False;
end;

function TGpuSampler.Open(const AVocab: Integer; const AMaxBatch: Integer;
  const ASoftcap: Single; const AHipStream: Pointer): Boolean;
var
  LStatus: Integer;
  LHandle: PG4SSampler;
begin
  Close();
  LHandle := nil;
  LStatus := g4s_create(@LHandle, AVocab, AMaxBatch, ASoftcap, AHipStream);
  if LStatus <> G4S_OK then
  begin
    // g4s_last_error(nil) holds the message of the failed create
    FHandle := nil;
    Exit(Fail(CSM_ERR_CREATE, LStatus));
  end;
  FHandle := LHandle;
  FVocab := AVocab;
  FMaxBatch := AMaxBatch;
  Result := True;
end;

procedure TGpuSampler.Close();
begin
  if FHandle <> nil then
  begin
    g4s_destroy(FHandle);
    FHandle := nil;
  end;
end;

function TGpuSampler.Sample(const ADevLogits: Pointer; const ADType: Integer;
  const AParams: PG4SParams; out ATokenId: Integer): Boolean;
var
  LU: Double;
  LId: Integer;
  LStatus: Integer;
begin
  ATokenId := -1;
  // System.Random is drawn only when the row draws, as DoSample does on
  // both of its paths (Model.pas:2723-2726, 2811-2813): a greedy call
  // (Temperature <= 0) leaves RandSeed where the reference leaves it.
  if AParams^.Temperature > 0.0 then
    LU := Random
  else
    LU := 0.0;
  LId := -1;
  LStatus := g4s_sample(FHandle, ADevLogits, ADType, FVocab, 1, AParams, @LU, @LId);
  if LStatus <> G4S_OK then
    Exit(Fail(CSM_ERR_SAMPLE, LStatus));
  ATokenId := LId;
  Result := True;
end;

function TGpuSampler.SampleBatch(const ADevLogits: Pointer; const ADType: Integer;
  const ARowStride: Int64; const ABatch: Integer; const AParams: PG4SParams;
  const AU: PDouble; const AIds: PInteger): Boolean;
var
  LStatus: Integer;
begin
  LStatus := g4s_sample(FHandle, ADevLogits, ADType, ARowStride, ABatch, AParams, AU, AIds);
  if LStatus <> G4S_OK then
    Exit(Fail(CSM_ERR_SAMPLE, LStatus));
  Result := True;
end;

function TGpuSampler.LmHeadQ4_0(const ADevWeights: Pointer; const ARows: Integer;
  const ACols: Integer; const ADevHidden: PSingle; const ABatch: Integer;
  const ADevLogits: PSingle; const ALogitsStride: Int64): Boolean;
var
  LStatus: Integer;
begin
  LStatus := g4s_lmhead_q4_0(FHandle, ADevWeights, ARows, ACols, ADevHidden, ABatch,
    ADevLogits, ALogitsStride);
  if LStatus <> G4S_OK then
    Exit(Fail(CSM_ERR_LMHEAD, LStatus));
  Result := True;
end;

function TGpuSampler.LmHeadSampleQ4_0(const ADevTiles: Pointer; const ACols: Integer;
  const ADevHidden: PSingle; const ABatch: Integer; const ADevLogits: PSingle;
  const AParams: PG4SParams; const AU: PDouble; const AIds: PInteger): Boolean;
var
  LStatus: Integer;
begin
  LStatus := g4s_lmhead_sample_q4_0(FHandle, ADevTiles, ACols, ADevHidden, ABatch, ADevLogits,
    FVocab, AParams, AU, AIds, nil);
  if LStatus <> G4S_OK then
    Exit(Fail(CSM_ERR_LMHEAD, LStatus));
  Result := True;
end;

{ TGpuWeightStore }

destructor TGpuWeightStore.Destroy();
begin
  Close();
  inherited;
end;

function TGpuWeightStore.LastError(): string;
begin
  Result := string(AnsiString(g4s_store_last_error(FHandle)));
end;

function TGpuWeightStore.Fail(const AStatus: Integer): Boolean;
begin
  GetErrors().Add(esError, CSM_ERR_STORE, 'Weight store status %d: %s', [AStatus, LastError()]);
  Result := False;
end;

function TGpuWeightStore.Open(const AVpkPath: string; const AManifestPath: string;
  const AWeightsPath: string): Boolean;
var
  LStatus: Integer;
  LHandle: PG4SStore;
  LPath, LManifest, LWeights: UTF8String;
  LPManifest, LPWeights: PAnsiChar;
begin
  Close();
  LHandle := nil;
  LPath := UTF8String(AVpkPath);
  LManifest := UTF8String(AManifestPath);
  LWeights := UTF8String(AWeightsPath);
  LPManifest := nil;
  LPWeights := nil;
  if AManifestPath <> '' then LPManifest := PAnsiChar(LManifest);
  if AWeightsPath <> '' then LPWeights := PAnsiChar(LWeights);
  LStatus := g4s_store_open(@LHandle, PAnsiChar(LPath), LPManifest, LPWeights);
  if LStatus <> G4S_OK then
  begin
    // g4s_store_last_error(nil) holds the message of the failed open
    FHandle := nil;
    Exit(Fail(LStatus));
  end;
  FHandle := LHandle;
  Result := True;
end;

procedure TGpuWeightStore.Close();
begin
  if FHandle <> nil then
  begin
    g4s_store_close(FHandle);
    FHandle := nil;
  end;
end;

function TGpuWeightStore.IsOpen(): Boolean;
begin
  Result := FHandle <> nil;
end;

function TGpuWeightStore.TensorCount(): Integer;
begin
  Result := g4s_store_tensor_count(FHandle);
end;

function TGpuWeightStore.FindTensor(const AName: string; out AInfo: TG4STensorInfo): Boolean;
var
  LName: UTF8String;
begin
  LName := UTF8String(AName);
  Result := g4s_store_find_tensor(FHandle, PAnsiChar(LName), @AInfo) = G4S_OK;
end;

function TGpuWeightStore.UploadQ4_0(const AName: string; const ALayout: Integer;
  const ADevDst: Pointer; const ADstBytes: UInt64; const AHipStream: Pointer): Boolean;
var
  LStatus: Integer;
  LName: UTF8String;
begin
  LName := UTF8String(AName);
  LStatus := g4s_store_upload_q4_0(FHandle, PAnsiChar(LName), ALayout, ADevDst, ADstBytes,
    AHipStream);
  if LStatus <> G4S_OK then
    Exit(Fail(LStatus));
  Result := True;
end;

end.
