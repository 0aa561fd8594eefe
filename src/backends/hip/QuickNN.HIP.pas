unit QuickNN.HIP;

{ MI355X (gfx950) backend for QuickNN's LLM decode path.

  A thin Object Pascal binding of libqnn_hip.so (include/qnn_hip.h, cdecl C
  ABI).  TQNNHIPContext has the method names, argument meaning and exception
  classes of the Vulkan resident context TQNNGPUContext
  (src/backends/vulkan/QuickNN.Vulkan.Context.API.inc:14-165), so the model
  units switch backends by the type of the context they create.

  The library enforces the reference's rules itself: one context at a time,
  bound to the creating thread; asynchronous recording, with Download and
  Flush waiting.  This unit only converts TMemoryBlock descriptors, maps status
  codes to exceptions, and keeps the WeightIdentity interfaces that
  OnWeightEvicted hands back.

  Methods of TQNNGPUContext that this backend does not provide raise
  ENotSupportedException: Attention (uncached), CopyCHWRect, and ConvRot
  weights (Rotation <> 0). }

interface

uses
  System.SysUtils, System.Math, System.Generics.Collections, QuickNN.Common;

const
{$IFDEF MSWINDOWS}
  QNN_LIB = 'qnn_hip.dll';
{$ELSE}
  QNN_LIB = 'libqnn_hip.so';
{$ENDIF}

  // Status codes (include/qnn_hip.h).
  QNN_OK = 0;
  QNN_NOT_HANDLED = 1;
  QNN_NOT_FOUND = 2;
  QNN_E_ARGUMENT = -1;
  QNN_E_RANGE = -2;
  QNN_E_NOT_SUPPORTED = -3;
  QNN_E_INVALID_OP = -4;
  QNN_E_FORMAT = -5;
  QNN_E_IO = -6;

  // TLLMInt4Scope ordinals for qnn_int4_cache_create.
  QNN_IQ_EXPERTS = 0;
  QNN_IQ_DENSE = 1;

  // Kernel op codes (Context.API.inc:167-258): the numbering is the op-code
  // ABI both backends share.  The HIP backend runs
  // GO_FILL, GO_NORM, GO_ADD, GO_SWIGLU, GO_FINITE, GO_SCALE, GO_LLM_CACHE_WRITE, GO_LLM_ROPE, GO_LLM_SEEN, GO_MOE_ROUTE, GO_MOE_GATHER, GO_MOE_SCATTER, GO_GEGLU, GO_SOFTCAP;
  // Kernel / KernelWeights with any other code raise ENotSupportedException.
  GO_FILL = 0; GO_CONV_ROT = 1; GO_NORM = 2; GO_UNARY = 3; GO_ADD = 4; GO_MOD_NORM = 5; GO_GATE_ADD = 6;
  GO_TEXT_ROPE = 7; GO_IMAGE_ROPE = 8; GO_SWIGLU = 9; GO_PACK_KV = 10; GO_SLICE = 11; GO_TIME = 12;
  GO_FINITE = 13; GO_CFG = 14; GO_GATHER = 15; GO_VISION_PATCH = 16; GO_VISION_POSITION = 17;
  GO_VISION_ROPE = 18; GO_PIXEL_INPUT = 19; GO_IM2COL = 20; GO_CONV_OUTPUT = 21; GO_LATENT_CHW = 22;
  GO_LATENT_NORMALIZE = 23; GO_NEAREST = 24; GO_UP_RESIDUAL = 25; GO_DOWN_RESIDUAL = 26; GO_PIXEL_OUTPUT = 27;
  GO_CHW_TO_ROWS = 28; GO_ROWS_TO_CHW = 29; GO_GROUP_NORM = 30; GO_AFFINE = 31; GO_ROTARY_CACHE = 32;
  GO_SINUSOIDAL = 33; GO_PATCH = 34; GO_LATENT_BN = 35; GO_PAD_END = 36; GO_RGB_OUTPUT = 37; GO_PAD_WEIGHT = 38;
  GO_SCATTER = 39; GO_ZI_ROPE = 40; GO_ZI_POSITION = 41; GO_FLUX_ROPE = 42; GO_SCALE = 43; GO_LLM_CACHE_WRITE = 44;
  GO_LLM_ROPE = 45; GO_LLM_SAMPLE = 46; GO_LLM_MATVEC = 47; GO_LLM_SEEN = 48; GO_LLM_MATVEC_BF16 = 49;
  GO_LLM_TOPK_TILE = 50; GO_LLM_TOPK_MERGE = 51; GO_MOE_ROUTE = 52; GO_MOE_GATHER = 53; GO_MOE_SCATTER = 54;
  GO_MOE_INT4_MATVEC = 55; GO_MOE_INT4_GEMM = 56; GO_HYBRID_INT4_GATHER = 57; GO_HYBRID_CONV_SCAN = 58;
  GO_HYBRID_QK_L2 = 59; GO_HYBRID_DELTA_GATES = 60; GO_HYBRID_DELTA_SCAN = 61; GO_HYBRID_GATED_NORM = 62;
  GO_HYBRID_ATTN_GATE = 63; GO_HYBRID_ROPE = 64; GO_GGUF_MATVEC = 65; GO_LLM_SWIGLU_VECTOR = 66;
  GO_GGUF_SWIGLU_VECTOR = 67; GO_INT4_SWIGLU_VECTOR = 68; GO_MOE_INT4_ACCUMULATE = 69; GO_CHW_RECT = 70;
  GO_GROUP_NORM_STATS = 71; GO_NORMALIZED_IM2COL = 72; GO_FLUX1_ROPE = 73; GO_T5_POSITION_BIAS = 74;
  GO_GEGLU = 75; GO_SOFTCAP = 76; GO_FLASH_GROUP_NORM = 77; GO_FLASH_HC_INIT = 78; GO_FLASH_HC_MIX = 79;
  GO_FLASH_HC_COMBINE = 80; GO_FLASH_PLE_GATE = 81; GO_FLASH_PLE_CONV = 82; GO_FLASH_QSA_POOL = 83;
  GO_FLASH_QSA_SCORE = 84; GO_FLASH_QSA_MASK = 85; GO_FLASH_SHARED_GATE = 86;

type
  EQNNHIPFormatError = class(Exception);   // ESafeTensorError / EGGUFError raised by the library's loaders

  // TMemoryBlock as it crosses the boundary (QuickNN.Common.pas:135-155).
  TQnnWeight = record
    Identity: UInt64;   // WeightIdentity as a key: non-zero, equal for the same immutable bytes
    Data: Pointer;      // DataPtr: element 0, before Offset
    Offset: Int64;
    Size: Int64;
    Shape0: Int64;
    Shape1: Int64;
    DataType: Int32;    // Ord(TQNNDataType)
    Encoding: Int32;    // Ord(TQNNWeightEncoding)
  end;
  PQnnWeight = ^TQnnWeight;

  // TQNNGPUStatus counters plus the HIP backend's own (QuickNN.Vulkan.pas:17-29).
  TQnnStatus = record
    GemmCalls, GGUFCalls, Int4Calls, MoECalls: UInt64;
    WeightUploads, WeightUploadBytes, WeightCacheHits, WeightCacheMisses, WeightEvictions: UInt64;
    Readbacks, Submissions: UInt64;
    WeightBytes, WeightLimit, ActivationBytes, ActivationPeakBytes: UInt64;
    MLPFused, LinearGrouped, MoEFused, MoERouteFused, GLUFused: UInt64;
    AsyncWeightBatches, AsyncWeightBytes: UInt64;
    GemmH16: UInt64;
  end;

  TQnnWeightEvictedFn = procedure(Identity: UInt64; User: Pointer); cdecl;
  TQnnProgressFn = procedure(Done, Total: Integer; User: Pointer); cdecl;

  // TSafeTensor as the library's loaders report it.
  TQnnTensorInfo = record
    Name: PAnsiChar;
    Data: Pointer;
    Shape: PInt64;
    Identity: UInt64;
    DataOffset, DataSize: Int64;
    Ndim, StDType, DataType, Encoding, FileIndex: Int32;
    StorageType: UInt32;
  end;

  TQnnTensorFileInfo = record
    Path, Architecture, HeaderJson: PAnsiChar;
    Data: Pointer;
    FileSize, HeaderSize, DataSize, Offset: Int64;
    IsGGUF, TensorCount: Int32;
  end;

  TQnnGGUFHeaderInfo = record
    Version, Alignment: UInt32;
    DataOffset: Int64;
    VocabularySize, TensorCount: Int32;
    Architecture, MetadataJson: PAnsiChar;
  end;

  TQnnGGUFTensor = record
    Name: PAnsiChar;
    Shape: PInt64;
    Offset, ByteSize: Int64;
    Ndim: Int32;
    StorageType: UInt32;
    Encoding: Int32;
  end;

// ---- errors and context lifetime
function qnn_last_error(Buf: PAnsiChar; Len: Integer): Integer; cdecl; external QNN_LIB;
function qnn_ctx_create(Device: Integer; WeightCacheBytes: UInt64; out Ctx: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_ctx_destroy(Ctx: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_get_status(Ctx: Pointer; out Status: TQnnStatus): Integer; cdecl; external QNN_LIB;
function qnn_reload_tuning: Integer; cdecl; external QNN_LIB;
function qnn_phase_trace(Ctx: Pointer; Dst: PUInt64; Count: UInt64; out Copied: UInt64): Integer; cdecl; external QNN_LIB;
function qnn_stream_read(Ctx: Pointer; Src: Pointer; Count: Integer; Dst: Pointer): Integer; cdecl; external QNN_LIB;
// ---- resident tensors
function qnn_tensor_new(Ctx: Pointer; Count: Integer; out T: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_recycle(Ctx: Pointer; var T: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_scratch(Ctx: Pointer; Slot, Count: Integer; out T: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_upload_raw(Ctx: Pointer; Data: Pointer; Count: Integer; out T: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_upload(Ctx: Pointer; W: PQnnWeight; out T: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_download(Ctx, T: Pointer; Dst: Pointer; Count: Integer): Integer; cdecl; external QNN_LIB;
function qnn_copy(Ctx, Dst, Src: Pointer; Count, DstOffset, SrcOffset: Integer): Integer; cdecl; external QNN_LIB;
function qnn_flush(Ctx: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_tensor_count(T: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_tensor_device_ptr(T: Pointer): Pointer; cdecl; external QNN_LIB;
// ---- weight residency and prefetch
function qnn_retain_weight(Ctx: Pointer; W: PQnnWeight; Rows, Cols: Integer): Integer; cdecl; external QNN_LIB;
function qnn_preload_weights(Ctx: Pointer; Ws: PQnnWeight; N: Integer; StagingLimit: UInt64): Integer; cdecl; external QNN_LIB;
function qnn_is_weight_resident(Ctx: Pointer; W: PQnnWeight; Rows, Cols: Integer; out Resident: Integer): Integer; cdecl; external QNN_LIB;
function qnn_weight_batch_capacity(Ctx: Pointer; out Bytes: UInt64): Integer; cdecl; external QNN_LIB;
function qnn_set_weight_evicted(Ctx: Pointer; Fn: TQnnWeightEvictedFn; User: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_enable_weight_prefetch(Ctx: Pointer; MaxLayerBytes: UInt64; out Enabled: Integer): Integer; cdecl; external QNN_LIB;
function qnn_begin_weight_prefetch(Ctx: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_prefetch_weights(Ctx: Pointer; Ws: PQnnWeight; N, DeferJoin: Integer): Integer; cdecl; external QNN_LIB;
function qnn_stage_weight_prefetch(Ctx: Pointer; Ws: PQnnWeight; N: Integer): Integer; cdecl; external QNN_LIB;
function qnn_complete_weight_prefetch(Ctx: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_activate_prefetched_weights(Ctx: Pointer; Ws: PQnnWeight; N: Integer; out Activated: Integer): Integer; cdecl; external QNN_LIB;
function qnn_seal_weight_prefetch(Ctx: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_end_weight_prefetch(Ctx: Pointer): Integer; cdecl; external QNN_LIB;
// ---- projections
function qnn_linear(Ctx, Dst, Src: Pointer; W, Scales, Bias: PQnnWeight; Rows, InDim, OutDim: Integer): Integer; cdecl; external QNN_LIB;
function qnn_q8_gemm_int8(Ctx, Dst, Src: Pointer; W: PQnnWeight; Rows, InDim, OutDim: Integer): Integer; cdecl; external QNN_LIB;
function qnn_vector_linear(Ctx, Dst, Src: Pointer; W: PQnnWeight; InDim, OutDim: Integer): Integer; cdecl; external QNN_LIB;
function qnn_int4_linear(Ctx, Dst, Src: Pointer; W: PQnnWeight; Rows, InDim, OutDim: Integer): Integer; cdecl; external QNN_LIB;
function qnn_int4_linear_noalloc(Ctx, Dst, Src: Pointer; W: PQnnWeight; Rows, InDim, OutDim: Integer): Integer; cdecl; external QNN_LIB;
function qnn_swiglu_vector(Ctx, Dst, Src: Pointer; Gate, Up: PQnnWeight; InDim, OutDim: Integer): Integer; cdecl; external QNN_LIB;
function qnn_int4_linear_accumulate(Ctx, Dst, Src, Probabilities: Pointer; W: PQnnWeight;
  InDim, OutDim, ProbIndex: Integer): Integer; cdecl; external QNN_LIB;
// ---- element-wise ops, the rest of the decode layer
function qnn_kernel(Ctx: Pointer; Op, N: Integer; Dst, A, B, C: Pointer; Args: PInteger; NArgs: Integer): Integer; cdecl; external QNN_LIB;
function qnn_kernel_weights(Ctx: Pointer; Op, N: Integer; Dst, A: Pointer; B, C: PQnnWeight;
  Args: PInteger; NArgs: Integer): Integer; cdecl; external QNN_LIB;
function qnn_gather(Ctx, Dst, Ids: Pointer; W, Scales: PQnnWeight; Rows, Dim, Vocab, Rotation: Integer): Integer; cdecl; external QNN_LIB;
function qnn_cached_attention(Ctx, Dst, Q, Cache: Pointer; QueryRows, Capacity, Heads, KvHeads, Dim, Position,
  Window: Integer; Softcap, Scale: Single; Masked: Integer): Integer; cdecl; external QNN_LIB;
function qnn_sample_token(Ctx, Dst, Logits, Seen: Pointer; Vocab, TopK: Integer;
  Temperature, TopP, Penalty, Uniform: Single): Integer; cdecl; external QNN_LIB;
function qnn_check_finite(Ctx, T: Pointer; Count: Integer): Integer; cdecl; external QNN_LIB;
// ---- routed experts on the device
function qnn_expert_set_create(Ctx: Pointer; Gate, Up, Down: PQnnWeight; Experts, Hidden, Inter: Integer;
  out ExpertSet: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_expert_set_destroy(Ctx, ExpertSet: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_moe_experts(Ctx, ExpertSet, Dst, Src, Routes: Pointer; Rows, TopK: Integer): Integer; cdecl; external QNN_LIB;
// ---- diagnostics
function qnn_dequantize(Ctx, Dst: Pointer; W: PQnnWeight; Rows, Cols: Integer): Integer; cdecl; external QNN_LIB;
function qnn_event_record(Ctx: Pointer; Slot: Integer): Integer; cdecl; external QNN_LIB;
function qnn_event_elapsed_ms(Ctx: Pointer; SlotBegin, SlotEnd: Integer; out Ms: Single): Integer; cdecl; external QNN_LIB;
function qnn_graph_begin(Ctx: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_graph_end(Ctx: Pointer; out GraphId: Integer): Integer; cdecl; external QNN_LIB;
function qnn_graph_launch(Ctx: Pointer; GraphId: Integer): Integer; cdecl; external QNN_LIB;
function qnn_stream(Ctx: Pointer): Pointer; cdecl; external QNN_LIB;
// ---- checkpoint files (for hosts without QuickNN.SafeTensors; the Pascal
//      engine keeps its own readers and passes their TMemoryBlocks instead)
function qnn_tensor_files_open(Path: PAnsiChar; out Files: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_tensor_files_open_shards(Dir, IndexFile, SingleFile: PAnsiChar; out Files: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_tensor_files_close(Files: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_tensor_files_count(Files: Pointer; out Count: Integer): Integer; cdecl; external QNN_LIB;
function qnn_tensor_files_file(Files: Pointer; FileIndex: Integer; out Info: TQnnTensorFileInfo): Integer; cdecl; external QNN_LIB;
function qnn_tensor_files_tensor(Files: Pointer; FileIndex, Index: Integer; out Info: TQnnTensorInfo): Integer; cdecl; external QNN_LIB;
function qnn_tensor_files_find(Files: Pointer; Name: PAnsiChar; out Info: TQnnTensorInfo): Integer; cdecl; external QNN_LIB;
function qnn_tensor_files_linear_weight(Files: Pointer; Name: PAnsiChar; out W: TQnnWeight): Integer; cdecl; external QNN_LIB;
function qnn_gguf_read_file(Path: PAnsiChar; WithMetadata, IncludeVocabulary: Integer; out Header: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_gguf_header_free(Header: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_gguf_header_get(Header: Pointer; out Info: TQnnGGUFHeaderInfo): Integer; cdecl; external QNN_LIB;
function qnn_gguf_header_tensor(Header: Pointer; Index: Integer; out Tensor: TQnnGGUFTensor): Integer; cdecl; external QNN_LIB;
function qnn_int4_cache_create(Sources: Pointer; Directory: PAnsiChar; Progress: TQnnProgressFn; User: Pointer;
  Scope: Integer; out Cache: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_int4_cache_destroy(Cache: Pointer): Integer; cdecl; external QNN_LIB;
function qnn_int4_cache_weight(Cache: Pointer; Name: PAnsiChar; Rows, Columns: Integer; out W: TQnnWeight): Integer; cdecl; external QNN_LIB;
function qnn_int4_cache_mapped_bytes(Cache: Pointer; out Bytes: UInt64): Integer; cdecl; external QNN_LIB;
function qnn_int4_cache_directory(Cache: Pointer): PAnsiChar; cdecl; external QNN_LIB;
function qnn_int4_source_fingerprint(Sources: Pointer; Out65: PAnsiChar): Integer; cdecl; external QNN_LIB;
// ---- host utilities
function qnn_int4_row_bytes(Cols: Integer): Integer; cdecl; external QNN_LIB;
function qnn_quantize_int4(Src: Pointer; DataType, Rows, Cols: Integer; Dst: PByte): Integer; cdecl; external QNN_LIB;
function qnn_gguf_quantize(Encoding: Integer; Src: PSingle; N: Int64; Dst: PByte): Integer; cdecl; external QNN_LIB;

type
  // TQNNGPUTensor: a context-owned fp32 device buffer of Count floats.
  TQNNHIPTensor = class
  private
    FHandle: Pointer;
  public
    Count: Integer;
    property Handle: Pointer read FHandle;
  end;

  TQNNHIPContext = class
  private
    FCtx: Pointer;
    FScratch: array[0..3] of TQNNHIPTensor;
    FOnWeightEvicted: TProc<IInterface>;
    // WeightIdentity interfaces the library may report back, by key.
    FIdentities: TDictionary<UInt64, IInterface>;
    procedure Check(const Status: Integer);
    function Wrap(const H: Pointer; const Count: Integer): TQNNHIPTensor;
    function Desc(const W: TMemoryBlock): TQnnWeight;
    function DescOrNil(const W: TMemoryBlock; out D: TQnnWeight): PQnnWeight;
    function Descs(const Weights: array of TMemoryBlock): TArray<TQnnWeight>;
    procedure SetOnWeightEvicted(const Value: TProc<IInterface>);
  public
    constructor Create(const Device: Integer = 0; const WeightCacheBytes: UInt64 = 0);
    destructor Destroy; override;
    function NewTensor(const Count: Integer): TQNNHIPTensor;
    procedure Recycle(var Tensor: TQNNHIPTensor);
    function Scratch(const Slot, Count: Integer): TQNNHIPTensor;
    procedure Flush;
    procedure RetainWeight(const Weight: TMemoryBlock; const Rows, Columns: Integer);
    procedure PreloadWeights(const Weights: array of TMemoryBlock; const StagingBytesLimit: UInt64 = 134217728);
    function EnableWeightPrefetch(const MaxLayerBytes: UInt64): Boolean;
    procedure BeginWeightPrefetch;
    procedure PrefetchWeights(const Weights: array of TMemoryBlock; const DeferJoin: Boolean = False);
    procedure StageWeightPrefetch(const Weights: array of TMemoryBlock);
    procedure CompleteWeightPrefetch;
    function ActivatePrefetchedWeights(const Weights: array of TMemoryBlock): Boolean;
    procedure SealWeightPrefetch;
    procedure EndWeightPrefetch;
    function WeightBatchCapacity: UInt64;
    function IsWeightResident(const Weight: TMemoryBlock; const Rows, Columns: Integer): Boolean;
    function Upload(const Data: TMemoryBlock): TQNNHIPTensor;
    function UploadRaw(const Data: Pointer; const Count: Integer): TQNNHIPTensor;
    procedure Download(const Tensor: TQNNHIPTensor; const Dst: Pointer; const Count: Integer = -1);
    procedure Copy(const Dst, Src: TQNNHIPTensor; const Count: Integer; const DstOffset: Integer = 0;
      const SrcOffset: Integer = 0);
    procedure CopyCHWRect(const Dst, Src: TQNNHIPTensor; const Channels, SrcWidth, SrcHeight, DstWidth, DstHeight,
      SrcX, SrcY, DstX, DstY, Width, Height: Integer);
    procedure Kernel(const Op, N: Integer; const Dst, A, B, C: TQNNHIPTensor; const Args: array of Integer);
    procedure KernelWeights(const Op, N: Integer; const Dst, A: TQNNHIPTensor; const B, C: TMemoryBlock;
      const Args: array of Integer);
    procedure Linear(const Dst, Src: TQNNHIPTensor; const Weight, Scales, Bias: TMemoryBlock;
      const Rows, InputDim, OutputDim: Integer; const Rotation: Integer = 0);
    procedure Attention(const Dst, Q, K, V: TQNNHIPTensor; const Rows, Heads, KvHeads, Dim, Causal: Integer;
      const Limits: TQNNHIPTensor = nil; const T5Bias: TQNNHIPTensor = nil);
    procedure VectorLinear(const Dst, Src: TQNNHIPTensor; const Weight: TMemoryBlock; const InputDim, OutputDim: Integer);
    function TrySwiGLUVector(const Dst, Src: TQNNHIPTensor; const Gate, Up: TMemoryBlock;
      const InputDim, OutputDim: Integer): Boolean;
    procedure Int4LinearAccumulate(const Dst, Src, Probabilities: TQNNHIPTensor; const Weight: TMemoryBlock;
      const InputDim, OutputDim, ProbabilityIndex: Integer);
    procedure Int4Linear(const Dst, Src: TQNNHIPTensor; const Weight: TMemoryBlock;
      const Rows, InputDim, OutputDim: Integer);
    procedure SampleToken(const Dst, Logits, Seen: TQNNHIPTensor; const Vocab, TopK: Integer;
      const Temperature, TopP, Penalty, Uniform: Single);
    procedure CachedAttention(const Dst, Q, Cache: TQNNHIPTensor;
      const QueryRows, Capacity, Heads, KvHeads, Dim, Position: Integer;
      const Window: Integer = 0; const Softcap: Single = 0; const Scale: Single = 0; const Masked: Boolean = False);
    procedure Gather(const Dst, Ids: TQNNHIPTensor; const Weight, Scales: TMemoryBlock;
      const Rows, Dim, Vocab, Rotation: Integer);
    procedure CheckFinite(const Tensor: TQNNHIPTensor; const Count: Integer = -1);
    function AllocatedBytes: UInt64;
    function ActivationBudget: UInt64;
    procedure TrimActivations;
    function PeakActivationBytes: UInt64;
    property OnWeightEvicted: TProc<IInterface> read FOnWeightEvicted write SetOnWeightEvicted;

    // HIP backend only (no TQNNGPUContext counterpart).
    // The routed experts of one MoE layer, resident as one set; MoEExperts
    // replaces the host loop of TLLMMoE.forward (LLM.MoE.pas:376-448).
    function CreateExpertSet(const Gates, Ups, Downs: array of TMemoryBlock; const Hidden, Inter: Integer): Pointer;
    procedure DestroyExpertSet(var ExpertSet: Pointer);
    procedure MoEExperts(const ExpertSet: Pointer; const Dst, Src, Routes: TQNNHIPTensor; const Rows, TopK: Integer);
    // Q8_0 prefill GEMM on int8 activations (per-32 quantiser).
    procedure Q8GemmInt8(const Dst, Src: TQNNHIPTensor; const Weight: TMemoryBlock;
      const Rows, InputDim, OutputDim: Integer);
    // Int4Linear without device allocation, for callers that cannot allocate
    // (graph capture, serving loops): resident weight, fixed 8 MiB scratch.
    procedure Int4LinearNoAlloc(const Dst, Src: TQNNHIPTensor; const Weight: TMemoryBlock;
      const Rows, InputDim, OutputDim: Integer);
    function Status: TQnnStatus;
  end;

{$IFDEF QNN_HIP}
  // With QNN_HIP defined, units that use QuickNN.HIP in place of
  // QuickNN.Vulkan compile unchanged against the same type names.
  TQNNGPUTensor = TQNNHIPTensor;
  TQNNGPUContext = TQNNHIPContext;
{$ENDIF}

// QNNGPUFloatBits (Context.API.inc:166): a float's bits as an Integer kernel argument.
function QNNGPUFloatBits(const Value: Single): Integer;

implementation

function QNNGPUFloatBits(const Value: Single): Integer;
begin
  Move(Value, Result, SizeOf(Result));
end;

procedure WeightEvictedThunk(Identity: UInt64; User: Pointer); cdecl;
var
  Ctx: TQNNHIPContext;
  Intf: IInterface;
begin
  Ctx := TQNNHIPContext(User);
  if not Ctx.FIdentities.TryGetValue(Identity, Intf) then
    Exit;
  Ctx.FIdentities.Remove(Identity);
  if Assigned(Ctx.FOnWeightEvicted) then
    Ctx.FOnWeightEvicted(Intf);
end;

// Status codes re-raise the reference's exception classes.
procedure TQNNHIPContext.Check(const Status: Integer);
var
  Buf: array[0..1023] of AnsiChar;
  Msg: string;
begin
  if Status >= 0 then
    Exit;
  qnn_last_error(@Buf[0], Length(Buf));
  Msg := string(UTF8String(PAnsiChar(@Buf[0])));
  case Status of
    QNN_E_ARGUMENT: raise EArgumentException.Create(Msg);
    QNN_E_RANGE: raise ERangeError.Create(Msg);
    QNN_E_NOT_SUPPORTED: raise ENotSupportedException.Create(Msg);
    QNN_E_FORMAT: raise EQNNHIPFormatError.Create(Msg);
    QNN_E_IO: raise EInOutError.Create(Msg);
  else
    raise EInvalidOp.Create(Msg);
  end;
end;

function TQNNHIPContext.Wrap(const H: Pointer; const Count: Integer): TQNNHIPTensor;
begin
  Result := TQNNHIPTensor.Create;
  Result.FHandle := H;
  Result.Count := Count;
end;

// The same immutable storage maps to the same key for the life of the
// process: the interface pointer of WeightIdentity (Common.pas:153-155).
function TQNNHIPContext.Desc(const W: TMemoryBlock): TQnnWeight;
var
  Key: UInt64;
begin
  if W.WeightIdentity = nil then
    raise EArgumentException.Create('GPU weights require an explicit immutable WeightIdentity');
  Key := UInt64(NativeUInt(Pointer(W.WeightIdentity)));
  if not FIdentities.ContainsKey(Key) then
    FIdentities.Add(Key, W.WeightIdentity);
  Result.Identity := Key;
  Result.Data := W.DataPtr;
  Result.Offset := W.Offset;
  Result.Size := W.Size;
  if Length(W.Shape) > 0 then
    Result.Shape0 := W.Shape[0]
  else
    Result.Shape0 := 1;
  if Length(W.Shape) > 1 then
    Result.Shape1 := W.Count div Max(Int64(1), W.Shape[0])
  else
    Result.Shape1 := 1;
  Result.DataType := Ord(W.DataType);
  Result.Encoding := Ord(W.Encoding);
end;

function TQNNHIPContext.DescOrNil(const W: TMemoryBlock; out D: TQnnWeight): PQnnWeight;
begin
  if W.DataPtr = nil then
    Exit(nil);
  D := Desc(W);
  Result := @D;
end;

function TQNNHIPContext.Descs(const Weights: array of TMemoryBlock): TArray<TQnnWeight>;
var
  I: Integer;
begin
  SetLength(Result, Length(Weights));
  for I := 0 to High(Weights) do
    Result[I] := Desc(Weights[I]);
end;

constructor TQNNHIPContext.Create(const Device: Integer; const WeightCacheBytes: UInt64);
begin
  inherited Create;
  FIdentities := TDictionary<UInt64, IInterface>.Create;
  Check(qnn_ctx_create(Device, WeightCacheBytes, FCtx));
end;

destructor TQNNHIPContext.Destroy;
var
  I: Integer;
begin
  for I := 0 to High(FScratch) do
    FreeAndNil(FScratch[I]);
  if FCtx <> nil then
    qnn_ctx_destroy(FCtx);
  FIdentities.Free;
  inherited;
end;

procedure TQNNHIPContext.SetOnWeightEvicted(const Value: TProc<IInterface>);
begin
  FOnWeightEvicted := Value;
  if Assigned(Value) then
    Check(qnn_set_weight_evicted(FCtx, WeightEvictedThunk, Self))
  else
    Check(qnn_set_weight_evicted(FCtx, nil, nil));
end;

function TQNNHIPContext.NewTensor(const Count: Integer): TQNNHIPTensor;
var
  H: Pointer;
begin
  Check(qnn_tensor_new(FCtx, Count, H));
  Result := Wrap(H, Count);
end;

procedure TQNNHIPContext.Recycle(var Tensor: TQNNHIPTensor);
begin
  if Tensor = nil then
    Exit;
  Check(qnn_recycle(FCtx, Tensor.FHandle));
  FreeAndNil(Tensor);
end;

function TQNNHIPContext.Scratch(const Slot, Count: Integer): TQNNHIPTensor;
var
  H: Pointer;
begin
  if (Slot < 0) or (Slot > High(FScratch)) then
    raise EArgumentException.Create('Invalid GPU scratch slot');
  Check(qnn_scratch(FCtx, Slot, Count, H));
  if (FScratch[Slot] = nil) or (FScratch[Slot].FHandle <> H) then
  begin
    FreeAndNil(FScratch[Slot]);
    FScratch[Slot] := Wrap(H, Count);
  end;
  FScratch[Slot].Count := qnn_tensor_count(H);
  Result := FScratch[Slot];
end;

procedure TQNNHIPContext.Flush;
begin
  Check(qnn_flush(FCtx));
end;

procedure TQNNHIPContext.RetainWeight(const Weight: TMemoryBlock; const Rows, Columns: Integer);
var
  W: TQnnWeight;
begin
  W := Desc(Weight);
  Check(qnn_retain_weight(FCtx, @W, Rows, Columns));
end;

procedure TQNNHIPContext.PreloadWeights(const Weights: array of TMemoryBlock; const StagingBytesLimit: UInt64);
var
  Ds: TArray<TQnnWeight>;
begin
  if Length(Weights) = 0 then
    Exit;
  Ds := Descs(Weights);
  Check(qnn_preload_weights(FCtx, @Ds[0], Length(Ds), StagingBytesLimit));
end;

function TQNNHIPContext.EnableWeightPrefetch(const MaxLayerBytes: UInt64): Boolean;
var
  Enabled: Integer;
begin
  Check(qnn_enable_weight_prefetch(FCtx, MaxLayerBytes, Enabled));
  Result := Enabled <> 0;
end;

procedure TQNNHIPContext.BeginWeightPrefetch;
begin
  Check(qnn_begin_weight_prefetch(FCtx));
end;

procedure TQNNHIPContext.PrefetchWeights(const Weights: array of TMemoryBlock; const DeferJoin: Boolean);
var
  Ds: TArray<TQnnWeight>;
begin
  if Length(Weights) = 0 then
    Exit;
  Ds := Descs(Weights);
  Check(qnn_prefetch_weights(FCtx, @Ds[0], Length(Ds), Ord(DeferJoin)));
end;

procedure TQNNHIPContext.StageWeightPrefetch(const Weights: array of TMemoryBlock);
var
  Ds: TArray<TQnnWeight>;
begin
  if Length(Weights) = 0 then
    Exit;
  Ds := Descs(Weights);
  Check(qnn_stage_weight_prefetch(FCtx, @Ds[0], Length(Ds)));
end;

procedure TQNNHIPContext.CompleteWeightPrefetch;
begin
  Check(qnn_complete_weight_prefetch(FCtx));
end;

function TQNNHIPContext.ActivatePrefetchedWeights(const Weights: array of TMemoryBlock): Boolean;
var
  Ds: TArray<TQnnWeight>;
  Activated: Integer;
begin
  if Length(Weights) = 0 then
    Exit(False);
  Ds := Descs(Weights);
  Check(qnn_activate_prefetched_weights(FCtx, @Ds[0], Length(Ds), Activated));
  Result := Activated <> 0;
end;

procedure TQNNHIPContext.SealWeightPrefetch;
begin
  Check(qnn_seal_weight_prefetch(FCtx));
end;

procedure TQNNHIPContext.EndWeightPrefetch;
begin
  Check(qnn_end_weight_prefetch(FCtx));
end;

function TQNNHIPContext.WeightBatchCapacity: UInt64;
begin
  Check(qnn_weight_batch_capacity(FCtx, Result));
end;

function TQNNHIPContext.IsWeightResident(const Weight: TMemoryBlock; const Rows, Columns: Integer): Boolean;
var
  W: TQnnWeight;
  R: Integer;
begin
  W := Desc(Weight);
  Check(qnn_is_weight_resident(FCtx, @W, Rows, Columns, R));
  Result := R <> 0;
end;

function TQNNHIPContext.Upload(const Data: TMemoryBlock): TQNNHIPTensor;
var
  W: TQnnWeight;
  H: Pointer;
begin
  W := Desc(Data);
  Check(qnn_upload(FCtx, @W, H));
  Result := Wrap(H, qnn_tensor_count(H));
end;

function TQNNHIPContext.UploadRaw(const Data: Pointer; const Count: Integer): TQNNHIPTensor;
var
  H: Pointer;
begin
  Check(qnn_upload_raw(FCtx, Data, Count, H));
  Result := Wrap(H, Count);
end;

procedure TQNNHIPContext.Download(const Tensor: TQNNHIPTensor; const Dst: Pointer; const Count: Integer);
begin
  Check(qnn_download(FCtx, Tensor.Handle, Dst, Count));
end;

procedure TQNNHIPContext.Copy(const Dst, Src: TQNNHIPTensor; const Count, DstOffset, SrcOffset: Integer);
begin
  Check(qnn_copy(FCtx, Dst.Handle, Src.Handle, Count, DstOffset, SrcOffset));
end;

procedure TQNNHIPContext.CopyCHWRect(const Dst, Src: TQNNHIPTensor; const Channels, SrcWidth, SrcHeight, DstWidth,
  DstHeight, SrcX, SrcY, DstX, DstY, Width, Height: Integer);
begin
  raise ENotSupportedException.Create('CopyCHWRect is not provided by the HIP backend');
end;

function TensorHandle(const T: TQNNHIPTensor): Pointer;
begin
  if T = nil then
    Result := nil
  else
    Result := T.Handle;
end;

procedure TQNNHIPContext.Kernel(const Op, N: Integer; const Dst, A, B, C: TQNNHIPTensor; const Args: array of Integer);
var
  P: PInteger;
begin
  if Length(Args) > 0 then
    P := @Args[0]
  else
    P := nil;
  Check(qnn_kernel(FCtx, Op, N, TensorHandle(Dst), TensorHandle(A), TensorHandle(B), TensorHandle(C), P, Length(Args)));
end;

procedure TQNNHIPContext.KernelWeights(const Op, N: Integer; const Dst, A: TQNNHIPTensor; const B, C: TMemoryBlock;
  const Args: array of Integer);
var
  DB, DC: TQnnWeight;
  P: PInteger;
begin
  if Length(Args) > 0 then
    P := @Args[0]
  else
    P := nil;
  Check(qnn_kernel_weights(FCtx, Op, N, TensorHandle(Dst), TensorHandle(A), DescOrNil(B, DB), DescOrNil(C, DC), P,
    Length(Args)));
end;

procedure TQNNHIPContext.Linear(const Dst, Src: TQNNHIPTensor; const Weight, Scales, Bias: TMemoryBlock;
  const Rows, InputDim, OutputDim: Integer; const Rotation: Integer);
var
  W, S, B: TQnnWeight;
begin
  if Rotation <> 0 then
    raise ENotSupportedException.Create('ConvRot weights are not handled by the HIP backend');
  W := Desc(Weight);
  Check(qnn_linear(FCtx, Dst.Handle, Src.Handle, @W, DescOrNil(Scales, S), DescOrNil(Bias, B), Rows, InputDim, OutputDim));
end;

procedure TQNNHIPContext.Attention(const Dst, Q, K, V: TQNNHIPTensor; const Rows, Heads, KvHeads, Dim, Causal: Integer;
  const Limits, T5Bias: TQNNHIPTensor);
begin
  raise ENotSupportedException.Create('Uncached attention is not provided by the HIP backend; use CachedAttention');
end;

procedure TQNNHIPContext.VectorLinear(const Dst, Src: TQNNHIPTensor; const Weight: TMemoryBlock;
  const InputDim, OutputDim: Integer);
var
  W: TQnnWeight;
begin
  W := Desc(Weight);
  Check(qnn_vector_linear(FCtx, Dst.Handle, Src.Handle, @W, InputDim, OutputDim));
end;

function TQNNHIPContext.TrySwiGLUVector(const Dst, Src: TQNNHIPTensor; const Gate, Up: TMemoryBlock;
  const InputDim, OutputDim: Integer): Boolean;
var
  G, U: TQnnWeight;
  St: Integer;
begin
  G := Desc(Gate);
  U := Desc(Up);
  St := qnn_swiglu_vector(FCtx, Dst.Handle, Src.Handle, @G, @U, InputDim, OutputDim);
  Check(St);
  Result := St = QNN_OK;  // QNN_NOT_HANDLED: the caller falls back to two projections + GO_SWIGLU
end;

procedure TQNNHIPContext.Int4LinearAccumulate(const Dst, Src, Probabilities: TQNNHIPTensor;
  const Weight: TMemoryBlock; const InputDim, OutputDim, ProbabilityIndex: Integer);
var
  W: TQnnWeight;
begin
  W := Desc(Weight);
  Check(qnn_int4_linear_accumulate(FCtx, Dst.Handle, Src.Handle, Probabilities.Handle, @W, InputDim, OutputDim,
    ProbabilityIndex));
end;

procedure TQNNHIPContext.Int4Linear(const Dst, Src: TQNNHIPTensor; const Weight: TMemoryBlock;
  const Rows, InputDim, OutputDim: Integer);
var
  W: TQnnWeight;
begin
  W := Desc(Weight);
  Check(qnn_int4_linear(FCtx, Dst.Handle, Src.Handle, @W, Rows, InputDim, OutputDim));
end;

procedure TQNNHIPContext.SampleToken(const Dst, Logits, Seen: TQNNHIPTensor; const Vocab, TopK: Integer;
  const Temperature, TopP, Penalty, Uniform: Single);
begin
  Check(qnn_sample_token(FCtx, Dst.Handle, Logits.Handle, Seen.Handle, Vocab, TopK, Temperature, TopP, Penalty,
    Uniform));
end;

procedure TQNNHIPContext.CachedAttention(const Dst, Q, Cache: TQNNHIPTensor;
  const QueryRows, Capacity, Heads, KvHeads, Dim, Position: Integer;
  const Window: Integer; const Softcap, Scale: Single; const Masked: Boolean);
begin
  Check(qnn_cached_attention(FCtx, Dst.Handle, Q.Handle, Cache.Handle, QueryRows, Capacity, Heads, KvHeads, Dim,
    Position, Window, Softcap, Scale, Ord(Masked)));
end;

procedure TQNNHIPContext.Gather(const Dst, Ids: TQNNHIPTensor; const Weight, Scales: TMemoryBlock;
  const Rows, Dim, Vocab, Rotation: Integer);
var
  W, S: TQnnWeight;
begin
  W := Desc(Weight);
  Check(qnn_gather(FCtx, Dst.Handle, Ids.Handle, @W, DescOrNil(Scales, S), Rows, Dim, Vocab, Rotation));
end;

procedure TQNNHIPContext.CheckFinite(const Tensor: TQNNHIPTensor; const Count: Integer);
var
  N: Integer;
begin
  if Count < 0 then
    N := Tensor.Count
  else
    N := Count;
  Check(qnn_check_finite(FCtx, Tensor.Handle, N));
end;

function TQNNHIPContext.Status: TQnnStatus;
begin
  Check(qnn_get_status(FCtx, Result));
end;

function TQNNHIPContext.AllocatedBytes: UInt64;
var
  S: TQnnStatus;
begin
  S := Status;
  Result := S.ActivationBytes + S.WeightBytes;
end;

function TQNNHIPContext.ActivationBudget: UInt64;
var
  S: TQnnStatus;
begin
  // Activations and weights share the device; the weight cache limit is what remains for weights.
  S := Status;
  Result := S.WeightLimit;
end;

procedure TQNNHIPContext.TrimActivations;
begin
  Flush;
end;

function TQNNHIPContext.PeakActivationBytes: UInt64;
begin
  Result := Status.ActivationPeakBytes;
end;

function TQNNHIPContext.CreateExpertSet(const Gates, Ups, Downs: array of TMemoryBlock;
  const Hidden, Inter: Integer): Pointer;
var
  G, U, D: TArray<TQnnWeight>;
begin
  if (Length(Gates) = 0) or (Length(Ups) <> Length(Gates)) or (Length(Downs) <> Length(Gates)) then
    raise EArgumentException.Create('Expert set needs equal, non-empty gate/up/down lists');
  G := Descs(Gates);
  U := Descs(Ups);
  D := Descs(Downs);
  Check(qnn_expert_set_create(FCtx, @G[0], @U[0], @D[0], Length(G), Hidden, Inter, Result));
end;

procedure TQNNHIPContext.DestroyExpertSet(var ExpertSet: Pointer);
begin
  if ExpertSet = nil then
    Exit;
  Check(qnn_expert_set_destroy(FCtx, ExpertSet));
  ExpertSet := nil;
end;

procedure TQNNHIPContext.MoEExperts(const ExpertSet: Pointer; const Dst, Src, Routes: TQNNHIPTensor;
  const Rows, TopK: Integer);
begin
  Check(qnn_moe_experts(FCtx, ExpertSet, Dst.Handle, Src.Handle, Routes.Handle, Rows, TopK));
end;

procedure TQNNHIPContext.Q8GemmInt8(const Dst, Src: TQNNHIPTensor; const Weight: TMemoryBlock;
  const Rows, InputDim, OutputDim: Integer);
var
  W: TQnnWeight;
begin
  W := Desc(Weight);
  Check(qnn_q8_gemm_int8(FCtx, Dst.Handle, Src.Handle, @W, Rows, InputDim, OutputDim));
end;

procedure TQNNHIPContext.Int4LinearNoAlloc(const Dst, Src: TQNNHIPTensor; const Weight: TMemoryBlock;
  const Rows, InputDim, OutputDim: Integer);
var
  W: TQnnWeight;
begin
  W := Desc(Weight);
  Check(qnn_int4_linear_noalloc(FCtx, Dst.Handle, Src.Handle, @W, Rows, InputDim, OutputDim));
end;

end.
