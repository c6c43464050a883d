// AttentionExecutor with the reference's call surface
// (AnimaXS/Runtime/Metal/AttentionExecutor.swift:5-12, 29-64, 97-133, 751-776) over
// anima_attention_*.  The DiT block, Qwen encoder, LLM adapter and VAE keep calling
// init / encode / execute / maximumScoreScratchBytes as they do today.
import CAnimaHIP

/// AttentionNumerics (AttentionExecutor.swift:5-12).
public enum AttentionNumerics: String, CaseIterable {
    case legacy
    case fp32ScoresAndSoftmax
    case bf16Compute = "bf16_compute"

    var code: Int32 {
        switch self {
        case .legacy: return Int32(ANIMA_NUMERICS_LEGACY.rawValue)
        case .fp32ScoresAndSoftmax: return Int32(ANIMA_NUMERICS_FP32_SCORES.rawValue)
        case .bf16Compute: return Int32(ANIMA_NUMERICS_BF16_COMPUTE.rawValue)
        }
    }
}

/// AttentionInputLayout (AttentionExecutor.swift:55-64); tokenStride in half elements.
public enum AttentionInputLayout: Equatable {
    case headMajor
    case tokenMajor(tokenStride: Int)

    public var isTokenMajor: Bool {
        if case .tokenMajor = self { return true }
        return false
    }

    var code: Int32 {
        switch self {
        case .headMajor: return Int32(ANIMA_LAYOUT_HEAD_MAJOR.rawValue)
        case .tokenMajor: return Int32(ANIMA_LAYOUT_TOKEN_MAJOR.rawValue)
        }
    }

    var tokenStride: Int64 {
        if case .tokenMajor(let stride) = self { return Int64(stride) }
        return 0
    }
}

/// DiTAttentionBackend (AttentionExecutor.swift:29-44) with the reference's case
/// names.  The two MPS score-tile backends keep their fp16 score and probability
/// round trips under legacy numerics (ANIMA_ATTENTION_BACKEND_LEGACY_MPS); the
/// streaming and flash backends, which keep fp32 softmax state, both run the MFMA
/// flash kernel.  `auto` and `generic` are the MI355X additions: the flash kernel
/// whenever its contract holds, and the fp32 diagnostic kernel.
public enum DiTAttentionBackend: String, CaseIterable {
    case legacyHeadMajorMPS
    case stridedTokenMajorMPS
    case streamingMPS
    case metalFlash
    case auto
    case generic

    var code: Int32 {
        switch self {
        case .legacyHeadMajorMPS, .stridedTokenMajorMPS: return Int32(ANIMA_ATTENTION_BACKEND_LEGACY_MPS.rawValue)
        case .streamingMPS, .auto: return Int32(ANIMA_ATTENTION_BACKEND_AUTO.rawValue)
        case .metalFlash: return Int32(ANIMA_ATTENTION_BACKEND_FLASH.rawValue)
        case .generic: return Int32(ANIMA_ATTENTION_BACKEND_GENERIC.rawValue)
        }
    }
}

/// Query-tiled scaled dot-product attention; non-reentrant like the reference's
/// executor (one caller at a time; executors may share a context).
public final class AttentionExecutor {
    public static let defaultTileRows = 128

    let handle: OpaquePointer
    public let context: HIPContext
    public let tileRows: Int
    public let numerics: AttentionNumerics
    public let layout: AttentionInputLayout
    public let attentionBackend: DiTAttentionBackend

    public init(context: HIPContext, tileRows: Int = AttentionExecutor.defaultTileRows,
                numerics: AttentionNumerics = .legacy,
                layout: AttentionInputLayout = .headMajor,
                attentionBackend: DiTAttentionBackend = .auto) {
        precondition(tileRows > 0)
        var config = anima_attention_config(
            tile_rows: Int32(tileRows), numerics: numerics.code, backend: attentionBackend.code,
            layout: layout.code, token_stride: layout.tokenStride, flash_rows: 0)
        var out: OpaquePointer?
        require(anima_attention_create(context.handle, &config, &out))
        handle = out!
        self.context = context
        self.tileRows = tileRows
        self.numerics = numerics
        self.layout = layout
        self.attentionBackend = attentionBackend
    }

    deinit { _ = anima_attention_destroy(handle) }

    /// AttentionExecutor.maximumScoreScratchBytes (AttentionExecutor.swift:112-120).
    public func maximumScoreScratchBytes(keyCount: Int, queryCount: Int? = nil) throws -> Int {
        var bytes: Int64 = 0
        try check(anima_attention_max_score_scratch_bytes(handle, Int64(keyCount), Int64(queryCount ?? 0), &bytes))
        return Int(bytes)
    }

    /// AttentionExecutor.encode (AttentionExecutor.swift:122-133): appends to the
    /// context's stream.  The trailing parameters are the library's extensions; their
    /// defaults give the reference's behaviour.
    public func encode(query: DeviceBuffer, queryOffset: Int = 0,
                       key: DeviceBuffer, keyOffset: Int = 0,
                       value: DeviceBuffer, valueOffset: Int = 0,
                       output: DeviceBuffer, outputOffset: Int = 0,
                       heads: Int, queryCount: Int, keyCount: Int, headDim: Int,
                       keyValueHeads: Int? = nil,
                       causal: Bool = false,
                       layout: AttentionInputLayout? = nil,
                       batch: Int = 1,
                       keyLengths: [Int32]? = nil,
                       scale: Float = 0,
                       prologue: anima_qk_prologue? = nil,
                       kvTokenStride: Int = 0) throws {
        try run(anima_attention_encode, query: query, queryOffset: queryOffset, key: key, keyOffset: keyOffset,
                value: value, valueOffset: valueOffset, output: output, outputOffset: outputOffset,
                heads: heads, queryCount: queryCount, keyCount: keyCount, headDim: headDim,
                keyValueHeads: keyValueHeads, causal: causal, layout: layout, batch: batch,
                keyLengths: keyLengths, scale: scale, prologue: prologue, kvTokenStride: kvTokenStride)
    }

    /// AttentionExecutor.execute (AttentionExecutor.swift:751-776): encode, then wait.
    public func execute(query: DeviceBuffer, queryOffset: Int = 0,
                        key: DeviceBuffer, keyOffset: Int = 0,
                        value: DeviceBuffer, valueOffset: Int = 0,
                        output: DeviceBuffer, outputOffset: Int = 0,
                        heads: Int, queryCount: Int, keyCount: Int, headDim: Int,
                        keyValueHeads: Int? = nil,
                        causal: Bool = false,
                        layout: AttentionInputLayout? = nil) throws {
        try run(anima_attention_execute, query: query, queryOffset: queryOffset, key: key, keyOffset: keyOffset,
                value: value, valueOffset: valueOffset, output: output, outputOffset: outputOffset,
                heads: heads, queryCount: queryCount, keyCount: keyCount, headDim: headDim,
                keyValueHeads: keyValueHeads, causal: causal, layout: layout, batch: 1,
                keyLengths: nil, scale: 0, prologue: nil, kvTokenStride: 0)
    }

    private func run(_ entry: (OpaquePointer?, UnsafePointer<anima_attention_args>?) -> anima_status,
                     query: DeviceBuffer, queryOffset: Int, key: DeviceBuffer, keyOffset: Int,
                     value: DeviceBuffer, valueOffset: Int, output: DeviceBuffer, outputOffset: Int,
                     heads: Int, queryCount: Int, keyCount: Int, headDim: Int,
                     keyValueHeads: Int?, causal: Bool, layout: AttentionInputLayout?, batch: Int,
                     keyLengths: [Int32]?, scale: Float, prologue: anima_qk_prologue?,
                     kvTokenStride: Int) throws {
        var args = anima_attention_args()
        args.query = query.raw; args.query_offset = Int64(queryOffset)
        args.key = key.raw; args.key_offset = Int64(keyOffset)
        args.value = value.raw; args.value_offset = Int64(valueOffset)
        args.output = output.raw; args.output_offset = Int64(outputOffset)
        args.heads = Int64(heads)
        args.query_count = Int64(queryCount)
        args.key_count = Int64(keyCount)
        args.head_dim = Int64(headDim)
        args.key_value_heads = Int64(keyValueHeads ?? 0)
        args.causal = causal ? 1 : 0
        args.layout = layout?.code ?? -1
        args.token_stride = layout?.tokenStride ?? 0
        args.batch = Int64(batch)
        args.key_lengths_on_device = 0
        args.scale = scale
        args.kv_token_stride = Int64(kvTokenStride)
        let lengths = keyLengths ?? []
        var pro = prologue ?? anima_qk_prologue()
        try lengths.withUnsafeBufferPointer { lengthBuffer in
            try withUnsafePointer(to: &pro) { proPointer in
                args.key_lengths = keyLengths == nil ? nil : lengthBuffer.baseAddress
                args.prologue = prologue == nil ? nil : proPointer
                try check(entry(handle, &args))
            }
        }
    }
}
