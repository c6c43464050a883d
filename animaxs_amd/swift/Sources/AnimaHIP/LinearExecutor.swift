// LinearExecutor with the reference's call surface
// (AnimaXS/Runtime/Metal/LinearExecutor.swift:10-29, 43-88, 386-438) over
// anima_linear_*: the packed W4/W8 (or fp16) [N, K] weight stays in its .animapk
// layout, and the GEMM dequantises it in registers ahead of the matrix cores.
import CAnimaHIP

/// StorageDtype (Runtime/Animapk/AnimapkTensor.swift:4-9): the pack's storage codes.
public enum StorageDtype: UInt8, Equatable {
    case w4 = 0
    case w8 = 1
    case fp16 = 2
    case fp32 = 3
}

/// DiTLinearFamily (LinearExecutor.swift:10-15).
public enum DiTLinearFamily {
    case attentionProjection
    case mlpUp
    case mlpDown
    case other

    var code: Int32 {
        switch self {
        case .attentionProjection: return Int32(ANIMA_FAMILY_ATTENTION_PROJECTION.rawValue)
        case .mlpUp: return Int32(ANIMA_FAMILY_MLP_UP.rawValue)
        case .mlpDown: return Int32(ANIMA_FAMILY_MLP_DOWN.rawValue)
        case .other: return Int32(ANIMA_FAMILY_OTHER.rawValue)
        }
    }
}

/// DiTLinearBackend (Runtime/Generation/InferenceOptimizationConfig.swift:7-30) with the
/// reference's case names.  dequantizedMPS keeps its shape (dequantise the whole
/// weight to fp16 scratch, then an fp16 GEMM); every direct / hybrid choice runs the
/// fused in-register-dequant MFMA GEMM, which is the fastest form for every family
/// on MI355X.
public enum DiTLinearBackend: String, CaseIterable {
    case dequantizedMPS
    case directQuantized
    case hybrid
    case aneHybridW8

    var code: Int32 {
        switch self {
        case .dequantizedMPS: return Int32(ANIMA_LINEAR_BACKEND_DEQUANT_THEN_GEMM.rawValue)
        case .directQuantized: return Int32(ANIMA_LINEAR_BACKEND_FUSED.rawValue)
        case .hybrid, .aneHybridW8: return Int32(ANIMA_LINEAR_BACKEND_AUTO.rawValue)
        }
    }
}

/// QuantizedLinearWeightBuffers (LinearExecutor.swift:18-29): buffers and metadata for a
/// packed [rows = N, columns = K] matrix; packedRowStride is bytes per row for W4/W8
/// and halfs per row for fp16.
public struct QuantizedLinearWeightBuffers {
    public let storage: StorageDtype
    public let packed: DeviceBuffer
    public let packedOffset: Int
    public let scale: DeviceBuffer?
    public let scaleOffset: Int
    public let zero: DeviceBuffer?
    public let zeroOffset: Int
    public let rows: Int
    public let columns: Int
    public let packedRowStride: Int

    public init(storage: StorageDtype, packed: DeviceBuffer, packedOffset: Int = 0,
                scale: DeviceBuffer?, scaleOffset: Int = 0, zero: DeviceBuffer?, zeroOffset: Int = 0,
                rows: Int, columns: Int, packedRowStride: Int) {
        self.storage = storage
        self.packed = packed
        self.packedOffset = packedOffset
        self.scale = scale
        self.scaleOffset = scaleOffset
        self.zero = zero
        self.zeroOffset = zeroOffset
        self.rows = rows
        self.columns = columns
        self.packedRowStride = packedRowStride
    }

    /// The C ABI view (anima_qweight), for the library entry points the wrappers do not cover.
    public var raw: anima_qweight {
        anima_qweight(storage: Int32(storage.rawValue),
                      packed: packed.raw, packed_offset: Int64(packedOffset),
                      scale: scale.raw, scale_offset: Int64(scaleOffset),
                      zero: zero.raw, zero_offset: Int64(zeroOffset),
                      rows: Int64(rows), columns: Int64(columns),
                      packed_row_stride: Int64(packedRowStride))
    }
}

public final class LinearExecutor {
    public static let defaultTileRows = 128

    let handle: OpaquePointer
    public let context: HIPContext
    public let tileRows: Int
    public let linearBackend: DiTLinearBackend
    public let family: DiTLinearFamily

    /// LinearExecutor.init (LinearExecutor.swift:64-75).  directMPSIO selects how the
    /// reference wraps MPS matrices; the HIP kernels read and write the caller's
    /// buffers in place either way, so it is accepted and has no effect.
    public init(context: HIPContext, tileRows: Int = LinearExecutor.defaultTileRows,
                directMPSIO: Bool = false,
                linearBackend: DiTLinearBackend = .directQuantized,
                family: DiTLinearFamily = .other) {
        precondition(tileRows > 0)
        var config = anima_linear_config(tile_rows: Int32(tileRows), backend: linearBackend.code)
        var out: OpaquePointer?
        require(anima_linear_create(context.handle, &config, &out))
        handle = out!
        self.context = context
        self.tileRows = tileRows
        self.linearBackend = linearBackend
        self.family = family
    }

    deinit { _ = anima_linear_destroy(handle) }

    /// LinearExecutor.encode (LinearExecutor.swift:79-88): output[M, N] = input[M, K] x W^T
    /// in fp16 with fp32 accumulation, appended to the context's stream.
    public func encode(input: DeviceBuffer, inputOffset: Int = 0,
                       weight: QuantizedLinearWeightBuffers,
                       output: DeviceBuffer, outputOffset: Int = 0,
                       inputRows: Int,
                       family: DiTLinearFamily = .other) throws {
        var w = weight.raw
        try check(anima_linear_encode(handle, input.raw, Int64(inputOffset), &w, output.raw,
                                      Int64(outputOffset), Int64(inputRows), family.code))
    }

    /// LinearExecutor.execute (LinearExecutor.swift:386-410): encode, then wait.
    public func execute(input: DeviceBuffer, inputOffset: Int = 0,
                        weight: QuantizedLinearWeightBuffers,
                        output: DeviceBuffer, outputOffset: Int = 0,
                        inputRows: Int,
                        family: DiTLinearFamily = .other) throws {
        var w = weight.raw
        try check(anima_linear_execute(handle, input.raw, Int64(inputOffset), &w, output.raw,
                                       Int64(outputOffset), Int64(inputRows), family.code))
    }
}
