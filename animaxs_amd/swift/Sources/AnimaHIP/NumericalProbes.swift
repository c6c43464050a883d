// The device side of NumericalMonitor (AnimaXS/Runtime/Diagnostics/NumericalMonitor.swift:
// 186-212, 320-358): a stats buffer of one uint32 quad per probe slot, its reset
// (beginRun) and the standalone fp16 / fp32 passes (encodeProbe / encodeProbeF32), all
// on the context's stream.  The buffer lives in device memory, so the caller copies a
// slot's four words back after synchronising and decodes them with ProbeStats.
import CAnimaHIP

public struct NumericalProbes {
    public let context: HIPContext
    public let stats: DeviceBuffer
    public let slots: Int

    public init(context: HIPContext, stats: DeviceBuffer, slots: Int) {
        precondition(slots >= 0 && stats.length >= slots * Int(ANIMA_PROBE_SLOT_UINTS) * 4)
        self.context = context
        self.stats = stats
        self.slots = slots
    }

    /// beginRun (:205-212): every slot to flags 0, max 0, first index 0xFFFFFFFF.
    public func beginRun() throws {
        try check(anima_numerics_probe_reset_encode(context.handle, stats.raw, Int32(slots)))
    }

    /// encodeProbe (:320-338): one pass over `count` fp16 values into `slot`.
    public func encodeProbe(values: DeviceBuffer, offset: Int = 0, count: Int, slot: Int) throws {
        try check(anima_numerics_probe_encode(context.handle, values.raw, Int64(offset), Int64(count),
                                              Int32(ANIMA_PROBE_F16.rawValue), stats.raw, Int32(slot)))
    }

    /// encodeProbeF32 (:340-358): one pass over `count` fp32 values into `slot`.
    public func encodeProbeF32(values: DeviceBuffer, offset: Int = 0, count: Int, slot: Int) throws {
        try check(anima_numerics_probe_encode(context.handle, values.raw, Int64(offset), Int64(count),
                                              Int32(ANIMA_PROBE_F32.rawValue), stats.raw, Int32(slot)))
    }
}

/// NumericalMonitor.Stats (:136-161) decoded from a slot's words
/// [flags, max |v| as fp32 bits, first index, reserved].
public struct ProbeStats: Equatable {
    public var flags: UInt32 = 0
    public var maxAbs: Float = 0
    public var firstIndex: UInt32 = .max

    public init() {}

    public init(words: [UInt32]) {
        precondition(words.count >= 3)
        flags = words[0]
        maxAbs = Float(bitPattern: words[1])
        firstIndex = words[2]
    }

    public var hasIssue: Bool { flags != 0 }
    public var hasNaN: Bool { flags & ANIMA_PROBE_FLAG_NAN != 0 }
    public var hasPosInf: Bool { flags & ANIMA_PROBE_FLAG_POS_INF != 0 }
    public var hasNegInf: Bool { flags & ANIMA_PROBE_FLAG_NEG_INF != 0 }
    public var hasHalfOverflow: Bool { flags & ANIMA_PROBE_FLAG_HALF_OVERFLOW != 0 }

    /// The reference's short condition text (:151-160) for the flags the passes set.
    public var condition: String {
        if hasNaN { return "NaN detected" }
        if hasPosInf { return "positive Inf detected" }
        if hasNegInf { return "negative Inf detected" }
        if hasHalfOverflow { return "value exceeded FP16 finite range" }
        return "non-finite value detected"
    }
}
