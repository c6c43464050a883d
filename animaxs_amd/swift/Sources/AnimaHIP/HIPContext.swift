// The MetalContext / MTLBuffer / AnimapkError analogs the executors below take
// (AnimaXS/Runtime/Metal/MetalContext.swift:14-81).  A Metal buffer plus byte offset
// becomes a device pointer with its byte length plus the same byte offset; a command
// buffer becomes the context's HIP stream.
import CAnimaHIP

/// Mirrors AnimapkError (thrown by the reference's validate/encode paths): every
/// non-zero anima_status carries the library's message text, which keeps the
/// reference's wording for the validation failures.
public enum AnimapkError: Error, Equatable {
    case validation(String)
    case unsupported(String)
    case device(String)
    case format(String)
    case io(String)
}

@inline(__always)
func check(_ status: anima_status) throws {
    if status == ANIMA_OK { return }
    let message = String(cString: anima_last_error())
    switch status {
    case ANIMA_E_UNSUPPORTED: throw AnimapkError.unsupported(message)
    case ANIMA_E_DEVICE: throw AnimapkError.device(message)
    case ANIMA_E_FORMAT: throw AnimapkError.format(message)
    case ANIMA_E_IO: throw AnimapkError.io(message)
    default: throw AnimapkError.validation(message)
    }
}

/// For the calls the reference guards with preconditions (executor construction, the
/// CPU decoders): a failure traps with the library's message, as a failed precondition
/// does there, so these entry points keep the reference's non-throwing signatures.
@inline(__always)
func require(_ status: anima_status) {
    if status == ANIMA_OK { return }
    preconditionFailure(String(cString: anima_last_error()))
}

/// A device allocation (hipMalloc or any device-visible pointer) and the bytes
/// addressable from it: the MTLBuffer of the reference signatures.
public struct DeviceBuffer {
    public let pointer: UnsafeMutableRawPointer
    public let length: Int

    public init(pointer: UnsafeMutableRawPointer, length: Int) {
        self.pointer = pointer
        self.length = length
    }

    /// The C ABI view, for the library entry points the wrappers do not cover.
    public var raw: anima_buffer { anima_buffer(ptr: pointer, length: Int64(length)) }
}

extension Optional where Wrapped == DeviceBuffer {
    var raw: anima_buffer { self?.raw ?? anima_buffer(ptr: nil, length: 0) }
}

/// MetalContext analog: one HIP device and the stream every encode appends to.
public final class HIPContext {
    let handle: OpaquePointer

    public init(device: Int32 = 0) throws {
        var out: OpaquePointer?
        try check(anima_ctx_create(device, &out))
        handle = out!
    }

    /// Replace the stream (a hipStream_t) the encodes append to; nil is the null stream.
    public func setStream(_ stream: UnsafeMutableRawPointer?) throws {
        try check(anima_ctx_set_stream(handle, stream))
    }

    /// Command-buffer completion: wait for everything encoded on the stream.
    public func synchronize() throws {
        try check(anima_ctx_synchronize(handle))
    }

    public static var abiVersion: Int32 { anima_abi_version() }

    deinit { _ = anima_ctx_destroy(handle) }
}
