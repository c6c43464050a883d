// QuantDecoders (AnimaXS/Runtime/Animapk/QuantDecoders.swift:17-164) over the library's
// CPU decoders: value = q * scale + zero per 64-wide group with fp16 scale / zero,
// groups reset at every row, W4 holding the even K index in the low nibble.  As in the
// reference, the decoders do not throw: an inconsistent shape traps.
import CAnimaHIP
import Foundation

public enum QuantDecoders {
    /// QuantDecoders.dequantW4 (:23-48).
    public static func dequantW4(data: Data, scale: Data, zero: Data, k: Int, groupSize: Int = 64) -> [Float] {
        precondition(k >= 0 && groupSize > 0)
        var out = [Float](repeating: 0, count: k)
        guard k > 0 else { return out }
        checkSizes(data, scale, zero, dataBytes: (k + 1) / 2, groups: (k + groupSize - 1) / groupSize)
        withBytes(data, scale, zero) { d, s, z in
            require(anima_dequant_w4(d, s, z, Int64(k), Int64(groupSize), &out))
        }
        return out
    }

    /// QuantDecoders.dequantW4Matrix (:54-87).
    public static func dequantW4Matrix(data: Data, scale: Data, zero: Data, rows: Int, cols: Int,
                                       groupSize: Int = 64) -> [Float] {
        precondition(rows >= 0 && cols >= 0 && groupSize > 0)
        var out = [Float](repeating: 0, count: rows * cols)
        guard rows > 0 && cols > 0 else { return out }
        checkSizes(data, scale, zero, dataBytes: rows * ((cols + 1) / 2),
                   groups: rows * ((cols + groupSize - 1) / groupSize))
        withBytes(data, scale, zero) { d, s, z in
            require(anima_dequant_w4_matrix(d, s, z, Int64(rows), Int64(cols), Int64(groupSize), &out))
        }
        return out
    }

    /// QuantDecoders.dequantW8 (:90-114).
    public static func dequantW8(data: Data, scale: Data, zero: Data, k: Int, groupSize: Int = 64) -> [Float] {
        precondition(k >= 0 && groupSize > 0)
        var out = [Float](repeating: 0, count: k)
        guard k > 0 else { return out }
        checkSizes(data, scale, zero, dataBytes: k, groups: (k + groupSize - 1) / groupSize)
        withBytes(data, scale, zero) { d, s, z in
            require(anima_dequant_w8(d, s, z, Int64(k), Int64(groupSize), &out))
        }
        return out
    }

    /// QuantDecoders.dequantW8Matrix (:117-147).
    public static func dequantW8Matrix(data: Data, scale: Data, zero: Data, rows: Int, cols: Int,
                                       groupSize: Int = 64) -> [Float] {
        precondition(rows >= 0 && cols >= 0 && groupSize > 0)
        var out = [Float](repeating: 0, count: rows * cols)
        guard rows > 0 && cols > 0 else { return out }
        checkSizes(data, scale, zero, dataBytes: rows * cols, groups: rows * ((cols + groupSize - 1) / groupSize))
        withBytes(data, scale, zero) { d, s, z in
            require(anima_dequant_w8_matrix(d, s, z, Int64(rows), Int64(cols), Int64(groupSize), &out))
        }
        return out
    }

    /// QuantDecoders.fp16ToFloat32 (:150-163).
    public static func fp16ToFloat32(_ bytes: Data, count: Int) -> [Float] {
        var out = [Float](repeating: 0, count: count)
        guard count > 0 else { return out }
        precondition(bytes.count >= 2 * count, "fp16 data holds fewer than count values")
        bytes.withUnsafeBytes { b in
            require(anima_fp16_to_float32(b.bindMemory(to: UInt16.self).baseAddress, Int64(count), &out))
        }
        return out
    }

    private static func checkSizes(_ data: Data, _ scale: Data, _ zero: Data, dataBytes: Int, groups: Int) {
        precondition(data.count >= dataBytes, "quantized data holds fewer bytes than the shape needs")
        precondition(scale.count >= 2 * groups && zero.count >= 2 * groups,
                     "scale / zero hold fewer fp16 values than the shape has groups")
    }

    private static func withBytes(_ data: Data, _ scale: Data, _ zero: Data,
                                  _ body: (UnsafePointer<UInt8>?, UnsafePointer<UInt16>?,
                                           UnsafePointer<UInt16>?) -> Void) {
        data.withUnsafeBytes { d in
            scale.withUnsafeBytes { s in
                zero.withUnsafeBytes { z in
                    body(d.bindMemory(to: UInt8.self).baseAddress,
                             s.bindMemory(to: UInt16.self).baseAddress,
                             z.bindMemory(to: UInt16.self).baseAddress)
                }
            }
        }
    }
}
