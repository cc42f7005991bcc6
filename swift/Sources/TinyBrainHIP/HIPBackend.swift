// HIPBackend.swift -- TinyBrain's backend protocols on libtinybrain_hip
// (MI355X, gfx950), through the C ABI in include/tinybrain_hip.h.
//
// Replaces MetalBackend (Sources/TinyBrainMetal/MetalBackend.swift) in the
// type-erased slot TinyBrainBackend.metalBackend (Backend.swift:29), which
// Tensor.matmul(QuantizedTensor) (QuantizedTensor.swift:627-643) and the
// dispatch helpers (Backend.swift:37-95) already look up; no call site of
// the runtime changes.  Every non-zero tbh_status becomes a Swift `throw`, on
// which the runtime falls back to its CPU path (QuantizedTensor.swift:634-642),
// exactly as for a Metal error.  Shape violations stay preconditions, as in
// MetalBackend.swift:895-897.
//
// Build: the reference's Package.swift gains
//   .systemLibrary(name: "CTinyBrainHIP", path: "Sources/CTinyBrainHIP"),
//   .target(name: "TinyBrainHIP", dependencies: ["TinyBrainRuntime", "CTinyBrainHIP"],
//           path: "Sources/TinyBrainHIP",
//           linkerSettings: [.unsafeFlags(["-L<dir of libtinybrain_hip.so>"])])
// and an app registers the backend where the umbrella registers Metal
// (Sources/TinyBrain/TinyBrain.swift:35-48):
//   TinyBrainBackend.metalBackend = try? HIPBackend()

import CTinyBrainHIP
import Foundation
import TinyBrainRuntime

public enum HIPError: Error, CustomStringConvertible {
    case status(Int32, String)

    public var description: String {
        switch self {
        case let .status(code, message): return "tbh_status \(code): \(message)"
        }
    }
}

@inline(__always) private func check(_ st: tbh_status) throws {
    if st != Int32(TBH_OK) { throw HIPError.status(st, String(cString: tbh_last_error())) }
}

/// A tensor's elements in row-major order, whatever its strides (the
/// reference's transpose() is a strided view; MetalBackend copies such views
/// with makeContiguousCopy, MetalBackend.swift:916, 1522-1550).
private func hostScalars(_ t: Tensor<Float>) -> [Float] {
    if t.isContiguous { return t.scalars }
    let dims = t.shape.dimensions, strides = t.shape.strides, raw = t.rawData
    var out = [Float](repeating: 0, count: t.shape.count)
    var index = [Int](repeating: 0, count: dims.count)
    for i in 0..<out.count {
        var offset = 0
        for d in 0..<dims.count { offset += index[d] * strides[d] }
        out[i] = raw[offset]
        var d = dims.count - 1
        while d >= 0 {
            index[d] += 1
            if index[d] < dims[d] { break }
            index[d] = 0
            d -= 1
        }
    }
    return out
}

public final class HIPBackend: QuantizedMatMulBackend, SoftmaxBackend, RMSNormBackend, ActivationBackend,
    AttentionBackend
{
    private let dev: OpaquePointer
    // One repacked device copy per QuantizedTensor.identifier, kept for the
    // backend's lifetime under a lock (MetalBackend.swift:33-34, 1282-1308).
    // Unlike the reference (cachedINT4Buffers, :1322-1359), INT4 is cached too.
    private var cache: [UUID: OpaquePointer] = [:]
    // Tensors whose flat INT4 data is the converter's [N, K] order
    // (Scripts/convert_model.py:489-502): groups run along K.
    private var converterLayout: Set<UUID> = []
    private let lock = NSLock()

    /// MetalBackend.isAvailable: a gfx950 device can be opened.
    public static var isAvailable: Bool {
        var d: OpaquePointer?
        guard tbh_device_open(0, &d) == Int32(TBH_OK), let dd = d else { return false }
        tbh_device_close(dd)
        return true
    }

    /// MetalBackend.init (MetalBackend.swift:38-56): throws off gfx950.
    public init(ordinal: Int32 = 0) throws {
        var d: OpaquePointer?
        try check(tbh_device_open(ordinal, &d))
        dev = d!
    }

    deinit {
        for w in cache.values { tbh_weight_destroy(w) }
        tbh_device_close(dev)
    }

    /// Marks an INT4 tensor loaded from a converter-written .tbf file (mode
    /// byte 3): its data is read with groups along K (TBH_LAYOUT_NK_FLAT).
    public func markConverterLayout(_ quantized: QuantizedTensor) {
        lock.lock()
        defer { lock.unlock() }
        converterLayout.insert(quantized.identifier)
    }

    /// Drops the device copy of a weight (no reference counterpart: the
    /// Metal cache is never evicted).
    public func evict(_ quantized: QuantizedTensor) {
        lock.lock()
        defer { lock.unlock() }
        if let w = cache.removeValue(forKey: quantized.identifier) { tbh_weight_destroy(w) }
    }

    private func weight(_ q: QuantizedTensor) throws -> OpaquePointer {
        lock.lock()
        defer { lock.unlock() }
        if let w = cache[q.identifier] { return w }
        let mode: Int32
        switch q.mode {
        case .symmetric: mode = Int32(TBH_MODE_SYMMETRIC)
        case .asymmetric: mode = Int32(TBH_MODE_ASYMMETRIC)
        case .perChannel: mode = Int32(TBH_MODE_PER_CHANNEL)
        case .int4: mode = Int32(TBH_MODE_INT4)
        case .int4PerChannel: mode = Int32(TBH_MODE_INT4_PER_CHANNEL)  // TBH_E_UNSUPPORTED: CPU fallback
        }
        let layout = converterLayout.contains(q.identifier) ? Int32(TBH_LAYOUT_NK_FLAT) : Int32(TBH_LAYOUT_KN_FLAT)
        var w: OpaquePointer?
        let zeroPoints = q.zeroPoints ?? []
        try q.data.withUnsafeBufferPointer { d in
            try q.scales.withUnsafeBufferPointer { s in
                try zeroPoints.withUnsafeBufferPointer { z in
                    var desc = tbh_qtensor_desc(
                        K: Int64(q.shape.dimensions[0]),
                        N: Int64(q.shape.dimensions[1]),
                        precision: q.precision == .int8 ? Int32(TBH_PREC_INT8) : Int32(TBH_PREC_INT4),
                        mode: mode,
                        layout: layout,
                        group_size: Int32(q.groupSize),
                        data: d.baseAddress,
                        data_bytes: Int64(d.count),
                        scales: s.baseAddress,
                        n_scales: Int64(s.count),
                        zero_points: q.zeroPoints == nil ? nil : z.baseAddress,
                        n_zero_points: Int64(z.count))
                    try check(tbh_weight_create(dev, &desc, &w))  // one-time repack; host arrays not kept
                }
            }
        }
        cache[q.identifier] = w!
        return w!
    }

    // MARK: QuantizedMatMulBackend (Backend.swift:173-175)

    public func matmulQuantized(_ input: Tensor<Float>, _ quantized: QuantizedTensor) throws -> Tensor<Float> {
        precondition(input.shape.dimensions.count == 2, "Input must be 2D")
        precondition(quantized.shape.dimensions.count == 2, "Weights must be 2D")
        precondition(input.shape.dimensions[1] == quantized.shape.dimensions[0], "Dimensions must match")
        let m = input.shape.dimensions[0], k = input.shape.dimensions[1]
        let n = quantized.shape.dimensions[1]
        let w = try weight(quantized)
        let x = hostScalars(input)
        var y = [Float](repeating: 0, count: m * n)
        try x.withUnsafeBufferPointer { xp in
            try y.withUnsafeMutableBufferPointer { yp in
                try check(tbh_matmul(dev, xp.baseAddress, Int64(m), Int64(k), w, yp.baseAddress))
            }
        }
        // Host-resident result: TensorStorage can only sync from an MTLBuffer
        // (TensorStorage.swift:82-97).
        return Tensor<Float>(shape: TensorShape(m, n), data: y)
    }

    /// QuantizedTensor.dequantize() (QuantizedTensor.swift:182-286) of the
    /// uploaded weight, bit-identical, as [K, N].
    public func dequantize(_ quantized: QuantizedTensor) throws -> Tensor<Float> {
        let w = try weight(quantized)
        let k = quantized.shape.dimensions[0], n = quantized.shape.dimensions[1]
        var out = [Float](repeating: 0, count: k * n)
        try out.withUnsafeMutableBufferPointer { op in try check(tbh_dequantize(dev, w, op.baseAddress)) }
        return Tensor<Float>(shape: TensorShape(k, n), data: out)
    }

    // MARK: SoftmaxBackend (Backend.swift:180-186)

    public func softmax(_ input: Tensor<Float>) throws -> Tensor<Float> {
        let count = input.shape.count
        guard count > 0 else { return input }
        let cols = input.shape.dimensions.last!
        var y = [Float](repeating: 0, count: count)
        try hostScalars(input).withUnsafeBufferPointer { x in
            try y.withUnsafeMutableBufferPointer { yp in
                try check(tbh_softmax(dev, x.baseAddress, Int64(count / cols), Int64(cols), yp.baseAddress))
            }
        }
        return Tensor<Float>(shape: input.shape, data: y)
    }

    // MARK: RMSNormBackend (Backend.swift:188-199)

    public func rmsnorm(_ input: Tensor<Float>, weight: Tensor<Float>, eps: Float) throws -> Tensor<Float> {
        precondition(input.shape.dimensions.count == 2, "rmsnorm input must be 2-D [tokens, hidden]")
        let rows = input.shape.dimensions[0], hidden = input.shape.dimensions[1]
        precondition(weight.shape.count == hidden, "weight size must equal hiddenDim")
        var y = [Float](repeating: 0, count: rows * hidden)
        try hostScalars(input).withUnsafeBufferPointer { x in
            try hostScalars(weight).withUnsafeBufferPointer { g in
                try y.withUnsafeMutableBufferPointer { yp in
                    try check(tbh_rmsnorm(dev, x.baseAddress, Int64(rows), Int64(hidden), g.baseAddress, eps,
                                          yp.baseAddress))
                }
            }
        }
        return Tensor<Float>(shape: input.shape, data: y)
    }

    // MARK: ActivationBackend (Backend.swift:222-228)

    public func silu(_ input: Tensor<Float>) throws -> Tensor<Float> {
        let count = input.shape.count
        guard count > 0 else { return input }
        var y = [Float](repeating: 0, count: count)
        try hostScalars(input).withUnsafeBufferPointer { x in
            try y.withUnsafeMutableBufferPointer { yp in
                try check(tbh_silu(dev, x.baseAddress, Int64(count), yp.baseAddress))
            }
        }
        return Tensor<Float>(shape: input.shape, data: y)
    }

    public func gelu(_ input: Tensor<Float>) throws -> Tensor<Float> {
        let count = input.shape.count
        guard count > 0 else { return input }
        var y = [Float](repeating: 0, count: count)
        try hostScalars(input).withUnsafeBufferPointer { x in
            try y.withUnsafeMutableBufferPointer { yp in
                try check(tbh_gelu(dev, x.baseAddress, Int64(count), yp.baseAddress))
            }
        }
        return Tensor<Float>(shape: input.shape, data: y)
    }

    // MARK: AttentionBackend (Backend.swift:201-220)

    public func attention(query: Tensor<Float>, keys: Tensor<Float>, values: Tensor<Float>,
                          mask: Tensor<Float>?, headDim: Int, numHeads: Int, numKVHeads: Int) throws -> Tensor<Float>
    {
        precondition(numHeads >= numKVHeads && numHeads % numKVHeads == 0,
                     "numHeads must be a multiple of numKVHeads")
        let q = query.shape.dimensions, k = keys.shape.dimensions
        var shape = tbh_attention_shape(
            batch: Int64(q.count == 3 ? q[0] : 1),
            seq_len: Int64(q.count == 3 ? q[1] : q[0]),
            kv_len: Int64(k.count == 3 ? k[1] : k[0]),
            head_dim: Int32(headDim),
            num_heads: Int32(numHeads),
            num_kv_heads: Int32(numKVHeads))
        var out = [Float](repeating: 0, count: query.shape.count)
        let maskScalars: [Float]? = mask.map { hostScalars($0) }
        try hostScalars(query).withUnsafeBufferPointer { qp in
            try hostScalars(keys).withUnsafeBufferPointer { kp in
                try hostScalars(values).withUnsafeBufferPointer { vp in
                    try out.withUnsafeMutableBufferPointer { op in
                        if let m = maskScalars {
                            try m.withUnsafeBufferPointer { mp in
                                try check(tbh_attention(dev, &shape, qp.baseAddress, kp.baseAddress, vp.baseAddress,
                                                        mp.baseAddress, op.baseAddress))
                            }
                        } else {
                            try check(tbh_attention(dev, &shape, qp.baseAddress, kp.baseAddress, vp.baseAddress,
                                                    nil, op.baseAddress))
                        }
                    }
                }
            }
        }
        return Tensor<Float>(shape: query.shape, data: out)
    }
}

extension TinyBrainBackend {
    /// Registers a HIPBackend in the slot the runtime dispatches through
    /// (Backend.swift:29), as the umbrella does for Metal
    /// (Sources/TinyBrain/TinyBrain.swift:35-48).  Returns false when no
    /// gfx950 device opens; the runtime then keeps its CPU paths.
    @discardableResult
    public static func enableHIP(ordinal: Int32 = 0) -> Bool {
        guard let backend = try? HIPBackend(ordinal: ordinal) else { return false }
        metalBackend = backend
        return true
    }
}
