// LSampRuntime.swift — what the MI355X sampling stage needs from the HIP
// runtime that produced the logits, and the small device-side helpers the
// conformers share.
//
// The reference's sampler protocols carry `MLXArray`s (Evaluate.swift:11-57,
// EngineLoopV2.swift:91-239).  On an MI355X deployment the arrays live in HIP
// device memory, owned by the model runtime; `LSampRuntime` is the one place
// that knows how to see such an array as a device pointer and how to wrap a
// device buffer back into an array, so the conformers below stay independent
// of that runtime.  Nothing here synchronizes with the host: every call is
// enqueued on the runtime's stream.

import CLSamp
import Foundation
import MLX

/// A [rows, vocab] (or [rows, window, vocab]) logits tensor in HIP device memory.
public struct LSampDeviceView {
    public var pointer: UnsafeRawPointer
    public var dtype: lsamp_dtype     // LSAMP_DTYPE_BF16 / F16 / F32
    public var shape: [Int]
    /// Elements between consecutive rows (the last dimension's stride).
    public var rowStride: Int64

    public init(pointer: UnsafeRawPointer, dtype: lsamp_dtype, shape: [Int], rowStride: Int64) {
        self.pointer = pointer
        self.dtype = dtype
        self.shape = shape
        self.rowStride = rowStride
    }
}

/// The HIP model runtime, as the sampling stage sees it.
public protocol LSampRuntime: AnyObject {
    /// The HIP device of the arrays.
    var device: Int32 { get }
    /// The hipStream_t on which the model's work is enqueued.
    var stream: UnsafeMutableRawPointer? { get }
    /// The device view of a logits array (no copy).
    func deviceView(_ array: MLXArray) -> LSampDeviceView
    /// Device memory for the adapter's own buffers (allocated once, reused).
    func allocate(bytes: Int) -> UnsafeMutableRawPointer
    /// Release memory from `allocate`, ordered on `stream` (as hipFreeAsync
    /// is): work already enqueued there may still read or write it.
    func free(_ pointer: UnsafeMutableRawPointer)
    /// Copy host bytes to device memory, ordered on `stream`.
    func upload(_ source: UnsafeRawPointer, to destination: UnsafeMutableRawPointer, bytes: Int)
    /// Copy device bytes to device memory, ordered on `stream`.
    func copyDevice(_ source: UnsafeRawPointer, to destination: UnsafeMutableRawPointer, bytes: Int)
    /// Arrays of the runtime over device buffers (no copy; the buffer must
    /// stay valid until the array has been consumed).
    func int32Array(_ pointer: UnsafeMutableRawPointer, shape: [Int]) -> MLXArray
    func float32Array(_ pointer: UnsafeMutableRawPointer, shape: [Int]) -> MLXArray
    func boolArray(_ pointer: UnsafeMutableRawPointer, shape: [Int]) -> MLXArray
    /// A logits array of `dtype` (bfloat16, float16 or float32) over a
    /// device buffer (no copy).
    func logitsArray(_ pointer: UnsafeMutableRawPointer, dtype: lsamp_dtype, shape: [Int]) -> MLXArray
}

/// A status check with the library's last error message (the xgrammar C ABI
/// convention, xgrammar_c.h:55-69).
@inline(__always)
func lsampCheck(_ status: lsamp_status, _ what: StaticString = #function) {
    precondition(status == LSAMP_OK, "\(what): \(String(cString: lsamp_last_error()))")
}

/// One lsamp_context: the device workspace for up to `maxRows` rows of up to
/// `maxVocab` logits.  Calls on one context must be ordered on one stream.
public final class LSampContext {
    public let handle: OpaquePointer

    public init(device: Int32, maxRows: Int32, maxVocab: Int32) {
        var h: OpaquePointer?
        lsampCheck(lsamp_context_create(device, maxRows, maxVocab, &h))
        handle = h!
    }

    deinit { lsamp_context_destroy(handle) }
}

/// A fixed-size device buffer of `count` values of T, owned by the adapter.
final class LSampDeviceBuffer<T> {
    let runtime: LSampRuntime
    let count: Int
    let raw: UnsafeMutableRawPointer

    init(_ runtime: LSampRuntime, count: Int) {
        self.runtime = runtime
        self.count = max(count, 1)
        raw = runtime.allocate(bytes: self.count * MemoryLayout<T>.stride)
    }

    var pointer: UnsafePointer<T> { UnsafePointer(raw.assumingMemoryBound(to: T.self)) }
    var mutablePointer: UnsafeMutablePointer<T> { raw.assumingMemoryBound(to: T.self) }

    /// Upload `values` (at most `count`) to the start of the buffer.
    func upload(_ values: [T]) {
        precondition(values.count <= count, "device buffer too small")
        guard !values.isEmpty else { return }
        values.withUnsafeBytes { bytes in
            runtime.upload(bytes.baseAddress!, to: raw, bytes: bytes.count)
        }
    }

    deinit { runtime.free(raw) }
}

/// A device buffer that grows on demand: a larger request replaces it (the
/// old memory is released through the runtime's stream-ordered free).
final class LSampGrowingBuffer<T> {
    let runtime: LSampRuntime
    private(set) var buffer: LSampDeviceBuffer<T>

    init(_ runtime: LSampRuntime, count: Int) {
        self.runtime = runtime
        buffer = LSampDeviceBuffer(runtime, count: count)
    }

    /// The buffer, at least `count` values long.
    func reserve(_ count: Int) -> LSampDeviceBuffer<T> {
        if count > buffer.count { buffer = LSampDeviceBuffer(runtime, count: max(count, 2 * buffer.count)) }
        return buffer
    }
}

/// Output buffers used in turn, so that a step's outputs stay valid while
/// the next step runs (chained decode reads step N's tokens after step N+1
/// has been enqueued).
final class LSampOutputRing<T> {
    private let slots: [LSampGrowingBuffer<T>]
    private var next = 0

    init(_ runtime: LSampRuntime, count: Int, depth: Int = 2) {
        slots = (0 ..< depth).map { _ in LSampGrowingBuffer<T>(runtime, count: count) }
    }

    /// The next buffer in turn, at least `count` values long (a larger
    /// request grows that slot).
    func take(_ count: Int = 0) -> LSampDeviceBuffer<T> {
        defer { next = (next + 1) % slots.count }
        return slots[next].reserve(count)
    }
}

/// Sparse penalty entries of one row: its distinct tokens with their counts
/// (`lsamp_penalty_entry`), in the order the counts were first seen.
struct LSampEntries {
    var index: [Int: Int] = [:]
    var entries: [lsamp_penalty_entry] = []

    mutating func add(_ token: Int, count: Int32 = 1, flags: UInt32 = 0, bias: Float = 0) {
        if let i = index[token] {
            entries[i].count += count
            entries[i].flags |= flags
            entries[i].bias += bias
        } else {
            index[token] = entries.count
            var e = lsamp_penalty_entry()
            e.token = Int32(token)
            e.count = count
            e.flags = flags
            e.bias = bias
            entries.append(e)
        }
    }
}
