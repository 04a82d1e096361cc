// LSampLogitSampler.swift — the single-stream mlx-lm path on the MI355X
// sampling stage: GenerateParameters.sampler() / .processor()
// (Evaluate.swift:328-387) as a LogitSampler + LogitProcessor pair.
//
// The reference applies the processor to the logits (penalties in the logits
// dtype, RepetitionContext / PresencePenaltyContext / FrequencyPenaltyContext,
// Evaluate.swift:586-693) and then the sampler draws (TopPSampler,
// CategoricalSampler, ArgMaxSampler, Evaluate.swift:394-510).  The processor
// keeps the penalty windows (the TokenRing of Evaluate.swift:518-570, on the
// host as distinct ids with flags and counts) and, by default, returns the
// penalized logits from lsamp_penalize, so that any processor after it
// (SampleTests.swift:431-454) sees what the reference's would.  With
// `fusedPenalties` the caller states that nothing follows the processor: it
// returns the logits unchanged and the sampler applies the windows in the
// same pass as the draw (lsamp_sample), one read of the logits instead of
// three.  A sampler without a processor draws from the unpenalized logits,
// as the reference's would.
//
// Shapes: [vocab] or [B, vocab] logits (the reference's processors broadcast
// one window over every row: every row reads the same entries through
// penalty_row_len).  Outputs wrap buffers the pair owns, used in turn (two
// each), so step N's token stays valid while step N + 1 is enqueued.

import CLSamp
import Foundation
import MLX

/// The penalty windows of one generation (GenerateParameters' contexts).
public final class LSampPenaltyWindows {
    let repetitionSize: Int      // 0 = no repetition context
    let presenceSize: Int        // 0 = no presence context
    let frequencySize: Int       // 0 = no frequency context
    var repetition: [Int] = []
    var presence: [Int] = []
    var frequency: [Int] = []

    init(contexts: Int32, parameters p: GenerateParameters) {
        repetitionSize = (contexts & 1) != 0 ? p.repetitionContextSize : 0
        presenceSize = (contexts & 2) != 0 ? p.presenceContextSize : 0
        frequencySize = (contexts & 4) != 0 ? p.frequencyContextSize : 0
    }

    private static func push(_ ring: inout [Int], _ tokens: [Int], _ size: Int) {
        guard size > 0 else { return }
        ring.append(contentsOf: tokens)
        if ring.count > size { ring.removeFirst(ring.count - size) }
    }

    func append(_ tokens: [Int]) {
        Self.push(&repetition, tokens, repetitionSize)
        Self.push(&presence, tokens, presenceSize)
        Self.push(&frequency, tokens, frequencySize)
    }

    /// The windows as lsamp_penalty_entry rows: LSAMP_PEN_REPETITION for ids
    /// in the repetition window, LSAMP_PEN_PRESENCE for ids in the presence
    /// window, count = occurrences in the frequency window.
    func entries() -> [lsamp_penalty_entry] {
        var e = LSampEntries()
        for t in repetition { e.add(t, count: 0, flags: LSAMP_PEN_REPETITION) }
        for t in presence { e.add(t, count: 0, flags: LSAMP_PEN_PRESENCE) }
        for t in frequency { e.add(t, count: 1) }
        return e.entries
    }

    /// FrequencyPenaltyContext subtracts a float32 histogram once its window
    /// holds a token (Evaluate.swift:649-657): 16-bit logits come out float32.
    var promotes: Bool { !frequency.isEmpty }

    func copy() -> LSampPenaltyWindows {
        let c = LSampPenaltyWindows(sizes: (repetitionSize, presenceSize, frequencySize))
        c.repetition = repetition
        c.presence = presence
        c.frequency = frequency
        return c
    }

    private init(sizes: (Int, Int, Int)) {
        (repetitionSize, presenceSize, frequencySize) = sizes
    }
}

/// The device side a generation's sampler and processor share: one
/// lsamp_context (their calls are ordered on the runtime's stream), the
/// resolved row parameters for up to `maxRows` rows, and the windows'
/// entries as every row reads them.
final class LSampSingleStream {
    let runtime: LSampRuntime
    let ctx: LSampContext
    let maxRows: Int
    let row: lsamp_row_params
    let params: LSampDeviceBuffer<lsamp_row_params>   // [maxRows] copies of `row`
    let rowPtr: LSampDeviceBuffer<Int32>              // [maxRows + 1] zeros
    let rowLen: LSampDeviceBuffer<Int32>              // [maxRows]
    let entries: LSampOutputRing<lsamp_penalty_entry>

    init(runtime: LSampRuntime, maxRows: Int, maxVocab: Int32, row: lsamp_row_params,
         maxEntries: Int) {
        self.runtime = runtime
        self.maxRows = maxRows
        self.row = row
        ctx = LSampContext(device: runtime.device, maxRows: Int32(maxRows), maxVocab: maxVocab)
        params = LSampDeviceBuffer(runtime, count: maxRows)
        params.upload([lsamp_row_params](repeating: row, count: maxRows))
        rowPtr = LSampDeviceBuffer(runtime, count: maxRows + 1)
        rowPtr.upload([Int32](repeating: 0, count: maxRows + 1))
        rowLen = LSampDeviceBuffer(runtime, count: maxRows)
        entries = LSampOutputRing(runtime, count: max(maxEntries, 1))
    }

    /// Rows of a [vocab] or [B, vocab] view.
    func rows(_ view: LSampDeviceView) -> Int {
        precondition(view.shape.count == 1 || view.shape.count == 2,
                     "logits must be [vocab] or [B, vocab]")
        let rows = view.shape.count == 2 ? view.shape[0] : 1
        precondition(rows >= 1 && rows <= maxRows, "\(rows) rows; the pair was made for \(maxRows)")
        return rows
    }

    /// The windows' entries on the device, one run read by all `rows` rows
    /// (every row starts at 0 with the same length).
    func upload(_ e: [lsamp_penalty_entry], rows: Int) -> UnsafePointer<lsamp_penalty_entry> {
        let buffer = entries.take(e.count)
        buffer.upload(e)
        rowLen.upload([Int32](repeating: Int32(e.count), count: rows))
        return buffer.pointer
    }
}

/// GenerateParameters.processor(): keeps the windows; `process` returns the
/// penalized logits (lsamp_penalize), or the logits unchanged when the
/// sampler applies the windows itself (`fusedPenalties`).
public struct LSampLogitProcessor: LogitProcessor {
    let windows: LSampPenaltyWindows
    let stage: LSampSingleStream
    let fused: Bool
    let outputs: LSampOutputRing<UInt8>

    init(windows: LSampPenaltyWindows, stage: LSampSingleStream, fused: Bool,
         outputs: LSampOutputRing<UInt8>) {
        self.windows = windows
        self.stage = stage
        self.fused = fused
        self.outputs = outputs
    }

    public mutating func prompt(_ prompt: MLXArray) {
        windows.append(prompt.asArray(Int.self))
    }

    /// PenaltyProcessor.process (Evaluate.swift:666-720): repetition, then
    /// presence, then frequency, in the logits dtype (float32 once the
    /// frequency window holds a token).  A processor whose windows are all
    /// empty returns the logits themselves, as each reference context does.
    public func process(logits: MLXArray) -> MLXArray {
        if fused { return logits }
        let e = windows.entries()
        guard !e.isEmpty else { return logits }
        let view = stage.runtime.deviceView(logits)
        let rows = stage.rows(view)
        let vocab = view.shape.last!
        let outDtype = windows.promotes ? LSAMP_DTYPE_F32 : view.dtype
        let width = outDtype == LSAMP_DTYPE_F32 ? 4 : 2
        let out = outputs.take(rows * vocab * width)
        var a = lsamp_penalize_args()
        a.rows = Int32(rows)
        a.vocab = Int32(vocab)
        a.dtype = Int32(view.dtype.rawValue)
        a.row_stride = view.rowStride
        a.logits = view.pointer
        a.params = stage.params.pointer
        a.penalty_row_ptr = stage.rowPtr.pointer
        a.penalty_row_len = stage.rowLen.pointer
        a.penalty_entries = stage.upload(e, rows: rows)
        a.out_dtype = Int32(outDtype.rawValue)
        a.out = out.raw
        lsampCheck(lsamp_penalize(stage.ctx.handle, &a, stage.runtime.stream))
        return stage.runtime.logitsArray(out.raw, dtype: outDtype, shape: view.shape)
    }

    /// The windows advance on the host: the token is read back here (the
    /// single-stream iterator reads every token to emit it).
    public mutating func didSample(token: MLXArray) {
        windows.append(token.asArray(Int.self))
    }

    public mutating func didEmit(token: Int) {}
    public mutating func finalizeGeneration() {}

    /// An independent processor: its own windows and output buffers, the
    /// same device context (calls stay ordered on the runtime's stream).  A
    /// copy is never fused: the sampler applies only the original's windows.
    public func copy() -> LSampLogitProcessor {
        LSampLogitProcessor(windows: windows.copy(), stage: stage, fused: false,
                            outputs: LSampOutputRing(stage.runtime, count: 1))
    }
}

/// GenerateParameters.sampler(), with the processor's penalties fused in
/// when the pair was made with `fusedPenalties`.
public final class LSampLogitSampler: LogitSampler {
    let stage: LSampSingleStream
    let windows: LSampPenaltyWindows?   // set only for a fused pair
    let uniforms: LSampOutputRing<Float>
    let tokens: LSampOutputRing<Int32>
    var uniformSource: () -> Float

    /// The sampler and its processor for `parameters`, resolved by the
    /// reference's factory rules (lsamp_resolve_generate_parameters).  The
    /// processor is nil where GenerateParameters.processor() returns nil.
    /// `fusedPenalties`: no other processor runs between this processor and
    /// the sampler, so the penalties may be applied inside the draw.
    public static func make(
        parameters p: GenerateParameters, runtime: LSampRuntime, maxVocab: Int32,
        maxRows: Int = 1, fusedPenalties: Bool = false,
        uniform: @escaping () -> Float = { Float.random(in: 0 ..< 1) }
    ) -> (sampler: LSampLogitSampler, processor: LSampLogitProcessor?) {
        var gp = lsamp_generate_parameters()
        gp.temperature = p.temperature
        gp.top_p = p.topP
        gp.top_k = Int32(p.topK)
        gp.min_p = p.minP
        if let r = p.repetitionPenalty {
            gp.has_repetition_penalty = 1
            gp.repetition_penalty = r
        }
        gp.repetition_context_size = Int32(p.repetitionContextSize)
        if let v = p.presencePenalty {
            gp.has_presence_penalty = 1
            gp.presence_penalty = v
        }
        gp.presence_context_size = Int32(p.presenceContextSize)
        if let v = p.frequencyPenalty {
            gp.has_frequency_penalty = 1
            gp.frequency_penalty = v
        }
        gp.frequency_context_size = Int32(p.frequencyContextSize)
        var row = lsamp_row_params()
        var contexts: Int32 = 0
        lsampCheck(lsamp_resolve_generate_parameters(&gp, &row, &contexts))
        let windows = contexts != 0 ? LSampPenaltyWindows(contexts: contexts, parameters: p) : nil
        let maxEntries = p.repetitionContextSize + p.presenceContextSize + p.frequencyContextSize
        let stage = LSampSingleStream(runtime: runtime, maxRows: maxRows, maxVocab: maxVocab,
                                      row: row, maxEntries: maxEntries)
        let sampler = LSampLogitSampler(
            stage: stage, windows: fusedPenalties ? windows : nil, uniform: uniform)
        let processor = windows.map {
            LSampLogitProcessor(windows: $0, stage: stage, fused: fusedPenalties,
                                outputs: LSampOutputRing(runtime, count: 1))
        }
        return (sampler, processor)
    }

    init(stage: LSampSingleStream, windows: LSampPenaltyWindows?, uniform: @escaping () -> Float) {
        self.stage = stage
        self.windows = windows
        self.uniformSource = uniform
        uniforms = LSampOutputRing(stage.runtime, count: stage.maxRows)
        tokens = LSampOutputRing(stage.runtime, count: stage.maxRows)
    }

    /// LogitSampler.sample(logits:): [vocab] logits give a scalar token,
    /// [B, vocab] logits [B] tokens (int32, on the device; no host
    /// synchronization here).
    public func sample(logits: MLXArray) -> MLXArray {
        let view = stage.runtime.deviceView(logits)
        let rows = stage.rows(view)
        let u = uniforms.take(rows)
        u.upload((0 ..< rows).map { _ in uniformSource() })
        let out = tokens.take(rows)
        var hostRows = [lsamp_row_params](repeating: stage.row, count: rows)
        var a = lsamp_sample_args()
        a.semantics = Int32(LSAMP_SEM_MLXLM.rawValue)
        a.rows = Int32(rows)
        a.vocab = Int32(view.shape.last!)
        a.dtype = Int32(view.dtype.rawValue)
        a.row_stride = view.rowStride
        a.logits = view.pointer
        a.params = stage.params.pointer
        if let e = windows?.entries(), !e.isEmpty {
            a.penalty_row_ptr = stage.rowPtr.pointer
            a.penalty_row_len = stage.rowLen.pointer
            a.penalty_entries = stage.upload(e, rows: rows)
        }
        a.uniforms = u.pointer
        a.tokens = out.mutablePointer
        hostRows.withUnsafeMutableBufferPointer { hp in
            a.params_host = UnsafePointer(hp.baseAddress)
            lsampCheck(lsamp_sample(stage.ctx.handle, &a, stage.runtime.stream))
        }
        let shape = view.shape.count == 2 ? [rows] : []
        return stage.runtime.int32Array(out.raw, shape: shape)
    }
}
