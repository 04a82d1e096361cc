// LSampLogitSampler.swift — the single-stream mlx-lm path on the MI355X
// sampling stage: GenerateParameters.sampler() / .processor()
// (Evaluate.swift:328-387) as a LogitSampler + LogitProcessor pair over one
// fused device call.
//
// The reference applies the processor to the logits (penalties in the logits
// dtype, RepetitionContext / PresencePenaltyContext / FrequencyPenaltyContext,
// Evaluate.swift:586-693) and then the sampler draws (TopPSampler,
// CategoricalSampler, ArgMaxSampler, Evaluate.swift:394-510).  lsamp_sample
// does both in one pass over the logits, in that order, so the pair shares
// one state object: the processor keeps the penalty windows (the TokenRing
// of Evaluate.swift:518-570, on the host as distinct ids with flags and
// counts) and returns the logits unchanged; the sampler passes the windows
// to the device with the draw.  A sampler without a processor draws from the
// unpenalized logits, as the reference's would.

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

/// GenerateParameters.processor(): keeps the windows; the device applies them.
public struct LSampLogitProcessor: LogitProcessor {
    let windows: LSampPenaltyWindows

    public mutating func prompt(_ prompt: MLXArray) {
        windows.append(prompt.asArray(Int.self))
    }

    /// Unchanged: the penalties are applied by LSampLogitSampler in the same
    /// pass as the draw.
    public func process(logits: MLXArray) -> MLXArray { logits }

    /// The windows advance on the host: the token is read back here (the
    /// single-stream iterator reads every token to emit it).
    public mutating func didSample(token: MLXArray) {
        windows.append(token.asArray(Int.self))
    }

    public mutating func didEmit(token: Int) {}
    public mutating func finalizeGeneration() {}

    public func copy() -> LSampLogitProcessor {
        LSampLogitProcessor(windows: windows.copy())
    }
}

/// GenerateParameters.sampler() with the processor's penalties fused in.
public final class LSampLogitSampler: LogitSampler {
    let runtime: LSampRuntime
    let ctx: LSampContext
    let row: lsamp_row_params
    let windows: LSampPenaltyWindows?
    let maxEntries: Int
    let devParams: LSampDeviceBuffer<lsamp_row_params>
    let devRowPtr: LSampDeviceBuffer<Int32>
    let devEntries: LSampDeviceBuffer<lsamp_penalty_entry>
    let devUniform: LSampDeviceBuffer<Float>
    let devTokens: LSampDeviceBuffer<Int32>
    var uniformSource: () -> Float

    /// The sampler and its processor for `parameters`, resolved by the
    /// reference's factory rules (lsamp_resolve_generate_parameters).  The
    /// processor is nil where GenerateParameters.processor() returns nil.
    public static func make(
        parameters p: GenerateParameters, runtime: LSampRuntime, maxVocab: Int32,
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
        let sampler = LSampLogitSampler(
            runtime: runtime, maxVocab: maxVocab, row: row, windows: windows,
            maxEntries: maxEntries, uniform: uniform)
        return (sampler, windows.map { LSampLogitProcessor(windows: $0) })
    }

    init(runtime: LSampRuntime, maxVocab: Int32, row: lsamp_row_params,
         windows: LSampPenaltyWindows?, maxEntries: Int, uniform: @escaping () -> Float) {
        self.runtime = runtime
        self.ctx = LSampContext(device: runtime.device, maxRows: 1, maxVocab: maxVocab)
        self.row = row
        self.windows = windows
        self.maxEntries = max(maxEntries, 1)
        self.uniformSource = uniform
        devParams = LSampDeviceBuffer(runtime, count: 1)
        devRowPtr = LSampDeviceBuffer(runtime, count: 2)
        devEntries = LSampDeviceBuffer(runtime, count: self.maxEntries)
        devUniform = LSampDeviceBuffer(runtime, count: 1)
        devTokens = LSampDeviceBuffer(runtime, count: 1)
        devParams.upload([row])
    }

    /// LogitSampler.sample(logits:): [1, vocab] (or [vocab]) logits in; the
    /// [1] int32 token out, on the device (no host synchronization here).
    public func sample(logits: MLXArray) -> MLXArray {
        let view = runtime.deviceView(logits)
        let entries = windows?.entries() ?? []
        devRowPtr.upload([0, Int32(entries.count)])
        devEntries.upload(entries)
        devUniform.upload([uniformSource()])
        var hostRow = row
        var a = lsamp_sample_args()
        a.semantics = Int32(LSAMP_SEM_MLXLM.rawValue)
        a.rows = 1
        a.vocab = Int32(view.shape.last!)
        a.dtype = Int32(view.dtype.rawValue)
        a.row_stride = view.rowStride
        a.logits = view.pointer
        a.params = devParams.pointer
        a.penalty_row_ptr = devRowPtr.pointer
        a.penalty_entries = devEntries.pointer
        a.uniforms = devUniform.pointer
        a.tokens = devTokens.mutablePointer
        withUnsafePointer(to: &hostRow) { hp in
            a.params_host = hp
            lsampCheck(lsamp_sample(ctx.handle, &a, runtime.stream))
        }
        return runtime.int32Array(devTokens.raw, shape: [1])
    }
}
