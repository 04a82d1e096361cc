// LSampStepSampler.swift — the batched CBv2 path on the MI355X sampling
// stage: a CBv2StepSampler (EngineLoopV2.swift:91-239) whose every draw is
// one lsamp_step call (CBv2DefaultSampler.sample, DefaultSamplerV2.swift:
// 84-181: draw, penalty commit, raw log-probabilities) and whose MTP verify
// entry points are lsamp_verify (DefaultSamplerV2.swift:310-580).
//
// State, as the reference keeps it (LogitsPipelineV2.swift:127-141, 357-384):
// each configured row's output counts and repetition window live in a device
// penalty table that lsamp_step updates after every draw, so a chained step
// (`pendingSampledTokens`) is already folded in on the device and no step
// reads anything back.  The table is rebuilt from `rowContext()` (prompt and
// confirmed outputs) whenever the batch's membership changes, plus the
// pending tokens committed once more on the device.  RNG: each row draws its
// uniform from the Philox key mix(seed, requestID, step) (SamplerV2.swift:
// 183-191, lsamp_rng_key), its step advancing by one per draw.

import CLSamp
import Foundation
import MLX

public final class LSampStepSampler: CBv2StepSampler {
    let runtime: LSampRuntime
    let ctx: LSampContext
    let maxRows: Int
    let vocab: Int32
    let capacity: Int32          // penalty entries per row
    let windowCapacity: Int32    // repetition ring slots per row
    let fallbackSeed: UInt64

    // configured batch
    var configuredIDs: [CBv2RequestID] = []
    var seeds: [UInt64] = []
    var steps: [UInt64] = []
    var rowParams: [lsamp_row_params] = []
    var pendingLogprobs: CBv2StepLogprobs?

    // device buffers (allocated once for maxRows)
    let devParams: LSampDeviceBuffer<lsamp_row_params>
    let devKeys: LSampDeviceBuffer<UInt64>
    let devTokens: LSampDeviceBuffer<Int32>
    let devFlags: LSampDeviceBuffer<UInt32>
    let devRowPtr: LSampDeviceBuffer<Int32>
    let devEntries: LSampDeviceBuffer<lsamp_penalty_entry>
    let devRowLen: LSampDeviceBuffer<Int32>
    let devWindowCount: LSampDeviceBuffer<Int32>
    let devWindow: LSampDeviceBuffer<Int32>
    let devRingPos: LSampDeviceBuffer<Int32>
    let devWindowSize: LSampDeviceBuffer<Int32>
    let devMode: LSampDeviceBuffer<UInt32>
    let devChosen: LSampDeviceBuffer<Float>
    let devTopValues: LSampDeviceBuffer<Float>
    let devTopIDs: LSampDeviceBuffer<Int32>
    static let maxTopLogprobs = 32

    public init(runtime: LSampRuntime, maxRows: Int, vocab: Int32, capacity: Int32,
                windowCapacity: Int32 = 64, fallbackSeed: UInt64 = 0) {
        self.runtime = runtime
        self.maxRows = maxRows
        self.vocab = vocab
        self.capacity = capacity
        self.windowCapacity = windowCapacity
        self.fallbackSeed = fallbackSeed
        ctx = LSampContext(device: runtime.device, maxRows: Int32(maxRows), maxVocab: vocab)
        devParams = LSampDeviceBuffer(runtime, count: maxRows)
        devKeys = LSampDeviceBuffer(runtime, count: maxRows)
        devTokens = LSampDeviceBuffer(runtime, count: maxRows)
        devFlags = LSampDeviceBuffer(runtime, count: maxRows)
        devRowPtr = LSampDeviceBuffer(runtime, count: maxRows + 1)
        devEntries = LSampDeviceBuffer(runtime, count: maxRows * Int(capacity))
        devRowLen = LSampDeviceBuffer(runtime, count: maxRows)
        devWindowCount = LSampDeviceBuffer(runtime, count: maxRows * Int(capacity))
        devWindow = LSampDeviceBuffer(runtime, count: maxRows * Int(windowCapacity))
        devRingPos = LSampDeviceBuffer(runtime, count: maxRows)
        devWindowSize = LSampDeviceBuffer(runtime, count: maxRows)
        devMode = LSampDeviceBuffer(runtime, count: maxRows)
        devChosen = LSampDeviceBuffer(runtime, count: maxRows)
        devTopValues = LSampDeviceBuffer(runtime, count: maxRows * Self.maxTopLogprobs)
        devTopIDs = LSampDeviceBuffer(runtime, count: maxRows * Self.maxTopLogprobs)
    }

    // MARK: - capabilities

    public var supportsMTPTargetPrefix: Bool { true }
    public var supportsMTPPenaltyVerification: Bool { true }

    // MARK: - configuration

    static func resolve(_ p: CBv2SamplingParams, vocab: Int32) -> lsamp_row_params {
        var sp = lsamp_cbv2_params()
        sp.temperature = p.temperature
        sp.top_p = p.topP
        sp.top_k = Int32(p.topK)
        sp.min_p = p.minP
        sp.repetition_penalty = p.repetitionPenalty
        sp.repetition_context_size = Int32(p.repetitionContextSize)
        sp.frequency_penalty = p.frequencyPenalty
        sp.presence_penalty = p.presencePenalty
        var row = lsamp_row_params()
        lsampCheck(lsamp_resolve_cbv2_params(&sp, vocab, &row))
        return row
    }

    var table: lsamp_penalty_table {
        var t = lsamp_penalty_table()
        t.rows = Int32(configuredIDs.count)
        t.capacity = capacity
        t.window_capacity = windowCapacity
        t.entries = devEntries.mutablePointer
        t.row_len = devRowLen.mutablePointer
        t.window_count = devWindowCount.mutablePointer
        t.window = devWindow.mutablePointer
        t.ring_pos = devRingPos.mutablePointer
        t.window_size = devWindowSize.pointer
        t.mode = devMode.pointer
        return t
    }

    /// Rebuild the batch's state from the confirmed history (membership
    /// change), then fold in the pending chained tokens on the device.
    func configure(_ rows: [CBv2SamplerRow], pending: MLXArray?) {
        precondition(rows.count <= maxRows, "batch larger than the sampler was made for")
        configuredIDs = rows.map(\.id)
        seeds = rows.map { $0.params.seed ?? fallbackSeed }
        steps = rows.map { UInt64($0.outputTokens.count) }
        rowParams = rows.map { Self.resolve($0.params, vocab: vocab) }
        var entries = [lsamp_penalty_entry](
            repeating: lsamp_penalty_entry(), count: rows.count * Int(capacity))
        var rowLen = [Int32](repeating: 0, count: rows.count)
        var windowCount = [Int32](repeating: 0, count: rows.count * Int(capacity))
        var window = [Int32](repeating: -1, count: rows.count * Int(windowCapacity))
        var ringPos = [Int32](repeating: 0, count: rows.count)
        var windowSize = [Int32](repeating: 1, count: rows.count)
        var mode = [UInt32](repeating: 0, count: rows.count)
        for (r, row) in rows.enumerated() {
            let p = row.params
            let reps = p.repetitionPenalty != 1 && p.repetitionContextSize > 0
            let counts = p.frequencyPenalty != 0 || p.presencePenalty != 0
            mode[r] = (counts ? LSAMP_STATE_COUNTS : 0) | (reps ? LSAMP_STATE_REPETITION : 0)
            windowSize[r] = Int32(min(max(p.repetitionContextSize, 1), Int(windowCapacity)))
            var e = LSampEntries()
            for (t, b) in p.logitBias { e.add(t, count: 0, bias: b) }
            if counts { for t in row.outputTokens { e.add(t) } }
            // the repetition window: the last tokens of prompt + outputs
            let history = row.promptTokens + row.outputTokens
            let w = reps ? Array(history.suffix(Int(windowSize[r]))) : []
            for t in w { e.add(t, count: 0, flags: LSAMP_PEN_REPETITION) }
            precondition(e.entries.count <= Int(capacity), "row history exceeds the table capacity")
            for (i, ent) in e.entries.enumerated() {
                entries[r * Int(capacity) + i] = ent
                windowCount[r * Int(capacity) + i] = Int32(w.filter { $0 == Int(ent.token) }.count)
            }
            rowLen[r] = Int32(e.entries.count)
            for (i, t) in w.enumerated() { window[r * Int(windowCapacity) + i] = Int32(t) }
            ringPos[r] = Int32(w.count) % windowSize[r]
        }
        devParams.upload(rowParams)
        devRowPtr.upload((0 ... rows.count).map { Int32($0) * capacity })
        devEntries.upload(entries)
        devRowLen.upload(rowLen)
        devWindowCount.upload(windowCount)
        devWindow.upload(window)
        devRingPos.upload(ringPos)
        devWindowSize.upload(windowSize)
        devMode.upload(mode)
        if let pending {
            // the chained step's tokens, committed into the rebuilt state
            var c = lsamp_commit_args()
            c.table = table
            c.vocab = vocab
            let view = runtime.deviceView(pending)
            c.tokens = view.pointer.assumingMemoryBound(to: Int32.self)
            lsampCheck(lsamp_commit(ctx.handle, &c, runtime.stream))
            for i in steps.indices { steps[i] += 1 }
        }
    }

    // MARK: - the draw

    public func sample(
        logits: MLXArray, params: [CBv2SamplingParams], requestIDs: [CBv2RequestID],
        stepIndex: Int, pendingSampledTokens: MLXArray?,
        rowContext: () -> [CBv2SamplerRow]
    ) -> MLXArray {
        if requestIDs != configuredIDs {
            configure(rowContext(), pending: pendingSampledTokens)
        }
        let rows = requestIDs.count
        devKeys.upload((0 ..< rows).map { lsamp_rng_key(seeds[$0], requestIDs[$0].raw, steps[$0]) })
        let view = runtime.deviceView(logits)
        let topK = min(params.map(\.topLogprobs).max() ?? 0, Self.maxTopLogprobs)

        var st = lsamp_step_args()
        st.sample.semantics = Int32(LSAMP_SEM_CBV2.rawValue)
        st.sample.rows = Int32(rows)
        st.sample.vocab = Int32(view.shape.last!)
        st.sample.dtype = Int32(view.dtype.rawValue)
        st.sample.row_stride = view.rowStride
        st.sample.logits = view.pointer
        st.sample.params = devParams.pointer
        st.sample.penalty_row_ptr = devRowPtr.pointer
        st.sample.penalty_entries = devEntries.pointer
        st.sample.penalty_row_len = devRowLen.pointer
        st.sample.philox_keys = devKeys.pointer
        st.sample.tokens = devTokens.mutablePointer
        st.sample.row_flags = devFlags.mutablePointer
        st.logprobs_top_k = topK > 0 ? Int32(topK) : -1
        st.chosen_logprob = devChosen.mutablePointer
        st.top_logprobs = devTopValues.mutablePointer
        st.top_ids = devTopIDs.mutablePointer
        var t = table
        rowParams.withUnsafeBufferPointer { hostParams in
            st.sample.params_host = hostParams.baseAddress
            withUnsafePointer(to: &t) { tp in
                st.table = tp
                lsampCheck(lsamp_step(ctx.handle, &st, runtime.stream))
            }
        }
        for i in steps.indices { steps[i] += 1 }
        pendingLogprobs = topK > 0
            ? CBv2StepLogprobs(
                rows: requestIDs, topLogprobsPerRow: params.map(\.topLogprobs),
                gathered: CBv2Logprobs.Gathered(
                    chosen: runtime.float32Array(devChosen.raw, shape: [rows]),
                    topValues: runtime.float32Array(devTopValues.raw, shape: [rows, topK]),
                    topIndices: runtime.int32Array(devTopIDs.raw, shape: [rows, topK])))
            : nil
        return runtime.int32Array(devTokens.raw, shape: [rows])
    }

    public func takeStepLogprobs() -> CBv2StepLogprobs? {
        defer { pendingLogprobs = nil }
        return pendingLogprobs
    }

    public func requestDidFinish(_ id: CBv2RequestID) {
        if configuredIDs.contains(id) { configuredIDs = [] }
    }

    public func mtpRoundDidCommit(requestIDs: [CBv2RequestID]) {
        configuredIDs = []
    }

    // MARK: - MTP verification

    /// uniforms[r, j]: the draw of output index stepBases[r] + j, keyed as
    /// the ordinary path keys it (SamplerV2.verifyExponentialNoise).
    func verifyUniforms(_ params: [CBv2SamplingParams], _ ids: [CBv2RequestID],
                        _ stepBases: [Int], window: Int) -> [Float] {
        var u = [Float]()
        u.reserveCapacity(ids.count * window)
        for r in ids.indices {
            let seed = params[r].seed ?? fallbackSeed
            for j in 0 ..< window {
                u.append(lsamp_rng_uniform(lsamp_rng_key(seed, ids[r].raw, UInt64(stepBases[r] + j)), 0))
            }
        }
        return u
    }

    func verify(mode: lsamp_verify_mode, logits: MLXArray, draftIDs: MLXArray?, delta: Float,
                params: [CBv2SamplingParams], requestIDs: [CBv2RequestID], stepBases: [Int],
                penalties: CBv2MTPVerifyPenalties?) -> (tokens: MLXArray, accept: MLXArray?) {
        let view = runtime.deviceView(logits)        // [S, W, V]
        let S = view.shape[0], W = view.shape[1]
        let uniforms = LSampDeviceBuffer<Float>(runtime, count: S * W)
        uniforms.upload(verifyUniforms(params, requestIDs, stepBases, window: W))
        let vparams = LSampDeviceBuffer<lsamp_row_params>(runtime, count: S)
        vparams.upload(params.map { Self.resolve($0, vocab: vocab) })
        let tokens = LSampDeviceBuffer<Int32>(runtime, count: S * W)
        let accepted = LSampDeviceBuffer<Int32>(runtime, count: S)
        let D = max(W - 1, 1)
        let accept = LSampDeviceBuffer<UInt8>(runtime, count: S * D)

        var a = lsamp_verify_args()
        a.mode = Int32(mode.rawValue)
        a.sequences = Int32(S)
        a.window = Int32(W)
        a.vocab = Int32(view.shape[2])
        a.dtype = Int32(view.dtype.rawValue)
        a.target_logits = view.pointer
        a.params = vparams.pointer
        a.uniforms = uniforms.pointer
        a.typical_delta = delta
        a.accepted = accepted.mutablePointer
        a.tokens = tokens.mutablePointer
        if let draftIDs { a.draft_tokens = runtime.deviceView(draftIDs).pointer.assumingMemoryBound(to: Int32.self) }
        a.accept_mask = draftIDs != nil ? accept.mutablePointer : nil

        // penalized windows: each sequence's confirmed output counts, and the
        // round's drafts before each position (CBv2MTPVerifyPenalties)
        var pen: (ptr: LSampDeviceBuffer<Int32>, ent: LSampDeviceBuffer<lsamp_penalty_entry>,
                  scratch: LSampDeviceBuffer<lsamp_penalty_entry>)?
        if let penalties {
            var rowPtr: [Int32] = [0]
            var all: [lsamp_penalty_entry] = []
            for r in 0 ..< S {
                var e = LSampEntries()
                for t in penalties.outputTokens[r] { e.add(t) }
                all.append(contentsOf: e.entries)
                rowPtr.append(Int32(all.count))
            }
            let longest = (0 ..< S).map { Int(rowPtr[$0 + 1] - rowPtr[$0]) }.max() ?? 0
            let drafts = penalties.drafts.map { runtime.deviceView($0) }
            let cap = longest + penalties.columnOffset + W
            let p = (ptr: LSampDeviceBuffer<Int32>(runtime, count: S + 1),
                     ent: LSampDeviceBuffer<lsamp_penalty_entry>(runtime, count: all.count),
                     scratch: LSampDeviceBuffer<lsamp_penalty_entry>(runtime, count: S * W * cap))
            p.ptr.upload(rowPtr)
            p.ent.upload(all)
            a.penalty_row_ptr = p.ptr.pointer
            a.penalty_entries = p.ent.pointer
            if let drafts {
                a.penalty_drafts = drafts.pointer.assumingMemoryBound(to: Int32.self)
                a.penalty_drafts_stride = Int32(drafts.rowStride)
            }
            a.penalty_column_offset = Int32(penalties.columnOffset)
            a.penalty_scratch = p.scratch.mutablePointer
            a.penalty_scratch_cap = Int32(cap)
            pen = p
        }
        lsampCheck(lsamp_verify(ctx.handle, &a, runtime.stream))
        // (the buffers are released once the arrays wrapping them are consumed:
        // the runtime keeps them alive with the arrays it returns)
        _ = pen
        return (runtime.int32Array(tokens.raw, shape: [S, W]),
                draftIDs != nil ? runtime.boolArray(accept.raw, shape: [S, D]) : nil)
    }

    public func mtpVerifySample(
        logits: MLXArray, params: [CBv2SamplingParams],
        requestIDs: [CBv2RequestID], stepBases: [Int]
    ) -> MLXArray? {
        verify(mode: LSAMP_VERIFY_EXACT, logits: logits, draftIDs: nil, delta: 0, params: params,
               requestIDs: requestIDs, stepBases: stepBases, penalties: nil).tokens
    }

    public func mtpVerifyTypical(
        logits: MLXArray, draftIDs: MLXArray, delta: Float,
        params: [CBv2SamplingParams], requestIDs: [CBv2RequestID], stepBases: [Int]
    ) -> (tokens: MLXArray, accept: MLXArray)? {
        let r = verify(mode: LSAMP_VERIFY_TYPICAL, logits: logits, draftIDs: draftIDs, delta: delta,
                       params: params, requestIDs: requestIDs, stepBases: stepBases, penalties: nil)
        return (r.tokens, r.accept!)
    }

    public func mtpVerifySample(
        logits: MLXArray, params: [CBv2SamplingParams],
        requestIDs: [CBv2RequestID], stepBases: [Int], penalties: CBv2MTPVerifyPenalties?
    ) -> MLXArray? {
        verify(mode: LSAMP_VERIFY_EXACT, logits: logits, draftIDs: nil, delta: 0, params: params,
               requestIDs: requestIDs, stepBases: stepBases, penalties: penalties).tokens
    }

    public func mtpVerifyTypical(
        logits: MLXArray, draftIDs: MLXArray, delta: Float,
        params: [CBv2SamplingParams], requestIDs: [CBv2RequestID], stepBases: [Int],
        penalties: CBv2MTPVerifyPenalties?
    ) -> (tokens: MLXArray, accept: MLXArray)? {
        // (with penalty entries, lsamp_verify accepts the rows that carry a
        // presence or frequency penalty exactly, as the reference does)
        let r = verify(mode: LSAMP_VERIFY_TYPICAL, logits: logits, draftIDs: draftIDs, delta: delta,
                       params: params, requestIDs: requestIDs, stepBases: stepBases,
                       penalties: penalties)
        return (r.tokens, r.accept!)
    }
}
