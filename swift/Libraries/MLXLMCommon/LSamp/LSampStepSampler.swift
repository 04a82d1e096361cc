// LSampStepSampler.swift — the batched CBv2 path on the MI355X sampling
// stage: a CBv2StepSampler (EngineLoopV2.swift:91-239) whose every draw is
// one lsamp_step call (CBv2DefaultSampler.sample, DefaultSamplerV2.swift:
// 84-181: draw, penalty commit, raw log-probabilities), whose grammar masks
// are assembled on the device (lsamp_mask_assemble, the constraint lifecycle
// of DefaultSamplerV2.swift:50-52, 183-206, 624-640) and whose MTP verify
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
//
// Outputs: the arrays a call returns wrap the sampler's own device buffers.
// Step outputs rotate through two buffers each, so step N's tokens stay valid
// while step N+1 is enqueued (chained decode reads them back after that);
// verify outputs likewise.  Inputs of a call are kept in buffers the sampler
// owns for its life (none is freed while a kernel may still read it).

import CLSamp
import Foundation
import MLX

public final class LSampStepSampler: CBv2StepSampler {
    let runtime: LSampRuntime
    let ctx: LSampContext
    let maxRows: Int
    let maxWindow: Int
    let vocab: Int32
    let capacity: Int32          // penalty entries per row
    let windowCapacity: Int32    // repetition ring slots per row
    let fallbackSeed: UInt64
    let words: Int32             // bitmask words per row

    // configured batch
    var configuredIDs: [CBv2RequestID] = []
    var seeds: [UInt64] = []
    var steps: [UInt64] = []
    var rowParams: [lsamp_row_params] = []
    var pendingLogprobs: CBv2StepLogprobs?

    // grammar constraints: host bookkeeping, the device pool and the step's mask
    let masks: LSampConstraintMasks
    let devMaskPool: LSampDeviceBuffer<UInt32>
    let devMask: LSampDeviceBuffer<UInt32>

    /// The state a speculative (chained, constrained) sample started from:
    /// what `redrawChainedSuccessor` restores (DefaultSamplerV2.swift:56-66).
    struct Speculation {
        let requestIDs: [CBv2RequestID]
        let params: [CBv2SamplingParams]
        let steps: [UInt64]
    }
    var speculation: Speculation?

    // device state and inputs (allocated once for maxRows)
    let devParams: LSampDeviceBuffer<lsamp_row_params>
    let devKeys: LSampDeviceBuffer<UInt64>
    let devRowPtr: LSampDeviceBuffer<Int32>
    let devEntries: LSampDeviceBuffer<lsamp_penalty_entry>
    let devRowLen: LSampDeviceBuffer<Int32>
    let devWindowCount: LSampDeviceBuffer<Int32>
    let devWindow: LSampDeviceBuffer<Int32>
    let devRingPos: LSampDeviceBuffer<Int32>
    let devWindowSize: LSampDeviceBuffer<Int32>
    let devMode: LSampDeviceBuffer<UInt32>
    // the penalty table as a speculative sample found it
    let snapEntries: LSampDeviceBuffer<lsamp_penalty_entry>
    let snapRowLen: LSampDeviceBuffer<Int32>
    let snapWindowCount: LSampDeviceBuffer<Int32>
    let snapWindow: LSampDeviceBuffer<Int32>
    let snapRingPos: LSampDeviceBuffer<Int32>
    // step outputs, in turn
    let outTokens: LSampOutputRing<Int32>
    let outFlags: LSampOutputRing<UInt32>
    let outChosen: LSampOutputRing<Float>
    let outTopValues: LSampOutputRing<Float>
    let outTopIDs: LSampOutputRing<Int32>
    static let maxTopLogprobs = 32
    // verification: inputs, outputs in turn, penalty buffers that grow
    let verUniforms: LSampDeviceBuffer<Float>
    let verParams: LSampDeviceBuffer<lsamp_row_params>
    let verAccepted: LSampDeviceBuffer<Int32>
    let verNoDrafts: LSampDeviceBuffer<Int32>   // -1 drafts for a draw-only verify
    let verTokens: LSampOutputRing<Int32>
    let verAccept: LSampOutputRing<UInt8>
    let verPenRowPtr: LSampDeviceBuffer<Int32>
    let verPenEntries: LSampGrowingBuffer<lsamp_penalty_entry>
    let verPenScratch: LSampGrowingBuffer<lsamp_penalty_entry>

    public init(runtime: LSampRuntime, maxRows: Int, vocab: Int32, capacity: Int32,
                windowCapacity: Int32 = 64, maxWindow: Int = 8, fallbackSeed: UInt64 = 0) {
        self.runtime = runtime
        self.maxRows = maxRows
        self.maxWindow = maxWindow
        self.vocab = vocab
        self.capacity = capacity
        self.windowCapacity = windowCapacity
        self.fallbackSeed = fallbackSeed
        words = (vocab + 31) / 32
        ctx = LSampContext(device: runtime.device, maxRows: Int32(maxRows * maxWindow),
                           maxVocab: vocab)
        masks = LSampConstraintMasks(maxRows: maxRows, vocab: Int(vocab))
        devMaskPool = LSampDeviceBuffer(runtime, count: Int(masks.poolRows) * Int(words))
        devMask = LSampDeviceBuffer(runtime, count: maxRows * Int(words))
        let cells = maxRows * Int(capacity), ring = maxRows * Int(windowCapacity)
        devParams = LSampDeviceBuffer(runtime, count: maxRows)
        devKeys = LSampDeviceBuffer(runtime, count: maxRows)
        devRowPtr = LSampDeviceBuffer(runtime, count: maxRows + 1)
        devEntries = LSampDeviceBuffer(runtime, count: cells)
        devRowLen = LSampDeviceBuffer(runtime, count: maxRows)
        devWindowCount = LSampDeviceBuffer(runtime, count: cells)
        devWindow = LSampDeviceBuffer(runtime, count: ring)
        devRingPos = LSampDeviceBuffer(runtime, count: maxRows)
        devWindowSize = LSampDeviceBuffer(runtime, count: maxRows)
        devMode = LSampDeviceBuffer(runtime, count: maxRows)
        snapEntries = LSampDeviceBuffer(runtime, count: cells)
        snapRowLen = LSampDeviceBuffer(runtime, count: maxRows)
        snapWindowCount = LSampDeviceBuffer(runtime, count: cells)
        snapWindow = LSampDeviceBuffer(runtime, count: ring)
        snapRingPos = LSampDeviceBuffer(runtime, count: maxRows)
        outTokens = LSampOutputRing(runtime, count: maxRows)
        outFlags = LSampOutputRing(runtime, count: maxRows)
        outChosen = LSampOutputRing(runtime, count: maxRows)
        outTopValues = LSampOutputRing(runtime, count: maxRows * Self.maxTopLogprobs)
        outTopIDs = LSampOutputRing(runtime, count: maxRows * Self.maxTopLogprobs)
        verUniforms = LSampDeviceBuffer(runtime, count: maxRows * maxWindow)
        verParams = LSampDeviceBuffer(runtime, count: maxRows)
        verAccepted = LSampDeviceBuffer(runtime, count: maxRows)
        verNoDrafts = LSampDeviceBuffer(runtime, count: maxRows * max(maxWindow - 1, 1))
        verNoDrafts.upload([Int32](repeating: -1, count: verNoDrafts.count))
        verTokens = LSampOutputRing(runtime, count: maxRows * maxWindow)
        verAccept = LSampOutputRing(runtime, count: maxRows * max(maxWindow - 1, 1))
        verPenRowPtr = LSampDeviceBuffer(runtime, count: maxRows + 1)
        verPenEntries = LSampGrowingBuffer(runtime, count: maxRows * 64)
        verPenScratch = LSampGrowingBuffer(runtime, count: maxRows * maxWindow * 64)
    }

    // MARK: - capabilities

    public var supportsTokenConstraints: Bool { true }
    public var supportsConstrainedChainedDecode: Bool { true }
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

    /// The device table's mutable arrays copied between the live table and
    /// the speculation snapshot (ordered on the stream).
    func copyTable(toSnapshot: Bool) {
        let rows = configuredIDs.count
        func copy<T>(_ live: LSampDeviceBuffer<T>, _ snap: LSampDeviceBuffer<T>, _ count: Int) {
            let bytes = count * MemoryLayout<T>.stride
            if toSnapshot {
                runtime.copyDevice(UnsafeRawPointer(live.raw), to: snap.raw, bytes: bytes)
            } else {
                runtime.copyDevice(UnsafeRawPointer(snap.raw), to: live.raw, bytes: bytes)
            }
        }
        copy(devEntries, snapEntries, rows * Int(capacity))
        copy(devRowLen, snapRowLen, rows)
        copy(devWindowCount, snapWindowCount, rows * Int(capacity))
        copy(devWindow, snapWindow, rows * Int(windowCapacity))
        copy(devRingPos, snapRingPos, rows)
    }

    /// Rebuild the batch's state from the confirmed history (membership
    /// change), then fold in the pending chained tokens on the device.
    func configure(_ rows: [CBv2SamplerRow], pending: MLXArray?) {
        precondition(rows.count <= maxRows, "batch larger than the sampler was made for")
        configuredIDs = rows.map(\.id)
        seeds = rows.map { $0.params.seed ?? fallbackSeed }
        steps = rows.map { UInt64($0.outputTokens.count) }
        rowParams = rows.map { Self.resolve($0.params, vocab: vocab) }
        masks.configure(rows)
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
            precondition(
                !reps || p.repetitionContextSize <= Int(windowCapacity),
                "repetition context \(p.repetitionContextSize) exceeds the sampler's window capacity \(windowCapacity)")
            windowSize[r] = Int32(max(p.repetitionContextSize, 1))
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
        // A chained successor over constrained rows samples before its
        // predecessor's token is confirmed: keep the state it starts from,
        // so that redrawChainedSuccessor can replay it exactly
        // (DefaultSamplerV2.swift:114-127).
        let speculative = pendingSampledTokens != nil && masks.hasRows(in: requestIDs)
        if speculative {
            masks.beginSpeculation()
            copyTable(toSnapshot: true)
            speculation = Speculation(requestIDs: requestIDs, params: params, steps: steps)
        } else {
            speculation = nil
        }
        return draw(logits: logits, params: params, requestIDs: requestIDs,
                    speculative: speculative)
    }

    /// One configured draw: the step's grammar masks (assembled on the
    /// device), then lsamp_step (transforms, mask, selection, state commit,
    /// raw log-probabilities).
    func draw(logits: MLXArray, params: [CBv2SamplingParams], requestIDs: [CBv2RequestID],
              speculative: Bool) -> MLXArray {
        let rows = requestIDs.count
        devKeys.upload((0 ..< rows).map { lsamp_rng_key(seeds[$0], requestIDs[$0].raw, steps[$0]) })
        let view = runtime.deviceView(logits)
        precondition(view.shape.last! == Int(vocab), "logits vocab \(view.shape.last!); the sampler was made for \(vocab)")
        let topK = min(params.map(\.topLogprobs).max() ?? 0, Self.maxTopLogprobs)
        let tokens = outTokens.take(), flags = outFlags.take()
        let chosen = outChosen.take(), topValues = outTopValues.take(), topIDs = outTopIDs.take()

        var st = lsamp_step_args()
        if let plan = masks.plan(requestIDs, speculative: speculative) {
            var m = lsamp_mask_assemble_args()
            m.rows = Int32(rows)
            m.vocab = vocab
            m.words = words
            m.pool_rows = masks.poolRows
            m.pool = devMaskPool.mutablePointer
            m.out = devMask.mutablePointer
            plan.rowSource.withUnsafeBufferPointer { src in
                plan.rowBuild.withUnsafeBufferPointer { build in
                    plan.idsPtr.withUnsafeBufferPointer { ptr in
                        plan.ids.withUnsafeBufferPointer { ids in
                            m.row_source = src.baseAddress
                            m.row_build = build.baseAddress
                            m.ids_ptr = ptr.baseAddress
                            m.ids = ids.baseAddress
                            lsampCheck(lsamp_mask_assemble(ctx.handle, &m, runtime.stream))
                        }
                    }
                }
            }
            st.sample.bitmask = devMask.pointer
            st.sample.mask_words = words
            st.sample.mask_bits = vocab
            st.sample.mask_tail = Int32(LSAMP_MASK_TAIL_FORBID.rawValue)
        }
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
        st.sample.tokens = tokens.mutablePointer
        st.sample.row_flags = flags.mutablePointer
        st.logprobs_top_k = topK > 0 ? Int32(topK) : -1
        st.chosen_logprob = chosen.mutablePointer
        st.top_logprobs = topValues.mutablePointer
        st.top_ids = topIDs.mutablePointer
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
                    chosen: runtime.float32Array(chosen.raw, shape: [rows]),
                    topValues: runtime.float32Array(topValues.raw, shape: [rows, topK]),
                    topIndices: runtime.int32Array(topIDs.raw, shape: [rows, topK])))
            : nil
        return runtime.int32Array(tokens.raw, shape: [rows])
    }

    public func takeStepLogprobs() -> CBv2StepLogprobs? {
        defer { pendingLogprobs = nil }
        return pendingLogprobs
    }

    // MARK: - the constraint lifecycle (DefaultSamplerV2.swift:183-206, 624-640)

    public func confirmSampledTokens(_ tokens: [Int], requestIDs: [CBv2RequestID]) {
        masks.confirm(tokens: tokens, requestIDs: requestIDs)
    }

    public func tokenConstraintFailure(for id: CBv2RequestID) -> String? {
        masks.failure(for: id)
    }

    public func takeInvalidatedChainedRows() -> [CBv2RequestID] {
        masks.takeInvalidated()
    }

    /// Exact redraw of the most recent speculative `sample`: the penalty
    /// table and per-row RNG steps it started from are restored, then the
    /// same draw runs with masks from the now-confirmed constraint state.
    /// The Philox keys are a pure function of (seed, request, step), so rows
    /// whose speculative mask was valid get the same token.
    public func redrawChainedSuccessor(logits: MLXArray, requestIDs: [CBv2RequestID]) -> MLXArray? {
        guard let s = speculation, s.requestIDs == requestIDs, requestIDs == configuredIDs
        else { return nil }
        speculation = nil
        copyTable(toSnapshot: false)
        steps = s.steps
        return draw(logits: logits, params: s.params, requestIDs: requestIDs, speculative: false)
    }

    public func requestDidFinish(_ id: CBv2RequestID) {
        masks.requestDidFinish(id)
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
        precondition(S <= maxRows && W <= maxWindow, "verify window larger than the sampler was made for")
        precondition(W >= 2, "MTP verify needs at least one draft position")
        if let draftIDs {
            precondition(draftIDs.ndim == 2 && draftIDs.dim(0) == S && draftIDs.dim(1) == W - 1,
                         "MTP draft ids must be [B, W - 1]")
        }
        verUniforms.upload(verifyUniforms(params, requestIDs, stepBases, window: W))
        verParams.upload(params.map { Self.resolve($0, vocab: vocab) })
        let tokens = verTokens.take()
        let D = max(W - 1, 1)
        let accept = verAccept.take()

        var a = lsamp_verify_args()
        a.mode = Int32(mode.rawValue)
        a.sequences = Int32(S)
        a.window = Int32(W)
        a.vocab = Int32(view.shape[2])
        a.dtype = Int32(view.dtype.rawValue)
        a.target_logits = view.pointer
        a.params = verParams.pointer
        a.uniforms = verUniforms.pointer
        a.typical_delta = delta
        a.accepted = verAccepted.mutablePointer
        a.tokens = tokens.mutablePointer
        // a draw-only verify (mtpVerifySample) has no drafts: every position
        // is compared with -1 and the acceptance outputs go unread
        a.draft_tokens = draftIDs.map {
            runtime.deviceView($0).pointer.assumingMemoryBound(to: Int32.self)
        } ?? verNoDrafts.pointer
        a.accept_mask = draftIDs != nil ? accept.mutablePointer : nil

        // penalized windows: each sequence's confirmed output counts, and the
        // round's drafts before each position (CBv2MTPVerifyPenalties)
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
            let cap = longest + penalties.columnOffset + W
            let ent = verPenEntries.reserve(all.count)
            let scratch = verPenScratch.reserve(S * W * cap)
            verPenRowPtr.upload(rowPtr)
            ent.upload(all)
            a.penalty_row_ptr = verPenRowPtr.pointer
            a.penalty_entries = ent.pointer
            // position j counts drafts[0 ..< columnOffset + j]: W >= 2 needs them
            guard let draftsArray = penalties.drafts else {
                preconditionFailure("MTP penalty verification needs the round's drafts")
            }
            let drafts = runtime.deviceView(draftsArray)
            precondition(drafts.shape.count == 2 && drafts.shape[0] == S
                             && drafts.shape[1] >= penalties.columnOffset + W - 1,
                         "MTP penalty drafts must be [B, >= columnOffset + W - 1]")
            a.penalty_drafts = drafts.pointer.assumingMemoryBound(to: Int32.self)
            a.penalty_drafts_stride = Int32(drafts.rowStride)
            a.penalty_column_offset = Int32(penalties.columnOffset)
            a.penalty_scratch = scratch.mutablePointer
            a.penalty_scratch_cap = Int32(cap)
        }
        lsampCheck(lsamp_verify(ctx.handle, &a, runtime.stream))
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
