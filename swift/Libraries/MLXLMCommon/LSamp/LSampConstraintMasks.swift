// LSampConstraintMasks.swift — CBv2TokenConstraintSampler's row state
// (ContinuousBatchingV2/TokenConstraintSamplerV2.swift:21-257) with its masks
// in a device pool of packed bitmask rows, assembled per step by
// lsamp_mask_assemble.
//
// The bookkeeping is the reference's, step for step: per constrained request
// the constraint state, the output tokens consumed, a latched failure, the
// speculation of a chained successor and an LRU of up to 8 masks keyed by the
// constraint's opt-in maskCacheKey.  Where the reference keeps each cached
// mask as an uploaded [1, vocab] bool array, here it is a row of the device
// pool: `plan` says, per output row, whether its mask is open (-1), a cached
// pool row, or a pool row to build from the allowed ids (a miss; only the ids
// travel to the device).  Pool rows [0, maxRows * 8) hold the LRU entries,
// handed out from a free list; output row r of a step uses pool row
// maxRows * 8 + r for a mask that is not cached (no key, or an impossible
// state).  The Python mirror is mlx-swift-lm_amd/lsamp/constraint.py.

import CLSamp
import Foundation
import MLX

/// The host descriptors of one lsamp_mask_assemble call.
struct LSampMaskPlan {
    var rowSource: [Int32]   // per output row: -1 open, else a pool row
    var rowBuild: [UInt8]    // 1 = build the pool row from the ids
    var idsPtr: [Int32]      // [rows + 1] offsets into ids
    var ids: [Int32]         // the allowed ids of the rows built
}

final class LSampConstraintMasks {
    static let cacheCapacity = 8

    /// The mask an in-flight chained successor was sampled under (:24-32).
    private struct Speculation {
        let state: Int
        let consumed: Int
        let failure: String?
    }

    /// Bounded per-row LRU of pool rows (MaskCache, :35-52): a lookup moves
    /// a hit to the most recent end; an insert drops the least recent when
    /// full.
    private struct MaskCache {
        var entries: [(key: Int, slot: Int32)] = []

        mutating func lookup(_ key: Int) -> Int32? {
            guard let i = entries.firstIndex(where: { $0.key == key }) else { return nil }
            let e = entries.remove(at: i)
            entries.append(e)
            return e.slot
        }

        /// Adds (key, slot); returns the pool rows the cache lets go.
        mutating func insert(_ key: Int, _ slot: Int32) -> [Int32] {
            var freed = entries.filter { $0.key == key }.map(\.slot)
            entries.removeAll { $0.key == key }
            if entries.count == LSampConstraintMasks.cacheCapacity {
                freed.append(entries.removeFirst().slot)
            }
            entries.append((key, slot))
            return freed
        }

        var slots: [Int32] { entries.map(\.slot) }

        /// Drops the least recent entry whose pool row is not in `avoid`.
        mutating func evictOldest(avoiding avoid: Set<Int32>) -> Int32? {
            guard let i = entries.firstIndex(where: { !avoid.contains($0.slot) }) else {
                return nil
            }
            return entries.remove(at: i).slot
        }
    }

    private struct RowState {
        let constraint: any CBv2TokenConstraint
        var state: Int
        var consumed: Int
        var failure: String?
        var speculation: Speculation?
        var successorFailure: String?
        var masks = MaskCache()
    }

    let maxRows: Int
    let vocab: Int
    let cacheRows: Int32
    let poolRows: Int32
    private var freeRows: [Int32]
    private var rows: [CBv2RequestID: RowState] = [:]
    private var invalidated: [CBv2RequestID] = []

    init(maxRows: Int, vocab: Int) {
        self.maxRows = maxRows
        self.vocab = vocab
        cacheRows = Int32(maxRows * Self.cacheCapacity)
        poolRows = cacheRows + Int32(maxRows)
        freeRows = Array((0 ..< cacheRows).reversed())  // popLast hands out row 0 first
    }

    var hasRows: Bool { !rows.isEmpty }

    func hasRows(in ids: [CBv2RequestID]) -> Bool {
        ids.contains { rows[$0] != nil }
    }

    private func release(_ row: RowState?) {
        if let row { freeRows.append(contentsOf: row.masks.slots) }
    }

    /// configure (:83-120): a row keeps its state when the constraint
    /// instance and the consumed count are unchanged; otherwise it is
    /// replayed from the initial state over the output tokens, keeping its
    /// masks only for the same constraint instance.
    func configure(_ descriptions: [CBv2SamplerRow]) {
        for row in descriptions {
            guard let constraint = row.tokenConstraint else {
                release(rows.removeValue(forKey: row.id))
                continue
            }
            let existing = rows[row.id]
            let same = existing.map {
                ObjectIdentifier($0.constraint) == ObjectIdentifier(constraint)
            } ?? false
            if let existing, same, existing.consumed == row.outputTokens.count { continue }
            var rebuilt = RowState(
                constraint: constraint, state: constraint.initialState, consumed: 0)
            if let existing, same { rebuilt.masks = existing.masks } else { release(existing) }
            for token in row.outputTokens {
                guard let next = constraint.nextState(state: rebuilt.state, tokenID: token) else {
                    rebuilt.failure = CBv2TokenConstraintFailure.impossibleState
                    break
                }
                rebuilt.state = next
                rebuilt.consumed += 1
            }
            rows[row.id] = rebuilt
        }
    }

    /// A speculative sample starts a new chain epoch (:124-126).
    func beginSpeculation() {
        invalidated.removeAll(keepingCapacity: true)
    }

    /// The mask bookkeeping of `mask` (:131-182) for one step: nil when no
    /// row is constrained (the logits go unmasked), else the assembly
    /// descriptors.  `speculative`: every row has one launched but
    /// unconfirmed sample; masks use the confirmed state with the
    /// successor's budget and latch nothing.
    func plan(_ requestIDs: [CBv2RequestID], speculative: Bool) -> LSampMaskPlan? {
        guard hasRows(in: requestIDs) else { return nil }
        precondition(requestIDs.count <= maxRows, "more rows than the masks were made for")
        let n = requestIDs.count
        var p = LSampMaskPlan(
            rowSource: [Int32](repeating: -1, count: n), rowBuild: [UInt8](repeating: 0, count: n),
            idsPtr: [Int32](repeating: 0, count: n + 1), ids: [])
        var inUse = Set<Int32>()  // pool rows this step reads or builds
        for (r, id) in requestIDs.enumerated() {
            p.idsPtr[r + 1] = p.idsPtr[r]
            guard var row = rows[id] else { continue }
            let consumed = row.consumed + (speculative ? 1 : 0)
            let remaining = max(0, row.constraint.maxTokens - consumed)
            let key = row.failure == nil
                ? row.constraint.maskCacheKey(state: row.state, remainingTokens: remaining) : nil
            var failure: String?
            if let key, let slot = row.masks.lookup(key) {
                p.rowSource[r] = slot
                inUse.insert(slot)
            } else {
                var allowed = row.failure == nil
                    ? row.constraint.allowedTokenIDs(state: row.state, remainingTokens: remaining)
                    : []
                if allowed.isEmpty || allowed.contains(where: { $0 < 0 || $0 >= vocab }) {
                    failure = CBv2TokenConstraintFailure.impossibleState
                    allowed = [row.constraint.fallbackTokenID]
                }
                var slot: Int32?
                if let key, failure == nil, let s = takeSlot(&row, of: id, avoiding: inUse) {
                    freeRows.append(contentsOf: row.masks.insert(key, s))
                    inUse.insert(s)
                    slot = s
                }
                // not cached: the step's own row (no key, an impossible
                // state, or no pool row free of this step's reads)
                p.rowSource[r] = slot ?? cacheRows + Int32(r)
                p.rowBuild[r] = 1
                p.ids.append(contentsOf: allowed.map { Int32($0) })
                p.idsPtr[r + 1] = p.idsPtr[r] + Int32(allowed.count)
            }
            if speculative {
                row.speculation = Speculation(state: row.state, consumed: row.consumed,
                                              failure: failure)
            } else {
                row.speculation = nil
                row.successorFailure = nil
                if let failure { row.failure = failure }
            }
            rows[id] = row
        }
        return p
    }

    /// A pool row for a new cache entry of `row`, taken before the cache
    /// changes: the row's own least recent entry when its cache is full, else
    /// a free row, else the least recent entry of another row's cache that
    /// this step does not read (the masks are only a cache).
    private func takeSlot(_ row: inout RowState, of rowID: CBv2RequestID,
                          avoiding inUse: Set<Int32>) -> Int32? {
        if row.masks.entries.count >= Self.cacheCapacity,
            let s = row.masks.evictOldest(avoiding: inUse)
        {
            return s
        }
        if let s = freeRows.popLast() { return s }
        for id in rows.keys where id != rowID {
            if let s = rows[id]!.masks.evictOldest(avoiding: inUse) { return s }
        }
        return nil
    }

    /// confirm(tokens:requestIDs:) (:201-235).
    func confirm(tokens: [Int], requestIDs: [CBv2RequestID]) {
        precondition(tokens.count == requestIDs.count)
        for (token, id) in zip(tokens, requestIDs) {
            guard var row = rows[id] else { continue }
            let speculation = row.speculation
            row.speculation = nil
            if let pending = row.successorFailure {
                row.failure = pending
                row.successorFailure = nil
            }
            if row.failure == nil {
                if let next = row.constraint.nextState(state: row.state, tokenID: token) {
                    row.state = next
                    row.consumed += 1
                } else {
                    row.failure = CBv2TokenConstraintFailure.impossibleState
                }
            }
            if let speculation {
                if row.failure == nil, speculation.state == row.state,
                    speculation.consumed + 1 == row.consumed
                {
                    row.successorFailure = speculation.failure
                } else {
                    invalidated.append(id)
                }
            }
            rows[id] = row
        }
    }

    func takeInvalidated() -> [CBv2RequestID] {
        defer { invalidated.removeAll(keepingCapacity: true) }
        return invalidated
    }

    func failure(for id: CBv2RequestID) -> String? { rows[id]?.failure }

    func requestDidFinish(_ id: CBv2RequestID) {
        release(rows.removeValue(forKey: id))
    }
}
