"""Grammar-constrained rows: the host bookkeeping of CBv2TokenConstraintSampler
(Libraries/MLXLMCommon/ContinuousBatchingV2/TokenConstraintSamplerV2.swift:
21-257) with its masks kept on the device.

The reference keeps, per constrained request, the constraint state, the
output tokens consumed, a latched failure, the speculation of a chained
(pipelined) successor and an LRU of up to 8 uploaded [1, vocab] bool masks
keyed by the constraint's opt-in `maskCacheKey`; `mask` builds each row's
mask (cache hit: no host work, no upload) and concatenates the rows.

Here the bookkeeping is the same, step for step, and the masks are packed
bitmask rows in a device pool (lsamp_mask_assemble).  `plan` returns, per
output row, where its mask comes from: -1 (an open row), a cached pool row,
or a pool row to build from the allowed ids (a miss; only the ids travel to
the device, through pinned double-buffered staging).  Pool rows
[0, max_rows * cache_capacity) hold the LRU entries, handed out from a free
list; row r of a step uses pool row max_rows * cache_capacity + r for a mask
that is not cached (no key, or an impossible state).

A constraint is any object with the members of CBv2TokenConstraint
(ToolConstraintV2.swift:23-67): `initial_state`, `max_tokens`,
`fallback_token_id`, `allowed_token_ids(state, remaining)`,
`next_state(state, token)` (None: not a valid transition) and optionally
`mask_cache_key(state, remaining)` (None disables caching).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

# CBv2TokenConstraintFailure.impossibleState
IMPOSSIBLE_STATE = "tool_constraint_impossible_state"
# MaskCache.capacity (TokenConstraintSamplerV2.swift:36)
MASK_CACHE_CAPACITY = 8


def _cache_key(constraint, state: int, remaining: int) -> Optional[int]:
    f = getattr(constraint, "mask_cache_key", None)
    return None if f is None else f(state, remaining)


@dataclass
class _Speculation:
    """The mask an in-flight chained successor was sampled under (:24-32)."""
    state: int
    consumed: int
    failure: Optional[str]


class _MaskCache:
    """Bounded per-row LRU of pool rows (MaskCache, :35-52): lookup moves a
    hit to the most recent end; insert drops the least recent when full."""

    def __init__(self, capacity: int):
        self.capacity = capacity
        self.entries: List[Tuple[int, int]] = []   # (key, pool row), least recent first

    def lookup(self, key: int) -> Optional[int]:
        for i, (k, slot) in enumerate(self.entries):
            if k == key:
                self.entries.append(self.entries.pop(i))
                return slot
        return None

    def insert(self, key: int, slot: int) -> List[int]:
        """Add (key, slot); returns the pool rows the cache let go."""
        freed = [s for k, s in self.entries if k == key]
        self.entries = [(k, s) for k, s in self.entries if k != key]
        if len(self.entries) == self.capacity:
            freed.append(self.entries.pop(0)[1])
        self.entries.append((key, slot))
        return freed

    def slots(self) -> List[int]:
        return [s for _, s in self.entries]

    def evict_oldest(self, avoid) -> Optional[int]:
        """Drop the least recent entry whose pool row is not in `avoid`;
        returns that pool row, or None."""
        for i, (_, slot) in enumerate(self.entries):
            if slot not in avoid:
                self.entries.pop(i)
                return slot
        return None


@dataclass
class _RowState:
    constraint: object
    state: int
    consumed: int
    failure: Optional[str] = None
    speculation: Optional[_Speculation] = None
    # a validated speculative mask failed; latched when the successor's
    # sample is confirmed (:62-66)
    successor_failure: Optional[str] = None
    masks: _MaskCache = field(default_factory=lambda: _MaskCache(MASK_CACHE_CAPACITY))


@dataclass
class MaskPlan:
    """The host descriptors of one lsamp_mask_assemble call."""
    row_source: np.ndarray   # [rows] int32: -1 open, else a pool row
    row_build: np.ndarray    # [rows] uint8: build the pool row from ids
    ids_ptr: np.ndarray      # [rows + 1] int32
    ids: np.ndarray          # [ids_ptr[-1]] int32

    @property
    def rows(self) -> int:
        return len(self.row_source)


class ConstraintMasks:
    """CBv2TokenConstraintSampler's row state with device-resident masks."""

    def __init__(self, max_rows: int, vocab: int, cache_capacity: int = MASK_CACHE_CAPACITY):
        self.max_rows = max_rows
        self.vocab = vocab
        self.words = (vocab + 31) // 32
        self.cache_capacity = cache_capacity
        self.cache_rows = max_rows * cache_capacity
        self.pool_rows = self.cache_rows + max_rows
        self._free = list(range(self.cache_rows - 1, -1, -1))   # pop() hands out row 0 first
        self.rows: Dict[int, _RowState] = {}
        self.invalidated: List[int] = []
        # test hooks (:70-73): builds from allowed ids, cached-mask reuses
        self.mask_build_count = 0
        self.mask_cache_hit_count = 0

    # ------------------------------------------------------------ row state
    def has_rows(self, ids: Optional[Sequence[int]] = None) -> bool:
        if ids is None:
            return bool(self.rows)
        return any(i in self.rows for i in ids)

    def _release(self, row: Optional[_RowState]):
        if row is not None:
            self._free.extend(row.masks.slots())
            row.masks.entries = []

    def configure(self, descriptions):
        """descriptions: (request_id, constraint or None, output_tokens) per
        row (configure, :83-120).  A row keeps its state when the constraint
        instance and the consumed count are unchanged; otherwise it is
        replayed from the initial state over the output tokens, keeping its
        masks only for the same constraint instance."""
        for rid, constraint, output in descriptions:
            existing = self.rows.get(rid)
            if constraint is None:
                self._release(self.rows.pop(rid, None))
                continue
            same = existing is not None and existing.constraint is constraint
            if same and existing.consumed == len(output):
                continue
            rebuilt = _RowState(constraint, constraint.initial_state, 0,
                                masks=_MaskCache(self.cache_capacity))
            if same:
                rebuilt.masks = existing.masks
            else:
                self._release(existing)
            for token in output:
                nxt = constraint.next_state(rebuilt.state, token)
                if nxt is None:
                    rebuilt.failure = IMPOSSIBLE_STATE
                    break
                rebuilt.state = nxt
                rebuilt.consumed += 1
            self.rows[rid] = rebuilt

    def begin_speculation(self):
        """A speculative sample starts a new chain epoch (:124-126)."""
        self.invalidated = []

    # ----------------------------------------------------------------- masks
    def plan(self, request_ids: Sequence[int], speculative: bool = False) -> Optional[MaskPlan]:
        """The mask bookkeeping of `mask` (:131-182) for one step: None when
        no row is constrained (the logits go unmasked), else the assembly
        descriptors.  `speculative`: every row has one launched-but-
        unconfirmed sample; masks use the confirmed state with the
        successor's budget and latch nothing."""
        if not self.has_rows(request_ids):
            return None
        if len(request_ids) > self.max_rows:
            raise ValueError(f"{len(request_ids)} rows exceed max_rows {self.max_rows}")
        n = len(request_ids)
        src = np.full(n, -1, np.int32)
        build = np.zeros(n, np.uint8)
        ptr = np.zeros(n + 1, np.int32)
        ids: List[np.ndarray] = []
        in_use = set()  # pool rows this step reads or builds
        for r, rid in enumerate(request_ids):
            row = self.rows.get(rid)
            if row is None:
                ptr[r + 1] = ptr[r]
                continue
            consumed = row.consumed + (1 if speculative else 0)
            remaining = max(0, row.constraint.max_tokens - consumed)
            key = _cache_key(row.constraint, row.state, remaining) if row.failure is None else None
            failure = None
            slot = row.masks.lookup(key) if key is not None else None
            if slot is not None:
                self.mask_cache_hit_count += 1
                src[r] = slot
                in_use.add(slot)
            else:
                allowed = (list(row.constraint.allowed_token_ids(row.state, remaining))
                           if row.failure is None else [])
                if not allowed or any(t < 0 or t >= self.vocab for t in allowed):
                    failure = IMPOSSIBLE_STATE
                    allowed = [row.constraint.fallback_token_id]
                self.mask_build_count += 1
                slot = None
                if key is not None and failure is None:
                    slot = self._take_slot(row, in_use)
                    if slot is not None:
                        self._free.extend(row.masks.insert(key, slot))
                        in_use.add(slot)
                if slot is None:
                    # not cached: the step's own row (no key, an impossible
                    # state, or no pool row free of this step's reads)
                    slot = self.cache_rows + r
                src[r] = slot
                build[r] = 1
                ids.append(np.asarray(allowed, np.int64).astype(np.int32))
                ptr[r + 1] = ptr[r] + len(allowed)
                if speculative:
                    row.speculation = _Speculation(row.state, row.consumed, failure)
                else:
                    row.speculation = None
                    row.successor_failure = None
                    if failure is not None:
                        row.failure = failure
                continue
            ptr[r + 1] = ptr[r]
            if speculative:
                row.speculation = _Speculation(row.state, row.consumed, failure)
            else:
                row.speculation = None
                row.successor_failure = None
        flat = np.concatenate(ids) if ids else np.zeros(0, np.int32)
        return MaskPlan(src, build, ptr, flat)

    def _take_slot(self, row: _RowState, in_use) -> Optional[int]:
        """A pool row for a new cache entry of `row`, taken before the cache
        changes: the row's own least recent entry when its cache is full (the
        LRU would drop it), else a free row, else the least recent entry of
        another row's cache that this step does not read (the masks are only
        a cache; that row rebuilds on its next miss).  None: every pool row
        is read by this step."""
        if len(row.masks.entries) >= row.masks.capacity:
            slot = row.masks.evict_oldest(in_use)
            if slot is not None:
                return slot
        if self._free:
            return self._free.pop()
        for other in self.rows.values():
            if other is row:
                continue
            slot = other.masks.evict_oldest(in_use)
            if slot is not None:
                return slot
        return None

    # ----------------------------------------------------------- confirmation
    def confirm(self, tokens: Sequence[int], request_ids: Sequence[int]):
        """confirm(tokens:requestIDs:) (:201-235): advance each constrained
        row by its confirmed token; a chained successor whose mask was not
        built from the state and budget now confirmed is reported through
        take_invalidated() for an exact redraw."""
        if len(tokens) != len(request_ids):
            raise ValueError("tokens and request_ids differ in length")
        for token, rid in zip(tokens, request_ids):
            row = self.rows.get(rid)
            if row is None:
                continue
            spec = row.speculation
            row.speculation = None
            if row.successor_failure is not None:
                row.failure = row.successor_failure
                row.successor_failure = None
            if row.failure is None:
                nxt = row.constraint.next_state(row.state, int(token))
                if nxt is not None:
                    row.state = nxt
                    row.consumed += 1
                else:
                    row.failure = IMPOSSIBLE_STATE
            if spec is not None:
                if (row.failure is None and spec.state == row.state
                        and spec.consumed + 1 == row.consumed):
                    row.successor_failure = spec.failure
                else:
                    self.invalidated.append(rid)

    def take_invalidated(self) -> List[int]:
        out, self.invalidated = self.invalidated, []
        return out

    def failure(self, rid: int) -> Optional[str]:
        row = self.rows.get(rid)
        return None if row is None else row.failure

    def confirmed_state(self, rid: int, output_token_count: int) -> Optional[int]:
        row = self.rows.get(rid)
        if row is None or row.failure is not None or row.consumed != output_token_count:
            return None
        return row.state

    def request_did_finish(self, rid: int):
        self._release(self.rows.pop(rid, None))
