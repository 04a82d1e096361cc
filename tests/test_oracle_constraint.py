"""CPU tests of the grammar-constraint row state (lsamp.constraint, a mirror of
CBv2TokenConstraintSampler, TokenConstraintSamplerV2.swift:21-257) and of the
oracle's mask assembly, pinned to the reference's constraint tests
(Tests/MLXLMTests/CBv2TokenConstraintSamplingTests.swift:80-356): each case
runs the row state, the oracle's assembled bitmask and the oracle's sampler,
and must give the reference's expected tokens and failures.  The mask cache
(LRU of 8, :35-52) and chained-decode validation (:201-235) are checked
against their stated rules."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from constraint_common import (CyclicKeyedConstraint, DenseTokenConstraint,
                               FixedTokenConstraint, ImpossibleTokenConstraint)
from lsamp import _ffi
from lsamp import workloads as W
from lsamp.constraint import IMPOSSIBLE_STATE, ConstraintMasks
from lsamp.history import Cbv2RowState, csr


def oracle_step(cm, pool, ids, logits, params, entries=None, speculative=False):
    logits = np.atleast_2d(np.asarray(logits, np.float32))
    V = logits.shape[1]
    plan = cm.plan(ids, speculative=speculative)
    kw = {}
    if plan is not None:
        words, _ = O.assemble_masks(plan, pool, V)
        kw.update(bitmask=words, mask_bits=V, mask_tail=_ffi.MASK_TAIL_FORBID)
    if entries is not None:
        kw["row_ptr"], kw["entries"] = csr(entries)
    out = O.sample(semantics=_ffi.SEM_CBV2, logits=logits, dtype=_ffi.DTYPE_F32,
                   params=W._params(params), uniforms=np.full(len(ids), 0.5, np.float32), **kw)
    return out["tokens"].tolist()


def fresh(rows, V):
    cm = ConstraintMasks(rows, V)
    return cm, np.zeros((cm.pool_rows, cm.words), np.uint32)


def test_greedy_sampler_enforces_the_constraint():
    # :80-101
    cm, pool = fresh(1, 4)
    cm.configure([(700, FixedTokenConstraint([1]), [])])
    assert oracle_step(cm, pool, [700], [0, 1, 2, 100], [W.resolve_cbv2(temperature=0, vocab=4)]) == [1]


def test_dense_allowlist_masks_its_excluded_token():
    # :103-128
    V = 32
    x = np.zeros(V, np.float32)
    x[30], x[31] = 10, 100
    cm, pool = fresh(1, V)
    cm.configure([(701, DenseTokenConstraint(V, 31), [])])
    assert oracle_step(cm, pool, [701], x, [W.resolve_cbv2(temperature=0, vocab=V)]) == [30]


def test_mixed_rows_never_share_grammar_state():
    # :130-177
    cm, pool = fresh(2, 4)
    c = FixedTokenConstraint([1, 2])
    p = [W.resolve_cbv2(temperature=0, vocab=4)] * 2
    x = [[0, 1, 2, 10], [0, 1, 2, 10]]
    cm.configure([(1, c, []), (2, None, [])])
    first = oracle_step(cm, pool, [1, 2], x, p)
    assert first == [1, 3]
    cm.confirm(first, [1, 2])
    cm.configure([(1, c, [1]), (2, None, [3])])
    assert oracle_step(cm, pool, [1, 2], x, p) == [2, 3]


def test_finished_request_id_reuse_rebuilds_fresh_state():
    # :179-204
    cm, pool = fresh(1, 4)
    c = FixedTokenConstraint([1, 2])
    p = [W.resolve_cbv2(temperature=0, vocab=4)]
    cm.configure([(4, c, [])])
    first = oracle_step(cm, pool, [4], [0, 1, 9, 8], p)
    assert first == [1]
    cm.confirm(first, [4])
    cm.request_did_finish(4)
    cm.configure([(4, c, [])])
    assert oracle_step(cm, pool, [4], [0, 1, 9, 8], p) == [1]


def test_impossible_state_fails_closed_on_the_stop_fallback():
    # :293-311
    cm, pool = fresh(1, 3)
    cm.configure([(77, ImpossibleTokenConstraint(), [])])
    assert oracle_step(cm, pool, [77], [0, 10, 20], [W.resolve_cbv2(temperature=0, vocab=3)]) == [0]
    assert cm.failure(77) == IMPOSSIBLE_STATE == "tool_constraint_impossible_state"


def test_grammar_mask_runs_before_top_k():
    # :313-331
    cm, pool = fresh(1, 4)
    cm.configure([(88, FixedTokenConstraint([1]), [])])
    p = [W.resolve_cbv2(temperature=1, top_p=1, top_k=1, vocab=4)]
    assert oracle_step(cm, pool, [88], [0, 1, 2, 100], p) == [1]


def test_sampling_transforms_cannot_resurrect_forbidden_logits():
    # :333-355: repetition penalty -1 over the prompt token 3 (logit 100)
    cm, pool = fresh(1, 4)
    cm.configure([(89, FixedTokenConstraint([1]), [])])
    p = [W.resolve_cbv2(temperature=1, top_p=1, top_k=1, repetition_penalty=-1,
                        repetition_context_size=64, vocab=4)]
    ent = [Cbv2RowState([3], [], 64, repetition_on=True, counts_on=False, vocab=4).entries()]
    assert oracle_step(cm, pool, [89], [0, 1, 2, 100], p, entries=ent) == [1]


def test_device_mask_words_match_the_bool_row():
    # deviceMask (:187-193): true exactly at the allowed ids; any id out of
    # range leaves the row false.  Unpacked with numpy's own bit order.
    rng = np.random.default_rng(3)
    for V in (1, 31, 32, 33, 1000, 151936):
        allowed = rng.choice(V, min(V, 50), replace=False)
        words = O.device_mask_words(allowed, V)
        assert words.shape == ((V + 31) // 32,)
        flags = np.unpackbits(words.view(np.uint8), bitorder="little")[:V].astype(bool)
        ref = np.zeros(V, bool)
        ref[allowed] = True
        assert np.array_equal(flags, ref)
        assert not np.unpackbits(words.view(np.uint8), bitorder="little")[V:].any()
        assert not O.device_mask_words(list(allowed) + [V], V).any()
        assert not O.device_mask_words([-1], V).any()


def test_mask_cache_hits_skip_allowed_ids_and_evict_least_recent():
    V = 4096
    c = CyclicKeyedConstraint(V, states=10, density=0.01, seed=1)
    cm, pool = fresh(1, V)
    cm.configure([(5, c, [])])
    seen = []
    for step in range(25):
        plan = cm.plan([5])
        O.assemble_masks(plan, pool, V)
        st = cm.rows[5].state
        seen.append(st)
        tok = int(c.sets[st][0])
        cm.confirm([tok], [5])
    # 10 states cycle; an LRU of 8 over a cycle of 10 never hits (each state
    # returns after 9 others): every step builds
    assert cm.mask_cache_hit_count == 0 and cm.mask_build_count == 25
    # a cycle of 4 states hits after the first round
    c4 = CyclicKeyedConstraint(V, states=4, density=0.01, seed=2)
    cm4, pool4 = fresh(1, V)
    cm4.configure([(6, c4, [])])
    for step in range(20):
        plan = cm4.plan([6])
        out, _ = O.assemble_masks(plan, pool4, V)
        st = cm4.rows[6].state
        assert np.array_equal(out[0], O.device_mask_words(c4.sets[st], V))
        cm4.confirm([int(c4.sets[st][0])], [6])
    assert cm4.mask_build_count == 4 and cm4.mask_cache_hit_count == 16
    assert c4.calls == 4                  # hits call no allowed_token_ids
    assert len(cm4.rows[6].masks.entries) == 4


def test_cache_slots_return_to_the_pool():
    V = 256
    cm, pool = fresh(2, V)
    c = CyclicKeyedConstraint(V, states=20, density=0.05, seed=3)
    cm.configure([(1, c, []), (2, c, [])])
    for _ in range(12):
        plan = cm.plan([1, 2])
        O.assemble_masks(plan, pool, V)
        cm.confirm([int(c.sets[cm.rows[i].state][0]) for i in (1, 2)], [1, 2])
    used = cm.rows[1].masks.slots() + cm.rows[2].masks.slots()
    assert len(used) == 16 and len(set(used)) == 16
    assert sorted(used + cm._free) == list(range(cm.cache_rows))
    cm.request_did_finish(1)
    cm.configure([(2, None, [])])
    assert sorted(cm._free) == list(range(cm.cache_rows))


def test_pool_past_max_rows_never_opens_a_row():
    """More live constrained requests than max_rows (parked or unfinished
    requests keep their 8 cached rows): once the pool is exhausted a miss
    takes another request's least recent row (or the step's own uncached
    row), never a row the same step reads, and no constrained row is ever
    planned as open (-1)."""
    V, rows = 512, 2
    cm, pool = fresh(rows, V)
    cs = {rid: CyclicKeyedConstraint(V, states=3, density=0.02, seed=40 + rid)
          for rid in range(6)}
    cm.configure([(rid, c, []) for rid, c in cs.items()])
    rng = np.random.default_rng(3)
    for step in range(60):
        batch = [int(v) for v in rng.choice(6, rows, replace=False)]
        plan = cm.plan(batch)
        assert (plan.row_source >= 0).all(), "a constrained row went open"
        out, _ = O.assemble_masks(plan, pool, V)
        for r, rid in enumerate(batch):
            st = cm.rows[rid].state
            assert np.array_equal(out[r], O.device_mask_words(cs[rid].sets[st], V)), (step, rid)
        cm.confirm([int(cs[rid].sets[cm.rows[rid].state][0]) for rid in batch], batch)
        used = [sl for row in cm.rows.values() for sl in row.masks.slots()]
        assert len(used) == len(set(used)) and -1 not in used
        assert sorted(used + cm._free) == list(range(cm.cache_rows))
    assert cm.mask_cache_hit_count > 0


def test_same_constraint_reconfigure_keeps_masks_new_instance_drops_them():
    V = 256
    cm, pool = fresh(1, V)
    c = CyclicKeyedConstraint(V, states=3, density=0.05, seed=4)
    cm.configure([(1, c, [])])
    O.assemble_masks(cm.plan([1]), pool, V)
    t0 = int(c.sets[0][0])
    cm.configure([(1, c, [t0])])          # consumed changes: replayed, masks kept
    assert cm.rows[1].state == 1 and len(cm.rows[1].masks.entries) == 1
    cm.configure([(1, CyclicKeyedConstraint(V, 3, 0.05, 4), [t0])])
    assert len(cm.rows[1].masks.entries) == 0
    cm.configure([(1, c, [t0, 99999])])   # an invalid transition latches the failure
    assert cm.failure(1) == IMPOSSIBLE_STATE


def test_chained_successor_validated_or_invalidated():
    """confirm (:201-235): a successor sampled under the confirmed state and
    budget is valid; one whose predecessor token moved the state elsewhere
    (here: the predecessor was never confirmed as the path token) is
    reported once through take_invalidated."""
    V = 64
    c = FixedTokenConstraint([5, 6, 7])
    cm, pool = fresh(1, V)
    cm.configure([(9, c, [])])
    plan = cm.plan([9])                               # step N: state 0
    assert plan.ids.tolist() == [5]
    cm.begin_speculation()
    spec = cm.plan([9], speculative=True)             # step N+1 from state 0 (stale)
    assert spec.ids.tolist() == [5]
    cm.confirm([5], [9])                              # N confirmed: state 0 -> 1
    assert cm.take_invalidated() == [9]               # successor built on state 0: redraw
    assert cm.take_invalidated() == []
    # a speculation built after confirming (state 1, consumed 1) validates
    cm.plan([9])
    cm.begin_speculation()
    cm.confirm([6], [9])
    assert cm.take_invalidated() == []
    assert cm.confirmed_state(9, 2) == 2 and cm.confirmed_state(9, 1) is None
