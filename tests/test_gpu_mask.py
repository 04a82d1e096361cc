"""GPU parity of the grammar-mask assembly (lsamp_mask_assemble;
CBv2TokenConstraintSampler.mask, TokenConstraintSamplerV2.swift:131-182)
through the C ABI: the assembled bitmask and the pool rows equal the oracle's
word for word over many steps of cached, built and open rows at the
151,936-token vocabulary; the out-of-range rule and its flag; back-to-back
calls that reuse and grow the pinned staging buffers; the reference's
constraint tests (CBv2TokenConstraintSamplingTests.swift:80-356) end to end
through lsamp_sample; and a grammar-constrained step of 64 rows against the
oracle's tokens."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from constraint_common import (CyclicKeyedConstraint, DenseTokenConstraint,
                               FixedTokenConstraint, ImpossibleTokenConstraint)
from lsamp import _ffi
from lsamp import workloads as W
from lsamp.constraint import IMPOSSIBLE_STATE, ConstraintMasks, MaskPlan
from lsamp.history import Cbv2RowState, csr

pytestmark = pytest.mark.gpu

V = 151936


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=64, max_vocab=V)
    yield c
    c.close()


def as_u32(t):
    return t.cpu().numpy().view(np.uint32)


def test_assembly_matches_the_oracle_over_many_steps(ctx):
    import torch
    rows = 48
    cm = ConstraintMasks(rows, V)
    pool = ctx.mask_pool(cm)
    opool = np.zeros((cm.pool_rows, cm.words), np.uint32)
    dens = [0.001, 0.02, 0.3, 1.0]
    cons = [None if r % 6 == 5 else
            CyclicKeyedConstraint(V, states=3 + r % 9, density=dens[r % 4], seed=r) for r in range(rows)]
    cons[7] = FixedTokenConstraint([11, 12, 13, 14, 15, 16, 17, 18, 19, 20] * 3)  # uncached builds
    ids = list(range(100, 100 + rows))
    cm.configure([(i, c, []) for i, c in zip(ids, cons)])
    flags = torch.zeros(rows, dtype=torch.int32, device="cuda")
    for step in range(14):
        plan = cm.plan(ids)
        got = ctx.assemble_masks(plan, pool, V, row_flags=flags)
        want, wflags = O.assemble_masks(plan, opool, V)
        torch.cuda.synchronize()
        assert np.array_equal(as_u32(got), want), f"step {step}"
        assert np.array_equal(flags.cpu().numpy().view(np.uint32), wflags)
        toks = []
        for r, i in enumerate(ids):
            row = cm.rows.get(i)
            toks.append(0 if row is None else
                        int(row.constraint.allowed_token_ids(row.state, 1)[0]))
        cm.confirm(toks, ids)
    assert cm.mask_cache_hit_count > 0 and cm.mask_build_count > 0
    assert np.array_equal(as_u32(pool), opool)


def test_out_of_range_ids_give_a_false_row_and_a_flag(ctx):
    import torch
    pool = torch.zeros((4, (V + 31) // 32), dtype=torch.int32, device="cuda")
    plan = MaskPlan(np.array([0, 1, -1, 2], np.int32), np.array([1, 1, 0, 1], np.uint8),
                    np.array([0, 3, 5, 5, 6], np.int32),
                    np.array([5, 70000, V - 1, 9, V, -3], np.int32))
    flags = torch.full((4,), 7, dtype=torch.int32, device="cuda")
    got = ctx.assemble_masks(plan, pool, V, row_flags=flags)
    opool = np.zeros((4, (V + 31) // 32), np.uint32)
    want, wflags = O.assemble_masks(plan, opool, V)
    torch.cuda.synchronize()
    assert np.array_equal(as_u32(got), want)
    assert flags.cpu().numpy().tolist() == [0, _ffi.MASK_ID_RANGE, 0, _ffi.MASK_ID_RANGE]
    assert not as_u32(got)[1].any() and (as_u32(got)[2] == 0xFFFFFFFF).all()


def test_back_to_back_calls_reuse_and_grow_the_staging(ctx):
    """Ten calls without a host synchronization in between, their id lists
    growing past the first staging allocation; every output is checked
    afterwards."""
    import torch
    rng = np.random.default_rng(5)
    pool = torch.zeros((16, (V + 31) // 32), dtype=torch.int32, device="cuda")
    opool = np.zeros((16, (V + 31) // 32), np.uint32)
    outs, wants = [], []
    for k in range(10):
        n = 8
        sizes = rng.integers(1, 2000 * (k + 1), n)
        ptr = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
        ids = rng.integers(0, V, int(ptr[-1])).astype(np.int32)
        src = rng.permutation(16)[:n].astype(np.int32)
        build = (rng.random(n) < 0.7).astype(np.uint8)
        plan = MaskPlan(src, build, ptr, ids)
        outs.append(ctx.assemble_masks(plan, pool, V))
        wants.append(O.assemble_masks(plan, opool, V)[0])
    torch.cuda.synchronize()
    for k, (g, w) in enumerate(zip(outs, wants)):
        assert np.array_equal(as_u32(g), w), f"call {k}"


def device_step(ctx, cm, pool, ids, logits, params, entries=None, vocab=None):
    import torch
    x = np.atleast_2d(np.asarray(logits, np.float32))
    Vx = x.shape[1]
    plan = cm.plan(ids)
    kw = {}
    if plan is not None:
        kw.update(bitmask=ctx.assemble_masks(plan, pool, Vx), mask_bits=Vx,
                  mask_tail=_ffi.MASK_TAIL_FORBID)
    if entries is not None:
        kw["row_ptr"], kw["entries"] = csr(entries)
    out = ctx.sample(torch.from_numpy(x).cuda(), W._params(params), semantics=_ffi.SEM_CBV2,
                     uniforms=np.full(len(ids), 0.5, np.float32), **kw)
    torch.cuda.synchronize()
    return out["tokens"].cpu().numpy().tolist()


def test_reference_constraint_cases_on_the_device(ctx):
    g4 = [W.resolve_cbv2(temperature=0, vocab=4)]
    cm = ConstraintMasks(2, 4)
    pool = ctx.mask_pool(cm)
    cm.configure([(700, FixedTokenConstraint([1]), [])])                       # :80-101
    assert device_step(ctx, cm, pool, [700], [0, 1, 2, 100], g4) == [1]
    cm.request_did_finish(700)
    cm32 = ConstraintMasks(1, 32)
    x = np.zeros(32, np.float32)
    x[30], x[31] = 10, 100
    cm32.configure([(701, DenseTokenConstraint(32, 31), [])])                  # :103-128
    assert device_step(ctx, cm32, ctx.mask_pool(cm32), [701], x,
                       [W.resolve_cbv2(temperature=0, vocab=32)]) == [30]
    c = FixedTokenConstraint([1, 2])                                           # :130-177
    cm.configure([(1, c, []), (2, None, [])])
    first = device_step(ctx, cm, pool, [1, 2], [[0, 1, 2, 10]] * 2, g4 * 2)
    assert first == [1, 3]
    cm.confirm(first, [1, 2])
    cm.configure([(1, c, [1]), (2, None, [3])])
    assert device_step(ctx, cm, pool, [1, 2], [[0, 1, 2, 10]] * 2, g4 * 2) == [2, 3]
    cm.request_did_finish(1)
    cm.configure([(4, c, [])])                                                 # :179-204
    assert device_step(ctx, cm, pool, [4], [0, 1, 9, 8], g4) == [1]
    cm.confirm([1], [4])
    cm.request_did_finish(4)
    cm.configure([(4, c, [])])
    assert device_step(ctx, cm, pool, [4], [0, 1, 9, 8], g4) == [1]
    cm.request_did_finish(4)
    cm.configure([(77, ImpossibleTokenConstraint(), [])])                      # :293-311
    assert device_step(ctx, cm, pool, [77], [0, 10, 20, -5], g4) == [0]
    assert cm.failure(77) == IMPOSSIBLE_STATE
    cm.request_did_finish(77)
    cm.configure([(88, FixedTokenConstraint([1]), [])])                        # :313-331
    assert device_step(ctx, cm, pool, [88], [0, 1, 2, 100],
                       [W.resolve_cbv2(temperature=1, top_p=1, top_k=1, vocab=4)]) == [1]
    cm.request_did_finish(88)
    cm.configure([(89, FixedTokenConstraint([1]), [])])                        # :333-355
    ent = [Cbv2RowState([3], [], 64, repetition_on=True, counts_on=False, vocab=4).entries()]
    assert device_step(ctx, cm, pool, [89], [0, 1, 2, 100],
                       [W.resolve_cbv2(temperature=1, top_p=1, top_k=1, repetition_penalty=-1,
                                       repetition_context_size=64, vocab=4)], entries=ent) == [1]


def test_constrained_step_matches_the_oracle(ctx):
    """64 rows of 151,936 fp32 logits, grammar rows of densities 0.1%, 2%, 30%,
    100% and an EOS-only row, repetition 1.1, T 0.6, top-p 0.9: tokens equal
    the oracle's on the oracle's own assembled bitmask."""
    import torch
    rows = 64
    rng = np.random.default_rng(11)
    x = rng.normal(0, 3, (rows, V)).astype(np.float32)
    cm = ConstraintMasks(rows, V)
    pool = ctx.mask_pool(cm)
    opool = np.zeros((cm.pool_rows, cm.words), np.uint32)
    dens = [0.001, 0.02, 0.3, 1.0]
    cons = [CyclicKeyedConstraint(V, 2, dens[r % 4], seed=50 + r) for r in range(rows - 1)]
    cons.append(FixedTokenConstraint([151645]))
    ids = list(range(rows))
    cm.configure([(i, c, []) for i, c in zip(ids, cons)])
    hist = [rng.integers(0, V, 20).tolist() for _ in range(rows)]
    ent = [Cbv2RowState(h, [], 20, repetition_on=True, counts_on=False, vocab=V).entries() for h in hist]
    rp, en = csr(ent)
    params = W._params([W.resolve_cbv2(temperature=0.6, top_p=0.9, repetition_penalty=1.1,
                                       repetition_context_size=20, vocab=V)] * rows)
    u = rng.random(rows, dtype=np.float32)
    plan = cm.plan(ids)
    bm = ctx.assemble_masks(plan, pool, V)
    words, _ = O.assemble_masks(plan, opool, V)
    got = ctx.sample(torch.from_numpy(x).cuda(), params, semantics=_ffi.SEM_CBV2, row_ptr=rp,
                     entries=en, bitmask=bm, mask_bits=V, uniforms=u)["tokens"]
    torch.cuda.synchronize()
    assert np.array_equal(as_u32(bm), words)
    ref = O.sample(semantics=_ffi.SEM_CBV2, logits=x, dtype=_ffi.DTYPE_F32, params=params,
                   row_ptr=rp, entries=en, bitmask=words, mask_bits=V, uniforms=u,
                   threads=8)["tokens"]
    tok = got.cpu().numpy()
    assert np.array_equal(tok, ref)
    assert tok[-1] == 151645


def test_chained_decode_with_redraw_equals_the_unchained_stream(ctx):
    """DefaultSamplerV2.swift:114-127, 206-240 (redrawChainedSuccessor): step
    N+1 is sampled before step N's token is confirmed, under masks from the
    confirmed state with N+1's budget; rows the confirmation invalidates are
    redrawn from the same logits and the same keys (a pure function of seed,
    request and step) with masks from the confirmed state.  The chained
    stream must equal the unchained one token for token.  Path constraints
    are invalidated every step; one-state constraints stay valid."""
    import torch
    rows, steps, Vs = 8, 6, 151936
    rng = np.random.default_rng(21)
    logits = [torch.from_numpy(rng.normal(0, 3, (rows, Vs)).astype(np.float32)).cuda()
              for _ in range(steps)]
    params = W._params([W.resolve_cbv2(temperature=0.8, top_k=50, top_p=0.95, vocab=Vs)] * rows)
    ids = list(range(300, 300 + rows))
    lib = _ffi.load_library()

    def keys(step):
        return np.array([lib.lsamp_rng_key(7, i, step) for i in ids], np.uint64)

    def constraints():
        cs = []
        for r in range(rows):
            if r % 4 == 0:
                cs.append(FixedTokenConstraint([int(t) for t in rng.integers(0, Vs, steps + 2)]))
            elif r % 4 == 1:
                cs.append(CyclicKeyedConstraint(Vs, states=1, density=0.05, seed=r))  # self-loop
            elif r % 4 == 2:
                cs.append(CyclicKeyedConstraint(Vs, states=3, density=0.02, seed=r))
            else:
                cs.append(None)
        return cs

    cons = constraints()

    def draw(cm, pool, step, plan):
        kw = {}
        if plan is not None:
            kw.update(bitmask=ctx.assemble_masks(plan, pool, Vs), mask_bits=Vs)
        out = ctx.sample(logits[step], params, semantics=_ffi.SEM_CBV2, philox_keys=keys(step), **kw)
        torch.cuda.synchronize()
        return out["tokens"].cpu().numpy().tolist()

    # unchained: mask from the confirmed state, sample, confirm
    cm = ConstraintMasks(rows, Vs)
    pool = ctx.mask_pool(cm)
    cm.configure([(i, c, []) for i, c in zip(ids, cons)])
    plain = []
    for step in range(steps):
        t = draw(cm, pool, step, cm.plan(ids))
        cm.confirm(t, ids)
        plain.append(t)

    # chained: step N+1 samples before step N is confirmed
    cm2 = ConstraintMasks(rows, Vs)
    pool2 = ctx.mask_pool(cm2)
    cm2.configure([(i, c, []) for i, c in zip(ids, cons)])
    chained = [draw(cm2, pool2, 0, cm2.plan(ids))]
    redraws = valid = 0
    for step in range(1, steps):
        cm2.begin_speculation()
        spec = draw(cm2, pool2, step, cm2.plan(ids, speculative=True))
        cm2.confirm(chained[-1], ids)
        bad = cm2.take_invalidated()
        if bad:
            redraws += 1
            t = draw(cm2, pool2, step, cm2.plan(ids))
            for r, i in enumerate(ids):
                if i not in bad and cons[r] is not None:
                    assert t[r] == spec[r], f"validated row {r} changed at step {step}"
                    valid += 1
        else:
            t = spec
        chained.append(t)
    assert chained == plain
    assert redraws == steps - 1 and valid > 0


@pytest.mark.parametrize("rows", [64, 256, 300])
def test_all_cached_steps_inline_and_staged(ctx, rows):
    """A step with no builds and at most 256 rows passes its pool rows in the
    kernel arguments; a larger one goes through the staging buffers.  Both
    equal the oracle's assembly after a building step."""
    import torch
    rng = np.random.default_rng(rows)
    Vs, P = 20000, rows + 8
    words = (Vs + 31) // 32
    pool = torch.zeros((P, words), dtype=torch.int32, device="cuda")
    opool = np.zeros((P, words), np.uint32)
    sizes = rng.integers(1, 3000, P)
    ptr = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    ids = rng.integers(0, Vs, int(ptr[-1])).astype(np.int32)
    build = MaskPlan(np.arange(P, dtype=np.int32), np.ones(P, np.uint8), ptr, ids)
    ctx.assemble_masks(build, pool, Vs)
    O.assemble_masks(build, opool, Vs)
    src = rng.integers(0, P, rows).astype(np.int32)
    src[rng.random(rows) < 0.2] = -1
    cached = MaskPlan(src, np.zeros(rows, np.uint8), np.zeros(rows + 1, np.int32),
                      np.zeros(0, np.int32))
    flags = torch.full((rows,), 9, dtype=torch.int32, device="cuda")
    got = ctx.assemble_masks(cached, pool, Vs, row_flags=flags)
    want, _ = O.assemble_masks(cached, opool, Vs)
    torch.cuda.synchronize()
    assert np.array_equal(as_u32(got), want)
    assert not flags.cpu().numpy().any()
