"""GPU tests of the coupled MTP proposal (lsamp_propose;
CBv2DefaultSampler.mtpCoupledProposal, DefaultSamplerV2.swift:310-374).

The reference's contract: the proposal uses the randomness the verifier
draws each position with, so a draft distribution equal to the target's is
always accepted, and a close one is accepted far more often than an
independent draw; any proposal leaves verification exact.  Checked here:
the proposal is the oracle's draw on the draft row with the verifier's
uniform; a draft equal to the target is accepted at every position (EXACT
verification); a perturbed draft is accepted more often with coupled
uniforms than with independent ones.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lsamp import _ffi
from lsamp import workloads as W

pytestmark = pytest.mark.gpu

V = 151936


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=512, max_vocab=V)
    yield c
    c.close()


def bf16(x):
    import torch
    b = W.f32_to_bf16_bits(np.ascontiguousarray(x, np.float32))
    return b, torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).cuda()


def windows(seed, S, Wn, noise):
    rng = np.random.default_rng(seed)
    prior = -1.1 * np.log(np.arange(1, V + 1, dtype=np.float64))
    t = np.stack([np.stack([rng.normal(0, 2.0, V) + prior[rng.permutation(V)] for _ in range(Wn)])
                  for _ in range(S)]).astype(np.float32)
    d = (t[:, :Wn - 1] + rng.normal(0, noise, (S, Wn - 1, V))).astype(np.float32)
    u = rng.random((S, Wn), dtype=np.float32)
    return rng, t, d, u


def params(S, **kw):
    ps = [W.resolve_cbv2(vocab=V, **kw) for _ in range(S)]
    ps[0] = W.resolve_cbv2(temperature=0.0, vocab=V)   # a greedy row: the mode
    return W._params(ps)


def test_proposal_is_the_draw_with_the_verifiers_uniform(ctx):
    import torch
    S = 16
    _, t, d, u = windows(1, S, 2, 0.5)
    pr = params(S, temperature=0.8, top_k=50, top_p=0.95, min_p=0.02)
    bits, dt = bf16(d[:, 0])
    got = ctx.propose(dt, pr, uniforms=u[:, 0]).cpu().numpy()
    ref = O.sample(semantics=_ffi.SEM_CBV2, logits=bits, dtype=_ffi.DTYPE_BF16, params=pr,
                   uniforms=u[:, 0], threads=8)["tokens"]
    assert np.array_equal(got, ref)
    assert got[0] == int(np.argmax(W.bf16_bits_to_f32(bits[0])))


def test_draft_equal_to_target_is_always_accepted(ctx):
    import torch
    S, Wn = 32, 4
    _, t, _, u = windows(2, S, Wn, 0.0)
    pr = params(S, temperature=0.9, top_p=0.95, top_k=100)
    tb, tt = bf16(t)
    drafts = np.zeros((S, Wn - 1), np.int32)
    for j in range(Wn - 1):
        drafts[:, j] = ctx.propose(tt[:, j], pr, uniforms=u[:, j]).cpu().numpy()
    out = ctx.verify(tt, None, drafts, pr, u, mode=_ffi.VERIFY_EXACT)
    torch.cuda.synchronize()
    assert (out["accepted"].cpu().numpy() == Wn - 1).all()


def test_coupling_raises_acceptance(ctx):
    import torch
    S, Wn = 64, 4
    rng, t, d, u = windows(3, S, Wn, 0.3)
    pr = params(S, temperature=1.0, top_p=0.9)
    tb, tt = bf16(t)
    _, dd = bf16(d)
    coupled = np.zeros((S, Wn - 1), np.int32)
    indep = np.zeros((S, Wn - 1), np.int32)
    u_ind = rng.random((S, Wn - 1), dtype=np.float32)
    for j in range(Wn - 1):
        coupled[:, j] = ctx.propose(dd[:, j], pr, uniforms=u[:, j]).cpu().numpy()
        indep[:, j] = ctx.propose(dd[:, j], pr, uniforms=u_ind[:, j]).cpu().numpy()
    a_c = ctx.verify(tt, None, coupled, pr, u, mode=_ffi.VERIFY_EXACT)["accept_mask"]
    a_i = ctx.verify(tt, None, indep, pr, u, mode=_ffi.VERIFY_EXACT)["accept_mask"]
    torch.cuda.synchronize()
    rc, ri = a_c.cpu().numpy().mean(), a_i.cpu().numpy().mean()
    assert rc > ri + 0.2, (rc, ri)
