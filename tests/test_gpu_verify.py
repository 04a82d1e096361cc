"""GPU parity of lsamp_verify (MTP speculative verification) against the
oracle, through the C ABI: RESIDUAL (textbook accept / residual / bonus),
EXACT and TYPICAL (DefaultSamplerV2.swift:378-380, 485-502) modes, small
hand-made windows and the measured 32 x 4 configuration.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lsamp import _ffi
from lsamp import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=512, max_vocab=262144)
    yield c
    c.close()


def to_dev(x, dtype):
    import torch
    if dtype == _ffi.DTYPE_F32:
        t = torch.from_numpy(np.ascontiguousarray(x, np.float32))
    elif dtype == _ffi.DTYPE_BF16:
        t = torch.from_numpy(np.ascontiguousarray(x, np.uint16).view(np.int16)).view(torch.bfloat16)
    else:
        t = torch.from_numpy(np.ascontiguousarray(x, np.uint16).view(np.int16)).view(torch.float16)
    return t.cuda()


def draw_drafts(draft, dtype, params, u):
    """Draft tokens drawn from the filtered draft distribution (oracle)."""
    S, D, V = draft.shape
    flat = draft.reshape(S * D, V)
    rp = np.repeat(np.asarray(params), D)
    out = O.sample(semantics=_ffi.SEM_CBV2, logits=flat, dtype=dtype, params=rp,
                   uniforms=np.asarray(u, np.float32).reshape(-1), threads=8)
    return out["tokens"].reshape(S, D)


def run_both(ctx, mode, target, draft, drafts, params, uniforms, dtype, delta=0.0):
    import torch
    g = ctx.verify(to_dev(target, dtype), None if draft is None else to_dev(draft, dtype),
                   drafts, params, uniforms, mode=mode, typical_delta=delta)
    torch.cuda.synchronize()
    g = {k: v.cpu().numpy() for k, v in g.items()}
    o = O.verify(mode=mode, target=target, draft=draft, draft_tokens=drafts, dtype=dtype,
                 params=params, uniforms=uniforms, typical_delta=delta, threads=8)
    return g, o


def check(g, o, label, typical=False):
    if typical:
        # decisions may differ only where p(draft) sits within 1e-6 of the
        # floor (the kernel derives p and H from fixed-point draw weights)
        near = np.abs(o["typical_margin"]) <= 1e-6
        assert np.array_equal(g["accept_mask"][~near], o["accept_mask"][~near]), label
        assert np.array_equal(g["tokens"], o["tokens"]), label
        return
    assert np.array_equal(g["accepted"], o["accepted"]), \
        f"{label}: accepted gpu {g['accepted']} oracle {o['accepted']}"
    assert np.array_equal(g["accept_mask"], o["accept_mask"]), label
    assert np.array_equal(g["tokens"], o["tokens"]), \
        f"{label}: tokens gpu {g['tokens']} oracle {o['tokens']}"


def small_case(seed, S=8, Wn=4, V=300, dtype=_ffi.DTYPE_F32, **pkw):
    rng = np.random.default_rng(seed)
    t = rng.normal(0, 2, (S, Wn, V)).astype(np.float32)
    d = (t[:, : Wn - 1] + rng.normal(0, 1, (S, Wn - 1, V))).astype(np.float32)
    if dtype == _ffi.DTYPE_BF16:
        t, d = W.f32_to_bf16_bits(t), W.f32_to_bf16_bits(d)
    params = W._params([W.resolve_cbv2(vocab=V, **pkw)] * S)
    drafts = draw_drafts(d, dtype, params, rng.random((S, Wn - 1), dtype=np.float32))
    u = rng.random((S, Wn), dtype=np.float32)
    return t, d, drafts, params, u


@pytest.mark.parametrize("pkw", [dict(temperature=1.0), dict(temperature=0.7, top_k=20),
                                 dict(temperature=1.3, top_k=5), dict(temperature=0.0)])
def test_residual_small(ctx, pkw):
    t, d, drafts, params, u = small_case(31, **pkw)
    g, o = run_both(ctx, _ffi.VERIFY_RESIDUAL, t, d, drafts, params, u, _ffi.DTYPE_F32)
    check(g, o, f"residual {pkw}")


def test_residual_rejects_and_accepts_everything(ctx):
    # drafts far from the target reject at position 0; drafts equal to the
    # target's own draws under equal distributions are always accepted
    t, d, drafts, params, u = small_case(32, temperature=1.0)
    g, o = run_both(ctx, _ffi.VERIFY_RESIDUAL, t, t[:, :-1].copy(), drafts, params, u,
                    _ffi.DTYPE_F32)
    check(g, o, "draft == target")
    assert (g["accepted"] == 3).all()
    bad = np.full_like(drafts, 299)
    dd = t[:, :-1].copy()
    dd[:, :, 299] = 30.0  # the draft is confident in a token the target finds unlikely
    g, o = run_both(ctx, _ffi.VERIFY_RESIDUAL, t, dd, bad, params, u, _ffi.DTYPE_F32)
    check(g, o, "confident wrong drafts")
    assert (g["accepted"] == 0).all()


@pytest.mark.parametrize("mode", [_ffi.VERIFY_EXACT, _ffi.VERIFY_TYPICAL])
@pytest.mark.parametrize("pkw", [dict(temperature=1.0), dict(temperature=0.5, top_k=2),
                                 dict(temperature=0.0)])
def test_exact_and_typical_small(ctx, mode, pkw):
    t, d, drafts, params, u = small_case(33, **pkw)
    g, o = run_both(ctx, mode, t, None, drafts, params, u, _ffi.DTYPE_F32,
                    delta=0.2 if mode == _ffi.VERIFY_TYPICAL else 0.0)
    check(g, o, f"mode {mode} {pkw}", typical=mode == _ffi.VERIFY_TYPICAL)


def test_typical_pinned_mask_on_gpu(ctx):
    # CBv2MTPTypicalAcceptanceTests.swift:35-110: mask [T,F,F,T,T,T]
    target = np.array([[[10, 10, -30, -30], [20, 0, 0, 0], [1, 2, 3, 4]],
                       [[1, 5, 2, 0], [0, 0, 9, 0], [3, 3, 3, 3]],
                       [[2, 2, 2, -30], [3, 0, 0, 0], [0, 1, 0, 0]]], np.float32)
    drafts = np.array([[0, 1], [2, 2], [0, 0]], np.int32)
    params = W._params([W.resolve_cbv2(temperature=1, vocab=4),
                        W.resolve_cbv2(temperature=0, vocab=4),
                        W.resolve_cbv2(temperature=1, vocab=4)])
    g, _ = run_both(ctx, _ffi.VERIFY_TYPICAL, target, None, drafts, params,
                    np.full((3, 3), 0.5, np.float32), _ffi.DTYPE_F32, delta=0.2)
    assert g["accept_mask"].reshape(-1).tolist() == [1, 0, 0, 1, 1, 1]


def test_config5_full(ctx):
    cfg = W.config5()
    drafts = draw_drafts(cfg["draft"], cfg["dtype"], cfg["params"], cfg["draft_uniforms"])
    g, o = run_both(ctx, _ffi.VERIFY_RESIDUAL, cfg["target"], cfg["draft"], drafts,
                    cfg["params"], cfg["uniforms"], cfg["dtype"])
    check(g, o, "config5")
    print(f"config5: accepted {g['accepted'].tolist()}")


@pytest.mark.parametrize("dtype,V,pkw", [
    (_ffi.DTYPE_BF16, 40003, dict(temperature=0.8, top_p=0.95)),
    (_ffi.DTYPE_F16, 20000, dict(temperature=1.0, min_p=0.02)),
    (_ffi.DTYPE_F32, 70001, dict(temperature=0.9, top_k=300)),
    (_ffi.DTYPE_BF16, 16384, dict(temperature=1.2)),
])
def test_residual_across_parts(ctx, dtype, V, pkw):
    # rows wider than one work-group's part: the residual sums are split over
    # several parts, the last part to finish draws (ragged last part, every dtype)
    rng = np.random.default_rng(V)
    S, Wn = 6, 3
    t = rng.normal(0, 3, (S, Wn, V)).astype(np.float32)
    d = (t[:, : Wn - 1] + rng.normal(0, 1.5, (S, Wn - 1, V))).astype(np.float32)
    if dtype == _ffi.DTYPE_BF16:
        t, d = W.f32_to_bf16_bits(t), W.f32_to_bf16_bits(d)
    elif dtype == _ffi.DTYPE_F16:
        t, d = t.astype(np.float16).view(np.uint16), d.astype(np.float16).view(np.uint16)
    params = W._params([W.resolve_cbv2(vocab=V, **pkw)] * S)
    drafts = draw_drafts(d, dtype, params, rng.random((S, Wn - 1), dtype=np.float32))
    u = rng.random((S, Wn), dtype=np.float32)
    for rep in range(2):  # twice: the parts' arrival counters return to zero
        g, o = run_both(ctx, _ffi.VERIFY_RESIDUAL, t, d, drafts, params, u, dtype)
        check(g, o, f"parts dtype {dtype} V {V} {pkw} rep {rep}")
    assert (g["accepted"] < Wn - 1).any(), "no rejection: the residual draw was not exercised"


@pytest.mark.parametrize("S,Wn,V,pkw", [
    (5, 2, 16385, dict(temperature=0.9, top_p=0.9)),   # one draft; a last part of one token
    (4, 6, 2049, dict(temperature=1.1)),               # a row inside one wave's first step
    (3, 6, 40000, dict(temperature=0.7, top_k=30)),    # long windows, later rejections
])
def test_residual_window_and_vocab_edges(ctx, S, Wn, V, pkw):
    rng = np.random.default_rng(V + Wn)
    t = rng.normal(0, 2.5, (S, Wn, V)).astype(np.float32)
    d = (t[:, : Wn - 1] + rng.normal(0, 1.5, (S, Wn - 1, V))).astype(np.float32)
    t, d = W.f32_to_bf16_bits(t), W.f32_to_bf16_bits(d)
    params = W._params([W.resolve_cbv2(vocab=V, **pkw)] * S)
    drafts = draw_drafts(d, _ffi.DTYPE_BF16, params, rng.random((S, Wn - 1), dtype=np.float32))
    u = rng.random((S, Wn), dtype=np.float32)
    g, o = run_both(ctx, _ffi.VERIFY_RESIDUAL, t, d, drafts, params, u, _ffi.DTYPE_BF16)
    check(g, o, f"S{S} W{Wn} V{V} {pkw}")


@pytest.mark.parametrize("sigma,pkw", [(1.0, dict(temperature=1.5)),
                                        (3.0, dict(temperature=1.0, top_p=0.9))])
def test_residual_at_the_maximum_vocabulary(sigma, pkw):
    # V = 524,288: 32 parts of eight 2,048-token spans each, so the finishing
    # wave scans all 256 spans' sums (four per lane); these rows put the
    # residual draw past token 262,144, in the spans of the third and fourth
    # lane rounds.  (Top-p over flat N(0, 1) rows would leave more than 4,096
    # tokens in the cut bin at this width: such rows fail closed by design.)
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    V, S, Wn = 524288, 6, 3
    rng = np.random.default_rng(524288 + len(pkw))
    t = rng.normal(0, sigma, (S, Wn, V)).astype(np.float32)
    d = (t[:, : Wn - 1] + rng.normal(0, 1.5, (S, Wn - 1, V))).astype(np.float32)
    t, d = W.f32_to_bf16_bits(t), W.f32_to_bf16_bits(d)
    params = W._params([W.resolve_cbv2(vocab=V, **pkw)] * S)
    drafts = draw_drafts(d, _ffi.DTYPE_BF16, params, rng.random((S, Wn - 1), dtype=np.float32))
    u = rng.random((S, Wn), dtype=np.float32)
    c = Context(0, max_rows=S * (2 * Wn - 1), max_vocab=V)
    try:
        for rep in range(2):
            g, o = run_both(c, _ffi.VERIFY_RESIDUAL, t, d, drafts, params, u, _ffi.DTYPE_BF16)
            check(g, o, f"V {V} {pkw} rep {rep}")
    finally:
        c.close()
    rej = [s for s in range(S) if o["accepted"][s] < Wn - 1]
    assert rej, "no rejection: the residual draw was not exercised"
    assert max(int(o["tokens"][s][o["accepted"][s]]) for s in rej) >= 262144
