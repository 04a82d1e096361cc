"""lsamp_penalize (the mlx-lm PenaltyProcessor as its own pass) against the
oracle, through the C ABI.

* The reference's composition test (SampleTests.swift:431-454): presence 0.5
  over a one-token window, then a custom ScaleProcessor(2) gives
  [2, 3, 6, 8]; scale-then-penalty would give 3.5 for token 1.
* Bit parity with the oracle's mlx-lm transform (which tests/
  test_oracle_penalty_dtype.py pins to exact single rounding): bf16, f16 and
  f32 logits, rows with their own repetition / presence / frequency windows,
  the output in the logits' dtype, or in float32 when a frequency penalty
  promotes it.
* Every bf16 and f16 pattern under a repetition penalty.
* One entry table shared by every row (penalty_row_len).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lsamp import _ffi
from lsamp import workloads as W
from lsamp.history import TokenRing, csr, mlxlm_entries

pytestmark = pytest.mark.gpu

F32, BF16, F16 = _ffi.DTYPE_F32, _ffi.DTYPE_BF16, _ffi.DTYPE_F16


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=64, max_vocab=262144)
    yield c
    c.close()


def torch_dtype(dt):
    import torch
    return {F32: torch.float32, BF16: torch.bfloat16, F16: torch.float16}[dt]


def to_bits(x, dt):
    x = np.asarray(x, np.float32)
    if dt == F32:
        return x.copy()
    if dt == BF16:
        return W.f32_to_bf16_bits(x)
    return x.astype(np.float16).view(np.uint16)


def device_logits(bits, dt):
    import torch
    if dt == F32:
        return torch.from_numpy(np.ascontiguousarray(bits, np.float32)).cuda()
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch_dtype(dt)).cuda()


def ring(tokens, size):
    r = TokenRing(size)
    r.load_prompt(tokens)
    return r


def test_custom_processor_after_the_penalties(ctx):
    """SampleTests.swift:431-454 through the C ABI: presence 0.5 over the
    prompt [1] (window 5), then ScaleProcessor(2)."""
    import torch
    p = W.resolve_mlxlm(temperature=0.0, presence_penalty=0.5, presence_context_size=5)
    row_ptr, ent = csr([mlxlm_entries(None, ring([1], 5), None)])
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0]], dtype=torch.float32, device="cuda")
    penalized = ctx.penalize(x, W._params([p]), row_ptr=row_ptr, entries=ent)
    scaled = penalized * 2.0  # ScaleProcessor(scale: 2)
    torch.cuda.synchronize()
    assert scaled.cpu().numpy().tolist() == [[2.0, 3.0, 6.0, 8.0]]


def _random_case(rng, rows, vocab, with_freq):
    params, ents = [], []
    for r in range(rows):
        hist = rng.integers(0, vocab, 64).tolist()
        rep = [None, 1.1, 1.3, 0.8][r % 4]
        pres = [0.5, None, 0.25, -0.5][(r // 2) % 4]
        freq = ([0.3, None, 0.1][r % 3]) if with_freq else None
        p = W.resolve_mlxlm(temperature=0.0, repetition_penalty=rep, repetition_context_size=20,
                            presence_penalty=pres, presence_context_size=12,
                            frequency_penalty=freq, frequency_context_size=32)
        rr = ring(hist, 20) if rep is not None else None
        pr = ring(hist, 12) if pres is not None else None
        fr = ring(hist, 32) if freq is not None else None
        params.append(p)
        ents.append(mlxlm_entries(rr, pr, fr))
    return params, ents


def _oracle_processed(bits, dt, params, row_ptr, ent):
    return O.sample(semantics=_ffi.SEM_MLXLM, logits=bits, dtype=dt, params=W._params(params),
                    row_ptr=row_ptr, entries=ent, uniforms=np.zeros(bits.shape[0], np.float32),
                    want_processed=True)["processed"]


@pytest.mark.parametrize("dt", [BF16, F16, F32], ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("with_freq", [False, True], ids=["dtype", "promoted"])
def test_penalize_equals_the_oracle(ctx, dt, with_freq):
    import torch
    rng = np.random.default_rng(5 + dt + 10 * with_freq)
    rows, vocab = 12, 40003
    x = rng.normal(0.0, 4.0, (rows, vocab)).astype(np.float32)
    bits = to_bits(x, dt)
    params, ents = _random_case(rng, rows, vocab, with_freq)
    row_ptr, ent = csr(ents)
    out_dtype = torch.float32 if with_freq else torch_dtype(dt)
    got = ctx.penalize(device_logits(bits, dt), W._params(params), row_ptr=row_ptr, entries=ent,
                       out_dtype=out_dtype)
    torch.cuda.synchronize()
    assert got.dtype == out_dtype
    g = got.float().cpu().numpy()
    want = _oracle_processed(bits, dt, params, row_ptr, ent)
    bad = g.view(np.uint32) != want.view(np.uint32)
    assert not bad.any(), f"{int(bad.sum())} values differ, first at {np.argwhere(bad)[0]}"
    # the entries changed something (the comparison is not of two copies)
    raw = (x if dt == F32 else W.bf16_bits_to_f32(bits) if dt == BF16
           else O.f16_to_f32(bits)).reshape(rows, vocab)
    assert (g != raw).sum() >= rows


@pytest.mark.parametrize("dt", [BF16, F16], ids=["bf16", "f16"])
def test_every_16bit_pattern(ctx, dt):
    """All finite bf16 / f16 patterns under repetition 1.1 and presence 0.5:
    the kernel's dtype rounding equals the oracle's (exact single rounding)."""
    import torch
    h = np.arange(1 << 16, dtype=np.uint16)
    xs = W.bf16_bits_to_f32(h) if dt == BF16 else O.f16_to_f32(h)
    bits = h[np.isfinite(xs)].reshape(1, -1)
    V = bits.shape[1]
    ent = np.zeros(V, O.PENALTY_DTYPE)
    ent["token"] = np.arange(V)
    ent["flags"] = _ffi.PEN_REPETITION | _ffi.PEN_PRESENCE
    p = W.resolve_mlxlm(temperature=0.0)
    p["repetition_penalty"], p["presence_penalty"] = 1.1, 0.5
    row_ptr = np.array([0, V], np.int32)
    got = ctx.penalize(device_logits(bits, dt), W._params([p]), row_ptr=row_ptr, entries=ent)
    torch.cuda.synchronize()
    g = got.float().cpu().numpy()
    want = _oracle_processed(bits, dt, [p], row_ptr, ent)
    assert np.array_equal(g.view(np.uint32), want.view(np.uint32))


def test_shared_entries_with_row_lengths(ctx):
    """One history for the whole batch (the reference's penalty contexts
    broadcast one window over [B, V]): every row start 0, row_len n."""
    import torch
    rng = np.random.default_rng(3)
    rows, vocab = 5, 1000
    x = rng.normal(0.0, 2.0, (rows, vocab)).astype(np.float32)
    p = W.resolve_mlxlm(temperature=0.0, repetition_penalty=1.2, repetition_context_size=10,
                        frequency_penalty=0.2, frequency_context_size=10)
    hist = rng.integers(0, vocab, 10).tolist()
    ent = mlxlm_entries(ring(hist, 10), None, ring(hist, 10))
    got = ctx.penalize(device_logits(x, F32), W._params([p] * rows),
                       row_ptr=np.zeros(rows + 1, np.int32), entries=ent,
                       row_len=np.full(rows, len(ent), np.int32))
    torch.cuda.synchronize()
    row_ptr, flat = csr([ent] * rows)
    want = _oracle_processed(x, F32, [p] * rows, row_ptr, flat)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
