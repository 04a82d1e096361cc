"""GPU parity of suppressed ids and of the mlx-lm processor chain order
(penalties -> custom (grammar mask) -> suppress; GenerationComponents.swift:
112-141, SuppressTokens.swift:67-81) against the oracle, through the C ABI."""
from __future__ import annotations

import numpy as np
import pytest

from common import compare, run_gpu, run_oracle
from lsamp import _ffi
from lsamp import workloads as W
from lsamp.history import Cbv2RowState, TokenRing, csr, mlxlm_entries

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=64, max_vocab=262144)
    yield c
    c.close()


def _cfg(semantics, x, params, us, dtype, entries=None, bitmask=None, mask_bits=0,
         mask_tail=0, suppress=None):
    cfg = dict(semantics=semantics, dtype=dtype, rows=x.shape[0], vocab=x.shape[1], logits=x,
               params=W._params(params), uniforms=np.asarray(us, np.float32), bitmask=bitmask,
               mask_bits=mask_bits, mask_tail=mask_tail, suppress_ids=suppress)
    if entries is not None:
        cfg["row_ptr"], cfg["entries"] = csr(entries)
    return cfg


def _rows(rng, B, V, dtype):
    prior = -1.1 * np.log(np.arange(1, V + 1, dtype=np.float64))
    x = np.stack([rng.normal(0.0, 3.0, V) + prior[rng.permutation(V)] for _ in range(B)])
    return W.f32_to_bf16_bits(x) if dtype == _ffi.DTYPE_BF16 else x.astype(np.float32)


def _top_ids(x, dtype, r, n):
    v = W.bf16_bits_to_f32(x[r]) if dtype == _ffi.DTYPE_BF16 else x[r]
    return np.argsort(-v, kind="stable")[:n]


@pytest.mark.parametrize("dtype", [_ffi.DTYPE_F32, _ffi.DTYPE_BF16])
@pytest.mark.parametrize("semantics", [_ffi.SEM_MLXLM, _ffi.SEM_CBV2])
def test_penalties_mask_and_suppress(ctx, semantics, dtype):
    """Full-vocabulary rows with penalties, a grammar bitmask and a suppress
    list that holds each row's best tokens, ids past the vocabulary and
    negative ids."""
    rng = np.random.default_rng(31 + semantics * 2 + dtype)
    V, B = 151936, 8
    x = _rows(rng, B, V, dtype)
    words = (V + 31) // 32
    bm = rng.integers(0, 2**32, (B, words), dtype=np.uint64).astype(np.uint32) | np.uint32(0x11111111)
    bm[3] = 0xFFFFFFFF  # an open row
    suppress = np.concatenate([_top_ids(x, dtype, 0, 3), _top_ids(x, dtype, 5, 2),
                               [V, V + 7, 262143, -1, -40]]).astype(np.int32)
    ents, params = [], []
    for r in range(B):
        hist = rng.integers(0, 3000, 200)
        if semantics == _ffi.SEM_MLXLM:
            rr, rp, rf = TokenRing(20), TokenRing(64), TokenRing(64)
            for t in (rr, rp, rf):
                t.load_prompt(hist)
            ents.append(mlxlm_entries(rr, rp, rf))
            params.append(W.resolve_mlxlm(temperature=[0.0, 0.7, 1.0, 0.9][r % 4],
                                          top_p=0.9, top_k=[0, 40][r % 2],
                                          repetition_penalty=1.2, presence_penalty=0.3,
                                          frequency_penalty=0.1))
        else:
            st = Cbv2RowState(prompt=hist[:40], output=hist[40:], repetition_window=32,
                              repetition_on=True, counts_on=True, vocab=V)
            ents.append(st.entries())
            params.append(W.resolve_cbv2(temperature=[0.0, 0.7, 1.0, 0.9][r % 4], top_p=0.9,
                                         top_k=[0, 40][r % 2], repetition_penalty=1.2,
                                         repetition_context_size=32, presence_penalty=0.3,
                                         frequency_penalty=0.1, vocab=V))
    cfg = _cfg(semantics, x, params, rng.random(B, dtype=np.float32), dtype, entries=ents,
               bitmask=bm, mask_bits=V - 5, mask_tail=_ffi.MASK_TAIL_KEEP, suppress=suppress)
    g = run_gpu(ctx, cfg)
    o = run_oracle(cfg)
    compare(cfg, g, o, label=f"suppress {semantics} {dtype}")
    for r in range(B):
        assert g["tokens"][r] not in set(suppress.tolist())
        for t in suppress:
            if 0 <= t < V:
                assert g["processed"][r, t] == -np.inf


@pytest.mark.parametrize("semantics", [_ffi.SEM_MLXLM, _ffi.SEM_CBV2])
def test_suppress_without_a_bitmask(ctx, semantics):
    # SuppressTokensTests.swift: the suppressed maximum is never drawn
    x = np.tile(np.array([0.5, 5.0, 1.0, 9.0, 2.0], np.float32), (4, 1))
    p = (W.resolve_mlxlm(temperature=0.0) if semantics == _ffi.SEM_MLXLM
         else W.resolve_cbv2(temperature=0.0, vocab=5))
    cfg = _cfg(semantics, x, [p] * 4, [0.1, 0.4, 0.6, 0.9], _ffi.DTYPE_F32,
               suppress=np.array([3, 258882], np.int32))
    g = run_gpu(ctx, cfg)
    compare(cfg, g, run_oracle(cfg), label="suppress no mask")
    assert (g["tokens"] == 1).all()


@pytest.mark.parametrize("mask_tail", [_ffi.MASK_TAIL_KEEP, _ffi.MASK_TAIL_FORBID])
def test_suppress_keeps_the_mask_tail_policy(ctx, mask_tail):
    """Bits past mask_bits follow the caller's tail policy after the fold."""
    rng = np.random.default_rng(5)
    V = 1000
    x = rng.normal(0, 2, (3, V)).astype(np.float32)
    bm = np.zeros((3, 30), np.uint32)  # covers 960 ids, mask_bits 900
    bm[:, :] = 0xF0F0F0F0
    p = W.resolve_cbv2(temperature=1.0, vocab=V)
    cfg = _cfg(_ffi.SEM_CBV2, x, [p] * 3, [0.2, 0.5, 0.8], _ffi.DTYPE_F32, bitmask=bm,
               mask_bits=900, mask_tail=mask_tail, suppress=np.array([950, 4, 5], np.int32))
    compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label=f"tail {mask_tail}")


def test_mlxlm_chain_order_on_the_device(ctx):
    """SampleTests.swift:431-454 order, with the grammar mask as the custom
    processor: a negative repetition penalty on masked / suppressed tokens
    leaves them -inf (mask-first would make them +inf and draw them)."""
    rng = np.random.default_rng(9)
    V, B = 4096, 4
    x = rng.normal(0, 1, (B, V)).astype(np.float32)
    x[:, 100] = 30.0  # masked maximum
    x[:, 200] = 25.0  # suppressed
    ring = TokenRing(8)
    ring.load_prompt([100, 200, 300])
    ents = [mlxlm_entries(ring, None, None)] * B
    p = W.resolve_mlxlm(temperature=0.8, top_k=5, repetition_penalty=-1.5,
                        repetition_context_size=8)
    bm = np.full((B, V // 32), 0xFFFFFFFF, np.uint32)
    bm[:, 100 // 32] &= ~np.uint32(1 << (100 % 32))
    cfg = _cfg(_ffi.SEM_MLXLM, x, [p] * B, rng.random(B, dtype=np.float32), _ffi.DTYPE_F32,
               entries=ents, bitmask=bm, mask_bits=V, suppress=np.array([200], np.int32))
    g = run_gpu(ctx, cfg)
    compare(cfg, g, run_oracle(cfg), label="chain order")
    assert (g["processed"][:, 100] == -np.inf).all() and (g["processed"][:, 200] == -np.inf).all()
    assert not np.isin(g["tokens"], [100, 200]).any()
