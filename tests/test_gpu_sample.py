"""GPU parity of lsamp_sample against the oracle (both semantics), through
the C ABI.  Small hand-made rows first, then the five measured
configurations at reduced and full size.
"""
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
    c = Context(0, max_rows=512, max_vocab=262144)
    yield c
    c.close()


def fixture16():
    """SamplerPenaltyTests.swift:25-31: 0.35 * ((5j + 3) mod 16)."""
    return np.array([0.35 * ((j * 5 + 3) % 16) for j in range(16)], np.float32)


def small_cfg(semantics, logits, params, uniforms, dtype=_ffi.DTYPE_F32, entries=None,
              bitmask=None, mask_bits=0, mask_tail=0):
    rows = logits.shape[0]
    cfg = dict(semantics=semantics, dtype=dtype, rows=rows, vocab=logits.shape[1],
               logits=logits, params=W._params(params), uniforms=np.asarray(uniforms, np.float32),
               bitmask=bitmask, mask_bits=mask_bits, mask_tail=mask_tail)
    if entries is not None:
        cfg["row_ptr"], cfg["entries"] = csr(entries)
    return cfg


GRID = (np.arange(64, dtype=np.float32) + 0.5) / 64.0


@pytest.mark.parametrize("semantics", [_ffi.SEM_MLXLM, _ffi.SEM_CBV2])
@pytest.mark.parametrize("top_p,min_p,top_k", [(0.9, 0.0, 6), (0.9, 0.2, 6), (1.0, 0.05, 3),
                                               (0.9, 0.05, 0), (0.6, 0.0, 0), (1.0, 0.0, 1),
                                               (1.0, 0.0, 0)])
def test_fixture16_filters_and_draw(ctx, semantics, top_p, min_p, top_k):
    x = np.tile(fixture16(), (len(GRID), 1))
    if semantics == _ffi.SEM_MLXLM:
        p = W.resolve_mlxlm(temperature=1.0, top_p=top_p, top_k=top_k, min_p=min_p)
    else:
        p = W.resolve_cbv2(temperature=1.0, top_p=top_p, top_k=top_k, min_p=min_p, vocab=16)
    cfg = small_cfg(semantics, x, [p] * len(GRID), GRID)
    compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label=f"fixture16 {semantics}")


@pytest.mark.parametrize("semantics", [_ffi.SEM_MLXLM, _ffi.SEM_CBV2])
def test_temperatures_and_greedy(ctx, semantics):
    rng = np.random.default_rng(7)
    x = rng.normal(0, 2, (24, 301)).astype(np.float32)
    params, us = [], rng.random(24, dtype=np.float32)
    for r in range(24):
        T = [0.0, 0.3, 0.7, 1.0, 1.6, 2.5][r % 6]
        if semantics == _ffi.SEM_MLXLM:
            params.append(W.resolve_mlxlm(temperature=T, top_p=[1.0, 0.8][r % 2],
                                          top_k=[0, 17][(r // 2) % 2]))
        else:
            params.append(W.resolve_cbv2(temperature=T, top_p=[1.0, 0.8][r % 2],
                                         top_k=[0, 17][(r // 2) % 2], vocab=301))
    cfg = small_cfg(semantics, x, params, us)
    compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label="temperatures")


def test_ties_and_nonfinite(ctx):
    # CBv2TopTwoTests.swift:46-53 rows: ties, +-inf, NaN, signed zeros
    rows = np.array([[7, 7, 7, -1, 0, 2], [np.nan, -np.inf, np.inf, np.nan, np.inf, 0],
                     [np.nan] * 6, [-0.0, 0.0, -1, -2, -3, -4],
                     [1.0001, 1.0002, 1.0003, 1, 0, -1]], np.float32)
    for sem in (_ffi.SEM_MLXLM, _ffi.SEM_CBV2):
        for T in (0.0, 1.0):
            for top_k in (0, 2):
                if sem == _ffi.SEM_MLXLM:
                    p = W.resolve_mlxlm(temperature=T, top_k=top_k)
                else:
                    p = W.resolve_cbv2(temperature=T, top_k=top_k, vocab=6)
                cfg = small_cfg(sem, rows, [p] * 5, [0.1, 0.5, 0.9, 0.3, 0.7])
                compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label=f"ties {sem} {T} {top_k}")


def test_mlxlm_top_p_over_long_tie_groups(ctx):
    """mlx-lm top-p on logits quantized to steps of 0.25 (tie groups of
    hundreds of tokens, so the finalize's candidate blocks of 64 hold groups
    that start and end inside a block and groups that cross its edges):
    tokens and keep sets equal the oracle's (Evaluate.swift:462-471, the
    stable ascending argsort's order among equal values)."""
    rng = np.random.default_rng(2024)
    rows, V = 16, 5003
    x = (np.round(rng.normal(0.0, 1.5, (rows, V)) * 4.0) / 4.0).astype(np.float32)
    params = [W.resolve_mlxlm(temperature=[0.7, 1.0][r % 2], top_p=[0.5, 0.8, 0.9, 0.97][r % 4])
              for r in range(rows)]
    for us in (rng.random(rows, dtype=np.float32), GRID[:rows]):
        cfg = small_cfg(_ffi.SEM_MLXLM, x, params, us)
        compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label="mlx-lm long tie groups")


@pytest.mark.parametrize("dtype", [_ffi.DTYPE_F32, _ffi.DTYPE_BF16])
def test_full_rows_with_many_minus_inf_logits(ctx, dtype):
    """Full-vocabulary rows (the fused histogram path) whose raw logits hold
    -inf runs and scatter, some NaN, and penalty entries on -inf tokens: the
    histogram's token counts leave out every -inf token, so keep sets,
    kept weights and tokens equal the oracle's."""
    rng = np.random.default_rng(4242 + dtype)
    V, R = 151936, 8
    x = rng.normal(0, 2.5, (R, V)).astype(np.float32)
    x[0, rng.random(V) < 0.3] = -np.inf
    x[1, rng.random(V) < 0.99] = -np.inf
    x[2, :] = -np.inf
    x[2, [5, 77777, V - 1]] = [1.0, 2.0, 1.5]
    x[3, rng.random(V) < 0.2] = -np.inf
    x[3, rng.random(V) < 0.01] = np.nan
    x[4, 30000:90000] = -np.inf  # whole slices
    x[5, ::2] = -np.inf
    x[6, rng.random(V) < 0.5] = -np.inf
    x[6, :64] += 12.0  # a few strong tokens over a thinned row
    xin = x if dtype == _ffi.DTYPE_F32 else W.f32_to_bf16_bits(x)
    us = rng.random(R, dtype=np.float32)
    for sem in (_ffi.SEM_MLXLM, _ffi.SEM_CBV2):
        ents = []
        for r in range(R):
            hist = np.concatenate([rng.integers(0, V, 24), np.nonzero(np.isneginf(x[r]))[0][:16]])
            if sem == _ffi.SEM_MLXLM:
                ring_r, ring_p, ring_f = TokenRing(32), TokenRing(32), TokenRing(32)
                for t in (ring_r, ring_p, ring_f):
                    t.load_prompt(hist)
                ents.append(mlxlm_entries(ring_r, ring_p, ring_f))
            else:
                st = Cbv2RowState(prompt=hist[:20], output=hist[20:], repetition_window=32,
                                  repetition_on=True, counts_on=True, bias={}, vocab=V)
                ents.append(st.entries())
        for pkw in (dict(temperature=0.9, top_p=0.9, min_p=0.02), dict(temperature=1.2, top_p=0.97)):
            if sem == _ffi.SEM_MLXLM:
                p = W.resolve_mlxlm(repetition_penalty=1.2, presence_penalty=0.3,
                                    frequency_penalty=0.1, **pkw)
            else:
                p = W.resolve_cbv2(vocab=V, repetition_penalty=1.2, repetition_context_size=32,
                                   presence_penalty=0.3, frequency_penalty=0.1, **pkw)
            cfg = small_cfg(sem, xin, [p] * R, us, dtype=dtype, entries=ents)
            compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label=f"-inf rows {sem} {pkw}")


def test_penalties_both_semantics(ctx):
    rng = np.random.default_rng(11)
    V = 1000
    x = rng.normal(0, 3, (6, V)).astype(np.float32)
    ents_a, ents_b = [], []
    for r in range(6):
        hist = rng.integers(0, 50, 40)
        ring_r, ring_p, ring_f = TokenRing(20), TokenRing(12), TokenRing(30)
        for t in (ring_r, ring_p, ring_f):
            t.load_prompt(hist)
        ents_a.append(mlxlm_entries(ring_r, ring_p, ring_f))
        st = Cbv2RowState(prompt=hist[:20], output=hist[20:], repetition_window=16,
                          repetition_on=True, counts_on=True,
                          bias={3: 2.5, 7: -4.0} if r % 2 else {}, vocab=V)
        ents_b.append(st.entries())
    pa = W.resolve_mlxlm(temperature=0.8, top_p=0.9, repetition_penalty=1.3,
                         presence_penalty=0.4, frequency_penalty=0.2)
    pb = W.resolve_cbv2(temperature=0.8, top_p=0.9, top_k=40, repetition_penalty=1.3,
                        repetition_context_size=16, presence_penalty=0.4, frequency_penalty=0.2,
                        vocab=V)
    us = rng.random(6, dtype=np.float32)
    for sem, ents, p in ((_ffi.SEM_MLXLM, ents_a, pa), (_ffi.SEM_CBV2, ents_b, pb)):
        cfg = small_cfg(sem, x, [p] * 6, us, entries=ents)
        compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label=f"penalties {sem}")


def test_bf16_mlxlm_penalties_round_in_dtype(ctx):
    rng = np.random.default_rng(12)
    V = 777
    x = W.f32_to_bf16_bits(rng.normal(0, 3, (4, V)).astype(np.float32))
    ents = []
    for r in range(4):
        ring = TokenRing(20)
        ring.load_prompt(rng.integers(0, V, 30))
        ents.append(mlxlm_entries(ring, ring, ring))
    p = W.resolve_mlxlm(temperature=0.7, top_k=30, repetition_penalty=1.1, presence_penalty=0.3,
                        frequency_penalty=0.1)
    cfg = small_cfg(_ffi.SEM_MLXLM, x, [p] * 4, rng.random(4, dtype=np.float32),
                    dtype=_ffi.DTYPE_BF16, entries=ents)
    compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label="bf16 mlx-lm")


def test_mask_tail_policies_and_eos_row(ctx):
    rng = np.random.default_rng(13)
    V = 200
    x = rng.normal(0, 3, (5, V)).astype(np.float32)
    words = 5  # 160 mask bits < V
    bm = rng.integers(0, 2**32, (5, words), dtype=np.uint64).astype(np.uint32)
    bm[4] = 0
    bm[4, 77 // 32] = 1 << (77 % 32)  # only token 77 allowed below mask_bits
    for tail in (_ffi.MASK_TAIL_KEEP, _ffi.MASK_TAIL_FORBID):
        p = W.resolve_cbv2(temperature=0.9, top_p=0.95, vocab=V)
        cfg = small_cfg(_ffi.SEM_CBV2, x, [p] * 5, rng.random(5, dtype=np.float32), bitmask=bm,
                        mask_bits=150, mask_tail=tail)
        g = run_gpu(ctx, cfg)
        compare(cfg, g, run_oracle(cfg), label=f"mask tail {tail}")
        if tail == _ffi.MASK_TAIL_FORBID:
            assert g["tokens"][4] == 77


def test_all_masked_row_is_empty(ctx):
    x = np.zeros((2, 64), np.float32)
    bm = np.zeros((2, 2), np.uint32)
    bm[1, 0] = 1 << 5
    p = W.resolve_cbv2(temperature=1.0, vocab=64)
    cfg = small_cfg(_ffi.SEM_CBV2, x, [p, p], [0.5, 0.5], bitmask=bm, mask_bits=64)
    g = run_gpu(ctx, cfg)
    compare(cfg, g, run_oracle(cfg), label="all masked")
    assert g["tokens"][0] == -1 and g["row_flags"][0] & _ffi.ROW_EMPTY
    assert g["tokens"][1] == 5


@pytest.mark.parametrize("V", [3, 19, 1023, 1025, 40001])
def test_odd_vocab_sizes(ctx, V):
    rng = np.random.default_rng(V)
    x = rng.normal(0, 2, (3, V)).astype(np.float32)
    p = W.resolve_cbv2(temperature=0.9, top_k=min(5, V), top_p=0.9, vocab=V)
    cfg = small_cfg(_ffi.SEM_CBV2, x, [p] * 3, rng.random(3, dtype=np.float32))
    compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label=f"V={V}")


@pytest.mark.parametrize("semantics", [_ffi.SEM_MLXLM, _ffi.SEM_CBV2])
@pytest.mark.parametrize("T,top_k,top_p,min_p", [
    (0.1, 50, 1.0, 0.0), (0.05, 1000, 1.0, 0.0), (0.2, 40, 0.9, 0.05),
    (2.0, 0, 0.95, 0.0), (5.0, 0, 0.99, 0.0), (3.0, 200, 0.9, 0.01)])
def test_temperature_extremes(ctx, semantics, T, top_k, top_p, min_p):
    """Low temperatures stretch the filter space (a top-k cut lies tens of
    nats below the maximum); high ones flatten it (a top-p cut lies deep in
    the distribution).  Full-vocabulary rows, both semantics."""
    rng = np.random.default_rng(int(T * 1000) + top_k)
    V, B = 151936, 6
    prior = -1.1 * np.log(np.arange(1, V + 1, dtype=np.float64))
    x = np.stack([rng.normal(0.0, 3.0, V) + prior[rng.permutation(V)] for _ in range(B)])
    x = x.astype(np.float32)
    if semantics == _ffi.SEM_MLXLM:
        p = W.resolve_mlxlm(temperature=T, top_p=top_p, top_k=top_k, min_p=min_p)
    else:
        p = W.resolve_cbv2(temperature=T, top_p=top_p, top_k=top_k, min_p=min_p, vocab=V)
    cfg = small_cfg(semantics, x, [p] * B, rng.random(B, dtype=np.float32))
    g = run_gpu(ctx, cfg)
    assert not (g["row_flags"] & _ffi.ROW_OVERFLOW).any(), "no row may overflow"
    compare(cfg, g, run_oracle(cfg), label=f"T={T} k={top_k} p={top_p} m={min_p}")


@pytest.mark.parametrize("n", [1, 2, 3, 4])
def test_configs_reduced(ctx, n):
    kw = {1: {}, 2: {"rows": 8}, 3: {"rows": 16}, 4: {"rows": 8}}
    if n == 4:
        cfg = W.config4(rows=8)
    else:
        cfg = W.WORKLOADS[n](**kw[n])
    g = run_gpu(ctx, cfg)
    o = run_oracle(cfg)
    compare(cfg, g, o, label=f"config{n} reduced")


@pytest.mark.parametrize("n", [1, 2, 3, 4])
def test_configs_full(ctx, n):
    cfg = W.WORKLOADS[n]()
    g = run_gpu(ctx, cfg)
    o = run_oracle(cfg, threads=16)
    boundary = compare(cfg, g, o, label=f"config{n}")
    print(f"config{n}: {len(boundary)} of {cfg['rows']} rows differ only at a top-p / min-p "
          f"boundary: {boundary}")
    # a row differs only where its boundary token's exact mass lies within
    # 1e-6 of the threshold; the kernel's masses are accurate to ~3e-7, so
    # such rows are rare (about 1 in 300 for wide nuclei)
    limit = 2 + cfg["rows"] // 64
    assert len(boundary) <= limit, f"config{n}: {len(boundary)} boundary rows (limit {limit})"
    if n == 4:
        assert g["tokens"][cfg["eos_row"]] == W.EOS_ID


def test_deterministic_replay(ctx):
    cfg = W.config2(rows=16)
    a = run_gpu(ctx, cfg)
    for _ in range(3):
        b = run_gpu(ctx, cfg)
        assert np.array_equal(a["tokens"], b["tokens"])
        assert np.array_equal(a["stats"], b["stats"])


@pytest.mark.parametrize("dtype", [_ffi.DTYPE_F32, _ffi.DTYPE_BF16])
def test_mask_ending_inside_a_later_slice(ctx, dtype):
    # a mask shorter than the vocabulary (100,003 bits: not a whole word)
    # ends inside a later slice, so the allow words each slice stages before
    # its first pass change policy mid-word and past the mask; strong tokens
    # past the mask are kept only under the KEEP tail.  Histogram-path rows
    # (the fused kernel) and top-k rows (the top-k kernel) both stage them.
    rng = np.random.default_rng(17 + dtype)
    V, R, nb = 151936, 4, 100003
    words = (nb + 31) // 32
    x = rng.normal(0, 3, (R, V)).astype(np.float32)
    x[:, 120000:120010] += 9.0
    x[:, nb - 3:nb + 3] += 8.0  # around the mask's last bit
    bits = rng.random((R, words * 32)) < 0.3
    bits[:, nb - 3:nb] = True
    bm = np.packbits(bits, axis=1, bitorder="little").view(np.uint32).copy()
    xin = x if dtype == _ffi.DTYPE_F32 else W.f32_to_bf16_bits(x)
    for tail in (_ffi.MASK_TAIL_KEEP, _ffi.MASK_TAIL_FORBID):
        for pkw in (dict(temperature=0.8, top_p=0.9), dict(temperature=0.8, top_k=40, top_p=0.95)):
            p = W.resolve_cbv2(vocab=V, **pkw)
            cfg = small_cfg(_ffi.SEM_CBV2, xin, [p] * R, rng.random(R, dtype=np.float32),
                            dtype=dtype, bitmask=bm, mask_bits=nb, mask_tail=tail)
            g = run_gpu(ctx, cfg)
            compare(cfg, g, run_oracle(cfg), label=f"mask to {nb} tail {tail} {pkw}")
            if tail == _ffi.MASK_TAIL_FORBID:
                assert (g["tokens"] < nb).all(), g["tokens"]
            else:
                assert (g["tokens"] >= nb).any(), g["tokens"]
