"""GPU parity of the short-list path's edge cases (top-k <= 256 rows), through
the C ABI: the conditions that send a row to the histogram path inside the
same launch, the largest short-list k, long penalty histories, and the
launch without optional outputs that the benchmark uses.
"""
from __future__ import annotations

import numpy as np
import pytest

from common import compare, run_gpu, run_oracle, to_torch_logits
from lsamp import _ffi
from lsamp import workloads as W
from lsamp.history import Cbv2RowState, csr

pytestmark = pytest.mark.gpu

V = 151936          # four slices of 38,912 tokens
SLICE = 38912


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=64, max_vocab=V)
    yield c
    c.close()


def bf16_cfg(x, params, uniforms, entries=None):
    cfg = dict(semantics=_ffi.SEM_CBV2, dtype=_ffi.DTYPE_BF16, rows=x.shape[0], vocab=x.shape[1],
               logits=W.f32_to_bf16_bits(x.astype(np.float32)), params=W._params(params),
               uniforms=np.asarray(uniforms, np.float32), bitmask=None, mask_bits=0)
    if entries is not None:
        cfg["row_ptr"], cfg["entries"] = csr(entries)
    return cfg


def base_rows(rng, rows):
    return rng.normal(0.0, 1.0, (rows, V))


def test_tied_top_overflows_the_short_list(ctx):
    """1,200 tokens tied at the top of one slice: that slice lists more keys
    than a short list holds and the row takes the histogram path."""
    rng = np.random.default_rng(71)
    x = base_rows(rng, 4)
    for r in range(4):
        pos = rng.choice(SLICE, 1200, replace=False) + (r % 4) * SLICE
        x[r, pos[pos < V]] = 6.0
    p = W.resolve_cbv2(temperature=0.8, top_k=50, top_p=0.95, vocab=V)
    cfg = bf16_cfg(x, [p] * 4, rng.random(4, dtype=np.float32))
    compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label="tied top")


def test_crowded_thread_overflows_the_staging(ctx):
    """The top tokens all sit in one thread's quads (same lane, every quad of
    the slice): the thread stages more quads than it has slots for and the
    row takes the histogram path."""
    rng = np.random.default_rng(72)
    x = base_rows(rng, 3)
    lane = 7
    for r in range(3):
        base = (r + 1) % 4 * SLICE
        pos = np.array([base + lane * 8 + e + g * 4096 for g in range(9) for e in range(8)])
        x[r, pos] = 6.0 + rng.random(pos.size)
    p = W.resolve_cbv2(temperature=0.7, top_k=40, top_p=0.9, min_p=0.02, vocab=V)
    cfg = bf16_cfg(x, [p] * 3, rng.random(3, dtype=np.float32))
    compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label="crowded thread")


@pytest.mark.parametrize("top_k", [1, 2, 64, 65, 255, 256, 257])
def test_short_list_k_range(ctx, top_k):
    """k around the one-wave tail (64) and the short-list limit (256)."""
    rng = np.random.default_rng(100 + top_k)
    prior = -1.1 * np.log(np.arange(1, V + 1, dtype=np.float64))
    x = np.stack([rng.normal(0.0, 3.0, V) + prior[rng.permutation(V)] for _ in range(4)])
    p = W.resolve_cbv2(temperature=0.9, top_k=top_k, top_p=0.97, min_p=0.01, vocab=V)
    cfg = bf16_cfg(x, [p] * 4, rng.random(4, dtype=np.float32))
    compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label=f"k={top_k}")


def test_long_history_beyond_the_prefetch(ctx):
    """About 5,000 distinct history tokens per row: past the 1,024 entries a
    work-group prefetches, so the rest go through the long-history loop."""
    rng = np.random.default_rng(73)
    prior = -1.1 * np.log(np.arange(1, V + 1, dtype=np.float64))
    rows = 4
    x = np.stack([rng.normal(0.0, 3.0, V) + prior[rng.permutation(V)] for _ in range(rows)])
    ents = []
    for _ in range(rows):
        hist = rng.integers(0, V, 5200)
        st = Cbv2RowState(prompt=[], output=hist, repetition_window=64, repetition_on=False,
                          counts_on=True, vocab=V)
        ents.append(st.entries())
    assert min(len(e) for e in ents) > 1024
    p = W.resolve_cbv2(temperature=0.8, top_k=50, top_p=0.95, min_p=0.05, presence_penalty=0.5,
                       frequency_penalty=0.3, vocab=V)
    cfg = bf16_cfg(x, [p] * rows, rng.random(rows, dtype=np.float32), entries=ents)
    compare(cfg, run_gpu(ctx, cfg), run_oracle(cfg), label="long history")


def test_launch_without_optional_outputs(ctx):
    """The benchmark's launch (tokens and flags only) draws the same tokens as
    the launch that also writes the processed logits, keep bytes and stats."""
    import torch
    cfg = W.config2(rows=16)
    full = run_gpu(ctx, cfg)
    lt = to_torch_logits(cfg)
    out = ctx.sample(lt, cfg["params"], semantics=cfg["semantics"], row_ptr=cfg["row_ptr"],
                     entries=cfg["entries"], uniforms=cfg["uniforms"])
    torch.cuda.synchronize()
    assert np.array_equal(out["tokens"].cpu().numpy(), full["tokens"])
    assert np.array_equal(out["row_flags"].cpu().numpy().astype(np.uint32), full["row_flags"])
