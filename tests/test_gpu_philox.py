"""GPU parity of the keyed draw (philox_keys instead of caller uniforms):
each row's key is SamplerV2.mix(seed, request id, step)
(SamplerV2.swift:134-155, 183-191) and its uniform Philox4x32-10 of the key,
which the oracle restates (lso_rng_uniform) and the Random123 known answers
pin.  A wrong device Philox round or float conversion changes tokens here."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from common import compare, run_gpu, run_oracle
from lsamp import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=256, max_vocab=262144)
    yield c
    c.close()


def _keys(rows, seed, step):
    return np.array([O.rng_key(seed, 1000 + r, step) for r in range(rows)], np.uint64)


@pytest.mark.parametrize("n,kw", [(2, {}), (3, {"rows": 32}), (4, {"rows": 16})])
def test_keyed_draw_matches_the_oracle(ctx, n, kw):
    cfg = W.WORKLOADS[n](**kw)
    for step in (0, 1, 57):
        keys = _keys(cfg["rows"], seed=20240501 + n, step=step)
        u = np.array([O.rng_uniform(int(k), 0) for k in keys], np.float32)
        g = run_gpu(ctx, cfg, philox_keys=keys)
        o = run_oracle(cfg, philox_keys=keys, threads=16)
        compare(cfg, g, o, label=f"config{n} philox step {step}", uniforms=u)
        # the keyed draw is the caller-uniform draw with the key's uniform
        gu = run_gpu(ctx, cfg, uniforms=u)
        assert np.array_equal(g["tokens"], gu["tokens"])
        assert np.array_equal(g["stats"]["kept_weight"], gu["stats"]["kept_weight"])
