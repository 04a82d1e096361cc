"""The one-pass top-k kernel (AUTO mode runs it on argmax rows and on CBv2
rows whose top-k is active and at most 64) against the oracle, on the cases
its design singles out:

* 16-bit rows with NaN, +inf and -inf anywhere, the slice's last quad
  included (the first pass flags them through a quad's maximum and a packed
  maximum of the raw half-words, and fixes those quads on a rare path);
* penalty entries in every quad position, slice edges and the vocabulary's
  last tokens included, and a history longer than the entries prefetched per
  work-group;
* K at the kernel's limit (64) and just past it (the fused kernel then runs);
* ties that overflow the candidate list (the exact radix select);
* rows whose length is not a multiple of 8 (unaligned 16-bit rows);
* the full batched-decode configuration, against the fused kernel.
"""
from __future__ import annotations

import numpy as np
import pytest

from common import compare, run_gpu, run_oracle, to_torch_logits
from lsamp import _ffi
from lsamp import workloads as W
from lsamp.api import PENALTY_DTYPE
from lsamp.history import csr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=512, max_vocab=262144)
    yield c
    c.close()


def to_bits(x: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == _ffi.DTYPE_BF16:
        return W.f32_to_bf16_bits(x.astype(np.float32))
    return x.astype(np.float16).view(np.uint16)


def cfg_of(logits_bits, dtype, params, uniforms, entries=None, vocab=None):
    rows, V = logits_bits.shape
    cfg = dict(semantics=_ffi.SEM_CBV2, dtype=dtype, rows=rows, vocab=V if vocab is None else vocab,
               logits=logits_bits, params=W._params(params),
               uniforms=np.asarray(uniforms, np.float32), bitmask=None, mask_bits=0, mask_tail=0)
    if entries is not None:
        cfg["row_ptr"], cfg["entries"] = csr(entries)
    return cfg


def check(ctx, cfg, label, topk=True):
    out = run_gpu(ctx, cfg)
    launch = ctx.last_launch()
    if topk:
        assert launch["fused"] == 2, f"{label}: the top-k kernel did not run ({launch})"
    else:
        assert launch["fused"] != 2, f"{label}: the top-k kernel ran ({launch})"
    compare(cfg, out, run_oracle(cfg), label=label)
    return out


SAMPLED = dict(temperature=0.8, top_k=20, top_p=0.9, min_p=0.05)
NO_MIN_P = dict(temperature=0.8, top_k=50, top_p=0.95, min_p=0.0)


@pytest.mark.parametrize("dtype", [_ffi.DTYPE_BF16, _ffi.DTYPE_F16])
@pytest.mark.parametrize("V", [40000, 151936])
def test_nonfinite_16bit(ctx, dtype, V):
    rng = np.random.default_rng(11 + V + dtype)
    R = 14
    x = rng.normal(0.0, 3.0, (R, V)).astype(np.float32)
    if dtype == _ffi.DTYPE_F16:
        x = np.clip(x, -60000, 60000)
    x[0, ::997] = np.nan                       # NaNs scattered
    x[1, V // 3] = np.inf                      # one +inf
    x[2, [5, V // 2, V - 9]] = np.inf          # +inf in several slices
    x[3, rng.choice(V, 40, replace=False)] = -np.inf  # -inf tokens (flag only)
    x[4, :] = np.nan                           # nearly all NaN
    x[4, rng.choice(V, 7, replace=False)] = rng.normal(0, 3, 7)
    x[5, V - 1] = np.nan                       # NaN in the last quad
    x[6, V - 1] = -np.inf                      # -inf in the last quad
    x[6, V - 2] = np.inf
    x[8, :] = -np.inf                          # nothing can be drawn
    x[9, 1000:1008] = [np.nan, np.inf, 1.0, np.nan, -np.inf, 2.0, np.inf, np.nan]  # one quad
    x[10, ::501] = np.nan                      # argmax rows
    x[11, V // 5] = np.inf
    x[12, V - 3:] = np.nan                     # min-p off: the thread-maximum bound
    x[13, ::7] = -np.inf
    params = [W.resolve_cbv2(**SAMPLED, vocab=V) for _ in range(R)]
    params[10] = params[11] = W.resolve_cbv2(temperature=0.0, vocab=V)
    params[12] = params[13] = W.resolve_cbv2(**NO_MIN_P, vocab=V)
    u = rng.random(R).astype(np.float32)
    check(ctx, cfg_of(to_bits(x, dtype), dtype, params, u), f"nonfinite dt{dtype} V{V}")


@pytest.mark.parametrize("dtype", [_ffi.DTYPE_BF16, _ffi.DTYPE_F16])
def test_penalty_entries_everywhere(ctx, dtype):
    """Entries on the tokens at every offset within a quad, on slice edges
    and on the vocabulary's last tokens; one row with a history longer than
    the per-work-group prefetch (1024 entries)."""
    V = 151936
    rng = np.random.default_rng(5 + dtype)
    R = 8
    x = rng.normal(0.0, 3.0, (R, V)).astype(np.float32)
    entries = []
    for r in range(R):
        if r == 3:
            toks = rng.choice(V, 3000, replace=False)
        else:
            edges = [k * step + d for step in (4096, 32768, 38912) for k in range(0, V // step + 1)
                     for d in (-1, 0, 7)]
            toks = np.unique(np.concatenate([
                np.array([t for t in edges if 0 <= t < V]),
                np.arange(V - 16, V),
                rng.choice(V, 300, replace=False)]))
        # make some entries the row's best tokens
        x[r, toks[:5]] = 14.0 + rng.random(5)
        counts = rng.integers(1, 9, len(toks))
        ent = np.zeros(len(toks), dtype=PENALTY_DTYPE)
        ent["token"] = toks
        ent["count"] = counts
        ent["flags"] = _ffi.PEN_REPETITION | _ffi.PEN_PRESENCE
        ent["bias"] = np.where(rng.random(len(toks)) < 0.1, rng.normal(0, 2, len(toks)), 0.0)
        entries.append(ent)
    params = [W.resolve_cbv2(temperature=0.8, top_k=50, top_p=0.95, min_p=0.05,
                             repetition_penalty=1.1, presence_penalty=0.5,
                             frequency_penalty=0.3, vocab=V) for _ in range(R)]
    params[6] = W.resolve_cbv2(temperature=0.0, repetition_penalty=1.3, presence_penalty=0.5,
                               vocab=V)
    params[7] = W.resolve_cbv2(temperature=1.0, top_k=64, top_p=1.0, presence_penalty=1.0,
                               frequency_penalty=0.5, vocab=V)
    u = rng.random(R).astype(np.float32)
    check(ctx, cfg_of(to_bits(x, dtype), dtype, params, u, entries=entries), f"entries dt{dtype}")


def test_k_limit(ctx):
    V = 151936
    rng = np.random.default_rng(3)
    x = rng.normal(0.0, 3.0, (4, V)).astype(np.float32)
    bits = to_bits(x, _ffi.DTYPE_BF16)
    u = rng.random(4).astype(np.float32)
    for k, topk in ((64, True), (65, False)):
        params = [W.resolve_cbv2(temperature=1.2, top_k=k, top_p=1.0, vocab=V)] * 4
        check(ctx, cfg_of(bits, _ffi.DTYPE_BF16, params, u), f"k={k}", topk=topk)


def test_ties_overflow_the_candidate_list(ctx):
    """Thousands of tokens share the largest values: the candidate list
    overflows and the slice's k-th key comes from the radix select."""
    V = 151936
    rng = np.random.default_rng(8)
    x = rng.normal(-20.0, 1.0, (6, V)).astype(np.float32)
    x[0, :] = 1.0                                   # every token equal
    x[1, rng.choice(V, 5000, replace=False)] = 3.0  # 5000-way tie at the top
    x[2, ::2] = 2.5                                 # half the row tied
    x[3, rng.choice(V, 3000, replace=False)] = 7.0
    x[3, rng.choice(V, 10, replace=False)] = 7.5
    x[4, :] = 0.0
    x[4, V - 40:] = 1.0                             # ties at the very end
    x[5, rng.choice(V, 2000, replace=False)] = 4.0
    params = [W.resolve_cbv2(**NO_MIN_P, vocab=V) for _ in range(6)]
    params[5] = W.resolve_cbv2(temperature=0.8, top_k=10, top_p=0.9, min_p=0.9, vocab=V)
    u = rng.random(6).astype(np.float32)
    check(ctx, cfg_of(to_bits(x, _ffi.DTYPE_BF16), _ffi.DTYPE_BF16, params, u), "ties")


@pytest.mark.parametrize("V", [151937, 40003, 1001])
def test_unaligned_rows(ctx, V):
    rng = np.random.default_rng(V)
    R = 5
    x = rng.normal(0.0, 3.0, (R, V)).astype(np.float32)
    x[1, V - 1] = np.nan
    x[2, V - 2] = np.inf
    toks = np.unique(np.concatenate([np.arange(V - 10, V), rng.choice(V, 200, replace=False)]))
    ent = np.zeros(len(toks), dtype=PENALTY_DTYPE)
    ent["token"], ent["count"], ent["flags"] = toks, 2, _ffi.PEN_PRESENCE | _ffi.PEN_REPETITION
    params = [W.resolve_cbv2(temperature=0.8, top_k=20, top_p=0.9, min_p=0.05,
                             presence_penalty=0.5, frequency_penalty=0.3,
                             repetition_penalty=1.2, vocab=V) for _ in range(R)]
    params[4] = W.resolve_cbv2(temperature=0.0, vocab=V)
    u = rng.random(R).astype(np.float32)
    check(ctx, cfg_of(to_bits(x, _ffi.DTYPE_BF16), _ffi.DTYPE_BF16, params, u,
                      entries=[ent] * R), f"unaligned V{V}")


def test_batched_decode_equals_fused(ctx):
    """The full batched-decode step: the top-k kernel and the fused kernel
    give the same tokens, flags, processed logits, keep sets and weights."""
    cfg = W.config2()
    a = run_gpu(ctx, cfg)
    assert ctx.last_launch()["fused"] == 2
    ctx.set_mode(_ffi.MODE_FUSED)
    try:
        b = run_gpu(ctx, cfg)
        assert ctx.last_launch()["fused"] == 1
    finally:
        ctx.set_mode(_ffi.MODE_AUTO)
    assert np.array_equal(a["tokens"], b["tokens"]), "tokens differ"
    assert np.array_equal(a["row_flags"], b["row_flags"]), "flags differ"
    assert np.array_equal(a["processed"].view(np.uint32), b["processed"].view(np.uint32)), \
        "processed logits differ"
    assert np.array_equal(a["keep"], b["keep"]), "keep sets differ"
    for f in ("kept", "token", "kept_weight", "probe_weight"):
        assert np.array_equal(a["stats"][f], b["stats"][f]), f"stats {f} differ"


@pytest.mark.parametrize("dtype", [_ffi.DTYPE_BF16, _ffi.DTYPE_F16])
def test_top_p_cuts_inside_top_k(ctx, dtype):
    # peaked rows (a head of 40 tokens spread over the slices) whose top-p
    # cut falls inside the top-k: the kernel's lower bound of the row's mass
    # (one exponential a quad) cannot decide the limit there, so the
    # finalizer waits for the slices' exact sums; Gaussian rows in the same
    # launch are decided by the bound; some head tokens are penalty entries
    rng = np.random.default_rng(71 + dtype)
    R, V = 24, 151936
    x = rng.normal(0, 2, (R, V)).astype(np.float32)
    entries = []
    params = []
    for r in range(R):
        head = rng.choice(V, 40, replace=False)
        if r % 4 != 3:
            x[r, head] = 12.0 - 0.4 * np.arange(40) + rng.normal(0, 0.05, 40)
        ent = np.zeros(8, dtype=PENALTY_DTYPE)
        ent["token"] = np.sort(head[::5])
        ent["count"] = rng.integers(1, 4, 8)
        ent["flags"] = _ffi.PEN_PRESENCE
        entries.append(ent)
        top_p = [0.3, 0.6, 0.9, 0.95, 0.99, 0.8][r % 6]
        params.append(W.resolve_cbv2(temperature=[0.7, 1.0, 1.3, 0.7][r // 6], top_k=[50, 64, 20][r % 3],
                                     top_p=top_p, min_p=0.0 if r % 2 else 0.01,
                                     presence_penalty=0.4, vocab=V))
    u = rng.random(R).astype(np.float32)
    check(ctx, cfg_of(to_bits(x, dtype), dtype, params, u, entries=entries), f"top-p in top-k dt{dtype}")


def test_params_host_mismatch_fails_closed(ctx):
    """The host copy of the parameters chooses the top-k kernel; rows whose
    device parameters it misdescribes (top-k 0, or past the kernel's limit)
    fail closed with token -1 and LSAMP_ROW_OVERFLOW instead of running a
    different sampler silently.  The other rows are exact, and the next
    step, with matching parameters, is exact too (the rows' hand-off state
    is not left behind)."""
    import torch
    from lsamp.api import to_device_bytes
    cfg = W.config2(rows=16)
    host = np.array(cfg["params"]).copy()
    dev = host.copy()
    dev[3]["top_k"] = 0        # histogram-path row: not the top-k kernel's
    dev[9]["top_k"] = 100      # past kTopkMaxK
    lt = to_torch_logits(cfg)
    prep = ctx.prepare_sample(lt, host, semantics=cfg["semantics"], row_ptr=cfg["row_ptr"],
                              entries=cfg["entries"], uniforms=cfg["uniforms"])
    prep.params.copy_(to_device_bytes(dev, lt.device))
    prep.launch()
    torch.cuda.synchronize()
    assert ctx.last_launch()["fused"] == 2
    tok = prep.tokens.cpu().numpy()
    flags = prep.row_flags.cpu().numpy().astype(np.uint32)
    ref = run_oracle(cfg)
    for r in range(16):
        if r in (3, 9):
            assert tok[r] == -1 and flags[r] & _ffi.ROW_OVERFLOW, (r, tok[r], flags[r])
        else:
            assert tok[r] == ref["tokens"][r] and flags[r] == ref["row_flags"][r], r
    out = run_gpu(ctx, cfg)   # the next step, parameters consistent again
    assert ctx.last_launch()["fused"] == 2
    compare(cfg, out, ref, label="step after the mismatch")
