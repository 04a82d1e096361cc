"""Synthetic inputs for the five measured configurations.

Each generator is seeded with numpy's PCG64 (`default_rng(1000 + n)` for
configuration n = 1..5); logits are drawn in float64 and rounded to the stored
dtype, and the stored tensor *is* the input.  Zipf(s) histories draw ranks k
with P(k) proportional to (k+1)^-s over the vocabulary and map them to token
ids through a per-row permutation.  Uniforms are float32 in [0, 1).

The returned dict holds host numpy arrays only:
  semantics, dtype, rows, vocab, logits (float32, or uint16 bf16 bits),
  params (structured, lsamp_row_params layout), row_ptr / entries (CSR of
  lsamp_penalty_entry) or None, bitmask / mask_bits or None, uniforms,
  and a `workload` description.  Config 5 holds the verify inputs instead.
"""
from __future__ import annotations

import numpy as np

from . import _ffi
from .api import PARAMS_DTYPE, PENALTY_DTYPE
from .history import Cbv2RowState, TokenRing, csr, mlxlm_entries

V_QWEN = 151936
V_256K = 262144
EOS_ID = 151645


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (uint16)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return b.astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def zipf_ranks(rng: np.random.Generator, s: float, V: int, n: int, cdf=None) -> np.ndarray:
    if cdf is None:
        p = (np.arange(1, V + 1, dtype=np.float64)) ** (-s)
        cdf = np.cumsum(p)
        cdf /= cdf[-1]
    r = np.searchsorted(cdf, rng.random(n), side="right")
    return np.minimum(r, V - 1)


def _zipf_cdf(s: float, V: int) -> np.ndarray:
    p = (np.arange(1, V + 1, dtype=np.float64)) ** (-s)
    cdf = np.cumsum(p)
    return cdf / cdf[-1]


def resolve_cbv2(temperature=1.0, top_p=1.0, top_k=0, min_p=0.0, repetition_penalty=1.0,
                 repetition_context_size=64, frequency_penalty=0.0, presence_penalty=0.0,
                 vocab=V_QWEN) -> dict:
    """LogitsPipelineV2.setRows resolution (LogitsPipelineV2.swift:188-227)."""
    greedy = np.float32(temperature) < np.float32(1e-5)
    r = dict(kind=_ffi.KIND_ARGMAX if greedy else _ffi.KIND_FILTERED,
             temperature=1.0 if greedy else temperature, top_k=0, top_p=2.0, min_p=0.0,
             repetition_penalty=1.0, presence_penalty=0.0, frequency_penalty=0.0)
    if not greedy:
        if 0 < top_k < vocab:
            r["top_k"] = top_k
        if 0.0 < top_p < 1.0:
            r["top_p"] = top_p
        elif top_p <= 0.0:
            r["top_p"] = 0.0
        if min_p > 0.0:
            r["min_p"] = min(min_p, 1.0)
    if repetition_penalty != 1.0 and repetition_context_size > 0:
        r["repetition_penalty"] = repetition_penalty
    if frequency_penalty != 0.0 or presence_penalty != 0.0:
        r["frequency_penalty"] = frequency_penalty
        r["presence_penalty"] = presence_penalty
    return r


def resolve_mlxlm(temperature=0.6, top_p=1.0, top_k=0, min_p=0.0, repetition_penalty=None,
                  repetition_context_size=20, presence_penalty=None, presence_context_size=20,
                  frequency_penalty=None, frequency_context_size=20) -> dict:
    """GenerateParameters.sampler() / .processor() (Evaluate.swift:328-387)."""
    uses_p = 0.0 < top_p < 1.0
    uses_k = top_k > 0
    uses_m = min_p > 0.0
    if temperature == 0:
        kind = _ffi.KIND_ARGMAX
    elif uses_p or uses_k or uses_m:
        kind = _ffi.KIND_FILTERED
    else:
        kind = _ffi.KIND_CATEGORICAL
    r = dict(kind=kind, temperature=temperature, top_p=top_p if uses_p else 1.0,
             top_k=top_k if uses_k else 0, min_p=min_p if uses_m else 0.0,
             repetition_penalty=1.0, presence_penalty=0.0, frequency_penalty=0.0)
    if (repetition_penalty is not None and repetition_penalty not in (0.0, 1.0)
            and repetition_context_size > 0):
        r["repetition_penalty"] = repetition_penalty
    if presence_penalty is not None and presence_penalty != 0.0 and presence_context_size > 0:
        r["presence_penalty"] = presence_penalty
    if frequency_penalty is not None and frequency_penalty != 0.0 and frequency_context_size > 0:
        r["frequency_penalty"] = frequency_penalty
    return r


def _params(rows):
    out = np.zeros(len(rows), PARAMS_DTYPE)
    for i, p in enumerate(rows):
        for k, v in p.items():
            out[i][k] = v
    return out


# ---------------------------------------------------------------- configs

def config1(vocab: int = V_QWEN) -> dict:
    """Single-row mlx-lm step: fp32 N(0,3^2) logits, 32 ids boosted +8,
    repetition 1.1 over the last 20 of a 512-token context, T=0.7, top-p 0.9."""
    rng = np.random.default_rng(1001)
    x = rng.normal(0.0, 3.0, vocab)
    boosted = rng.choice(vocab, 32, replace=False)
    x[boosted] += 8.0
    logits = x.astype(np.float32)[None, :]
    context = rng.integers(0, vocab, 512)
    ring = TokenRing(20)
    ring.load_prompt(context)
    row_ptr, entries = csr([mlxlm_entries(repetition=ring)])
    params = _params([resolve_mlxlm(temperature=0.7, top_p=0.9, repetition_penalty=1.1,
                                    repetition_context_size=20)])
    uniforms = rng.random(1, dtype=np.float32)
    return dict(name="c1", semantics=_ffi.SEM_MLXLM, dtype=_ffi.DTYPE_F32, rows=1, vocab=vocab,
                logits=logits, params=params, row_ptr=row_ptr, entries=entries, bitmask=None,
                mask_bits=0, uniforms=uniforms,
                workload=f"mlx-lm step B=1 V={vocab} fp32 rep1.1/20 T0.7 top-p0.9")


def config2(rows: int = 64, vocab: int = V_QWEN) -> dict:
    """Batched CBv2 step: bf16 N(0,3^2) + Zipf(1.1) log-prior per row, 2048-token
    Zipf(1.1) output histories with presence 0.5 / frequency 0.3, T=0.8,
    top-k 50, top-p 0.95, min-p 0.05."""
    rng = np.random.default_rng(1002)
    cdf = _zipf_cdf(1.1, vocab)
    prior = -1.1 * np.log(np.arange(1, vocab + 1, dtype=np.float64))
    logits = np.empty((rows, vocab), np.uint16)
    ents = []
    for r in range(rows):
        perm = rng.permutation(vocab)
        x = rng.normal(0.0, 3.0, vocab)
        x[perm] += prior
        logits[r] = f32_to_bf16_bits(x.astype(np.float32))
        hist = perm[zipf_ranks(rng, 1.1, vocab, 2048, cdf)]
        st = Cbv2RowState(prompt=[], output=hist, repetition_window=64, repetition_on=False,
                          counts_on=True, vocab=vocab)
        ents.append(st.entries())
    row_ptr, entries = csr(ents)
    p = resolve_cbv2(temperature=0.8, top_k=50, top_p=0.95, min_p=0.05, presence_penalty=0.5,
                     frequency_penalty=0.3, vocab=vocab)
    params = _params([p] * rows)
    uniforms = rng.random(rows, dtype=np.float32)
    return dict(name="c2", semantics=_ffi.SEM_CBV2, dtype=_ffi.DTYPE_BF16, rows=rows, vocab=vocab,
                logits=logits, params=params, row_ptr=row_ptr, entries=entries, bitmask=None,
                mask_bits=0, uniforms=uniforms,
                workload=f"CBv2 decode step B={rows} V={vocab} bf16 pres0.5 freq0.3 T0.8 "
                         "top-k50 top-p0.95 min-p0.05")


def config3(rows: int = 256, vocab: int = V_256K) -> dict:
    """Continuous-batching mixed step: bf16 N(0,4^2); 25% greedy rows; others
    T~U[0.3,1.2], top-k in {0,20,100}, top-p~U[0.8,1.0]; repetition
    U[1.0,1.3] over the last 64 tokens of 4096-token Zipf histories."""
    rng = np.random.default_rng(1003)
    cdf = _zipf_cdf(1.1, vocab)
    n_greedy = rows // 4
    greedy = set(rng.choice(rows, n_greedy, replace=False).tolist())
    logits = np.empty((rows, vocab), np.uint16)
    plist, ents = [], []
    for r in range(rows):
        x = rng.normal(0.0, 4.0, vocab)
        logits[r] = f32_to_bf16_bits(x.astype(np.float32))
        perm = rng.permutation(vocab)
        hist = perm[zipf_ranks(rng, 1.1, vocab, 4096, cdf)]
        rep = float(np.float32(rng.uniform(1.0, 1.3)))
        if r in greedy:
            p = resolve_cbv2(temperature=0.0, repetition_penalty=rep, repetition_context_size=64,
                             vocab=vocab)
        else:
            p = resolve_cbv2(temperature=float(np.float32(rng.uniform(0.3, 1.2))),
                             top_k=int(rng.choice([0, 20, 100])),
                             top_p=float(np.float32(rng.uniform(0.8, 1.0))),
                             repetition_penalty=rep, repetition_context_size=64, vocab=vocab)
        plist.append(p)
        st = Cbv2RowState(prompt=[], output=hist, repetition_window=64,
                          repetition_on=p["repetition_penalty"] != 1.0, counts_on=False,
                          vocab=vocab)
        ents.append(st.entries())
    row_ptr, entries = csr(ents)
    uniforms = rng.random(rows, dtype=np.float32)
    return dict(name="c3", semantics=_ffi.SEM_CBV2, dtype=_ffi.DTYPE_BF16, rows=rows, vocab=vocab,
                logits=logits, params=_params(plist), row_ptr=row_ptr, entries=entries,
                bitmask=None, mask_bits=0, uniforms=uniforms,
                workload=f"CBv2 mixed step B={rows} V={vocab} bf16 25% greedy rep/64")


def config4(rows: int = 64, vocab: int = V_QWEN) -> dict:
    """Grammar-constrained CBv2 step: fp32 N(0,3^2); packed uint32 bitmask per
    row with density cycling {0.1%, 2%, 30%, 100%}, one EOS-only row;
    repetition 1.1 over a 20-token history, T=0.6, top-p 0.9."""
    rng = np.random.default_rng(1004)
    words = (vocab + 31) // 32
    logits = rng.normal(0.0, 3.0, (rows, vocab)).astype(np.float32)
    bitmask = np.zeros((rows, words), np.uint32)
    densities = [0.001, 0.02, 0.30, 1.0]
    eos_row = rows - 1
    ents = []
    for r in range(rows):
        allowed = np.zeros(words * 32, bool)
        if r == eos_row:
            allowed[min(EOS_ID, vocab - 1)] = True
        else:
            d = densities[r % 4]
            if d >= 1.0:
                allowed[:vocab] = True
            else:
                n = max(1, int(round(d * vocab)))
                allowed[rng.choice(vocab, n, replace=False)] = True
        bits = np.packbits(allowed.reshape(-1, 32)[:, ::-1], axis=1)  # MSB-first bytes of each word
        bitmask[r] = bits.view(">u4").reshape(-1).astype(np.uint32)
        hist = rng.integers(0, vocab, 20)
        st = Cbv2RowState(prompt=[], output=hist, repetition_window=20, repetition_on=True,
                          counts_on=False, vocab=vocab)
        ents.append(st.entries())
    row_ptr, entries = csr(ents)
    p = resolve_cbv2(temperature=0.6, top_p=0.9, repetition_penalty=1.1,
                     repetition_context_size=20, vocab=vocab)
    uniforms = rng.random(rows, dtype=np.float32)
    return dict(name="c4", semantics=_ffi.SEM_CBV2, dtype=_ffi.DTYPE_F32, rows=rows, vocab=vocab,
                logits=logits, params=_params([p] * rows), row_ptr=row_ptr, entries=entries,
                bitmask=bitmask, mask_bits=vocab, uniforms=uniforms, eos_row=eos_row,
                workload=f"CBv2 grammar step B={rows} V={vocab} fp32 bitmask rep1.1/20 T0.6 "
                         "top-p0.9")


def config5(sequences: int = 32, window: int = 4, vocab: int = V_QWEN) -> dict:
    """MTP verify: target [S, W, V] bf16 N(0,3^2), draft [S, W-1, V] = target
    + N(0,1^2) (bf16), T=0.8, top-p 0.95 (CBv2 transform); uniforms for the
    draft draws, the acceptance tests and the residual / bonus draw."""
    rng = np.random.default_rng(1005)
    D = window - 1
    tgt = rng.normal(0.0, 3.0, (sequences, window, vocab)).astype(np.float32)
    tgt_bits = f32_to_bf16_bits(tgt)
    tgt_f = bf16_bits_to_f32(tgt_bits)
    dr = tgt_f[:, :D, :].astype(np.float64) + rng.normal(0.0, 1.0, (sequences, D, vocab))
    dr_bits = f32_to_bf16_bits(dr.astype(np.float32))
    p = resolve_cbv2(temperature=0.8, top_p=0.95, vocab=vocab)
    draft_uniforms = rng.random((sequences, D), dtype=np.float32)
    verify_uniforms = rng.random((sequences, window), dtype=np.float32)
    return dict(name="c5", semantics=_ffi.SEM_CBV2, dtype=_ffi.DTYPE_BF16, sequences=sequences,
                window=window, vocab=vocab, target=tgt_bits, draft=dr_bits,
                params=_params([p] * sequences), draft_uniforms=draft_uniforms,
                uniforms=verify_uniforms,
                workload=f"MTP verify S={sequences} W={window} V={vocab} bf16 T0.8 top-p0.95")


WORKLOADS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


def algorithmic_bytes(cfg: dict) -> int:
    """Bytes one step must move at minimum: the logits once, the sparse
    penalty table, the bitmask, uniforms, params and the tokens written."""
    if cfg["name"] == "c5":
        S, W, V = cfg["sequences"], cfg["window"], cfg["vocab"]
        return (S * W * V + S * (W - 1) * V) * 2 + S * (W - 1) * 4 + S * W * 4 + S * W * 4
    es = 4 if cfg["dtype"] == _ffi.DTYPE_F32 else 2
    B, V = cfg["rows"], cfg["vocab"]
    total = B * V * es + B * 4 + B * 4 + B * 32
    if cfg.get("entries") is not None:
        total += len(cfg["entries"]) * 16 + (B + 1) * 4
    if cfg.get("bitmask") is not None:
        total += cfg["bitmask"].nbytes
    return total
