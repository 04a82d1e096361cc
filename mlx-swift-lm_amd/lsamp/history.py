"""Host-side penalty state: builds the sparse per-row entry tables
(lsamp_penalty_entry) the kernels consume, from token histories.

This is where the reference's stateful penalty bookkeeping lives on the host:

* TokenRing (Evaluate.swift:518-570): ring of the last W token ids, loaded
  from a flattened prompt and appended one token per step; the three mlx-lm
  penalty contexts each own one (repetition, presence, frequency), each with
  its own context size.
* CBv2 state (LogitsPipelineV2.setRows :150-262, commit :357-384): the
  repetition window is the last W tokens of prompt + output (a ring with
  eviction); frequency / presence count output tokens only (unwindowed);
  logit bias per token.

Both produce entries {token, count, flags, bias}, one per distinct token id.
"""
from __future__ import annotations

from collections import Counter, deque
from typing import Dict, Iterable, List, Optional, Sequence

import numpy as np

from . import _ffi
from .api import PENALTY_DTYPE


class TokenRing:
    """Ring of the most recent `capacity` token ids (Evaluate.swift:518-570).

    `buffer` keeps the reference's slot layout (zero-padded, write index
    wrapping), so `valid_tokens` returns the ids in the same order the
    reference's `validTokens` does."""

    def __init__(self, capacity: int):
        if capacity <= 0:
            raise ValueError("capacity must be positive")
        self.capacity = capacity
        self.buffer = [0] * capacity
        self.count = 0
        self.write_index = 0

    @property
    def valid_tokens(self) -> Optional[List[int]]:
        if self.count == 0:
            return None
        return self.buffer[: self.count] if self.count < self.capacity else list(self.buffer)

    def load_prompt(self, prompt: Sequence[int]) -> None:
        tokens = [int(t) for t in np.asarray(prompt).reshape(-1)]
        n = len(tokens)
        if n <= self.capacity:
            self.buffer = tokens + [0] * (self.capacity - n)
            self.count = n
            self.write_index = n % self.capacity
        else:
            self.buffer = tokens[-self.capacity:]
            self.count = self.capacity
            self.write_index = 0

    def append(self, token: int) -> None:
        self.buffer[self.write_index] = int(token)
        self.write_index = (self.write_index + 1) % self.capacity
        self.count = min(self.count + 1, self.capacity)


def mlxlm_entries(repetition: Optional[TokenRing] = None, presence: Optional[TokenRing] = None,
                  frequency: Optional[TokenRing] = None) -> np.ndarray:
    """Entries of one row for the mlx-lm PenaltyProcessor: REPETITION flag for
    ids in the repetition ring, PRESENCE flag for ids in the presence ring,
    count = occurrences in the frequency ring."""
    flags: Dict[int, int] = {}
    counts: Counter = Counter()
    if repetition is not None and repetition.valid_tokens is not None:
        for t in repetition.valid_tokens:
            flags[t] = flags.get(t, 0) | _ffi.PEN_REPETITION
    if presence is not None and presence.valid_tokens is not None:
        for t in presence.valid_tokens:
            flags[t] = flags.get(t, 0) | _ffi.PEN_PRESENCE
    if frequency is not None and frequency.valid_tokens is not None:
        counts.update(frequency.valid_tokens)
    ids = sorted(set(flags) | set(counts))
    out = np.zeros(len(ids), PENALTY_DTYPE)
    for i, t in enumerate(ids):
        out[i] = (t, counts.get(t, 0), flags.get(t, 0), 0.0)
    return out


class Cbv2RowState:
    """Penalty state of one CBv2 row (LogitsPipelineV2.swift:150-262, 357-384).

    `window` is the ring of the last W ids of prompt + output with -1 for empty
    slots and the same write position the reference keeps, so eviction on
    `commit` matches `repWindowCounts` exactly."""

    def __init__(self, prompt: Sequence[int], output: Sequence[int], repetition_window: int,
                 repetition_on: bool, counts_on: bool, bias: Optional[Dict[int, float]] = None,
                 vocab: Optional[int] = None):
        self.vocab = vocab
        self.repetition_on = repetition_on
        self.counts_on = counts_on
        self.W = max(1, int(repetition_window))
        self.bias = {int(k): float(v) for k, v in (bias or {}).items()
                     if k >= 0 and (vocab is None or k < vocab)}
        history = [int(t) for t in prompt] + [int(t) for t in output]
        recent = history[-self.W:] if history else []
        self.window = [-1] * self.W
        for j, t in enumerate(recent):
            self.window[j] = t if t >= 0 else -1
        self.ring_pos = 0 if len(recent) == self.W else len(recent)
        self.output_counts: Counter = Counter(t for t in output if self._in_vocab(t))

    def _in_vocab(self, t: int) -> bool:
        return t >= 0 and (self.vocab is None or t < self.vocab)

    def commit(self, token: int) -> None:
        """LogitsPipelineV2.commit for one row (:357-384).  A token outside
        [0, vocab) -- the -1 of an EMPTY / OVERFLOW / TIMEOUT row, which the
        reference never produces -- commits nothing, as lsamp_commit and the
        oracle's lso_penalty_commit do: the ring does not advance."""
        token = int(token)
        if not self._in_vocab(token):
            return
        if self.counts_on:
            self.output_counts[token] += 1
        if self.repetition_on:
            self.window[self.ring_pos] = token
            self.ring_pos = (self.ring_pos + 1) % self.W

    def entries(self) -> np.ndarray:
        flags: Dict[int, int] = {}
        if self.repetition_on:
            for t in self.window:
                if self._in_vocab(t):
                    flags[t] = _ffi.PEN_REPETITION
        counts = self.output_counts if self.counts_on else Counter()
        ids = sorted(set(flags) | set(counts) | set(self.bias))
        out = np.zeros(len(ids), PENALTY_DTYPE)
        for i, t in enumerate(ids):
            out[i] = (t, counts.get(t, 0), flags.get(t, 0), self.bias.get(t, 0.0))
        return out


def csr(entries_per_row: Sequence[np.ndarray]):
    """Per-row entry arrays -> (row_ptr [B+1] int32, entries)."""
    sizes = [len(e) for e in entries_per_row]
    row_ptr = np.zeros(len(sizes) + 1, np.int32)
    row_ptr[1:] = np.cumsum(sizes)
    entries = (np.concatenate(entries_per_row) if sizes and sum(sizes)
               else np.zeros(0, PENALTY_DTYPE))
    return row_ptr, entries.astype(PENALTY_DTYPE)
