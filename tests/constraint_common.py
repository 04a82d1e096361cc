"""Token constraints of the reference's constraint tests
(Tests/MLXLMTests/CBv2TokenConstraintSamplingTests.swift:6-58) and a keyed
automaton for the mask cache, shared by the CPU and GPU tests."""
from __future__ import annotations

import numpy as np


class FixedTokenConstraint:
    """One allowed token per state, along a fixed path (:6-28)."""

    def __init__(self, path):
        self.path = list(path)
        self.initial_state = 0
        self.max_tokens = len(self.path)
        self.fallback_token_id = self.path[-1] if self.path else 0

    def allowed_token_ids(self, state, remaining):
        if not (0 <= state < len(self.path)) or remaining <= 0:
            return []
        return [self.path[state]]

    def next_state(self, state, token):
        if not (0 <= state < len(self.path)) or token != self.path[state]:
            return None
        return state + 1


class ImpossibleTokenConstraint:
    """Every state is impossible (:30-38)."""
    initial_state, max_tokens, fallback_token_id = 0, 4, 0

    def allowed_token_ids(self, state, remaining):
        return []

    def next_state(self, state, token):
        return None


class DenseTokenConstraint:
    """Every token but one (:40-58)."""
    initial_state, max_tokens, fallback_token_id = 0, 1, 0

    def __init__(self, vocab, excluding):
        self.allowed = [t for t in range(vocab) if t != excluding]
        self.excluded = excluding

    def allowed_token_ids(self, state, remaining):
        return self.allowed if remaining > 0 else []

    def next_state(self, state, token):
        return None if token == self.excluded else 1


class CyclicKeyedConstraint:
    """A keyed automaton over `states` states, each allowing a fixed random
    subset of the vocabulary; the cache key is the state (the allowed set
    ignores the budget while it is positive)."""

    def __init__(self, vocab, states, density, seed, max_tokens=10_000, fallback=0):
        rng = np.random.default_rng(seed)
        self.sets = [np.sort(rng.choice(vocab, max(1, int(vocab * density)), replace=False))
                     for _ in range(states)]
        self.initial_state, self.max_tokens, self.fallback_token_id = 0, max_tokens, fallback
        self.calls = 0

    def allowed_token_ids(self, state, remaining):
        self.calls += 1
        return self.sets[state].tolist() if remaining > 0 else []

    def next_state(self, state, token):
        return (state + 1) % len(self.sets) if token in set(self.sets[state].tolist()) else None

    def mask_cache_key(self, state, remaining):
        return state if remaining > 0 else None
