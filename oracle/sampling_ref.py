"""Restatement of the top-k / top-p sampler's rule in numpy (float64), for the tests only.

The reference calls ``flashinfer.sampling.top_k_top_p_sampling_from_logits(logits, top_k=,
top_p=, deterministic=True)`` (ecahlang/main.py:377-379, 400-402, 489-491, 582-584); FlashInfer
(0.6.5, not vendored here) is the arithmetic.  Its published contract, with the default
``filter_apply_order="top_k_first"``: keep the top-k tokens of softmax(logits), renormalise, keep
the top-p nucleus of that, sample.  Its random stream is its own, so a draw is compared through
the uniform number that selects it: this restatement maps (row, u) to a token by inverse CDF in
vocabulary order, the same rule the kernel implements, and the tests check distributions
against it rather than FlashInfer's exact draws ("parity unpinned" for the draw itself; the kept
set and the distribution are pinned by closed forms in tests/test_oracle_sampling.py).

  K = {i : x_i >= k-th largest x}            (everything when k <= 0 or k >= V; ties kept)
  S = {i in K : x_i >= t}, t the largest logit with mass({j in K : x_j >= t}) >= top_p * mass(K)
  token = first i in S (vocabulary order) with cumulative mass over S > u * mass(S)
"""
from __future__ import annotations

import numpy as np


def kept_set(x: np.ndarray, top_k: int, top_p: float) -> np.ndarray:
    """Boolean mask of S for one row of logits."""
    x = np.asarray(x, dtype=np.float64)
    V = x.shape[0]
    ok = ~np.isnan(x)
    xs = np.where(ok, x, -np.inf)
    keep = ok.copy()
    if 0 < top_k < V:
        kth = np.sort(xs)[::-1][top_k - 1]
        keep &= xs >= kth
    if top_p < 1.0:
        m = np.exp(xs - xs[ok].max()) * keep
        need = max(top_p, 0.0) * m.sum()
        vals = np.unique(xs[keep])[::-1]  # distinct kept logits, descending
        acc = 0.0
        t = vals[-1]
        for v in vals:
            acc += m[xs == v].sum()
            if acc >= need:
                t = v
                break
        keep &= xs >= t
    return keep


def probabilities(x: np.ndarray, top_k: int, top_p: float) -> np.ndarray:
    """The distribution the sampler draws from (zero outside S)."""
    x = np.asarray(x, dtype=np.float64)
    keep = kept_set(x, top_k, top_p)
    xs = np.where(np.isnan(x), -np.inf, x)
    m = np.exp(xs - xs[keep].max()) * keep
    return m / m.sum()


def sample(x: np.ndarray, top_k: int, top_p: float, u: float) -> int:
    """Inverse CDF in vocabulary order: the first token of S whose cumulative mass exceeds u."""
    p = probabilities(x, top_k, top_p)
    c = np.cumsum(p)
    return int(min(np.searchsorted(c, u * c[-1], side="right"), len(c) - 1))
