"""Sampling helpers and the accept rule of one verify pass, restated.

Reference: draftkv/engine.py:25-41 (``_softmax``, ``_probs``), :101-106
(``_sample``), :188-213 (accept loop, bonus token, residual resample).

The reference samples with ``rng.choice(V, p=p/s)``. numpy's Generator
implements that as ``searchsorted(cdf, rng.random(), side="right")`` with
``cdf = cumsum(p); cdf /= cdf[-1]`` -- one 64-bit draw per call, also when p
is one-hot. ``sample_u`` takes that uniform explicitly so the oracle and the
HIP accept kernel can be fed the same draw; ``tests/test_oracle_engine.py``
pins the equivalence by running numpy.
"""

from __future__ import annotations

import numpy as np


def softmax64(x):                                         # engine.py:25-28
    x = x - x.max(-1, keepdims=True)
    e = np.exp(x)
    return e / e.sum(-1, keepdims=True)


def probs(logits: np.ndarray, temperature: float) -> np.ndarray:   # engine.py:36-41
    if temperature <= 0.0:
        p = np.zeros_like(logits, dtype=np.float64)
        p[int(np.argmax(logits))] = 1.0
        return p
    return softmax64(logits.astype(np.float64) / temperature)


def sample_u(p: np.ndarray, u: float) -> int:
    """``_sample`` (engine.py:101-106) with the uniform supplied: clip at 0,
    then the first index whose normalised cumulative sum exceeds ``u``.
    (The ``rng.integers`` branch for an all-zero p is not reachable from
    softmax or residual inputs and is not restated.)"""
    p = np.clip(p, 0.0, None)
    s = p.sum()
    if s <= 0:
        raise ValueError("all-zero distribution")
    c = np.cumsum(p / s)
    c /= c[-1]
    return int(np.searchsorted(c, u, side="right"))


def accept(target_logits, draft_tokens, draft_probs, temperature, uniforms):
    """One verify decision (engine.py:188-213).

    target_logits (gamma+1, V) float32; draft_tokens (gamma,); draft_probs
    list of gamma (V,) float64 (``_probs`` of the drafter's logits);
    uniforms: the draws the reference would make, in order -- one per
    tested position (sampling mode only), then one for the final token.

    Returns ``(accepted, next_token, n_uniforms_used)``.
    """
    gamma = len(draft_tokens)
    used = 0
    accepted = 0
    for i in range(gamma):
        if temperature <= 0.0:
            ok = int(np.argmax(target_logits[i])) == int(draft_tokens[i])
        else:
            p = probs(target_logits[i], temperature)
            q = draft_probs[i]
            d = int(draft_tokens[i])
            ratio = p[d] / q[d] if q[d] > 0 else 0.0
            ok = uniforms[used] < min(1.0, ratio)
            used += 1
        if not ok:
            break
        accepted += 1
    if accepted == gamma:
        nxt = sample_u(probs(target_logits[gamma], temperature), uniforms[used])
        used += 1
    else:
        p = probs(target_logits[accepted], temperature)
        if temperature <= 0.0:
            nxt = int(np.argmax(target_logits[accepted]))
        else:
            resid = np.clip(p - draft_probs[accepted], 0.0, None)
            nxt = sample_u(resid if resid.sum() > 0 else p, uniforms[used])
            used += 1
    return accepted, nxt, used
