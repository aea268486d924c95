"""Masked softmax attention over a cache read, restated.

Reference call sites (identical maths in all three models):
draftkv/model.py:117-127, draftkv/gpt2.py:197-206, draftkv/llama.py:202-218.

numpy 2 promotion is part of the semantics: ``einsum(q, k)`` in float32 (or
float64 when the Llama RoPE made q/k float64) divided by ``np.sqrt(D)`` (a
float64 numpy scalar) is float64, so the mask and softmax run in float64 and
the probabilities are cast to float32 before the PV product.
"""

from __future__ import annotations

import numpy as np


def softmax64(x: np.ndarray, axis: int = -1) -> np.ndarray:
    x = x - x.max(axis=axis, keepdims=True)
    e = np.exp(x)
    return e / e.sum(axis=axis, keepdims=True)


def attend(q, ck, cv, cpos, pos, n_rep: int = 1):
    """q (T, H, D); ck/cv (Tk, Hkv, D); cpos (Tk,), pos (T,).

    Returns ``(out (T, H, D) float32, probs (T, H, Tk) float32,
    mass_probs (T, Hkv, Tk) float32)`` where ``mass_probs`` is what the model
    hands to ``note_attention`` (probabilities summed over each GQA query group,
    llama.py:213-216; equal to ``probs`` for multi-head attention).
    """
    T, H, D = q.shape
    if n_rep > 1:
        ck = np.repeat(ck, n_rep, axis=1)
        cv = np.repeat(cv, n_rep, axis=1)
    scores = np.einsum("qhd,khd->qhk", q, ck) / np.sqrt(D)
    masked = np.asarray(cpos)[None, :] > np.asarray(pos)[:, None]
    scores = np.where(masked[:, None, :], -np.inf, scores)
    probs = softmax64(scores, axis=-1).astype(np.float32)
    if n_rep > 1:
        mass_probs = probs.reshape(T, H // n_rep, n_rep, -1).sum(axis=2)
    else:
        mass_probs = probs
    out = np.einsum("qhk,khd->qhd", probs, cv)
    return out, probs, mass_probs


def row_mass(mass_probs: np.ndarray) -> np.ndarray:
    """What ``note_attention`` adds to each row's score (compress.py:148): the
    float32 sum over (queries, heads)."""
    return mass_probs.sum(axis=(0, 1))
