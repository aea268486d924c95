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


def attend_blas(q, ck, cv, cpos, pos, n_rep: int = 1):
    """``attend``'s output through matrix products instead of ``einsum`` (no
    GQA repeat: each KV head's query rows are multiplied as one block), for
    benchmark-size checks where the einsum loops take minutes. Same
    promotion: scores in float64 when q or the keys are float64, else float32
    then float64 after the division by sqrt(D); softmax in float64; float32
    probabilities times V. Only the order of the float32 additions differs
    from ``attend`` (within float32 rounding of it, checked on the CPU).
    Returns out (T, H, D)."""
    T, H, D = q.shape
    Tk, Hkv = ck.shape[0], ck.shape[1]
    if H != Hkv * n_rep:
        raise ValueError("query heads must be n_rep times the KV heads")
    qg = np.ascontiguousarray(q.reshape(T, Hkv, n_rep, D).transpose(1, 0, 2, 3).reshape(Hkv, T * n_rep, D))
    s = np.matmul(qg, np.ascontiguousarray(ck.transpose(1, 2, 0)))          # (Hkv, T*n_rep, Tk)
    s = s.reshape(Hkv, T, n_rep, Tk).transpose(1, 0, 2, 3).reshape(T, H, Tk) / np.sqrt(D)
    masked = np.asarray(cpos)[None, :] > np.asarray(pos)[:, None]
    s = np.where(masked[:, None, :], -np.inf, s)
    probs = softmax64(s, axis=-1).astype(np.float32)
    pg = np.ascontiguousarray(probs.reshape(T, Hkv, n_rep, Tk).transpose(1, 0, 2, 3).reshape(Hkv, T * n_rep, Tk))
    out = np.matmul(pg, np.ascontiguousarray(cv.transpose(1, 0, 2)))       # (Hkv, T*n_rep, D)
    return out.reshape(Hkv, T, n_rep, D).transpose(1, 0, 2, 3).reshape(T, H, D)
