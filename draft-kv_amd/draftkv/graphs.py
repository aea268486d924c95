"""HIP-graph replay of the draft step of a decode round.

A draft step (engine.py:173-185 of the reference: one forward of the pending
token against the drafter mirror, then a sample) is a few hundred short
kernels; at small batch the host cannot issue them as fast as the GPU runs
them. ``DraftStepGraph`` records one step -- embed, every layer's projections,
mirror append/evict and drafter attention, the head and the sample -- as one
HIP graph (torch.cuda.CUDAGraph) and replays it for the round's later steps.

What a step reads that changes from step to step sits in fixed device
buffers the graph was recorded with:
  * ``tok``: the token fed in; the sample writes the next one back in place;
  * ``inp``: the uniforms (float64 [b]), start positions, row counts (int32
    [b]) and the mirror's eviction budgets (int32 [n_layers, b]).
The host computes ``inp`` for all of a round's steps at once (the budgets
follow the mirror's ``seen`` counter step by step, as eager forwards would
move it) and ships them in one copy; each replay is preceded by a
device-to-device copy of its row. The graph holds raw pointers to the
mirror's buffers, the RoPE table and its own scratch (a private workspace),
so it is keyed on them and recorded again when any of them changes.

``FullStepGraph`` does the same for a round that declines to draft (gamma
0: engine.py:147-153 of the reference, one forward of the pending token
against the full cache, then a sample). It reads the start positions, row
counts and uniforms from its own fixed buffer; the full cache's block tables
are a device tensor that never moves (new blocks are written into it by
``reserve`` before the replay), and its attention is recorded for every key
up to the batch's position bound (the launch grows with that bound, the
arithmetic of each sequence does not: chunks past a sequence's end are
skipped, and the merge covers its own chunks only).
"""

from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import ops


def graph_key(model, comp, b: int, temperature: float) -> tuple:
    cs = getattr(model, "_cs", None)
    return (b, float(temperature), tuple(comp.cfgs), comp.cap, comp.page_stride, comp.pages.data_ptr(),
            comp.pos.data_ptr(), comp.score.data_ptr(), comp.n_rows.data_ptr(),
            None if cs is None else (cs.data_ptr(), model._cs_len))


class DraftStepGraph:
    """One recorded draft step for a fixed (model, mirror layout, arms, batch,
    temperature); see the module docstring."""

    def __init__(self, model, comp, b: int, temperature: float, pool) -> None:
        if model.device.type != "cuda":
            raise RuntimeError("draft-step graphs need a ROCm device")
        L = comp.n_layers
        dev = model.device
        self.model, self.comp, self.b, self.L, self.T = model, comp, b, L, float(temperature)
        self.key = graph_key(model, comp, b, temperature)
        # [u as 2b words | start b | count b | budgets L*b]
        self.n_words = 4 * b + L * b
        self.inp = torch.zeros(self.n_words, dtype=torch.int32, device=dev)
        self.u = self.inp[: 2 * b].view(torch.float64)
        self.start = self.inp[2 * b: 3 * b]
        self.count = self.inp[3 * b: 4 * b]
        self.budgets = self.inp[4 * b:].view(L, b)
        self.tok = torch.zeros(b, dtype=torch.int32, device=dev)
        self.stats = ops.row_stats(b, dev)   # the sampled rows' normalisers (for the verify decision)
        self.ws = ops.Workspace()
        self._rows_host: Optional[torch.Tensor] = None
        self._rows_dev: Optional[torch.Tensor] = None
        self._copied: Optional[torch.cuda.Event] = None   # the last copy out of the pinned rows
        self.replays = 0
        cs, cs_len = (None, 0)
        if model.rope_theta is not None:
            cs, cs_len = model._cos_sin(1)        # the table already sized by the eager forwards
        attn = model.mirror_attn(comp, b, self.start, self.budgets, self.count)
        self.graph = torch.cuda.CUDAGraph()
        with ops.private_workspace(self.ws):
            with torch.cuda.graph(self.graph, pool=pool):
                lg = model._core(self.tok, self.start, b, 1, attn, cs, cs_len)[:, 0]
                ops.sample(lg, self.T, self.u, out=self.tok, stats_out=self.stats if self.T > 0 else None)
        self.logits = lg

    def _rows(self, n: int):
        if self._rows_host is None or self._rows_host.shape[0] < n:
            self._rows_host = torch.empty((n, self.n_words), dtype=torch.int32, pin_memory=True)
            self._rows_dev = torch.empty((n, self.n_words), dtype=torch.int32, device=self.model.device)
        return self._rows_host, self._rows_dev

    def run(self, x0: torch.Tensor, starts: np.ndarray, act: np.ndarray, u: np.ndarray, draft_tok: torch.Tensor,
            draft_logits: Optional[torch.Tensor], col0: int = 0,
            draft_stats: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Run len(starts) steps from token x0 (int32 [b], device): step i
        appends at starts[i] (int [b]) the rows act (0/1 [b]) with uniforms
        u[i] ([b]); tokens go to draft_tok[:, col0 + i], logits (when given)
        to draft_logits[col0 + i] (step-major: one contiguous copy) and the
        rows' normalisers (when given) to draft_stats[col0 + i]. The mirror's
        ``seen`` advances as the eager
        steps would move it. Returns the last sampled token (a device view)."""
        steps, b = len(starts), self.b
        if steps == 0:
            return x0
        if self._copied is not None:
            self._copied.synchronize()          # the pinned rows are free again
        host, dev = self._rows(steps)
        rows = host.numpy()
        for i in range(steps):
            st = np.where(act > 0, starts[i], 0)
            budgets = self.comp.step_budgets(st, act)
            rows[i, : 2 * b] = np.ascontiguousarray(u[i], np.float64).view(np.int32)
            rows[i, 2 * b: 3 * b] = st
            rows[i, 3 * b: 4 * b] = act
            rows[i, 4 * b:] = budgets.reshape(-1)
        dev[:steps].copy_(host[:steps], non_blocking=True)
        self._copied = torch.cuda.Event()
        self._copied.record()
        self.tok.copy_(x0)
        for i in range(steps):
            self.inp.copy_(dev[i])
            self.graph.replay()
            self.replays += 1
            if draft_logits is not None:
                draft_logits[col0 + i].copy_(self.logits)
            if draft_stats is not None:
                draft_stats[col0 + i].copy_(self.stats)
            draft_tok[:, col0 + i].copy_(self.tok)
        return self.tok


def full_graph_key(model, full, b: int, temperature: float, max_len: int) -> tuple:
    cs = getattr(model, "_cs", None)
    return (b, float(temperature), full.store.data_ptr(), full.d_tables.data_ptr(), int(max_len),
            full.chunk_keys, None if cs is None else (cs.data_ptr(), model._cs_len))


class FullStepGraph:
    """One recorded gamma-0 step (a plain forward of the pending token over the
    full cache and its sample) for a fixed (model, full cache, batch,
    temperature); see the module docstring."""

    def __init__(self, model, full, b: int, temperature: float, max_len: int, pool) -> None:
        """max_len: a bound on every sequence's key count (its last position + 1)
        over the graph's life; the RoPE table is grown to it first."""
        if model.device.type != "cuda":
            raise RuntimeError("full-step graphs need a ROCm device")
        dev = model.device
        self.model, self.full, self.b, self.T = model, full, b, float(temperature)
        self.max_len = max_len = int(min(max_len, full.max_tokens))
        cs, cs_len = (None, 0)
        if model.rope_theta is not None:
            cs, cs_len = model._cos_sin(max_len)
        self.key = full_graph_key(model, full, b, temperature, max_len)
        # [u as 2b words | start b | count b]
        self.n_words = 4 * b
        self.inp = torch.zeros(self.n_words, dtype=torch.int32, device=dev)
        self.u = self.inp[: 2 * b].view(torch.float64)
        self.start = self.inp[2 * b: 3 * b]
        self.count = self.inp[3 * b:]
        self.tok = torch.zeros(b, dtype=torch.int32, device=dev)
        self.ws = ops.Workspace()
        self._host = torch.empty(self.n_words, dtype=torch.int32, pin_memory=True)
        self._copied: Optional[torch.cuda.Event] = None
        self.replays = 0
        attn = model.paged_attn(full, self.start, self.count, max_len)
        self.graph = torch.cuda.CUDAGraph()
        with ops.private_workspace(self.ws):
            with torch.cuda.graph(self.graph, pool=pool):
                lg = model._core(self.tok, self.start, b, 1, attn, cs, cs_len)[:, 0]
                ops.sample(lg, self.T, self.u, out=self.tok)
        self.logits = lg

    def run(self, x0: torch.Tensor, start: np.ndarray, act: np.ndarray, u: np.ndarray) -> torch.Tensor:
        """One step from token x0 (int32 [b], device): sequence s appends its
        row at start[s] when act[s] (rows of inactive sequences are neither
        written nor read), samples with uniform u[s]. The caller reserves the
        cache's blocks before and commits the rows after. Returns the sampled
        tokens (a new device tensor)."""
        b = self.b
        if self._copied is not None:
            self._copied.synchronize()            # the pinned row is free again
        row = self._host.numpy()
        row[: 2 * b] = np.ascontiguousarray(u, np.float64).view(np.int32)
        row[2 * b: 3 * b] = np.where(act > 0, start, 0)
        row[3 * b:] = act
        self.inp.copy_(self._host, non_blocking=True)
        self._copied = torch.cuda.Event()
        self._copied.record()
        self.tok.copy_(x0)
        self.graph.replay()
        self.replays += 1
        return self.tok.clone()
