"""The draft/verify loop on the GPU.

Reference: draftkv/engine.py:25-223. Same invariant -- the caches hold K/V for
positions 0 .. len(tokens)-2 and the last token is pending -- the same round
(draft gamma tokens against the compressed mirror, verify gamma+1 rows against
the full cache, accept, roll back the full cache, resync the mirror) and the
same results (``GenerationResult``, ``RoundLog``).

What differs is where the work happens. A round runs a whole batch of
sequences in lockstep: every forward, sample and accept decision is a device
launch over the batch, and the host reads back one small block per round
(accepted counts, next tokens, draft tokens, uniforms consumed) to do the
bookkeeping the reference does in Python.

Random numbers follow the reference's stream exactly: sequence s draws from
``np.random.default_rng(seed + s)`` (sequence 0 is the reference's
``self.rng``). A round pre-draws its uniforms on the host -- one per draft
sample, then up to gamma accept tests plus one final sample -- and afterwards
rewinds the generator and advances it by the number the device decisions
consumed, so the stream stays where the reference's would be.
"""

from __future__ import annotations

import time
import warnings
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np
import torch

from . import ops
from .compress import CompressedKVCache
from .paged import PagedKVCache, auto_chunk_keys
from .graphs import DraftStepGraph, FullStepGraph, full_graph_key, graph_key
from .config import CompressionConfig
from .controller import Controller, FixedPolicy


def _layer_cfgs(cfg, n_layers: int) -> list:                        # engine.py:31-33
    return list(cfg.cfgs) if hasattr(cfg, "cfgs") else [cfg] * n_layers


@dataclass
class RoundLog:                                                     # engine.py:44-50
    cfg: CompressionConfig
    gamma: int
    accepted: int
    emitted: int
    ctx: int


@dataclass
class GenerationResult:                                             # engine.py:53-73
    tokens: list
    rounds: list = field(default_factory=list)
    draft_steps: int = 0
    verify_passes: int = 0
    cache_rebuilds: int = 0
    layers_rebuilt: int = 0

    @property
    def new_tokens(self) -> int:
        return sum(r.emitted for r in self.rounds)

    @property
    def acceptance_rate(self) -> float:
        drafted = sum(r.gamma for r in self.rounds)
        return sum(r.accepted for r in self.rounds) / drafted if drafted else float("nan")

    @property
    def tokens_per_verify(self) -> float:
        return self.new_tokens / self.verify_passes if self.verify_passes else float("nan")


class DraftKVEngine:
    """Self-speculative decoding where the drafter is the target model reading
    a compressed copy of its own KV cache (engine.py:76-99). Greedy output is
    identical to full-KV decoding; sampled output follows the speculative
    rejection rule."""

    def __init__(self, model, controller: Optional[Controller] = None, seed: int = 0,
                 full_cache_factory=None) -> None:
        self.model = model
        self.controller = controller or FixedPolicy(CompressionConfig(4, 0.5), 4)
        self.seed = seed
        self.rng = np.random.default_rng(seed)
        self._rngs = {0: self.rng}
        # swappable authoritative cache (engine.py:96-98); called with no
        # arguments and must hold as many sequences as the call has prompts
        self.full_cache_factory = full_cache_factory
        self.last_full = None       # the full cache of the last call (inspection, tests)
        self.last_mirror = None
        self.draft_graphs = True    # replay draft steps from recorded HIP graphs (DecodeBatch)

    # ------------------------------------------------------------------ util
    def _g(self, s: int) -> np.random.Generator:
        g = self._rngs.get(s)
        if g is None:
            g = self._rngs[s] = np.random.default_rng(self.seed + s)
        return g

    def _new_full(self, batch: int, max_tokens: int, span: Optional[int] = None):
        """The full cache of one call: ``max_tokens`` rows per sequence, and the
        attention key chunk chosen from ``span`` (longest prompt + new tokens;
        default max_tokens), which plain and speculative decoding of the same
        request share -- their rows then merge the same chunk partials in the
        same order, so the greedy outputs stay identical whatever room each
        path reserves."""
        if self.full_cache_factory is not None:
            c = self.full_cache_factory()
            if getattr(c, "batch", 1) != batch:
                raise ValueError(f"full_cache_factory made a cache for {getattr(c, 'batch', 1)} sequences, "
                                 f"need {batch}")
            return c
        ck = auto_chunk_keys(batch, self.model.n_kv_heads, max_tokens if span is None else span)
        return self.model.new_cache(batch=batch, max_tokens=max_tokens, chunk_keys=ck)

    def _prefill(self, prompts, full) -> None:
        lens = np.array([len(p) for p in prompts], np.int64)
        T = int(lens.max()) - 1
        if T <= 0:
            return
        tk = np.zeros((len(prompts), T), np.int32)
        for s, p in enumerate(prompts):
            tk[s, : len(p) - 1] = p[:-1]
        self.model.forward_batch(torch.as_tensor(tk).to(self.model.device), full, [0] * len(prompts), lens - 1)

    def _pending(self, toks) -> torch.Tensor:
        return ops.to_device(np.array([t[-1] for t in toks], np.int32), self.model.device)

    @staticmethod
    def _check_prompts(prompts, vocab: int):
        out = []
        for p in prompts:
            p = [int(x) for x in p]
            if not p:
                raise ValueError("prompts must hold at least one token")
            if min(p) < 0 or max(p) >= vocab:
                raise IndexError("token id out of range")
            out.append(p)
        return out

    # -------------------------------------------------------------- baseline
    def generate_baseline(self, prompt, max_new_tokens: int, temperature: float = 0.0) -> list:
        """Plain full-KV autoregressive decoding -- the reference output (engine.py:108-119)."""
        return self.generate_baseline_batch([prompt], max_new_tokens, temperature)[0]

    def generate_baseline_batch(self, prompts: Sequence, max_new_tokens: int, temperature: float = 0.0) -> list:
        model = self.model
        toks = self._check_prompts(prompts, model.vocab_size)
        b = len(toks)
        span = max(len(t) for t in toks) + max_new_tokens
        full = self._new_full(b, span + 16, span)
        self.last_full = full
        self._prefill(toks, full)
        dev = model.device
        x = self._pending(toks)
        start = np.array([len(t) - 1 for t in toks], np.int64)
        out = torch.empty((b, max_new_tokens), dtype=torch.int32, device=dev)
        u = np.stack([self._g(s).random(max_new_tokens) for s in range(b)], 1) if max_new_tokens else None
        u_d = torch.as_tensor(np.ascontiguousarray(u)).to(dev) if max_new_tokens else None
        for i in range(max_new_tokens):
            logits = model.forward_batch(x[:, None], full, start + i)[:, 0]
            x = ops.sample(logits, temperature, u_d[i])
            out[:, i] = x
        res = out.cpu().numpy()
        return [toks[s] + [int(v) for v in res[s]] for s in range(b)]

    # --------------------------------------------------------------- draftkv
    def generate(self, prompt, max_new_tokens: int, temperature: float = 0.0,
                 context_key: Optional[str] = None) -> GenerationResult:      # engine.py:122-223
        return self.generate_batch([prompt], max_new_tokens, temperature, context_key)[0]

    def generate_batch(self, prompts: Sequence, max_new_tokens: int, temperature: float = 0.0,
                       context_key: Optional[str] = None) -> list:
        """Decode every prompt with self-speculative rounds run in lockstep.

        One controller decision (config, gamma) per round serves the batch;
        gamma is capped by the largest remaining budget, and each sequence's
        output is cut to ``max_new_tokens`` at the end (with one prompt this is
        exactly the reference's cap ``min(gamma, budget - 1)``)."""
        toks = self._check_prompts(prompts, self.model.vocab_size)
        plen = np.array([len(t) for t in toks], np.int64)
        full = self._new_full(len(toks), rows_needed(plen, max_new_tokens, self.controller),
                              int(plen.max()) + max_new_tokens)
        self._prefill(toks, full)
        batch = DecodeBatch(self, toks, full, max_new_tokens, temperature, context_key)
        while batch.step():
            pass
        return batch.results()


def gamma_bound(controller, max_new_tokens: int) -> int:
    """The longest draft a round can run: the engine caps gamma at the largest
    remaining budget minus one (engine.py:175), and a controller that states
    its own bound (``gamma_max``, or a fixed ``gamma``) caps it further."""
    bound = max(int(max_new_tokens) - 1, 0)
    for attr in ("gamma_max", "gamma"):
        g = getattr(controller, attr, None)
        if isinstance(g, (int, np.integer)) and g >= 0:
            return min(bound, int(g))
    return bound


def rows_needed(plen, max_new_tokens: int, controller) -> int:
    """Cache rows per sequence that decoding ``max_new_tokens`` after prompts of
    lengths ``plen`` can write. A sequence is decoded while it has produced
    fewer than max_new tokens, so its pending position is at most
    len + max_new - 2, and a round writes gamma + 1 rows from there. In a
    batch, one gamma serves every sequence, so a sequence one token short of
    its budget still writes the whole verify block."""
    return int(np.max(plen)) + int(max_new_tokens) + gamma_bound(controller, max_new_tokens)


_RECORD = object()   # DecodeBatch._draft_graph: record a graph after this round's first step


class _Landed:
    """Event stand-in for a host tensor (nothing to wait for)."""

    def query(self) -> bool:
        return True

    def synchronize(self) -> None:
        pass


class DecodeBatch:
    """A batch in the middle of self-speculative decoding: token lists, the
    full cache (holding positions 0 .. len-2 of every sequence), the drafter
    mirror and the per-sequence random streams. ``step()`` runs one round
    (engine.py:138-221) for every unfinished sequence."""

    def __init__(self, engine: DraftKVEngine, toks: list, full, max_new_tokens: int, temperature: float = 0.0,
                 context_key: Optional[str] = None, reserve_cfgs: Sequence = (),
                 graphs: Optional[bool] = None) -> None:
        self.engine, self.model = engine, engine.model
        self.toks = toks
        self.full = full
        engine.last_full = full
        self.plen = np.array([len(t) for t in toks], np.int64)
        self.max_new = max_new_tokens
        self.T = float(temperature)
        self.key = context_key
        self.b = len(toks)
        self.res = [GenerationResult(tokens=toks[s]) for s in range(self.b)]
        self.comp: Optional[CompressedKVCache] = None
        self.comp_cfg = None
        # the mirror never holds more rows per segment than the sequence has positions
        need = rows_needed(self.plen, max_new_tokens, engine.controller)
        self.cap_tokens = min(int(getattr(full, "max_tokens", need) or need), need)
        self.last_emitted = 0             # tokens emitted by the last step, summed over the batch
        # arms the mirror may switch to: its pages are sized for the widest from the start
        self.reserve_cfgs = list(reserve_cfgs) or list(getattr(engine.controller, "arms", ()))
        # draft steps replayed from recorded HIP graphs (one per mirror layout)
        if graphs is None:
            graphs = getattr(engine, "draft_graphs", True)
        self.use_graphs = bool(graphs) and self.model.device.type == "cuda"
        self._graphs: dict = {}
        self._pool = None
        self._pending_key = None
        self.last_draft = None            # (tokens [b, gamma], logits [gamma, b, V]) of the last round's draft steps
        self.phases = None                # a calibrate.PhaseLog to record per-round phase times
        # A round that declines to draft (gamma 0) does not wait for its token:
        # the next round reads it from the device (_dev_pending), and the host
        # copy lands in a pinned buffer and fills the placeholder appended to
        # the token list when resolve_tokens() (or a drafted round's read-back)
        # comes to it. The token streams are the same; only the wait moves.
        self._dev_pending = None          # device int32 [b]: every sequence's last token
        self._deferred: list = []         # (pinned int32 [b], event, sequences, list positions)

    def _sync(self, start) -> None:
        self.comp.sync_from(self.full, start)

    # ------------------------------------------------------------ draft-step graphs
    def _draft_graph(self, n, act, gamma):
        """The recorded draft step for the mirror's current layout, _RECORD when
        this round should record one after an eager first step, or None (no
        graphs). Grows the mirror and the RoPE table for the round's positions
        first, so nothing the graph points at moves during the round."""
        model, comp, b = self.model, self.comp, self.b
        last = np.where(act > 0, n - 2 + gamma, 0)
        if model.pos_table is not None and int(last.max()) >= model.pos_table.shape[0]:
            raise IndexError(f"position {int(last.max())} beyond the position table ({model.pos_table.shape[0]})")
        model.prepare_mirror(comp, b, int((last + act).max()))
        if model.rope_theta is not None:
            model._cos_sin(int(last.max()) + 1)
        key = graph_key(model, comp, b, self.T)
        g = self._graphs.get(key)
        if g is not None:
            return g
        self._pending_key = key
        return _RECORD

    def _record_graph(self):
        key = self._pending_key
        try:
            if self._pool is None:
                self._pool = torch.cuda.graph_pool_handle()
            g = DraftStepGraph(self.model, self.comp, self.b, self.T, self._pool)
        except Exception as e:            # keep decoding eagerly
            warnings.warn(f"draft-step graph recording failed ({e}); decoding eagerly")
            self.use_graphs = False
            return None
        if g.key != key:
            raise RuntimeError("the mirror moved while a draft-step graph was recorded")
        while len(self._graphs) >= 4:     # a few arms' layouts; the oldest goes first
            self._graphs.pop(next(iter(self._graphs)))
        self._graphs[key] = g
        return g

    # ------------------------------------------------------------ gamma-0 step graphs
    def _full_key(self):
        """The key of the gamma-0 step graph for the current full cache, or
        None where none applies (a cache without device block tables)."""
        full, model = self.full, self.model
        if not isinstance(full, PagedKVCache) or not getattr(full, "_ready", True):
            return None
        if model.rope_theta is not None:
            model._cos_sin(min(self.cap_tokens, full.max_tokens))   # never regrown under the graph
        return full_graph_key(model, full, self.b, self.T, min(self.cap_tokens, full.max_tokens))

    def _full_graph(self, n, act):
        """The recorded gamma-0 step, or None: the round then runs eagerly and
        records one after (its first run warms every kernel and GEMM shape)."""
        model = self.model
        last = np.where(act > 0, n - 1, 0)
        if model.pos_table is not None and int(last.max()) >= model.pos_table.shape[0]:
            raise IndexError(f"position {int(last.max())} beyond the position table ({model.pos_table.shape[0]})")
        key = self._full_key()
        return None if key is None else self._graphs.get(key)

    def _record_full_graph(self) -> None:
        key = self._full_key()
        if key is None or key in self._graphs:
            return
        try:
            if self._pool is None:
                self._pool = torch.cuda.graph_pool_handle()
            g = FullStepGraph(self.model, self.full, self.b, self.T, min(self.cap_tokens, self.full.max_tokens),
                              self._pool)
        except Exception as e:            # keep decoding eagerly
            warnings.warn(f"gamma-0 step graph recording failed ({e}); decoding eagerly")
            self.use_graphs = False
            return
        if g.key != key:
            raise RuntimeError("the full cache moved while a gamma-0 step graph was recorded")
        while len(self._graphs) >= 4:
            self._graphs.pop(next(iter(self._graphs)))
        self._graphs[key] = g

    def _pending_dev(self) -> torch.Tensor:
        """The last token of every sequence as a device int32 [b]."""
        if self._dev_pending is not None:
            return self._dev_pending
        return self.engine._pending(self.toks)

    def resolve_tokens(self, wait: bool = True) -> None:
        """Write the tokens of declined rounds into the token lists (waiting
        for their copies when ``wait``; else only those already landed)."""
        keep = []
        for hbuf, ev, seqs, at in self._deferred:
            if not wait and not ev.query():
                keep.append((hbuf, ev, seqs, at))
                continue
            ev.synchronize()
            v = hbuf.numpy()
            for s, j in zip(seqs, at):
                self.toks[s][j] = int(v[s])
        self._deferred = keep

    def results(self) -> list:
        self.resolve_tokens()
        for s in range(self.b):
            del self.toks[s][int(self.plen[s]) + self.max_new:]
            self.res[s].tokens = self.toks[s]
        return self.res

    def step(self) -> bool:
        eng, model, toks, full, res, b, T = self.engine, self.model, self.toks, self.full, self.res, self.b, self.T
        dev, V = model.device, model.vocab_size
        n = np.array([len(t) for t in toks], np.int64)          # caches cover 0 .. n-2
        produced = n - self.plen
        active = produced < self.max_new
        self.last_emitted = 0
        self.last_draft = None
        if not active.any():
            self.resolve_tokens()
            return False
        self.resolve_tokens(wait=False)
        act = active.astype(np.int64)
        budget = np.where(active, self.max_new - produced, 0)
        ctx = int(n[active].max())
        cfg, gamma = eng.controller.select(ctx, self.key)
        gamma = min(int(gamma), max(int(budget.max()) - 1, 0))
        # a round writes rows n-1 .. n-1+gamma of every active sequence: never
        # more than the caches were sized for (a controller past its own bound)
        room = int(getattr(full, "max_tokens", 0) or 0)
        if room:
            gamma = max(0, min(gamma, room - int(n[active].max()), self.cap_tokens - int(n[active].max())))
        flen = full.lengths()

        ph, ev = self.phases, {}
        if gamma <= 0:
            u = np.array([eng._g(s).random() if active[s] else 0.5 for s in range(b)])
            if ph is not None:
                ev["d1"] = ph.event()
            graph = None
            if self.use_graphs:
                full.reserve(act)         # first: the pool may grow (and move) to take the rows
                graph = self._full_graph(n, act)
            if graph is not None:
                tok = graph.run(self._pending_dev(), n - 1, act, u)
                full.commit(act)
            else:
                u_d = ops.to_device(u, dev)
                logits = model.forward_batch(self._pending_dev()[:, None], full, n - 1, act)[:, 0]
                tok = ops.sample(logits, T, u_d)
                if self.use_graphs:
                    self._record_full_graph()
            if ph is not None:
                ev["v1"] = ph.event()
            # no wait: the next round reads tok on the device; the host copy
            # fills the placeholders when resolved
            if tok.device.type == "cuda":
                hbuf = torch.empty(tok.shape, dtype=tok.dtype, pin_memory=True)
                hbuf.copy_(tok, non_blocking=True)
                landed = torch.cuda.Event()
                landed.record()
                self._dev_pending = tok
            else:
                hbuf, landed = tok, _Landed()
            h0 = time.perf_counter()
            seqs = np.flatnonzero(active)
            for s in seqs:
                toks[s].append(-1)
                res[s].verify_passes += 1
                res[s].rounds.append(RoundLog(cfg, 0, 0, 1, int(n[s])))
            self._deferred.append((hbuf, landed, seqs, [len(toks[s]) - 1 for s in seqs]))
            self.last_emitted = int(active.sum())
            hs = time.perf_counter() - h0
            if ph is not None:
                ev["s0"] = ph.event()
            if self.comp is not None:
                self._sync(np.where(active, n - 1, full.lengths()))
            if ph is not None:
                ev["end"] = ph.event()
                ph.add(cfg, 0, ev, self.last_emitted, hs)
            return True

        # -- drafter's cache: build once, then rebuild only the layers that changed
        if self.comp is None:
            self.comp = CompressedKVCache(model.n_layers, cfg, batch=b, cap=self.cap_tokens, device=dev,
                                          reserve_cfgs=[c for a in self.reserve_cfgs
                                                        for c in _layer_cfgs(a, model.n_layers)])
            self.comp.sync_from(full, 0)
            self.comp_cfg = cfg
            for r in res:
                r.cache_rebuilds += 1
        elif self.comp_cfg != cfg:
            old, new = _layer_cfgs(self.comp_cfg, model.n_layers), _layer_cfgs(cfg, model.n_layers)
            changed = [L for L in range(model.n_layers) if old[L] != new[L]]
            self.comp.rebuild_layers(full, changed, new)
            self.comp_cfg = cfg
            for r in res:
                r.cache_rebuilds += 1
                r.layers_rebuilt += len(changed)
        comp = self.comp
        eng.last_mirror = comp

        # -- uniforms: gamma draft samples, then gamma+1 for verify
        states = {}
        u_draft = np.full((gamma, b), 0.5)
        u_ver = np.full((b, gamma + 1), 0.5)
        for s in np.flatnonzero(active):
            g = eng._g(s)
            u_draft[:, s] = g.random(gamma)
            states[s] = g.bit_generator.state
            u_ver[s] = g.random(gamma + 1)
        u_draft_d = ops.to_device(u_draft, dev)
        u_ver_d = ops.to_device(u_ver, dev)

        # -- draft
        x = self._pending_dev()
        pending = x
        draft_tok = torch.empty((b, gamma), dtype=torch.int32, device=dev)
        draft_logits = torch.empty((gamma, b, V), dtype=torch.float32, device=dev) if T > 0 else None   # step-major
        # the draft rows' normalisers, kept from each step's sample for the decision (as the
        # reference keeps the drafter's distributions, engine.py:176-179)
        draft_stats = ops.row_stats(b, dev, (gamma,)) if T > 0 else None
        graph = self._draft_graph(n, act, gamma) if self.use_graphs else None
        # with a graph for this layout recorded, every step replays it; on the
        # layout's first round step 0 runs eagerly (warming every kernel and GEMM
        # shape) and the graph is recorded after it
        n_eager = gamma if graph is None else (1 if graph is _RECORD else 0)
        if ph is not None:
            ev["d0"] = ph.event()
        for i in range(n_eager):
            lg = model.forward_batch(x[:, None], comp, n - 1 + i, act)[:, 0]
            if draft_logits is not None:
                draft_logits[i].copy_(lg)
            x = ops.sample(lg, T, u_draft_d[i], stats_out=None if draft_stats is None else draft_stats[i])
            draft_tok[:, i] = x
        if graph is _RECORD:
            graph = self._record_graph()
        if graph is not None:
            graph.run(x, [n - 1 + i for i in range(n_eager, gamma)], act, u_draft[n_eager:], draft_tok,
                      draft_logits, col0=n_eager, draft_stats=draft_stats)
        self.last_draft = (draft_tok, draft_logits)
        if ph is not None:
            ev["d1"] = ph.event()

        # -- verify
        block = torch.cat([pending[:, None], draft_tok], 1).contiguous()
        logits = model.forward_batch(block, full, n - 1, act * (gamma + 1))
        acc, nxt, used = ops.accept(logits, draft_logits, draft_tok, T, u_ver_d, draft_stats)
        if ph is not None:
            ev["v1"] = ph.event()
        host = torch.cat([torch.stack([acc, nxt, used], 1), draft_tok], 1).cpu().numpy()
        self.resolve_tokens()             # the read-back above waited for every earlier copy
        self._dev_pending = None

        # -- rollback and resync first (queued on the device), then the host's
        # bookkeeping, which runs while the device resyncs the mirror
        seqs = np.flatnonzero(active)
        cut = flen.copy()
        cut[seqs] = n[seqs] + host[seqs, 0]
        if ph is not None:
            ev["s0"] = ph.event()
        full.truncate(cut)
        self._sync(np.where(active, n - 1, full.lengths()))
        if ph is not None:
            ev["end"] = ph.event()
        h0 = time.perf_counter()
        emitted_total = 0
        for s in seqs:
            a, nx, k = int(host[s, 0]), int(host[s, 1]), int(host[s, 2])
            emitted = [int(t) for t in host[s, 3: 3 + a]] + [nx]
            toks[s].extend(emitted)
            emitted_total += len(emitted)
            g = eng._g(s)
            g.bit_generator.state = states[s]
            g.bit_generator.advance(k)
            eng.controller.update(cfg, gamma, a, int(n[s]), self.key)
            res[s].rounds.append(RoundLog(cfg, gamma, a, len(emitted), int(n[s])))
            res[s].draft_steps += gamma
            res[s].verify_passes += 1
        hs = time.perf_counter() - h0
        self.last_emitted = emitted_total
        if ph is not None:
            ph.add(cfg, gamma, ev, emitted_total, hs)
        return True
