"""The draft -> verify -> accept -> roll back/resync loop, restated.

Reference: draftkv/engine.py:76-223 (``DraftKVEngine.generate`` and
``generate_baseline``). Invariant (engine.py:1-12): the caches hold positions
``0 .. len(tokens)-2``; the last token is pending.

The random stream is ``np.random.default_rng(seed)``; every draw the reference
makes -- one per ``_sample`` (the drafter's, the bonus/residual one) and one
per tested position in sampling mode -- is taken in the reference's order.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .caches import CompressedKVCache, FullKVCache
from .config import Cfg
from .sampling import probs, sample_u


@dataclass
class Round:
    cfg: object
    gamma: int
    accepted: int
    emitted: int
    ctx: int


@dataclass
class Result:
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


def _layer_cfgs(cfg, n_layers):                            # engine.py:31-33
    return list(cfg) if isinstance(cfg, (list, tuple)) else [cfg] * n_layers


class Engine:
    def __init__(self, model, policy, seed: int = 0, full_cache_factory=None):
        """``policy(ctx) -> (cfg, gamma)`` (a fixed policy in the tests)."""
        self.model = model
        self.policy = policy
        self.rng = np.random.default_rng(seed)
        self.full_cache_factory = full_cache_factory or (lambda: FullKVCache(model.n_layers))

    def _sample(self, p):                                  # engine.py:101-106
        return sample_u(p, self.rng.random())

    def generate_baseline(self, prompt, max_new_tokens, temperature=0.0):   # engine.py:109-120
        tokens = list(prompt)
        cache = self.full_cache_factory()
        if len(tokens) > 1:
            self.model.forward(np.array(tokens[:-1]), cache, 0)
        for _ in range(max_new_tokens):
            logits = self.model.forward(np.array([tokens[-1]]), cache, len(tokens) - 1)[-1]
            tokens.append(self._sample(probs(logits, temperature)))
        return tokens

    def generate(self, prompt, max_new_tokens, temperature=0.0, trace=None):   # engine.py:123-223
        m = self.model
        tokens = list(prompt)
        full = self.full_cache_factory()
        if len(tokens) > 1:
            m.forward(np.array(tokens[:-1]), full, 0)
        comp, comp_cfg = None, None
        res = Result(tokens=tokens)
        while len(tokens) - len(prompt) < max_new_tokens:
            n = len(tokens)
            budget = max_new_tokens - (n - len(prompt))
            cfg, gamma = self.policy(n)
            gamma = min(gamma, max(budget - 1, 0))
            if gamma <= 0:
                logits = m.forward(np.array([tokens[-1]]), full, n - 1)[-1]
                tokens.append(self._sample(probs(logits, temperature)))
                res.verify_passes += 1
                res.rounds.append(Round(cfg, 0, 0, 1, n))
                if comp is not None:
                    comp.sync_from(full, n - 1)
                continue
            if comp is None:
                comp = CompressedKVCache(m.n_layers, _layer_cfgs(cfg, m.n_layers))
                comp.sync_from(full, 0)
                comp_cfg = cfg
                res.cache_rebuilds += 1
            elif comp_cfg != cfg:
                old, new = _layer_cfgs(comp_cfg, m.n_layers), _layer_cfgs(cfg, m.n_layers)
                changed = [L for L in range(m.n_layers) if old[L] != new[L]]
                comp.rebuild_layers(full, changed, new)
                comp_cfg = cfg
                res.cache_rebuilds += 1
                res.layers_rebuilt += len(changed)
            drafts, qs, dlogits = [], [], []
            x = tokens[-1]
            for i in range(gamma):
                lg = m.forward(np.array([x]), comp, n - 1 + i)[-1]
                q = probs(lg, temperature)
                x = self._sample(q)
                drafts.append(x)
                qs.append(q)
                dlogits.append(lg)
            res.draft_steps += gamma
            tl = m.forward(np.array([tokens[-1]] + drafts), full, n - 1)
            res.verify_passes += 1
            acc = 0
            for i in range(gamma):
                if temperature <= 0.0:
                    ok = int(np.argmax(tl[i])) == drafts[i]
                else:
                    p = probs(tl[i], temperature)
                    d = drafts[i]
                    ratio = p[d] / qs[i][d] if qs[i][d] > 0 else 0.0
                    ok = self.rng.random() < min(1.0, ratio)
                if not ok:
                    break
                acc += 1
            emitted = list(drafts[:acc])
            if acc == gamma:
                nxt = self._sample(probs(tl[gamma], temperature))
            else:
                p = probs(tl[acc], temperature)
                if temperature <= 0.0:
                    nxt = int(np.argmax(tl[acc]))
                else:
                    resid = np.clip(p - qs[acc], 0.0, None)
                    nxt = self._sample(resid if resid.sum() > 0 else p)
            emitted.append(nxt)
            tokens.extend(emitted)
            if trace is not None:
                trace.append(dict(n=n, drafts=drafts, draft_logits=dlogits, target_logits=tl,
                                  accepted=acc, next=nxt))
            full.truncate(n + acc)
            comp.sync_from(full, n - 1)
            res.rounds.append(Round(cfg, gamma, acc, len(emitted), n))
        res.tokens = tokens
        return res


def fixed(cfg: Cfg, gamma: int):
    return lambda ctx: (cfg, gamma)
