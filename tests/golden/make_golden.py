"""Writes tests/golden/reference_vectors.npz from the reference implementation.

Run in the build container (where the read-only reference checkout exists):

    python tests/golden/make_golden.py /root/reference

It imports the reference's ``draftkv`` package and records, for small seeded
cases, the quantities that only the reference itself pins:

* exact float32 logits of ``demo_model``, ``demo_llama`` (GQA + bias) and a
  small random GPT-2 forward (numpy float64 promotion included);
* the drafter mirror after a greedy run with keep < 1: per-layer kept
  positions and accumulated scores (steady-state heavy-hitter eviction);
* per-round accepted counts and emitted tokens of greedy keep < 1 runs;
* emitted tokens and per-round accepted counts of temperature-sampling runs
  for a fixed seed (the reference's draw order);
* quantize() outputs for a few shapes (group 64, the reference default).

The oracle tests compare the numpy restatement under ``oracle/`` with these
vectors; nothing at run time (tests on the GPU box, smoke, bench) reads the
reference.
"""

from __future__ import annotations

import os
import sys

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_vectors.npz")


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from draftkv import CompressionConfig, DraftKVEngine, FixedPolicy
    from draftkv.compress import CompressedKVCache, FullKVCache, quantize
    from draftkv.gpt2 import GPT2
    from draftkv.llama import demo_llama
    from draftkv.model import demo_model

    out: dict[str, np.ndarray] = {}

    # quantize
    rng = np.random.default_rng(7)
    for i, (shape, bits) in enumerate([((5, 2, 16), 4), ((3, 4, 64), 8), ((2, 3, 80), 2), ((4, 1, 128), 3)]):
        x = (rng.standard_normal(shape) * (i + 1)).astype(np.float32)
        out[f"quant{i}_x"] = x
        out[f"quant{i}_bits"] = np.int64(bits)
        out[f"quant{i}_deq"] = quantize(x, bits)

    # forwards
    m = demo_model()
    toks = np.random.default_rng(11).integers(0, m.vocab_size, 40)
    out["tiny_tokens"] = toks
    out["tiny_logits"] = m.forward(toks, FullKVCache(m.n_layers), 0)
    ml = demo_llama(n_heads=8, n_kv_heads=2, attn_bias=True, seed=3)
    out["llama_tokens"] = toks
    out["llama_logits"] = ml.forward(toks, FullKVCache(ml.n_layers), 0)
    gcfg = dict(n_layer=2, n_embd=32, n_head=4, vocab_size=97, n_positions=256)
    grng = np.random.default_rng(5)
    gw = {}
    d, ff = 32, 128
    gw["wte.weight"] = (grng.standard_normal((97, d)) * 0.02).astype(np.float32)
    gw["wpe.weight"] = (grng.standard_normal((256, d)) * 0.02).astype(np.float32)
    for i in range(2):
        p = f"h.{i}."
        for n, s in (("attn.c_attn.weight", (d, 3 * d)), ("attn.c_proj.weight", (d, d)),
                     ("mlp.c_fc.weight", (d, ff)), ("mlp.c_proj.weight", (ff, d))):
            gw[p + n] = (grng.standard_normal(s) * 0.2).astype(np.float32)
        for n, s in (("attn.c_attn.bias", 3 * d), ("attn.c_proj.bias", d), ("mlp.c_fc.bias", ff),
                     ("mlp.c_proj.bias", d), ("ln_1.bias", d), ("ln_2.bias", d)):
            gw[p + n] = (grng.standard_normal(s) * 0.1).astype(np.float32)
        gw[p + "ln_1.weight"] = (1 + grng.standard_normal(d) * 0.1).astype(np.float32)
        gw[p + "ln_2.weight"] = (1 + grng.standard_normal(d) * 0.1).astype(np.float32)
    gw["ln_f.weight"] = np.ones(d, np.float32)
    gw["ln_f.bias"] = np.zeros(d, np.float32)
    for k, v in gw.items():
        out["gpt2w_" + k] = v
    g = GPT2(gw, gcfg)
    gt = np.random.default_rng(12).integers(0, 97, 30)
    out["gpt2_tokens"] = gt
    out["gpt2_logits"] = g.forward(gt, FullKVCache(2), 0)

    # greedy keep<1 runs: accepted sequence + final mirror state
    prompt = [int(x) for x in np.random.default_rng(0).integers(0, m.vocab_size, 192)]
    out["run_prompt"] = np.array(prompt)
    for j, (bits, keep, gamma) in enumerate([(4, 0.5, 3), (2, 0.25, 6), (3, 0.5, 4)]):
        cfg = CompressionConfig(bits, keep)
        eng = DraftKVEngine(m, FixedPolicy(cfg, gamma), seed=0)
        r = eng.generate(prompt, 32, 0.0)
        out[f"greedy{j}_cfg"] = np.array([bits, keep, gamma], np.float64)
        out[f"greedy{j}_tokens"] = np.array(r.tokens)
        out[f"greedy{j}_accepted"] = np.array([x.accepted for x in r.rounds])
    # mirror state after drafting (steady-state eviction), driven by hand so the
    # cache object is reachable
    full = FullKVCache(m.n_layers)
    m.forward(np.array(prompt[:-1]), full, 0)
    comp = CompressedKVCache(m.n_layers, CompressionConfig(4, 0.25))
    comp.sync_from(full, 0)
    x = prompt[-1]
    n = len(prompt)
    drafted = []
    for i in range(8):
        lg = m.forward(np.array([x]), comp, n - 1 + i)[-1]
        x = int(np.argmax(lg))
        drafted.append(x)
    out["mirror_drafts"] = np.array(drafted)
    for L in range(m.n_layers):
        out[f"mirror_pos{L}"] = np.array(comp.pos[L])
        out[f"mirror_score{L}"] = np.array(comp.score[L])

    # temperature runs
    pr = [int(x) for x in np.random.default_rng(3).integers(0, m.vocab_size, 64)]
    out["temp_prompt"] = np.array(pr)
    for j, (bits, keep, gamma, seed) in enumerate([(8, 1.0, 4, 4), (2, 0.25, 6, 4)]):
        r = DraftKVEngine(m, FixedPolicy(CompressionConfig(bits, keep), gamma), seed=seed).generate(pr, 24, 1.0)
        out[f"temp{j}_cfg"] = np.array([bits, keep, gamma, seed], np.float64)
        out[f"temp{j}_tokens"] = np.array(r.tokens)
        out[f"temp{j}_accepted"] = np.array([x.accepted for x in r.rounds])
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, sum(v.nbytes for v in out.values()), "bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
