#!/usr/bin/env python3
"""Throughput of the self-speculative decode round on one MI355X.

Default workload (``--workload e2e``): Llama-3-8B shape (32 layers, d_model
4096, 32/8 GQA heads, head_dim 128, SwiGLU 14336, RoPE theta 500000, vocab
128256), bf16 random weights N(0, 0.02), batch 32, context 32768 tokens of
synthetic bf16 KV (N(0,1), 1% outlier channels x8) in 16-token pages with
shuffled block tables, drafter arms int8 group-64 keep 1.0 and int4 group-32
(fp16 scale/zero) keep 0.25 switched every 64 rounds, or half way through
the timed rounds when fewer than 128 are timed (each switch requantizes the
mirror), gamma chosen each round by the cost model (at most 20; 0 = a plain
full-KV step), temperature 0.8 rejection sampling. A step is one decode round over the
batch: gamma draft forwards against the mirror (replayed from a recorded HIP
graph per mirror layout; ``--eager`` runs them op by op), one gamma+1-row
verify forward against the full cache, acceptance, rollback and mirror
resync.

Printed on one line: accepted (emitted) tokens per second over the timed
rounds, plus ``roofline`` for the drafter attention (algorithmic bytes per
call / average call time from HIP events on the launch stream vs 8 TB/s;
with graphs the calls are timed right after the rounds on the run's own
mirror, under each arm) and ``cpu_baseline`` (the numpy oracle on a bounded
sample of the same round).

``--workload kernels`` times the attention kernels alone at the same shape
(drafter pass and 9-query verify pass over rotating layers) for profiling;
``--workload requant`` the mirror rebuild of an arm switch; ``--workload
accept`` one verify decision over the batch.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "draft-kv_amd"))

HBM_PEAK_GBS = 8000.0
METRIC = "accepted tok/s, Llama-3-8B shape b=32 ctx32k; drafter attn HBM GB/s vs peak"


def log(msg: str) -> None:
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=96)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--period", type=int, default=64)
    ap.add_argument("--baseline-steps", type=int, default=8)
    ap.add_argument("--workload", choices=["e2e", "kernels", "copy", "requant", "accept", "gemm"], default="e2e")
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--gamma", type=int, default=20)
    ap.add_argument("--verify-gamma", type=int, default=8,
                    help="--workload kernels: the verify pass runs verify_gamma + 1 queries per sequence")
    ap.add_argument("--temperature", type=float, default=0.8)
    ap.add_argument("--recompute-draft-stats", action="store_true",
                    help="accept workload: recompute the draft rows' normalisers in the call")
    ap.add_argument("--bits", type=int, default=4)
    ap.add_argument("--keep", type=float, default=0.25)
    ap.add_argument("--group", type=int, default=32)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-calibrate", action="store_true",
                    help="choose gamma with the nominal 8 TB/s cost model instead of one fitted to this device")
    ap.add_argument("--eager", action="store_true", help="run the draft steps eagerly (no HIP graphs)")
    return ap.parse_args()


# ---------------------------------------------------------------- synthetic KV
def fill_kv(store, n_heads: int, bs: int, d: int, seed: int = 1) -> None:
    """Fill the paged store with N(0,1) bf16 values, 1% of channels x8 (K pages
    are [head][row][d], V pages [head][d][row]); one 128 MB random tile is
    generated and copied over the store."""
    import torch
    per = store.shape[1]
    half = n_heads * bs * d
    rows = max(1, min(store.shape[0], (128 << 20) // (per * 2)))
    g = torch.Generator(device=store.device)
    g.manual_seed(seed)
    tile = torch.randn((rows, per), generator=g, device=store.device, dtype=torch.float32)
    n_out = max(1, round(0.01 * d))
    ch = torch.randperm(d, generator=torch.Generator().manual_seed(seed))[:n_out].tolist()
    k = tile[:, :half].view(rows, n_heads, bs, d)
    v = tile[:, half:].view(rows, n_heads, d, bs)
    for c in ch:
        k[..., c] *= 8.0
        v[:, :, c, :] *= 8.0
    tile = tile.to(store.dtype)
    for i in range(0, store.shape[0], rows):
        n = min(rows, store.shape[0] - i)
        store[i: i + n].copy_(tile[:n])


def shuffled_full_cache(L, H, D, batch, ctx, extra, dtype, seed=0):
    """Paged bf16 cache with ctx-1 synthetic rows per sequence and layer, in
    16-token blocks handed out from a shuffled free list."""
    import numpy as np
    from draftkv import PagedKVCache
    bs = 16
    max_tokens = ctx + extra
    nb = L * -(-max_tokens // bs)
    full = PagedKVCache(L, H, D, block_size=bs, n_blocks=nb, dtype=dtype, batch=batch, max_tokens=max_tokens)
    rng = np.random.default_rng(seed)
    for p in full.pools:
        rng.shuffle(p._stack)
    full.reserve([ctx - 1] * batch)
    fill_kv(full.store, H, bs, D)
    full.commit([ctx - 1] * batch)
    return full


def measured_traffic(key: str):
    """HBM bytes per call of a kernel, from the FETCH_SIZE / WRITE_SIZE counter
    runs summarised in profiles/ (scaled by a copy kernel of known size), or None."""
    path = os.path.join(ROOT, "profiles", "roofline_traffic.json")
    try:
        with open(path) as f:
            return float(json.load(f)[key]["traffic_bytes_per_call"])
    except (OSError, KeyError, ValueError):
        return None


def drafter_bytes(rows_per_seq, n_kv_heads, d, bits, group, q_heads):
    """Algorithmic bytes of one drafter attention call: codes + fp16 scale/zero
    for K and V of every kept row and KV head, the fp32 query and output, and a
    4-byte attention mass per kept row."""
    per_row = n_kv_heads * 2 * (d * bits / 8 + 4 * math.ceil(d / group))
    rows = float(sum(rows_per_seq))
    b = len(rows_per_seq)
    return rows * per_row + 2 * b * q_heads * d * 4 + rows * 4


def verify_bytes(ctx_per_seq, n_kv_heads, d, T, q_heads):
    """Algorithmic bytes of one verify attention call: bf16 K and V of every
    row and KV head, fp32 queries and outputs."""
    rows = float(sum(ctx_per_seq))
    b = len(ctx_per_seq)
    return rows * n_kv_heads * 2 * d * 2 + 2 * b * T * q_heads * d * 4


class EventTimer:
    """HIP events around every call of a bound method, on torch's current stream
    (the stream every draftkv launch goes to); ``tag(*args)`` is recorded per call."""

    def __init__(self, obj, name, tag=None):
        import torch
        self.obj, self.name = obj, name
        self.orig = getattr(obj, name)
        self.pairs, self.tags = [], []
        self.on = False

        def wrapped(*a, **k):
            if not self.on:
                return self.orig(*a, **k)
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            if tag is not None:
                self.tags.append(tag(*a, **k))
            s.record()
            r = self.orig(*a, **k)
            e.record()
            self.pairs.append((s, e))
            return r

        setattr(obj, name, wrapped)

    def restore(self):
        self.on = False
        setattr(self.obj, self.name, self.orig)

    def times_ms(self):
        return [s.elapsed_time(e) for s, e in self.pairs]

    def mean_us(self):
        if not self.pairs:
            return float("nan")
        return 1000.0 * sum(self.times_ms()) / len(self.pairs)


# ---------------------------------------------------------------- CPU baseline
def splitk_bytes(rows_per_seq, n_kv_heads, d, bits, group, q_heads):
    """Algorithmic bytes of the drafter's split-K kernel: codes + fp16
    scale/zero of every kept row and KV head, and the fp32 query (the mass
    and the output belong to the two passes after it)."""
    per_row = n_kv_heads * 2 * (d * bits / 8 + 4 * math.ceil(d / group))
    return float(sum(rows_per_seq)) * per_row + len(rows_per_seq) * q_heads * d * 4


def segment_path(arm, batch, n_kv_heads, d, q_heads) -> bool:
    """Whether dkv_drafter_attention runs the segment kernel for this arm and
    shape (one 8-wave block per sequence and KV head: 4-bit codes, head_dim
    128, 4 query heads and 4 groups per KV head, fp16 meta, batch x KV heads
    >= 256); it then writes the output and the mass itself, so its
    algorithmic bytes are the whole call's."""
    return (arm.bits <= 4 and d == 128 and q_heads == 4 * n_kv_heads and d // arm.group == 4
            and arm.scale_fp16 and batch * n_kv_heads >= 256)


def time_verify(full, n_q_heads: int, T: int, reps: int = 2):
    """Verify attention timed on the run's own full cache: T N(0,1) query rows
    per sequence at its last T positions, every layer, ``reps`` times, one
    HIP event pair per call on the launch stream. Returns (us per call, calls)."""
    import torch
    b = full.batch
    lens = full.lengths().astype("int64")
    g = torch.Generator(device=full.device)
    g.manual_seed(8)
    q = torch.randn((b, T, n_q_heads, full.d_head), generator=g, device=full.device)
    start = torch.as_tensor((lens - T).astype("int32")).to(full.device)
    max_len = int(lens.max())
    full.attend(0, q, start, max_len)
    torch.cuda.synchronize()
    t = EventTimer(full, "attend")
    t.on = True
    for _ in range(reps):
        for layer in range(full.n_layers):
            full.attend(layer, q, start, max_len)
    torch.cuda.synchronize()
    t.restore()
    return t.mean_us(), len(t.pairs)


def time_drafter(comp, full, arms, n_q_heads: int, reps: int = 4) -> dict:
    """Drafter attention timed on the decode run's own mirror, rebuilt under
    each arm in turn: every layer, ``reps`` times, with N(0,1) queries and the
    attention mass on (as in the draft steps). HIP events on the launch
    stream time each whole call and, through the library's timing hook, its
    segment (or split-K) kernel alone, with the events carried by that
    kernel's own launch. Returns {arm: {"call": [bytes, us, calls],
    "splitk": [bytes, us, calls]}}."""
    import numpy as np
    import torch
    from draftkv import ops
    L, b = comp.n_layers, comp.batch
    g = torch.Generator(device=comp.device)
    g.manual_seed(7)
    q = torch.randn((b, n_q_heads, comp.d_head), generator=g, device=comp.device)
    out = {}
    for arm in arms:
        if list(comp.cfgs) != [arm] * L:
            comp.rebuild_layers(full, list(range(L)), [arm] * L)
        comp.attend(0, q)
        torch.cuda.synchronize()
        rows = comp.rows()
        cb = kb = 0.0
        for layer in range(L):
            r = rows[:, layer].astype(np.float64)
            cb += reps * drafter_bytes(r, comp.n_kv_heads, comp.d_head, arm.bits, arm.group, n_q_heads)
            kfn = drafter_bytes if segment_path(arm, b, comp.n_kv_heads, comp.d_head, n_q_heads) else splitk_bytes
            kb += reps * kfn(r, comp.n_kv_heads, comp.d_head, arm.bits, arm.group, n_q_heads)
        # whole calls back to back, then the split-K kernel of each call
        # (again back to back: one event pair per call, summed at the end)
        t = EventTimer(comp, "attend")
        t.on = True
        for _ in range(reps):
            for layer in range(L):
                comp.attend(layer, q)
        torch.cuda.synchronize()
        t.restore()
        ops.drafter_kernel_timing(True)
        for _ in range(reps):
            for layer in range(L):
                comp.attend(layer, q)
        k_ms, k_n = ops.drafter_kernel_total_ms()
        ops.drafter_kernel_timing(False)
        torch.cuda.synchronize()
        out[arm] = {"call": [cb, sum(t.times_ms()) * 1e3, len(t.pairs)],
                    "splitk": [kb, k_ms * 1e3, k_n]}
    return out


def cpu_baseline(ctx: int, T: float, arms: list):
    """The numpy oracle on a bounded sample of the timed rounds: for each arm
    the GPU ran, one sequence, one decode round (gamma drafts at the arm's
    mean timed gamma, verify, accept, rollback, resync) of the Llama-3-8B
    shape with no decoder layer and with one over ctx synthetic rows, the
    per-layer time extrapolated to 32 layers; first with every BLAS thread,
    then with one. ``arms``: [(bits, keep, group, gamma, rounds, tokens per
    round per sequence)] as measured on the GPU. The rate mixes the arms' rounds
    as the timed region did: sum(rounds x tokens per round) / sum(rounds x
    round time). Returns (tok/s all threads, tok/s 1 thread, threads, sample)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    w = _oracle_llama_weights(ctx)
    per_arm, lines = [], []
    for bits, keep, group, gamma, rounds, tpr in arms:
        t_all = _oracle_round_time(w, ctx, gamma, T, bits, keep, group)
        with threadpool_limits(limits=1):
            t_one = _oracle_round_time(w, ctx, gamma, T, bits, keep, group)
        per_arm.append((rounds, tpr, t_all[2], t_one[2]))
        lines.append(f"int{bits} g{group} keep {keep} at gamma {gamma}: 0/1 layers {t_all[0]:.2f}/{t_all[1]:.2f} s, "
                     f"32 layers {t_all[2]:.1f} s per round ({t_one[2]:.1f} s on 1 thread), "
                     f"{tpr:.2f} tokens/round over {rounds} GPU rounds")
    tok = sum(r * t for r, t, _, _ in per_arm)
    v_all = tok / sum(r * a for r, _, a, _ in per_arm)
    v_one = tok / sum(r * o for r, _, _, o in per_arm)
    sample = ("numpy oracle, 1 sequence, one decode round per timed arm of the Llama-3-8B shape at ctx "
              f"{ctx} (T {T}), timed with 0 and 1 decoder layers and extrapolated to 32; "
              + "; ".join(lines) + "; rate = the timed region's round mix over the oracle's round times")
    return v_all, v_one, blas_threads(), sample


def _oracle_llama_weights(ctx: int):
    """One decoder layer, embedding and head of the Llama-3-8B shape (float32,
    uniform +-0.035, the oracle's own draw), ctx-1 rows of N(0,1) K/V per
    layer and a ctx-token prompt."""
    import numpy as np
    d, H, KV, D, ff, V = 4096, 32, 8, 128, 14336, 128256
    rng = np.random.default_rng(0)

    def R(*shape):
        return ((rng.random(shape, dtype=np.float32) - 0.5) * np.float32(0.0693)).astype(np.float32)

    emb = R(V, d)
    layer_w = {}
    for i in range(1):
        p = f"model.layers.{i}."
        layer_w[p + "input_layernorm.weight"] = np.ones(d, np.float32)
        layer_w[p + "post_attention_layernorm.weight"] = np.ones(d, np.float32)
        layer_w[p + "self_attn.q_proj.weight"] = R(H * D, d)
        layer_w[p + "self_attn.k_proj.weight"] = R(KV * D, d)
        layer_w[p + "self_attn.v_proj.weight"] = R(KV * D, d)
        layer_w[p + "self_attn.o_proj.weight"] = R(d, H * D)
        layer_w[p + "mlp.gate_proj.weight"] = R(ff, d)
        layer_w[p + "mlp.up_proj.weight"] = R(ff, d)
        layer_w[p + "mlp.down_proj.weight"] = R(d, ff)
    kv = [(rng.standard_normal((ctx - 1, KV, D)).astype(np.float32),
           rng.standard_normal((ctx - 1, KV, D)).astype(np.float32))]
    prompt = [int(x) for x in rng.integers(0, V, ctx)]
    return {"emb": emb, "layers": layer_w, "kv": kv, "prompt": prompt}


def _oracle_round_time(w, ctx, gamma, T, bits, keep, group):
    """Seconds of one oracle decode round with no decoder layer (embedding,
    head, sampling, accept) and with one, and the 32-layer extrapolation."""
    import numpy as np
    from oracle.caches import CompressedKVCache, FullKVCache
    from oracle.config import Cfg
    from oracle.engine import Engine, fixed
    from oracle.models import LlamaLike
    d, H, KV, D, V = 4096, 32, 8, 128, 128256
    emb, layer_w, kv, prompt = w["emb"], w["layers"], w["kv"], w["prompt"]
    cfg = Cfg(bits, keep, group=group, meta="f16")
    times = []
    for n_layers in (0, 0, 1):        # the first pass only pages the head in
        wl = {"model.embed_tokens.weight": emb, "model.norm.weight": np.ones(d, np.float32)}
        wl.update({k: v for k, v in layer_w.items() if int(k.split(".")[2]) < n_layers})
        c = dict(num_hidden_layers=n_layers, hidden_size=d, num_attention_heads=H, num_key_value_heads=KV,
                 head_dim=D, vocab_size=V, rms_norm_eps=1e-5, rope_theta=500000.0)
        m = LlamaLike(wl, c)

        full = FullKVCache(n_layers)
        for L in range(n_layers):
            full.append(L, kv[L][0], kv[L][1], np.arange(ctx - 1))
        eng = Engine(m, fixed(cfg, gamma), seed=0)
        comp = CompressedKVCache(n_layers, cfg)
        comp.sync_from(full, 0)
        # one round, timed: drafts + verify + accept + rollback + resync
        t0 = time.perf_counter()
        _oracle_one_round(eng, m, prompt, full, comp, gamma, T)
        times.append(time.perf_counter() - t0)
    t0, t1 = times[1], times[2]
    return t0, t1, t0 + 32 * max(t1 - t0, 1e-9)


def _oracle_one_round(eng, m, prompt, full, comp, gamma, T):
    """engine.py:173-221 for one round on prepared caches (the oracle engine's
    loop body, without its prefill); returns tokens emitted."""
    import numpy as np
    from oracle.sampling import probs
    tokens = list(prompt)
    n = len(tokens)
    drafts, qs = [], []
    x = tokens[-1]
    for i in range(gamma):
        lg = m.forward(np.array([x]), comp, n - 1 + i)[-1]
        q = probs(lg, T)
        x = eng._sample(q)
        drafts.append(x)
        qs.append(q)
    tl = m.forward(np.array([tokens[-1]] + drafts), full, n - 1)
    acc = 0
    for i in range(gamma):
        p = probs(tl[i], T)
        d = drafts[i]
        ratio = p[d] / qs[i][d] if qs[i][d] > 0 else 0.0
        if not eng.rng.random() < min(1.0, ratio):
            break
        acc += 1
    if acc == gamma:
        eng._sample(probs(tl[gamma], T))
    else:
        p = probs(tl[acc], T)
        resid = np.clip(p - qs[acc], 0.0, None)
        eng._sample(resid if resid.sum() > 0 else p)
    full.truncate(n + acc)
    comp.sync_from(full, n - 1)
    return acc + 1


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info
        n = [i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"]
        if n:
            return int(max(n))
    except Exception:
        pass
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


# ---------------------------------------------------------------- workloads
class ScheduledArms:
    """Arms switched on a fixed schedule (every ``period`` rounds), gamma chosen
    each round by the cost model from a decayed Beta posterior of the current
    arm's per-token acceptance (the controller protocol, controller.py:29-33).
    Gamma 0 -- a plain full-KV step -- when no draft length beats it, as the
    reference's controller declines to draft (controller.py:149-152)."""

    def __init__(self, arms, period, cost, ctx, gamma_max=20, decay=0.98):
        from draftkv.throughput import best_gamma
        self.best_gamma = best_gamma
        self.arms, self.period, self.cost, self.ctx = list(arms), period, cost, ctx
        self.gamma_max, self.decay = gamma_max, decay
        self.post = {a: [2.0, 1.0] for a in self.arms}
        self.round = 0
        self.gammas = []

    def select(self, ctx, key=None):
        arm = self.arms[(self.round // self.period) % len(self.arms)]
        a, b = self.post[arm]
        g, _ = self.best_gamma(self.cost, arm, a / (a + b), ctx, self.gamma_max)
        self.round += 1
        self.gammas.append(g)
        self.last_arm = arm
        return arm, g

    def update(self, cfg, gamma, accepted, ctx, key=None):
        p = self.post[cfg]
        p[0] = self.decay * p[0] + accepted
        p[1] = self.decay * p[1] + (1 if accepted < gamma else 0)


def run_e2e(args):
    import numpy as np
    import torch
    from draftkv import CompressionConfig, CostModel, DraftKVEngine
    from draftkv import ops
    from draftkv.calibrate import calibrate
    from draftkv.compress import _budget
    from draftkv.engine import DecodeBatch
    from draftkv.llama import LLAMA3_8B, LlamaLike

    cfgL = dict(LLAMA3_8B, num_hidden_layers=args.layers)
    L, Hkv, D, Hq = cfgL["num_hidden_layers"], cfgL["num_key_value_heads"], cfgL["head_dim"], \
        cfgL["num_attention_heads"]
    b, ctx = args.batch, args.ctx
    gmax = args.gamma
    rounds = args.warmup + args.steps
    cal_gammas = (1, min(4, gmax))
    cal_rounds = 0 if args.no_calibrate else 3 + 2 * (1 + 2 * len(cal_gammas))
    max_new = rounds * (gmax + 1) + cal_rounds * (max(cal_gammas) + 1) + args.baseline_steps + 2
    log(f"random Llama-3-8B-shape weights ({L} layers, bf16)")
    model = LlamaLike.random(cfgL, seed=0, std=0.02, dtype=torch.bfloat16)
    wbytes = float(sum(t.numel() * t.element_size() for p in model.layers
                       for t in (p.wqkv, p.wo, p.w1, p.w2))) + model.head.numel() * 2
    torch.cuda.synchronize()
    log(f"synthetic full cache: batch {b}, ctx {ctx}, {L} layers")
    full = shuffled_full_cache(L, Hkv, D, b, ctx, max_new + 16, torch.bfloat16)
    torch.cuda.synchronize()
    rng = np.random.default_rng(0)
    toks = [[int(x) for x in rng.integers(0, cfgL["vocab_size"], ctx)] for _ in range(b)]
    arms = [CompressionConfig(8, 1.0, group=64, scale_fp16=True),
            CompressionConfig(args.bits, args.keep, group=args.group, scale_fp16=True)]
    cost = CostModel(n_layers=L, n_kv_heads=Hkv, d_head=D, weight_bytes=wbytes, bandwidth=HBM_PEAK_GBS * 1e9,
                     batch=b)
    ctrl = ScheduledArms(arms, args.period, cost, ctx, gamma_max=gmax)
    eng = DraftKVEngine(model, ctrl, seed=0)
    batch = DecodeBatch(eng, toks, full, max_new, args.temperature, reserve_cfgs=arms, graphs=not args.eager)
    log("warmup rounds (the first builds the drafter mirror)")
    for _ in range(max(1, args.warmup)):
        batch.step()
    torch.cuda.synchronize()
    calibrated = None
    if not args.no_calibrate:
        # fit the cost model's time terms to this device: full-KV steps, then
        # each arm at two draft lengths (real decode rounds, before the timed ones)
        log(f"calibrating the cost model ({cal_rounds} rounds)")
        # (the arms in reverse, so the mirror ends up as the first timed round needs it)
        calibrated = calibrate(batch, cost, arms[::-1], gammas=cal_gammas, reps=2)
        ctrl.cost = calibrated
        torch.cuda.synchronize()
    comp = batch.comp
    # drafter calls are timed live when the draft steps run eagerly; replayed
    # draft-step graphs never pass through the Python call, so then the
    # drafter is timed right after the rounds, on the same mirror
    live = not batch.use_graphs
    t_draft = EventTimer(comp, "attend", tag=lambda layer, *a, **k: (comp.cfgs[layer], comp.seen.copy())) \
        if live else None
    # verify attention: the rounds only note each call's query count (an event
    # pair per call would put two markers, about 5 us of idle GPU each, into
    # every layer of every verify forward); the calls are timed after the rounds
    ver_T = []
    ver_orig = full.attend

    def ver_note(layer, q, *a, **k):
        ver_T.append(int(q.shape[1]))
        return ver_orig(layer, q, *a, **k)

    full.attend = ver_note
    t_req = EventTimer(comp, "rebuild_layers")
    timers = [t for t in (t_draft, t_req) if t is not None]
    for t in timers:
        t.on = True
    # the timed rounds cover both arms: the first arm for `period` rounds, then
    # the second; with fewer than 2 x period timed rounds the switch comes
    # half way through (so the requantize of the switch is timed too)
    period = args.period if args.steps >= 2 * args.period else max(1, args.steps // 2)
    ctrl.period, ctrl.round = period, 0
    log(f"timing {args.steps} rounds (arm switch every {period} rounds)")
    emitted = 0
    # arm -> [seconds, tokens, rounds]: the rounds of one arm run back to back,
    # and the device is drained once at each switch (and at the end), so an
    # arm's time holds all of its rounds' device work, its requantize included
    arm_time = {}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    seg_arm, seg_t0 = None, t0
    for _ in range(args.steps):
        nxt = ctrl.arms[(ctrl.round // ctrl.period) % len(ctrl.arms)]
        if seg_arm is not None and nxt != seg_arm:
            torch.cuda.synchronize()
            now = time.perf_counter()
            arm_time[seg_arm][0] += now - seg_t0
            seg_t0 = now
        seg_arm = nxt
        batch.step()
        emitted += batch.last_emitted
        at = arm_time.setdefault(ctrl.last_arm, [0.0, 0, 0])
        at[1] += batch.last_emitted
        at[2] += 1
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    arm_time[seg_arm][0] += t0 + dt - seg_t0
    batch.resolve_tokens()     # the declined rounds' tokens, already on the host
    for t in timers:
        t.on = False
    del full.attend            # the class method again
    per_arm = {}
    for r in batch.res:
        for x in r.rounds[-args.steps:]:
            st = per_arm.setdefault(x.cfg.label(), [0, 0, 0, 0])   # accepted, drafted, rounds, declined
            st[0] += x.accepted
            st[1] += x.gamma
            st[2] += 1
            st[3] += x.gamma == 0
    # drafter attention during the rounds (eager steps only): bytes of each
    # timed call from the rows the mirror held
    live_calls = {}
    if live:
        for (s_ev, e_ev), (cfg, seen) in zip(t_draft.pairs, t_draft.tags):
            rows = [min(int(n), _budget(cfg, int(n))) for n in seen]
            nbytes = drafter_bytes(rows, Hkv, D, cfg.bits, cfg.group, Hq)
            c = live_calls.setdefault(cfg, [0.0, 0.0, 0])
            c[0] += nbytes
            c[1] += s_ev.elapsed_time(e_ev) * 1e3
            c[2] += 1
    log("drafter attention and its dominant kernel timed on the run's mirror, under each arm")
    timed = time_drafter(comp, full, arms, Hq)
    main_arm = arms[1]
    seg = segment_path(main_arm, b, Hkv, D, Hq)
    mb, mus, mn = timed[main_arm]["call"]
    kbytes, kus, kn = timed[main_arm]["splitk"]
    achieved = kbytes / (kus * 1e-6) / 1e9
    traffic = None
    if (b, ctx, main_arm.bits, main_arm.group, main_arm.keep_frac) == (32, 32768, 4, 32, 0.25):
        traffic = measured_traffic("drafter_splitk_int4_g32_keep0.25_b32_ctx32k")
    # verify attention at the rounds' most frequent query count, every layer,
    # on the run's own cache (HIP events per call, as the rounds would be timed)
    v_T = max(set(ver_T), key=ver_T.count) if ver_T else 1
    v_us, v_n = time_verify(full, Hq, v_T)
    v_bytes = verify_bytes(full.lengths().astype(np.float64), Hkv, D, v_T, Hq)
    # plain full-KV decoding on the same cache (one token per sequence per step)
    log(f"baseline: {args.baseline_steps} full-KV decode steps")
    dev = model.device
    x = torch.as_tensor(np.array([t[-1] for t in batch.toks], np.int32)).to(dev)
    start = np.array([len(t) - 1 for t in batch.toks], np.int64)
    full.truncate(start)
    u = torch.rand((args.baseline_steps + 1, b), dtype=torch.float64, device=dev)
    lg = model.forward_batch(x[:, None], full, start)[:, 0]
    x = ops.sample(lg, args.temperature, u[0])
    torch.cuda.synchronize()
    tb0 = time.perf_counter()
    for i in range(args.baseline_steps):
        lg = model.forward_batch(x[:, None], full, start + 1 + i)[:, 0]
        x = ops.sample(lg, args.temperature, u[i + 1])
    x.cpu()
    torch.cuda.synchronize()
    base_tps = b * args.baseline_steps / (time.perf_counter() - tb0)
    value = emitted / dt
    # measured round speedup per arm against the cost model at 8 TB/s: its
    # ceiling (alpha -> 1, gamma -> inf) and its prediction at the measured
    # acceptance and mean gamma of that arm
    cost_model = {}
    cost_cal = {}
    for arm, (secs, tok, nr) in arm_time.items():
        st_ = per_arm.get(arm.label(), [0, 0, 0, 0])
        alpha_a = st_[0] / max(st_[1], 1)
        gam = max(1, round(st_[1] / max(st_[2], 1)))
        meas = (tok / secs) / base_tps
        # the model's best round at the measured acceptance (any gamma up to the bench's bound): what
        # the arm could reach on this workload however fast the kernels were, next to its ceiling
        best_g = max(range(1, args.gamma + 1), key=lambda g_: cost.speedup(arm, g_, alpha_a, ctx))
        best = cost.speedup(arm, best_g, alpha_a, ctx)
        cost_model[arm.label()] = {
            "rounds": nr, "tok_s": tok / secs, "measured_speedup": meas,
            "ceiling": cost.ceiling(arm, ctx), "frac_of_ceiling": meas / cost.ceiling(arm, ctx),
            "modeled_speedup": cost.speedup(arm, gam, alpha_a, ctx), "gamma": gam, "alpha": alpha_a,
            "frac_of_modeled": meas / cost.speedup(arm, gam, alpha_a, ctx),
            "best_modeled_speedup_at_alpha": best, "best_gamma_at_alpha": best_g,
            "best_at_alpha_frac_of_ceiling": best / cost.ceiling(arm, ctx)}
        if calibrated is not None:
            declined = st_[3] // max(b, 1)
            cost_cal[arm.label()] = {
                "ceiling": calibrated.ceiling(arm, ctx), "frac_of_ceiling": meas / calibrated.ceiling(arm, ctx),
                "modeled_speedup": calibrated.speedup(arm, gam, alpha_a, ctx),
                "frac_of_modeled": meas / calibrated.speedup(arm, gam, alpha_a, ctx),
                "declined_rounds": declined}
    if calibrated is not None:
        cost_cal["params"] = {
            "bandwidth_GBs": calibrated.bandwidth / 1e9, "full_kv_bandwidth_GBs": calibrated.full_kv_bandwidth / 1e9,
            "compute_per_token_us": calibrated.compute_per_token * 1e6,
            "fixed_draft_us": calibrated.fixed_draft * 1e6, "fixed_verify_us": calibrated.fixed_verify * 1e6,
            "resync_per_token_us": calibrated.resync_per_token * 1e6,
            "controller_overhead_us": calibrated.controller_overhead * 1e6}
    acc_total = sum(v[0] for v in per_arm.values())
    drafted = sum(v[1] for v in per_arm.values())
    alpha = {k: v[0] / max(v[1], 1) for k, v in per_arm.items()}
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": 1000.0 * dt / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init bf16 weights N(0,0.02); random token ids; synthetic N(0,1) KV with 1% "
                "outlier channels x8 written straight into the paged cache in place of a 32k prefill)",
        "config": {"workload": f"Llama-3-8B-shape decode rounds, batch {b}, ctx {ctx}, drafter arms int8 g64 "
                               f"keep 1.0 / int{args.bits} g{args.group} keep {args.keep} (fp16 scale/zero) "
                               f"switched every {period} rounds of the timed region (every {args.period}, or half "
                               f"way when fewer than {2 * args.period} rounds are timed), gamma by cost model (max {gmax}; 0 = a "
                               f"full-KV step when drafting does not pay; "
                               f"{'nominal 8 TB/s' if calibrated is None else 'fitted to this device'}), "
                               f"T {args.temperature} rejection sampling, 16-token pages, shuffled block tables",
                   "layers": L, "batch": b, "ctx": ctx, "temperature": args.temperature, "switch_period": period,
                   "rounds_per_arm": {k: v[2] // b for k, v in per_arm.items()},
                   "tok_s_per_arm": {a.label(): v[1] / v[0] for a, v in arm_time.items()},
                   "gamma_mean_per_arm": {k: v[1] / max(v[2], 1) for k, v in per_arm.items()},
                   "acceptance_per_arm": alpha, "acceptance": acc_total / max(drafted, 1),
                   "gamma_mean": float(np.mean(ctrl.gammas[-args.steps:])),
                   "tokens_per_round": emitted / args.steps / b,
                   "full_kv_decode_tok_s": base_tps, "speedup_vs_full_kv_decode": value / base_tps,
                   "requantize_ms": [round(t, 3) for t in t_req.times_ms()],
                   "draft_graphs": batch.use_graphs, "cost_model_8tbs": cost_model,
                   "cost_model_calibrated": cost_cal if calibrated is not None else None},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "traffic_source": "profiles/attention_hbm_traffic_b32_ctx32k.md (FETCH_SIZE x 2.0 + "
                                       "WRITE_SIZE, copy-kernel calibrated)" if traffic else None,
                     "kernel": f"drafter attention {'segment' if seg else 'split-K'} kernel, "
                               f"{main_arm.label()} g{main_arm.group} (the dominant kernel of "
                               "dkv_drafter_attention)",
                     "bytes_per_launch": kbytes / max(kn, 1), "us_per_launch": kus / max(kn, 1), "launches": kn,
                     "call": {"what": "segment kernel + mass sum" if seg else
                              "split-K + combine + mass", "bytes_per_call": mb / max(mn, 1),
                              "us_per_call": mus / max(mn, 1), "GB/s": mb / (mus * 1e-6) / 1e9,
                              "frac": mb / (mus * 1e-6) / 1e9 / HBM_PEAK_GBS, "calls": mn}},
        "kernels": {"verify_attention": {"us_per_call": v_us, "bytes_per_call": v_bytes,
                                         "GB/s": v_bytes / (v_us * 1e-6) / 1e9, "calls": v_n, "queries": v_T,
                                         "calls_in_rounds": len(ver_T)}},
    }
    for cfg, d in timed.items():
        (nb, us, n), (kb_, kus_, kn_) = d["call"], d["splitk"]
        out["kernels"][f"drafter_attention {cfg.label()} g{cfg.group}"] = {
            "us_per_call": us / n, "bytes_per_call": nb / n, "GB/s": nb / (us * 1e-6) / 1e9, "calls": n,
            "splitk_us": kus_ / kn_, "splitk_GB/s": kb_ / (kus_ * 1e-6) / 1e9}
    for cfg, (nb, us, n) in live_calls.items():
        out["kernels"][f"drafter_attention {cfg.label()} g{cfg.group} (live, in the rounds)"] = {
            "us_per_call": us / n, "bytes_per_call": nb / n, "GB/s": nb / (us * 1e-6) / 1e9, "calls": n}
    log(f"{emitted} tokens in {dt:.3f} s ({value:.1f} tok/s); full-KV decode {base_tps:.1f} tok/s; "
        f"acceptance {alpha}")
    del batch, comp, full, model, eng
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        log("cpu baseline (numpy oracle, bounded sample of the timed arms)")
        timed_arms = []
        for arm in arms:
            st_ = per_arm.get(arm.label())
            if not st_:
                continue
            nr = st_[2] // b
            timed_arms.append((arm.bits, arm.keep_frac, arm.group, round(st_[1] / max(st_[2], 1)), nr,
                               arm_time[arm][1] / max(arm_time[arm][2], 1) / b))
        v, v1, threads, sample = cpu_baseline(ctx, args.temperature, timed_arms)
        out["cpu_baseline"] = {"value": v, "unit": "tok/s", "cores": threads, "kind": "port",
                               "value_1thread": v1, "sample": sample}
    else:
        out["cpu_baseline"] = None
    return out


def run_kernels(args):
    """Attention kernels alone at the Llama-3-8B attention shape: drafter pass
    (1 query/sequence, int4 group-32 keep 0.25 mirror) and verify pass
    (gamma+1 queries/sequence over the bf16 cache), rotating over layers so no
    layer is re-read from cache."""
    import numpy as np
    import torch
    from draftkv import CompressedKVCache, CompressionConfig
    L = max(2, min(args.layers, 8))
    Hkv, D, Hq = 8, 128, 32
    b, ctx, gamma = args.batch, args.ctx, args.verify_gamma
    log(f"synthetic full cache: batch {b}, ctx {ctx}, {L} layers")
    full = shuffled_full_cache(L, Hkv, D, b, ctx + 1, gamma + 16, torch.bfloat16)
    arm = CompressionConfig(args.bits, args.keep, group=args.group, scale_fp16=True)
    comp = CompressedKVCache(L, arm, batch=b, cap=ctx + 64)
    comp.sync_from(full, 0)
    dev = full.store.device
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    qd = torch.randn((b, Hq, D), generator=g, device=dev)
    qv = torch.randn((b, gamma + 1, Hq, D), generator=g, device=dev)
    q1 = torch.randn((b, 1, Hq, D), generator=g, device=dev)
    start = torch.full((b,), ctx - 1 - gamma, dtype=torch.int32, device=dev)
    start1 = torch.full((b,), ctx - 1, dtype=torch.int32, device=dev)
    max_len = ctx

    def one_pass():
        for layer in range(L):
            comp.attend(layer, qd)
        for layer in range(L):
            full.attend(layer, qv, start, max_len)
        for layer in range(L):
            tdec.obj.attend_decode(layer, q1, start1, max_len)

    full.attend_decode = full.attend
    td, tv = EventTimer(comp, "attend"), EventTimer(full, "attend")
    tdec = EventTimer(full, "attend_decode")
    for _ in range(args.warmup):
        one_pass()
    torch.cuda.synchronize()
    td.on = tv.on = tdec.on = True
    for _ in range(args.steps):
        one_pass()
    torch.cuda.synchronize()
    rows = comp.rows().astype(np.float64).mean(axis=1)
    d_bytes = drafter_bytes(rows, Hkv, D, args.bits, args.group, Hq)
    v_bytes = verify_bytes(np.full(b, ctx - 1.0 - gamma / 2), Hkv, D, gamma + 1, Hq)
    dec_bytes = verify_bytes(np.full(b, ctx - 1.0), Hkv, D, 1, Hq)
    d_us, v_us, dec_us = td.mean_us(), tv.mean_us(), tdec.mean_us()
    achieved = d_bytes / (d_us * 1e-6) / 1e9
    return {
        "metric": "drafter / verify attention kernels, Llama-3-8B attention shape b=32 ctx32k",
        "value": achieved, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": (d_us + v_us) * L / 1000.0, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int4/bf16", "data": "synthetic",
        "config": {"workload": f"attention microbench b={b} ctx={ctx} int{args.bits} g{args.group} "
                               f"keep {args.keep} / verify {gamma + 1} queries", "layers": L},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "bytes_per_call": d_bytes,
                     "us_per_call": d_us},
        "kernels": {"verify_attention": {"us_per_call": v_us, "bytes_per_call": v_bytes,
                                         "GB/s": v_bytes / (v_us * 1e-6) / 1e9, "T": gamma + 1},
                    "decode_attention": {"us_per_call": dec_us, "bytes_per_call": dec_bytes,
                                         "GB/s": dec_bytes / (dec_us * 1e-6) / 1e9, "T": 1}},
        "cpu_baseline": None,
    }


def run_copy(args):
    """A plain device-to-device copy of 1 GiB, repeated: the reference dispatch
    for scaling FETCH_SIZE / WRITE_SIZE counter readings to bytes."""
    import torch
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / max(args.steps, 1)
    return {"metric": "device copy 1 GiB (counter calibration)", "value": 2 * n / dt / 1e9, "unit": "GB/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": dt * 1e3,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8", "data": "synthetic",
            "config": {"workload": "copy 1 GiB device to device", "bytes_read": n, "bytes_written": n}}


def run_requant(args):
    """Requantize alone (the mirror rebuild on an arm switch) at the
    Llama-3-8B attention shape: every layer of a batch x ctx mirror rebuilt
    from the bf16 full cache, alternating int8 group-64 keep 1.0 and
    int{bits} group-{group} keep {keep} (fp16 scale/zero), each call timed
    with HIP events on the launch stream. Algorithmic bytes: the kept rows'
    bf16 K and V read, their codes and scale/zero pairs written, and 12 B of
    position and score per kept row."""
    import numpy as np
    import torch
    from draftkv import CompressedKVCache, CompressionConfig
    from draftkv.compress import _budget
    L, Hkv, D = args.layers, 8, 128
    b, ctx = args.batch, args.ctx
    log(f"synthetic full cache: batch {b}, ctx {ctx}, {L} layers")
    full = shuffled_full_cache(L, Hkv, D, b, ctx, 16, torch.bfloat16)
    arms = [CompressionConfig(8, 1.0, group=64, scale_fp16=True),
            CompressionConfig(args.bits, args.keep, group=args.group, scale_fp16=True)]
    comp = CompressedKVCache(L, arms[0], batch=b, cap=ctx + 64, reserve_cfgs=arms)
    comp.sync_from(full, 0)
    t = EventTimer(comp, "rebuild_layers")
    for i in range(args.warmup):
        comp.rebuild_layers(full, list(range(L)), [arms[(i + 1) % 2]] * L)
    torch.cuda.synchronize()
    t.on = True
    tags = []
    for i in range(2 * args.steps):
        arm = arms[(args.warmup + i + 1) % 2]
        comp.rebuild_layers(full, list(range(L)), [arm] * L)
        tags.append(arm)
    torch.cuda.synchronize()
    t.restore()
    n = full.lengths()
    out_k = {}
    for arm, ms in zip(tags, t.times_ms()):
        kept = np.array([min(int(x), _budget(arm, int(x))) for x in n], np.float64)
        ng = -(-D // arm.group)
        per_row = Hkv * 2 * (D * 2 + D * arm.bits / 8 + ng * 4)
        nbytes = L * float(kept.sum()) * (per_row + 12)
        c = out_k.setdefault(f"{arm.label()} g{arm.group}", [0.0, 0.0, 0])
        c[0] += nbytes
        c[1] += ms * 1e3
        c[2] += 1
    kern = {k: {"us_per_call": v[1] / v[2], "bytes_per_call": v[0] / v[2], "GB/s": v[0] / (v[1] * 1e-6) / 1e9,
                "calls": v[2]} for k, v in out_k.items()}
    main = kern[f"{arms[1].label()} g{arms[1].group}"]
    return {"metric": f"requantize (mirror rebuild of {L} layers) GB/s, b={b} ctx={ctx}", "value": main["GB/s"],
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": main["us_per_call"] / 1e3, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16->int", "data": "synthetic",
            "config": {"workload": f"requantize {L} layers, batch {b}, ctx {ctx}, alternating arms"},
            "roofline": {"bound": "hbm", "achieved": main["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": main["GB/s"] / HBM_PEAK_GBS, "traffic": None},
            "kernels": kern, "cpu_baseline": None}


def run_accept(args):
    """Acceptance alone: one verify decision over the batch (target logits
    [batch, gamma+1, vocab] and draft logits [batch, gamma, vocab], float32
    N(0, 2^2), temperature rejection sampling), timed per call with HIP
    events. As in the decode round, the draft rows' normalisers come from the
    draft steps' samples (computed before the timed calls);
    --recompute-draft-stats times the call that recomputes them instead.
    Algorithmic bytes: every target logit read once, plus one draft row per
    sequence (the residual's q; every draft logit when recomputing)."""
    import torch
    from draftkv import ops
    b, g, V = args.batch, args.gamma, 128256
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    target = 2.0 * torch.randn((b, g + 1, V), generator=gen, device=dev)
    draft = 2.0 * torch.randn((g, b, V), generator=gen, device=dev)   # step-major, as the draft steps write it
    tok = torch.randint(0, V, (b, g), generator=gen, device=dev, dtype=torch.int32)
    u = torch.rand((b, g + 1), generator=gen, device=dev, dtype=torch.float64)
    T = args.temperature
    ds = None
    if T > 0 and not args.recompute_draft_stats:   # what the draft steps' samples leave behind
        ds = ops.row_stats(b, dev, (g,))
        for i in range(g):
            ops.sample(draft[i], T, u[:, i].contiguous(), stats_out=ds[i])
    for _ in range(args.warmup):
        ops.accept(target, draft, tok, T, u, ds)
    torch.cuda.synchronize()
    evs = []
    for _ in range(args.steps):
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_ev.record()
        ops.accept(target, draft, tok, T, u, ds)
        e_ev.record()
        evs.append((s_ev, e_ev))
    torch.cuda.synchronize()
    us = 1e3 * sum(a.elapsed_time(c) for a, c in evs) / len(evs)
    nbytes = 4.0 * b * ((2 * g + 1) if ds is None else (g + 2)) * V
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"metric": f"accept (verify decision) GB/s, b={b} gamma={g} vocab={V}", "value": gbs, "unit": "GB/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": us / 1e3,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32/f64",
            "data": "synthetic",
            "config": {"workload": f"accept b={b} gamma={g} T={T}",
                       "draft_stats": "recomputed" if ds is None else "from the draft samples"},
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "traffic": None, "bytes_per_call": nbytes, "us_per_call": us},
            "cpu_baseline": None}


def run_gemm(args):
    """The four projection GEMMs of a Llama-3-8B decoder layer (qkv 6144x4096,
    o 4096x4096 on the float32 attention output, gate/up 28672x4096 with the
    SwiGLU epilogue, down 4096x14336), bf16 weights N(0, 0.02), at the row
    counts of a b=32 decode step (M = 32), a gamma-2 verify (96) and a gamma-8
    verify (288), rotating over 8 layers' weights (3.5 GB, so every call
    streams its weights from HBM), stored tiled as the bf16 models store them
    (``ops.TiledW``). The 8 calls of a shape run back to back between one
    pair of HIP events on the launch stream; algorithmic bytes: the weights
    once, x once, y once."""
    import torch
    from draftkv import ops
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    d, ff, nq = 4096, 14336, 6144
    nl = 8
    shapes = {"qkv": (nq, d, torch.bfloat16, False), "o": (d, d, torch.float32, False),
              "gate_up": (2 * ff, d, torch.bfloat16, True), "down": (d, ff, torch.bfloat16, False)}
    W = {k: [ops.TiledW(torch.empty((n, kk), dtype=torch.bfloat16, device=dev).normal_(0, 0.02, generator=g))
             for _ in range(nl)] for k, (n, kk, _, _) in shapes.items()}
    res = {}
    for M in (32, 96, 288):
        X = {k: torch.randn((M, kk), generator=g, device=dev).to(xd) for k, (n, kk, xd, _) in shapes.items()}
        # one event pair around the nl calls of a shape (back to back, as in a
        # forward; a pair around every call would add its markers' idle gaps)
        per = {}
        for rep in range(args.warmup + args.steps):
            for k, (n, kk, xd, sw) in shapes.items():
                s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s_ev.record()
                for i in range(nl):
                    ops.gemm_bf16(X[k], W[k][i], None, torch.bfloat16, swiglu=sw)
                e_ev.record()
                if rep >= args.warmup:
                    per.setdefault(k, []).append((s_ev, e_ev))
        torch.cuda.synchronize()
        row = {}
        tot_b = tot_us = 0.0
        for k, (n, kk, xd, sw) in shapes.items():
            us = 1e3 * sum(a.elapsed_time(c) for a, c in per[k]) / (len(per[k]) * nl)
            nbytes = n * kk * 2 + M * kk * (4 if xd == torch.float32 else 2) + M * (n // 2 if sw else n) * 2
            row[k] = {"us": us, "GB/s": nbytes / (us * 1e-6) / 1e9, "frac": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}
            tot_b += nbytes
            tot_us += us
        row["layer"] = {"us": tot_us, "GB/s": tot_b / (tot_us * 1e-6) / 1e9,
                        "frac": tot_b / (tot_us * 1e-6) / 1e9 / HBM_PEAK_GBS}
        res[f"M={M}"] = row
        log(f"M={M}: layer {tot_us:.1f} us, {row['layer']['GB/s']:.0f} GB/s")
    main_ = res["M=32"]["layer"]
    return {"metric": "Llama-3-8B layer GEMMs (bf16 weights) GB/s at M=32", "value": main_["GB/s"], "unit": "GB/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": main_["us"] / 1e3,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "qkv / o / gate_up+SwiGLU / down GEMMs of a Llama-3-8B layer, M = 32, 96, 288"},
            "roofline": {"bound": "hbm", "achieved": main_["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": main_["frac"], "traffic": None},
            "kernels": res, "cpu_baseline": None}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the decode round runs on a "
              "single MI355X; multi-GPU sharding is a design note, not a measured path)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    out = {"e2e": run_e2e, "kernels": run_kernels, "copy": run_copy, "requant": run_requant,
           "accept": run_accept, "gemm": run_gemm}[args.workload](args)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
