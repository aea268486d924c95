"""The drafter's kernels at the Llama-3-8B attention shape the benchmark runs
(32 query heads, 8 KV heads, head_dim 128; batch 32, ~32k positions per
sequence in a bf16 cache of 16-token pages with shuffled block tables),
against the oracle through the C ABI.

At this shape the mirror is built by the compile-time requantize kernel (bf16
source, 16-token blocks, head_dim 128), the int4 group-32 arm's attention
streams 32-row pages through the LDS ring of its split-K kernel (every wave
walks many pages, so the ring wraps and the pipelined page loop runs), and
the int8 group-64 fp16-meta arm runs the register-staged kernel -- the paths
toy shapes never reach. Sequence lengths are ragged (32767 - 37 s), so the
recent window of the keep-0.25 arm starts at a different offset inside a
16-token block in every sequence.

Bit-exact: kept positions, codes and scale/zero bit patterns after the
build, an arm switch, a draft step with eviction by the accumulated mass,
and the rollback resync. Attention: 2e-3 relative / 1e-3 absolute against
the float32 oracle; attention mass: 1e-4 relative.

The verify pass (gamma + 1 query rows per sequence over
the full bf16 cache) is checked at the same shape with the cache's own key
chunk (8192 keys: four chunk partials merged per row) for T = 1, 9 and 17
rows, which run the MFMA kernel with 1, 4 and 8 waves; and at batch 1 with
262144 positions (2048-key chunks, 128 partials per row) for T = 17.

The oracle quantizes only the kept rows of a build: its quantizer works row
by row (compress.py:38-43), so that equals quantizing every row and then
evicting (checked on the CPU in test_oracle_caches.py).
"""

import concurrent.futures as cf

import numpy as np
import pytest
import torch

from oracle import caches as oc
from oracle.attention import attend, attend_blas, row_mass
from oracle.config import Cfg, budget, closed_form_kept
from oracle.quant import quantize_codes

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-3, 1e-3
B, CTX, HKV, HQ, D, L = 32, 32768, 8, 32, 128, 2
LAYER = 1                              # the layer under test (layer 0 holds other rows)
INT4 = Cfg(4, 0.25, group=32, meta="f16")
INT8 = Cfg(8, 1.0, group=64, meta="f16")
INT4H = Cfg(4, 0.5, group=32, meta="f16")    # ~16k rows: 64 pages per wave of the segment kernel
LENS = np.array([CTX - 1 - 37 * s for s in range(B)], np.int64)
_POOL = cf.ThreadPoolExecutor(8)       # the numpy oracle per sequence (it releases the GIL)


def _dcfg(c: Cfg):
    from draftkv import CompressionConfig
    return CompressionConfig(c.bits, c.keep_frac, c.sink, c.recent, c.group, c.meta == "f16")


@pytest.fixture(scope="module")
def cache(dev):
    """A bf16 paged cache of L layers at the benchmark shape: N(0,1) K/V with
    two outlier channels x8, ragged lengths, shuffled free lists. Returns the
    device cache and the host copy (bf16) of layer LAYER."""
    import draftkv
    maxt = CTX + 64
    full = draftkv.PagedKVCache(L, HKV, D, 16, L * (maxt // 16), "bf16", batch=B, max_tokens=maxt)
    rng = np.random.default_rng(2)
    for p in full.pools:
        rng.shuffle(p._stack)
    full.reserve(LENS)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    T = int(LENS.max())
    cnt = torch.tensor(LENS, dtype=torch.int32, device=dev)
    st0 = torch.zeros(B, dtype=torch.int32, device=dev)
    host = None
    for layer in range(L):
        kv = []
        for _ in range(2):
            x = torch.randn((B, T, HKV, D), generator=g, device=dev, dtype=torch.float32)
            x[..., [5, 77]] *= 8.0
            kv.append(x.bfloat16())
            del x
        full.append_layer(layer, kv[0], kv[1], st0, cnt)
        if layer == LAYER:
            host = (kv[0].cpu(), kv[1].cpu())
        del kv
    full.commit(LENS)
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    yield full, host
    del full
    torch.cuda.empty_cache()


def _rows(host, s, idx):
    """float32 (len(idx), HKV, D) K and V rows of sequence s at positions idx."""
    i = torch.as_tensor(np.asarray(idx, np.int64))
    return host[0][s].index_select(0, i).float().numpy(), host[1][s].index_select(0, i).float().numpy()


def _mirror(cfgs, reserve):
    import draftkv
    return draftkv.CompressedKVCache(L, [_dcfg(c) for c in cfgs], batch=B, cap=CTX + 64,
                                     reserve_cfgs=[_dcfg(c) for c in reserve])


def _oracle_state(host, s, cfg, pos):
    """The oracle's quantized rows of sequence s at positions pos: (kq, vq),
    each (codes, scale, lo, deq)."""
    k, v = _rows(host, s, pos)
    return quantize_codes(k, cfg.bits, cfg.group, cfg.meta), quantize_codes(v, cfg.bits, cfg.group, cfg.meta)


def _same_codes(g, kq, vq, what):
    assert np.array_equal(g["k_codes"], kq[0]), what + ": K codes"
    assert np.array_equal(g["v_codes"], vq[0]), what + ": V codes"
    for name, a, b in (("k_scale", g["k_scale"], kq[1]), ("k_lo", g["k_lo"], kq[2]),
                       ("v_scale", g["v_scale"], vq[1]), ("v_lo", g["v_lo"], vq[2])):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{what}: {name} bits"


def _check_build(md, host, cfg, seqs):
    """Every listed sequence's mirror equals the oracle's build/rebuild:
    closed-form kept set (all-zero scores), codes and meta bit for bit."""
    gs = {s: md.read_codes(LAYER, s) for s in seqs}

    def one(s):
        n = int(LENS[s])
        kept = closed_form_kept(n, cfg, n)
        g = gs[s]
        assert g["pos"].tolist() == kept, f"seq {s}: kept positions"
        assert not g["score"].any(), f"seq {s}: scores not reset"
        kq, vq = _oracle_state(host, s, cfg, kept)
        _same_codes(g, kq, vq, f"seq {s}")
        return s

    assert sorted(_POOL.map(one, seqs)) == sorted(seqs)


def test_requantize_both_arms_and_switches_bit_exact(dev, cache):
    """sync_from(full, 0) and rebuild_layers (an arm switch each way) at the
    benchmark shape: the compile-time requantize kernel against the oracle,
    for every sequence of the int4 arm (the window starts mid-block) and a
    spread of the int8 arm's."""
    full, host = cache
    md = _mirror([INT8] * L, [INT8, INT4])
    md.sync_from(full, 0)
    _check_build(md, host, INT8, [0, 7, 18, 31])
    md.rebuild_layers(full, [LAYER], [_dcfg(INT8), _dcfg(INT4)])
    assert md.cfgs[LAYER] == _dcfg(INT4) and md.cfgs[0] == _dcfg(INT8)
    _check_build(md, host, INT4, list(range(B)))
    # back to int8: the pages held int4 rows in another layout
    md.rebuild_layers(full, [LAYER], [_dcfg(INT8), _dcfg(INT8)])
    _check_build(md, host, INT8, [3, 12, 25])
    # the other layer was never touched
    g0 = md.read_codes(0, 5)
    assert g0["pos"].tolist() == list(range(int(LENS[5])))


@pytest.mark.parametrize("cfg", [INT4, INT8, INT4H], ids=["int4g32f16keep0.25", "int8g64f16keep1", "int4g32f16keep0.5"])
def test_drafter_attention_and_mass_match_oracle(dev, cache, cfg):
    """One query row per sequence over the mirror built at the benchmark
    shape: every sequence's output within tolerance of the oracle's, and the
    attention mass added to every kept row's score. The int4 arms run the
    segment kernel (one block per sequence and KV head); at keep 0.5 its waves
    hold more pages than their logit registers and spill the rest."""
    full, host = cache
    md = _mirror([cfg] * L, [cfg])
    md.sync_from(full, 0)
    rng = np.random.default_rng(11)
    q = (rng.standard_normal((B, HQ, D)) * 2.0).astype(np.float32)
    out = md.attend(LAYER, torch.from_numpy(q).to(dev), want_mass=True).cpu().numpy()
    gs = {s: md.read_codes(LAYER, s) for s in range(B)}

    def one(s):
        n = int(LENS[s])
        kept = closed_form_kept(n, cfg, n)
        g = gs[s]
        assert g["pos"].tolist() == kept
        kq, vq = _oracle_state(host, s, cfg, kept)
        ref, _, mp = attend(q[s][None], kq[3], vq[3], np.asarray(kept), np.array([n]), HQ // HKV)
        np.testing.assert_allclose(out[s], ref[0], rtol=RTOL, atol=ATOL, err_msg=f"seq {s}")
        np.testing.assert_allclose(g["score"], row_mass(mp).astype(np.float64), rtol=1e-4, atol=1e-7,
                                   err_msg=f"seq {s} mass")
        return s

    assert sorted(_POOL.map(one, range(B))) == list(range(B))


def test_draft_step_eviction_and_resync_match_oracle(dev, cache):
    """After an attention pass has filled the scores: one draft step appends
    the row at position n (the keep-0.25 arm evicts the lowest (score,
    position) unprotected row), then the rollback resync rewrites positions
    >= n - 2 from the full cache. The kept sets, the new rows' codes and the
    scores equal the oracle's, which is handed the device's scores."""
    full, host = cache
    cfg = INT4
    md = _mirror([cfg] * L, [cfg])
    md.sync_from(full, 0)
    rng = np.random.default_rng(12)
    q = (rng.standard_normal((B, HQ, D)) * 2.0).astype(np.float32)
    md.attend(LAYER, torch.from_numpy(q).to(dev), want_mass=True)
    before = {s: md.read_codes(LAYER, s) for s in range(B)}
    # the drafted row of every sequence (bf16 values, as a bf16 forward makes them)
    kn = torch.randn((B, 1, HKV, D), generator=torch.Generator().manual_seed(3)).bfloat16().float()
    vn = torch.randn((B, 1, HKV, D), generator=torch.Generator().manual_seed(4)).bfloat16().float()
    bud = md.begin_step(LENS, np.ones(B, np.int64))
    md.append_layer(LAYER, kn.to(dev), vn.to(dev), torch.tensor(LENS, dtype=torch.int32, device=dev), bud[LAYER])
    after = {s: md.read_codes(LAYER, s) for s in range(B)}
    # rollback: positions >= n-2 come back from the full cache (which holds 0 .. n-1)
    start = LENS - 2
    md.sync_from(full, start)
    synced = {s: md.read_codes(LAYER, s) for s in range(B)}

    def one(s):
        n = int(LENS[s])
        b0 = before[s]
        kq, vq = _oracle_state(host, s, cfg, b0["pos"])
        o = oc.CompressedKVCache(1, cfg)
        o._cat(0, kq[3], vq[3], kq, vq, b0["pos"].astype(np.int64), b0["score"].copy())
        o.seen_positions = n
        o.append(0, kn[s].numpy(), vn[s].numpy(), [n])
        a = after[s]
        assert len(o.pos[0]) == budget(cfg, n + 1)
        assert a["pos"].tolist() == o.pos[0].tolist(), f"seq {s}: kept set after the draft step"
        assert np.array_equal(a["score"], o.score[0]), f"seq {s}: scores after the draft step"
        _same_codes(a, o.kq[0], o.vq[0], f"seq {s} draft step")
        # resync (compress.py:190-207): truncate at start, append the true rows, evict
        o.truncate(int(start[s]))
        kt, vt = _rows(host, s, np.arange(start[s], n))
        o.append(0, kt, vt, np.arange(start[s], n))
        y = synced[s]
        assert y["pos"].tolist() == o.pos[0].tolist(), f"seq {s}: kept set after the resync"
        assert np.array_equal(y["score"], o.score[0]), f"seq {s}: scores after the resync"
        _same_codes(y, o.kq[0], o.vq[0], f"seq {s} resync")
        return len(o.pos[0])

    kept = list(_POOL.map(one, range(B)))
    assert md.rows()[:, LAYER].tolist() == kept


@pytest.mark.parametrize("T", [1, 3, 5, 9, 17])
def test_verify_attention_matches_oracle(dev, cache, T):
    """T query rows per sequence at positions n-T .. n-1 over keys 0 .. own
    position of the benchmark cache (ragged ~32k rows, shuffled 16-token bf16
    pages), with the key chunk the cache picks for its shape: every sequence
    within 2e-3 / 1e-3 of the oracle (llama.py:202-218 via engine.py:184-185).
    T = 1, 3, 5, 9, 17 make 1, 1, 2, 3, 5 sixteen-row query tiles, so the
    kernel runs with 1, 1, 2, 4 and 8 waves per workgroup; T = 3 (the verify
    pass at gamma 2, the benchmark's usual one) leaves 4 of its tile's 16 rows
    empty, T = 5 (gamma 4) 12 of its second tile's."""
    full, host = cache
    assert full.chunk_keys == 8192
    rng = np.random.default_rng(20 + T)
    q = rng.standard_normal((B, T, HQ, D)).astype(np.float32)
    start = torch.tensor(LENS - T, dtype=torch.int32, device=dev)
    out = full.attend(LAYER, torch.from_numpy(q).to(dev), start, int(LENS.max())).cpu().numpy()

    def one(s):
        n = int(LENS[s])
        k, v = host[0][s, :n].float().numpy(), host[1][s, :n].float().numpy()
        ref = attend_blas(q[s], k, v, np.arange(n), np.arange(n - T, n), HQ // HKV)
        np.testing.assert_allclose(out[s], ref, rtol=RTOL, atol=ATOL, err_msg=f"T {T} seq {s}")
        return s

    assert sorted(_POOL.map(one, range(B))) == list(range(B))


def test_verify_attention_long_context_matches_oracle(dev):
    """Batch 1 with 262144 positions (the long-context workload) in
    shuffled 16-token bf16 pages: the cache's key chunk is 2048, so each of
    the 17 query rows merges up to 128 chunk partials. Every row and head
    within 2e-3 / 1e-3 of the oracle."""
    import draftkv
    ctx, T = 262144, 17
    maxt = ctx + 64
    full = draftkv.PagedKVCache(1, HKV, D, 16, maxt // 16, "bf16", batch=1, max_tokens=maxt)
    assert full.chunk_keys == 2048
    rng = np.random.default_rng(5)
    rng.shuffle(full.pools[0]._stack)
    full.reserve([ctx])
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    kv = []
    for _ in range(2):
        x = torch.randn((1, ctx, HKV, D), generator=g, device=dev, dtype=torch.float32)
        x[..., [5, 77]] *= 8.0
        kv.append(x.bfloat16())
        del x
    full.append_layer(0, kv[0], kv[1], torch.zeros(1, dtype=torch.int32, device=dev),
                      torch.tensor([ctx], dtype=torch.int32, device=dev))
    full.commit([ctx])
    k, v = kv[0][0].float().cpu().numpy(), kv[1][0].float().cpu().numpy()
    del kv
    q = rng.standard_normal((1, T, HQ, D)).astype(np.float32)
    start = torch.tensor([ctx - T], dtype=torch.int32, device=dev)
    out = full.attend(0, torch.from_numpy(q).to(dev), start, ctx).cpu().numpy()[0]
    del full
    torch.cuda.empty_cache()
    rep = HQ // HKV

    def one(h):   # one KV head and its query group at a time
        ref = attend_blas(q[0][:, h * rep:(h + 1) * rep], k[:, h:h + 1], v[:, h:h + 1], np.arange(ctx),
                          np.arange(ctx - T, ctx), rep)
        np.testing.assert_allclose(out[:, h * rep:(h + 1) * rep], ref, rtol=RTOL, atol=ATOL, err_msg=f"KV head {h}")
        return h

    assert sorted(_POOL.map(one, range(HKV))) == list(range(HKV))
