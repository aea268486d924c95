"""Host-side API of the product package, on CPU: the cost model against the
reference's published ceilings (README.md:82-86) and its own test
expectations (tests/test_math.py, tests/test_llama.py:98-132), the arm space,
and the block pool's allocator semantics (paged.py:33-73)."""

import numpy as np
import pytest

from draftkv import (BlockPool, BlockPoolExhausted, CompressionConfig, CostModel, LayerPlan, best_gamma,
                     default_arms, expected_tokens, plan_blocks_needed)


@pytest.mark.parametrize("batch,ctxs,want", [(1, (1024, 32768, 262144), (1.008, 1.222, 2.417)),
                                             (32, (1024, 32768, 262144), (1.222, 4.342, 6.538))])
def test_ceiling_reproduces_published_rows(batch, ctxs, want):
    # README.md:82-85: 4b/keep0.5, HBM-resident cache, Llama-3-8B shape, 2 TB/s; the
    # reference prices fp16 scale/zero pairs per 64 channels (config.py:39-48)
    cm = CostModel(batch=batch)
    got = tuple(round(cm.ceiling(F16(4, 0.5), c), 3) for c in ctxs)
    assert got == want


def test_offloaded_ceiling_row():
    # README.md:86: full cache offloaded over PCIe5 (64 GB/s), 1 GB HBM budget
    cm = CostModel(full_kv_bandwidth=6.4e10, hbm_kv_budget=1e9)
    got = [round(cm.ceiling(F16(4, 0.5), c), 2) for c in (1024, 32768, 262144)]
    assert got == [1.26, 9.04, 7.97]


def test_mi355x_target_ceilings():
    cm = CostModel(bandwidth=8e12, batch=32)
    assert cm.ceiling(F16(4, 0.25), 32768) == pytest.approx(5.967, abs=1e-3)
    assert cm.ceiling(F16(8, 1.0), 32768) == pytest.approx(1.724, abs=1e-3)


def F16(bits, keep, group=64):
    return CompressionConfig(bits, keep, group=group, scale_fp16=True)


def test_bytes_per_entry_prices_the_stored_group_and_meta():
    # reference formula (config.py:39-48): D*bits/8 + 4*ceil(D/64) -- fp16 scale and zero per 64 channels
    for d in (64, 80, 128):
        for b in (2, 3, 4, 8):
            assert F16(b, 1.0).bytes_per_entry(d) == d * b / 8 + 4 * -(-d // 64)
    assert F16(4, 0.25, 32).bytes_per_entry(128) == 64 + 4 * 4          # int4 g32: 80 B
    assert CompressionConfig(4, 0.25, group=32).bytes_per_entry(128) == 64 + 8 * 4   # f32 meta: 96 B
    assert F16(8, 1.0).bytes_per_entry(128, group=32) == 128 + 16
    assert CompressionConfig(16, 1.0).bytes_per_entry(128) == 256
    # the cost model prices the g32 arm's larger meta
    cm = CostModel(bandwidth=8e12, batch=32)
    assert cm.draft_kv_bytes(F16(4, 0.25, 32), 32768) == pytest.approx(
        cm.draft_kv_bytes(F16(4, 0.25), 32768) * 80 / 72)


def test_expected_tokens_and_speedup_bound():          # reference tests/test_math.py:8-55
    for g in (1, 4, 9):
        assert expected_tokens(0.0, g) == pytest.approx(1.0)
        assert expected_tokens(1.0, g) == pytest.approx(g + 1)
    for a in (0.5, 0.8, 0.95):
        assert expected_tokens(a, 1000) == pytest.approx(1 / (1 - a), rel=1e-6)
    cm = CostModel(full_kv_bandwidth=6.4e10, hbm_kv_budget=1e9)
    for ctx in (512, 8192, 131072):
        for cfg in (CompressionConfig(16, 1.0), CompressionConfig(4, 0.5), CompressionConfig(2, 0.25)):
            ceil = cm.ceiling(cfg, ctx)
            assert all(cm.speedup(cfg, g, 0.999, ctx) <= ceil + 1e-9 for g in range(1, 32))
    gs = [best_gamma(cm, CompressionConfig(4, 0.5), a, 32768, 16)[0] for a in (0.1, 0.3, 0.5, 0.7, 0.9, 0.99)]
    assert gs == sorted(gs)
    assert CostModel().ceiling(CompressionConfig(2, 0.25), 512) < 1.02


def test_gqa_breakeven_scales_with_ratio():            # reference tests/test_llama.py:98-122
    cfg = CompressionConfig(4, 0.5)
    base = dict(n_layers=32, d_head=128, weight_bytes=16e9, bandwidth=2.0e12)

    def breakeven(n_kv, target=1.5):
        cm = CostModel(n_kv_heads=n_kv, **base)
        lo, hi = 128, 8_000_000
        while lo < hi:
            mid = (lo + hi) // 2
            if cm.ceiling(cfg, mid) >= target:
                hi = mid
            else:
                lo = mid + 1
        return lo

    mha, gqa4, gqa8 = breakeven(32), breakeven(8), breakeven(4)
    assert gqa4 / mha == pytest.approx(4.0, rel=0.1) and gqa8 / mha == pytest.approx(8.0, rel=0.1)


def test_config_validation_and_arms():
    with pytest.raises(ValueError):
        CompressionConfig(5, 1.0)
    with pytest.raises(ValueError):
        CompressionConfig(4, 0.0)
    arms = default_arms()
    assert len(arms) == 15 and arms == sorted(arms)
    sizes = [CompressionConfig(b, 1.0).bytes_per_entry(128) for b in (2, 3, 4, 8, 16)]
    assert sizes == sorted(sizes) and sizes[-1] == 256
    plan = LayerPlan.uniform(CompressionConfig(4, 0.25), 32)
    cm = CostModel()
    assert cm.draft_kv_bytes(plan, 32768) == pytest.approx(cm.draft_kv_bytes(CompressionConfig(4, 0.25), 32768))


def test_block_pool_semantics():
    pool = BlockPool(8, 16)
    got = [pool.allocate() for _ in range(5)]
    assert got == [7, 6, 5, 4, 3]
    pool.free(5)
    assert pool.allocate() == 5
    for b in got:
        pool.free(b)
    pool.check_invariants()
    p2 = BlockPool(2, 16)
    a, b = p2.allocate(), p2.allocate()
    with pytest.raises(BlockPoolExhausted):
        p2.allocate()
    p2.free(a)
    with pytest.raises(RuntimeError, match="double free"):
        p2.free(a)
    assert plan_blocks_needed(33, 3, 16) == 9


def test_paged_reserve_truncate_match_reference_allocator():
    """The batched cache's vectorized reserve/truncate hand out and return
    blocks exactly as the reference's per-layer appends and truncate do
    (paged.py:112-162), sequence by sequence: same block tables, same free
    lists, same lengths. Host logic only (a CPU store of tiny rows)."""
    from draftkv.paged import PagedKVCache
    from oracle.caches import PagedKVCache as RefPaged
    L, b, bs, nb = 3, 4, 4, 256
    pc = PagedKVCache(L, 1, 2, block_size=bs, n_blocks=nb, batch=b, max_tokens=200, device="cpu")
    refs = [RefPaged(L, 1, 2, bs, nb) for _ in range(b)]
    rng = np.random.default_rng(0)
    for _ in range(60):
        if rng.random() < 0.6:
            cnt = rng.integers(0, 9, b)
            pc.reserve(cnt)
            pc.commit(cnt)
            for s in range(b):
                n = refs[s].length
                z = np.zeros((int(cnt[s]), 1, 2), np.float32)
                if cnt[s] > 0:
                    for layer in range(L):
                        refs[s].append(layer, z, z, np.arange(n, n + cnt[s]))
        else:
            cut = np.maximum(pc.lengths() - rng.integers(0, 6, b), 0)
            pc.truncate(cut)
            for s in range(b):
                refs[s].truncate(int(cut[s]))
        for s in range(b):
            assert [pc.tables[s, ly, : pc.table_len[s, ly]].tolist() for ly in range(L)] == refs[s].block_table
            assert pc.pools[s]._stack == refs[s].pool.free_list
            pc.pools[s].check_invariants()
        assert pc.lengths().tolist() == [r.length for r in refs]
    # the device table mirror holds every live block id (physical = local + s * n_blocks)
    for s in range(b):
        for ly in range(L):
            n = int(pc.table_len[s, ly])
            assert (pc.d_tables[s, ly, :n].numpy() == pc.tables[s, ly, :n] + s * nb).all()
    with pytest.raises(BlockPoolExhausted):
        pc.reserve([1000, 0, 0, 0])


def test_growing_full_cache_reserve_matches_block_by_block():
    """FullKVCache grows its pools instead of running dry; the vectorized
    reserve hands out the same ids, and ends with the same pool size, as
    allocating block by block through _ensure_capacity (its batch-1 path)."""
    from draftkv.compress import FullKVCache
    a = FullKVCache(2, 1, 2, batch=3, device="cpu", block_size=4, max_tokens=4096)
    b = FullKVCache(2, 1, 2, batch=3, device="cpu", block_size=4, max_tokens=4096)
    rng = np.random.default_rng(1)
    for _ in range(12):
        cnt = rng.integers(0, 90, 3)
        a.reserve(cnt)
        a.commit(cnt)
        for layer in range(2):
            for s in range(3):
                if cnt[s] > 0:
                    b._ensure_capacity(s, layer, int(cnt[s]))
        b._upload()
        b.commit(cnt)
        assert a.n_blocks == b.n_blocks
        assert (a.tables == b.tables).all() and (a.table_len == b.table_len).all()
        assert all(p._stack == q._stack for p, q in zip(a.pools, b.pools))
        assert (a.d_tables.numpy() == b.d_tables.numpy()).all()


def test_tiled_weight_layout_and_round_trip():
    """ops.TiledW puts element (16 fn + c, 128 kb + 32 j + 8 q + e) of a bf16
    [N, K] weight at (fn * K/128 + kb) * 2048 + j * 512 + (16 q + c) * 8 + e
    (the MFMA A-operand order the tiled GEMM reads), and rows() gives the
    matrix back; shapes it cannot tile are refused. Two weights whose
    entries are their row and their column (exact in bf16) locate every
    element."""
    import itertools
    import torch
    from draftkv import ops
    N, K = 48, 256
    rows = torch.arange(N, dtype=torch.float32)[:, None].expand(N, K).contiguous().to(torch.bfloat16)
    cols = torch.arange(K, dtype=torch.float32)[None, :].expand(N, K).contiguous().to(torch.bfloat16)
    tr, tc = ops.TiledW(rows).t.reshape(-1), ops.TiledW(cols).t.reshape(-1)
    assert tr.numel() == N * K
    for fn, kb, j, q, c, e in itertools.product(range(N // 16), range(K // 128), range(4), range(4), range(16), range(8)):
        off = ((fn * (K // 128) + kb) * 4 + j) * 512 + (16 * q + c) * 8 + e
        assert int(tr[off]) == 16 * fn + c and int(tc[off]) == 128 * kb + 32 * j + 8 * q + e
    w = torch.randn((N, K)).to(torch.bfloat16)
    assert torch.equal(ops.TiledW(w).rows(), w)
    for bad in (torch.zeros((24, 256), dtype=torch.bfloat16), torch.zeros((32, 192), dtype=torch.bfloat16),
                torch.zeros((32, 256), dtype=torch.float32)):
        assert not ops.tile_ok(bad)
        with pytest.raises(ValueError):
            ops.TiledW(bad)


class _Made(Exception):
    pass


class _StubModel:
    """Just enough of a model for the engine to size a full cache: records
    new_cache's arguments and stops there (no device needed)."""

    vocab_size, n_kv_heads = 1000, 8

    def __init__(self):
        self.calls = []

    def new_cache(self, **kw):
        self.calls.append(kw)
        raise _Made


@pytest.mark.parametrize("plen,n_new,gamma", [(22000, 1024, 20), (22000, 1024, None), (4000, 300, 8),
                                              (130000, 256, 16)])
def test_baseline_and_speculative_caches_share_the_key_chunk(plen, n_new, gamma):
    """Plain and speculative decoding of one request size their full caches
    differently (16 rows of slack vs the longest draft), but the attention
    key chunk -- which fixes how a row's chunk partials are merged -- comes
    from what both share, so greedy speculative output can equal the
    baseline bit for bit."""
    from draftkv import DraftKVEngine, FixedPolicy
    from draftkv.paged import auto_chunk_keys

    class NoBound:
        def select(self, ctx, key=None):
            return CompressionConfig(4, 0.5), 20

        def update(self, *a, **k):
            pass

    m = _StubModel()
    ctrl = FixedPolicy(CompressionConfig(4, 0.5), gamma) if gamma is not None else NoBound()
    eng = DraftKVEngine(m, ctrl)
    prompts = [[1] * plen] * 32
    for call in (lambda: eng.generate_baseline_batch(prompts, n_new), lambda: eng.generate_batch(prompts, n_new)):
        with pytest.raises(_Made):
            call()
    base, spec = m.calls
    assert base["chunk_keys"] == spec["chunk_keys"] == auto_chunk_keys(32, 8, plen + n_new)
