"""Pins the oracle caches against the reference's own expectations
(tests/test_paged.py, tests/test_lossless.py:60-77, tests/test_adaptive.py:130-153)
and against closed forms of the eviction rule (compress.py:154-179)."""

import numpy as np
import pytest

from oracle.caches import (BlockPool, BlockPoolExhausted, CompressedKVCache, FullKVCache,
                           PagedKVCache, plan_blocks_needed)
from oracle.config import Cfg, budget, closed_form_kept
from oracle.models import demo_model


def _paged(m, block_size=16, n_blocks=512):
    return PagedKVCache(m.n_layers, m.n_heads, m.d_head, block_size, n_blocks)


def test_pool_lifo_order_and_invariants():           # paged.py:42-59
    pool = BlockPool(8, 16)
    got = [pool.allocate() for _ in range(5)]
    assert got == [7, 6, 5, 4, 3]
    pool.check_invariants()
    pool.free(5)
    assert pool.allocate() == 5                       # freed block is reused first
    for b in got:
        pool.free(b)
    pool.check_invariants()
    assert pool.n_used == 0 and pool.n_free == 8


def test_pool_rejects_double_free_and_exhaustion():   # reference test_paged.py:33-42
    pool = BlockPool(2, 16)
    a, b = pool.allocate(), pool.allocate()
    with pytest.raises(BlockPoolExhausted):
        pool.allocate()
    pool.free(a)
    with pytest.raises(RuntimeError, match="double free"):
        pool.free(a)
    pool.free(b)


@pytest.mark.parametrize("block_size", [1, 4, 16, 64])
def test_paged_matches_contiguous(block_size):        # reference test_paged.py:44-55
    m = demo_model()
    toks = np.random.default_rng(0).integers(0, m.vocab_size, 100)
    full, paged = FullKVCache(m.n_layers), _paged(m, block_size)
    assert np.array_equal(m.forward(toks, full, 0), m.forward(toks, paged, 0))
    for L in range(m.n_layers):
        for a, b in zip(full.read(L), paged.read(L)):
            assert np.array_equal(a, b)


def test_truncate_keeps_tail_block():                  # reference test_paged.py:58-68
    m = demo_model()
    paged = _paged(m, 16)
    m.forward(np.random.default_rng(1).integers(0, m.vocab_size, 64), paged, 0)
    before = paged.blocks_in_use
    paged.truncate(33)
    paged.pool.check_invariants()
    assert paged.length == 33 and paged.blocks_in_use == 3 * m.n_layers < before


def test_rollback_cycles_do_not_leak():                # reference test_paged.py:71-85
    m = demo_model()
    rng = np.random.default_rng(2)
    paged = _paged(m, 8, 256)
    m.forward(rng.integers(0, m.vocab_size, 40), paged, 0)
    base = paged.blocks_in_use
    for _ in range(60):
        n = paged.length
        m.forward(rng.integers(0, m.vocab_size, 6), paged, n)
        paged.truncate(n)
        paged.pool.check_invariants()
        assert paged.length == n
    assert paged.blocks_in_use == base


def test_exhaustion_raises():                           # reference test_paged.py:88-92
    m = demo_model()
    with pytest.raises(BlockPoolExhausted):
        m.forward(np.arange(64) % m.vocab_size, _paged(m, 8, m.n_layers), 0)


def test_blocks_needed_and_fragmentation():             # reference test_paged.py:95-100,119-124
    m = demo_model()
    for ctx in (1, 15, 16, 17, 100):
        p = _paged(m, 16)
        m.forward(np.arange(ctx) % m.vocab_size, p, 0)
        assert p.blocks_in_use == plan_blocks_needed(ctx, m.n_layers, 16)
    p = _paged(m, 16)
    m.forward(np.arange(33) % m.vocab_size, p, 0)
    assert p.fragmentation() == pytest.approx(1 - 33 / 48)


def test_first_block_table_is_interleaved_lifo():
    # one forward appends layer 0, then layer 1, ...: with 33 tokens and block
    # size 16 layer 0 takes 511, 510, 509, layer 1 takes 508, 507, 506, ...
    m = demo_model()
    p = _paged(m, 16, 512)
    m.forward(np.arange(33) % m.vocab_size, p, 0)
    assert p.block_table == [[511, 510, 509], [508, 507, 506], [505, 504, 503]]


def test_resync_row_count():                            # reference test_lossless.py:60-77
    m = demo_model()
    prompt = np.random.default_rng(0).integers(0, m.vocab_size, 192)
    full = FullKVCache(m.n_layers)
    m.forward(prompt, full, 0)
    comp = CompressedKVCache(m.n_layers, Cfg(8, 1.0))
    comp.sync_from(full, 0)
    assert comp.length == full.length
    comp.truncate(10)
    assert comp.length == 10
    assert comp.sync_from(full, 10) == (192 - 10) * m.n_layers
    assert comp.length == 192


def test_only_changed_layers_rebuilt():                 # reference test_adaptive.py:130-153
    m = demo_model()
    full = FullKVCache(m.n_layers)
    m.forward(np.arange(64) % m.vocab_size, full, 0)
    comp = CompressedKVCache(m.n_layers, [Cfg(8, 1.0)] * m.n_layers)
    comp.sync_from(full, 0)
    before = [comp.read(L)[0].copy() for L in range(m.n_layers)]
    cfgs = [Cfg(8, 1.0)] * m.n_layers
    cfgs[1] = Cfg(2, 0.25)
    assert comp.rebuild_layers(full, [1], cfgs) == 64
    for L in range(m.n_layers):
        assert np.array_equal(comp.read(L)[0], before[L]) == (L != 1)


@pytest.mark.parametrize("keep,sink,recent", [(0.25, 4, 32), (0.5, 4, 32), (0.3, 2, 5),
                                              (0.5, 0, 8), (0.25, 4, 0)])
@pytest.mark.parametrize("n", [10, 36, 37, 100, 257])
def test_build_eviction_closed_form(keep, sink, recent, n):
    """A build appends n rows with score 0 and evicts once: the survivors are the
    sink oldest plus the newest B - sink (B = budget), by brute force over the
    stable (score, index) order."""
    cfg = Cfg(4, keep, sink, recent)
    rng = np.random.default_rng(n)
    k = rng.standard_normal((n, 2, 16)).astype(np.float32)
    comp = CompressedKVCache(1, cfg)
    comp.append(0, k, k, np.arange(n))
    assert comp.pos[0].tolist() == closed_form_kept(n, cfg, n)
    B = budget(cfg, n)
    assert comp.length == (n if (n <= B or recent == 0) else B)


def test_budget_rounds_half_to_even():
    assert budget(Cfg(4, 0.5, 0, 1), 5) == 2           # round(2.5) == 2
    assert budget(Cfg(4, 0.5, 0, 1), 7) == 4           # round(3.5) == 4
    assert budget(Cfg(4, 0.25, 4, 32), 10) == 36       # floor at sink + recent


def test_heavy_hitters_survive_eviction():
    """Steady state: with scores accumulated, the lowest-mass unprotected rows
    go first and ties fall back to the oldest position."""
    cfg = Cfg(8, 0.5, 1, 2)
    comp = CompressedKVCache(1, cfg)
    x = np.ones((6, 1, 4), np.float32)
    comp.append(0, x, x, np.arange(6))                 # budget 3 -> keep {0, 4, 5}
    assert comp.pos[0].tolist() == [0, 4, 5]
    comp.score[0][:] = [0.0, 9.0, 0.0]                 # make row at pos 4 heavy
    comp.append(0, x[:4], x[:4], np.arange(6, 10))     # budget 5: rows 0,4,5,6,7,8,9
    # unprotected: 4 (score 9), 5, 6, 7 (score 0) -> drop the two oldest zeros: 5, 6
    assert comp.pos[0].tolist() == [0, 4, 7, 8, 9]


@pytest.mark.parametrize("cfg", [Cfg(4, 0.25, group=32, meta="f16"), Cfg(8, 1.0, group=64, meta="f16"),
                                 Cfg(2, 0.5), Cfg(3, 0.3, 2, 5)])
def test_build_equals_quantizing_only_the_kept_rows(cfg):
    """A build (sync_from(full, 0): quantize every row, then one eviction with
    all scores 0) leaves exactly the closed-form kept rows, each quantized as
    if it were quantized alone: the quantizer works row by row, so parity
    tests at large shapes may quantize only the kept rows."""
    from oracle.quant import quantize_codes
    rng = np.random.default_rng(cfg.bits)
    n, H, D = 1001, 3, 128
    k = rng.standard_normal((n, H, D)).astype(np.float32)
    v = rng.standard_normal((n, H, D)).astype(np.float32)
    full = FullKVCache(1)
    full.append(0, k, v, np.arange(n))
    comp = CompressedKVCache(1, cfg)
    comp.sync_from(full, 0)
    kept = closed_form_kept(n, cfg, n)
    assert comp.pos[0].tolist() == kept
    for got, x in ((comp.kq[0], k), (comp.vq[0], v)):
        want = quantize_codes(x[kept], cfg.bits, cfg.group, cfg.meta)
        for a, b in zip(got, want[:3]):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
