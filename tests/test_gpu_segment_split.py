"""The drafter's int4 segment kernel when the segments alone do not fill the
chip (batch x KV heads < 256): every (sequence, KV head) segment is cut into
blocks of whole pages, each block leaves its merged partial and its kept
probabilities, and a second kernel merges the blocks and adds the attention
mass to the scores.

Shapes: the long-context workload (batch 1, 262144 positions, Llama-3-8B
attention heads: 32 query heads, 8 KV heads, head_dim 128; int4 group 32,
fp16 meta, keep 0.25: 65536 kept rows = 2048 pages per segment, 33 blocks
each) and ragged small batches (segments of 1 row to a few thousand, so
blocks without pages, one-page blocks and partial last pages occur).

Attention: 2e-3 relative / 1e-3 absolute against the float32 oracle
(compress.py:135-142, llama.py:202-218); attention mass added to each kept
row's score (compress.py:144-151, llama.py:213-216): 1e-4 relative.
"""

import numpy as np
import pytest
import torch

from oracle.attention import attend, row_mass
from oracle.config import Cfg, closed_form_kept
from oracle.quant import quantize_codes

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-3, 1e-3
HKV, HQ, D = 8, 32, 128


def _dcfg(c: Cfg):
    from draftkv import CompressionConfig
    return CompressionConfig(c.bits, c.keep_frac, c.sink, c.recent, c.group, c.meta == "f16")


def _build(dev, lens, seed, cfg):
    """A one-layer bf16 paged cache holding lens[s] N(0,1) rows (two outlier
    channels x8) per sequence in shuffled 16-token pages, and the drafter
    mirror built from it. Returns (mirror, host K, host V) with host arrays
    float32 [b][max_len][HKV][D]."""
    import draftkv
    b, T = len(lens), int(max(lens))
    maxt = T + 64
    full = draftkv.PagedKVCache(1, HKV, D, 16, maxt // 16 + 1, "bf16", batch=b, max_tokens=maxt)
    rng = np.random.default_rng(seed)
    for p in full.pools:
        rng.shuffle(p._stack)
    full.reserve(lens)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    kv = []
    for _ in range(2):
        x = torch.randn((b, T, HKV, D), generator=g, device=dev, dtype=torch.float32)
        x[..., [5, 77]] *= 8.0
        kv.append(x.bfloat16())
        del x
    full.append_layer(0, kv[0], kv[1], torch.zeros(b, dtype=torch.int32, device=dev),
                      torch.tensor(lens, dtype=torch.int32, device=dev))
    full.commit(lens)
    md = draftkv.CompressedKVCache(1, [_dcfg(cfg)], batch=b, cap=maxt, reserve_cfgs=[_dcfg(cfg)])
    md.sync_from(full, 0)
    host = kv[0].float().cpu().numpy(), kv[1].float().cpu().numpy()
    del full, kv
    torch.cuda.empty_cache()
    return md, host


def _check(dev, md, host, lens, cfg, seed):
    rng = np.random.default_rng(seed)
    b = len(lens)
    q = (rng.standard_normal((b, HQ, D)) * 2.0).astype(np.float32)
    out = md.attend(0, torch.from_numpy(q).to(dev), want_mass=True).cpu().numpy()
    for s in range(b):
        n = int(lens[s])
        g = md.read_codes(0, s)
        kept = closed_form_kept(n, cfg, n)
        assert g["pos"].tolist() == kept, f"seq {s}: kept positions"
        idx = np.asarray(kept)
        kq = quantize_codes(host[0][s, idx], cfg.bits, cfg.group, cfg.meta)
        vq = quantize_codes(host[1][s, idx], cfg.bits, cfg.group, cfg.meta)
        ref, _, mp = attend(q[s][None], kq[3], vq[3], idx, np.array([n]), HQ // HKV)
        np.testing.assert_allclose(out[s], ref[0], rtol=RTOL, atol=ATOL, err_msg=f"seq {s} (n {n})")
        np.testing.assert_allclose(g["score"], row_mass(mp).astype(np.float64), rtol=1e-4, atol=1e-7,
                                   err_msg=f"seq {s} (n {n}) mass")


def test_long_context_int4_drafter_matches_oracle(dev):
    """Batch 1, 262144 positions, int4 g32 keep 0.25: the split segment path."""
    cfg = Cfg(4, 0.25, group=32, meta="f16")
    lens = np.array([262144], np.int64)
    md, host = _build(dev, lens, 31, cfg)
    _check(dev, md, host, lens, cfg, 32)


@pytest.mark.parametrize("keep", [0.25, 0.5, 1.0])
def test_ragged_small_batch_int4_drafter_matches_oracle(dev, keep):
    """Batch 5 of ragged segments (1 to 9000 rows): 40 segments, so each is
    cut into 7 blocks, many without pages or with a single partial page."""
    cfg = Cfg(4, keep, group=32, meta="f16")
    lens = np.array([1, 37, 700, 4097, 9000], np.int64)
    md, host = _build(dev, lens, 41 + int(keep * 4), cfg)
    _check(dev, md, host, lens, cfg, 42)


def test_repeated_passes_accumulate_mass(dev):
    """Two passes with different queries: each adds its mass to the scores
    (the second pass must not see the first one's kept values)."""
    cfg = Cfg(4, 0.25, group=32, meta="f16")
    lens = np.array([20000, 3333], np.int64)
    md, host = _build(dev, lens, 51, cfg)
    rng = np.random.default_rng(52)
    total = [np.zeros(len(closed_form_kept(int(n), cfg, int(n)))) for n in lens]
    for _ in range(2):
        q = (rng.standard_normal((2, HQ, D)) * 2.0).astype(np.float32)
        md.attend(0, torch.from_numpy(q).to(dev), want_mass=True)
        for s in range(2):
            n = int(lens[s])
            idx = np.asarray(closed_form_kept(n, cfg, n))
            kq = quantize_codes(host[0][s, idx], cfg.bits, cfg.group, cfg.meta)
            vq = quantize_codes(host[1][s, idx], cfg.bits, cfg.group, cfg.meta)
            _, _, mp = attend(q[s][None], kq[3], vq[3], idx, np.array([n]), HQ // HKV)
            total[s] += row_mass(mp).astype(np.float64)
    for s in range(2):
        np.testing.assert_allclose(md.read_codes(0, s)["score"], total[s], rtol=1e-4, atol=1e-7)
