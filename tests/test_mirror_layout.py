"""The drafter mirror's page layout on the host side: the slot map is a
bijection onto the page tensor's rows for every capacity (whole chunks of 8
pages and a tail), and growing the mirror moves each page's bytes to its new
slot. Runs on the CPU: the mirror's storage is plain torch memory."""

import numpy as np
import pytest
import torch


def _cache(L, b, H, D, cap, cfg):
    import draftkv
    return draftkv.CompressedKVCache(L, cfg, n_kv_heads=H, d_head=D, batch=b, cap=cap, device="cpu")


@pytest.mark.parametrize("L,b,H", [(1, 1, 1), (3, 5, 3), (2, 32, 8)])
@pytest.mark.parametrize("npg", [1, 7, 8, 9, 13, 16, 17, 128, 243])
def test_page_slots_are_a_bijection(L, b, H, npg):
    from draftkv import CompressionConfig
    c = _cache(L, b, H, 64, 32, CompressionConfig(4, 1.0, group=32, scale_fp16=True))
    s = c.page_slots(32 * npg)
    n = L * b * H * npg
    assert s.shape == (L, b * H, npg)
    assert int(s.min()) == 0 and int(s.max()) == n - 1
    assert torch.unique(s).numel() == n
    # a layer's pages are one contiguous range
    for layer in range(L):
        assert int(s[layer].min()) == layer * b * H * npg and int(s[layer].max()) == (layer + 1) * b * H * npg - 1
    # within a whole chunk a segment's pages are consecutive slots
    nf = npg // 8
    if nf:
        d = s[:, :, : 8 * nf].reshape(L, b * H, nf, 8).diff(dim=-1)
        assert bool((d == 1).all())


def test_page_slots_closed_form_small():
    """Two segments, 10 pages (one chunk of 8, then 2 each): segment 0's chunk,
    segment 1's chunk, segment 0's tail, segment 1's tail."""
    from draftkv import CompressionConfig
    c = _cache(1, 1, 2, 64, 32, CompressionConfig(8, 1.0))
    s = c.page_slots(320)[0]
    assert s[0].tolist() == [0, 1, 2, 3, 4, 5, 6, 7, 16, 17]
    assert s[1].tolist() == [8, 9, 10, 11, 12, 13, 14, 15, 18, 19]


@pytest.mark.parametrize("ocap,ncap", [(32 * 9, 32 * 20), (32 * 8, 32 * 24), (32 * 3, 32 * 5), (32 * 16, 32 * 17)])
def test_regrow_keeps_every_page(ocap, ncap):
    from draftkv import CompressionConfig
    narrow, wide = CompressionConfig(4, 1.0, group=32, scale_fp16=True), CompressionConfig(8, 1.0)
    L, b, H = 2, 3, 2
    c = _cache(L, b, H, 64, ocap, narrow)
    g = torch.Generator().manual_seed(ocap + ncap)
    c.pages.copy_(torch.randint(0, 256, c.pages.shape, generator=g, dtype=torch.uint8))
    c.pos.copy_(torch.randint(0, 1 << 20, c.pos.shape, generator=g, dtype=torch.int32))
    c.score.copy_(torch.rand(c.score.shape, generator=g, dtype=torch.float64))
    old = c.pages[c.page_slots(ocap)].clone()            # (L, segments, pages, stride)
    opos, oscore, ostride = c.pos.clone(), c.score.clone(), c.page_stride
    c._regrow(ncap, [wide])
    assert c.cap == ncap and c.page_stride >= ostride
    new = c.pages[c.page_slots(ncap)[:, :, : ocap // 32]]
    assert torch.equal(new[..., :ostride], old)
    assert torch.equal(c.pos[..., :ocap], opos) and bool((c.pos[..., ocap:] == -1).all())
    assert torch.equal(c.score[..., :ocap], oscore)
