"""A drafter mirror grown past its row capacity (and to wider pages) reads
back the same rows and attends the same as before: the host's page slot map
and the kernels' page addressing agree, whole chunks and tails alike."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ocap,ncap", [(32 * 9, 32 * 20), (32 * 12, 32 * 13)])
def test_regrown_mirror_reads_and_attends_the_same(dev, ocap, ncap):
    import draftkv
    from draftkv import CompressionConfig
    narrow, wide = CompressionConfig(4, 1.0, group=32, scale_fp16=True), CompressionConfig(8, 1.0)
    L, H, D, Hq, n = 2, 3, 64, 6, ocap - 20
    rng = np.random.default_rng(ocap)
    c = draftkv.CompressedKVCache(L, narrow, n_kv_heads=H, d_head=D, cap=ocap, device=dev)
    for layer in range(L):
        k = rng.standard_normal((n, H, D)).astype(np.float32)
        v = rng.standard_normal((n, H, D)).astype(np.float32)
        c.append(layer, k, v, np.arange(n))
    q = torch.from_numpy(rng.standard_normal((1, Hq, D)).astype(np.float32)).to(dev)
    before = [c.read(layer) for layer in range(L)]
    att = [c.attend(layer, q, want_mass=False).cpu() for layer in range(L)]
    c._regrow(ncap, [wide])
    assert c.cap == ncap
    for layer in range(L):
        for x, y in zip(before[layer], c.read(layer)):
            np.testing.assert_array_equal(np.asarray(x), np.asarray(y))
        torch.testing.assert_close(c.attend(layer, q, want_mass=False).cpu(), att[layer], rtol=1e-6, atol=1e-6)
