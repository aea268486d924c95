"""HIP kernels against the oracle, through the C ABI (via draftkv.ops and the
device caches). Integer/byte/index results are compared bit for bit; float
attention within 2e-3 relative / 1e-3 absolute of the float32 numpy oracle."""

import numpy as np
import pytest
import torch

from oracle import caches as oc
from oracle.attention import attend, row_mass
from oracle.config import Cfg
from oracle.quant import quantize_codes
from oracle.sampling import accept as o_accept
from oracle.sampling import probs as o_probs
from oracle.sampling import sample_u

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-3, 1e-3


def _dk():
    import draftkv
    from draftkv import ops
    return draftkv, ops


def _bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).bfloat16().float().numpy()


# ------------------------------------------------------------------ quantize
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("d,group", [(16, 64), (64, 64), (128, 32), (80, 64), (40, 32), (128, 128)])
@pytest.mark.parametrize("meta", ["f32", "f16"])
def test_quantize_bit_exact(dev, bits, d, group, meta):
    _, ops = _dk()
    rng = np.random.default_rng(bits * 1000 + d + group)
    x = rng.standard_normal((37, 3, d)).astype(np.float32)
    x[:, :, rng.integers(0, d, max(1, d // 100))] *= 8.0           # outlier channels
    x[0, 0, :] = 1.25                                               # a constant row
    x[1, 1, :] = 0.0
    codes, scale, lo, deq = ops.quantize_codes(torch.from_numpy(x).to(dev), bits, group, meta == "f16")
    oc_, os_, ol_, od_ = quantize_codes(x, bits, group, meta)
    assert np.array_equal(codes.cpu().numpy(), oc_)
    assert np.array_equal(scale.cpu().numpy().view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(lo.cpu().numpy().view(np.uint32), ol_.view(np.uint32))
    assert np.array_equal(deq.cpu().numpy().view(np.uint32), od_.view(np.uint32))


def test_quantize_api_numpy_roundtrip(dev):
    draftkv, _ = _dk()
    from oracle.quant import quantize as oq
    x = np.random.default_rng(3).standard_normal((16, 8, 64)).astype(np.float32)
    for b in (2, 3, 4, 8, 16):
        assert np.array_equal(draftkv.quantize(x, b), oq(x, b))


# ------------------------------------------------------------------ paged append
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("block_size", [1, 4, 16, 64])
def test_paged_tables_and_rows_match_reference(dev, dtype, block_size):
    draftkv, _ = _dk()
    L, H, D = 3, 4, 16
    rng = np.random.default_rng(block_size)
    ref = oc.PagedKVCache(L, H, D, block_size, 512)
    pc = draftkv.PagedKVCache(L, H, D, block_size, 512, dtype="bf16" if dtype == "bf16" else np.float32)
    n = 0
    for T in (33, 1, 5, 1, 17):
        for layer in range(L):
            k = rng.standard_normal((T, H, D)).astype(np.float32)
            v = rng.standard_normal((T, H, D)).astype(np.float32)
            if dtype == "bf16":
                k, v = _bf16(k), _bf16(v)
            pos = np.arange(n, n + T)
            ref.append(layer, k, v, pos)
            pc.append(layer, k, v, pos)
        n += T
        if T == 1:
            ref.truncate(n - 1)
            pc.truncate(n - 1)
            n -= 1
    assert pc.block_table == ref.block_table
    assert pc.blocks_in_use == ref.blocks_in_use
    assert pc.fragmentation() == pytest.approx(ref.fragmentation())
    pc.pool.check_invariants()
    for layer in range(L):
        for a, b in zip(pc.read(layer), ref.read(layer)):
            assert np.array_equal(a, b)


# ------------------------------------------------------------------ paged attention
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("Hq,Hkv,D", [(4, 4, 16), (8, 2, 64), (32, 8, 128), (9, 3, 64)])
@pytest.mark.parametrize("chunk", [32, 64, 512])
def test_paged_attention_matches_oracle(dev, dtype, Hq, Hkv, D, chunk):
    draftkv, _ = _dk()
    rng = np.random.default_rng(Hq + D + chunk)
    b, n, T = 3, 150, 5
    pc = draftkv.PagedKVCache(1, Hkv, D, 16, 64, dtype="bf16" if dtype == "bf16" else np.float32, batch=b,
                              chunk_keys=chunk)
    k = rng.standard_normal((b, n + T, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((b, n + T, Hkv, D)).astype(np.float32)
    if dtype == "bf16":
        k, v = _bf16(k), _bf16(v)
    # ragged: sequence s holds n - 7*s positions before the T queries
    starts = [n - 7 * s for s in range(b)]
    pc.reserve([n + T] * b)
    st0 = torch.zeros(b, dtype=torch.int32, device=dev)
    kk = np.zeros_like(k)
    vv = np.zeros_like(v)
    for s in range(b):
        m = starts[s] + T
        kk[s, :m], vv[s, :m] = k[s, :m], v[s, :m]
    pc.append_layer(0, torch.from_numpy(kk).to(dev), torch.from_numpy(vv).to(dev), st0,
                    torch.tensor([starts[s] + T for s in range(b)], dtype=torch.int32, device=dev))
    q = rng.standard_normal((b, T, Hq, D)).astype(np.float32)
    st = torch.tensor(starts, dtype=torch.int32, device=dev)
    out = pc.attend(0, torch.from_numpy(q).to(dev), st, max_len=n + T).cpu().numpy()
    for s in range(b):
        m = starts[s] + T
        ref, _, _ = attend(q[s], kk[s, :m], vv[s, :m], np.arange(m), np.arange(starts[s], m), Hq // Hkv)
        np.testing.assert_allclose(out[s], ref, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("dtype,Hq,Hkv,D", [("f32", 4, 2, 16), ("bf16", 8, 2, 128), ("bf16", 4, 4, 64),
                                            ("f32", 32, 8, 128)])
def test_paged_attention_ignores_rows_past_count(dev, dtype, Hq, Hkv, D):
    """A ragged forward (a prefill of prompts of different lengths): sequence
    s appends count[s] of the T rows, and the positions past start + count
    hold whatever the pool held before -- here NaN bytes. Valid rows must
    match the oracle over the appended keys alone (a masked key's V times a
    zero probability would be NaN), padding rows must stay finite, and a
    sequence that appended nothing reads zeros."""
    draftkv, _ = _dk()
    rng = np.random.default_rng(D + Hq)
    b, T = 3, 40
    counts = [40, 23, 0]
    pc = draftkv.PagedKVCache(1, Hkv, D, 16, 64, dtype="bf16" if dtype == "bf16" else np.float32, batch=b,
                              chunk_keys=32)
    pc.store.view(torch.uint8).fill_(0xFF)            # stale NaN in every page
    pc.reserve(counts)
    k = rng.standard_normal((b, T, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((b, T, Hkv, D)).astype(np.float32)
    if dtype == "bf16":
        k, v = _bf16(k), _bf16(v)
    st0 = torch.zeros(b, dtype=torch.int32, device=dev)
    cnt = torch.tensor(counts, dtype=torch.int32, device=dev)
    pc.append_layer(0, torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev), st0, cnt)
    q = rng.standard_normal((b, T, Hq, D)).astype(np.float32)
    out = pc.attend(0, torch.from_numpy(q).to(dev), st0, max_len=T, count=cnt).cpu().numpy()
    assert np.isfinite(out).all()
    for s, m in enumerate(counts):
        if m:
            ref, _, _ = attend(q[s, :m], k[s, :m], v[s, :m], np.arange(m), np.arange(m), Hq // Hkv)
            np.testing.assert_allclose(out[s, :m], ref, rtol=RTOL, atol=ATOL)
    assert not out[2].any()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("Hq,Hkv,D,g,n", [(8, 2, 64, 8, 700), (32, 8, 128, 16, 2600), (9, 3, 64, 4, 1030),
                                          (4, 4, 128, 1, 64)])
def test_verify_is_batch_invariant_with_decode(dev, dtype, Hq, Hkv, D, g, n):
    """A verify pass over gamma+1 queries gives each row the bit pattern the
    one-token decode step at that position gives (the losslessness contract),
    also when the rows span several query-tile groups and key super-chunks."""
    draftkv, _ = _dk()
    rng = np.random.default_rng(7 + g)
    b = 2
    pc = draftkv.PagedKVCache(1, Hkv, D, 16, 256, dtype="bf16" if dtype == "bf16" else np.float32, batch=b,
                              chunk_keys=256)
    k = rng.standard_normal((b, n + g, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((b, n + g, Hkv, D)).astype(np.float32)
    pc.reserve([n + g] * b)
    pc.append_layer(0, torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev),
                    torch.zeros(b, dtype=torch.int32, device=dev))
    q = torch.from_numpy(rng.standard_normal((b, g + 1, Hq, D)).astype(np.float32)).to(dev)
    start = torch.full((b,), n - 1, dtype=torch.int32, device=dev)
    ver = pc.attend(0, q, start, max_len=n + g)
    for t in range(g + 1):
        one = pc.attend(0, q[:, t:t + 1].contiguous(), start + t, max_len=n + g)
        assert torch.equal(one[:, 0], ver[:, t]), t


# ------------------------------------------------------------------ mirror maintenance
def _full_pair(L, H, D, n, rng, dev, dtype=np.float32):
    """An oracle FullKVCache and a device PagedKVCache holding the same rows."""
    import draftkv
    full_o = oc.FullKVCache(L)
    full_d = draftkv.PagedKVCache(L, H, D, 16, 4096, dtype=dtype, max_tokens=8192)
    ks = [rng.standard_normal((n, H, D)).astype(np.float32) for _ in range(L)]
    vs = [rng.standard_normal((n, H, D)).astype(np.float32) for _ in range(L)]
    for layer in range(L):
        full_o.append(layer, ks[layer], vs[layer], np.arange(n))
        full_d.append(layer, ks[layer], vs[layer], np.arange(n))
    return full_o, full_d, ks, vs


def _same_mirror(mo, md, L, codes=True):
    for layer in range(L):
        g = md.read_codes(layer)
        assert g["pos"].tolist() == mo.pos[layer].tolist(), layer
        if codes and mo.kq[layer] is not None:
            assert np.array_equal(g["k_codes"], mo.kq[layer][0])
            assert np.array_equal(g["v_codes"], mo.vq[layer][0])
            assert np.array_equal(g["k_scale"], mo.kq[layer][1])
            assert np.array_equal(g["v_lo"], mo.vq[layer][2])
        k, v, p = md.read(layer)
        ko, vo, po = mo.read(layer)
        assert np.array_equal(k, ko) and np.array_equal(v, vo)


# (8-bit arms that evict: with head_dim a multiple of 64 their pages are in
# the attention kernel's lane load order, which the appends, the compaction
# moves and the rebuilds must all write)
ARMS = [Cfg(8, 1.0), Cfg(8, 0.5), Cfg(8, 0.4, 2, 8, group=32, meta="f16"), Cfg(4, 0.5),
        Cfg(4, 0.25, group=32, meta="f16"), Cfg(2, 0.25), Cfg(3, 0.5, 2, 5), Cfg(16, 0.5), Cfg(4, 0.3, 4, 0)]


def _dcfg(c: Cfg):
    from draftkv import CompressionConfig
    return CompressionConfig(c.bits, c.keep_frac, c.sink, c.recent, c.group, c.meta == "f16")


@pytest.mark.parametrize("arm", ARMS, ids=lambda c: f"{c.bits}b{c.keep_frac}g{c.group}{c.meta}s{c.sink}r{c.recent}")
def test_build_and_rebuild_match_reference(dev, arm):
    draftkv, _ = _dk()
    rng = np.random.default_rng(arm.bits)
    L, H, D, n = 3, 2, 64, 300
    full_o, full_d, _, _ = _full_pair(L, H, D, n, rng, dev)
    mo = oc.CompressedKVCache(L, [Cfg(8, 1.0)] * L)
    md = draftkv.CompressedKVCache(L, [_dcfg(Cfg(8, 1.0))] * L)
    assert md.sync_from(full_d, 0) == mo.sync_from(full_o, 0)
    _same_mirror(mo, md, L)
    cfgs_o = [Cfg(8, 1.0)] * L
    cfgs_o[1] = arm
    assert md.rebuild_layers(full_d, [1], [_dcfg(c) for c in cfgs_o]) == mo.rebuild_layers(full_o, [1], cfgs_o)
    _same_mirror(mo, md, L)


@pytest.mark.parametrize("D", [32, 64])
@pytest.mark.parametrize("arm", ARMS, ids=lambda c: f"{c.bits}b{c.keep_frac}g{c.group}{c.meta}s{c.sink}r{c.recent}")
def test_steady_state_eviction_truncate_and_resync(dev, arm, D):
    """Drafting appends one row at a time with accumulated scores; the
    victims, the compaction, truncation and the per-round resync must leave
    the same rows (positions, codes, scores) as the reference."""
    draftkv, _ = _dk()
    rng = np.random.default_rng(11 + arm.bits + D)
    L, H, n = 2, 2, 120
    full_o, full_d, _, _ = _full_pair(L, H, D, n, rng, dev)
    mo = oc.CompressedKVCache(L, [arm] * L)
    md = draftkv.CompressedKVCache(L, [_dcfg(arm)] * L)
    mo.sync_from(full_o, 0)
    md.sync_from(full_d, 0)
    _same_mirror(mo, md, L)
    pos = n
    for rnd in range(6):
        for step in range(5):
            # identical scores on both sides (distinct values, plus a tie)
            for layer in range(L):
                nr = mo.pos[layer].size
                sc = np.round(rng.random(nr) * 4, 1)
                mo.score[layer][:] = sc
                dpos = md.pos[0, layer, :nr].cpu().numpy()
                # device rows are in storage order: map by position
                lut = {int(p): float(s) for p, s in zip(mo.pos[layer], sc)}
                md.score[0, layer, :nr] = torch.tensor([lut[int(p)] for p in dpos], dtype=torch.float64,
                                                       device=dev)
            for layer in range(L):
                k = rng.standard_normal((1, H, D)).astype(np.float32)
                v = rng.standard_normal((1, H, D)).astype(np.float32)
                mo.append(layer, k, v, [pos])
                md.append(layer, k, v, [pos])
            pos += 1
            _same_mirror(mo, md, L)
        # rollback: 2 of the 5 drafted positions accepted; the full cache gets
        # the 3 true rows (2 accepted + the next one) and the mirror resyncs
        # from the last committed position
        full_o.truncate(pos - 5)
        full_d.truncate(pos - 5)
        for layer in range(L):
            k = rng.standard_normal((3, H, D)).astype(np.float32)
            v = rng.standard_normal((3, H, D)).astype(np.float32)
            full_o.append(layer, k, v, np.arange(pos - 5, pos - 2))
            full_d.append(layer, k, v, np.arange(pos - 5, pos - 2))
        start = pos - 6
        assert md.sync_from(full_d, start) == mo.sync_from(full_o, start)
        pos = pos - 2
        _same_mirror(mo, md, L)
        assert md.seen_positions == mo.seen_positions


# ------------------------------------------------------------------ drafter attention
@pytest.mark.parametrize("arm", [Cfg(8, 1.0), Cfg(8, 0.5, group=32, meta="f16"), Cfg(4, 0.25, group=32, meta="f16"),
                                 Cfg(16, 0.5), Cfg(2, 0.5)],
                         ids=lambda c: f"{c.bits}b{c.keep_frac}")
@pytest.mark.parametrize("Hq,Hkv,D", [(4, 4, 16), (32, 8, 128), (9, 3, 64)])
def test_drafter_attention_and_mass(dev, arm, Hq, Hkv, D):
    draftkv, _ = _dk()
    rng = np.random.default_rng(Hq * D + arm.bits)
    L, n = 1, 1500
    full_o, full_d, _, _ = _full_pair(L, Hkv, D, n, rng, dev)
    mo = oc.CompressedKVCache(L, [arm])
    md = draftkv.CompressedKVCache(L, [_dcfg(arm)])
    mo.sync_from(full_o, 0)
    md.sync_from(full_d, 0)
    q = rng.standard_normal((1, Hq, D)).astype(np.float32) * 2.0
    nr = mo.pos[0].size
    before = md.read_codes(0)["score"].copy()
    out = md.attend(0, torch.from_numpy(q).to(dev), want_mass=True).cpu().numpy()
    ck, cv, cpos = mo.read(0)
    ref, _, mp = attend(q, ck, cv, cpos, np.array([n - 1]), Hq // Hkv)
    np.testing.assert_allclose(out, ref, rtol=RTOL, atol=ATOL)
    mass = md.read_codes(0)["score"] - before
    np.testing.assert_allclose(mass, row_mass(mp).astype(np.float64), rtol=1e-4, atol=1e-7)
    assert mass.shape == (nr,)


@pytest.mark.parametrize("arm,D", [(Cfg(8, 1.0), 64), (Cfg(8, 0.5, group=32, meta="f16"), 64),
                                   (Cfg(4, 0.5), 64), (Cfg(4, 0.25, group=32, meta="f16"), 64),
                                   (Cfg(8, 1.0), 128), (Cfg(8, 0.5, group=64, meta="f16"), 128)],
                         ids=lambda x: f"{x.bits}b{x.keep_frac}{x.meta}" if isinstance(x, Cfg) else f"D{x}")
def test_drafter_attention_merged_blocks(dev, arm, D):
    """512 (sequence, KV head) segments (batch 64, 8 KV heads, 32 query
    heads): one block per segment fills the device, so the register-staged
    kernel runs as 8-wave blocks that merge their waves' partials in LDS and
    write the output and row statistics themselves (no combine kernel).
    Ragged lengths (300 - 3 s rows) leave some waves of every block with no
    page. Every sequence's output and the mass added to its kept rows match
    the oracle's."""
    import draftkv
    b, Hkv, Hq = 64, 8, 32
    lens = np.array([300 - 3 * s for s in range(b)], np.int64)
    T = int(lens.max())
    full = draftkv.PagedKVCache(1, Hkv, D, 16, T // 16 + 2, dtype=np.float32, batch=b, max_tokens=T + 32)
    full.reserve(lens)
    rng = np.random.default_rng(D + arm.bits)
    k = rng.standard_normal((b, T, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((b, T, Hkv, D)).astype(np.float32)
    full.append_layer(0, torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev),
                      torch.zeros(b, dtype=torch.int32, device=dev), torch.tensor(lens, dtype=torch.int32, device=dev))
    full.commit(lens)
    md = draftkv.CompressedKVCache(1, [_dcfg(arm)], batch=b, cap=T + 32)
    md.sync_from(full, 0)
    q = (rng.standard_normal((b, Hq, D)) * 2.0).astype(np.float32)
    out = md.attend(0, torch.from_numpy(q).to(dev), want_mass=True).cpu().numpy()
    for s in range(b):
        n = int(lens[s])
        g = md.read_codes(0, s)
        pos = g["pos"].astype(np.int64)
        kq = quantize_codes(k[s][pos], arm.bits, arm.group, arm.meta)
        vq = quantize_codes(v[s][pos], arm.bits, arm.group, arm.meta)
        ref, _, mp = attend(q[s][None], kq[3], vq[3], pos, np.array([n]), Hq // Hkv)
        np.testing.assert_allclose(out[s], ref[0], rtol=RTOL, atol=ATOL, err_msg=f"seq {s}")
        np.testing.assert_allclose(g["score"], row_mass(mp).astype(np.float64), rtol=1e-4, atol=1e-7,
                                   err_msg=f"seq {s} mass")


def test_splitk_timing_hook_times_each_call(dev):
    """The benchmark hook records events around the split-K kernel only: its
    time is positive and below the whole call's, and off means no events."""
    draftkv, _ = _dk()
    from draftkv import ops
    rng = np.random.default_rng(5)
    _, full_d, _, _ = _full_pair(1, 8, 128, 3000, rng, dev)
    md = draftkv.CompressedKVCache(1, [_dcfg(Cfg(4, 0.25, group=32, meta="f16"))])
    md.sync_from(full_d, 0)
    q = torch.from_numpy(rng.standard_normal((1, 32, 128)).astype(np.float32)).to(dev)
    ops.drafter_kernel_timing(True)
    try:
        for _ in range(3):
            s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s_ev.record()
            md.attend(0, q, want_mass=True)
            e_ev.record()
            k_ms = ops.drafter_kernel_last_ms()
            torch.cuda.synchronize()
            assert 0.0 < k_ms <= s_ev.elapsed_time(e_ev) + 1e-3
        # back to back: one pair per call, summed once at the end
        ops.drafter_kernel_timing(True)
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_ev.record()
        for _ in range(5):
            md.attend(0, q, want_mass=True)
        e_ev.record()
        total, n = ops.drafter_kernel_total_ms()
        torch.cuda.synchronize()
        assert n == 5 and 0.0 < total <= s_ev.elapsed_time(e_ev) + 1e-3
    finally:
        ops.drafter_kernel_timing(False)


# ------------------------------------------------------------------ sampling and accept
@pytest.mark.parametrize("V", [128, 50257, 128256])
@pytest.mark.parametrize("T", [0.0, 0.8, 1.0])
def test_sample_matches_numpy_choice(dev, V, T):
    _, ops = _dk()
    rng = np.random.default_rng(V)
    b = 6
    logits = (rng.standard_normal((b, V)) * 3).astype(np.float32)
    logits[1, 7] = logits[1].max() + 0.0          # tie for argmax -> first index
    logits[1, 3] = logits[1, 7]
    u = rng.random(b)
    tok = ops.sample(torch.from_numpy(logits).to(dev), T, torch.from_numpy(u).to(dev)).cpu().numpy()
    for s in range(b):
        assert tok[s] == sample_u(o_probs(logits[s], T), u[s]), s


def _accept_case(ops, dev, b, gamma, V, T, seed, stats=False):
    """Target rows near a shared base, draft rows near it too, drafted tokens
    mostly the target's argmax (long accepted runs) and sometimes not; the
    device decision against the oracle rule for every sequence. stats: the
    draft rows' normalisers come from dkv_sample on each draft step's logits
    (as the decode round passes them), and the decision also equals the one
    that recomputes them."""
    rng = np.random.default_rng(seed)
    base = rng.standard_normal((b, 1, V)).astype(np.float32) * 2
    target = (base + 0.3 * rng.standard_normal((b, gamma + 1, V))).astype(np.float32)
    draft = (base[:, :1] + 0.3 * rng.standard_normal((b, gamma, V))).astype(np.float32)
    toks = np.zeros((b, gamma), np.int32)
    for s in range(b):
        for i in range(gamma):
            toks[s, i] = int(np.argmax(target[s, i])) if rng.random() < 0.95 else int(rng.integers(V))
    u = rng.random((b, gamma + 1))
    # the draft steps' logits go to the library step-major: [gamma, batch, vocab]
    t_d, d_d, k_d, u_d = (torch.from_numpy(np.ascontiguousarray(x)).to(dev)
                          for x in (target, draft.transpose(1, 0, 2), toks, u))
    acc, nxt, used = ops.accept(t_d, d_d, k_d, T, u_d)
    acc, nxt, used = acc.cpu().numpy(), nxt.cpu().numpy(), used.cpu().numpy()
    if stats and T > 0:
        ds = ops.row_stats(b, dev, (gamma,))
        for i in range(gamma):
            ops.sample(d_d[i], T, u_d[:, i].contiguous(), stats_out=ds[i])
        got = [x.cpu().numpy() for x in ops.accept(t_d, d_d, k_d, T, u_d, ds)]
        for x, y, name in zip((acc, nxt, used), got, ("accepted", "next_token", "n_uniforms")):
            assert np.array_equal(x, y), name
    for s in range(b):
        qs = [o_probs(draft[s, i], T) for i in range(gamma)]
        ra, rn, ru = o_accept(target[s], toks[s].tolist(), qs, T, u[s])
        assert (acc[s], nxt[s], used[s]) == (ra, rn, ru), (s, (acc[s], nxt[s], used[s]), (ra, rn, ru))
    return acc


@pytest.mark.parametrize("T", [0.0, 0.8])
@pytest.mark.parametrize("b,gamma", [(32, 2), (32, 3), (32, 8), (32, 16), (32, 20), (4, 80)])
def test_accept_matches_reference_rule_at_bench_points(dev, T, b, gamma):
    """Where the benchmark runs the decision: batch 32, the Llama-3-8B
    vocabulary (128256), gamma from the 2-3 its controller settles on up to
    its bound of 20, greedy and T = 0.8; and
    a draft longer than one 64-position block of the decide kernel. Accepted
    counts, next tokens and uniforms consumed equal the oracle rule's
    (engine.py:188-213) for every sequence."""
    _, ops = _dk()
    acc = _accept_case(ops, dev, b, gamma, 128256, T, 1000 + gamma + int(T * 10), stats=True)
    assert acc.max() > 0


@pytest.mark.parametrize("V", [128256, 50257])
def test_sample_row_stats_are_the_float64_normaliser(dev, V):
    """dkv_sample's row statistics: m = max(x) * (1/T), s = the sum over the
    row of exp(x/T - m) in float64 (within 1e-13 relative of numpy's), 1/s;
    a ragged batch of 7 rows with -inf and -30000 entries; odd vocab takes the
    float read path."""
    _, ops = _dk()
    rng = np.random.default_rng(V + 3)
    b, T = 7, 0.8
    x = (rng.standard_normal((b, V)) * 3).astype(np.float32)
    x[2, :50] = -np.inf
    x[3, 7] = -30000.0
    st = ops.row_stats(b, dev)
    ops.sample(torch.from_numpy(x).to(dev), T, torch.from_numpy(rng.random(b)).to(dev), stats_out=st)
    st = st.cpu().numpy()
    iT = 1.0 / float(np.float32(T))   # the library takes T as float32
    for s in range(b):
        m = float(x[s].max()) * iT
        y = x[s].astype(np.float64) * iT - m
        S = float(np.exp(y).sum())
        assert st[s, 0] == m, s
        assert abs(st[s, 1] - S) <= 1e-13 * S, (s, st[s, 1], S)
        assert abs(st[s, 2] * st[s, 1] - 1.0) <= 1e-15, s


@pytest.mark.parametrize("T", [0.0, 0.8])
@pytest.mark.parametrize("gamma", [1, 4, 8])
def test_accept_matches_reference_rule(dev, T, gamma):
    _, ops = _dk()
    rng = np.random.default_rng(gamma * 10 + int(T * 10))
    b, V = 16, 5000
    base = rng.standard_normal((b, 1, V)).astype(np.float32) * 2
    target = (base + 0.3 * rng.standard_normal((b, gamma + 1, V))).astype(np.float32)
    draft = (base[:, :1] + 0.3 * rng.standard_normal((b, gamma, V))).astype(np.float32)
    toks = np.zeros((b, gamma), np.int32)
    for s in range(b):
        for i in range(gamma):
            # mostly the target argmax so long runs get accepted, sometimes not
            toks[s, i] = int(np.argmax(target[s, i])) if rng.random() < 0.8 else int(rng.integers(V))
    u = rng.random((b, gamma + 1))
    acc, nxt, used = ops.accept(torch.from_numpy(target).to(dev),
                                torch.from_numpy(np.ascontiguousarray(draft.transpose(1, 0, 2))).to(dev),
                                torch.from_numpy(toks).to(dev), T, torch.from_numpy(u).to(dev))
    acc, nxt, used = acc.cpu().numpy(), nxt.cpu().numpy(), used.cpu().numpy()
    for s in range(b):
        qs = [o_probs(draft[s, i], T) for i in range(gamma)]
        ra, rn, ru = o_accept(target[s], toks[s].tolist(), qs, T, u[s])
        assert (acc[s], nxt[s], used[s]) == (ra, rn, ru), s


@pytest.mark.parametrize("V", [128256, 50257])
def test_accept_all_zero_residual_falls_back_to_p(dev, V):
    """A rejection where p and q are the same row (the drafted token's
    probability underflows to 0, so the ratio test fails) leaves an all-zero
    residual; the next token is then drawn from p itself (engine.py:210-211).
    Other sequences of the batch reject with a real residual or accept every
    position. Decisions equal the oracle rule's; a target view that starts
    off a 16-byte boundary takes the scalar read path."""
    _, ops = _dk()
    rng = np.random.default_rng(V + 7)
    b, gamma, T = 12, 3, 0.8
    target = (rng.standard_normal((b, gamma + 1, V)) * 2).astype(np.float32)
    draft = (target[:, :gamma] + 0.2 * rng.standard_normal((b, gamma, V))).astype(np.float32)
    toks = np.argmax(target[:, :gamma], axis=2).astype(np.int32)
    for s in range(0, b, 3):                        # p == q at the rejected row, p[d] = q[d] = 0
        r = (s // 3) % gamma
        toks[s, r] = 11
        target[s, r, 11] = -30000.0
        draft[s, : r + 1] = target[s, : r + 1]      # (ratio 1 before it: accepted)
    for s in range(1, b, 3):                        # q far above p at a random token: a plain rejection
        r, d = s % gamma, int(rng.integers(V))
        toks[s, r] = d
        draft[s, r, d] = target[s, r].max() + 6.0
    u = rng.random((b, gamma + 1))
    t_dev = torch.from_numpy(target).to(dev)
    cases = [t_dev]
    if V % 4 == 0:
        flat = torch.empty(t_dev.numel() + 1, dtype=torch.float32, device=dev)
        flat[1:].copy_(t_dev.reshape(-1))
        cases.append(flat[1:].view(b, gamma + 1, V))   # 4 bytes past an aligned start
    for tgt in cases:
        acc, nxt, used = ops.accept(tgt, torch.from_numpy(np.ascontiguousarray(draft.transpose(1, 0, 2))).to(dev),
                                    torch.from_numpy(toks).to(dev), T,
                                    torch.from_numpy(u).to(dev))
        acc, nxt, used = acc.cpu().numpy(), nxt.cpu().numpy(), used.cpu().numpy()
        for s in range(b):
            qs = [o_probs(draft[s, i], T) for i in range(gamma)]
            want = o_accept(target[s], toks[s].tolist(), qs, T, u[s])
            assert (acc[s], nxt[s], used[s]) == want, (s, (acc[s], nxt[s], used[s]), want)
        assert (acc[0::3] == (np.arange(0, b, 3) // 3) % gamma).all()
