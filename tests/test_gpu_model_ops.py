"""The model-forward kernels (include/draftkv_hip.h "model forward ops") against
plain PyTorch float32 references of the same ops, with float32 and bf16 inputs
and row counts that exercise the 2-D grids (1, 7, 32 and 300 rows)."""

import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ops():
    from draftkv import ops
    return ops


ROWS = [1, 7, 32, 300]


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("d", [64, 100, 576, 768, 4096, 8192])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_add_rmsnorm_and_layernorm(dev, rows, d, xdt):
    ops = _ops()
    g = torch.Generator(device=dev).manual_seed(rows * 7 + d)
    h0 = torch.randn((rows, d), generator=g, device=dev)
    x = torch.randn((rows, d), generator=g, device=dev).to(xdt)
    bias = torch.randn((d,), generator=g, device=dev).to(xdt)
    w = (1 + 0.1 * torch.randn((d,), generator=g, device=dev)).to(xdt)
    b = (0.1 * torch.randn((d,), generator=g, device=dev)).to(xdt)
    for ln in (False, True):
        h = h0.clone()
        out = ops.add_norm(h, x, bias, w, b if ln else None, 1e-5, ln, torch.float32)
        ref_h = h0 + x.float() + bias.float()
        if ln:
            mu = ref_h.mean(-1, keepdim=True)
            var = ((ref_h - mu) ** 2).mean(-1, keepdim=True)
            ref = (ref_h - mu) / torch.sqrt(var + 1e-5) * w.float() + b.float()
        else:
            ref = ref_h / torch.sqrt((ref_h * ref_h).mean(-1, keepdim=True) + 1e-5) * w.float()
        torch.testing.assert_close(h, ref_h, rtol=1e-6, atol=1e-6)
        torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)
        o16 = ops.add_norm(h0.clone(), x, bias, w, b if ln else None, 1e-5, ln, torch.bfloat16)
        assert o16.dtype == torch.bfloat16
        torch.testing.assert_close(o16.float(), ref.bfloat16().float(), rtol=0, atol=0.02 * ref.abs().max().item())
    plain = ops.rmsnorm(h0, w, 1e-6)
    torch.testing.assert_close(plain, h0 / torch.sqrt((h0 * h0).mean(-1, keepdim=True) + 1e-6) * w.float(),
                               rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("hq,hkv,d", [(4, 4, 16), (32, 8, 128), (9, 3, 64)])
@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_qkv_split_rope(dev, rows, hq, hkv, d, rope, xdt):
    ops = _ops()
    g = torch.Generator(device=dev).manual_seed(rows + hq + d)
    n = (hq + 2 * hkv) * d
    qkv = torch.randn((rows, n), generator=g, device=dev).to(xdt)
    bias = torch.randn((n,), generator=g, device=dev).to(xdt)
    pos = torch.randint(0, 5000, (rows,), generator=g, device=dev, dtype=torch.int32)
    max_pos = 8192
    inv = 1.0 / (500000.0 ** (np.arange(0, d, 2) / d))
    ang = np.outer(np.arange(max_pos), inv)
    cs = torch.as_tensor(np.stack([np.cos(ang), np.sin(ang)]).astype(np.float32)).to(dev)
    q, k, v = ops.qkv_split(qkv, bias, hq, hkv, d, pos if rope else None, cs if rope else None, max_pos)
    x = qkv.float() + bias.float()
    rq = x[:, : hq * d].view(rows, hq, d)
    rk = x[:, hq * d: (hq + hkv) * d].view(rows, hkv, d)
    rv = x[:, (hq + hkv) * d:].view(rows, hkv, d)
    if rope:
        c = cs[0][pos.long()].repeat(1, 2)[:, None, :]
        s = cs[1][pos.long()].repeat(1, 2)[:, None, :]

        def rot(t):
            return torch.cat([-t[..., d // 2:], t[..., : d // 2]], -1)

        rq, rk = rq * c + rot(rq) * s, rk * c + rot(rk) * s
    torch.testing.assert_close(q, rq, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(k, rk, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(v, rv, rtol=0, atol=0)


@pytest.mark.parametrize("rows", ROWS)
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_activations(dev, rows, xdt):
    ops = _ops()
    g = torch.Generator(device=dev).manual_seed(rows)
    ff = 1536
    gu = (2 * torch.randn((rows, 2 * ff), generator=g, device=dev)).to(xdt)
    ref = torch.nn.functional.silu(gu[:, :ff].float()) * gu[:, ff:].float()
    torch.testing.assert_close(ops.silu_mul(gu), ref, rtol=1e-5, atol=1e-5)
    x = (2 * torch.randn((rows, 3072), generator=g, device=dev)).to(xdt)
    bias = torch.randn((3072,), generator=g, device=dev)
    xb = x.float() + bias
    ref = 0.5 * xb * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (xb + 0.044715 * xb ** 3)))
    torch.testing.assert_close(ops.bias_gelu(x, bias), ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(ops.relu(x), torch.relu(x.float()), rtol=0, atol=0)
    h = torch.randn((rows, 3072), generator=g, device=dev)
    ref = h + x.float() + bias
    torch.testing.assert_close(ops.add_(h, x, bias), ref, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("M,N,K", [(1, 97, 64), (9, 200, 130), (300, 64, 768)])
@pytest.mark.parametrize("layout", [0, 1])
def test_gemm_f32_and_batch_invariance(dev, M, N, K, layout):
    ops = _ops()
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    x = torch.randn((M, K), generator=g, device=dev)
    w = torch.randn((K, N) if layout == 0 else (N, K), generator=g, device=dev)
    bias = torch.randn((N,), generator=g, device=dev)
    ref = x.double() @ (w.double() if layout == 0 else w.double().t()) + bias.double()
    out = ops.gemm_f32(x, w, layout, bias)
    torch.testing.assert_close(out.double(), ref, rtol=1e-4, atol=1e-4)
    acc = torch.randn((M, N), generator=g, device=dev)
    got = ops.gemm_f32(x, w, layout, bias, out=acc.clone(), accumulate=True)
    torch.testing.assert_close(got.double(), ref + acc.double(), rtol=1e-4, atol=1e-4)
    # one row alone == the same row inside the batch, bit for bit
    r = M // 2
    one = ops.gemm_f32(x[r:r + 1].contiguous(), w, layout, bias)
    assert torch.equal(one[0], out[r])


@pytest.mark.parametrize("M,N,K,with_bias", [(1, 64, 128, False), (5, 96, 160, True), (6, 1024, 4096, True),
                                             (8, 4096, 14336, False), (17, 6144, 4096, False),
                                             (32, 4096, 4096, True), (33, 512, 14336, False),
                                             (96, 6144, 4096, True), (200, 1024, 2048, False), (64, 272, 96, True),
                                             (544, 4096, 4096, False), (32, 28672, 4096, True),
                                             (96, 28672, 4096, False), (160, 6144, 4096, False),
                                             (288, 4096, 4096, True), (288, 28672, 4096, False),
                                             # larger verify blocks: up to six m tiles, a partial last
                                             # fragment, the 28672-row weight at 16 fragments
                                             (65, 4096, 4096, False), (300, 6144, 4096, True),
                                             (352, 1024, 4096, False), (672, 4096, 1024, True),
                                             (256, 28672, 4096, False), (130, 4096, 14336, False),
                                             # W ending inside a 16-row fragment (a tied GPT-2 head: 50257 rows)
                                             (1, 50257, 768, False), (5, 50257, 768, True), (33, 50257, 768, False),
                                             (3, 40, 4096, True), (96, 1001, 2048, True), (17, 23, 96, True)])
def test_gemm_bf16_matches_fp32_and_is_batch_invariant(dev, M, N, K, with_bias):
    """bf16 x @ W^T (+ b) against the float32 product of the same bf16 values
    (one rounding to bf16 apart), float32 output too, and every row equal to
    the same row computed alone or in a smaller batch, bit for bit. The
    shapes take every launch plan: one or two W fragments per wave, x tiles
    of 16 to 128 rows, several M tiles, K chunks split over workgroups
    (partials + ordered reduce) or summed inside one, the small-M kernel that
    splits K among the waves of a workgroup, 128-k blocks and the 32-k
    tail, the 7-wave workgroups of the 28672-row gate/up weight (whose
    rows must equal those of the 4-wave plan at M = 96), x tiles cut evenly
    (M = 96: one of 96 rows; 160: two of 80; 288: three of 96), and any N: a last
    fragment of fewer than 16 W rows (odd N: element stores) in the main and
    the small-M kernels."""
    ops = _ops()
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    w = (0.05 * torch.randn((N, K), generator=g, device=dev)).to(torch.bfloat16)
    bias = torch.randn((N,), generator=g, device=dev).to(torch.bfloat16) if with_bias else None
    ref = x.float() @ w.float().t()
    if bias is not None:
        ref = ref + bias.float()
    y = ops.gemm_bf16(x, w, bias)
    assert y.dtype == torch.bfloat16 and y.shape == (M, N)
    # one rounding of a float32 sum: within 2^-8 relative plus the sum's own error
    torch.testing.assert_close(y.float(), ref, rtol=2 ** -8, atol=1e-3 * math.sqrt(K / 128))
    y32 = ops.gemm_bf16(x, w, bias, out_dtype=torch.float32)
    torch.testing.assert_close(y32, ref, rtol=1e-5, atol=2e-4 * math.sqrt(K / 128))
    assert torch.equal(y32.to(torch.bfloat16), y)
    for r in sorted({0, M // 2, M - 1}):
        one = ops.gemm_bf16(x[r:r + 1].contiguous(), w, bias)
        assert torch.equal(one[0], y[r])
    if M > 17:
        part = ops.gemm_bf16(x[3:17].contiguous(), w, bias)
        assert torch.equal(part, y[3:17])


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (5, 96, 160), (8, 512, 14336), (32, 4096, 4096),
                                   (96, 1024, 2048), (200, 272, 96), (288, 4096, 4096), (130, 6144, 4096),
                                   (352, 1024, 1024)])
def test_gemm_bf16_float32_x_equals_converting_first(dev, M, N, K):
    """A float32 x is rounded to bf16 (nearest even) as the kernels read it:
    the result is bit for bit that of x.to(bfloat16), for every launch plan."""
    ops = _ops()
    g = torch.Generator(device=dev).manual_seed(M * 7 + N + K)
    x = torch.randn((M, K), generator=g, device=dev) * 3.0
    w = (0.05 * torch.randn((N, K), generator=g, device=dev)).to(torch.bfloat16)
    bias = torch.randn((N,), generator=g, device=dev).to(torch.bfloat16)
    for b in (None, bias):
        assert torch.equal(ops.gemm_bf16(x, w, b), ops.gemm_bf16(x.to(torch.bfloat16), w, b))
        assert torch.equal(ops.gemm_bf16(x, w, b, out_dtype=torch.float32),
                           ops.gemm_bf16(x.to(torch.bfloat16), w, b, out_dtype=torch.float32))


@pytest.mark.parametrize("M,ff,K", [(1, 2048, 4096), (5, 48, 160), (8, 512, 2048), (32, 14336, 4096),
                                    (96, 512, 1024), (200, 136, 96), (288, 14336, 4096), (160, 512, 1024),
                                    # 7-wave workgroups with x tiles of 48 to 128 rows (the Llama-3-8B gate/up)
                                    (96, 14336, 4096), (65, 14336, 4096), (128, 14336, 4096), (40, 14336, 4096)])
def test_gemm_bf16_swiglu_epilogue_equals_unfused(dev, M, ff, K):
    """The SwiGLU epilogue (interleaved gate/up rows) gives bit for bit the
    unfused result: the [gate; up] GEMM rounded to bf16, then the SwiGLU
    kernel -- for every launch plan, bf16 and float32 x."""
    ops = _ops()
    g = torch.Generator(device=dev).manual_seed(M + ff + K)
    w = (0.05 * torch.randn((2 * ff, K), generator=g, device=dev)).to(torch.bfloat16)
    wi = w.view(2, ff, K).transpose(0, 1).reshape(2 * ff, K).contiguous()
    x = torch.randn((M, K), generator=g, device=dev) * 2.0
    for xx in (x, x.to(torch.bfloat16)):
        ref = ops.silu_mul(ops.gemm_bf16(xx, w), torch.bfloat16)
        got = ops.gemm_bf16(xx, wi, swiglu=True)
        assert got.shape == (M, ff) and torch.equal(got, ref)


@pytest.mark.parametrize("M,N,K", [(32, 4096, 4096), (96, 4096, 14336), (1, 4096, 4096), (288, 4096, 4096),
                                   (32, 256, 512)])
@pytest.mark.parametrize("layer_norm", [False, True])
def test_add_norm_on_deferred_partials_equals_gemm_then_add_norm(dev, M, N, K, layer_norm):
    """A GEMM that leaves its per-chunk partials (DKV_GEMM_DEFER) to the
    residual add + norm gives bit for bit the GEMM's bf16 output followed by
    the add-norm: the same out and the same updated residual, with a bias,
    float32 and bf16 x; plans without partials return the tensor as usual."""
    ops = _ops()
    g = torch.Generator(device=dev).manual_seed(M * 7 + N + K + layer_norm)
    w = (0.05 * torch.randn((N, K), generator=g, device=dev)).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(N, generator=g, device=dev)).to(torch.bfloat16)
    nb = (0.1 * torch.randn(N, generator=g, device=dev)).to(torch.bfloat16)
    bias = (0.1 * torch.randn(N, generator=g, device=dev)).to(torch.bfloat16)
    h0 = torch.randn((M, N), generator=g, device=dev)
    x = torch.randn((M, K), generator=g, device=dev) * 2.0
    planned = ops.lib().dkv_gemm_bf16_partials(M, N, K)
    for xx in (x, x.to(torch.bfloat16)):
        y = ops.gemm_bf16(xx, w)
        h_ref = h0.clone()
        ref = ops.add_norm(h_ref, y, bias, nw, nb, 1e-5, layer_norm, torch.bfloat16)
        p = ops.gemm_bf16(xx, w, defer=True)
        assert isinstance(p, ops.Partials) == (planned > 0)
        h_got = h0.clone()
        got = ops.add_norm(h_got, p, bias, nw, nb, 1e-5, layer_norm, torch.bfloat16)
        assert torch.equal(got, ref) and torch.equal(h_got, h_ref)
    if (M, N, K) == (32, 4096, 4096):
        assert planned > 1, "the Llama-3-8B o projection at M = 32 should run with partials"


@pytest.mark.parametrize("M,rope,bias", [(32, True, False), (96, True, True), (3, False, True), (32, False, False),
                                         (288, True, False)])
def test_qkv_split_on_deferred_partials_equals_gemm_then_split(dev, M, rope, bias):
    """qkv_split reading the qkv GEMM's deferred partials equals the split of
    the GEMM's bf16 output bit for bit (q, k, v; RoPE and a projection bias)."""
    ops = _ops()
    Hq, Hkv, D, K = 32, 8, 128, 4096
    N = (Hq + 2 * Hkv) * D
    g = torch.Generator(device=dev).manual_seed(M + 31 * rope + bias)
    w = (0.05 * torch.randn((N, K), generator=g, device=dev)).to(torch.bfloat16)
    b = (0.1 * torch.randn(N, generator=g, device=dev)).to(torch.bfloat16) if bias else None
    x = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    pos = torch.randint(0, 4000, (M,), generator=g, device=dev, dtype=torch.int32)
    cs, n = None, 0
    if rope:
        n = 4096
        inv = 1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
        ang = torch.outer(torch.arange(n, dtype=torch.float64), inv)
        cs = torch.stack([ang.cos(), ang.sin()]).float().to(dev).contiguous()
    ref = ops.qkv_split(ops.gemm_bf16(x, w), b, Hq, Hkv, D, pos, cs, n)
    p = ops.gemm_bf16(x, w, defer=True)
    assert isinstance(p, ops.Partials) == (ops.lib().dkv_gemm_bf16_partials(M, N, K) > 0)
    got = ops.qkv_split(p, b, Hq, Hkv, D, pos, cs, n)
    for r, o in zip(ref, got):
        assert torch.equal(r, o)


@pytest.mark.parametrize("M,N,K,with_bias", [(1, 4096, 4096, False), (6, 1024, 4096, True), (8, 4096, 14336, False),
                                             (17, 6144, 4096, True), (32, 4096, 4096, False),
                                             (32, 28672, 4096, False), (12, 28672, 4096, True),
                                             (96, 6144, 4096, False), (200, 1024, 2048, True), (96, 4096, 14336, False),
                                             (288, 28672, 4096, False), (288, 4096, 4096, True),
                                             (352, 6144, 4096, False)])
def test_gemm_bf16_tiled_weights_equal_row_major(dev, M, N, K, with_bias):
    """W stored in 16x128 tiles (ops.TiledW, DKV_GEMM_WTILED) gives bit for bit
    the row-major product on every launch plan (small-M in-workgroup split, x
    tiles of 16-128 rows, one or two fragments per wave, 7-wave workgroups,
    partials + reduce or deferred to the consumer, float32 output, float32 x,
    the SwiGLU epilogue)."""
    ops = _ops()
    g = torch.Generator(device=dev).manual_seed(M * 3 + N + K)
    w = (0.05 * torch.randn((N, K), generator=g, device=dev)).to(torch.bfloat16)
    wt = ops.TiledW(w)
    assert torch.equal(wt.rows(), w)
    bias = (0.1 * torch.randn(N, generator=g, device=dev)).to(torch.bfloat16) if with_bias else None
    x = torch.randn((M, K), generator=g, device=dev)
    for xx in (x, x.to(torch.bfloat16)):
        assert torch.equal(ops.gemm_bf16(xx, wt, bias), ops.gemm_bf16(xx, w, bias))
        assert torch.equal(ops.gemm_bf16(xx, wt, bias, out_dtype=torch.float32),
                           ops.gemm_bf16(xx, w, bias, out_dtype=torch.float32))
    if not with_bias:   # the deferred partials (the op workspace holds one set at a time)
        pr = ops.gemm_bf16(x, w, defer=True)
        ref = pr.part.view(torch.float32)[: pr.n_part * M * N].clone() if isinstance(pr, ops.Partials) else pr
        pt = ops.gemm_bf16(x, wt, defer=True)
        assert isinstance(pt, ops.Partials) == isinstance(pr, ops.Partials)
        got = pt.part.view(torch.float32)[: pt.n_part * M * N] if isinstance(pt, ops.Partials) else pt
        assert torch.equal(got, ref)
    if N % 32 == 0:
        assert torch.equal(ops.gemm_bf16(x, wt, swiglu=True), ops.gemm_bf16(x, w, swiglu=True))


def test_gemm_bf16_rejects_unsupported_operands(dev):
    ops = _ops()
    x = torch.zeros((4, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.gemm_bf16(x, torch.zeros((40, 64), dtype=torch.bfloat16, device=dev), swiglu=True)   # SwiGLU: N % 16
    with pytest.raises(ValueError):
        ops.gemm_bf16(x[:, :48].contiguous(), torch.zeros((32, 48), dtype=torch.bfloat16, device=dev))   # K % 32
    with pytest.raises(ValueError):
        ops.gemm_bf16(x, torch.zeros((32, 64), dtype=torch.bfloat16, device=dev),
                      torch.zeros((32,), dtype=torch.float32, device=dev))            # bias dtype
    with pytest.raises(ValueError):
        ops.gemm_bf16(x.to(torch.float16), torch.zeros((32, 64), dtype=torch.bfloat16, device=dev))   # x dtype
    with pytest.raises(ValueError):
        ops.gemm_bf16(x, torch.zeros((32, 64), dtype=torch.bfloat16, device=dev),
                      torch.zeros((32,), dtype=torch.bfloat16, device=dev), swiglu=True)   # SwiGLU takes no bias


def test_embed_with_positions(dev):
    ops = _ops()
    g = torch.Generator(device=dev).manual_seed(3)
    table = torch.randn((50, 96), generator=g, device=dev).bfloat16()
    pos_t = torch.randn((40, 96), generator=g, device=dev).bfloat16()
    tok = torch.randint(0, 50, (33,), generator=g, device=dev, dtype=torch.int32)
    pos = torch.randint(0, 40, (33,), generator=g, device=dev, dtype=torch.int32)
    out = ops.embed(table, tok, pos_t, pos)
    torch.testing.assert_close(out, table.float()[tok.long()] + pos_t.float()[pos.long()], rtol=0, atol=0)


def test_library_stream_is_torchs_current_stream(dev):
    """Every launch goes to torch's current stream: the default stream, a
    side stream entered with torch.cuda.stream, and back."""
    from draftkv import ops
    assert ops._stream() == torch.cuda.current_stream().cuda_stream
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        assert ops._stream() == s.cuda_stream
    assert ops._stream() == torch.cuda.current_stream().cuda_stream
