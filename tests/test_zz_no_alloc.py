"""dkv_accept_noalloc -- the accept decision with its workspace in the
library's static device scratch (no allocation) -- against dkv_accept with a
caller workspace, through the C ABI: accepted counts, next tokens and draws
consumed equal bit for bit, greedy and sampled, on two calls in a row (the
second smaller, so it runs over what the first left in the scratch), and a
request larger than the scratch is refused before any launch."""

import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(seed, b, gamma, V, dev):
    rng = np.random.default_rng(seed)
    base = rng.standard_normal((b, 1, V)).astype(np.float32) * 2
    target = (base + 0.3 * rng.standard_normal((b, gamma + 1, V))).astype(np.float32)
    draft = (base[:, :1] + 0.3 * rng.standard_normal((b, gamma, V))).astype(np.float32)
    toks = np.zeros((b, gamma), np.int32)
    for s in range(b):
        for i in range(gamma):
            toks[s, i] = int(np.argmax(target[s, i])) if rng.random() < 0.8 else int(rng.integers(V))
    u = rng.random((b, gamma + 1))
    # draft logits step-major, [gamma, batch, vocab], as the library takes them
    return [torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in (target, draft.transpose(1, 0, 2), toks, u)]


def _run(fn_noalloc, target, draft, toks, u, T):
    from draftkv._lib import check, lib
    b, g1, V = target.shape
    gamma = g1 - 1
    outs = [torch.full((b,), -7, dtype=torch.int32, device=target.device) for _ in range(3)]
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = (target.data_ptr(), draft.data_ptr(), toks.data_ptr(), b, gamma, V, float(T), u.data_ptr(), None,
            *(o.data_ptr() for o in outs))
    if fn_noalloc:
        check(lib().dkv_accept_noalloc(*args, stream), "dkv_accept_noalloc")
    else:
        nbytes = lib().dkv_accept_workspace(b, gamma, V)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=target.device)
        check(lib().dkv_accept(*args, ws.data_ptr(), nbytes, stream), "dkv_accept")
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs]


@pytest.mark.parametrize("T", [0.0, 0.8])
def test_noalloc_equals_workspace_entry_point_twice(dev, T):
    for seed, (b, gamma, V) in ((1, (16, 8, 50257)), (2, (5, 2, 3000))):
        target, draft, toks, u = _case(seed + int(T * 10), b, gamma, V, dev)
        want = _run(False, target, draft, toks, u, T)
        got = _run(True, target, draft, toks, u, T)
        for w, g, name in zip(want, got, ("accepted", "next_token", "n_uniforms")):
            assert np.array_equal(w, g), (b, gamma, V, name)
        assert (want[0] >= 0).all() and (want[0] <= gamma).all()


def test_noalloc_refuses_more_than_the_scratch(dev):
    """A request whose workspace exceeds the static scratch is refused with
    DKV_ECAPACITY before any launch. Its inputs and outputs are real device
    tensors of the request's sizes: what is tested is the refusal, never a
    launch on pointers that do not hold the data."""
    from draftkv._lib import lib
    L = lib()
    b, gamma, V = 256, 40, 65536
    nbytes = L.dkv_accept_workspace(b, gamma, V)
    assert nbytes > (16 << 20)   # DKV_ACCEPT_SCRATCH_BYTES
    target = torch.zeros((b, gamma + 1, V), dtype=torch.float32, device=dev)
    draft = torch.zeros((gamma, b, V), dtype=torch.float32, device=dev)
    toks = torch.zeros((b, gamma), dtype=torch.int32, device=dev)
    u = torch.zeros((b, gamma + 1), dtype=torch.float64, device=dev)
    outs = [torch.zeros(b, dtype=torch.int32, device=dev) for _ in range(3)]
    rc = L.dkv_accept_noalloc(target.data_ptr(), draft.data_ptr(), toks.data_ptr(), b, gamma, V, 0.8, u.data_ptr(),
                              None, *(o.data_ptr() for o in outs), None)
    torch.cuda.synchronize()
    assert rc == -4 and b"static scratch" in L.dkv_last_error()
    assert all(not o.any() for o in outs)     # nothing ran
