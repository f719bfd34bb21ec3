"""dwm_moe_dispatch_noalloc (the dispatch without a workspace or any
allocation) through the C ABI against dwm_moe_dispatch with a workspace:
bit-identical outputs on two calls in a row, the second smaller, both on
the three-launch path that uses the static counters; and the size limit
rejected on the host before any device work."""
import ctypes

import numpy as np
import pytest
import torch

from dw_tpu_amd import _lib


def _outs(n, E, dev):
    z = lambda k: torch.full((k,), -7, dtype=torch.int32, device=dev)  # noqa: E731
    return z(n), z(n), z(n), z(E), z(E + 1), torch.zeros(1, dtype=torch.int32, device=dev)


def _dispatch(ids, T, topk, E, dev, noalloc):
    perm, tok, rev, gs, go, flags = _outs(T * topk, E, dev)
    st = _lib.stream_handle(dev)
    args = (_lib.ptr(ids), T, topk, E, _lib.ptr(perm), _lib.ptr(tok), _lib.ptr(rev), _lib.ptr(gs), _lib.ptr(go),
            _lib.ptr(flags))
    if noalloc:
        _lib.call("dwm_moe_dispatch_noalloc", *args, st)
    else:
        b = ctypes.c_int64(0)
        _lib.call("dwm_moe_dispatch_workspace_size", T * topk, E, ctypes.byref(b))
        ws = torch.empty(b.value, dtype=torch.uint8, device=dev)
        _lib.call("dwm_moe_dispatch", *args, _lib.ptr(ws), st)
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in (perm, tok, rev, gs, go, flags)]


@pytest.mark.gpu
def test_noalloc_dispatch_matches_workspace_dispatch(dev):
    rng = np.random.default_rng(11)
    E, topk = 256, 8
    for T in (6000, 1500):  # 48000 then 12000 ids: both above the one-block path
        ids_np = rng.integers(0, E, (T, topk)).astype(np.int32)
        ids_np[0, 0] = E + 3  # an invalid id: flagged and ordered last
        ids = torch.from_numpy(ids_np).to(dev)
        want = _dispatch(ids, T, topk, E, dev, noalloc=False)
        got = _dispatch(ids, T, topk, E, dev, noalloc=True)
        for a, b in zip(got, want):
            assert np.array_equal(a, b)
        assert got[5][0] == 1
        perm = got[0]
        assert np.array_equal(perm, np.argsort(np.where(ids_np.ravel() < E, ids_np.ravel(), E), kind="stable"))


def test_noalloc_dispatch_rejects_sizes_past_its_scratch():
    _lib.load()
    T, topk, E = 1 << 18, 8, 1024  # 2048 chunks x 1025 counters > 2^20 words
    with pytest.raises(_lib.Unsupported, match="static scratch"):
        _lib.call("dwm_moe_dispatch_noalloc", ctypes.c_void_p(16), T, topk, E, ctypes.c_void_p(16),
                  ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), None, None, None)


def _static_outs(n, E, dev):
    return [torch.full((k,), -7, dtype=torch.int32, device=dev) for k in (n, n, n, E, E + 1)] + [
        torch.zeros(1, dtype=torch.int32, device=dev)]


@pytest.mark.gpu
def test_noalloc_dispatch_under_graph_capture(dev):
    """The no-alloc dispatch captured into a HIP graph and replayed with new
    ids copied in, eager work and synchronisations between the replays; every
    replay bit-identical to dwm_moe_dispatch with a workspace.  The 2048-id
    batch is captured with no earlier no-alloc call of its size class (it
    never looks the static array up); the 20,000-id batch (three launches
    on the static counters) is captured after one eager call, as the header
    asks of batches above 8192 ids."""
    rng = np.random.default_rng(5)
    for T, topk, E in ((256, 8, 32), (2500, 8, 256)):
        n = T * topk
        ids = torch.zeros((T, topk), dtype=torch.int32, device=dev)
        outs = _static_outs(n, E, dev)
        args = lambda: (_lib.ptr(ids), T, topk, E) + tuple(_lib.ptr(t) for t in outs)  # noqa: E731
        if n > 8192:
            _lib.call("dwm_moe_dispatch_noalloc", *args(), _lib.stream_handle(dev))
            torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs[5].zero_()  # flags start at zero on every replay (a fill kernel, not a memset node)
            _lib.call("dwm_moe_dispatch_noalloc", *args(), _lib.stream_handle(dev))
        torch.cuda.synchronize()
        for rep in range(4):
            ids_np = rng.integers(0, E, (T, topk)).astype(np.int32)
            if rep == 2:
                ids_np[1, 3] = E + 5  # an invalid id: flagged and ordered last
            ids.copy_(torch.from_numpy(ids_np))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got = [t.cpu().numpy().copy() for t in outs]
            want = _dispatch(ids, T, topk, E, dev, noalloc=False)
            for a, b in zip(got, want):
                assert np.array_equal(a, b), (T, E, rep)
            assert got[5][0] == (1 if rep == 2 else 0)
