"""gmm_v2's cache of prepacked raw weights (host logic, no GPU): one prepack
per live, unmodified (rhs, rhs_scale) pair; an in-place change, another
tensor, or the flags it was prepacked with make a new one."""
import importlib

import torch

g = importlib.import_module("dw_tpu_amd.gmm_v2")  # the package attribute gmm_v2 is the function


def test_prepack_cache_hits_and_misses(monkeypatch):
    calls = []

    def fake_prepack(rhs, rhs_scale, rhs_fp4_codes=False, gate_up=False, transpose_rhs=False):
        calls.append((id(rhs), rhs_fp4_codes, gate_up, transpose_rhs))
        return object()

    monkeypatch.setattr(g, "prepack_fp4", fake_prepack)
    g.clear_prepack_cache()
    rhs = torch.zeros(2, 64, 8, dtype=torch.uint8)
    sc = torch.zeros(2, 2, 1, 16, dtype=torch.uint8)
    w1 = g._prepack_cached(rhs, sc, True, False)
    assert g._prepack_cached(rhs, sc, True, False) is w1 and len(calls) == 1
    assert g._prepack_cached(rhs, sc, True, True) is not w1 and len(calls) == 2  # gate/up layout
    assert g._prepack_cached(rhs, sc, True, False, True) is not w1 and len(calls) == 3  # transposed source
    calls.pop()
    rhs.add_(1)  # in place: the version counter moves
    w3 = g._prepack_cached(rhs, sc, True, False)
    assert w3 is not w1 and len(calls) == 3
    sc[0, 0, 0, 0] = 7  # an in-place write to the scales
    assert g._prepack_cached(rhs, sc, True, False) is not w3 and len(calls) == 4
    other = rhs.clone()
    assert g._prepack_cached(other, sc, True, False) is not w3 and len(calls) == 5
    g.clear_prepack_cache()
    g._prepack_cached(rhs, sc, True, False)
    assert len(calls) == 6


def test_prepack_cache_is_bounded(monkeypatch):
    monkeypatch.setattr(g, "prepack_fp4", lambda *a, **k: object())
    g.clear_prepack_cache()
    keep = [(torch.zeros(1, 32, 2, dtype=torch.uint8), torch.zeros(1, 1, 1, 4, dtype=torch.uint8)) for _ in range(20)]
    for r, s in keep:
        g._prepack_cached(r, s, False, False)
    assert len(g._prepack_cache) == g._PREPACK_CACHE_SIZE
    g.clear_prepack_cache()
