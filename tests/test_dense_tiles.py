"""Dense FP8 launch selection on the host: the override file's checks, the
mapping between the reference's (mode, tm, tk, tn) tiles and the library's
launch plans, and try_dense_fp8's fail-closed checks
(kernels/tpu_inference/kernels/experimental/dense_fp8.py:80-163,
dense_fp8_tiles.py:11-58).  CPU only: plans are host logic of the library."""
import json

import pytest
import torch

from dw_tpu_amd import _lib, dense_fp8
from dw_tpu_amd import dense_fp8_tiles as tiles


def _doc(entries, **kw):
    d = {"version": 1, "device": tiles.DEVICE, "entries": entries}
    d.update(kw)
    return d


def _entry(m, k, n, mode="native", tm=128, tk=None, tn=128, **kw):
    e = {"m": m, "k": k, "n": n, "mode": mode, "tm": tm, "tk": k if tk is None else tk, "tn": tn}
    e.update(kw)
    return e


def test_table_entries_become_launches():
    t = tiles.parse_table(_doc([
        _entry(128, 7168, 4096, tm=256, tk=7168, stages=3),
        _entry(64, 7168, 4096, mode="megablox", tm=64, tk=1792),
        _entry(4, 7168, 4096, tm=16, tn=16),
        {"m": 1024, "k": 7168, "n": 4096, "mode": "baseline"},
    ]))
    assert t[(128, 7168, 4096)] == ("native", 256, 7168, 128) and t[(128, 7168, 4096)].stages == 3
    assert t[(64, 7168, 4096)] == ("megablox", 64, 1792, 128) and t[(64, 7168, 4096)].stages == 2
    assert t[(4, 7168, 4096)] == ("native", 16, 7168, 16)
    assert t[(1024, 7168, 4096)] is None
    p = tiles.tile_to_plan(t[(64, 7168, 4096)], 64, 7168, 4096)
    assert p.astuple() == (_lib.DENSE_TILED, 64, 128, 4, 2)


@pytest.mark.parametrize("doc", [
    [],                                                              # not an object
    {"version": 2, "device": tiles.DEVICE, "entries": []},            # version
    {"version": True, "device": tiles.DEVICE, "entries": []},         # bool is not a version
    {"version": 1, "device": "TPU v6 lite", "entries": []},           # device
    {"version": 1, "device": tiles.DEVICE, "entries": {}},            # entries not a list
    _doc(["x"]),                                                     # entry not an object
    _doc([_entry(16, 7168, "4096")]),                                # non-integer dimension
    _doc([_entry(0, 7168, 4096)]),                                   # non-positive dimension
    _doc([_entry(128, 7168, 4096, mode="pre")]),                     # mode without a kernel here
    _doc([_entry(128, 7168, 4096, tk=1000)]),                        # tk off the 128 grid
    _doc([_entry(128, 7168, 4096, tk=1920)]),                        # 4 runs of 15 K blocks are really 14
    _doc([_entry(128, 7168, 4096, tm=8)]),                           # no such MFMA tile
    _doc([_entry(128, 7168, 4096, tm=0)]),                           # no such tile
    _doc([_entry(128, 7168, 4096, tm=256, stages=4)]),               # W8A16 256-row ring of 4 exceeds LDS
    _doc([_entry(128, 7168, 4000)]),                                 # MFMA needs N % 128 == 0
    _doc([_entry(32, 7168, 4096, tm=16, tn=16)]),                    # skinny kernel is for M <= 16
    _doc([_entry(4, 7168, 4096, tm=16, tn=16, tk=896)]),             # skinny kernel covers all of K
    _doc([_entry(64, 7168, 4096, mode="megablox", tm=32, tn=128)]),  # no such tiled shape
    _doc([{"m": 16, "k": 7168, "n": 4096, "mode": "baseline"}] * 2),  # duplicate
])
def test_malformed_tables_raise(doc):
    with pytest.raises(ValueError):
        tiles.parse_table(doc)


def test_overrides_read_from_env(tmp_path, monkeypatch):
    p = tmp_path / "tiles.json"
    p.write_text(json.dumps(_doc([{"m": 1, "k": 1024, "n": 512, "mode": "baseline"},
                                  _entry(300, 1024, 512, tm=256, tk=512, stages=3)])))
    monkeypatch.setenv(tiles.ENV_VAR, str(p))
    tiles._read.cache_clear()
    try:
        assert dense_fp8.select_tile(1, 1024, 512) is None  # baseline keeps the caller's path
        assert dense_fp8.select_tile(2, 1024, 512) == ("native", 16, 1024, 16)
        assert dense_fp8.select_tile(300, 1024, 512) == ("native", 256, 512, 128)
    finally:
        monkeypatch.delenv(tiles.ENV_VAR)
        tiles._read.cache_clear()


@pytest.mark.parametrize("m,k,n,want,stages", [
    (1, 7168, 4096, ("native", 16, 7168, 16), 2),        # skinny
    (16, 7168, 4096, ("native", 16, 7168, 16), 2),
    (128, 7168, 4096, ("native", 128, 896, 128), 3),     # 32 tiles x 8 K runs
    (1024, 7168, 4096, ("native", 128, 7168, 128), 3),   # 256 tiles: no split; one round: 3-stage ring
    (4096, 7168, 4096, ("native", 256, 7168, 128), 2),   # 256-row tiles fill the grid alone
    (64, 7168, 4000, ("megablox", 64, 512, 128), 2),     # N % 128 != 0: the tiled kernel, 14 K runs
])
def test_select_tile_is_the_library_plan(m, k, n, want, stages):
    t = dense_fp8.select_tile(m, k, n)
    assert t == want and t.stages == stages
    plan = tiles.default_plan(m, k, n)
    assert tiles.tile_to_plan(t, m, k, n).astuple() == plan.astuple()


@pytest.mark.parametrize("m", [1, 16, 17, 64, 128, 255, 256, 1024, 4096])
def test_w8a8_plans_round_trip(m):
    plan = tiles.default_plan(m, 7168, 4096, w8a8=True)
    t = tiles.plan_to_tile(plan, 7168)
    assert tiles.tile_to_plan(t, m, 7168, 4096, w8a8=True).astuple() == plan.astuple()
    if m >= 256:
        assert (plan.tile_m, plan.stages) == (256, 3)


def test_select_tile_rejects_unaligned():
    assert dense_fp8.select_tile(4, 1000, 512) is None
    assert dense_fp8.select_tile(4, 1024, 500) is None
    assert dense_fp8.select_tile(0, 1024, 512) is None


def test_plan_workspace_matches_ksplit():
    t = dense_fp8.select_tile(128, 7168, 4096)
    plan = tiles.tile_to_plan(t, 128, 7168, 4096)
    import ctypes
    b = ctypes.c_int64(0)
    _lib.call("dwm_dense_fp8_plan_workspace_size", 128, 7168, 4096, ctypes.byref(plan), ctypes.byref(b))
    assert b.value == 8 * 128 * 4096 * 4


def test_try_dense_fp8_fail_closed_on_host():
    x = torch.zeros((4, 256), dtype=torch.bfloat16)
    w = torch.zeros((256, 128), dtype=torch.float8_e4m3fn)
    s = torch.ones((2, 1, 128), dtype=torch.float32)
    assert dense_fp8.try_dense_fp8(x.float(), w, s) is None            # x not bf16
    assert dense_fp8.try_dense_fp8(x, w.view(torch.uint8), s) is None  # w not e4m3
    assert dense_fp8.try_dense_fp8(x, w, s.double()) is None           # scale not f32
    assert dense_fp8.try_dense_fp8(x, w, torch.ones((2, 128))) is None # scale shape
    assert dense_fp8.try_dense_fp8(x, w, s) is None                    # host tensors: no kernel
