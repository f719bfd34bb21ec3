"""Dense FP8 tile table validation and try_dense_fp8's fail-closed checks
(dense_fp8_tiles.py:11-58, dense_fp8.py:140-163).  CPU only."""
import json

import pytest
import torch

from dw_tpu_amd import dense_fp8, dense_fp8_tiles as tiles


def _table(entries, **kw):
    d = {"version": 1, "device": tiles.DEVICE, "entries": entries}
    d.update(kw)
    return d


def test_valid_table_and_baseline_entry():
    t = tiles.validate_table(_table([
        {"m": 16, "k": 7168, "n": 4096, "mode": "native", "tm": 16, "tk": 1024, "tn": 512},
        {"m": 128, "k": 7168, "n": 4096, "mode": "baseline"},
    ]))
    assert t[(16, 7168, 4096)] == ("native", 16, 1024, 512)
    assert t[(128, 7168, 4096)] is None


@pytest.mark.parametrize("bad", [
    {"version": 2, "device": tiles.DEVICE, "entries": []},
    {"version": 1, "device": "TPU v6 lite", "entries": []},
    {"version": 1, "device": tiles.DEVICE, "entries": {}},
    _table(["x"]),
    _table([{"m": 16, "k": 7168, "n": "4096", "mode": "native", "tm": 16, "tk": 1024, "tn": 512}]),
    _table([{"m": 16, "k": 7000, "n": 4096, "mode": "native", "tm": 16, "tk": 1000, "tn": 512}]),
    _table([{"m": 16, "k": 7168, "n": 4096, "mode": "pre", "tm": 16, "tk": 1024, "tn": 512}]),
    _table([{"m": 16, "k": 7168, "n": 4096, "mode": "native", "tm": 16, "tk": 1000, "tn": 512}]),
    _table([{"m": 16, "k": 7168, "n": 4096, "mode": "native", "tm": 0, "tk": 1024, "tn": 512}]),
    _table([{"m": 128, "k": 7168, "n": 4096, "mode": "native", "tm": 8, "tk": 1024, "tn": 512}]),
    _table([{"m": 16, "k": 7168, "n": 4096, "mode": "baseline"}, {"m": 16, "k": 7168, "n": 4096, "mode": "baseline"}]),
])
def test_invalid_tables_raise(bad):
    with pytest.raises(ValueError):
        tiles.validate_table(bad)


def test_overrides_from_env(tmp_path, monkeypatch):
    p = tmp_path / "tiles.json"
    p.write_text(json.dumps(_table([{"m": 1, "k": 1024, "n": 512, "mode": "baseline"}])))
    monkeypatch.setenv("DSV4_DENSE_FP8_TILES", str(p))
    tiles._load.cache_clear()
    assert dense_fp8.select_tile(1, 1024, 512) is None  # baseline keeps the caller's path
    assert dense_fp8.select_tile(2, 1024, 512) == ("native", 16, 128, 64)
    monkeypatch.delenv("DSV4_DENSE_FP8_TILES")
    tiles._load.cache_clear()


def test_select_tile_rejects_unaligned():
    assert dense_fp8.select_tile(4, 1000, 512) is None
    assert dense_fp8.select_tile(4, 1024, 500) is None
    assert dense_fp8.select_tile(4096, 7168, 4096) == ("native", 128, 128, 128)


def test_try_dense_fp8_fail_closed_on_host():
    x = torch.zeros((4, 256), dtype=torch.bfloat16)
    w = torch.zeros((256, 128), dtype=torch.float8_e4m3fn)
    s = torch.ones((2, 1, 128), dtype=torch.float32)
    assert dense_fp8.try_dense_fp8(x.float(), w, s) is None            # x not bf16
    assert dense_fp8.try_dense_fp8(x, w.view(torch.uint8), s) is None  # w not e4m3
    assert dense_fp8.try_dense_fp8(x, w, s.double()) is None           # scale not f32
    assert dense_fp8.try_dense_fp8(x, w, torch.ones((2, 128))) is None # scale shape
    assert dense_fp8.try_dense_fp8(x, w, s) is None                    # host tensors: no kernel
