"""Validated, immutable per-process dense FP8 tile overrides (no device work).

Mirrors kernels/tpu_inference/kernels/experimental/dense_fp8_tiles.py:11-58:
a JSON table named by the DSV4_DENSE_FP8_TILES environment variable, read
once and validated fail-closed (ValueError on any malformed entry).  Entries
select per-(M, K, N) tiles or "baseline" (keep the caller's path).  The
device string is this build's target.
"""
import functools
import json
import os

DEVICE = "AMD Instinct MI355X"
ROWS = frozenset(range(1, 34)) | {64, 65, 128, 129, 256, 257, 512, 513, 1024, 4096}
MODES = ("native", "megablox")


def validate_table(data):
    if not isinstance(data, dict) or type(data.get("version")) is not int or data["version"] != 1:
        raise ValueError("dense FP8 tile table requires version=1")
    if data.get("device") != DEVICE:
        raise ValueError(f"dense FP8 tile table requires device {DEVICE!r}")
    if not isinstance(data.get("entries"), list):
        raise ValueError("dense FP8 tile table requires entries list")
    table = {}
    for row in data["entries"]:
        if not isinstance(row, dict):
            raise ValueError("tile entry must be an object")
        dims = tuple(row.get(key) for key in ("m", "k", "n"))
        if any(type(x) is not int for x in dims):
            raise ValueError("tile dimensions must be integers")
        m, k, n = dims
        if m not in ROWS or k % 128 or n % 16 or k <= 0 or n <= 0 or dims in table:
            raise ValueError(f"unsupported or duplicate dense tile: {dims}")
        mode = row.get("mode")
        if mode == "baseline":
            table[dims] = None
            continue
        if mode not in MODES:
            raise ValueError("only native/megablox/baseline tiles are supported")
        tile = tuple(row.get(key) for key in ("tm", "tk", "tn"))
        if any(type(x) is not int or x <= 0 for x in tile):
            raise ValueError("tile sizes must be positive integers")
        tm, tk, tn = tile
        if m % tm or k % tk or n % tn or tk % 128 or tn % 16:
            raise ValueError("tile must divide dimensions; K tiles align to 128, N tiles to 16")
        if tm != m and tm % 16:
            raise ValueError("partial M tiles must align to 16")
        table[dims] = (mode, tm, tk, tn)
    return table


@functools.lru_cache(maxsize=None)
def _load(path):
    # Read once: changing the file later cannot change the process's choices.
    with open(path, encoding="utf-8") as handle:
        return validate_table(json.load(handle))


def overrides():
    """Set DSV4_DENSE_FP8_TILES before startup; absent means unchanged defaults."""
    path = os.environ.get("DSV4_DENSE_FP8_TILES", "")
    return _load(path) if path else {}
