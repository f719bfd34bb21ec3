"""Dense FP8 launch selection: tiles as the reference names them, plans as
this library launches them, and the per-process override file.

The reference picks a dense tile as ``(mode, tm, tk, tn)``
(kernels/tpu_inference/kernels/experimental/dense_fp8.py:80-138) and lets a
JSON file named by ``DSV4_DENSE_FP8_TILES`` pin it per (M, K, N)
(dense_fp8_tiles.py:11-58).  Both the tuple and the file's schema are kept,
so a caller's table and its unpacking of ``select_tile`` work unchanged.
What they mean here is a launch of this library's kernels
(``struct dwm_dense_plan``):

  mode "native"    tm = tn = 16: the skinny kernel (M <= 16; its 16 waves
                   split K inside one block, so tk = K);
                   tm = 128 or 256, tn = 128: the MFMA tile kernel;
  mode "megablox"  the general tiled kernel, tm x tn = 16 x 64, 64 x 128 or
                   128 x 128 (any N % 16 == 0);
  tk               the K depth one block covers: K / tk blocks share an
                   output tile and their f32 partials are added in order;
  "stages"         optional ring depth (LDS stages of the MFMA kernel);
  mode "baseline"  no launch: ``try_dense_fp8`` returns None.

Table entries are checked by the library's own plan rules when the file is
read (``dwm_dense_fp8_plan_check``, host code only), so a table can name
only launches that exist.  A malformed file raises ValueError.
"""
import ctypes
import functools
import json
import os

from . import _lib

ENV_VAR = "DSV4_DENSE_FP8_TILES"
DEVICE = "AMD Instinct MI355X"
FORMAT_VERSION = 1

_KERNEL_OF_MODE = {"native": None, "megablox": _lib.DENSE_TILED}


class DenseTile(tuple):
    """``(mode, tm, tk, tn)`` -- the reference's ``select_tile`` value --
    with the ring depth as ``.stages`` (0: the library's usual depth for the
    tile)."""

    def __new__(cls, mode, tm, tk, tn, stages=0):
        self = super().__new__(cls, (mode, tm, tk, tn))
        self.stages = stages
        return self

    mode = property(lambda self: self[0])
    tm = property(lambda self: self[1])
    tk = property(lambda self: self[2])
    tn = property(lambda self: self[3])

    def __repr__(self):
        return f"DenseTile{tuple(self)!r}(stages={self.stages})"


def _usual_stages(kernel, tile_m, w8a8):
    if kernel == _lib.DENSE_MFMA:
        if w8a8:
            return 4 if tile_m == 128 else 3
        return 3 if tile_m == 128 else 2
    return 2


def plan_to_tile(plan, k):
    """The ``DenseTile`` describing a ``_lib.DensePlan`` at depth K."""
    kb = k // 128
    if plan.kernel == _lib.DENSE_SKINNY:
        return DenseTile("native", plan.tile_m, k, plan.tile_n, plan.stages)
    tk = 128 * -(-kb // plan.ksplit)
    mode = "megablox" if plan.kernel == _lib.DENSE_TILED else "native"
    return DenseTile(mode, plan.tile_m, tk, plan.tile_n, plan.stages)


def tile_to_plan(tile, m, k, n, w8a8=False):
    """The ``_lib.DensePlan`` a tile names at M x K x N; ValueError if the
    tile names no launch of this library (checked by the library itself)."""
    mode, tm, tk, tn = tile
    stages = getattr(tile, "stages", 0)
    if mode not in _KERNEL_OF_MODE:
        raise ValueError(f"dense tile mode {mode!r} is not one of {sorted(_KERNEL_OF_MODE)}")
    if any(type(v) is not int for v in (tm, tk, tn, stages)):
        raise ValueError(f"dense tile sizes must be integers: {tile!r}")
    if tk <= 0 or tk % 128:
        raise ValueError(f"tk={tk} must be a positive multiple of 128 (the scale block)")
    kernel = _KERNEL_OF_MODE[mode]
    if kernel is None:
        kernel = _lib.DENSE_SKINNY if (tm, tn) == (16, 16) else _lib.DENSE_MFMA
    if kernel == _lib.DENSE_SKINNY:
        if tk != k:
            raise ValueError(f"the skinny kernel covers all of K in one block: tk must be {k}")
        ksplit = 16
    else:
        ksplit = -(-(k // 128) // (tk // 128))
    plan = _lib.DensePlan(kernel, tm, tn, ksplit, stages or _usual_stages(kernel, tm, w8a8))
    if kernel != _lib.DENSE_SKINNY and plan_to_tile(plan, k)[2] != tk:
        raise ValueError(f"tk={tk} does not split K={k} into whole runs of its own depth")
    try:
        _lib.call("dwm_dense_fp8_plan_check", m, k, n, int(bool(w8a8)), ctypes.byref(plan))
    except _lib.Unsupported as exc:
        raise ValueError(str(exc)) from None
    return plan


def default_plan(m, k, n, w8a8=False):
    """The plan the library launches when none is given."""
    plan = _lib.DensePlan()
    _lib.call("dwm_dense_fp8_plan", m, k, n, int(bool(w8a8)), ctypes.byref(plan))
    return plan


def parse_table(data):
    """JSON document -> {(m, k, n): DenseTile or None}."""
    if not isinstance(data, dict):
        raise ValueError("dense tile file: the document must be a JSON object")
    if data.get("version") != FORMAT_VERSION or type(data.get("version")) is not int:
        raise ValueError(f"dense tile file: version must be {FORMAT_VERSION}")
    if data.get("device") != DEVICE:
        raise ValueError(f"dense tile file: written for {data.get('device')!r}, this library runs on {DEVICE!r}")
    rows = data.get("entries")
    if not isinstance(rows, list):
        raise ValueError("dense tile file: 'entries' must be a list")
    out = {}
    for i, row in enumerate(rows):
        if not isinstance(row, dict):
            raise ValueError(f"dense tile file: entry {i} is not an object")
        key = tuple(row.get(f) for f in ("m", "k", "n"))
        if any(type(v) is not int or v <= 0 for v in key):
            raise ValueError(f"dense tile file: entry {i} needs positive integer m, k, n")
        if key in out:
            raise ValueError(f"dense tile file: (m, k, n) = {key} appears twice")
        if row.get("mode") == "baseline":
            out[key] = None
            continue
        tile = DenseTile(row.get("mode"), row.get("tm"), row.get("tk"), row.get("tn"), row.get("stages", 0))
        try:
            plan = tile_to_plan(tile, *key)
        except ValueError as exc:
            raise ValueError(f"dense tile file: entry {i} {key}: {exc}") from None
        out[key] = DenseTile(*tile, plan.stages)
    return out


validate_table = parse_table  # the reference's name for the same check


@functools.lru_cache(maxsize=None)
def _read(path):
    with open(path, encoding="utf-8") as fh:
        return parse_table(json.load(fh))


def overrides():
    """{(m, k, n): DenseTile or None} from the file named by
    DSV4_DENSE_FP8_TILES ({} when unset).  The file is read once per path."""
    path = os.environ.get(ENV_VAR)
    return _read(path) if path else {}
