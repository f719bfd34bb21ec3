"""roctx ranges around the package's operations, for `rocprofv3
--marker-trace` (the ROCm build of torch.cuda.nvtx is roctx).

Off by default: a disabled range costs one flag test.  On with the
environment variable DWTPU_ROCTX=1 or ``enable(True)``.  Every C-ABI call
through ``_lib.call`` gets a range named by its entry point (``dwm_*``);
composite operations (the expert block) add their own around those.
"""
import contextlib
import functools
import os

_on = os.environ.get("DWTPU_ROCTX", "").strip() not in ("", "0")


def enable(on: bool = True) -> None:
    """Turns the ranges on or off for this process."""
    global _on
    _on = bool(on)


def enabled() -> bool:
    return _on


@contextlib.contextmanager
def op_range(name: str):
    """A roctx range around the body when ranges are on."""
    if not _on:
        yield
        return
    import torch
    torch.cuda.nvtx.range_push(name)
    try:
        yield
    finally:
        torch.cuda.nvtx.range_pop()


def traced(name: str):
    """Decorator form of ``op_range``."""
    def wrap(fn):
        @functools.wraps(fn)
        def inner(*a, **k):
            if not _on:
                return fn(*a, **k)
            with op_range(name):
                return fn(*a, **k)
        return inner
    return wrap
