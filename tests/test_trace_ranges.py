"""roctx ranges (dw_tpu_amd._trace): off by default, on through enable() or
DWTPU_ROCTX; every C-ABI call through _lib.call is wrapped in a range named
by its entry point.  CPU only: torch's range calls need no GPU."""
import subprocess
import sys

import pytest
import torch

from dw_tpu_amd import _lib, _trace


def test_calls_are_wrapped_when_on(monkeypatch):
    pushed = []
    monkeypatch.setattr(torch.cuda.nvtx, "range_push", lambda n: pushed.append(("push", n)))
    monkeypatch.setattr(torch.cuda.nvtx, "range_pop", lambda: pushed.append(("pop", None)))
    _trace.enable(True)
    try:
        _lib.call("dwm_row_gather", None, 4, 16, None, 0, None, None)  # zero rows: returns OK, no launch
        with pytest.raises(ValueError):
            _lib.call("dwm_moe_combine", None, 5, 4, 8, None, None, _lib.F32, 2, 2, None, _lib.BF16, None)
    finally:
        _trace.enable(False)
    assert pushed == [("push", "dwm_row_gather"), ("pop", None), ("push", "dwm_moe_combine"), ("pop", None)]


def test_switch_and_decorator(monkeypatch):
    """Whatever DWTPU_ROCTX this process started with (a marker-trace pass
    sets it), enable(False) turns the ranges off and enable(True) on."""
    pushed = []
    monkeypatch.setattr(torch.cuda.nvtx, "range_push", lambda n: pushed.append(n))
    monkeypatch.setattr(torch.cuda.nvtx, "range_pop", lambda: None)
    was = _trace.enabled()
    monkeypatch.delenv("DWTPU_ROCTX", raising=False)
    _trace.enable(False)

    @_trace.traced("op")
    def f(x):
        return x + 1

    assert not _trace.enabled()
    assert f(1) == 2 and pushed == []
    _trace.enable(True)
    try:
        assert f(2) == 3 and pushed == ["op"]
    finally:
        _trace.enable(was)


@pytest.mark.parametrize("value,want", [(None, "False"), ("1", "True")])
def test_environment_switch_and_default(value, want):
    """Off by default in a clean environment; DWTPU_ROCTX=1 turns it on."""
    code = "from dw_tpu_amd import _trace; print(_trace.enabled())"
    import os
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "dw-tpu_amd")
    env = {k: v for k, v in os.environ.items() if k != "DWTPU_ROCTX"}
    env["PYTHONPATH"] = pkg
    if value is not None:
        env["DWTPU_ROCTX"] = value
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert out.stdout.strip() == want, out.stderr[-500:]
