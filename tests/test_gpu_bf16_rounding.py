"""The library's f32 -> bf16 conversion (every bf16 output of the grouped
matmul epilogues, combine, dense reduce and router weights) is gfx950's
packed v_cvt_pk_bf16_f32.  dwtpu_bf16_check (built with the library from
dw-tpu_amd/csrc/bf16_check.hip) converts all 2^32 f32 bit patterns, in both
halves of the packed result, through the library's own helper and compares
each against round to nearest even with the quiet-NaN rule written out in
integer arithmetic, the rule of the oracle's bf16_bits (oracle/numerics.py)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "dw-tpu_amd", "dw_tpu_amd", "dwtpu_bf16_check")


@pytest.mark.gpu
def test_bf16_conversion_is_round_to_nearest_even_on_every_input(dev):
    assert os.path.isfile(CHECK), "dwtpu_bf16_check is not built (make -C dw-tpu_amd/csrc)"
    r = subprocess.run([CHECK], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches: 0" in r.stdout
