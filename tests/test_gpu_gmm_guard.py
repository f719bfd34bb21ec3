"""The grouped matmul's guard against device group sizes that do not fit M.

group_sizes lives on the device and the host cannot check it, so the tile
list skips every tile whose rows start at or past M and clips the tile that
straddles M (find_tile in csrc/gmm_tiles.h).  Here the sizes sum to
M + 300.  lhs and out are allocated with padding rows past M (more than the
excess), so even a missing guard would read and write inside the
allocations; the test checks that the padding rows of out are untouched and
that rows [0, M) equal, bit for bit, a run whose sizes are cut to fit M
(every row's result depends on its own lhs row and expert only), for the
bf16 and the MX kernels."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import bf16_tensor
from dw_tpu_amd import _lib
from oracle.numerics import bf16_bits

pytestmark = pytest.mark.gpu

SENTINEL = 0x1234  # bf16 bits no result row holds here


def _call_gmm(mode, lhs, mx, M, K, N, pw, gs, E, out):
    P = ctypes.c_void_p
    st = _lib.stream_handle(lhs.device)
    tail = (P(pw.weight.data_ptr()), P(pw.scale.data_ptr()), P(gs.data_ptr()), E, None, E, N, P(out.data_ptr()),
            _lib.BF16, 0, _lib.ACT_NONE, st)
    if mode == "bf16":
        _lib.call("dwm_gmm_fp4", P(lhs.data_ptr()), M, K, *tail)
    else:
        # without row_idx the MX lhs is the first M rows of the (padded) codes
        _lib.call("dwm_gmm_fp4_mx", P(mx.codes.data_ptr()), P(mx.scales.data_ptr()), M, None, M, K, *tail)
    torch.cuda.synchronize()


@pytest.mark.parametrize("mode", ["bf16", "mx"])
@pytest.mark.parametrize("sizes", [(100, 0, 250, 200, 250),    # the fourth group straddles M, the last lies past it
                                   (600, 200, 0, 0, 0),        # the first group alone runs past M
                                   (0, 0, 500, 300, 0)])       # the second group starts exactly at M
def test_group_sizes_past_m_stay_inside_m(dev, rng, mode, sizes):
    from dw_tpu_amd import fp4_weight_to_codes, mx_quantize
    E, K, N, M = 5, 512, 512, 500
    assert sum(sizes) == M + 300
    pad = 400  # > the 300 excess rows, and more than one 96-row tile
    lhs_bits = bf16_bits(rng.standard_normal((M + pad, K)).astype(np.float32))
    lhs = bf16_tensor(lhs_bits, dev)
    mx = mx_quantize(lhs) if mode == "mx" else None
    rhs = torch.from_numpy(rng.integers(0, 256, (E, K, N // 2), dtype=np.uint8)).to(dev)
    sc = torch.from_numpy(rng.integers(123, 130, (E, K // 32, 1, N), dtype=np.uint8)).to(dev)
    pw = fp4_weight_to_codes(rhs, sc)
    out = torch.full((M + pad, N), SENTINEL, dtype=torch.int16, device=dev).view(torch.bfloat16)
    gs = torch.tensor(sizes, dtype=torch.int32, device=dev)
    _call_gmm(mode, lhs, mx, M, K, N, pw, gs, E, out)
    got = out.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.all(got[M:] == SENTINEL), "rows past M were written"
    # the same rows with the sizes cut to fit M
    fit = np.minimum(np.asarray(sizes), np.maximum(0, M - np.concatenate([[0], np.cumsum(sizes)[:-1]])))
    assert fit.sum() == M
    ref = torch.full((M + pad, N), SENTINEL, dtype=torch.int16, device=dev).view(torch.bfloat16)
    _call_gmm(mode, lhs, mx, M, K, N, pw, torch.tensor(fit, dtype=torch.int32, device=dev), E, ref)
    want = ref.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got[:M], want[:M])
