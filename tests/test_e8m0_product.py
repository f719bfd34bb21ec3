"""The product's e8m0_encode / e8m0_decode (dw_tpu_amd.e8m0_scale) against
the oracle's restatement of e8m0_scale.py:28-40: every one of the 256 codes,
and the lossless predicate on crafted scales.  The CPU case runs the torch
bit operations on host tensors; the GPU case on device tensors."""
import numpy as np
import pytest
import torch

from dw_tpu_amd import e8m0_decode, e8m0_encode
from oracle import fp4


def _scales():
    """Every power of two with an f32 exponent field 0..255 (0 -> +0.0,
    255 -> inf), and scales each failing the lossless rule one way."""
    pow2 = (np.arange(256, dtype=np.uint32) << 23).view(np.float32)
    bad = np.array([-1.0, 3.0, 0.75, np.float32(2.0) * (1 + 2 ** -23), -0.0, np.inf, np.nan,
                    np.float32(1e-45), np.float32(2 ** -127)], np.float32)
    return pow2, bad


def _check(device):
    pow2, bad = _scales()
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).to(device)
    got = e8m0_decode(codes).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), fp4.e8m0_decode(np.arange(256, dtype=np.uint8)).view(np.uint32))
    enc, ok = e8m0_encode(torch.from_numpy(pow2[:255]).to(device))
    want, want_ok = fp4.e8m0_encode(pow2[:255])
    assert np.array_equal(enc.cpu().numpy(), want) and bool(ok) is want_ok is True
    # decode(encode(s)) == s bit for bit for every lossless scale
    assert np.array_equal(e8m0_decode(enc).cpu().numpy().view(np.uint32), pow2[:255].view(np.uint32))
    for v in list(bad) + [pow2[255]]:
        s = np.array([1.0, v, 0.5], np.float32)
        enc, ok = e8m0_encode(torch.from_numpy(s).to(device))
        want, want_ok = fp4.e8m0_encode(s)
        assert np.array_equal(enc.cpu().numpy(), want), v
        assert bool(ok) is want_ok is False, v
    # bf16 input widens exactly
    enc, ok = e8m0_encode(torch.tensor([0.25, 8.0, 0.0], dtype=torch.bfloat16, device=device))
    assert enc.cpu().tolist() == [125, 130, 0] and bool(ok)


def test_e8m0_product_on_host():
    _check("cpu")


@pytest.mark.gpu
def test_e8m0_product_on_device(dev):
    _check(dev)
