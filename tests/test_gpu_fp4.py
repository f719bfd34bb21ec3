"""FP4 decode, e2m1 -> code re-encoding and the prepack on the GPU: bit-exact
against the oracle over every nibble, byte and scale code."""
import numpy as np
import pytest
import torch

from conftest import bf16_bits
from oracle import fp4
from oracle.numerics import bf16_bits as to_bf16_bits

pytestmark = pytest.mark.gpu


def _all_bytes():
    return np.arange(256, dtype=np.uint8)


def test_e2m1_to_codes_all_bytes(dev):
    from dw_tpu_amd import e2m1_to_codes
    b = np.tile(_all_bytes(), 37)  # odd multiple of 256 exercises the tail
    got = e2m1_to_codes(torch.from_numpy(b).to(dev)).cpu().numpy()
    want = fp4.pack_nibbles(fp4.e2m1_to_codes(fp4.unpack_nibbles(b[None]))[0][None])[0]
    assert np.array_equal(got, want)


def test_decode_codes_all_bytes_bit_exact(dev):
    from dw_tpu_amd import decode_codes
    b = _all_bytes()
    got = bf16_bits(decode_codes(torch.from_numpy(b).to(dev)))
    want = to_bf16_bits(fp4.decode_codes(fp4.unpack_nibbles(b)))
    assert np.array_equal(got, want)  # includes code 8 (q = -8 -> -8.0) and +0 for -0


@pytest.mark.parametrize("fmt", ["e2m1", "codes"])
def test_decode_with_every_scale_code(dev, fmt):
    """bf16(decode(q)) * bf16(2^(c-127)) for every byte and every e8m0 code
    0..254 (code 0 = +0.0 keeps the sign of the value)."""
    from dw_tpu_amd import _lib
    from dw_tpu_amd.gmm_v2 import decode_fp4
    nib = np.tile(np.arange(16, dtype=np.uint8), 2)            # one 32-block
    if fmt == "codes":
        nib = fp4.e2m1_to_codes(nib)
    blocks = np.tile(nib, 255)                                  # 255 blocks
    packed = fp4.pack_nibbles(blocks)
    scales = np.arange(255, dtype=np.uint8)
    got = bf16_bits(decode_fp4(torch.from_numpy(packed).to(dev),
                               _lib.FP4_E2M1 if fmt == "e2m1" else _lib.FP4_CODES,
                               torch.from_numpy(scales).to(dev)))
    codes = blocks if fmt == "codes" else fp4.e2m1_to_codes(blocks)
    w = fp4.dequant_fp4_block(codes.reshape(255 * 32, 1), fp4.e8m0_decode(scales).reshape(255, 1, 1))
    want = to_bf16_bits(w.reshape(-1))
    assert np.array_equal(got, want)


def test_decode_flags_code_255(dev):
    from dw_tpu_amd import _lib
    from dw_tpu_amd.gmm_v2 import decode_fp4
    packed = torch.zeros(16, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError, match="255"):
        decode_fp4(packed, _lib.FP4_E2M1, torch.tensor([255], dtype=torch.uint8, device=dev))


def test_prepack_layout_matches_definition(dev, rng):
    """Every prepacked byte equals the documented layout of the reference
    [E, K, N/2] weight, and every scale byte its [E, K/32, N] code; columns
    past N (padding to 64) hold zero codes and scale code 127."""
    from dw_tpu_amd import prepack_fp4
    E, K, N = 2, 640, 80  # K/64 = 10 steps, N = 64 + 16: the second group is 3/4 padding
    G, T, KB = 2, K // 64, K // 128
    rhs = rng.integers(0, 256, (E, K, N // 2), dtype=np.uint8)
    sc = rng.integers(1, 255, (E, K // 32, 1, N), dtype=np.uint8)
    w = prepack_fp4(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev))
    wp = w.weight.cpu().numpy().reshape(E, G, T, 2, 64, 16)
    sp = w.scale.cpu().numpy().reshape(E, G, KB, 64, 4)
    nib = fp4.unpack_nibbles(rhs)  # [E, K, N]
    nib = np.where(nib == 8, 0, nib)  # -0 -> +0
    for e in range(E):
        for g in range(G):
            for t in range(T):
                for j in range(2):
                    for lane in range(64):
                        c, h = lane % 32, lane // 32
                        n = 64 * g + 32 * j + c
                        ks = 64 * t + 32 * h + np.arange(32)
                        if n < N:
                            want = fp4.pack_nibbles(nib[e, ks, n][None])[0]
                            code = sc[e, (64 * t + 32 * h) // 32, 0, n]
                        else:
                            want = np.zeros(16, np.uint8)
                            code = 127
                        assert np.array_equal(wp[e, g, t, j, lane], want)
                        assert sp[e, g, t // 2, lane, 2 * (t % 2) + j] == code


def test_prepack_rejects_bad_scales(dev):
    from dw_tpu_amd import prepack_fp4
    rhs = torch.zeros((1, 128, 16), dtype=torch.uint8, device=dev)
    bad = torch.full((1, 4, 1, 32), 3.0, dtype=torch.float32, device=dev)
    with pytest.raises(ValueError, match="power of two"):
        prepack_fp4(rhs, bad)
    ok = torch.full((1, 4, 1, 32), 0.25, dtype=torch.bfloat16, device=dev)
    prepack_fp4(rhs, ok)
    codes = torch.full((1, 128, 16), 0x88, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError, match="code 8"):
        prepack_fp4(codes, torch.full((1, 4, 1, 32), 127, dtype=torch.uint8, device=dev), rhs_fp4_codes=True)
