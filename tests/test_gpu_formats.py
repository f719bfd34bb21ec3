"""Checkpoint weight formats on the GPU (dwm_mxfp4_requant,
dwm_fp8_block_requant): bit-exact against oracle/checkpoint.py, including
every checkpoint scale code, -0, NaN / overflow groups and both layouts, end
to end into the gmm's prepacked weights, and at full checkpoint size."""
import numpy as np
import pytest
import torch

from oracle import checkpoint as C
from oracle.numerics import to_e4m3

pytestmark = pytest.mark.gpu


def _pack_k(codes):
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)


def _unpack_n(packed):
    """[E, K, N/2] bytes -> [E, K, N] nibbles (even n in the low nibble)."""
    out = np.empty(packed.shape[:-1] + (2 * packed.shape[-1],), np.uint8)
    out[..., 0::2] = packed & 0xF
    out[..., 1::2] = packed >> 4
    return out


def _run_mxfp4(dev, codes, scales, interleave):
    from dw_tpu_amd import mxfp4_requant
    blocks = _pack_k(codes)
    q, sc, st = mxfp4_requant(torch.from_numpy(blocks).to(dev), torch.from_numpy(scales).to(dev), interleave)
    wq, wsc, lossy, nonfinite = C.mxfp4_requant(blocks, scales, interleave)
    got_q = _unpack_n(q.cpu().numpy())
    got_sc = sc.cpu().numpy()[:, :, 0, :]
    assert np.array_equal(got_q, wq), np.argwhere(got_q != wq)[:5]
    assert np.array_equal(got_sc, wsc), np.argwhere(got_sc != wsc)[:5]
    assert (st.inexact_groups, st.nonfinite_groups) == (lossy, nonfinite)
    return st


@pytest.mark.parametrize("interleave", [False, True])
@pytest.mark.parametrize("e,n,k", [(3, 256, 384), (2, 512, 512)])  # the 128x64-tile and 256x256-tile kernels
def test_mxfp4_random_bit_exact(dev, rng, interleave, e, n, k):
    codes = rng.integers(0, 16, (e, n, k), dtype=np.uint8)
    scales = rng.integers(100, 140, (e, n, k // 32)).astype(np.uint8)
    st = _run_mxfp4(dev, codes, scales, interleave)
    assert st.exact


def test_mxfp4_every_scale_code_and_block_maximum(dev, rng):
    # 256 columns x 8 groups: every checkpoint scale code 0..255 appears with
    # blocks whose maximum magnitude runs over the 8 e2m1 magnitudes.
    e, n, k = 1, 256, 256
    codes = np.zeros((e, n, k), np.uint8)
    scales = np.zeros((e, n, k // 32), np.uint8)
    for col in range(n):
        for g in range(k // 32):
            top = (col + g) % 8
            blk = rng.integers(0, top + 1, 32).astype(np.uint8) | (rng.integers(0, 2, 32).astype(np.uint8) << 3)
            blk[rng.integers(0, 32)] = top
            codes[0, col, 32 * g:32 * g + 32] = blk
            scales[0, col, g] = (col * 8 + g * 37) % 256
    st = _run_mxfp4(dev, codes, scales, False)
    assert st.nonfinite_groups > 0 and st.inexact_groups > 0  # codes 255 / 254 x 6 and subnormal scales occur


def test_mxfp4_zero_and_negative_zero_groups(dev):
    codes = np.zeros((1, 64, 128), np.uint8)
    codes[0, 1] = 8
    codes[0, 2, 5] = 9  # -0.5 among zeros
    scales = np.full((1, 64, 4), 127, np.uint8)
    st = _run_mxfp4(dev, codes, scales, False)
    assert st.exact


def test_load_mxfp4_moe_weight_matches_oracle_prepack(dev, rng):
    from dw_tpu_amd import fp4_weight_to_codes, load_mxfp4_moe_weight
    e, n, k = 2, 128, 256
    codes = rng.integers(0, 16, (e, n, k), dtype=np.uint8)
    scales = rng.integers(110, 135, (e, n, k // 32)).astype(np.uint8)
    w = load_mxfp4_moe_weight(torch.from_numpy(_pack_k(codes)).to(dev), torch.from_numpy(scales).to(dev))
    wq, wsc, _, _ = C.mxfp4_requant(_pack_k(codes), scales)
    ref = fp4_weight_to_codes(torch.from_numpy((wq[..., 0::2] | (wq[..., 1::2] << 4)).astype(np.uint8)).to(dev),
                              torch.from_numpy(wsc[:, :, None, :].copy()).to(dev))
    assert torch.equal(w.weight, ref.weight) and torch.equal(w.scale, ref.scale)
    with pytest.raises(ValueError):
        bad = scales.copy()
        bad[0, 0, 0] = 255
        load_mxfp4_moe_weight(torch.from_numpy(_pack_k(codes)).to(dev), torch.from_numpy(bad).to(dev))


def _run_fp8(dev, wc, scale, input_nk):
    from dw_tpu_amd import fp8_block_requant
    w_out, s_out, st = fp8_block_requant(torch.from_numpy(wc).to(dev), torch.from_numpy(scale).to(dev),
                                         "nk" if input_nk else "kn")
    qc, s, inexact, nonfinite = C.fp8_block_requant(wc, scale, input_nk)
    got_w = w_out.cpu().numpy()
    got_s = s_out.cpu().numpy()[:, 0, :]
    assert np.array_equal(got_w, qc), np.argwhere(got_w != qc)[:5]
    assert np.array_equal(got_s.view(np.uint32), s.view(np.uint32)) or np.array_equal(got_s, s, equal_nan=True)
    assert (st.inexact_groups, st.nonfinite_groups) == (inexact, nonfinite)
    return st


@pytest.mark.parametrize("input_nk", [True, False])
@pytest.mark.parametrize("k,n", [(512, 384), (384, 512)])
def test_fp8_block_requant_pow2_scales_exact(dev, rng, input_nk, k, n):
    wc = to_e4m3((rng.standard_normal((k, n)) * 3).astype(np.float32))
    scale = np.ldexp(np.float32(1), rng.integers(-12, 0, (k // 128, n // 128))).astype(np.float32)
    if input_nk:
        wc, scale = wc.T.copy(), scale.T.copy()
    st = _run_fp8(dev, wc, scale, input_nk)
    assert st.exact


def test_fp8_block_requant_general_scales_and_edges(dev, rng):
    k, n = 256, 256
    wc = rng.integers(0, 256, (k, n), dtype=np.uint8)          # every code, NaNs (0x7F, 0xFF) included
    scale = (rng.random((k // 128, n // 128)) * 0.02 + 1e-4).astype(np.float32)
    scale[0, 0] = np.float32(2.0 ** -140)                       # subnormal products
    st = _run_fp8(dev, wc, scale, False)
    assert st.nonfinite_groups > 0 and st.inexact_groups > 0
    wc2 = wc.copy()
    wc2[(wc2 & 0x7F) == 0x7F] = 0x80                            # no NaN: -0 instead
    _run_fp8(dev, wc2, scale, False)


def test_mxfp4_full_size_gate_up_checkpoint(dev):
    # The whole 32-expert gate/up checkpoint (N = 2 x 2048 interleaved w1/w3
    # columns, K = 7168) in one call: the first and the last expert bit-exact
    # against the oracle, the status counters over every expert.
    e, n, k = 32, 4096, 7168
    g = torch.Generator(device=dev).manual_seed(7)
    blocks = torch.randint(0, 256, (e, n, k // 2), dtype=torch.uint8, device=dev, generator=g)
    scales = torch.randint(110, 135, (e, n, k // 32), dtype=torch.uint8, device=dev, generator=g)
    planted = [(0, 5, 3), (0, 4095, 223), (13, 2048, 100), (31, 1, 0), (31, 3000, 77)]
    for ex, col, grp in planted:
        scales[ex, col, grp] = 255  # a NaN scale: the whole group is non-finite
    from dw_tpu_amd import mxfp4_requant
    q, sc, st = mxfp4_requant(blocks, scales, True)
    torch.cuda.synchronize()
    assert (st.inexact_groups, st.nonfinite_groups) == (0, len(planted))
    for ex in (0, e - 1):
        wq, wsc, lossy, nonfinite = C.mxfp4_requant(blocks[ex:ex + 1].cpu().numpy(),
                                                    scales[ex:ex + 1].cpu().numpy(), True)
        assert lossy == 0 and nonfinite == sum(p[0] == ex for p in planted)
        got_q = _unpack_n(q[ex:ex + 1].cpu().numpy())
        assert np.array_equal(got_q, wq), (ex, np.argwhere(got_q != wq)[:5])
        got_sc = sc[ex:ex + 1].cpu().numpy()[:, :, 0, :]
        assert np.array_equal(got_sc, wsc), (ex, np.argwhere(got_sc != wsc)[:5])


@pytest.mark.parametrize("input_nk", [True, False])
def test_fp8_block_requant_full_size(dev, rng, input_nk):
    # A whole DeepSeek FP8 projection (N = 4096, K = 7168) with general block
    # scales: bit-exact codes and scales, and the same inexact-block count.
    n, k = 4096, 7168
    wc = rng.integers(0, 256, (n, k), dtype=np.uint8)
    wc[(wc & 0x7F) == 0x7F] = 0  # no NaN codes: every block finite
    scale = (rng.random((n // 128, k // 128)) * 0.02 + 1e-4).astype(np.float32)
    if not input_nk:
        wc, scale = wc.T.copy(), scale.T.copy()
    st = _run_fp8(dev, wc, scale, input_nk)
    assert st.nonfinite_groups == 0 and st.inexact_groups > 0
