"""Seeded random shapes for the grouped matmul on the GPU, against the
float64 oracle under the stated bounds (bf16 path: oracle.gmm.error_bound
terms; MX path: plus the in-block alignment term; fused activations:
oracle.moe_block.act_bound).

The cases vary what the device tile list does: group counts and sizes with
empty groups (16-row block classes 1 .. 6, full and partial row tiles),
column counts that leave part-filled 512- and 256-column tiles, expert-
parallel windows, and totals near the CU count, where the narrow split cuts
some classes into 256-column tiles and not others.  MX cases below K = 4096
with 97 .. 192 rows per group on average take the stacked row halves, and
cases with 8192 .. 10240 columns fill the CUs (the kernel without narrow
tiles)."""
import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from oracle import fp4, gmm, quant
from oracle import moe_block as omb
from oracle.numerics import bf16_bits as to_bf16_bits
from oracle.numerics import bf16_to_f32

pytestmark = pytest.mark.gpu


def _case(seed):
    r = np.random.default_rng(1000 + seed)
    mx = bool(seed % 3 == 2)
    act = [None, None, "silu_and_mul_with_clamp", "gelu"][seed % 4]
    K = int(r.choice([128, 256, 4096 if mx and seed % 2 else 256]))
    if seed % 5 == 4:
        # near the CU count: 24 .. 30 local groups of 60 .. 96 rows, 8 column tiles
        E = int(r.integers(24, 31))
        sizes = r.integers(60, 97, E)
        N = 4096
    elif seed % 6 == 1 and not mx:
        # enough tiles to fill the CUs: the kernel without narrow tiles
        E = int(r.integers(10, 19))
        sizes = r.integers(60, 260, E)
        N = int(64 * r.integers(128, 161))
        K = 128
    else:
        E = int(r.integers(1, 20))
        sizes = r.integers(0, 260, E)
        sizes[r.random(E) < 0.25] = 0
        N = int(64 * r.integers(1, 20))
    go, e_local = 0, E
    if seed % 7 == 3 and E > 2:
        go = int(r.integers(0, E // 2))
        e_local = int(r.integers(1, E - go + 1))
    return dict(mx=mx, act=act, K=K, N=N, sizes=[int(x) for x in sizes], go=go, e_local=e_local,
                bias=bool(seed % 2), r=r)


@pytest.mark.parametrize("seed", range(30))
def test_gmm_random_shapes(dev, seed):
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2
    c = _case(seed)
    r, K, N, sizes, go, e_local, act, mx = c["r"], c["K"], c["N"], c["sizes"], c["go"], c["e_local"], c["act"], c["mx"]
    M = sum(sizes)
    if M == 0:
        sizes[0] = 5
        M = 5
    lhs_bits = to_bf16_bits(r.standard_normal((M, K)).astype(np.float32))
    rhs = r.integers(0, 256, (e_local, K, N // 2), dtype=np.uint8)
    sc = r.integers(122, 128, (e_local, K // 32, 1, N), dtype=np.uint8)
    bias = (r.standard_normal((e_local, N)) * 4).astype(np.float32) if c["bias"] else None
    gs = np.array(sizes, np.int32)
    pw = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev), gate_up=act is not None)
    window = go > 0 or e_local < len(sizes)
    out = gmm_v2(bf16_tensor(lhs_bits, dev), pw, torch.from_numpy(gs).to(dev),
                 rhs_bias=None if bias is None else torch.from_numpy(bias).to(dev),
                 group_offset=go if window else None, fuse_act=act, preferred_element_type=torch.float32,
                 zero_initialize=window, lhs_quant_dtype=torch.float8_e4m3fn if mx else None)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    a = bf16_to_f32(lhs_bits)
    if mx:
        a = quant.mx_dequantize(*quant.mx_quantize_e4m3(a))
    n = rhs.shape[2] * 2
    b = rhs[:, :, np.arange(n) // 2]
    nib = np.where(np.arange(n) % 2 == 1, b >> 4, b & 0xF).astype(np.uint8)
    w = gmm.dequant_rhs(fp4.e2m1_to_codes(nib), fp4.e8m0_decode(sc))
    y64, written = gmm.gmm(a, None, None, gs, group_offset=go, out_dtype="float64", w=w, bias=bias)
    acc_err = K * 2.0 ** -24 * gmm.abs_product(a, w, gs, group_offset=go) + 2.0 ** -24 * np.abs(y64)
    if mx:
        acc_err += gmm.MX_BLOCK_TERM * gmm.block_max_product(a, w, gs, group_offset=go)
    if act is None:
        want, bound = y64, 2.0 ** -24 * np.abs(y64) + acc_err
    else:
        want, bound = omb.apply_act(y64, act), omb.act_bound(y64, acc_err, act)
    if window:
        assert np.all(got[~written] == 0)
    err = np.abs(got[written] - want[written])
    assert np.all(np.isfinite(got[written]))
    assert np.all(err <= bound[written]), (seed, float((err / bound[written]).max()))
