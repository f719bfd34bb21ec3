"""The grouped matmul's epilogue on the GPU: gmm_v2's rhs_bias and every
fused activation of apply_act_fn
(patches/tpu-inference-experimental/fused-moe-fp4/0901-...:57-66), on the
bf16 path and on the MX path (both of its kernels: K < 4096 and K >= 4096),
against the float64 oracle:

* no activation: |y - y64| within oracle.gmm.error_bound (bf16 lhs) or
  mx_error_bound (MX), y64 = lhs @ w + bias;
* an activation: |h - act(y64)| within oracle.moe_block.act_bound, with the
  accumulator error of the matching gmm bound (plus one f32 rounding of the
  bias add) propagated through the activation's Lipschitz constants.
"""
import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from oracle import fp4, gmm, quant
from oracle import moe_block as omb
from oracle.numerics import bf16_bits as to_bf16_bits
from oracle.numerics import bf16_to_f32

pytestmark = pytest.mark.gpu

ACTS = [None, "silu_and_mul_with_clamp", "silu", "gelu", "swigluoai"]


def _case(rng, sizes, K, N):
    E = len(sizes)
    lhs_bits = to_bf16_bits(rng.standard_normal((sum(sizes), K)).astype(np.float32))
    rhs = rng.integers(0, 256, (E, K, N // 2), dtype=np.uint8)
    sc = rng.integers(122, 128, (E, K // 32, 1, N), dtype=np.uint8)
    bias = (rng.standard_normal((E, N)) * 4).astype(np.float32)
    return lhs_bits, rhs, sc, np.array(sizes, np.int32), bias


def _w(rhs, sc):
    n = rhs.shape[2] * 2
    b = rhs[:, :, np.arange(n) // 2]
    nib = np.where(np.arange(n) % 2 == 1, b >> 4, b & 0xF).astype(np.uint8)
    return gmm.dequant_rhs(fp4.e2m1_to_codes(nib), fp4.e8m0_decode(sc))


def _run(dev, lhs_bits, rhs, sc, gs, bias, act, mx, out_dtype=torch.bfloat16, bias_dtype=torch.float32, idx=None):
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2
    pw = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev), gate_up=act is not None)
    b = None if bias is None else torch.from_numpy(bias).to(dev).to(bias_dtype)
    out = gmm_v2(bf16_tensor(lhs_bits, dev), pw, torch.from_numpy(gs).to(dev), rhs_bias=b, fuse_act=act,
                 preferred_element_type=out_dtype, lhs_quant_dtype=torch.float8_e4m3fn if mx else None,
                 lhs_row_indices=idx)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("K", [256, 4096])
@pytest.mark.parametrize("mx", [False, True])
def test_bias_and_activation(dev, rng, mx, K, act):
    N = 192
    lhs_bits, rhs, sc, gs, bias = _case(rng, [40, 0, 70, 33], K, N)
    out = _run(dev, lhs_bits, rhs, sc, gs, bias, act, mx)
    a = bf16_to_f32(lhs_bits)
    if mx:
        a = quant.mx_dequantize(*quant.mx_quantize_e4m3(a))
    w = _w(rhs, sc)
    y64, _ = gmm.gmm(a, None, None, gs, out_dtype="float64", w=w, bias=bias)
    ap = gmm.abs_product(a, w, gs)
    acc_err = K * 2.0 ** -24 * ap + 2.0 ** -24 * np.abs(y64)
    if mx:
        acc_err += gmm.MX_BLOCK_TERM * gmm.block_max_product(a, w, gs)
    got = bf16_to_f32(bf16_bits(out)).astype(np.float64)
    if act is None:
        want, bound = y64, 2.0 ** -8 * np.abs(y64) + acc_err
    else:
        want, bound = omb.apply_act(y64, act), omb.act_bound(y64, acc_err, act)
    err = np.abs(got - want)
    assert np.all(np.isfinite(got))
    assert np.all(err <= bound), (float(err.max()), float((err / bound).max()))
    print(mx, K, act, gmm.error_stats(got, want), flush=True)


@pytest.mark.parametrize("mx", [False, True])
def test_bias_dtypes_and_shapes(dev, rng, mx):
    """A bf16 bias gives the bits of the same values in f32 ([E, N] and
    [E, 1, N] alike), f32 output included; no bias differs."""
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2
    K, N = 256, 144
    lhs_bits, rhs, sc, gs, bias = _case(rng, [17, 64, 0, 9], K, N)
    bias_b = to_bf16_bits(bias)
    bias_f = bf16_to_f32(bias_b)
    kw = dict(lhs_quant_dtype=torch.float8_e4m3fn if mx else None)
    pw = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev))
    lhs, g = bf16_tensor(lhs_bits, dev), torch.from_numpy(gs).to(dev)
    for od in (torch.bfloat16, torch.float32):
        y_f = gmm_v2(lhs, pw, g, rhs_bias=torch.from_numpy(bias_f).to(dev), preferred_element_type=od, **kw)
        y_b = gmm_v2(lhs, pw, g, rhs_bias=bf16_tensor(bias_b, dev)[:, None, :], preferred_element_type=od, **kw)
        y_0 = gmm_v2(lhs, pw, g, preferred_element_type=od, **kw)
        torch.cuda.synchronize()
        assert torch.equal(y_f, y_b)
        assert not torch.equal(y_f, y_0)


@pytest.mark.parametrize("mx", [False, True])
def test_bias_with_fused_gather(dev, rng, mx):
    """lhs_row_indices with a bias and an activation gives the bits of the
    gathered copy through the same call."""
    from dw_tpu_amd import row_gather
    K, N, T = 256, 128, 90
    sizes = [30, 0, 50, 12]
    _, rhs, sc, gs, bias = _case(rng, sizes, K, N)
    hidden_bits = to_bf16_bits(rng.standard_normal((T, K)).astype(np.float32))
    idx = torch.from_numpy(rng.integers(0, T, sum(sizes)).astype(np.int32)).to(dev)
    x_bits = bf16_bits(row_gather(bf16_tensor(hidden_bits, dev), idx))
    for act in (None, "swigluoai"):
        want = _run(dev, x_bits, rhs, sc, gs, bias, act, mx)
        got = _run(dev, hidden_bits, rhs, sc, gs, bias, act, mx, idx=idx)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("mx", [False, True])
@pytest.mark.parametrize("act", [None, "gelu"])
def test_bias_with_group_offset_window(dev, rng, mx, act):
    """An expert-parallel window (group_offset, E_local < num_groups): the
    bias row of local expert g - group_offset is added to group g's rows only,
    and rows outside the window are zero (zero_initialize)."""
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2
    K, N = 256, 128
    sizes = [20, 33, 0, 41, 7, 50]
    go, e_local = 2, 3
    lhs_bits = to_bf16_bits(rng.standard_normal((sum(sizes), K)).astype(np.float32))
    rhs = rng.integers(0, 256, (e_local, K, N // 2), dtype=np.uint8)
    sc = rng.integers(122, 128, (e_local, K // 32, 1, N), dtype=np.uint8)
    bias = (rng.standard_normal((e_local, N)) * 4).astype(np.float32)
    gs = np.array(sizes, np.int32)
    pw = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev), gate_up=act is not None)
    out = gmm_v2(bf16_tensor(lhs_bits, dev), pw, torch.from_numpy(gs).to(dev),
                 rhs_bias=torch.from_numpy(bias).to(dev), group_offset=go, fuse_act=act,
                 preferred_element_type=torch.float32, lhs_quant_dtype=torch.float8_e4m3fn if mx else None)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    a = bf16_to_f32(lhs_bits)
    if mx:
        a = quant.mx_dequantize(*quant.mx_quantize_e4m3(a))
    w = _w(rhs, sc)
    y64, written = gmm.gmm(a, None, None, gs, group_offset=go, out_dtype="float64", w=w, bias=bias)
    ap = gmm.abs_product(a, w, gs, group_offset=go)
    acc_err = K * 2.0 ** -24 * ap + 2.0 ** -24 * np.abs(y64)
    if mx:
        acc_err += gmm.MX_BLOCK_TERM * gmm.block_max_product(a, w, gs, group_offset=go)
    if act is None:
        want, bound = y64, 2.0 ** -24 * np.abs(y64) + acc_err
    else:
        want, bound = omb.apply_act(y64, act), omb.act_bound(y64, acc_err, act)
    assert np.all(got[~written] == 0)
    err = np.abs(got[written] - want[written])
    assert np.all(err <= bound[written]), float((err / bound[written]).max())


@pytest.mark.parametrize("act", [None, "silu_and_mul_with_clamp"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("window", [False, True])
def test_remainder_rows_every_count(dev, rng, act, out_dtype, window):
    """Row tiles of every 16-row block count (1 .. 6) and fill, the first and
    last rows of a block included, with a bias and N = 640 (a 512-column tile
    and a part-filled one; as 256-column tiles, one of them past N by two
    groups).  The tile list leaves most CUs idle, so every class runs as
    narrow tiles; with `window` a 12,288-row group outside the expert-parallel
    window (group_offset 1) comes first, so the launch sizes its grid for
    that many rows and runs the kernel without narrow tiles on the same
    local groups.  Against the float64 oracle under the bounds above; rows
    outside the window are zero."""
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2
    K, N = 256, 640
    local = [1, 16, 17, 32, 33, 48, 49, 64, 0, 65, 80, 81, 96, 97, 112, 113, 160, 161, 177, 192, 5]
    sizes = ([12288] if window else []) + local
    go = 1 if window else 0
    e_local = len(local)
    lhs_bits = to_bf16_bits(rng.standard_normal((sum(sizes), K)).astype(np.float32))
    rhs = rng.integers(0, 256, (e_local, K, N // 2), dtype=np.uint8)
    sc = rng.integers(122, 128, (e_local, K // 32, 1, N), dtype=np.uint8)
    bias = (rng.standard_normal((e_local, N)) * 4).astype(np.float32)
    gs = np.array(sizes, np.int32)
    pw = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev), gate_up=act is not None)
    out = gmm_v2(bf16_tensor(lhs_bits, dev), pw, torch.from_numpy(gs).to(dev),
                 rhs_bias=torch.from_numpy(bias).to(dev), group_offset=go if window else None, fuse_act=act,
                 preferred_element_type=out_dtype, zero_initialize=window)
    torch.cuda.synchronize()
    a = bf16_to_f32(lhs_bits)
    w = _w(rhs, sc)
    y64, written = gmm.gmm(a, None, None, gs, group_offset=go, out_dtype="float64", w=w, bias=bias)
    ap = gmm.abs_product(a, w, gs, group_offset=go)
    acc_err = K * 2.0 ** -24 * ap + 2.0 ** -24 * np.abs(y64)
    if out_dtype == torch.float32:
        got = out.cpu().numpy().astype(np.float64)
        rnd = 2.0 ** -24
    else:
        got = bf16_to_f32(bf16_bits(out)).astype(np.float64)
        rnd = 2.0 ** -8
    if act is None:
        want, bound = y64, rnd * np.abs(y64) + acc_err
    else:
        want, bound = omb.apply_act(y64, act), omb.act_bound(y64, acc_err, act)
    assert int(written.sum()) == sum(local)
    assert np.all(got[~written] == 0)
    err = np.abs(got[written] - want[written])
    assert np.all(np.isfinite(got))
    assert np.all(err <= bound[written]), (float(err.max()), float((err / bound[written]).max()))


@pytest.mark.parametrize("act", [None, "swigluoai"])
def test_mx_row_halves(dev, rng, act):
    """The 64-deep MX kernel's stacked row halves (192 x 256 tiles, used
    below K = 4096 when the groups average 97 .. 192 rows): groups of
    1 .. 193 rows, so a half holds 0 .. 3 row blocks and a consumer may have
    no rows; a bias; N = 320, so the second 256-column tile holds one group
    and three past N.  Against the float64 MX oracle under the bounds above."""
    K, N = 256, 320
    sizes = [1, 97, 150, 192, 193, 0, 64, 128]
    assert 96 * len(sizes) < sum(sizes) <= 192 * len(sizes)
    lhs_bits, rhs, sc, gs, bias = _case(rng, sizes, K, N)
    out = _run(dev, lhs_bits, rhs, sc, gs, bias, act, True)
    a = quant.mx_dequantize(*quant.mx_quantize_e4m3(bf16_to_f32(lhs_bits)))
    w = _w(rhs, sc)
    y64, _ = gmm.gmm(a, None, None, gs, out_dtype="float64", w=w, bias=bias)
    ap = gmm.abs_product(a, w, gs)
    acc_err = K * 2.0 ** -24 * ap + 2.0 ** -24 * np.abs(y64) + gmm.MX_BLOCK_TERM * gmm.block_max_product(a, w, gs)
    got = bf16_to_f32(bf16_bits(out)).astype(np.float64)
    if act is None:
        want, bound = y64, 2.0 ** -8 * np.abs(y64) + acc_err
    else:
        want, bound = omb.apply_act(y64, act), omb.act_bound(y64, acc_err, act)
    err = np.abs(got - want)
    assert np.all(np.isfinite(got))
    assert np.all(err <= bound), (float(err.max()), float((err / bound).max()))


@pytest.mark.parametrize("act", [None, "silu_and_mul_with_clamp"])
def test_mx_row_halves_with_fused_gather(dev, rng, act):
    """The stacked-halves MX tiles with lhs_row_indices give the bits of the
    gathered copy through the same call (row indices read per half)."""
    from dw_tpu_amd import row_gather
    K, N, T = 256, 320, 300
    sizes = [1, 97, 150, 192, 193, 0, 64, 128]
    assert 96 * len(sizes) < sum(sizes) <= 192 * len(sizes)
    _, rhs, sc, gs, bias = _case(rng, sizes, K, N)
    hidden_bits = to_bf16_bits(rng.standard_normal((T, K)).astype(np.float32))
    idx = torch.from_numpy(rng.integers(0, T, sum(sizes)).astype(np.int32)).to(dev)
    x_bits = bf16_bits(row_gather(bf16_tensor(hidden_bits, dev), idx))
    want = _run(dev, x_bits, rhs, sc, gs, bias, act, True)
    got = _run(dev, hidden_bits, rhs, sc, gs, bias, act, True, idx=idx)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
