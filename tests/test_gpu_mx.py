"""MX mode of the FP4 grouped matmul on the GPU (gmm_v2 with
lhs_quant_dtype=float8_e4m3fn): the lhs quantization bit for bit against the
oracle (oracle.quant.mx_quantize_e4m3, the reference's power-of-two block
quantizer at block 32), and the scaled-MFMA gmm against the float64 product
of the dequantized operands under the stated tolerance
(oracle.gmm.mx_error_bound)

    |y - y64| <= u_out * |y64| + K * 2^-24 * sum_k |a_k w_k|
                 + 2^-11 * sum_b max_{k in b} |a_k w_k|

(u_out = 2^-8 for bf16 output, 2^-24 for f32; a = the dequantized e4m3 lhs;
b = the 32-value K-blocks).  The last term is the scaled MFMA's in-block
alignment, which test_mx_mfma_block_alignment measures.  The quantization
error itself (MX output against the bf16 path's float64 result) is
reported, not bounded per element.
"""
import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from oracle import fp4, gmm, quant
from oracle.numerics import bf16_bits as to_bf16_bits
from oracle.numerics import bf16_to_f32

pytestmark = pytest.mark.gpu


def _mx_gpu(dev, x_bits):
    from dw_tpu_amd import mx_quantize
    q = mx_quantize(bf16_tensor(x_bits, dev))
    torch.cuda.synchronize()
    return q.codes.cpu().numpy(), q.scales.cpu().numpy()


def _special_rows(rng, K):
    """Rows built to hit every branch of the scale rule: blocks of zeros
    (both signs), NaN / inf blocks, absmax exactly 448 * 2^e and one bf16
    ulp either side, bf16 subnormals, the largest bf16 values, e4m3 ties."""
    nb = K // 32
    rows = []
    for kind in range(8):
        x = rng.standard_normal(K).astype(np.float32) * np.float32(2.0 ** rng.integers(-20, 20))
        xb = x.reshape(nb, 32)
        for b in range(nb):
            sel = (b + kind) % 8
            if sel == 0:
                xb[b] = 0.0
                xb[b, ::3] = -0.0
            elif sel == 1:
                xb[b, rng.integers(32)] = [np.nan, np.inf, -np.inf][b % 3]
            elif sel == 2:
                e = int(rng.integers(-100, 100))
                xb[b] *= np.float32(2.0 ** -40)
                xb[b, 5] = np.float32(448.0 * 2.0 ** e)           # absmax exactly 448 * 2^e
            elif sel == 3:
                e = int(rng.integers(-100, 100))
                xb[b] *= np.float32(2.0 ** -40)
                xb[b, 7] = np.float32(1.7578125 * 2.0 ** (e + 8))  # one bf16 ulp above 1.75 * 2^(e+8)
            elif sel == 4:
                xb[b] = np.float32(2.0 ** -133) * rng.integers(-127, 128, 32)  # bf16 subnormals
            elif sel == 5:
                xb[b, :4] = np.float32(3.3e38) * np.array([1, -1, 0.5, -0.25], np.float32)
            elif sel == 6:
                # halfway between e4m3 neighbours after scaling: RNE ties
                xb[b] = np.float32(2.0 ** 10) * (np.float32(17.0) + rng.integers(0, 2, 32) * 2) / 16
                xb[b, 0] = np.float32(448.0 * 2.0 ** 10)
        rows.append(xb.reshape(K))
    return np.stack(rows)


@pytest.mark.parametrize("rows,K", [(1, 32), (3, 128), (64, 1024), (257, 7168)])
def test_mx_quant_bit_exact(dev, rng, rows, K):
    x = rng.standard_normal((rows, K)).astype(np.float32) * np.float32(3.0)
    if rows >= 8:
        x[:8] = _special_rows(rng, K)
    x_bits = to_bf16_bits(x)
    codes, scales = _mx_gpu(dev, x_bits)
    want_c, want_s = quant.mx_quantize_e4m3(bf16_to_f32(x_bits))
    assert np.array_equal(scales, want_s), np.argwhere(scales != want_s)[:5]
    assert np.array_equal(codes, want_c), np.argwhere(codes != want_c)[:5]


def _mx_case(rng, sizes, K, N, extra_rows=0):
    E = len(sizes)
    M = int(sum(sizes)) + extra_rows
    lhs_bits = to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    rhs = rng.integers(0, 256, (E, K, N // 2), dtype=np.uint8)
    sc = rng.integers(123, 130, (E, K // 32, 1, N), dtype=np.uint8)
    return lhs_bits, rhs, sc, np.array(sizes, np.int32)


def _w(rhs, sc):
    n = rhs.shape[2] * 2
    b = rhs[:, :, np.arange(n) // 2]
    nib = np.where(np.arange(n) % 2 == 1, b >> 4, b & 0xF).astype(np.uint8)
    return gmm.dequant_rhs(fp4.e2m1_to_codes(nib), fp4.e8m0_decode(sc))


def _oracle_mx(lhs_bits, w, gs, group_offset=0):
    """float64 MX product, |a| |w| term and written mask, from the oracle's
    quantization of the lhs."""
    c, s = quant.mx_quantize_e4m3(bf16_to_f32(lhs_bits))
    a = quant.mx_dequantize(c, s)
    y64, written = gmm.gmm(a, None, None, gs, group_offset=group_offset, out_dtype="float64", w=w)
    ap = gmm.abs_product(a, w, gs, group_offset=group_offset)
    bm = gmm.block_max_product(a, w, gs, group_offset=group_offset)
    return y64, (ap, bm), written


def _check(out, y64, terms, K, out_dtype, mask=None):
    y = out.float().cpu().numpy().astype(np.float64)
    kind = "float32" if out_dtype == torch.float32 else "bfloat16"
    ap, bm = terms
    if mask is not None:
        y, y64, ap, bm = y[mask], y64[mask], ap[mask], bm[mask]
    bound = gmm.mx_error_bound(y64, ap, bm, K, kind)
    err = np.abs(y - y64)
    stats = gmm.error_stats(y, y64)
    stats["max_err_over_tol"] = float((err / np.maximum(bound, 1e-300)).max()) if err.size else 0.0
    assert np.all(np.isfinite(y))
    assert np.all(err <= bound), stats
    return stats


def _gmm_mx(dev, lhs_bits, rhs, sc, gs, out_dtype=torch.bfloat16, group_offset=None, zero_init=True,
            fuse_act=None):
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2
    pw = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev),
                             gate_up=fuse_act is not None)
    out = gmm_v2(bf16_tensor(lhs_bits, dev), pw, torch.from_numpy(np.asarray(gs, np.int32)).to(dev),
                 group_offset=group_offset, preferred_element_type=out_dtype, zero_initialize=zero_init,
                 lhs_quant_dtype=torch.float8_e4m3fn, fuse_act=fuse_act)
    torch.cuda.synchronize()
    return out


CASES = [  # K < 4096: the 64-deep kernel; K >= 4096: the 128-deep one
    ([5], 128, 16),
    ([1, 0, 15, 16, 17], 128, 96),
    ([31, 32, 33, 0, 3], 256, 272),
    ([127, 128, 129, 0, 3], 256, 272),
    ([300, 0, 0, 64, 257], 1024, 512),
    ([0, 0, 0], 128, 64),
    ([5], 4096, 16),
    ([1, 0, 15, 16, 17, 95, 97], 4096, 96),
    ([127, 0, 129, 8], 4224, 656),
]


@pytest.mark.parametrize("sizes,K,N", CASES)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gmm_mx_random_shapes(dev, rng, sizes, K, N, out_dtype):
    lhs_bits, rhs, sc, gs = _mx_case(rng, sizes, K, N)
    out = _gmm_mx(dev, lhs_bits, rhs, sc, gs, out_dtype=out_dtype)
    if out.shape[0]:
        y64, ap, _ = _oracle_mx(lhs_bits, _w(rhs, sc), gs)
        print(sizes, K, N, _check(out, y64, ap, K, out_dtype), flush=True)


def test_gmm_mx_prequantized_lhs_and_repeat_runs(dev, rng):
    """An MxLhs passed directly gives the bits of lhs_quant_dtype on bf16, and
    repeated runs are bitwise identical."""
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2, mx_quantize
    lhs_bits, rhs, sc, gs = _mx_case(rng, [100, 3, 0, 200], 512, 256)
    a = _gmm_mx(dev, lhs_bits, rhs, sc, gs)
    b = _gmm_mx(dev, lhs_bits, rhs, sc, gs)
    pw = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev))
    c = gmm_v2(mx_quantize(bf16_tensor(lhs_bits, dev)), pw, torch.from_numpy(gs).to(dev))
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(a.view(torch.int16), c.view(torch.int16))


@pytest.mark.parametrize("K", [128, 4096])
def test_gmm_mx_group_offset_and_zero_init(dev, rng, K):
    sizes = [20, 35, 0, 50, 9]
    lhs_bits, rhs, sc, gs = _mx_case(rng, sizes, K, 64, extra_rows=7)
    out = _gmm_mx(dev, lhs_bits, rhs[1:4], sc[1:4], gs, group_offset=1)
    y64, ap, written = _oracle_mx(lhs_bits, _w(rhs[1:4], sc[1:4]), gs, group_offset=1)
    assert list(np.nonzero(written)[0]) == list(range(20, 105))
    y = out.float().cpu().numpy()
    assert np.all(y[~written] == 0)
    _check(out, y64, ap, K, torch.bfloat16, mask=written)
    out2 = _gmm_mx(dev, lhs_bits, rhs[1:4], sc[1:4], gs, group_offset=1, zero_init=False)
    assert torch.equal(out2[20:105].view(torch.int16), out[20:105].view(torch.int16))


@pytest.mark.parametrize("K", [256, 4096])
@pytest.mark.parametrize("fused_act", [False, True])
def test_gmm_mx_fused_row_gather_equals_gather_then_gmm(dev, rng, fused_act, K):
    """lhs_row_indices in the MX mode gives the bits of quantizing the
    gathered rows: quantization is per row, so quantizing the tokens once and
    gathering their codes and scales is the same."""
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2, mx_quantize, row_gather
    T, N = 150, 192
    sizes = [37, 0, 120, 64, 9]
    M = sum(sizes)
    hidden = bf16_tensor(to_bf16_bits(rng.standard_normal((T, K)).astype(np.float32)), dev)
    idx_np = rng.integers(0, T, M).astype(np.int32)
    idx_np[3], idx_np[50], idx_np[M - 1] = -1, T + 7, -T - 5
    idx = torch.from_numpy(idx_np).to(dev)
    rhs = torch.from_numpy(rng.integers(0, 256, (len(sizes), K, N // 2), dtype=np.uint8)).to(dev)
    sc = torch.from_numpy(rng.integers(123, 130, (len(sizes), K // 32, 1, N), dtype=np.uint8)).to(dev)
    w = fp4_weight_to_codes(rhs, sc, gate_up=fused_act)
    gs = torch.from_numpy(np.array(sizes, np.int32)).to(dev)
    act = "silu_and_mul_with_clamp" if fused_act else None
    want = gmm_v2(row_gather(hidden, idx), w, gs, fuse_act=act, lhs_quant_dtype=torch.float8_e4m3fn)
    got = gmm_v2(mx_quantize(hidden), w, gs, fuse_act=act, lhs_row_indices=idx)
    torch.cuda.synchronize()
    assert got.shape == want.shape
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("K", [512, 4096])
def test_gmm_mx_fused_activation(dev, rng, K):
    """gmm1 with the fused activation in the MX mode against the oracle's
    activation of the float64 MX product (oracle.moe_block's propagated
    bound)."""
    from oracle import moe_block as omb
    N = 256
    lhs_bits, rhs, sc, gs = _mx_case(rng, [60, 0, 130, 7], K, N)
    out = _gmm_mx(dev, lhs_bits, rhs, sc, gs, fuse_act="silu_and_mul_with_clamp")
    y64, (ap, bm), _ = _oracle_mx(lhs_bits, _w(rhs, sc), gs)
    h = bf16_to_f32(bf16_bits(out)).astype(np.float64)
    act64 = omb.silu_and_mul_clamp(y64)
    bound = omb.act_output_bound(act64, omb.act_error_bound(y64, K * 2.0 ** -24 * ap + gmm.MX_BLOCK_TERM * bm))
    assert np.all(np.abs(h - act64) <= bound)


@pytest.mark.parametrize("name", ["cpu_plumbing", "decode_gate_up", "decode_down", "prefill"])
def test_gmm_mx_workloads(dev, rng, name):
    """Every gmm workload in the MX mode: the GPU quantization of sampled rows
    bit for bit, the gmm against the float64 MX oracle on sampled rows and
    columns (all of cpu_plumbing), and the quantization error against the
    bf16 path's float64 result reported."""
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2, mx_quantize
    from dw_tpu_amd.workloads import make_gmm_workload
    wl = make_gmm_workload(name)
    pw = fp4_weight_to_codes(torch.from_numpy(wl.rhs_e2m1).to(dev), torch.from_numpy(wl.scale_codes).to(dev))
    lhs = bf16_tensor(wl.lhs_bits, dev)
    q = mx_quantize(lhs)
    out = gmm_v2(q, pw, torch.from_numpy(wl.group_sizes).to(dev))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    if name == "cpu_plumbing":
        rows, cols = np.arange(wl.M), np.arange(wl.N)
    else:
        rows, cols = gmm.sample_rows_cols(wl.group_sizes, wl.N, rng)
    r_t = torch.from_numpy(rows).to(dev)
    codes, scales = q.codes[r_t].cpu().numpy(), q.scales[r_t].cpu().numpy()
    want_c, want_s = quant.mx_quantize_e4m3(bf16_to_f32(wl.lhs_bits[rows]))
    assert np.array_equal(codes, want_c) and np.array_equal(scales, want_s)
    starts = np.concatenate([[0], np.cumsum(wl.group_sizes)])
    grp = np.searchsorted(starts, rows, side="right") - 1
    sub_gs = np.bincount(grp, minlength=wl.E).astype(np.int32)
    b = wl.rhs_e2m1[:, :, cols // 2]
    nib = np.where(cols % 2 == 1, b >> 4, b & 0xF).astype(np.uint8)
    w = gmm.dequant_rhs(fp4.e2m1_to_codes(nib), fp4.e8m0_decode(wl.scale_codes[..., cols]))
    y64, ap, _ = _oracle_mx(wl.lhs_bits[rows], w, sub_gs)
    got = out[r_t][:, torch.from_numpy(cols).to(dev)]
    stats = _check(got, y64, ap, wl.K, torch.bfloat16)
    # The distance a caller sees: the MX output against the reference's W4A16
    # result (the lhs quantization included).  bench.py's CPU leg reports the
    # same figures for each <name>_mx line, from the same oracle functions.
    y_w4a16 = gmm.w4a16_rows(wl.lhs_bits[rows], wl.rhs_e2m1, wl.scale_codes, wl.group_sizes, rows, cols)
    assert np.allclose(y_w4a16, gmm.gmm(bf16_to_f32(wl.lhs_bits[rows]), None, None, sub_gs,
                                        out_dtype="float64", w=w)[0], rtol=0, atol=0)
    vs = gmm.error_stats(got.float().cpu().numpy(), y_w4a16)
    stats["vs_w4a16_max_abs"], stats["vs_w4a16_rel_fro"] = vs["max_abs"], vs["rel_fro"]
    print(name, stats, flush=True)
    assert stats["vs_w4a16_rel_fro"] < 0.05


@pytest.mark.parametrize("name", ["decode_gate_up", "prefill"])
def test_gmm_mx_full_size_exact_scaling(dev, name):
    """Doubling the bf16 lhs doubles every scale and keeps every code, so the
    MX gmm's f32 output doubles bit for bit at the full workload."""
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2
    from dw_tpu_amd.workloads import make_gmm_workload
    wl = make_gmm_workload(name)
    pw = fp4_weight_to_codes(torch.from_numpy(wl.rhs_e2m1).to(dev), torch.from_numpy(wl.scale_codes).to(dev))
    lhs = bf16_tensor(wl.lhs_bits, dev)
    gs = torch.from_numpy(wl.group_sizes).to(dev)
    kw = dict(preferred_element_type=torch.float32, lhs_quant_dtype=torch.float8_e4m3fn)
    y1 = gmm_v2(lhs, pw, gs, **kw)
    y2 = gmm_v2(lhs * 2, pw, gs, **kw)
    torch.cuda.synchronize()
    assert torch.equal(y2, y1 * 2)
    assert torch.isfinite(y1).all()


def test_mx_mfma_block_alignment(dev):
    """The scaled MFMA's accumulation inside one 32-value K-block, measured
    on crafted rows (weights all 1.0): a product of 448 with 31 small ones of
    one sign, of both signs, and with a cancelling -448.  Every error stays
    within half the stated in-block term (2^-12 of the block's largest
    product), and products in different blocks combine exactly to 2^-20."""
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2, mx_quantize
    K, N = 128, 64
    pw = fp4_weight_to_codes(torch.from_numpy(np.full((1, K, N // 2), 0x22, np.uint8)).to(dev),
                             torch.from_numpy(np.full((1, K // 32, 1, N), 127, np.uint8)).to(dev))
    rows = []
    for v in [1.0, 0.375, 0.0625, 0.046875, 2.0 ** -5, 2.0 ** -6, 2.0 ** -7, 2.0 ** -9, 3 * 2.0 ** -9]:
        for sgn in (1, -1):
            r = np.zeros(K, np.float32); r[0] = 448.0; r[1:32] = sgn * v; rows.append(r)
        r = np.zeros(K, np.float32); r[0] = 448.0; r[1:32:2] = v; r[2:32:2] = -v / 2; rows.append(r)
        r = np.zeros(K, np.float32); r[0] = 448.0; r[1] = -448.0; r[2:32] = v; rows.append(r)
    in_block = len(rows)
    for j in range(0, 20):  # 448 in block 0, 32 x 1.25 2^-j in block 1 (own scale)
        r = np.zeros(K, np.float32); r[0] = 448.0; r[32:64] = np.float32(1.25 * 2.0 ** -j); rows.append(r)
    x = np.stack(rows)
    q = mx_quantize(bf16_tensor(to_bf16_bits(x), dev))
    y = gmm_v2(q, pw, torch.tensor([x.shape[0]], dtype=torch.int32, device=dev),
               preferred_element_type=torch.float32)[:, 0].cpu().numpy().astype(np.float64)
    torch.cuda.synchronize()
    want = quant.mx_dequantize(q.codes.cpu().numpy(), q.scales.cpu().numpy()).astype(np.float64).sum(1)
    err = np.abs(y - want) / 448.0
    print("in-block max error / largest product: %.3e; across blocks: %.3e" % (err[:in_block].max(),
                                                                             err[in_block:].max()))
    assert err[:in_block].max() <= gmm.MX_BLOCK_TERM / 2
    assert err[in_block:].max() <= 2.0 ** -20
