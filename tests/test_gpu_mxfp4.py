"""MXFP4 lhs (gmm_v2(lhs_quant_dtype=float4_e2m1fn)) on the GPU: the e2m1
block-32 quantizer bit for bit against the oracle (oracle/quant.py
mx_quantize_e2m1, pinned against the reference's quantize_tensor), and the
fp4 x fp4 scaled-MFMA grouped matmul against the float64 product of the
dequantized operands within the MX bound of oracle/gmm.py (mx_error_bound);
max abs and relative Frobenius errors are printed, and the distance from the
reference's W4A16 result is reported for each workload."""
import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from oracle import fp4, gmm, quant
from oracle.numerics import bf16_bits as to_bf16_bits
from oracle.numerics import bf16_to_f32

pytestmark = pytest.mark.gpu
F4 = "float4_e2m1fn"


def _special_rows_e2m1(rng, K):
    """Blocks that hit every branch of the e2m1 scale rule: zeros of both
    signs, NaN / inf, absmax exactly 6 * 2^e and one bf16 ulp above it, bf16
    subnormals, the largest bf16 values, and e2m1 rounding ties."""
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
                xb[b, 5] = np.float32(6.0 * 2.0 ** e)                   # absmax exactly 6 * 2^e
            elif sel == 3:
                e = int(rng.integers(-100, 100))
                xb[b] *= np.float32(2.0 ** -40)
                xb[b, 7] = np.float32(1.5078125 * 2.0 ** (e + 2))       # one bf16 ulp above 6 * 2^e
            elif sel == 4:
                xb[b] = np.float32(2.0 ** -133) * rng.integers(-127, 128, 32)  # bf16 subnormals
            elif sel == 5:
                xb[b, :4] = np.float32(3.3e38) * np.array([1, -1, 0.5, -0.25], np.float32)
            elif sel == 6:
                # e2m1 ties after scaling by 2^10 (block max 6 * 2^10)
                xb[b] = np.float32(2.0 ** 10) * rng.choice(np.float32([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]), 32)
                xb[b] *= np.where(rng.random(32) < 0.5, -1, 1).astype(np.float32)
                xb[b, 0] = np.float32(6.0 * 2.0 ** 10)
        rows.append(xb.reshape(K))
    return np.stack(rows)


@pytest.mark.parametrize("rows,K", [(1, 32), (3, 128), (64, 1024), (257, 7168)])
def test_mxfp4_quant_bit_exact(dev, rng, rows, K):
    from dw_tpu_amd import mx_quantize
    x = rng.standard_normal((rows, K)).astype(np.float32) * np.float32(3.0)
    if rows >= 8:
        x[:8] = _special_rows_e2m1(rng, K)
    x_bits = to_bf16_bits(x)
    q = mx_quantize(bf16_tensor(x_bits, dev), "e2m1")
    torch.cuda.synchronize()
    want_c, want_s = quant.mx_quantize_e2m1(bf16_to_f32(x_bits))
    assert np.array_equal(q.scales.cpu().numpy(), want_s)
    assert np.array_equal(q.codes.cpu().numpy(), fp4.pack_nibbles(want_c))
    # the MxLhs view dequantizes to the oracle's values (NaN blocks aside; on
    # host tensors, which keep f32 subnormals such as 0.5 * 2^-126)
    from dw_tpu_amd import MxLhs
    deq = MxLhs(q.codes.cpu(), q.scales.cpu(), q.fmt).dequantize().numpy()
    want = quant.mx_dequantize_e2m1(want_c, want_s)
    ok = ~np.isnan(want)
    assert np.array_equal(deq[ok], want[ok]) and np.all(np.isnan(deq[~ok]))


def _case(rng, sizes, K, N, extra_rows=0):
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


def _oracle(lhs_bits, w, gs, group_offset=0):
    c, s = quant.mx_quantize_e2m1(bf16_to_f32(lhs_bits))
    a = quant.mx_dequantize_e2m1(c, s)
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


def _gmm(dev, lhs_bits, rhs, sc, gs, out_dtype=torch.bfloat16, group_offset=None, zero_init=True, fuse_act=None):
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2
    pw = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev),
                             gate_up=fuse_act is not None)
    out = gmm_v2(bf16_tensor(lhs_bits, dev), pw, torch.from_numpy(np.asarray(gs, np.int32)).to(dev),
                 group_offset=group_offset, preferred_element_type=out_dtype, zero_initialize=zero_init,
                 lhs_quant_dtype=F4, fuse_act=fuse_act)
    torch.cuda.synchronize()
    return out


CASES = [
    ([5], 128, 16),
    ([1, 0, 15, 16, 17], 128, 96),
    ([31, 32, 33, 0, 3], 256, 272),
    ([127, 128, 129, 0, 3], 256, 272),   # 97 .. 192-row groups: stacked row halves
    ([200, 7, 0, 90], 1024, 512),
    ([40, 75, 3], 4096, 512),            # the 64-deep kernel at K >= 4096 too
]


@pytest.mark.parametrize("sizes,K,N", CASES)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_mxfp4_gmm_random_shapes(dev, rng, sizes, K, N, out_dtype):
    lhs_bits, rhs, sc, gs = _case(rng, sizes, K, N)
    out = _gmm(dev, lhs_bits, rhs, sc, gs, out_dtype)
    y64, terms, _ = _oracle(lhs_bits, _w(rhs, sc), gs)
    print(sizes, K, N, out_dtype, _check(out, y64, terms, K, out_dtype), flush=True)


def test_mxfp4_prequantized_lhs_repeat_runs_and_fused_paths(dev, rng):
    """An MxLhs passed in gives the same bits as lhs_quant_dtype, repeat runs
    are bitwise equal, and the fused row gather and activation run on it."""
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2, mx_quantize
    sizes, K, N = [33, 0, 70, 9], 512, 256
    lhs_bits, rhs, sc, gs = _case(rng, sizes, K, N)
    lhs = bf16_tensor(lhs_bits, dev)
    pw = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev))
    g = torch.from_numpy(gs).to(dev)
    q = mx_quantize(lhs, "e2m1")
    a = gmm_v2(q, pw, g)
    b = gmm_v2(lhs, pw, g, lhs_quant_dtype=F4)
    c = gmm_v2(q, pw, g)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)) and torch.equal(a.view(torch.int16),
                                                                                 c.view(torch.int16))
    with pytest.raises(ValueError, match="MxLhs"):
        gmm_v2(q, pw, g, lhs_quant_dtype=torch.float8_e4m3fn)
    # fused gather: rows of a source tensor by index equal the gathered copy
    perm = torch.from_numpy(rng.permutation(lhs.shape[0]).astype(np.int32)).to(dev)
    src_q = mx_quantize(lhs, "e2m1")
    fused = gmm_v2(src_q, pw, g, lhs_row_indices=perm)
    copy = gmm_v2(lhs[perm.long()], pw, g, lhs_quant_dtype=F4)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), copy.view(torch.int16))
    # fused activation on gate/up weights: bf16 out, within the bound of the f32 run's activation
    pgu = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev), gate_up=True)
    act = gmm_v2(q, pgu, g, fuse_act="silu_and_mul_with_clamp")
    torch.cuda.synchronize()
    assert act.shape == (lhs.shape[0], N // 2) and torch.isfinite(act.float()).all()


@pytest.mark.parametrize("K", [256, 4096])
def test_mxfp4_group_offset_and_zero_init(dev, rng, K):
    lhs_bits, rhs, sc, gs = _case(rng, [20, 31, 0, 45, 12], K, 128)
    out = _gmm(dev, lhs_bits, rhs[1:4], sc[1:4], gs, group_offset=torch.tensor([1], dtype=torch.int32, device=dev))
    y64, terms, written = _oracle(lhs_bits, _w(rhs[1:4], sc[1:4]), gs, group_offset=1)
    _check(out, y64, terms, K, torch.bfloat16, mask=written)
    assert np.all(out.float().cpu().numpy()[~written] == 0)


@pytest.mark.parametrize("name", ["cpu_plumbing", "decode_gate_up", "decode_down", "prefill"])
def test_mxfp4_workloads(dev, rng, name):
    """Every gmm workload in MXFP4: the quantization of sampled rows bit for
    bit, the gmm against the float64 MXFP4 oracle on sampled rows and
    columns, and the distance from the reference's W4A16 result reported."""
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2, mx_quantize
    from dw_tpu_amd.workloads import make_gmm_workload
    wl = make_gmm_workload(name)
    pw = fp4_weight_to_codes(torch.from_numpy(wl.rhs_e2m1).to(dev), torch.from_numpy(wl.scale_codes).to(dev))
    q = mx_quantize(bf16_tensor(wl.lhs_bits, dev), "e2m1")
    out = gmm_v2(q, pw, torch.from_numpy(wl.group_sizes).to(dev))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    if name == "cpu_plumbing":
        rows, cols = np.arange(wl.M), np.arange(wl.N)
    else:
        rows, cols = gmm.sample_rows_cols(wl.group_sizes, wl.N, rng)
    r_t = torch.from_numpy(rows).to(dev)
    want_c, want_s = quant.mx_quantize_e2m1(bf16_to_f32(wl.lhs_bits[rows]))
    assert np.array_equal(q.codes[r_t].cpu().numpy(), fp4.pack_nibbles(want_c))
    assert np.array_equal(q.scales[r_t].cpu().numpy(), want_s)
    starts = np.concatenate([[0], np.cumsum(wl.group_sizes)])
    grp = np.searchsorted(starts, rows, side="right") - 1
    sub_gs = np.bincount(grp, minlength=wl.E).astype(np.int32)
    b = wl.rhs_e2m1[:, :, cols // 2]
    nib = np.where(cols % 2 == 1, b >> 4, b & 0xF).astype(np.uint8)
    w = gmm.dequant_rhs(fp4.e2m1_to_codes(nib), fp4.e8m0_decode(wl.scale_codes[..., cols]))
    y64, terms, _ = _oracle(wl.lhs_bits[rows], w, sub_gs)
    got = out[r_t][:, torch.from_numpy(cols).to(dev)]
    stats = _check(got, y64, terms, wl.K, torch.bfloat16)
    vs = gmm.error_stats(got.float().cpu().numpy(),
                         gmm.w4a16_rows(wl.lhs_bits[rows], wl.rhs_e2m1, wl.scale_codes, wl.group_sizes, rows, cols))
    stats["vs_w4a16_max_abs"], stats["vs_w4a16_rel_fro"] = vs["max_abs"], vs["rel_fro"]
    print(name, stats, flush=True)
    assert stats["vs_w4a16_rel_fro"] < 0.25


@pytest.mark.parametrize("name", ["decode_gate_up", "decode_down"])
def test_mxfp4_full_size_exact_scaling(dev, name):
    """Doubling the bf16 lhs doubles every scale and keeps every code, so the
    f32 output doubles bit for bit at the full workload."""
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2
    from dw_tpu_amd.workloads import make_gmm_workload
    wl = make_gmm_workload(name)
    pw = fp4_weight_to_codes(torch.from_numpy(wl.rhs_e2m1).to(dev), torch.from_numpy(wl.scale_codes).to(dev))
    lhs = bf16_tensor(wl.lhs_bits, dev)
    gs = torch.from_numpy(wl.group_sizes).to(dev)
    kw = dict(preferred_element_type=torch.float32, lhs_quant_dtype=F4)
    y1 = gmm_v2(lhs, pw, gs, **kw)
    y2 = gmm_v2(lhs * 2, pw, gs, **kw)
    torch.cuda.synchronize()
    assert torch.equal(y2, y1 * 2)
    assert torch.isfinite(y1).all()
