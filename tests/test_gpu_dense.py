"""Dense FP8 GEMM (W8A16 and W8A8) on the GPU against the float64 oracle,
with the stated bound of oracle.dense_fp8.error_bound; max abs and relative
Frobenius errors are printed."""
import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from oracle import dense_fp8 as odf
from oracle import gmm as ogmm
from oracle.numerics import E4M3_VALUES, bf16_to_f32

pytestmark = pytest.mark.gpu


def _check(out, y64, ap, K):
    y = bf16_to_f32(bf16_bits(out)).astype(np.float64)
    bound = odf.error_bound(y64, ap, K)
    err = np.abs(y - y64)
    stats = ogmm.error_stats(y, y64)
    assert np.all(np.isfinite(y))
    assert np.all(err <= bound), (stats, float((err / np.maximum(bound, 1e-300)).max()))
    return stats


@pytest.mark.parametrize("M,K,N", [(1, 1024, 512), (3, 256, 48), (16, 1024, 512), (17, 512, 256),
                                   (100, 1024, 384), (128, 1024, 512), (300, 768, 256), (256, 512, 128),
                                   (513, 1024, 640), (1900, 256, 4096)])  # the last: 256-row tiles, ragged M
def test_w8a16_small_shapes(dev, M, K, N):
    from dw_tpu_amd.dense_fp8 import matmul
    from dw_tpu_amd.workloads import make_dense_workload
    wl = make_dense_workload(M, K, N, seed=77)
    x = bf16_tensor(wl.x_bits, dev)
    w = torch.from_numpy(wl.wq).to(dev).view(torch.float8_e4m3fn)
    s = torch.from_numpy(wl.s_w8a16).to(dev)
    out = matmul(x, w, s)
    xf = bf16_to_f32(wl.x_bits)
    y64 = odf.matmul_w8a16(xf, wl.wq, wl.s_w8a16, out_dtype="float64")
    print(M, K, N, _check(out, y64, odf.abs_product_w8a16(xf, wl.wq, wl.s_w8a16), K))


@pytest.mark.parametrize("M,K,N", [(1, 1024, 512), (16, 1024, 512), (33, 512, 256), (128, 1024, 512),
                                   (257, 768, 384), (256, 512, 128), (600, 1024, 640),
                                   (200, 5120, 4096)])  # the last: 10 K blocks per split, two row-scale chunks
def test_w8a8_small_shapes(dev, M, K, N):
    from dw_tpu_amd.dense_fp8 import matmul_w8a8
    from dw_tpu_amd.workloads import make_dense_workload
    wl = make_dense_workload(M, K, N, seed=78)
    out = matmul_w8a8(torch.from_numpy(wl.xq).to(dev), torch.from_numpy(wl.sx).to(dev),
                      torch.from_numpy(wl.wq).to(dev), torch.from_numpy(wl.sw).to(dev))
    y64 = odf.matmul_w8a8(wl.xq, wl.sx, wl.wq, wl.sw, out_dtype="float64")
    print(M, K, N, _check(out, y64, odf.abs_product_w8a8(wl.xq, wl.sx, wl.wq, wl.sw), K))


@pytest.mark.parametrize("M", [16, 300])
def test_dense_reference_acceptance_policy(dev, M):
    """The reference's kernel-acceptance rule
    (results/dsv4-dense-gemm-kernel-1/NOTES.md:26-27), with the oracle's f32
    per-K-block accumulation (the reference kernel's structure) as the
    current kernel: RMS error <= 1.10x and max abs error <= 2x of its error
    against float64, for both variants."""
    from dw_tpu_amd.dense_fp8 import matmul, matmul_w8a8
    from dw_tpu_amd.workloads import make_dense_workload
    K, N = 2048, 512
    wl = make_dense_workload(M, K, N, seed=79)
    x = bf16_tensor(wl.x_bits, dev)
    out16 = matmul(x, torch.from_numpy(wl.wq).to(dev).view(torch.float8_e4m3fn), torch.from_numpy(wl.s_w8a16).to(dev))
    out8 = matmul_w8a8(torch.from_numpy(wl.xq).to(dev), torch.from_numpy(wl.sx).to(dev),
                       torch.from_numpy(wl.wq).to(dev), torch.from_numpy(wl.sw).to(dev))
    xf = bf16_to_f32(wl.x_bits)
    cases = [(out16, odf.matmul_w8a16(xf, wl.wq, wl.s_w8a16, out_dtype="float64"),
              odf.matmul_w8a16(xf, wl.wq, wl.s_w8a16, accumulate="f32")),
             (out8, odf.matmul_w8a8(wl.xq, wl.sx, wl.wq, wl.sw, out_dtype="float64"),
              odf.matmul_w8a8(wl.xq, wl.sx, wl.wq, wl.sw, accumulate="f32"))]
    for out, y64, ybase in cases:
        ok, st = ogmm.acceptance_policy(bf16_to_f32(bf16_bits(out)), ybase, y64)
        print(M, st, flush=True)
        assert ok, st


@pytest.mark.parametrize("M", [1, 16, 128, 1024, 4096])
def test_dense_fp8_workload_sampled(dev, M):
    """The dense_fp8 workload (K=7168, N=4096) at every M: sampled rows x
    columns against the oracle, both variants, prepacked weights."""
    from dw_tpu_amd.dense_fp8 import matmul, matmul_w8a8, prepack_fp8, try_dense_fp8
    from dw_tpu_amd.workloads import make_dense_workload
    wl = make_dense_workload(M)
    rng = np.random.Generator(np.random.PCG64(M))
    rows = np.unique(np.r_[0, M - 1, rng.integers(0, M, 14)])
    cols = np.unique(np.r_[0, wl.N - 1, rng.integers(0, wl.N, 46)])
    pw = prepack_fp8(torch.from_numpy(wl.wq).to(dev))
    x = bf16_tensor(wl.x_bits, dev)
    s = torch.from_numpy(wl.s_w8a16).to(dev)
    out16 = try_dense_fp8(x, pw, s)
    assert out16 is not None
    xf = bf16_to_f32(wl.x_bits)[rows]
    wq_c = wl.wq[:, cols]
    s_c = wl.s_w8a16[:, :, cols]
    y64 = odf.matmul_w8a16(xf, wq_c, s_c, out_dtype="float64")
    got = out16[torch.from_numpy(rows).to(dev)][:, torch.from_numpy(cols).to(dev)]
    print("w8a16", M, _check(got, y64, odf.abs_product_w8a16(xf, wq_c, s_c), wl.K))
    out8 = matmul_w8a8(torch.from_numpy(wl.xq).to(dev), torch.from_numpy(wl.sx).to(dev), pw,
                       torch.from_numpy(wl.sw).to(dev))
    # W8A8 oracle on the sampled rows / columns: per-column weight block scale
    sw_c = np.repeat(wl.sw, 128, axis=1)[:, cols]
    xv = E4M3_VALUES[wl.xq[rows]].astype(np.float64)
    wv = E4M3_VALUES[wq_c].astype(np.float64)
    y64 = np.zeros((len(rows), len(cols)))
    ap = np.zeros_like(y64)
    for kb in range(wl.K // 128):
        sl = slice(kb * 128, kb * 128 + 128)
        f = wl.sx[rows, kb][:, None].astype(np.float64) * sw_c[kb][None, :]
        y64 += (xv[:, sl] @ wv[sl]) * f
        ap += (np.abs(xv[:, sl]) @ np.abs(wv[sl])) * np.abs(f)
    got = out8[torch.from_numpy(rows).to(dev)][:, torch.from_numpy(cols).to(dev)]
    print("w8a8", M, _check(got, y64, ap, wl.K))


def test_dense_repeatable_and_prepack_equivalent(dev):
    from dw_tpu_amd.dense_fp8 import matmul, prepack_fp8
    from dw_tpu_amd.workloads import make_dense_workload
    wl = make_dense_workload(16, 1024, 512, seed=3)
    x = bf16_tensor(wl.x_bits, dev)
    w = torch.from_numpy(wl.wq).to(dev)
    s = torch.from_numpy(wl.s_w8a16).to(dev)
    a = matmul(x, w, s)
    b = matmul(x, prepack_fp8(w), s)
    c = matmul(x, w.view(torch.float8_e4m3fn), s)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(a.view(torch.int16), c.view(torch.int16))


def test_dense_full_size_exact_scaling(dev):
    """At M = 4096 (K=7168, N=4096): doubling the bf16 activations doubles the
    W8A16 output exactly (every product, partial sum and scale product scales
    by a power of two); doubling the W8A8 row scales does the same."""
    from dw_tpu_amd.dense_fp8 import matmul, matmul_w8a8, prepack_fp8
    from dw_tpu_amd.workloads import make_dense_workload
    wl = make_dense_workload(4096)
    pw = prepack_fp8(torch.from_numpy(wl.wq).to(dev))
    x = bf16_tensor(wl.x_bits, dev)
    s16 = torch.from_numpy(wl.s_w8a16).to(dev)
    a = matmul(x, pw, s16).float()
    b = matmul(x * 2, pw, s16).float()
    assert torch.equal(b, a * 2)
    xq, sx, sw = (torch.from_numpy(v).to(dev) for v in (wl.xq, wl.sx, wl.sw))
    a8 = matmul_w8a8(xq, sx, pw, sw).float()
    b8 = matmul_w8a8(xq, sx * 2, pw, sw).float()
    torch.cuda.synchronize()
    assert torch.equal(b8, a8 * 2)
