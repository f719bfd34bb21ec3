"""Seeded random shapes for the dense FP8 GEMM on the GPU, against the
float64 oracle under the stated bound (oracle.dense_fp8.error_bound).

The cases vary the launch the library plans (section "Launch plans" of
csrc/dense_fp8.hip): M <= 16 takes the skinny kernel; N % 128 != 0 the
tiled kernel; otherwise the MFMA tile kernel, whose K split (and so the
split-K sum in run order, its loads 1, 2, 4 or 8 runs at a time) follows
from the tile count and K.  W8A16 runs every case; W8A8 the cases whose N is
a multiple of 128 (its weight scales are 128 x 128 blocks)."""
import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from oracle import dense_fp8 as odf
from oracle import gmm as ogmm
from oracle.numerics import bf16_to_f32

pytestmark = pytest.mark.gpu


def _case(seed):
    r = np.random.default_rng(2000 + seed)
    if seed % 4 == 0:
        M = int(r.integers(1, 17))
    elif seed % 4 == 1:
        M = int(r.integers(17, 129))
    else:
        M = int(r.integers(17, 401))
    K = 128 * int(r.integers(1, 17))
    N = 16 * int(r.integers(1, 65)) if seed % 3 == 0 else 128 * int(r.integers(1, 9))
    return M, K, N


def _check(out, y64, ap, K):
    y = bf16_to_f32(bf16_bits(out)).astype(np.float64)
    bound = odf.error_bound(y64, ap, K)
    err = np.abs(y - y64)
    assert np.all(np.isfinite(y))
    assert np.all(err <= bound), float((err / np.maximum(bound, 1e-300)).max())
    return ogmm.error_stats(y, y64)


@pytest.mark.parametrize("seed", range(24))
def test_dense_random_shapes(dev, seed):
    from dw_tpu_amd.dense_fp8 import last_plan, matmul, matmul_w8a8
    from dw_tpu_amd.workloads import make_dense_workload
    M, K, N = _case(seed)
    wl = make_dense_workload(M, K, N, seed=90 + seed)
    x = bf16_tensor(wl.x_bits, dev)
    w = torch.from_numpy(wl.wq).to(dev).view(torch.float8_e4m3fn)
    out16 = matmul(x, w, torch.from_numpy(wl.s_w8a16).to(dev))
    torch.cuda.synchronize()
    plan16 = last_plan().astuple()
    xf = bf16_to_f32(wl.x_bits)
    st16 = _check(out16, odf.matmul_w8a16(xf, wl.wq, wl.s_w8a16, out_dtype="float64"),
                  odf.abs_product_w8a16(xf, wl.wq, wl.s_w8a16), K)
    print(seed, (M, K, N), "w8a16 plan", plan16, st16, flush=True)
    if N % 128:
        return
    out8 = matmul_w8a8(torch.from_numpy(wl.xq).to(dev), torch.from_numpy(wl.sx).to(dev),
                       torch.from_numpy(wl.wq).to(dev), torch.from_numpy(wl.sw).to(dev))
    torch.cuda.synchronize()
    plan8 = last_plan().astuple()
    st8 = _check(out8, odf.matmul_w8a8(wl.xq, wl.sx, wl.wq, wl.sw, out_dtype="float64"),
                 odf.abs_product_w8a8(wl.xq, wl.sx, wl.wq, wl.sw), K)
    print(seed, (M, K, N), "w8a8 plan", plan8, st8, flush=True)
