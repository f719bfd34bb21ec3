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
from oracle.numerics import bf16_bits as f32_to_bf16_bits

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


_M, _K, _N = 160, 2048, 512  # 2 x 4 MFMA tiles: the default plan splits K 16 ways


@pytest.mark.parametrize("tile,plan", [
    (None, (2, 128, 128, 16, 3)),                            # the library's plan
    (("native", 256, 2048, 128, 2), (2, 256, 128, 1, 2)),    # one 256-row tile per column tile, no split
    (("native", 128, 512, 128, 4), (2, 128, 128, 4, 4)),     # 4 K runs, 4-stage ring
    (("native", 128, 512, 128, 3), (2, 128, 128, 4, 3)),     # 4 K runs, 3-stage ring
    (("megablox", 64, 1024, 128, 2), (3, 64, 128, 2, 2)),    # the general tiled kernel, 2 K runs
    (("megablox", 16, 2048, 64, 2), (3, 16, 64, 1, 2)),
])
def test_w8a16_tile_choice_is_launched(dev, tile, plan):
    """A tile given to matmul is the launch the library makes (its plan read
    back from the library), and every plan stays within the dense bound."""
    from dw_tpu_amd.dense_fp8 import last_plan, matmul
    from dw_tpu_amd.dense_fp8_tiles import DenseTile
    from dw_tpu_amd.workloads import make_dense_workload
    wl = make_dense_workload(_M, _K, _N, seed=81)
    x = bf16_tensor(wl.x_bits, dev)
    w = torch.from_numpy(wl.wq).to(dev).view(torch.float8_e4m3fn)
    s = torch.from_numpy(wl.s_w8a16).to(dev)
    if tile is None:
        out = matmul(x, w, s)
    else:
        t = DenseTile(*tile)
        out = matmul(x, w, s, mode=t.mode, tm=t.tm, tk=t.tk, tn=t.tn, stages=t.stages)
    torch.cuda.synchronize()
    assert last_plan().astuple() == plan
    xf = bf16_to_f32(wl.x_bits)
    y64 = odf.matmul_w8a16(xf, wl.wq, wl.s_w8a16, out_dtype="float64")
    print(tile, _check(out, y64, odf.abs_product_w8a16(xf, wl.wq, wl.s_w8a16), _K))


@pytest.mark.parametrize("tk", [1024, 512, 384, 128])  # 2, 4, 6 (runs of 3, 3, 3, 3, 3, 1) and 16 K runs
def test_w8a16_ring_depth_keeps_bits(dev, tk):
    """With the same K runs, the ring depth only reschedules the same
    products: 2, 3 and 4 stages give the same bits, through the split-K sum
    in run order (this grid is small: the sum issues the loads of 2, 4 or 8
    runs at a time, the last chunk of 6 and 16 runs partly past the end)."""
    from dw_tpu_amd.dense_fp8 import last_plan, matmul
    from dw_tpu_amd.workloads import make_dense_workload
    wl = make_dense_workload(_M, _K, _N, seed=84)
    x = bf16_tensor(wl.x_bits, dev)
    w = torch.from_numpy(wl.wq).to(dev).view(torch.float8_e4m3fn)
    s = torch.from_numpy(wl.s_w8a16).to(dev)
    runs = -(-(_K // 128) // (tk // 128))
    outs = []
    for stages in (2, 3, 4):
        outs.append(matmul(x, w, s, mode="native", tm=128, tk=tk, tn=128, stages=stages))
        torch.cuda.synchronize()
        assert last_plan().astuple() == (2, 128, 128, runs, stages)
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
    xf = bf16_to_f32(wl.x_bits)
    _check(outs[0], odf.matmul_w8a16(xf, wl.wq, wl.s_w8a16, out_dtype="float64"),
           odf.abs_product_w8a16(xf, wl.wq, wl.s_w8a16), _K)


def test_override_file_steers_try_dense_fp8(dev, tmp_path, monkeypatch):
    """An entry of the DSV4_DENSE_FP8_TILES file changes what try_dense_fp8
    launches (dense_fp8.py:115-163 with dense_fp8_tiles.py:52-58); a
    "baseline" entry returns None."""
    import json
    from dw_tpu_amd import dense_fp8_tiles as tiles
    from dw_tpu_amd.dense_fp8 import last_plan, try_dense_fp8
    from dw_tpu_amd.workloads import make_dense_workload
    p = tmp_path / "tiles.json"
    p.write_text(json.dumps({"version": 1, "device": tiles.DEVICE, "entries": [
        {"m": _M, "k": _K, "n": _N, "mode": "native", "tm": 256, "tk": 1024, "tn": 128, "stages": 3},
        {"m": _M + 1, "k": _K, "n": _N, "mode": "baseline"}]}))
    monkeypatch.setenv(tiles.ENV_VAR, str(p))
    tiles._read.cache_clear()
    try:
        wl = make_dense_workload(_M, _K, _N, seed=82)
        w = torch.from_numpy(wl.wq).to(dev).view(torch.float8_e4m3fn)
        s = torch.from_numpy(wl.s_w8a16).to(dev).reshape(_K // 128, 1, _N)
        out = try_dense_fp8(bf16_tensor(wl.x_bits, dev), w, s)
        torch.cuda.synchronize()
        assert out is not None and last_plan().astuple() == (2, 256, 128, 2, 3)
        xf = bf16_to_f32(wl.x_bits)
        _check(out, odf.matmul_w8a16(xf, wl.wq, wl.s_w8a16, out_dtype="float64"),
               odf.abs_product_w8a16(xf, wl.wq, wl.s_w8a16), _K)
        x1 = torch.zeros((_M + 1, _K), dtype=torch.bfloat16, device=dev)
        assert try_dense_fp8(x1, w, s) is None
    finally:
        monkeypatch.delenv(tiles.ENV_VAR)
        tiles._read.cache_clear()


@pytest.mark.parametrize("tile,plan", [
    (None, (2, 128, 128, 16, 4)),
    (("native", 128, 1024, 128, 3), (2, 128, 128, 2, 3)),
    (("native", 256, 2048, 128, 3), (2, 256, 128, 1, 3)),
])
def test_w8a8_tile_choice_is_launched(dev, tile, plan):
    from dw_tpu_amd.dense_fp8 import last_plan, matmul_w8a8
    from dw_tpu_amd.dense_fp8_tiles import DenseTile
    from dw_tpu_amd.workloads import make_dense_workload
    wl = make_dense_workload(_M, _K, _N, seed=83)
    out = matmul_w8a8(torch.from_numpy(wl.xq).to(dev), torch.from_numpy(wl.sx).to(dev),
                      torch.from_numpy(wl.wq).to(dev), torch.from_numpy(wl.sw).to(dev),
                      tile=None if tile is None else DenseTile(*tile))
    torch.cuda.synchronize()
    assert last_plan().astuple() == plan
    y64 = odf.matmul_w8a8(wl.xq, wl.sx, wl.wq, wl.sw, out_dtype="float64")
    print(tile, _check(out, y64, odf.abs_product_w8a8(wl.xq, wl.sx, wl.wq, wl.sw), _K))


def _dense_inputs(dev, M, K, N, seed):
    from dw_tpu_amd.workloads import make_dense_workload
    wl = make_dense_workload(M, K, N, seed=seed)
    x = bf16_tensor(wl.x_bits, dev)
    w = torch.from_numpy(wl.wq).to(dev).view(torch.float8_e4m3fn)
    return wl, x, w


def test_same_math_modes_are_bitwise_equal(dev):
    """"wide", "flipped" and "megablox" compute the native arithmetic
    (reference dense_fp8.py:1-5, 33-53): the same launch, the same bits."""
    from dw_tpu_amd.dense_fp8 import matmul
    for M in (4, 128):
        wl, x, w = _dense_inputs(dev, M, 1024, 512, 81)
        s = torch.from_numpy(wl.s_w8a16).to(dev)
        ref = bf16_bits(matmul(x, w, s))
        for mode in ("wide", "flipped", "megablox"):
            assert np.array_equal(bf16_bits(matmul(x, w, s, mode=mode)), ref), (M, mode)


@pytest.mark.parametrize("M,tile", [(16, ("native", 16, 1024, 1024)),     # the reference's defaults
                                    (4, ("native", 4, 1024, 2048)),       # _TUNED entries
                                    (512, ("megablox", 128, 1024, 2048))])
def test_reference_tiles_take_the_library_plan_with_a_warning(dev, M, tile):
    """A tile of the reference's TPU tables names no launch here: matmul warns
    and runs the library's own plan, with the same bits."""
    from dw_tpu_amd.dense_fp8 import matmul
    wl, x, w = _dense_inputs(dev, M, 2048, 4096, 82)
    s = torch.from_numpy(wl.s_w8a16).to(dev)
    mode, tm, tk, tn = tile
    with pytest.warns(UserWarning, match="names no launch"):
        got = matmul(x, w, s, mode=mode, tm=tm, tk=tk, tn=tn)
    assert np.array_equal(bf16_bits(got), bf16_bits(matmul(x, w, s)))


@pytest.mark.parametrize("M,K,N", [(1, 1024, 512), (17, 512, 256), (64, 1024, 384), (128, 1024, 512),
                                   (300, 768, 4096)])
def test_pre_mode_against_oracle(dev, M, K, N):
    """mode="pre" (reference dense_fp8.py:33-43): x @ bf16(w * bf16(s)) in
    f32 against the float64 oracle of the same rounding, within the stated
    dense bound (computed on the pre weights)."""
    from dw_tpu_amd.dense_fp8 import matmul
    wl, x, w = _dense_inputs(dev, M, K, N, 83)
    out = matmul(x, w, torch.from_numpy(wl.s_w8a16).to(dev), mode="pre")
    xf = bf16_to_f32(wl.x_bits)
    y64 = odf.matmul_pre(xf, wl.wq, wl.s_w8a16, out_dtype="float64")
    ap = np.abs(xf.astype(np.float64)) @ np.abs(odf.pre_weight(wl.wq, wl.s_w8a16).astype(np.float64))
    print(M, K, N, _check(out, y64, ap, K))


def test_pre_mode_products_bit_exact(dev):
    """One-hot activation rows make each output element a single rounded
    product: y[m, n] = bf16(w[k_m, n] * bf16(s[k_m // 128, n])) bit for bit
    (random non-power-of-two scales, every K block and column)."""
    from dw_tpu_amd.dense_fp8 import matmul
    M, K, N = 96, 1024, 256
    wl, _, w = _dense_inputs(dev, M, K, N, 84)
    rng = np.random.default_rng(85)
    s = (rng.random((K // 128, 1, N)) * 3.0 + 0.01).astype(np.float32)
    ks = rng.integers(0, K, M)
    x = np.zeros((M, K), np.float32)
    x[np.arange(M), ks] = 1.0
    out = matmul(bf16_tensor(f32_to_bf16_bits(x), dev), w, torch.from_numpy(s).to(dev), mode="pre")
    want = odf.pre_weight(wl.wq, s)[ks]
    assert np.array_equal(bf16_to_f32(bf16_bits(out)), want)


def test_pre_mode_power_of_two_scales_equal_native_on_its_plan(dev):
    """With power-of-two scales every pre product is exact, so "pre" and the
    native scaling on the same launch plan give the same bits."""
    from dw_tpu_amd.dense_fp8 import last_plan, matmul
    from dw_tpu_amd.dense_fp8_tiles import plan_to_tile
    rng = np.random.default_rng(86)
    for M, K, N in ((16, 1024, 512), (200, 2048, 384)):
        wl, x, w = _dense_inputs(dev, M, K, N, 87)
        s = torch.from_numpy(np.ldexp(np.float32(1), rng.integers(-8, 3, (K // 128, 1, N))).astype(np.float32)).to(dev)
        pre = bf16_bits(matmul(x, w, s, mode="pre"))
        t = plan_to_tile(last_plan(), K)
        nat = bf16_bits(matmul(x, w, s, mode=t.mode, tm=t.tm, tk=t.tk, tn=t.tn, stages=t.stages))
        assert np.array_equal(pre, nat), (M, K, N, t)


@pytest.mark.parametrize("w8a8", [False, True])
def test_dense_timeline_build_same_bits(dev, w8a8):
    """The timeline build (libdwtpu_moe_timeline.so, what bench.py --probe
    dense_steps loads) runs the dense MFMA kernel with per-wave cycle sums
    compiled in: the same output bits as the library (8 K runs, split-K
    reduce included), one record per wave of every block, each wave's step
    count that of its K run (W8A16 two 64-deep steps per 128-deep K block,
    W8A8 one), and its phases within its own entry-to-exit cycles."""
    import ctypes
    import os
    from dw_tpu_amd import _lib
    from dw_tpu_amd.dense_fp8 import last_plan, matmul, matmul_w8a8, prepack_fp8
    from dw_tpu_amd.dense_fp8_tiles import DenseTile
    from dw_tpu_amd.workloads import make_dense_workload
    tl = ctypes.CDLL(os.path.join(os.path.dirname(_lib.LIB_PATH), "libdwtpu_moe_timeline.so"))
    for n in ("dwm_dense_fp8_w8a16_plan", "dwm_dense_fp8_w8a8_plan"):
        getattr(tl, n).argtypes = _lib.SIGNATURES[n]
    tl.dwm_dense_steps_set.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    M, K, N = 128, 2048, 1024  # 8 column tiles x 8 K runs of 2 K blocks: 64 blocks
    wl = make_dense_workload(M, K, N, seed=85)
    pw = prepack_fp8(torch.from_numpy(wl.wq).to(dev))
    x = bf16_tensor(wl.x_bits, dev)
    xq, sx, sw = (torch.from_numpy(v).to(dev) for v in (wl.xq, wl.sx, wl.sw))
    s16 = torch.from_numpy(wl.s_w8a16.reshape(K // 128, N)).to(dev)
    plan = _lib.DensePlan(2, 128, 128, 8, 4 if w8a8 else 3)
    if w8a8:
        y = matmul_w8a8(xq, sx, pw, sw, tile=DenseTile("native", 128, 256, 128, 4))
    else:
        y = matmul(x, pw, torch.from_numpy(wl.s_w8a16).to(dev), mode="native", tm=128, tk=256, tn=128, stages=3)
    torch.cuda.synchronize()
    assert last_plan().astuple() == plan.astuple()
    out = torch.empty_like(y)
    ws = torch.empty(8 * M * N * 4, dtype=torch.uint8, device=dev)
    waves, slots = 16 * 64, 10
    buf = torch.zeros(waves * slots, dtype=torch.int64, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    assert tl.dwm_dense_steps_set(P(buf), waves) == 0
    if w8a8:
        rc = tl.dwm_dense_fp8_w8a8_plan(P(xq), P(sx), M, K, N, P(pw.weight), P(sw), P(out), ctypes.byref(plan),
                                        P(ws), ws.numel(), _lib.stream_handle(dev))
    else:
        rc = tl.dwm_dense_fp8_w8a16_plan(P(x), M, K, N, P(pw.weight), P(s16), P(out), ctypes.byref(plan), P(ws),
                                         ws.numel(), _lib.stream_handle(dev))
    torch.cuda.synchronize()
    assert tl.dwm_dense_steps_set(None, 0) == 0
    assert rc == 0
    assert torch.equal(out.view(torch.int16), y.view(torch.int16))
    d = buf.view(waves, slots).cpu().numpy().astype(np.int64)
    per_block = 4 if w8a8 else 8
    live = d[:, 8] != 0
    assert live.sum() == 64 * per_block
    assert np.all((np.arange(waves) % 16)[live] < per_block)
    d = d[live]
    assert np.all(d[:, 5] == (2 if w8a8 else 4))
    assert np.all(d[:, 0] + d[:, 1] + d[:, 2] + d[:, 3] + d[:, 4] <= d[:, 9])
    assert np.all(d[:, 7] < d[:, 8])
