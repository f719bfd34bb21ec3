"""Pins the oracle's gmm, dispatch, combine, requantization and dense FP8
math with brute force, closed forms, invariants and the reference's own
exactness tests.  CPU only, small shapes."""
import numpy as np
import pytest

from oracle import dense_fp8, fp4, gmm, moe, quant
from oracle.numerics import E4M3_VALUES, round_bf16, to_e4m3


# --------------------------------------------------------------------------- gmm

def _tiny_gmm_case(rng, sizes, K=64, N=32):
    E = len(sizes)
    M = int(sum(sizes))
    lhs = round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    nib = rng.integers(0, 16, (E, K, N), dtype=np.uint8)
    codes = fp4.e2m1_to_codes(nib)
    exps = rng.integers(-4, 3, (E, K // 32, 1, N))
    scale = np.ldexp(np.float32(1), exps).astype(np.float32)
    return lhs, nib, codes, exps, scale, np.array(sizes, np.int32)


def test_gmm_matches_triple_loop(rng):
    lhs, nib, codes, exps, scale, gs = _tiny_gmm_case(rng, [3, 0, 5, 2], K=64, N=8)
    out, written = gmm.gmm(lhs, codes, scale, gs, out_dtype="float64")
    # brute force straight from the e2m1 table and 2^exponent, row by row
    row = 0
    for g, sz in enumerate(gs):
        for r in range(row, row + sz):
            for n in range(8):
                acc = 0.0
                for k in range(64):
                    acc += float(lhs[r, k]) * float(fp4.E2M1_VALUES[nib[g, k, n]]) * 2.0 ** exps[g, k // 32, 0, n]
                assert out[r, n] == pytest.approx(acc, rel=1e-12, abs=1e-12)
        row += sz
    assert written.all()


def test_gmm_group_offset_and_unwritten_rows(rng):
    lhs, nib, codes, exps, scale, gs = _tiny_gmm_case(rng, [2, 3, 4, 1])
    # local experts are groups 1..2: rows 2..8 written, rows 0,1,9 not
    out, written = gmm.gmm(lhs, codes[1:3], scale[1:3], gs, group_offset=1, zero_initialize=True)
    assert list(np.nonzero(written)[0]) == list(range(2, 9))
    assert np.all(out[~written] == 0)
    full, _ = gmm.gmm(lhs, codes, scale, gs)
    assert np.array_equal(out[written], full[written])
    out2, _ = gmm.gmm(lhs, codes[1:3], scale[1:3], gs, group_offset=1, zero_initialize=False)
    assert np.isnan(out2[~written]).all()


def test_gmm_groups_are_independent_and_row_permutation_equivariant(rng):
    lhs, nib, codes, exps, scale, gs = _tiny_gmm_case(rng, [4, 6])
    out, _ = gmm.gmm(lhs, codes, scale, gs, out_dtype="float64")
    p = np.r_[rng.permutation(4), 4 + rng.permutation(6)]
    outp, _ = gmm.gmm(lhs[p], codes, scale, gs, out_dtype="float64")
    assert np.allclose(outp, out[p], rtol=1e-14, atol=0)
    # changing expert 0's weights leaves group 1's rows bit-identical
    codes2 = codes.copy()
    codes2[0] = fp4.e2m1_to_codes(rng.integers(0, 16, codes[0].shape, dtype=np.uint8))
    out2, _ = gmm.gmm(lhs, codes2, scale, gs, out_dtype="float64")
    assert np.array_equal(out2[4:], out[4:])


def test_gmm_error_bound_accepts_f32_and_rejects_planted_mistakes(rng):
    K, N = 256, 64
    lhs, nib, codes, exps, scale, gs = _tiny_gmm_case(rng, [40, 0, 24], K=K, N=N)
    w = gmm.dequant_rhs(codes, scale)
    y64, written = gmm.gmm(lhs, None, None, gs, out_dtype="float64", w=w)
    absprod = gmm.abs_product(lhs, w, gs)
    bound = gmm.error_bound(y64, absprod, K)
    y32, _ = gmm.gmm(lhs, None, None, gs, accumulate="f32", w=w)
    assert np.all(np.abs(y32 - y64) <= bound)
    # planted: drop the block scale of one K block of expert 2 (a dropped term)
    s_bad = scale.copy()
    s_bad[2, 3] = 1.0
    y_bad, _ = gmm.gmm(lhs, codes, s_bad, gs)
    assert np.any(np.abs(y_bad - y64) > bound)
    # planted: transposed nibble order within a byte (a swapped index)
    w_swap = gmm.dequant_rhs(codes[..., ::-1].copy(), scale[..., ::-1].copy())[..., ::-1]
    y_swap, _ = gmm.gmm(lhs, None, None, gs, w=np.ascontiguousarray(w_swap[:, :, ::-1]))
    assert np.any(np.abs(y_swap - y64) > bound)
    # planted: wrong sign of the decoded codes
    y_neg, _ = gmm.gmm(lhs, None, None, gs, w=-w)
    assert np.any(np.abs(y_neg - y64) > bound)


def test_gmm_seq32_is_the_sequential_f32_sum(rng):
    lhs, nib, codes, exps, scale, gs = _tiny_gmm_case(rng, [3, 0, 2], K=64, N=4)
    w = gmm.dequant_rhs(codes, scale)
    ys, _ = gmm.gmm(lhs, None, None, gs, out_dtype="float64", accumulate="seq32", w=w)
    # per element, an explicit f32 running sum in k order (bit for bit)
    starts = gmm.group_starts(gs)
    for g, sz in enumerate(gs):
        for r in range(starts[g], starts[g] + sz):
            for n in range(4):
                acc = np.float32(0)
                for k in range(64):
                    acc = np.float32(acc + np.float32(lhs[r, k] * w[g, k, n]))
                assert ys[r, n] == float(acc)
    # and within the sequential-summation bound (K - 1) u sum|a w| of float64
    K = 1024
    lhs, nib, codes, exps, scale, gs = _tiny_gmm_case(rng, [17, 9], K=K, N=16)
    w = gmm.dequant_rhs(codes, scale)
    ys, _ = gmm.gmm(lhs, None, None, gs, out_dtype="float64", accumulate="seq32", w=w)
    y64, _ = gmm.gmm(lhs, None, None, gs, out_dtype="float64", w=w)
    ap = gmm.abs_product(lhs, w, gs)
    assert np.all(np.abs(ys - y64) <= (K - 1) * 2.0 ** -24 * ap)
    assert np.any(ys != y64)  # it does round


def test_w4a16_rows_and_sampling_match_the_full_product():
    """The sampled W4A16 reference (used for the MX mode's distance) is the
    full float64 gmm's rows and columns; the sample has the first, last and
    one more row of every non-empty group, and columns 0 and N - 1."""
    from dw_tpu_amd.workloads import make_gmm_workload
    from oracle.numerics import bf16_to_f32
    wl = make_gmm_workload("cpu_plumbing")
    rows, cols = gmm.sample_rows_cols(wl.group_sizes, wl.N, np.random.default_rng(3), ncols=20)
    starts = np.concatenate([[0], np.cumsum(wl.group_sizes)])
    for s0, g in zip(starts[:-1], wl.group_sizes):
        if g > 0:
            assert s0 in rows and s0 + g - 1 in rows
    assert cols[0] == 0 and cols[-1] == wl.N - 1
    full, _ = gmm.gmm(bf16_to_f32(wl.lhs_bits), fp4.e2m1_to_codes(fp4.unpack_nibbles(wl.rhs_e2m1)),
                      fp4.e8m0_decode(wl.scale_codes), wl.group_sizes, out_dtype="float64")
    got = gmm.w4a16_rows(wl.lhs_bits[rows], wl.rhs_e2m1, wl.scale_codes, wl.group_sizes, rows, cols)
    np.testing.assert_allclose(got, full[np.ix_(rows, cols)], rtol=1e-13, atol=1e-9)


def test_gmm_acceptance_policy(rng):
    K = 512
    lhs, nib, codes, exps, scale, gs = _tiny_gmm_case(rng, [40, 24], K=K, N=32)
    w = gmm.dequant_rhs(codes, scale)
    y64, _ = gmm.gmm(lhs, None, None, gs, out_dtype="float64", w=w)
    ys, _ = gmm.gmm(lhs, None, None, gs, out_dtype="float32", accumulate="seq32", w=w)
    yb, _ = gmm.gmm(lhs, None, None, gs, out_dtype="float32", accumulate="f32", w=w)
    ok, st = gmm.acceptance_policy(ys, ys, y64)
    assert ok and st["rms"] == st["rms_base"]
    ok, _ = gmm.acceptance_policy(yb, ys, y64)  # a blocked BLAS sum is at least as accurate
    assert ok
    # planted: a 4-ulp-scale perturbation of every element fails it
    bad = (ys.astype(np.float64) + 4 * np.abs(ys - y64).max()).astype(np.float32)
    ok, _ = gmm.acceptance_policy(bad, ys, y64)
    assert not ok


# ---------------------------------------------------------------------- dispatch

@pytest.mark.parametrize("T,topk,E", [(1, 1, 1), (5, 2, 3), (64, 2, 8), (37, 8, 32), (300, 6, 256)])
def test_dispatch_matches_brute_force(rng, T, topk, E):
    ids = rng.integers(0, E, (T, topk)).astype(np.int32)
    perm, tok, rev, gs, off = moe.dispatch(ids, E)
    flat = ids.reshape(-1)
    brute = sorted(range(flat.size), key=lambda j: (flat[j], j))  # stable by construction
    assert list(perm) == brute
    # moe_fast_dispatch.py:18-19 identity
    assert np.array_equal(tok, np.arange(T).repeat(topk)[perm])
    assert np.array_equal(perm[rev], np.arange(flat.size))
    assert np.array_equal(gs, [int((flat == e).sum()) for e in range(E)])
    assert off[0] == 0 and off[-1] == flat.size and np.array_equal(np.diff(off), gs)
    # rows of each group are contiguous and in increasing (token, slot) order
    for e in range(E):
        seg = perm[off[e]:off[e + 1]]
        assert np.all(flat[seg] == e) and np.all(np.diff(seg) > 0)


def test_gather_rows_jax_index_semantics():
    h = np.arange(12, dtype=np.float32).reshape(6, 2)
    got = moe.gather_rows(h, np.array([0, 5, -1, -6, 7, -9]))
    assert np.array_equal(got[:, 0], [0, 10, 10, 0, 10, 0])


def test_combine_matches_scalar_loop(rng):
    T, topk, H = 7, 3, 5
    x = round_bf16(rng.standard_normal((T * topk, H)).astype(np.float32) * 3)
    idx = rng.permutation(T * topk).astype(np.int32)
    w = rng.random((T, topk)).astype(np.float32)
    got = moe.combine(x, idx, w, topk, out_dtype="float32")
    for t in range(T):
        for h in range(H):
            acc = np.float32(0.0)
            for k in range(topk):
                acc = np.float32(acc + np.float32(x[idx[t * topk + k], h] * w[t, k]))
            assert got[t, h] == acc
    # the summation order is part of the definition: k = 0, 1, 2 left to right
    x2 = np.array([[1.0], [2.0 ** -24], [2.0 ** -24]], np.float32)
    w2 = np.ones((1, 3), np.float32)
    fwd = moe.combine(x2, np.array([0, 1, 2]), w2, 3, out_dtype="float32")
    late = moe.combine(x2, np.array([1, 2, 0]), w2, 3, out_dtype="float32")
    assert fwd[0, 0] == 1.0  # each 2^-24 is half an ulp of 1.0: ties to even
    assert late[0, 0] == np.float32(1.0 + 2.0 ** -23)


def test_combine_zero_start_sign():
    # sum starts from +0.0: a single -0.0 product yields +0.0
    x = np.array([[-0.0]], np.float32)
    out = moe.combine(x, np.array([0]), np.ones((1, 1), np.float32), 1, out_dtype="float32")
    assert out[0, 0] == 0.0 and not np.signbit(out[0, 0])


def test_route_topk_tie_break_and_mask():
    logits = np.array([[1.0, 3.0, 3.0, 0.0], [0.0, 0.0, 0.0, 0.0]], np.float32)
    w, ids = moe.route_topk(logits, 2)
    assert ids[0].tolist() == [1, 2] and ids[1].tolist() == [0, 1]
    w, ids = moe.route_topk(logits, 2, num_valid_tokens=1)
    assert ids[1].tolist() == [0, 0] and np.all(w[1] == 0)
    w, _ = moe.route_topk(logits, 2, renormalize=True)
    assert np.allclose(w.sum(-1), 1.0)


# ------------------------------------------------------------ requantization

def test_pow2_requant_reproduces_mxfp4_exactly(rng):
    # patches/tpu-inference/0001-...:131-157, restated with numpy draws:
    # random e2m1 codes + e8m0 exponents in [-20, 5) per 32-block.
    shape = (4, 64, 256)
    nib = rng.integers(0, 16, shape, dtype=np.uint8)
    values = fp4.E2M1_VALUES[nib]
    exps = rng.integers(-20, 5, shape[:-1] + (shape[-1] // 32,))
    scale = np.ldexp(np.float32(1), exps).astype(np.float32)
    original = (values.reshape(*shape[:-1], -1, 32) * scale[..., None]).reshape(shape)
    q, s = quant.quantize_tensor_pow2(original, "e2m1", -1, 32)
    rt = quant.dequantize(q, s, "e2m1", -1, 32)
    assert np.array_equal(rt, original)
    # the default absmax scale (not rounded to a power of two) is not exact
    xb = original.reshape(*shape[:-1], -1, 32)
    s_abs = (np.abs(xb).max(-1, keepdims=True) / np.float32(6.0)).astype(np.float32)
    q_abs = quant.to_e2m1(xb / np.where(s_abs == 0, 1, s_abs))
    lossy = (fp4.E2M1_VALUES[q_abs] * s_abs).reshape(shape)
    assert not np.all(lossy == original)


def test_pow2_requant_fp8_128x128_to_1x128_exactly(rng):
    # patches/tpu-inference/0001-...:110-130: 128x128 ue8m0 blocks requantized
    # to 1x128 blocks along K round-trip exactly.
    K, N = 512, 384
    wq = to_e4m3(rng.standard_normal((K, N)).astype(np.float32))
    exps = rng.integers(-12, 0, (K // 128, N // 128))
    s = np.ldexp(np.float32(1), exps).astype(np.float32)
    original = E4M3_VALUES[wq] * np.repeat(np.repeat(s, 128, 0), 128, 1)
    q, s2 = quant.quantize_tensor_pow2(original, "e4m3", 0, 128)
    assert s2.shape == (K // 128, N)
    rt = quant.dequantize(q, s2, "e4m3", 0, 128)
    assert np.array_equal(rt, original)


def test_pow2_ceil_closed_form():
    s = np.array([0.5, 0.75, 1.0, 1.0000001, 3.0, 1e-30, 0.0, -2.0], np.float32)
    got = quant.pow2_ceil(s)
    want = [0.5, 1.0, 1.0, 2.0, 4.0, 2.0 ** np.ceil(np.log2(1e-30)), 0.0, -2.0]
    assert np.allclose(got, np.array(want, np.float32), rtol=0, atol=0)


def test_act_quant_reference_cases(rng):
    # fp8_fake_quant reference (0001-...:47-56): an all-zero row stays zero
    # (amax floor 1e-4), the result is idempotent, rope channels untouched.
    x = (rng.standard_normal((37, 512)) * 3).astype(np.float32)
    x[3] = 0
    x = round_bf16(x)
    y = quant.act_quant_ue8m0(x, 64, 448)
    assert np.all(y[3] == 0)
    assert np.array_equal(y[:, 448:], x[:, 448:])
    assert np.array_equal(quant.act_quant_ue8m0(y, 64, 448), y)
    rel = np.abs(y[:, :448] - x[:, :448]) / np.maximum(np.abs(x[:, :448]), 1e-30)
    big = np.abs(x[:, :448]) > np.abs(x[:, :448]).max() / 64
    assert rel[big].max() <= 2.0 ** -4


# ------------------------------------------------------------------- dense fp8

def test_dense_w8a16_brute_force(rng):
    M, K, N = 3, 256, 4
    x = round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    wq = to_e4m3(rng.standard_normal((K, N)).astype(np.float32))
    s = rng.random((K // 128, 1, N)).astype(np.float32)
    got = dense_fp8.matmul_w8a16(x, wq, s, out_dtype="float64")
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for kb in range(K // 128):
                part = sum(float(x[m, k]) * float(E4M3_VALUES[wq[k, n]]) for k in range(kb * 128, kb * 128 + 128))
                acc += part * float(s[kb, 0, n])
            assert got[m, n] == pytest.approx(acc, rel=1e-12)


def test_dense_w8a8_brute_force(rng):
    M, K, N = 2, 256, 256
    xq = to_e4m3(rng.standard_normal((M, K)).astype(np.float32))
    wq = to_e4m3(rng.standard_normal((K, N)).astype(np.float32))
    sx = rng.random((M, K // 128)).astype(np.float32)
    sw = rng.random((K // 128, N // 128)).astype(np.float32)
    got = dense_fp8.matmul_w8a8(xq, sx, wq, sw, out_dtype="float64")
    for m in range(M):
        for n in (0, 127, 128, 255):
            acc = 0.0
            for kb in range(2):
                part = sum(float(E4M3_VALUES[xq[m, k]]) * float(E4M3_VALUES[wq[k, n]])
                           for k in range(kb * 128, kb * 128 + 128))
                acc += part * float(sx[m, kb]) * float(sw[kb, n // 128])
            assert got[m, n] == pytest.approx(acc, rel=1e-12)


def _e4m3_code(v):
    return int(np.flatnonzero(E4M3_VALUES == v)[0])


@pytest.mark.parametrize("w,s,want", [
    (1.125, 1.0078125, 1.1328125),   # 1.1337890625 = 145.125 ulps of 2^-7: rounds down
    (1.5, 1.0078125, 1.515625),      # 1.51171875 = 193.5 ulps: a tie, to the even 194
    (1.75, 1.0078125, 1.765625),     # 1.763671875 = 225.75 ulps: rounds up
    (1.5, 1.005859375, 1.515625),    # the scale rounds to bf16 first (1 + 2^-7), then the tie
    (-3.0, 0.3, -0.90234375),        # bf16(0.3) = 0.30078125; -0.90234375 = -231 ulps of 2^-8: exact
    (448.0, 2.0 ** -10, 0.4375),     # power-of-two scales are exact
])
def test_dense_pre_weight_rounding_hand_cases(w, s, want):
    """The "pre" weight bf16(w * bf16(s)) on hand-computed cases: round to
    nearest even after an exact product, and the scale rounded to bf16
    before the product (the fourth case gives 1.5078125 if it is not)."""
    codes = np.zeros((128, 1), np.uint8)
    codes[5, 0] = _e4m3_code(w)
    got = dense_fp8.pre_weight(codes, np.full((1, 1, 1), s, np.float32))
    assert got[5, 0] == want
    assert np.all(np.delete(got[:, 0], 5) == 0.0)


def test_dense_pre_equals_native_for_power_of_two_scales(rng):
    """With power-of-two scales the pre rounding is exact, so "pre" and the
    native per-block scaling are the same sum (float64, up to summation
    order); the scale is per (128-deep K block, column), not transposed."""
    M, K, N = 4, 384, 40
    x = round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    wq = to_e4m3(rng.standard_normal((K, N)).astype(np.float32))
    s = np.ldexp(np.float32(1), rng.integers(-6, 4, (K // 128, 1, N))).astype(np.float32)
    pre = dense_fp8.matmul_pre(x, wq, s, out_dtype="float64")
    nat = dense_fp8.matmul_w8a16(x, wq, s, out_dtype="float64")
    np.testing.assert_allclose(pre, nat, rtol=1e-12, atol=1e-12)
    # a planted mistake -- the scale indexed by (column, K block) -- is caught
    bad = dense_fp8.matmul_pre(x, wq, s.reshape(N, 1, K // 128).transpose(2, 1, 0).copy()[::-1], out_dtype="float64")
    assert not np.allclose(bad, nat, rtol=1e-6)


def test_block_quantizers_bound_and_shape(rng):
    w = rng.standard_normal((256, 384)).astype(np.float32)
    q, s = quant.quantize_fp8_blocks(w)
    assert s.shape == (2, 3)
    deq = E4M3_VALUES[q] * np.repeat(np.repeat(s, 128, 0), 128, 1)
    assert np.all(np.abs(deq - w) <= np.abs(w) * 2 ** -4 + np.repeat(np.repeat(s, 128, 0), 128, 1) * 2 ** -9)
    xq, sx = quant.quantize_fp8_rows(w)
    assert sx.shape == (256, 3)
