"""MoE dispatch, row gather and combine on the GPU: bit-exact against the
oracle (indices, group sizes / offsets, gathered rows, combined rows)."""
import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from oracle import moe
from oracle.numerics import bf16_bits as to_bf16_bits, bf16_to_f32

pytestmark = pytest.mark.gpu


def _dispatch(dev, ids, E, check=False):
    from dw_tpu_amd import moe_dispatch
    d = moe_dispatch(torch.from_numpy(ids).to(dev), E, check=check)
    return [t.cpu().numpy() for t in d]


# Batches of up to 8192 ids take a one-block kernel (with at most 63
# experts the register-count kernel, E = 63 and a ragged last round here;
# with more the LDS-histogram one, E = 64 here), larger ones the
# three-launch path: both sides of each boundary are covered.  In the
# three-launch path the scan splits the chunk counters into runs per expert
# column (E + 1 <= 512 columns: 2 .. 1024 runs), or walks whole columns
# (E = 1024: more columns than the scan's threads).
@pytest.mark.parametrize("T,topk,E", [(1, 1, 1), (3, 2, 8), (64, 2, 8), (256, 8, 32), (512, 8, 32),
                                      (1000, 6, 256), (8192, 8, 32), (130, 8, 1024), (4096, 1, 3),
                                      (1024, 8, 1024), (8192, 1, 5), (8193, 1, 7), (2731, 3, 64),
                                      (2048, 8, 1024), (16384, 8, 256), (65536, 8, 32), (9000, 1, 1),
                                      (1000, 5, 63), (700, 8, 64), (1, 7, 2), (8191, 1, 1)])
def test_dispatch_bit_exact(dev, rng, T, topk, E):
    ids = rng.integers(0, E, (T, topk)).astype(np.int32)
    got = _dispatch(dev, ids, E)
    want = moe.dispatch(ids, E)
    for g, w, name in zip(got, want, ["perm", "tok_sorted", "revert", "group_sizes", "group_offsets"]):
        assert np.array_equal(g, w), name


@pytest.mark.parametrize("name", ["cpu_plumbing", "decode_gate_up", "decode_down", "prefill"])
def test_dispatch_workload_routing(dev, name):
    from dw_tpu_amd.workloads import make_gmm_workload
    wl = make_gmm_workload(name, with_data=False)
    got = _dispatch(dev, wl.topk_ids, wl.E)
    want = moe.dispatch(wl.topk_ids, wl.E)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)
    assert np.array_equal(got[3], wl.group_sizes)


def test_dispatch_skewed_and_invalid_ids(dev, rng):
    ids = np.zeros((700, 4), np.int32)  # every id equal: one group of 2800
    got = _dispatch(dev, ids, 16)
    want = moe.dispatch(ids, 16)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)
    bad = rng.integers(0, 8, (50, 2)).astype(np.int32)
    bad[7, 1] = 8
    bad[20, 0] = -1
    with pytest.raises(ValueError, match="outside"):
        _dispatch(dev, bad, 8, check=True)
    perm, tok, rev, gs, off = _dispatch(dev, bad, 8)
    valid = (bad.reshape(-1) >= 0) & (bad.reshape(-1) < 8)
    assert gs.sum() == valid.sum() and off[-1] == valid.sum()
    assert set(perm[off[-1]:]) == set(np.nonzero(~valid)[0])  # invalid ids last
    assert np.array_equal(perm[rev], np.arange(bad.size))
    # the same on the three-launch path (more than 8192 ids): invalid ids sort
    # as one extra key E after every valid one, stably
    big = rng.integers(0, 8, (3000, 3)).astype(np.int32)
    big[5, 2], big[2999, 0], big[1500, 1] = 8, -3, 100
    got = _dispatch(dev, big, 8)
    perm, tok, rev, gs, off = moe.dispatch(np.where((big >= 0) & (big < 8), big, 8), 9)
    for g, w in zip(got, (perm, tok, rev, gs[:8], off[:9])):
        assert np.array_equal(g, w)


@pytest.mark.parametrize("T,H,dtype", [(64, 1024, torch.bfloat16), (513, 7168, torch.bfloat16),
                                       (10, 100, torch.bfloat16), (33, 96, torch.float32), (7, 3, torch.bfloat16)])
def test_row_gather_bitwise(dev, rng, T, H, dtype):
    from dw_tpu_amd import row_gather
    src = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(dtype).to(dev)
    idx = rng.integers(-T, 2 * T, 3 * T).astype(np.int32)  # includes negative and out-of-range
    got = row_gather(src, torch.from_numpy(idx).to(dev)).cpu()
    want = moe.gather_rows(src.cpu().float().numpy(), idx)
    assert np.array_equal(got.float().numpy(), want)


@pytest.mark.parametrize("T,topk,H", [(64, 8, 1024), (513, 3, 7168), (10, 2, 100), (7, 5, 3)])
def test_dispatch_gather_floor_div_bitwise(dev, rng, T, topk, H):
    """fast_dispatch_gather computes argsort // topk inside the gather
    (moe_fast_dispatch.py:41-44, 188-194): floor division, then JAX gather
    index semantics, for any argsort values (negative and past T * topk
    included) and unaligned rows."""
    from dw_tpu_amd import fast_dispatch_gather
    src = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16).to(dev)
    idx = rng.integers(-2 * T * topk, 2 * T * topk, 3 * T * topk).astype(np.int32)
    got = fast_dispatch_gather(src, torch.from_numpy(idx).to(dev), topk).cpu()
    want = moe.gather_rows(src.cpu().float().numpy(), np.floor_divide(idx, topk))
    assert np.array_equal(got.float().numpy(), want)


def test_fast_dispatch_gather_workload(dev):
    from dw_tpu_amd import fast_dispatch_gather, moe_dispatch
    from dw_tpu_amd.workloads import make_gmm_workload
    wl = make_gmm_workload("decode_down")
    rng = np.random.Generator(np.random.PCG64(5))
    hidden_bits = to_bf16_bits(rng.standard_normal((wl.T, wl.K)).astype(np.float32))
    hidden = bf16_tensor(hidden_bits, dev)
    d = moe_dispatch(torch.from_numpy(wl.topk_ids).to(dev), wl.E)
    x = fast_dispatch_gather(hidden, d.topk_argsort_indices, wl.topk)
    want = hidden_bits[d.token_indices_sorted.cpu().numpy()]
    assert np.array_equal(bf16_bits(x), want)


@pytest.mark.parametrize("T,topk,H", [(512, 8, 7168), (64, 2, 512), (5, 3, 100), (1, 1, 8), (300, 6, 4096)])
@pytest.mark.parametrize("x_dtype,w_dtype,out_dtype", [
    (torch.bfloat16, torch.float32, torch.bfloat16),
    (torch.bfloat16, torch.bfloat16, torch.bfloat16),
    (torch.float32, torch.float32, torch.float32),
    (torch.bfloat16, torch.float32, torch.float32),
])
def test_combine_bit_exact(dev, rng, T, topk, H, x_dtype, w_dtype, out_dtype):
    from dw_tpu_amd import fast_combine
    x = torch.from_numpy((rng.standard_normal((T * topk, H)) * 4).astype(np.float32)).to(x_dtype)
    idx = rng.permutation(T * topk).astype(np.int32)
    w = torch.from_numpy(rng.random((T, topk)).astype(np.float32)).to(w_dtype)
    got = fast_combine(x.to(dev), torch.from_numpy(idx).to(dev), w.to(dev), topk, out_dtype=out_dtype).cpu()
    want = moe.combine(x.float().numpy(), idx, w.float().numpy(), topk,
                       out_dtype="bfloat16" if out_dtype == torch.bfloat16 else "float32")
    g = got.float().numpy()
    assert np.array_equal(g, want)
    assert np.array_equal(np.signbit(g), np.signbit(want))


def test_dispatch_gmm_combine_pipeline(dev):
    """decode_down: dispatch -> gather -> gmm -> combine, with the combine
    bit-exact to the oracle applied to the GPU's own gmm output, and the
    dispatch indices bit-exact."""
    from dw_tpu_amd import fast_combine, fast_dispatch_gather, fp4_weight_to_codes, gmm_wrapper, moe_dispatch
    from dw_tpu_amd.workloads import make_gmm_workload
    wl = make_gmm_workload("decode_down", scale_m=0.25)
    rng = np.random.Generator(np.random.PCG64(9))
    hidden_bits = to_bf16_bits(rng.standard_normal((wl.T, wl.K)).astype(np.float32))
    hidden = bf16_tensor(hidden_bits, dev)
    ids = torch.from_numpy(wl.topk_ids).to(dev)
    d = moe_dispatch(ids, wl.E)
    x = fast_dispatch_gather(hidden, d.topk_argsort_indices, wl.topk)
    pw = fp4_weight_to_codes(torch.from_numpy(wl.rhs_e2m1).to(dev), torch.from_numpy(wl.scale_codes).to(dev))
    y = gmm_wrapper(x, pw, None, None, d.group_sizes, None)
    out = fast_combine(y, d.topk_argsort_revert_indices, torch.from_numpy(wl.topk_weights).to(dev), wl.topk)
    torch.cuda.synchronize()
    want = moe.combine(bf16_to_f32(bf16_bits(y)), d.topk_argsort_revert_indices.cpu().numpy(), wl.topk_weights,
                       wl.topk)
    assert np.array_equal(bf16_to_f32(bf16_bits(out)), want)
