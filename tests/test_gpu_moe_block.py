"""The expert block on the GPU: gmm1 with the fused silu_and_mul_with_clamp
activation against the float64 oracle, and the whole block (dispatch ->
gather -> gmm1 + act -> gmm2 -> combine) checked stage by stage on the
kernel's own intermediates.

Stated tolerance of the fused activation output (oracle.moe_block):
    |h - act(acc64)| <= 2^-8 (|act64| + p) + p + 2^-20 |act64|,
    p = act_error_bound(acc64, K 2^-24 sum_k |a_k w_k|)
the gmm1 f32 accumulation bound propagated through clip and silu (whose
slope is below 1.1), plus bf16 rounding and the f32 evaluation of silu.
gmm2 uses the gmm bound on the exact bf16 activation it was given; dispatch,
gather and combine are bit-exact."""
import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from oracle import fp4, gmm, moe
from oracle import moe_block as omb
from oracle.numerics import bf16_bits as np_bf16_bits
from oracle.numerics import bf16_to_f32

pytestmark = pytest.mark.gpu


def _weights(rng, E, K, N, lo=121, hi=130):
    rhs = rng.integers(0, 256, (E, K, N // 2), dtype=np.uint8)
    sc = rng.integers(lo, hi, (E, K // 32, 1, N), dtype=np.uint8)
    return rhs, sc


def _dequant(rhs, sc, cols=None):
    n = rhs.shape[2] * 2
    cols = np.arange(n) if cols is None else np.asarray(cols)
    b = rhs[:, :, cols // 2]
    nib = np.where(cols % 2 == 1, b >> 4, b & 0xF).astype(np.uint8)
    return gmm.dequant_rhs(fp4.e2m1_to_codes(nib), fp4.e8m0_decode(sc[..., cols]))


def _check_act(h, lhs_f32, w_gu, gs, K, out_kind="bfloat16", rows=None):
    """h [M, I] from the kernel vs the oracle activation of lhs @ w_gu (w_gu [E, K, 2I])."""
    acc64, written = gmm.gmm(lhs_f32, None, None, gs, out_dtype="float64", w=w_gu)
    ap = gmm.abs_product(lhs_f32, w_gu, gs)
    acc_err = K * 2.0 ** -24 * ap
    act64 = omb.silu_and_mul_clamp(acc64)
    bound = omb.act_output_bound(act64, omb.act_error_bound(acc64, acc_err))
    if out_kind == "bfloat16":
        y = bf16_to_f32(bf16_bits(h)).astype(np.float64)
    else:
        y = h.cpu().numpy().astype(np.float64)
    sel = written if rows is None else rows
    err = np.abs(y[sel] - act64[sel])
    assert np.all(np.isfinite(y[sel]))
    assert np.all(err <= bound[sel]), float((err / np.maximum(bound[sel], 1e-300)).max())
    clamped = float(np.mean(np.abs(acc64[sel]) > omb.SWIGLU_LIMIT))
    return gmm.error_stats(y[sel], act64[sel]), clamped


@pytest.mark.parametrize("sizes,K,I", [([5, 0, 33, 64, 97], 256, 64), ([1, 130, 0, 17], 512, 96),
                                       ([200, 3], 1024, 32)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_fused_gmm1_activation(dev, rng, sizes, K, I, out_dtype):
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2
    E, N, M = len(sizes), 2 * I, sum(sizes)
    lhs_bits = np_bf16_bits(rng.standard_normal((M, K), dtype=np.float32))
    rhs, sc = _weights(rng, E, K, N)
    w = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev), gate_up=True)
    g = torch.tensor(sizes, dtype=torch.int32, device=dev)
    h = gmm_v2(bf16_tensor(lhs_bits, dev), w, g, fuse_act="silu_and_mul_with_clamp",
               preferred_element_type=out_dtype)
    assert tuple(h.shape) == (M, I)
    stats, clamped = _check_act(h, bf16_to_f32(lhs_bits), _dequant(rhs, sc), np.asarray(sizes), K,
                                "bfloat16" if out_dtype == torch.bfloat16 else "float32")
    assert 0.05 < clamped < 0.95  # both sides of the swiglu limit are exercised
    print(sizes, K, I, stats, clamped)


def test_fused_needs_gate_up_weights(dev, rng):
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2
    rhs, sc = _weights(rng, 2, 128, 64)
    g = torch.tensor([3, 4], dtype=torch.int32, device=dev)
    x = bf16_tensor(np_bf16_bits(rng.standard_normal((7, 128), dtype=np.float32)), dev)
    plain = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev))
    gu = fp4_weight_to_codes(torch.from_numpy(rhs).to(dev), torch.from_numpy(sc).to(dev), gate_up=True)
    with pytest.raises(ValueError):
        gmm_v2(x, plain, g, fuse_act="silu_and_mul_with_clamp")
    with pytest.raises(ValueError):
        gmm_v2(x, gu, g)


def _block_case(rng, T, E, topk, H, I, empty=()):
    logits = rng.standard_normal((T, E)).astype(np.float32)
    for e in empty:
        logits[:, e] = -np.inf
    p = moe.softmax_f32(logits)
    wts, ids = moe.top_k(p, topk)
    hidden_bits = np_bf16_bits(rng.standard_normal((T, H), dtype=np.float32))
    w13 = _weights(rng, E, H, 2 * I)
    w2 = _weights(rng, E, I, H, lo=118, hi=124)
    return ids.astype(np.int32), wts.astype(np.float32), hidden_bits, w13, w2


@pytest.mark.parametrize("f32_reduce", [False, True])
def test_moe_block_stagewise(dev, rng, f32_reduce):
    from dw_tpu_amd import fp4_weight_to_codes, moe_block
    T, E, topk, H, I = 64, 8, 2, 256, 128
    ids, wts, hidden_bits, (r13, s13), (r2, s2) = _block_case(rng, T, E, topk, H, I, empty=(5,))
    w13 = fp4_weight_to_codes(torch.from_numpy(r13).to(dev), torch.from_numpy(s13).to(dev), gate_up=True)
    w2 = fp4_weight_to_codes(torch.from_numpy(r2).to(dev), torch.from_numpy(s2).to(dev))
    hidden = bf16_tensor(hidden_bits, dev)
    r = moe_block(hidden, torch.from_numpy(ids).to(dev), torch.from_numpy(wts).to(dev), w13, w2, E,
                  f32_reduce=f32_reduce, return_intermediates=True)
    torch.cuda.synchronize()
    # dispatch and gather: bit-exact
    perm, tok, rev, gs, _ = moe.dispatch(ids, E)
    assert np.array_equal(r.dispatch.group_sizes.cpu().numpy(), gs)
    assert np.array_equal(r.dispatch.token_indices_sorted.cpu().numpy(), tok)
    assert np.array_equal(bf16_bits(r.x), hidden_bits[tok])
    # gmm1 + activation within the stated bound
    stats, _ = _check_act(r.h, bf16_to_f32(hidden_bits[tok]), _dequant(r13, s13), gs, H)
    # gmm2 on the kernel's exact bf16 activation within the gmm bound
    h_f32 = bf16_to_f32(bf16_bits(r.h))
    w2f = _dequant(r2, s2)
    y64, _ = gmm.gmm(h_f32, None, None, gs, out_dtype="float64", w=w2f)
    ap = gmm.abs_product(h_f32, w2f, gs)
    kind = "float32" if f32_reduce else "bfloat16"
    y = r.y.cpu().numpy().astype(np.float64) if f32_reduce else bf16_to_f32(bf16_bits(r.y)).astype(np.float64)
    assert np.all(np.abs(y - y64) <= gmm.error_bound(y64, ap, I, kind))
    # combine of the kernel's gmm2 output: bit-exact
    want = moe.combine(y.astype(np.float32), rev, wts, topk, out_dtype="bfloat16")
    assert np.array_equal(bf16_bits(r.out), np_bf16_bits(want))
    print(stats)


@pytest.mark.parametrize("f32_reduce", [False, True])
@pytest.mark.parametrize("fmt", ["e4m3", "e2m1"])
def test_moe_block_mx_stagewise(dev, rng, f32_reduce, fmt):
    """The block in the MX modes (lhs_quant_dtype=float8_e4m3fn, or
    float4_e2m1fn: MXFP4): dispatch and combine bit-exact; gmm1 + activation
    on the quantized hidden rows and gmm2 on the quantized activation, each
    within the MX bound (oracle.gmm.mx_error_bound propagated through the
    activation)."""
    from dw_tpu_amd import fp4_weight_to_codes, moe_block
    from oracle import quant
    qdt = torch.float8_e4m3fn if fmt == "e4m3" else "float4_e2m1fn"

    def mxq(x):  # the oracle's quantize-dequantize of the chosen format
        if fmt == "e4m3":
            return quant.mx_dequantize(*quant.mx_quantize_e4m3(x))
        return quant.mx_dequantize_e2m1(*quant.mx_quantize_e2m1(x))
    T, E, topk, H, I = 64, 8, 2, 256, 128
    ids, wts, hidden_bits, (r13, s13), (r2, s2) = _block_case(rng, T, E, topk, H, I, empty=(2,))
    w13 = fp4_weight_to_codes(torch.from_numpy(r13).to(dev), torch.from_numpy(s13).to(dev), gate_up=True)
    w2 = fp4_weight_to_codes(torch.from_numpy(r2).to(dev), torch.from_numpy(s2).to(dev))
    r = moe_block(bf16_tensor(hidden_bits, dev), torch.from_numpy(ids).to(dev), torch.from_numpy(wts).to(dev), w13,
                  w2, E, f32_reduce=f32_reduce, return_intermediates=True, lhs_quant_dtype=qdt)
    torch.cuda.synchronize()
    perm, tok, rev, gs, _ = moe.dispatch(ids, E)
    assert np.array_equal(r.dispatch.group_sizes.cpu().numpy(), gs)
    # gmm1: the quantized hidden rows, gathered
    a = mxq(bf16_to_f32(hidden_bits))[tok]
    w13f = _dequant(r13, s13)
    acc64, _ = gmm.gmm(a, None, None, gs, out_dtype="float64", w=w13f)
    acc_err = H * 2.0 ** -24 * gmm.abs_product(a, w13f, gs) + gmm.MX_BLOCK_TERM * gmm.block_max_product(a, w13f, gs)
    h = bf16_to_f32(bf16_bits(r.h)).astype(np.float64)
    err = np.abs(h - omb.apply_act(acc64, "silu_and_mul_with_clamp"))
    assert np.all(err <= omb.act_bound(acc64, acc_err, "silu_and_mul_with_clamp"))
    # gmm2: the kernel's activation, quantized
    hq = mxq(bf16_to_f32(bf16_bits(r.h)))
    w2f = _dequant(r2, s2)
    y64, _ = gmm.gmm(hq, None, None, gs, out_dtype="float64", w=w2f)
    kind = "float32" if f32_reduce else "bfloat16"
    bound = gmm.mx_error_bound(y64, gmm.abs_product(hq, w2f, gs), gmm.block_max_product(hq, w2f, gs), I, kind)
    y = r.y.cpu().numpy().astype(np.float64) if f32_reduce else bf16_to_f32(bf16_bits(r.y)).astype(np.float64)
    assert np.all(np.abs(y - y64) <= bound)
    want = moe.combine(y.astype(np.float32), rev, wts, topk, out_dtype="bfloat16")
    assert np.array_equal(bf16_bits(r.out), np_bf16_bits(want))


def test_moe_block_mx_graph_replays_equal_eager(dev, rng):
    """MoeBlockGraph in the MX mode: every replay (with eager work and
    synchronisations between) gives the eager block's bits."""
    from dw_tpu_amd import MoeBlockGraph, fp4_weight_to_codes, moe_block
    T, E, topk, H, I = 48, 8, 2, 256, 128
    ids, wts, hidden_bits, (r13, s13), (r2, s2) = _block_case(rng, T, E, topk, H, I)
    w13 = fp4_weight_to_codes(torch.from_numpy(r13).to(dev), torch.from_numpy(s13).to(dev), gate_up=True)
    w2 = fp4_weight_to_codes(torch.from_numpy(r2).to(dev), torch.from_numpy(s2).to(dev))
    args = (bf16_tensor(hidden_bits, dev), torch.from_numpy(ids).to(dev), torch.from_numpy(wts).to(dev))
    g = MoeBlockGraph(*args, w13, w2, E, lhs_quant_dtype=torch.float8_e4m3fn)
    for _ in range(3):
        want = moe_block(*args, w13, w2, E, lhs_quant_dtype=torch.float8_e4m3fn)
        torch.cuda.synchronize()
        got = g(*args).clone()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_moe_block_decode_size_sampled(dev, rng):
    """Real decode shapes (256 tokens x top-8, 32 experts, H=7168, I=2048):
    gmm1 + activation and gmm2 on sampled rows and columns, combine exact."""
    from dw_tpu_amd import fp4_weight_to_codes, moe_block
    T, E, topk, H, I = 256, 32, 8, 7168, 2048
    ids, wts, hidden_bits, (r13, s13), (r2, s2) = _block_case(rng, T, E, topk, H, I, empty=(3, 11))
    w13 = fp4_weight_to_codes(torch.from_numpy(r13).to(dev), torch.from_numpy(s13).to(dev), gate_up=True)
    w2 = fp4_weight_to_codes(torch.from_numpy(r2).to(dev), torch.from_numpy(s2).to(dev))
    r = moe_block(bf16_tensor(hidden_bits, dev), torch.from_numpy(ids).to(dev), torch.from_numpy(wts).to(dev),
                  w13, w2, E, return_intermediates=True)
    torch.cuda.synchronize()
    perm, tok, rev, gs, _ = moe.dispatch(ids, E)
    starts = gmm.group_starts(gs)
    rows = np.unique(np.concatenate([[s, s + n - 1] for s, n in zip(starts, gs) if n > 0]))
    cols = rng.choice(I, 24, replace=False)
    # gmm1 + act on sampled rows x cols (gate column c and up column I + c)
    x = bf16_to_f32(hidden_bits[tok])
    wg = _dequant(r13, s13, np.concatenate([cols, I + cols]))
    h = bf16_to_f32(bf16_bits(r.h))[:, cols]
    sub = np.zeros(h.shape[0], bool)
    sub[rows] = True
    acc64, _ = gmm.gmm(x, None, None, gs, out_dtype="float64", w=wg)
    ap = gmm.abs_product(x, wg, gs)
    act64 = omb.silu_and_mul_clamp(acc64)
    bound = omb.act_output_bound(act64, omb.act_error_bound(acc64, H * 2.0 ** -24 * ap))
    assert np.all(np.abs(h[sub] - act64[sub]) <= bound[sub])
    # gmm2 on the kernel's activation, sampled columns
    hc = bf16_to_f32(bf16_bits(r.h))
    c2 = rng.choice(H, 24, replace=False)
    w2f = _dequant(r2, s2, c2)
    y64, _ = gmm.gmm(hc, None, None, gs, out_dtype="float64", w=w2f)
    y = bf16_to_f32(bf16_bits(r.y))[:, c2].astype(np.float64)
    assert np.all(np.abs(y - y64) <= gmm.error_bound(y64, gmm.abs_product(hc, w2f, gs), I, "bfloat16"))
    # combine: exact on the kernel's gmm2 output (all columns)
    want = moe.combine(bf16_to_f32(bf16_bits(r.y)), rev, wts, topk, out_dtype="bfloat16")
    assert np.array_equal(bf16_bits(r.out), np_bf16_bits(want))


def test_moe_block_graph_replays_match_eager(dev, rng):
    """The captured block, replayed several times with new inputs and eager
    work (and synchronisations) in between, gives the eager block's bits
    every time."""
    from dw_tpu_amd import MoeBlockGraph, fp4_weight_to_codes, moe_block
    T, E, topk, H, I = 64, 8, 2, 256, 128
    ids, wts, hidden_bits, (r13, s13), (r2, s2) = _block_case(rng, T, E, topk, H, I, empty=(3,))
    w13 = fp4_weight_to_codes(torch.from_numpy(r13).to(dev), torch.from_numpy(s13).to(dev), gate_up=True)
    w2 = fp4_weight_to_codes(torch.from_numpy(r2).to(dev), torch.from_numpy(s2).to(dev))
    g = MoeBlockGraph(bf16_tensor(hidden_bits, dev), torch.from_numpy(ids).to(dev), torch.from_numpy(wts).to(dev),
                      w13, w2, E)
    for rep in range(4):
        ids_r, wts_r, hb_r, _, _ = _block_case(rng, T, E, topk, H, I, empty=(rep % E,))
        hidden, tid, tw = bf16_tensor(hb_r, dev), torch.from_numpy(ids_r).to(dev), torch.from_numpy(wts_r).to(dev)
        want = moe_block(hidden, tid, tw, w13, w2, E)
        torch.cuda.synchronize()
        got = g(hidden, tid, tw).clone()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), rep
        # eager work between replays
        moe_block(hidden, tid, tw, w13, w2, E)
        torch.cuda.synchronize()


def test_moe_block_graph_with_group_offset(dev, rng):
    """An expert-parallel shard (group_offset as an int) captured and replayed."""
    from dw_tpu_amd import MoeBlockGraph, fp4_weight_to_codes, moe_block
    T, E, topk, H, I = 48, 8, 2, 256, 128
    ids, wts, hidden_bits, (r13, s13), (r2, s2) = _block_case(rng, T, E, topk, H, I)
    lo, hi = 2, 6  # this shard's experts
    w13 = fp4_weight_to_codes(torch.from_numpy(r13[lo:hi]).to(dev), torch.from_numpy(s13[lo:hi]).to(dev),
                              gate_up=True)
    w2 = fp4_weight_to_codes(torch.from_numpy(r2[lo:hi]).to(dev), torch.from_numpy(s2[lo:hi]).to(dev))
    hidden, tid, tw = bf16_tensor(hidden_bits, dev), torch.from_numpy(ids).to(dev), torch.from_numpy(wts).to(dev)
    want = moe_block(hidden, tid, tw, w13, w2, E, group_offset=lo)
    g = MoeBlockGraph(hidden, tid, tw, w13, w2, E, group_offset=lo)
    for _ in range(3):
        got = g().clone()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
