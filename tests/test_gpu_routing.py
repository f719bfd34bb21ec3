"""The router and dedupe_topk on the GPU (dwm_route_topk, dwm_dedupe_topk)
against oracle/moe.py: expert ids exact, weights within the f32 evaluation
error of exp / log1p / sqrt (the reference's score functions are not
vendored, so their last bits are unpinned), dedupe_topk bit-exact."""
import numpy as np
import pytest
import torch

from oracle import moe
from oracle.numerics import round_bf16

pytestmark = pytest.mark.gpu


def _check(dev, logits, k, score, renorm=False, bias=None, hash_ids=None, nvalid=None, in_dtype=torch.float32,
           w_dtype=torch.float32):
    from dw_tpu_amd import fused_moe_fp4_routing
    lt = torch.from_numpy(logits).to(dev).to(in_dtype)
    lf = lt.float().cpu().numpy()  # the values the kernel sees
    extra = {}
    if bias is not None:
        extra["e_score_correction_bias"] = torch.from_numpy(bias).to(dev)
    if hash_ids is not None:
        extra["hash_based_topk_indices"] = torch.from_numpy(hash_ids).to(dev)
    if nvalid is not None:
        extra["num_valid_tokens"] = nvalid
    w, ids = fused_moe_fp4_routing(lt, k, renorm, score, w_dtype, extra)
    assert not extra  # popped, as the reference does
    ww, wid = moe.route_topk(lf, k, renormalize=renorm, num_valid_tokens=nvalid, scoring_fn=score, bias=bias,
                             hash_ids=hash_ids)
    got_ids = ids.cpu().numpy()
    assert np.array_equal(got_ids, wid), np.argwhere(got_ids != wid)[:5]
    got = w.float().cpu().numpy()
    tol = 8e-7 * np.abs(ww) + 1e-30
    if w_dtype == torch.bfloat16:
        # one bf16 ulp: the f32 weights may straddle a rounding boundary
        tol = 2.0 ** -7 * np.abs(ww) + 1e-30
        ww = round_bf16(ww)
    assert (np.abs(got - ww) <= tol).all(), np.max(np.abs(got - ww) / np.maximum(np.abs(ww), 1e-30))


@pytest.mark.parametrize("E,k", [(32, 8), (256, 8), (384, 6), (1024, 16), (64, 64)])
@pytest.mark.parametrize("score", ["softmax", "sigmoid", "sqrtsoftplus"])
def test_route_topk_plain(dev, rng, E, k, score):
    logits = (rng.standard_normal((300, E)) * 2).astype(np.float32)
    _check(dev, logits, k, score)


@pytest.mark.parametrize("score", ["softmax", "sigmoid", "sqrtsoftplus"])
def test_route_topk_bias_renorm_mask(dev, rng, score):
    E, k = 256, 8
    logits = rng.standard_normal((513, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    _check(dev, logits, k, score, renorm=True, bias=bias, nvalid=400)
    _check(dev, logits, k, score, renorm=False, bias=bias, nvalid=0)


def test_route_topk_hash_and_dtypes(dev, rng):
    E, k = 128, 6
    logits = rng.standard_normal((257, E)).astype(np.float32)
    hid = rng.integers(0, E, (257, k)).astype(np.int32)
    _check(dev, logits, k, "sqrtsoftplus", renorm=True, hash_ids=hid)
    _check(dev, logits, k, "softmax", in_dtype=torch.bfloat16, w_dtype=torch.bfloat16)
    _check(dev, logits, k, "sigmoid", renorm=True, in_dtype=torch.bfloat16, w_dtype=torch.bfloat16, nvalid=100)


def test_route_topk_ties_go_to_the_lower_expert(dev):
    logits = np.zeros((8, 64), np.float32)
    logits[:, 40] = 1.0
    logits[:, 7] = 1.0
    _check(dev, logits, 4, "softmax")  # 7, 40, then 0, 1 among the equal rest


@pytest.mark.parametrize("score", ["softmax", "sqrtsoftplus"])
def test_route_topk_approx_branch(dev, rng, score):
    """MOE_APPROX_TOPK (0901-...:671-675): after hash routing, before the
    bias, so a correction bias is popped but not applied; the exact top-k of
    the unbiased scores (a valid approx_max_k result for any recall target).
    Hash routing still takes precedence."""
    from dw_tpu_amd import fused_moe_fp4_routing
    E, k, T = 256, 8, 300
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.5).astype(np.float32)
    lt = torch.from_numpy(logits).to(dev)
    bt = torch.from_numpy(bias).to(dev)
    extra = {"e_score_correction_bias": bt}
    w, ids = fused_moe_fp4_routing(lt, k, True, score, torch.float32, extra, approx_topk=True, recall_target=0.9)
    assert not extra
    w0, ids0 = fused_moe_fp4_routing(lt, k, True, score, torch.float32, {})
    assert torch.equal(ids, ids0) and torch.equal(w, w0)
    ww, wid = moe.route_topk(logits, k, renormalize=True, scoring_fn=score)
    assert np.array_equal(ids.cpu().numpy(), wid)
    wb, idb = fused_moe_fp4_routing(lt, k, True, score, torch.float32, {"e_score_correction_bias": bt})
    assert not torch.equal(idb, ids)  # the bias does change the exact branch's choice here
    hid = torch.from_numpy(rng.integers(0, E, (T, k)).astype(np.int32)).to(dev)
    wh, idh = fused_moe_fp4_routing(lt, k, True, score, torch.float32, {"hash_based_topk_indices": hid},
                                    approx_topk=True)
    assert torch.equal(idh, hid)


@pytest.mark.parametrize("k,E", [(8, 256), (8, 12), (6, 6), (3, 2), (64, 300)])
def test_dedupe_topk_bit_exact(dev, rng, k, E):
    from dw_tpu_amd import dedupe_topk
    ids = rng.integers(0, min(E, 5), (333, k)).astype(np.int32)
    w = rng.random((333, k)).astype(np.float32)
    w[0, 0] = -0.0
    gw, gi = dedupe_topk(torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev), E)
    ww, wi = moe.dedupe_topk(w, ids, E)
    assert np.array_equal(gi.cpu().numpy(), wi)
    assert np.array_equal(gw.cpu().numpy().view(np.uint32), ww.view(np.uint32))
