"""MoE routing, dispatch permutation, row gather and combine -- numpy restatement.

Test infrastructure only (see oracle/__init__.py).

Reference files restated here:
* patches/tpu-inference-experimental/fused-moe-fp4/0901-...:656-687
  (_fused_moe_fp4_routing: top-k routing "exactly as fused_moe_func")
* 0901-...:98-121 (dedupe_topk)
* patches/tpu-inference-ext/0101-...:131 (top-k weights cast to the hidden dtype)
* patches/tpu-inference-ext/0405-moe-fast-dispatch.patch:70-98 (argsort,
  token_indices_sorted, group_sizes via one_hot(...).sum(0), row gather)
* kernels/tpu_inference/layers/common/moe_fast_dispatch.py:14-44, 188-194
* kernels/tpu_inference/layers/common/moe_fast_combine.py:14-54
"""
import numpy as np

from .numerics import round_bf16


def softmax_f32(logits: np.ndarray) -> np.ndarray:
    """exp(x - max) / sum(exp(x - max)) along the last axis, in f32."""
    x = np.asarray(logits, np.float32)
    z = np.exp(x - x.max(axis=-1, keepdims=True))
    return (z / z.sum(axis=-1, keepdims=True)).astype(np.float32)


def top_k(x: np.ndarray, k: int):
    """Largest k along the last axis, descending; ties keep the lower index
    first (lax.top_k)."""
    order = np.argsort(-np.asarray(x), axis=-1, kind="stable")[..., :k]
    return np.take_along_axis(x, order, axis=-1), order.astype(np.int32)


def scoring(logits: np.ndarray, scoring_fn: str) -> np.ndarray:
    """Router scores in f32 along the last axis (apply_scoring_fn, called at
    0901-...:667; its body is not vendored, so these are the functions'
    definitions): "softmax" exp(x - max) / sum; "sigmoid" 1 / (1 + exp(-x));
    "sqrtsoftplus" sqrt(log(1 + exp(x))), the DeepSeek V4 router score
    (0901-...:176, :517 name it), with softplus in its overflow-free form
    max(x, 0) + log1p(exp(-|x|))."""
    x = np.asarray(logits, np.float32)
    if scoring_fn == "softmax":
        return softmax_f32(x)
    if scoring_fn == "sigmoid":
        return (np.float32(1) / (np.float32(1) + np.exp(-x))).astype(np.float32)
    if scoring_fn == "sqrtsoftplus":
        sp = (np.maximum(x, np.float32(0)) + np.log1p(np.exp(-np.abs(x)))).astype(np.float32)
        return np.sqrt(sp).astype(np.float32)
    raise ValueError(f"unknown scoring_fn {scoring_fn!r}")


def route_topk(logits, topk: int, renormalize: bool = False, num_valid_tokens=None,
               weight_dtype: str = "float32", scoring_fn: str = "softmax", bias=None, hash_ids=None):
    """scoring -> (hash ids | top_k of score + bias | top_k) -> optional
    renormalize -> invalid-token mask -> cast (0901-...:656-687).

    With ``bias`` (e_score_correction_bias) the experts are chosen on
    score + bias and weighted by the unbiased score; with ``hash_ids``
    (hash_based_topk_indices) the experts are given and weighted by their
    scores.  Invalid tokens get expert 0 and weight 0 (0901-...:682-686).
    The renormalizing sum runs over k in order.
    """
    p = scoring(logits, scoring_fn)
    if hash_ids is not None:
        ids = np.asarray(hash_ids, np.int32)
        w = np.take_along_axis(p, ids, axis=-1)
    elif bias is not None:
        _, ids = top_k((p + np.asarray(bias, np.float32)[None, :]).astype(np.float32), topk)
        w = np.take_along_axis(p, ids, axis=-1)
    else:
        w, ids = top_k(p, topk)
    w = w.astype(np.float32)
    if renormalize:
        tot = np.zeros(w.shape[:-1] + (1,), np.float32)
        for j in range(w.shape[-1]):
            tot = (tot + w[..., j:j + 1]).astype(np.float32)
        w = (w / tot).astype(np.float32)
    if num_valid_tokens is not None:
        valid = (np.arange(w.shape[0]) < num_valid_tokens)[:, None]
        ids = np.where(valid, ids, 0).astype(np.int32)
        w = np.where(valid, w, 0.0).astype(np.float32)
    if weight_dtype == "bfloat16":
        w = round_bf16(w)
    return w.astype(np.float32), ids.astype(np.int32)


def dedupe_topk(topk_weights, topk_ids, num_experts: int):
    """Makes each token's expert ids distinct (0901-...:98-121): for
    j = 1 .. topk-1, a repeat of an earlier id adds its weight (f32) to the
    first occurrence and is re-pointed at the first candidate in
    arange(min(2 topk, E)) that no column of the token currently holds
    (candidate 0 when all are held), with weight 0.  The add runs for every
    token (adding +0.0 when there is no repeat), as the reference's
    scatter-add does."""
    w = np.asarray(topk_weights, np.float32).copy()
    ids = np.asarray(topk_ids, np.int32).copy()
    topk = ids.shape[-1]
    cand = np.arange(min(2 * topk, num_experts), dtype=np.int32)
    rows = np.arange(w.shape[0])
    for j in range(1, topk):
        same = ids[:, :j] == ids[:, j:j + 1]
        dup = same.any(axis=-1)
        first = np.argmax(same, axis=-1)
        add = np.where(dup, w[:, j], np.float32(0)).astype(np.float32)
        w[rows, first] = (w[rows, first] + add).astype(np.float32)
        used = (ids[:, :, None] == cand[None, None, :]).any(axis=1)
        free = cand[np.argmin(used, axis=-1)]
        ids[:, j] = np.where(dup, free, ids[:, j])
        w[:, j] = np.where(dup, np.float32(0), w[:, j])
    return w, ids


def dispatch(topk_ids: np.ndarray, num_experts: int):
    """Expert-sorted dispatch indices for topk_ids [T, topk].

    * perm = stable argsort of the flattened ids (0405-...:73; jnp.argsort
      is stable, so equal experts keep increasing j = t * topk + k);
    * tok_sorted = perm // topk (moe_fast_dispatch.py:41-44, equal to
      arange(T).repeat(topk)[perm], :18-19);
    * revert = inverse permutation of perm (the combine's indices,
      moe_fast_combine.py:14-22): perm[revert[j]] == j;
    * group_sizes = bincount(ids, E) (0405-...:85-87);
    * group_offsets = exclusive prefix sum of group_sizes, plus the total.
    """
    ids = np.asarray(topk_ids, np.int32)
    topk = ids.shape[-1]
    flat = ids.reshape(-1)
    perm = np.argsort(flat, kind="stable").astype(np.int32)
    tok_sorted = (perm // topk).astype(np.int32)
    revert = np.empty_like(perm)
    revert[perm] = np.arange(perm.size, dtype=np.int32)
    gs = np.bincount(flat, minlength=num_experts)[:num_experts].astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(gs)]).astype(np.int32)
    return perm, tok_sorted, revert, gs, offsets


def gather_rows(hidden: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """hidden[idx] with JAX gather index semantics: negative indices wrap
    once, then indices are clamped into range (moe_fast_dispatch.py:194)."""
    n = hidden.shape[0]
    i = np.asarray(idx, np.int64)
    i = np.where(i < 0, i + n, i)
    i = np.clip(i, 0, n - 1)
    return hidden[i]


def combine(x: np.ndarray, indices: np.ndarray, topk_weights: np.ndarray, topk: int,
            out_dtype: str = "bfloat16") -> np.ndarray:
    """out[t] = round(sum_k f32(x[idx[t*topk+k]]) * f32(w[t, k])).

    moe_fast_combine.py:44-54: f32 products, summed left to right over
    k = 0..topk-1 starting from +0.0, one rounding to out_dtype.  numpy
    evaluates the product and the add as two rounded f32 ops (no FMA).
    ``x`` holds bf16-exact or f32 values as float32.
    """
    x = np.asarray(x, np.float32)
    w = np.asarray(topk_weights, np.float32)
    t = w.shape[0]
    idx = np.asarray(indices).reshape(t, topk)
    acc = np.zeros((t, x.shape[1]), np.float32)
    for k in range(topk):
        rows = gather_rows(x, idx[:, k])
        acc = acc + rows * w[:, k:k + 1]
    if out_dtype == "bfloat16":
        return round_bf16(acc)
    return acc
