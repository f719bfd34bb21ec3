"""Dense FP8 block-quantized GEMM -- numpy restatement.

Test infrastructure only (see oracle/__init__.py).

* W8A16: kernels/tpu_inference/kernels/experimental/dense_fp8.py:23-59.
  For each 128-row K block kb: acc += dot(x_bf16[:, kb], w_e4m3[kb, :]) (f32)
  * s[kb, :] (f32), acc initialised to zero; stored as bf16.
* W8A16 "pre" mode: dense_fp8.py:33-43 -- the weight tile is widened to
  bf16, each weight multiplied by bf16(s[kb, n]) with the product rounded to
  bf16, then one f32 dot over K (no scale after the dot).
* W8A8 (activations e4m3 with per-(token, 128-K) f32 scales, weights e4m3 with
  128x128 f32 block scales): no reference kernel; the closed form is
  out[m, n] = sum_kb sx[m, kb] * sw[kb, n // 128] * dot(xq[m, kb], wq[kb, n]).
"""
import numpy as np

from .numerics import E4M3_VALUES, round_bf16


def matmul_w8a16(x, w_codes, s, accumulate: str = "f64", out_dtype: str = "bfloat16"):
    """x [M, K] f32 (bf16-exact); w_codes [K, N] e4m3 codes; s [K/128, 1, N] f32."""
    x = np.asarray(x, np.float32)
    m, k = x.shape
    n = w_codes.shape[1]
    w = E4M3_VALUES[np.asarray(w_codes)].astype(np.float32)
    s = np.asarray(s, np.float32).reshape(k // 128, n)
    dt = np.float64 if accumulate == "f64" else np.float32
    acc = np.zeros((m, n), dt)
    for kb in range(k // 128):
        part = x[:, kb * 128:(kb + 1) * 128].astype(dt) @ w[kb * 128:(kb + 1) * 128].astype(dt)
        acc = acc + part * s[kb].astype(dt)[None, :]
    if out_dtype == "bfloat16":
        return round_bf16(acc.astype(np.float32))
    return acc


def pre_weight(w_codes, s):
    """The "pre" mode's bf16 weight (dense_fp8.py:39-41):
    w_pre[k, n] = bf16(e4m3(w[k, n]) * bf16(s[k // 128, n])), each rounding
    to nearest even.  The f32 product of a bf16 and an e4m3 value is exact,
    so this is the correctly rounded bf16 product.  Returns float32."""
    w = E4M3_VALUES[np.asarray(w_codes)].astype(np.float32)
    k, n = w.shape
    sb = round_bf16(np.asarray(s, np.float32).reshape(k // 128, n))
    prod = (w.reshape(k // 128, 128, n) * sb[:, None, :]).reshape(k, n)
    return round_bf16(prod.astype(np.float32))


def matmul_pre(x, w_codes, s, accumulate: str = "f64", out_dtype: str = "bfloat16"):
    """The "pre" mode: x [M, K] f32 (bf16-exact) @ pre_weight(w_codes, s)."""
    x = np.asarray(x, np.float32)
    dt = np.float64 if accumulate == "f64" else np.float32
    acc = x.astype(dt) @ pre_weight(w_codes, s).astype(dt)
    if out_dtype == "bfloat16":
        return round_bf16(acc.astype(np.float32))
    return acc


def matmul_w8a8(xq, sx, wq, sw, accumulate: str = "f64", out_dtype: str = "bfloat16"):
    """xq [M, K] e4m3 codes, sx [M, K/128] f32; wq [K, N] e4m3, sw [K/128, N/128] f32."""
    xv = E4M3_VALUES[np.asarray(xq)].astype(np.float32)
    wv = E4M3_VALUES[np.asarray(wq)].astype(np.float32)
    m, k = xv.shape
    n = wv.shape[1]
    dt = np.float64 if accumulate == "f64" else np.float32
    sx = np.asarray(sx, np.float32)
    sw_full = np.repeat(np.asarray(sw, np.float32), 128, axis=1)[:, :n]  # [K/128, N]
    acc = np.zeros((m, n), dt)
    for kb in range(k // 128):
        part = xv[:, kb * 128:(kb + 1) * 128].astype(dt) @ wv[kb * 128:(kb + 1) * 128].astype(dt)
        acc = acc + part * (sx[:, kb:kb + 1].astype(dt) * sw_full[kb][None, :].astype(dt))
    if out_dtype == "bfloat16":
        return round_bf16(acc.astype(np.float32))
    return acc


def abs_product_w8a16(x, w_codes, s):
    """sum_k |x_mk| |w_kn s_kn| (float64), for the error bound."""
    k = x.shape[1]
    n = w_codes.shape[1]
    w = np.abs(E4M3_VALUES[np.asarray(w_codes)].astype(np.float64))
    s = np.abs(np.asarray(s, np.float64).reshape(k // 128, 1, n))
    w = (w.reshape(k // 128, 128, n) * s).reshape(k, n)
    return np.abs(np.asarray(x, np.float64)) @ w


def abs_product_w8a8(xq, sx, wq, sw):
    """sum_k |xq_mk sx_m,kb| |wq_kn sw_kb,n/128| (float64), for the error bound."""
    xv = np.abs(E4M3_VALUES[np.asarray(xq)].astype(np.float64))
    wv = np.abs(E4M3_VALUES[np.asarray(wq)].astype(np.float64))
    m, k = xv.shape
    n = wv.shape[1]
    xs = (xv.reshape(m, k // 128, 128) * np.abs(np.asarray(sx, np.float64))[:, :, None]).reshape(m, k)
    swf = np.repeat(np.abs(np.asarray(sw, np.float64)), 128, axis=1)[:, :n]
    ws = (wv.reshape(k // 128, 128, n) * swf[:, None, :]).reshape(k, n)
    return xs @ ws


def error_bound(y64, absprod, k, out_dtype="bfloat16"):
    """Stated tolerance for a dense FP8 output element against float64:

        |y - y64| <= u_out |y64| + (K + 3 K/128) 2^-24 sum_k |x_k w_k s_k|

    u_out = 2^-8 for bf16 output; the second term covers any f32 order of
    the 128-long partial dots, the f32 scale products and the sum over K
    blocks (and the sx * sw product of the W8A8 variant).
    """
    u_out = 2.0 ** -8 if out_dtype == "bfloat16" else 2.0 ** -24
    return u_out * np.abs(y64) + (k + 3 * (k // 128)) * 2.0 ** -24 * absprod
