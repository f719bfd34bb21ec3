"""Ragged grouped matmul (tokamax gmm_v2 with FP4 codes) -- numpy restatement.

Test infrastructure only (see oracle/__init__.py).

Semantics restated from:
* patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:58-66 (decode each rhs
  tile to the lhs dtype inside the kernel), :93-96 (lhs is not quantized when
  rhs is emulated fp4), :128-141 (rhs_fp4_codes requires uint4 rhs).
* patches/tpu-inference/0001-dsv4-v6e-enablement.patch:214-233 (gmm_wrapper
  calls gmm_v2 with zero_initialize=False).
* patches/tpu-inference-ext/0103-...:94-97 (rows outside the local groups are
  left unwritten when zero_initialize is False).
* patches/tpu-inference-ext/0106-...:243-250 (f32 output variant).

Rows [off_g, off_g + size_g) of the expert-sorted lhs, for each local group
g in [group_offset, group_offset + E_local), are multiplied by
dequant(rhs[g - group_offset]); off_g is the exclusive prefix sum of ALL
group sizes.  Accumulation is f32 in the reference; its order inside the
un-vendored kernel is unknown, so this oracle offers the float64 product of
the exact bf16 inputs (the closed form) and an f32 BLAS product.
"""
import numpy as np

from .fp4 import dequant_fp4_block
from .numerics import round_bf16


def group_starts(group_sizes: np.ndarray) -> np.ndarray:
    gs = np.asarray(group_sizes, np.int64)
    return np.concatenate([[0], np.cumsum(gs)])[:-1]


def dequant_rhs(codes: np.ndarray, scale: np.ndarray, block: int = 32) -> np.ndarray:
    """codes [E, K, N] uint4 values; scale [E, K/block, 1, N] f32 -> f32 [E, K, N]."""
    e, k, n = codes.shape
    scale = np.asarray(scale, np.float32).reshape(e, k // block, 1, n)
    return np.stack([dequant_fp4_block(codes[i], scale[i], block) for i in range(e)])


def gmm(lhs, codes, scale, group_sizes, group_offset: int = 0, out_dtype: str = "bfloat16",
        accumulate: str = "f64", zero_initialize: bool = True, w=None, bias=None):
    """Returns (out [M, N] float32 or float64 values, written-row mask [M]).

    lhs: [M, K] float32 holding bf16-exact values.  codes: [E_local, K, N]
    uint4 code values (0..15).  scale: [E_local, K/32, 1, N] f32.
    ``w`` may pass a precomputed ``dequant_rhs`` result.  ``bias``
    ([E_local, N]) is gmm_v2's rhs_bias: added to each local group's rows
    (in the accumulation dtype) before the output rounding.
    With out_dtype 'bfloat16' the result is rounded to bf16 (RNE); with
    'float32' to f32; with 'float64' it is returned unrounded.
    accumulate: 'f64' (exact up to float64 rounding), 'f32' (BLAS) or
    'seq32' (f32 running sum over k in order).
    """
    lhs = np.asarray(lhs, np.float32)
    m, k = lhs.shape
    e_local = codes.shape[0] if w is None else w.shape[0]
    n = codes.shape[2] if w is None else w.shape[2]
    if w is None:
        w = dequant_rhs(codes, scale)
    starts = group_starts(group_sizes)
    gs = np.asarray(group_sizes, np.int64)
    out = np.zeros((m, n), np.float64)
    written = np.zeros(m, bool)
    for g in range(group_offset, min(group_offset + e_local, len(gs))):
        r0, r1 = int(starts[g]), int(starts[g] + gs[g])
        r1 = min(r1, m)
        if r1 <= r0:
            continue
        a = lhs[r0:r1]
        if accumulate == "f64":
            y = a.astype(np.float64) @ w[g - group_offset].astype(np.float64)
        elif accumulate == "seq32":
            # f32 running sum over k in order of the exact bf16 x bf16
            # products (each fits f32): the plain sequential-accumulation
            # kernel, the baseline of the acceptance policy below.
            wg = w[g - group_offset].astype(np.float32)
            acc = np.zeros((r1 - r0, n), np.float32)
            for kk in range(k):
                acc += a[:, kk:kk + 1] * wg[kk:kk + 1, :]
            y = acc.astype(np.float64)
        else:
            y = (a @ w[g - group_offset].astype(np.float32)).astype(np.float64)
        if bias is not None:
            b = np.asarray(bias[g - group_offset], np.float64)
            y = y + b if accumulate == "f64" else (y.astype(np.float32) + b.astype(np.float32)).astype(np.float64)
        out[r0:r1] = y
        written[r0:r1] = True
    if out_dtype == "bfloat16":
        out = round_bf16(out.astype(np.float32))
    elif out_dtype == "float32":
        out = out.astype(np.float32)
    if not zero_initialize:
        out = np.where(written[:, None], out, np.nan)
    return out, written


def abs_product(lhs, w, group_sizes, group_offset: int = 0):
    """sum_k |a_mk| |w_kn| per output element (float64): the scale of the
    f32 accumulation error term of the tolerance."""
    m = lhs.shape[0]
    starts = group_starts(group_sizes)
    gs = np.asarray(group_sizes, np.int64)
    out = np.zeros((m, w.shape[2]), np.float64)
    for g in range(group_offset, min(group_offset + w.shape[0], len(gs))):
        r0, r1 = int(starts[g]), min(int(starts[g] + gs[g]), m)
        if r1 > r0:
            out[r0:r1] = np.abs(lhs[r0:r1]).astype(np.float64) @ np.abs(w[g - group_offset]).astype(np.float64)
    return out


def error_bound(y64, absprod, k: int, out_dtype: str = "bfloat16"):
    """Stated tolerance for a gmm output element against the float64 value:

        |y - y64| <= u_out * |y64| + K * 2^-24 * sum_k |a_k w_k|

    u_out = 2^-8 (bf16 round to nearest) or 2^-24 (f32); the second term
    bounds any order of f32 accumulation of K exact bf16 x bf16 products.
    """
    u_out = 2.0 ** -8 if out_dtype == "bfloat16" else 2.0 ** -24
    return u_out * np.abs(y64) + k * 2.0 ** -24 * absprod


def error_stats(y, y64, mask=None):
    """max abs error and relative Frobenius error against float64."""
    y = np.asarray(y, np.float64)
    y64 = np.asarray(y64, np.float64)
    if mask is not None:
        y, y64 = y[mask], y64[mask]
    d = y - y64
    den = np.linalg.norm(y64)
    return {"max_abs": float(np.abs(d).max()) if d.size else 0.0,
            "rel_fro": float(np.linalg.norm(d) / den) if den > 0 else float(np.linalg.norm(d))}


def sample_rows_cols(group_sizes, n, rng, ncols=64):
    """Rows and columns on which full-size workloads are checked: the first,
    last and one random row of every non-empty group, and columns 0, N - 1
    and ncols - 2 random ones (sorted, unique)."""
    gs = np.asarray(group_sizes, np.int64)
    starts = np.concatenate([[0], np.cumsum(gs)])
    rows = np.unique(np.concatenate([[s, s + g - 1, s + rng.integers(0, g)]
                                     for s, g in zip(starts[:-1], gs) if g > 0]))
    cols = np.unique(np.r_[0, n - 1, rng.integers(0, n, ncols - 2)])
    return rows, cols


def w4a16_rows(lhs_bits_rows, rhs_e2m1, scale_codes, group_sizes, rows, cols):
    """The reference's W4A16 result (bf16 lhs times exactly decoded e2m1 x
    e8m0 weights, patches/tokamax/0001-...:58-66, 93-96) in float64 for the
    given rows (lhs_bits_rows: their bf16 bit patterns) and columns of a
    grouped matmul over all groups: rhs_e2m1 [E, K, N/2] packed nibbles
    (low nibble = even column), scale_codes [E, K/32, 1, N] e8m0 codes."""
    from .fp4 import e2m1_to_codes, e8m0_decode
    from .numerics import bf16_to_f32
    cols = np.asarray(cols)
    b = rhs_e2m1[:, :, cols // 2]
    nib = np.where(cols % 2 == 1, b >> 4, b & 0xF).astype(np.uint8)
    w = dequant_rhs(e2m1_to_codes(nib), e8m0_decode(scale_codes[..., cols]))
    starts = np.concatenate([[0], np.cumsum(np.asarray(group_sizes, np.int64))])
    grp = np.searchsorted(starts, rows, side="right") - 1
    sub_gs = np.bincount(grp, minlength=len(group_sizes)).astype(np.int32)
    y64, _ = gmm(bf16_to_f32(lhs_bits_rows), None, None, sub_gs, out_dtype="float64", w=w)
    return y64


def acceptance_policy(y, y_base, y64, mask=None):
    """The reference's kernel-acceptance rule
    (results/dsv4-dense-gemm-kernel-1/NOTES.md:26-27): against the float64
    result, a new kernel's RMS error is at most 1.10x, and its max abs error
    at most 2x, those of the current kernel (here ``y_base``, the
    sequential-f32 accumulation).  Returns (passed, stats)."""
    y, y_base, y64 = (np.asarray(v, np.float64) for v in (y, y_base, y64))
    if mask is not None:
        y, y_base, y64 = y[mask], y_base[mask], y64[mask]
    d, db = y - y64, y_base - y64
    rms, rms_b = float(np.sqrt(np.mean(d * d))), float(np.sqrt(np.mean(db * db)))
    mx, mx_b = float(np.abs(d).max()), float(np.abs(db).max())
    st = {"rms": rms, "rms_base": rms_b, "max_abs": mx, "max_abs_base": mx_b}
    return rms <= 1.10 * rms_b and mx <= 2.0 * mx_b, st


MX_BLOCK_TERM = 2.0 ** -11


def block_max_product(lhs, w, group_sizes, group_offset: int = 0, block: int = 32):
    """sum over 32-value K-blocks b of max_{k in b} |a_mk| |w_kn| per output
    element (float64): the scale of the scaled MFMA's in-block alignment
    error in the MX tolerance below."""
    lhs = np.abs(np.asarray(lhs, np.float64))
    m, k = lhs.shape
    starts = group_starts(group_sizes)
    gs = np.asarray(group_sizes, np.int64)
    out = np.zeros((m, w.shape[2]), np.float64)
    for g in range(group_offset, min(group_offset + w.shape[0], len(gs))):
        r0, r1 = int(starts[g]), min(int(starts[g] + gs[g]), m)
        if r1 <= r0:
            continue
        wg = np.abs(np.asarray(w[g - group_offset], np.float64))
        for b0 in range(0, k, block):
            a = lhs[r0:r1, b0:b0 + block]
            wb = wg[b0:b0 + block]
            mx = np.zeros((r1 - r0, wg.shape[1]))
            for kk in range(a.shape[1]):
                np.maximum(mx, a[:, kk:kk + 1] * wb[kk:kk + 1, :], out=mx)
            out[r0:r1] += mx
    return out


def mx_error_bound(y64, absprod, blockmax, k: int, out_dtype: str = "bfloat16"):
    """Stated tolerance of the MX mode (e4m3 lhs x e2m1 rhs on the gfx950
    scaled MFMA) against the float64 product of the dequantized operands:

        |y - y64| <= u_out |y64| + K 2^-24 sum_k |a_k w_k|
                     + 2^-11 sum_b max_{k in b} |a_k w_k|

    The last term is the instruction's own accumulation: within one 32-value
    K-block it aligns the products to the block's largest and truncates
    toward zero (measured on MI355X: errors up to 2^-12 of that product;
    sums of different blocks combine exact to 2^-20), taken here with a
    factor 2 margin.  The first two terms are those of ``error_bound``."""
    return error_bound(y64, absprod, k, out_dtype) + MX_BLOCK_TERM * blockmax
