"""Writes the golden fixtures under tests/golden/ from the oracle.

The reference holds no golden vectors for this path (its gmm, dispatch and
combine live in un-vendored code), so these fixtures are the oracle's own
outputs on small fixed inputs, written once and committed: they pin the
oracle against drift and give the GPU tests fixed expected values.

    python tests/golden/make_golden.py        # rewrites the fixtures
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "dw-tpu_amd")]

from oracle import fp4, gmm, moe  # noqa: E402
from oracle.numerics import E4M3_VALUES, bf16_bits, bf16_to_f32  # noqa: E402


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def tables():
    e4 = E4M3_VALUES.astype(np.float32)
    return {"e2m1_values": [float(v) for v in fp4.E2M1_VALUES],
            "e2m1_to_codes": [int(c) for c in fp4.e2m1_to_codes(np.arange(16, dtype=np.uint8))],
            "decode_codes": [float(v) for v in fp4.decode_codes(np.arange(16, dtype=np.uint8))],
            "e8m0_f32_bits": [int(b) for b in fp4.e8m0_decode(np.arange(256, dtype=np.uint8)).astype(np.float32)
                              .view(np.uint32)],
            "e4m3_f32_bits": [int(b) for b in e4.view(np.uint32)]}


def dispatch_case():
    rng = np.random.Generator(np.random.PCG64(2024))
    ids = rng.integers(0, 9, (37, 3)).astype(np.int32)
    ids[5] = [4, 4, 4]          # repeats within a token
    ids[:, 2][ids[:, 2] == 7] = 1
    perm, tok, rev, gs, off = moe.dispatch(ids, 9)
    return dict(ids=ids, perm=perm, tok_sorted=tok, revert=rev, group_sizes=gs, group_offsets=off)


def combine_case():
    rng = np.random.Generator(np.random.PCG64(2025))
    t, topk, h = 8, 3, 40
    x_bits = bf16_bits(rng.standard_normal((t * topk, h)).astype(np.float32) * 3)
    rev = rng.permutation(t * topk).astype(np.int32)
    w = rng.random((t, topk)).astype(np.float32)
    out = moe.combine(bf16_to_f32(x_bits), rev, w, topk, out_dtype="bfloat16")
    return dict(x_bits=x_bits, revert=rev, weights=w, out_bits=bf16_bits(out))


def gmm_tiny_case():
    rng = np.random.Generator(np.random.PCG64(2026))
    sizes = np.array([3, 0, 7], np.int32)
    k, n = 128, 16
    lhs_bits = bf16_bits(rng.standard_normal((int(sizes.sum()), k)).astype(np.float32))
    nib = rng.integers(0, 16, (3, k, n), dtype=np.uint8)
    sc = rng.integers(123, 130, (3, k // 32, 1, n), dtype=np.uint8)
    w = gmm.dequant_rhs(fp4.e2m1_to_codes(nib), fp4.e8m0_decode(sc))
    y64, _ = gmm.gmm(bf16_to_f32(lhs_bits), None, None, sizes, out_dtype="float64", w=w)
    ap = gmm.abs_product(bf16_to_f32(lhs_bits), w, sizes)
    return dict(lhs_bits=lhs_bits, rhs_e2m1=fp4.pack_nibbles(nib), scale_codes=sc, group_sizes=sizes,
                y64=y64, abs_product=ap)


def cpu_plumbing():
    from dw_tpu_amd.workloads import make_gmm_workload
    wl = make_gmm_workload("cpu_plumbing")
    rows, cols = np.arange(4), np.arange(256)
    w = gmm.dequant_rhs(fp4.e2m1_to_codes(fp4.unpack_nibbles(wl.rhs_e2m1)), fp4.e8m0_decode(wl.scale_codes))
    lhs = bf16_to_f32(wl.lhs_bits)
    y64, _ = gmm.gmm(lhs, None, None, wl.group_sizes, out_dtype="float64", w=w)
    ap = gmm.abs_product(lhs, w, wl.group_sizes)
    return ({"sha256": {"topk_ids": sha(wl.topk_ids), "lhs_bits": sha(wl.lhs_bits), "rhs_e2m1": sha(wl.rhs_e2m1),
                        "scale_codes": sha(wl.scale_codes)},
             "group_sizes": [int(g) for g in wl.group_sizes], "rows": rows.tolist(), "cols": [0, 256]},
            dict(y64=y64[np.ix_(rows, cols)], abs_product=ap[np.ix_(rows, cols)]))


def main():
    json.dump(tables(), open(os.path.join(HERE, "fp4_tables.json"), "w"), indent=0)
    np.savez(os.path.join(HERE, "dispatch_small.npz"), **dispatch_case())
    np.savez(os.path.join(HERE, "combine_small.npz"), **combine_case())
    np.savez(os.path.join(HERE, "gmm_tiny.npz"), **gmm_tiny_case())
    meta, arrays = cpu_plumbing()
    json.dump(meta, open(os.path.join(HERE, "gmm_cpu_plumbing.json"), "w"), indent=1)
    np.savez(os.path.join(HERE, "gmm_cpu_plumbing_slice.npz"), **arrays)


if __name__ == "__main__":
    main()
