"""The committed golden fixtures (tests/golden/, written by make_golden.py
from the oracle): the oracle still reproduces them on the CPU, and the GPU
path matches them -- bit-exact for decode, dispatch and combine, within the
stated bound for the gmm."""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor
from oracle import fp4, gmm, moe
from oracle.numerics import E4M3_VALUES, bf16_to_f32

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _npz(name):
    return dict(np.load(os.path.join(GOLDEN, name)))


def _json(name):
    return json.load(open(os.path.join(GOLDEN, name)))


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ------------------------------------------------------------------ oracle (CPU)

def test_oracle_reproduces_the_fp4_and_fp8_tables():
    t = _json("fp4_tables.json")
    assert [float(v) for v in fp4.E2M1_VALUES] == t["e2m1_values"]
    assert fp4.e2m1_to_codes(np.arange(16, dtype=np.uint8)).tolist() == t["e2m1_to_codes"]
    assert [float(v) for v in fp4.decode_codes(np.arange(16, dtype=np.uint8))] == t["decode_codes"]
    e8 = fp4.e8m0_decode(np.arange(256, dtype=np.uint8)).astype(np.float32).view(np.uint32)
    assert e8.tolist() == t["e8m0_f32_bits"]
    assert E4M3_VALUES.astype(np.float32).view(np.uint32).tolist() == t["e4m3_f32_bits"]


def test_oracle_reproduces_dispatch_and_combine():
    d = _npz("dispatch_small.npz")
    for got, key in zip(moe.dispatch(d["ids"], 9), ["perm", "tok_sorted", "revert", "group_sizes", "group_offsets"]):
        assert np.array_equal(got, d[key]), key
    c = _npz("combine_small.npz")
    out = moe.combine(bf16_to_f32(c["x_bits"]), c["revert"], c["weights"], c["weights"].shape[1])
    from oracle.numerics import bf16_bits as np_bits
    assert np.array_equal(np_bits(out), c["out_bits"])


def test_oracle_reproduces_the_gmm_fixtures():
    g = _npz("gmm_tiny.npz")
    w = gmm.dequant_rhs(fp4.e2m1_to_codes(fp4.unpack_nibbles(g["rhs_e2m1"])), fp4.e8m0_decode(g["scale_codes"]))
    y64, _ = gmm.gmm(bf16_to_f32(g["lhs_bits"]), None, None, g["group_sizes"], out_dtype="float64", w=w)
    assert np.array_equal(y64, g["y64"])
    from dw_tpu_amd.workloads import make_gmm_workload
    meta, sl = _json("gmm_cpu_plumbing.json"), _npz("gmm_cpu_plumbing_slice.npz")
    wl = make_gmm_workload("cpu_plumbing")  # the seeded generator still makes the same inputs
    for key, h in meta["sha256"].items():
        assert _sha(getattr(wl, key)) == h, key
    assert wl.group_sizes.tolist() == meta["group_sizes"]
    rows, (c0, c1) = meta["rows"], meta["cols"]
    w = gmm.dequant_rhs(fp4.e2m1_to_codes(fp4.unpack_nibbles(wl.rhs_e2m1[:, :, c0 // 2:c1 // 2])),
                        fp4.e8m0_decode(wl.scale_codes[..., c0:c1]))
    y64, _ = gmm.gmm(bf16_to_f32(wl.lhs_bits), None, None, wl.group_sizes, out_dtype="float64", w=w)
    assert np.allclose(y64[rows], sl["y64"], rtol=1e-13, atol=0)


# --------------------------------------------------------------------- GPU path

@pytest.mark.gpu
def test_gpu_matches_the_decode_tables(dev):
    from dw_tpu_amd import _lib
    from dw_tpu_amd.gmm_v2 import decode_fp4
    t = _json("fp4_tables.json")
    nib = torch.arange(256, dtype=torch.uint8, device=dev)  # every byte: two e2m1 nibbles
    got = decode_fp4(nib, _lib.FP4_E2M1).float().cpu().numpy()
    want = np.array([[t["e2m1_values"][b & 15], t["e2m1_values"][b >> 4]] for b in range(256)], np.float32)
    assert np.array_equal(got.reshape(-1), want.reshape(-1))


@pytest.mark.gpu
def test_gpu_matches_the_dispatch_and_combine_fixtures(dev):
    from dw_tpu_amd import fast_combine, moe_dispatch
    d = _npz("dispatch_small.npz")
    r = moe_dispatch(torch.from_numpy(d["ids"]).to(dev), 9)
    got = [r.topk_argsort_indices, r.token_indices_sorted, r.topk_argsort_revert_indices, r.group_sizes,
           r.group_offsets]
    for g, key in zip(got, ["perm", "tok_sorted", "revert", "group_sizes", "group_offsets"]):
        assert np.array_equal(g.cpu().numpy(), d[key]), key
    c = _npz("combine_small.npz")
    topk = c["weights"].shape[1]
    out = fast_combine(bf16_tensor(c["x_bits"], dev), torch.from_numpy(c["revert"]).to(dev),
                       torch.from_numpy(c["weights"]).to(dev), topk, mode=2, out_dtype=torch.bfloat16)
    assert np.array_equal(bf16_bits(out), c["out_bits"])


@pytest.mark.gpu
def test_gpu_gmm_matches_the_gmm_fixtures_within_the_bound(dev):
    from dw_tpu_amd import fp4_weight_to_codes, gmm_v2
    g = _npz("gmm_tiny.npz")
    pw = fp4_weight_to_codes(torch.from_numpy(g["rhs_e2m1"]).to(dev), torch.from_numpy(g["scale_codes"]).to(dev))
    out = gmm_v2(bf16_tensor(g["lhs_bits"], dev), pw, torch.from_numpy(g["group_sizes"]).to(dev))
    y = bf16_to_f32(bf16_bits(out)).astype(np.float64)
    assert np.all(np.abs(y - g["y64"]) <= gmm.error_bound(g["y64"], g["abs_product"], g["lhs_bits"].shape[1]))
    from dw_tpu_amd.workloads import make_gmm_workload
    meta, sl = _json("gmm_cpu_plumbing.json"), _npz("gmm_cpu_plumbing_slice.npz")
    wl = make_gmm_workload("cpu_plumbing")
    pw = fp4_weight_to_codes(torch.from_numpy(wl.rhs_e2m1).to(dev), torch.from_numpy(wl.scale_codes).to(dev))
    out = gmm_v2(bf16_tensor(wl.lhs_bits, dev), pw, torch.from_numpy(wl.group_sizes).to(dev))
    rows, (c0, c1) = meta["rows"], meta["cols"]
    y = bf16_to_f32(bf16_bits(out[rows, c0:c1])).astype(np.float64)
    assert np.all(np.abs(y - sl["y64"]) <= gmm.error_bound(sl["y64"], sl["abs_product"], wl.K))
