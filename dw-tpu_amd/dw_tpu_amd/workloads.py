"""Seeded synthetic inputs of the MoE hot-path workloads (numpy PCG64).

Five workloads, each reproducible bit for bit from its seed:

* ``cpu_plumbing``  -- 8 experts, 64 tokens top-2, K=1024, N=512.
* ``decode_gate_up`` -- 32 local experts, 256 tokens top-8 (experts 3, 11,
  19, 27 never routed: guaranteed empty groups), K=7168, N=2x2048.
* ``decode_down``   -- 32 local experts, 512 tokens top-8, K=2048, N=7168,
  with dispatch / combine (f32 softmax routing weights).
* ``prefill``       -- 8192 tokens top-8 over 32 local experts with Zipf(1.1)
  expert popularity (3 experts never routed), K=7168, N=4096.
* ``dense_fp8``     -- K=7168, N=4096, M in {1, 16, 128, 1024, 4096}.

Router logits are N(0,1); weights and ids come from softmax -> top-k.  lhs
values are N(0,1) rounded to bf16.  FP4 weights are uniform over the 16 e2m1
nibbles, packed two per byte (element 2j low); e8m0 scale exponents are
uniform in [-4, 2] (codes 123..129).  Arrays are numpy; bf16 is carried as
uint16 bit patterns.
"""
from dataclasses import dataclass, field

import numpy as np
import torch

GMM_WORKLOADS = {
    "cpu_plumbing": dict(E=8, T=64, topk=2, K=1024, N=512, seed=1001, empty=(), zipf=None),
    "decode_gate_up": dict(E=32, T=256, topk=8, K=7168, N=4096, seed=1002, empty=(3, 11, 19, 27), zipf=None),
    "decode_down": dict(E=32, T=512, topk=8, K=2048, N=7168, seed=1003, empty=(), zipf=None),
    "prefill": dict(E=32, T=8192, topk=8, K=7168, N=4096, seed=1004, empty=(5, 17, 29), zipf=1.1),
}
DENSE_FP8 = dict(K=7168, N=4096, M=(1, 16, 128, 1024, 4096), seed=1005)


def bf16_bits_from_f32(x: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 (nearest even) and return the uint16 bits."""
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def f32_from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _softmax(x):
    z = np.exp(x - x.max(-1, keepdims=True))
    return (z / z.sum(-1, keepdims=True)).astype(np.float32)


def route(rng, T, E, topk, empty=(), zipf=None):
    """Returns (topk_ids int32 [T, topk], topk_weights f32 [T, topk])."""
    if zipf is None:
        logits = rng.standard_normal((T, E)).astype(np.float32)
        for e in empty:
            logits[:, e] = -np.inf
        p = _softmax(logits)
        ids = np.argsort(-p, axis=-1, kind="stable")[:, :topk].astype(np.int32)
        w = np.take_along_axis(p, ids, axis=-1).astype(np.float32)
        return ids, w
    # Zipf popularity p_e ~ rank^-s over a random expert order; per token, k
    # distinct experts without replacement by Gumbel-top-k on log p.
    order = rng.permutation(E)
    rank = np.empty(E, np.int64)
    rank[order] = np.arange(1, E + 1)
    logp = -zipf * np.log(rank.astype(np.float64))
    for e in empty:
        logp[e] = -np.inf
    g = rng.gumbel(size=(T, E))
    ids = np.argsort(-(logp[None, :] + g), axis=-1, kind="stable")[:, :topk].astype(np.int32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    w = np.take_along_axis(_softmax(logits), ids, axis=-1).astype(np.float32)
    return ids, w


@dataclass
class GmmWorkload:
    name: str
    E: int
    T: int
    topk: int
    K: int
    N: int
    seed: int
    topk_ids: np.ndarray = field(repr=False)      # int32 [T, topk]
    topk_weights: np.ndarray = field(repr=False)  # f32 [T, topk]
    group_sizes: np.ndarray = field(repr=False)   # int32 [E]
    lhs_bits: np.ndarray = field(repr=False)      # uint16 [M, K], expert-sorted rows
    rhs_e2m1: np.ndarray = field(repr=False)      # uint8 [E, K, N/2]
    scale_codes: np.ndarray = field(repr=False)   # uint8 [E, K/32, 1, N]

    @property
    def M(self):
        return self.T * self.topk

    def weight_bytes(self):
        """Packed fp4 bytes + e8m0 scale bytes of the experts that own rows."""
        nonempty = int((self.group_sizes > 0).sum())
        return nonempty * (self.K * self.N // 2 + (self.K // 32) * self.N)

    def algorithmic_bytes(self, out_bytes=2):
        """HBM bytes one gmm call must move at least: non-empty experts'
        weights and scales, the lhs once and the output once."""
        return self.weight_bytes() + self.M * self.K * 2 + self.M * self.N * out_bytes

    def flops(self):
        return 2 * self.M * self.K * self.N


def make_gmm_workload(name: str, scale_m: float = 1.0, with_data: bool = True) -> GmmWorkload:
    """Builds a named workload.  ``scale_m`` < 1 shrinks T (a faster variant
    with the same K, N, E for tests); ``with_data=False`` draws only the
    routing (identical to the full workload's) and leaves the arrays None."""
    cfg = GMM_WORKLOADS[name]
    rng = np.random.Generator(np.random.PCG64(cfg["seed"]))
    E, topk, K, N = cfg["E"], cfg["topk"], cfg["K"], cfg["N"]
    T = max(1, int(round(cfg["T"] * scale_m)))
    ids, w = route(rng, T, E, topk, cfg["empty"], cfg["zipf"])
    gs = np.bincount(ids.reshape(-1), minlength=E).astype(np.int32)
    M = T * topk
    if not with_data:
        return GmmWorkload(name, E, T, topk, K, N, cfg["seed"], ids, w, gs, None, None, None)
    lhs = bf16_bits_from_f32(rng.standard_normal((M, K), dtype=np.float32))
    rhs = rng.integers(0, 256, size=(E, K, N // 2), dtype=np.uint8)
    sc = rng.integers(123, 130, size=(E, K // 32, 1, N), dtype=np.uint8)
    return GmmWorkload(name, E, T, topk, K, N, cfg["seed"], ids, w, gs, lhs, rhs, sc)


@dataclass
class DenseWorkload:
    M: int
    K: int
    N: int
    x_bits: np.ndarray = field(repr=False)   # uint16 [M, K] bf16 activations
    xq: np.ndarray = field(repr=False)       # uint8 [M, K] e4m3 activations
    sx: np.ndarray = field(repr=False)       # f32 [M, K/128]
    wq: np.ndarray = field(repr=False)       # uint8 [K, N] e4m3 weights
    sw: np.ndarray = field(repr=False)       # f32 [K/128, N/128] block scales
    s_w8a16: np.ndarray = field(repr=False)  # f32 [K/128, 1, N] per-(K-block, column) scales


def _e4m3_codes(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def make_dense_workload(M: int, K: int = DENSE_FP8["K"], N: int = DENSE_FP8["N"],
                        seed: int = DENSE_FP8["seed"]) -> DenseWorkload:
    """Weights N(0,1) quantised per 128x128 block by absmax/448 to e4m3
    (128 x 16 blocks when N is not a multiple of 128, for small test shapes);
    activations N(0,1) quantised per (token, 128-K group) the same way."""
    rng = np.random.Generator(np.random.PCG64(seed + M))
    w = rng.standard_normal((K, N), dtype=np.float32)
    bn = 128 if N % 128 == 0 else 16
    wb = w.reshape(K // 128, 128, N // bn, bn)
    sw = (np.abs(wb).max(axis=(1, 3)) / np.float32(448.0)).astype(np.float32)
    wq = _e4m3_codes((wb / sw[:, None, :, None]).reshape(K, N))
    x = rng.standard_normal((M, K), dtype=np.float32)
    xb = x.reshape(M, K // 128, 128)
    sx = (np.abs(xb).max(axis=2) / np.float32(448.0)).astype(np.float32)
    xq = _e4m3_codes((xb / sx[:, :, None]).reshape(M, K))
    s16 = np.repeat(sw, bn, axis=1)[:, None, :].astype(np.float32)  # [K/128, 1, N]
    return DenseWorkload(M, K, N, bf16_bits_from_f32(x), xq, sx, wq, sw, s16)
