#!/usr/bin/env python3
"""FP4 MoE grouped-matmul throughput on one MI355X.

A step is one FP4 grouped matmul (gmm_v2 with prepacked e2m1 + e8m0 weights)
over one batch of routed rows of the decode gate+up workload: 32 local
experts, 256 tokens x top-8 (M = 2048 routed rows, 4 guaranteed-empty
experts), K = 7168, N = 2 x 2048, bf16 activations, bf16 output.  Inputs are
resident in HBM before the timed region; the weight set is rotated over
copies larger than the 256 MB Infinity Cache so the stream comes from HBM.

`value` is algorithmic HBM GB/s (non-empty experts' packed weights + scales,
lhs once, output once) divided by the step time measured with HIP events on
the stream the kernels run on: the median of 9 samples of --steps
back-to-back launches (the gmm and dense lines in `extra`: of 3).  The
headline runs the reference's W4A16 arithmetic (bf16 lhs, exactly decoded
fp4 weights, bf16 MFMA).
`extra` reports the other workloads (decode down-projection with dispatch /
combine, prefill) the same way, each gmm workload again in the MX mode
(`<name>_mx`: e4m3 lhs with e8m0 block-32 scales on the scaled MFMA, a
lossier computation, with the quantization kernel timed alone and with the
gmm; `<name>_mxfp4`: the same with an e2m1 lhs, fp4 x fp4, lossier still),
the expert block, dense FP8, router and format kernels.
`cpu_baseline` times the numpy oracle of the same math on a bounded sample of
experts on this host's cores (and one expert on one thread), the same for
prefill and a dense GEMM, and reports the max abs and relative Frobenius
error of one expert's GPU output rows against the oracle's float64 product.
The same leg adds `vs_w4a16` to each `<name>_mx` / `<name>_mxfp4` line:
the output's max abs and relative Frobenius distance from the reference's
W4A16 result (float64, sampled rows and columns), the lhs quantization
included.

The headline is timed last, right after the `extra` workloads (its inputs
are in HBM beforehand), so that the GPU runs at the clock it holds under
continuous load: after about a second without GPU work the power manager
lowers the clock and ramps it back up over tens of milliseconds of load, so
a few warmup launches after a host-side pause time part of that ramp
(decode_gate_up: 170-185 us/step after an idle second, 142-155 us/step
right after GPU load).  With `--extra none` it runs after the input upload
alone.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--extra all|none]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "dw-tpu_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "FP4 MoE gmm TFLOP/s + HBM GB/s (% of peak) at decode & prefill sizes"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
FP4_PEAK_TFLOPS = 10100.0
ONLY_CHOICES = ("decode_gate_up", "decode_down", "prefill", "decode_gate_up_mx", "decode_down_mx", "prefill_mx",
                "decode_gate_up_mxfp4", "decode_down_mxfp4", "prefill_mxfp4",
                "dense_M1", "dense_M16", "dense_M128", "dense_M1024", "dense_M4096")
MALL_BYTES = 256 * 2 ** 20
HEADLINE_SAMPLES = 9  # timed samples of the headline; value is their median


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _to_dev_bf16(bits, dev):
    import numpy as np
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(dev)


class GmmBench:
    """Device-resident inputs of one gmm workload plus a raw C-ABI launcher.

    mode "bf16": dwm_gmm_fp4 (the reference's W4A16 arithmetic); mode "mx":
    dwm_gmm_fp4_mx on the lhs quantized once beforehand (e4m3 codes + e8m0
    block-32 scales); mode "mxfp4": dwm_gmm_fp4_mxfp4 on an e2m1 lhs.
    ``quant_step`` times the quantization."""

    def __init__(self, wl, dev, copies, mode="bf16"):
        import torch
        from dw_tpu_amd import _lib, fp4_weight_to_codes, mx_quantize
        self.wl = wl
        self.mode = mode
        self.lib = _lib.load()
        rhs = torch.from_numpy(wl.rhs_e2m1).to(dev)
        sc = torch.from_numpy(wl.scale_codes).to(dev)
        self.weights = [fp4_weight_to_codes(rhs, sc) for _ in range(copies)]
        del rhs, sc
        self.lhs = [_to_dev_bf16(wl.lhs_bits, dev) for _ in range(copies if mode == "bf16" else 1)]
        self.gs = torch.from_numpy(wl.group_sizes).to(dev)
        self.out = [torch.empty((wl.M, wl.N), dtype=torch.bfloat16, device=dev) for _ in range(copies)]
        self.stream = _lib.stream_handle(dev)
        P = ctypes.c_void_p
        self.args = []
        if mode in ("mx", "mxfp4"):
            fmt = "e2m1" if mode == "mxfp4" else "e4m3"
            self.mx = mx_quantize(self.lhs[0], fmt)
            self.qcodes = torch.empty_like(self.mx.codes)
            self.qscales = torch.empty_like(self.mx.scales)
            self.quant_args = (P(self.lhs[0].data_ptr()), wl.M, wl.K, P(self.qcodes.data_ptr()),
                               P(self.qscales.data_ptr()), self.stream)
            self.quant_fn = self.lib.dwm_mx_quant_e2m1 if mode == "mxfp4" else self.lib.dwm_mx_quant_e4m3
        for i in range(copies):
            w = self.weights[i]
            tail = (P(w.weight.data_ptr()), P(w.scale.data_ptr()), P(self.gs.data_ptr()), wl.E, None, wl.E, wl.N,
                    P(self.out[i].data_ptr()), _lib.BF16, 0, _lib.ACT_NONE, self.stream)
            if mode == "mx":
                self.args.append((P(self.mx.codes.data_ptr()), P(self.mx.scales.data_ptr()), wl.M, None, wl.M,
                                  wl.K) + tail)
            elif mode == "mxfp4":  # no bias: (weight, scale, bias NULL, bias dtype 0, ...)
                self.args.append((P(self.mx.codes.data_ptr()), P(self.mx.scales.data_ptr()), wl.M, None, wl.M,
                                  wl.K) + tail[:2] + (None, 0) + tail[2:])
            else:
                self.args.append((P(self.lhs[i].data_ptr()), wl.M, wl.K) + tail)
        self.fn = {"mx": self.lib.dwm_gmm_fp4_mx, "mxfp4": self.lib.dwm_gmm_fp4_mxfp4}.get(mode, self.lib.dwm_gmm_fp4)

    def step(self, i):
        rc = self.fn(*self.args[i % len(self.args)])
        if rc:
            raise RuntimeError(self.lib.dwm_last_error().decode())

    def quant_step(self, i):
        rc = self.quant_fn(*self.quant_args)
        if rc:
            raise RuntimeError(self.lib.dwm_last_error().decode())

    def quant_and_step(self, i):
        self.quant_step(i)
        self.step(i)


def time_steps(step, steps, warmup):
    """Average ms per step over `steps` back-to-back launches (HIP events on
    torch's current stream, which is the stream the kernels are launched on)."""
    import torch
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        step(warmup + i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_median(step, steps, warmup, n=3):
    """Median over n samples of time_steps (the first after `warmup` untimed
    launches, the others straight after it)."""
    s = sorted([time_steps(step, steps, warmup)] + [time_steps(step, steps, 0) for _ in range(n - 1)])
    return s[len(s) // 2]


def gmm_result(wl, ms, mode="bf16"):
    """Throughput of one gmm launch.  Algorithmic bytes: the non-empty
    experts' packed weights and e8m0 scales, the lhs once (bf16, or e4m3
    codes + block-32 scales in the MX mode) and the bf16 output once."""
    bts = wl.algorithmic_bytes()
    if mode == "mx":
        bts += wl.M * wl.K // 32 - wl.M * wl.K  # e4m3 codes + scales in place of bf16
    elif mode == "mxfp4":
        bts += wl.M * wl.K // 32 - wl.M * wl.K * 3 // 2  # e2m1 codes + scales in place of bf16
    fl = wl.flops()
    gbs = bts / (ms * 1e-3) / 1e9
    tfl = fl / (ms * 1e-3) / 1e12
    r = {"ms": round(ms, 5), "GB_s": round(gbs, 1), "TFLOP_s": round(tfl, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    if mode == "mx":
        r["mfma_fp8_frac"] = round(tfl / FP8_PEAK_TFLOPS, 4)
        r["dtype"] = "e4m3 lhs (e8m0 block-32 scales) x e2m1 weights, scaled MFMA, f32 accumulate"
    elif mode == "mxfp4":
        r["mfma_fp4_frac"] = round(tfl / FP4_PEAK_TFLOPS, 4)
        r["mfma_fp8_frac"] = round(tfl / FP8_PEAK_TFLOPS, 4)
        r["dtype"] = "e2m1 lhs (e8m0 block-32 scales) x e2m1 weights, scaled MFMA, f32 accumulate"
    else:
        r["mfma_bf16_frac"] = round(tfl / BF16_PEAK_TFLOPS, 4)
    r.update({"bytes": bts, "flops": fl, "M": wl.M, "K": wl.K, "N": wl.N, "E": wl.E,
              "nonempty_groups": int((wl.group_sizes > 0).sum())})
    return r


def copies_for(wl):
    return max(1, min(4, -(-2 * MALL_BYTES // max(1, wl.weight_bytes()))))


def bench_gmm(name, dev, steps, warmup, mode="bf16"):
    from dw_tpu_amd.workloads import make_gmm_workload
    wl = make_gmm_workload(name)
    b = GmmBench(wl, dev, copies_for(wl), mode)
    ms = time_steps(b.step, steps, warmup)
    return wl, b, ms


def prep_gmm(name, dev, steps, warmup):
    """The bf16 gmm of one workload: inputs now, timing in the returned run()."""
    from dw_tpu_amd.workloads import make_gmm_workload
    wl = make_gmm_workload(name)
    b = GmmBench(wl, dev, copies_for(wl))

    def run():
        return {name: gmm_result(wl, time_median(b.step, steps, warmup))}
    return run


def prep_gmm_mx(name, dev, steps, warmup, keep=None, mode="mx"):
    """The MX mode of one gmm workload: the gmm on the quantized lhs, the
    lhs quantization (bf16 [M, K] -> e4m3 + scales), and the two back to back
    (what gmm_v2(lhs_quant_dtype=float8_e4m3fn) runs on a bf16 lhs).  With
    ``keep`` (a dict), keep[name] = (workload, device output of the timed
    gmm) for the CPU leg's distance from the W4A16 result."""
    from dw_tpu_amd.workloads import make_gmm_workload
    wl = make_gmm_workload(name)
    b = GmmBench(wl, dev, copies_for(wl), mode)

    def run():
        r = gmm_result(wl, time_median(b.step, steps, warmup), mode)
        if keep is not None:
            keep[f"{name}_{mode}"] = (wl, b.out[0])
        q_ms = time_steps(b.quant_step, steps, warmup)
        qb = wl.M * wl.K * 2 + (wl.M * wl.K // 2 if mode == "mxfp4" else wl.M * wl.K) + wl.M * wl.K // 32
        r["quant"] = {"ms": round(q_ms, 5), "GB_s": round(qb / (q_ms * 1e-3) / 1e9, 1),
                      "hbm_frac": round(qb / (q_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": qb}
        both = time_steps(b.quant_and_step, steps, warmup)
        r["ms_with_quant"] = round(both, 5)
        r["TFLOP_s_with_quant"] = round(wl.flops() / (both * 1e-3) / 1e12, 1)
        return {f"{name}_{mode}": r}
    return run


def bench_gmm_mx(name, dev, steps, warmup, mode="mx"):
    return prep_gmm_mx(name, dev, steps, warmup, mode=mode)()[f"{name}_{mode}"]


def prep_dispatch_combine(dev, steps, warmup):
    """decode_down routing through the C ABI with preallocated outputs:
    dispatch indices for 512 tokens x top-8 over 32 experts, the row gather
    of hidden [512, 2048] into [4096, 2048], and the combine of the
    down-projection output [4096, 7168] back to [512, 7168].

    The gather and combine rotate over input/output sets of more than twice
    the 256 MB Infinity Cache, so each launch reads its inputs from HBM.
    Algorithmic bytes: the gather reads each source row once (the 2 MB
    hidden, whose rows it reads 8 times from cache) and writes the 16.8 MB
    routed copy; the combine reads y once, writes out once, plus indices and
    weights."""
    import numpy as np
    import torch
    from dw_tpu_amd import _lib
    from dw_tpu_amd.workloads import make_gmm_workload
    lib = _lib.load()
    wl = make_gmm_workload("decode_down", with_data=False)
    n = wl.M
    i32 = dict(dtype=torch.int32, device=dev)
    ids = torch.from_numpy(wl.topk_ids).to(dev)
    perm, tok, rev = (torch.empty(n, **i32) for _ in range(3))
    gs, goff, flags = torch.empty(wl.E, **i32), torch.empty(wl.E + 1, **i32), torch.zeros(1, **i32)
    wsb = ctypes.c_int64()
    _lib.call("dwm_moe_dispatch_workspace_size", n, wl.E, ctypes.byref(wsb))
    ws = torch.empty(wsb.value, dtype=torch.uint8, device=dev)
    st = _lib.stream_handle(dev)
    P = _lib.ptr
    disp_args = (P(ids), wl.T, wl.topk, wl.E, P(perm), P(tok), P(rev), P(gs), P(goff), P(flags), P(ws), st)
    rng = np.random.Generator(np.random.PCG64(11))
    hidden0 = torch.from_numpy(rng.standard_normal((wl.T, wl.K), dtype=np.float32)).to(torch.bfloat16).to(dev)
    y0 = torch.from_numpy(rng.standard_normal((n, wl.N), dtype=np.float32)).to(torch.bfloat16).to(dev)
    w = torch.from_numpy(wl.topk_weights).to(dev)

    def call(fn, args):
        rc = fn(*args)
        if rc:
            raise RuntimeError(lib.dwm_last_error().decode())

    call(lib.dwm_moe_dispatch, disp_args)  # the gather and combine read its indices
    set_bytes = (wl.T + n) * wl.K * 2
    gc = -(-2 * MALL_BYTES // set_bytes)
    hiddens = [hidden0.clone() for _ in range(gc)]
    xs = [torch.empty((n, wl.K), dtype=torch.bfloat16, device=dev) for _ in range(gc)]
    gargs = [(P(hiddens[c]), wl.T, wl.K * 2, P(tok), n, P(xs[c]), st) for c in range(gc)]
    set_bytes = (n + wl.T) * wl.N * 2
    cc = -(-2 * MALL_BYTES // set_bytes)
    ys = [y0.clone() for _ in range(cc)]
    outs = [torch.empty((wl.T, wl.N), dtype=torch.bfloat16, device=dev) for _ in range(cc)]
    cargs = [(P(ys[c]), _lib.BF16, n, wl.N, P(rev), P(w), _lib.F32, wl.T, wl.topk, P(outs[c]), _lib.BF16, st)
             for c in range(cc)]

    # The argument tuples hold raw device addresses: the closure keeps the
    # tensors behind them alive (freed, their memory would go to later inputs).
    keep = (ids, perm, tok, rev, gs, goff, flags, ws, hidden0, y0, w, hiddens, xs, ys, outs)

    def run():
        assert keep
        res = {}
        ms = time_steps(lambda i: call(lib.dwm_moe_dispatch, disp_args), steps, warmup)
        res["dispatch"] = {"ms": round(ms, 5), "ids": n, "experts": wl.E, "kernels": 1 if n <= 8192 else 3,
                           "note": "launch-latency bound (one 1024-thread block)"}
        ms = time_steps(lambda i: call(lib.dwm_row_gather, gargs[i % gc]), steps, warmup)
        gb = wl.T * wl.K * 2 + n * wl.K * 2 + n * 4
        res["row_gather"] = {"ms": round(ms, 5), "GB_s": round(gb / (ms * 1e-3) / 1e9, 1), "rows": n, "H": wl.K,
                             "hbm_frac": round(gb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": gb,
                             "rotated_sets": gc}
        ms = time_steps(lambda i: call(lib.dwm_moe_combine, cargs[i % cc]), steps, warmup)
        gb = n * wl.N * 2 + wl.T * wl.N * 2 + n * 8
        res["combine"] = {"ms": round(ms, 5), "GB_s": round(gb / (ms * 1e-3) / 1e9, 1), "T": wl.T, "topk": wl.topk,
                          "H": wl.N, "hbm_frac": round(gb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": gb,
                          "rotated_sets": cc}
        return res
    return run


def _block_weights(dev, E, H, I, copies):
    """Random gate/up and down expert weights (prepacked), ``copies`` sets."""
    import torch
    from dw_tpu_amd import fp4_weight_to_codes
    w13s, w2s = [], []
    for _ in range(copies):
        r13 = torch.randint(0, 256, (E, H, I), dtype=torch.uint8, device=dev)   # [E, H, 2I] packed
        s13 = torch.randint(121, 130, (E, H // 32, 1, 2 * I), dtype=torch.uint8, device=dev)
        w13s.append(fp4_weight_to_codes(r13, s13, gate_up=True))
        r2 = torch.randint(0, 256, (E, I, H // 2), dtype=torch.uint8, device=dev)
        s2 = torch.randint(118, 124, (E, I // 32, 1, H), dtype=torch.uint8, device=dev)
        w2s.append(fp4_weight_to_codes(r2, s2))
        del r13, s13, r2, s2
    return w13s, w2s


def _block_result(wl, ms, H, I):
    nonempty = int((wl.group_sizes > 0).sum())
    n = wl.M
    wbytes = nonempty * (H * 2 * I // 2 + H // 32 * 2 * I + I * H // 2 + I // 32 * H)
    # hidden read once, h written by gmm1 and read by gmm2, y written by gmm2
    # and read by the combine, out written (gmm1 reads the routed rows of
    # hidden itself: no gathered copy)
    act_bytes = wl.T * H * 2 + 2 * n * I * 2 + 2 * n * H * 2 + wl.T * H * 2
    flops = 2 * n * H * 2 * I + 2 * n * I * H
    gbs = (wbytes + act_bytes) / (ms * 1e-3) / 1e9
    return {"ms": round(ms, 5), "GB_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "TFLOP_s": round(flops / (ms * 1e-3) / 1e12, 1), "mfma_bf16_frac": round(flops / (ms * 1e-3) / 1e12
                                                                                   / BF16_PEAK_TFLOPS, 4),
            "bytes": wbytes + act_bytes, "flops": flops, "T": wl.T, "topk": wl.topk, "H": H, "I": I, "E": wl.E,
            "nonempty_groups": nonempty}


def prep_moe_block(dev, steps, warmup):
    """The expert block through ``moe_block``: dispatch + gmm1 over the routed
    rows of hidden [T, 7168] (gathered inside the gmm) x [7168, 2x2048] with
    the fused silu_and_mul_with_clamp + gmm2 [., 2048] x [2048, 7168] +
    combine to [T, 7168], over 32 experts.  Decode: 256 tokens x top-8
    (decode_gate_up routing), also replayed from a captured HIP graph;
    prefill: 8192 tokens x top-8 (the prefill workload's skewed routing).
    Two weight copies are rotated."""
    import numpy as np
    import torch
    from dw_tpu_amd import MoeBlockGraph, moe_block
    from dw_tpu_amd.workloads import make_gmm_workload
    copies = 2
    cases = []
    for name, key in (("decode_gate_up", "moe_block_decode"), ("prefill", "moe_block_prefill")):
        wl = make_gmm_workload(name, with_data=False)
        H, I, E = wl.K, wl.N // 2, wl.E
        w13s, w2s = _block_weights(dev, E, H, I, copies)
        rng = np.random.Generator(np.random.PCG64(12))
        hidden = torch.from_numpy(rng.standard_normal((wl.T, H), dtype=np.float32)).to(torch.bfloat16).to(dev)
        ids = torch.from_numpy(wl.topk_ids).to(dev)
        wts = torch.from_numpy(wl.topk_weights).to(dev)
        graphs = None
        if name == "decode_gate_up":
            # the same block captured once per weight copy (MoeBlockGraph) and replayed
            graphs = [MoeBlockGraph(hidden, ids, wts, w13s[c], w2s[c], E) for c in range(copies)]
        cases.append((name, key, wl, H, I, E, w13s, w2s, hidden, ids, wts, graphs))

    def run():
        res = {}
        for name, key, wl, H, I, E, w13s, w2s, hidden, ids, wts, graphs in cases:
            ms = time_steps(lambda i: moe_block(hidden, ids, wts, w13s[i % copies], w2s[i % copies], E), steps,
                            warmup)
            res[key] = _block_result(wl, ms, H, I)
            # The same block in the MX mode (e4m3 activations with e8m0
            # block-32 scales into both gmm: a lossier computation).
            ms_mx = time_steps(lambda i: moe_block(hidden, ids, wts, w13s[i % copies], w2s[i % copies], E,
                                                   lhs_quant_dtype=torch.float8_e4m3fn), steps, warmup)
            mx = _block_result(wl, ms_mx, H, I)
            res[key + "_mx"] = {"ms": mx["ms"], "TFLOP_s": mx["TFLOP_s"],
                                "mfma_fp8_frac": round(mx["TFLOP_s"] / FP8_PEAK_TFLOPS, 4),
                                "note": "the same block with lhs_quant_dtype=float8_e4m3fn (hidden and the "
                                        "activation quantized in the step)"}
            if graphs is not None:
                ms_graph = time_steps(lambda i: graphs[i % copies](), steps, warmup)
                g = _block_result(wl, ms_graph, H, I)
                res["moe_block_decode_graph"] = {"ms": g["ms"], "GB_s": g["GB_s"], "TFLOP_s": g["TFLOP_s"],
                                                 "note": "the same block replayed from a captured HIP graph"}
        return res
    return run


def prep_routing(dev, steps, warmup):
    """The router (dwm_route_topk) at the decode workload's routing (256
    tokens, 32 experts, top-8 softmax) and at a DeepSeek-V4-like prefill
    (8192 tokens, 256 experts, top-8 sqrtsoftplus + correction bias +
    renormalize), f32 logits, bf16 weights.  Bytes = logits + ids + weights."""
    import torch
    from dw_tpu_amd import _lib
    lib = _lib.load()
    st = _lib.stream_handle(dev)
    cases = []
    for name, T, E, k, fn, biased in (("route_decode", 256, 32, 8, 0, False),
                                      ("route_prefill_dsv4", 8192, 256, 8, 2, True)):
        g = torch.Generator(device="cpu").manual_seed(T + E)
        logits = torch.randn((T, E), generator=g).to(dev)
        bias = (torch.randn((E,), generator=g) * 0.1).to(dev) if biased else None
        w = torch.empty((T, k), dtype=torch.bfloat16, device=dev)
        ids = torch.empty((T, k), dtype=torch.int32, device=dev)
        args = (_lib.ptr(logits), _lib.F32, T, E, k, fn, _lib.ptr(bias), None, 1 if biased else 0, None,
                _lib.ptr(w), _lib.BF16, _lib.ptr(ids), st)

        cases.append((name, T, E, k, biased, args, (logits, bias, w, ids)))

    def step(args):
        if lib.dwm_route_topk(*args):
            raise RuntimeError(lib.dwm_last_error().decode())

    def run():
        res = {}
        for name, T, E, k, biased, args, _ in cases:
            ms = time_steps(lambda i: step(args), steps, warmup)
            b = T * E * 4 + T * k * 6 + (E * 4 if biased else 0)
            res[name] = {"ms": round(ms, 5), "GB_s": round(b / (ms * 1e-3) / 1e9, 1), "bytes": b, "T": T, "E": E,
                         "topk": k}
        return res
    return run


def prep_formats(dev, steps, warmup):
    """Checkpoint weight formats (load-time kernels) at the decode shapes:
    an MXFP4 expert checkpoint of the gate/up weight (32 experts, N = 4096,
    K = 7168: [E, N, K/2] codes + [E, N, K/32] scales -> [E, K, N/2] +
    [E, K/32, N]) and a DeepSeek FP8 128x128-block weight (N = 4096,
    K = 7168, [N, K] -> [K, N]), through the C ABI with preallocated outputs.
    Bytes = every input and output byte once."""
    import torch
    from dw_tpu_amd import _lib
    lib = _lib.load()
    st = _lib.stream_handle(dev)
    E, N, K = 32, 4096, 7168
    blocks = torch.randint(0, 256, (E, N, K // 2), dtype=torch.uint8, device=dev)
    scales = torch.randint(110, 135, (E, N, K // 32), dtype=torch.uint8, device=dev)
    codes = torch.empty((E, K, N // 2), dtype=torch.uint8, device=dev)
    scode = torch.empty((E, K // 32, N), dtype=torch.uint8, device=dev)
    status = torch.empty(2, dtype=torch.int32, device=dev)
    args = (_lib.ptr(blocks), _lib.ptr(scales), E, N, K, 0, _lib.ptr(codes), _lib.ptr(scode), _lib.ptr(status), st)

    def run_mx(i):
        if lib.dwm_mxfp4_requant(*args):
            raise RuntimeError(lib.dwm_last_error().decode())
    b_mx = 2 * (blocks.numel() + scales.numel())
    w = torch.randint(0, 0x7E, (N, K), dtype=torch.uint8, device=dev)
    wsc = torch.full((N // 128, K // 128), 2.0 ** -8, dtype=torch.float32, device=dev)
    w_out = torch.empty((K, N), dtype=torch.uint8, device=dev)
    s_out = torch.empty((K // 128, N), dtype=torch.float32, device=dev)
    args8 = (_lib.ptr(w), _lib.ptr(wsc), K, N, 1, _lib.ptr(w_out), _lib.ptr(s_out), _lib.ptr(status), st)

    def run_f8(i):
        if lib.dwm_fp8_block_requant(*args8):
            raise RuntimeError(lib.dwm_last_error().decode())
    b_f8 = 2 * w.numel() + 4 * (wsc.numel() + s_out.numel())
    # The argument tuples hold raw device addresses: the closure keeps the
    # tensors behind them alive.
    keep = (blocks, scales, codes, scode, status, w, wsc, w_out, s_out)

    def run():
        assert keep
        res = {}
        ms = time_steps(run_mx, steps, warmup)
        res["mxfp4_requant"] = {"ms": round(ms, 5), "GB_s": round(b_mx / (ms * 1e-3) / 1e9, 1),
                                "hbm_frac": round(b_mx / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": b_mx,
                                "E": E, "N": N, "K": K}
        ms = time_steps(run_f8, steps, warmup)
        res["fp8_block_requant"] = {"ms": round(ms, 5), "GB_s": round(b_f8 / (ms * 1e-3) / 1e9, 1),
                                    "hbm_frac": round(b_f8 / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": b_f8,
                                    "N": N, "K": K}
        return res
    return run


def prep_dense(dev, steps, warmup, ms_list=(1, 16, 128, 1024, 4096)):
    """Dense FP8 GEMM (K=7168, N=4096) at each M, W8A16 and W8A8, through
    the C ABI with prepacked weights; 10 rotated weight copies (~290 MB) keep
    the small-M weight stream out of the Infinity Cache."""
    import torch
    from dw_tpu_amd import _lib
    from dw_tpu_amd.dense_fp8 import prepack_fp8
    from dw_tpu_amd.workloads import make_dense_workload
    lib = _lib.load()
    st = _lib.stream_handle(dev)
    P = _lib.ptr
    cases = []
    for m in ms_list:
        wl = make_dense_workload(m)
        k, n = wl.K, wl.N
        copies = 10 if m <= 128 else 1
        w = torch.from_numpy(wl.wq).to(dev)
        pws = [prepack_fp8(w) for _ in range(copies)]
        del w
        x = _to_dev_bf16(wl.x_bits, dev)
        xq = torch.from_numpy(wl.xq).to(dev)
        sx = torch.from_numpy(wl.sx).to(dev)
        s16 = torch.from_numpy(wl.s_w8a16.reshape(k // 128, n)).to(dev)
        sw = torch.from_numpy(wl.sw).to(dev)
        out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        wsb = ctypes.c_int64()
        _lib.call("dwm_dense_fp8_workspace_size", m, k, n, ctypes.byref(wsb))
        ws = torch.empty(max(1, wsb.value), dtype=torch.uint8, device=dev)
        cases.append((m, k, n, copies, pws, x, xq, sx, s16, sw, out, ws, wsb.value))

    def run():
        res = {}
        for m, k, n, copies, pws, x, xq, sx, s16, sw, out, ws, wsb in cases:
            def run16(i):
                rc = lib.dwm_dense_fp8_w8a16(P(x), m, k, n, P(pws[i % copies].weight), P(s16), P(out), P(ws), wsb,
                                             st)
                if rc:
                    raise RuntimeError(lib.dwm_last_error().decode())

            def run8(i):
                rc = lib.dwm_dense_fp8_w8a8(P(xq), P(sx), m, k, n, P(pws[i % copies].weight), P(sw), P(out), P(ws),
                                            wsb, st)
                if rc:
                    raise RuntimeError(lib.dwm_last_error().decode())

            fl = 2 * m * k * n
            for tag, fn, xbytes in (("w8a16", run16, m * k * 2 + (k // 128) * n * 4),
                                    ("w8a8", run8, m * k + m * (k // 128) * 4 + (k // 128) * (n // 128) * 4)):
                ms = time_median(fn, steps, warmup)
                bts = k * n + xbytes + m * n * 2
                gbs = bts / (ms * 1e-3) / 1e9
                tf = fl / (ms * 1e-3) / 1e12
                peak_key, peak = ("mfma_fp8_frac", FP8_PEAK_TFLOPS) if tag == "w8a8" else ("mfma_bf16_frac",
                                                                                        BF16_PEAK_TFLOPS)
                res[f"dense_{tag}_M{m}"] = {"ms": round(ms, 5), "GB_s": round(gbs, 1), "TFLOP_s": round(tf, 2),
                                            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), peak_key: round(tf / peak, 4),
                                            "bytes": bts, "flops": fl}
        return res
    return run


TIMELINE_SLOTS = 24  # words per block record of the timeline build (kTlSlots in csrc/gmm_fp4.hip)
DENSE_STEP_SLOTS = 10  # words per wave record of the dense step accounting (kDsSlots in csrc/dense_fp8.hip)
GMM_STEP_SLOTS = 10  # words per wave record of the gmm step accounting (kGsSlots in csrc/gmm_fp4.hip)


def probe_gmm_steps(dev, names=("decode_gate_up", "decode_down", "prefill")):
    """Profiling aid (``--probe gmm_steps``): where a 64-deep K step of the
    bf16 gmm goes, from the library's timeline build (the same kernels with
    per-wave s_memtime sums compiled in), one launch per workload after at
    least 0.2 s of warmup launches.  Every wave of a tile block sums its shader
    cycles waiting before each barrier (producers: vmcnt for their loads;
    consumers: their LDS reads), at the barrier, and working between barriers.
    Reported per K step (the sums over the T + 1 barriers, the epilogue's
    included, over the T steps) and per tile shape (16-row blocks, narrow tiles apart)
    for the older and the younger consumer of each SIMD (waves 0-3 and 4-7)
    and the producers (waves 8-11), with the role's prologue (start to the
    first wait) and end (last barrier to stores issued), and the shader clock
    (s_memtime against s_memrealtime)."""
    import numpy as np
    import torch
    from dw_tpu_amd import _lib, fp4_weight_to_codes
    from dw_tpu_amd.workloads import make_gmm_workload
    lib = ctypes.CDLL(os.path.join(os.path.dirname(_lib.LIB_PATH), "libdwtpu_moe_timeline.so"))
    for n, a in _lib.SIGNATURES.items():
        f = getattr(lib, n)
        f.argtypes = a
        f.restype = _lib._RESTYPES.get(n, ctypes.c_int)
    lib.dwm_gmm_steps_set.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    st = _lib.stream_handle(dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    out_all = {}
    for name in names:
        wl = make_gmm_workload(name)
        pw = fp4_weight_to_codes(torch.from_numpy(wl.rhs_e2m1).to(dev), torch.from_numpy(wl.scale_codes).to(dev))
        lhs = torch.from_numpy(wl.lhs_bits.view(np.int16)).view(torch.bfloat16).to(dev)
        gs = torch.from_numpy(wl.group_sizes).to(dev)
        out = torch.empty((wl.M, wl.N), dtype=torch.bfloat16, device=dev)
        waves = 16 * 16384
        buf = torch.zeros(waves * GMM_STEP_SLOTS, dtype=torch.int64, device=dev)

        def launch():
            rc = lib.dwm_gmm_fp4(P(lhs), wl.M, wl.K, P(pw.weight), P(pw.scale), P(gs), wl.E, None, wl.E, wl.N,
                                 P(out), _lib.BF16, 0, 0, st)
            if rc:
                raise RuntimeError(lib.dwm_last_error().decode())

        if lib.dwm_gmm_steps_set(None, 0):
            raise RuntimeError(lib.dwm_last_error().decode())
        t_end = time.time() + 0.2
        n = 0
        while n < 30 or time.time() < t_end:
            for _ in range(10):
                launch()
            n += 10
            torch.cuda.synchronize()
        if lib.dwm_gmm_steps_set(P(buf), waves):
            raise RuntimeError(lib.dwm_last_error().decode())
        launch()
        torch.cuda.synchronize()
        lib.dwm_gmm_steps_set(None, 0)
        d = buf.view(waves, GMM_STEP_SLOTS).cpu().numpy().astype(np.int64)
        wave = np.arange(waves) % 16
        live = d[:, 8] != 0
        d, wave = d[live], wave[live]
        role, rows, narrow = d[:, 6] & 0xFF, (d[:, 6] >> 8) & 0xFFFF, (d[:, 6] >> 24) & 1
        # T + 1 barriers (the K steps' and the epilogue's) around T steps of work.
        steps = np.maximum(d[:, 5] - 1, 1).astype(np.float64)
        clock = float(d[:, 9].sum() / ((d[:, 8] - d[:, 7]).sum() / 100.0) / 1e3)
        shapes = {}
        for nh in sorted(set(((rows + 15) // 16).tolist())):
            for nw in (0, 1):
                tile = ((rows + 15) // 16 == nh) & (narrow == nw)
                if not tile.any():
                    continue
                roles = {}
                for rname, sel in (("older consumer", (role == 2) & (wave < 4)),
                                   ("younger consumer", (role == 2) & (wave >= 4)),
                                   ("producer", role == 1)):
                    m = tile & sel
                    if not m.any():
                        continue
                    roles[rname] = {"waves": int(m.sum()),
                                    "wait_per_step": round(float((d[m, 1] / steps[m]).mean()), 1),
                                    "barrier_per_step": round(float((d[m, 2] / steps[m]).mean()), 1),
                                    "work_per_step": round(float((d[m, 3] / steps[m]).mean()), 1),
                                    "prologue": round(float(d[m, 0].mean()), 1),
                                    "end": round(float(d[m, 4].mean()), 1)}
                shapes[f"{nh} blocks{' narrow' if nw else ''}"] = {
                    "tiles": int((tile & (role == 1) & (wave == 8)).sum()),
                    "barriers": int(np.median(d[tile, 5])), "roles": roles}
        out_all[name] = {"shader_clock_GHz": round(clock, 3), "shapes": shapes}
        log(f"gmm steps {name}: {out_all[name]}")
    return out_all


def probe_dense_steps(dev, ms_list=(128, 1024)):
    """Profiling aid (``--probe dense_steps``): where a K step of the dense
    FP8 MFMA tile kernel goes, from the library's timeline build (the same
    kernels with per-wave s_memtime sums compiled in): one launch of the
    library's default plan per (M, variant) after at least 0.2 s of warmup
    launches (K = 7168, N = 4096, the dense workload).  Each wave sums its
    shader cycles waiting for data, at barriers and working between barriers;
    reported per step, separately for the first and the second wave of each
    SIMD (waves w and w + 4 of an 8-wave block), with the prologue (entry to
    the first wait), the epilogue (loop end to its stores complete) and the
    shader clock (s_memtime against s_memrealtime)."""
    import numpy as np
    import torch
    from dw_tpu_amd import _lib
    from dw_tpu_amd.dense_fp8 import prepack_fp8
    from dw_tpu_amd.workloads import make_dense_workload
    lib = ctypes.CDLL(os.path.join(os.path.dirname(_lib.LIB_PATH), "libdwtpu_moe_timeline.so"))
    for n, a in _lib.SIGNATURES.items():
        f = getattr(lib, n)
        f.argtypes = a
        f.restype = _lib._RESTYPES.get(n, ctypes.c_int)
    lib.dwm_dense_steps_set.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    st = _lib.stream_handle(dev)
    P = _lib.ptr
    res = {}
    for m in ms_list:
        wl = make_dense_workload(m)
        k, n = wl.K, wl.N
        pw = prepack_fp8(torch.from_numpy(wl.wq).to(dev))
        x = _to_dev_bf16(wl.x_bits, dev)
        xq, sx, sw = (torch.from_numpy(v).to(dev) for v in (wl.xq, wl.sx, wl.sw))
        s16 = torch.from_numpy(wl.s_w8a16.reshape(k // 128, n)).to(dev)
        out = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        wsb = ctypes.c_int64()
        _lib.call("dwm_dense_fp8_workspace_size", m, k, n, ctypes.byref(wsb))
        ws = torch.empty(max(1, wsb.value), dtype=torch.uint8, device=dev)
        for tag in ("w8a16", "w8a8"):
            def launch():
                if tag == "w8a16":
                    rc = lib.dwm_dense_fp8_w8a16(P(x), m, k, n, P(pw.weight), P(s16), P(out), P(ws), wsb.value, st)
                else:
                    rc = lib.dwm_dense_fp8_w8a8(P(xq), P(sx), m, k, n, P(pw.weight), P(sw), P(out), P(ws),
                                                wsb.value, st)
                if rc:
                    raise RuntimeError(lib.dwm_last_error().decode())

            if lib.dwm_dense_steps_set(None, 0):
                raise RuntimeError(lib.dwm_last_error().decode())
            t_end = time.time() + 0.2
            done = 0
            while done < 100 or time.time() < t_end:
                for _ in range(20):
                    launch()
                done += 20
                torch.cuda.synchronize()
            plan = _lib.DensePlan()
            if lib.dwm_dense_fp8_last_plan(ctypes.byref(plan)):
                raise RuntimeError(lib.dwm_last_error().decode())
            waves = 16 * 4096
            buf = torch.zeros(waves * DENSE_STEP_SLOTS, dtype=torch.int64, device=dev)
            if lib.dwm_dense_steps_set(P(buf), waves):
                raise RuntimeError(lib.dwm_last_error().decode())
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            launch()
            e1.record()
            torch.cuda.synchronize()
            lib.dwm_dense_steps_set(None, 0)
            d = buf.view(waves, DENSE_STEP_SLOTS).cpu().numpy().astype(np.int64)
            wave = np.arange(waves) % 16
            live = d[:, 8] != 0
            d, wave = d[live], wave[live]
            nw = int(wave.max()) + 1
            steps = d[:, 5].astype(np.float64)
            clock = float(d[:, 9].sum() / ((d[:, 8] - d[:, 7]).sum() / 100.0) / 1e3)
            pos = {}
            for name, sel in (("first wave of a SIMD", wave < 4), ("second wave of a SIMD", wave >= 4)):
                if not sel.any():
                    continue
                pos[name] = {"wait_per_step": round(float((d[sel, 1] / steps[sel]).mean()), 1),
                             "barrier_per_step": round(float((d[sel, 2] / steps[sel]).mean()), 1),
                             "work_per_step": round(float((d[sel, 3] / steps[sel]).mean()), 1),
                             "prologue": round(float(d[sel, 0].mean()), 1),
                             "epilogue": round(float(d[sel, 4].mean()), 1)}
            res[f"dense_{tag}_M{m}"] = {
                "plan": [plan.kernel, plan.tile_m, plan.tile_n, plan.ksplit, plan.stages],
                "event_us": round(e0.elapsed_time(e1) * 1e3, 2), "waves": int(len(d)), "waves_per_block": nw,
                "steps_per_wave": float(np.median(steps)), "shader_clock_GHz": round(clock, 3),
                "launch_span_us": round(float((d[:, 8].max() - d[:, 7].min()) / 100.0), 2),
                "cycles": pos}
            log(f"dense steps M={m} {tag}: {res[f'dense_{tag}_M{m}']}")
    return res


def probe_timeline(dev, names=("decode_gate_up", "decode_down", "prefill")):
    """Profiling aid (``--probe timeline``): the bf16 gmm's per-block
    timeline from the library's timeline build (libdwtpu_moe_timeline.so:
    the same kernels with s_memrealtime / s_memtime stores compiled in), one
    launch per workload after at least 0.2 s of warmup launches.  Per block: entry, the
    tile's rows, consumer wave 0's first barrier / K-loop end / stores issued,
    every wave's exit (100 MHz realtime, one clock for all XCDs) and wave 0's
    shader-clock counter.  Reports, per row-block count (narrow tiles apart),
    the blocks' spans from entry to the last wave's exit; the mean phases of
    consumer wave 0; tiles per CU and the quantiles of the tile blocks'
    start times (the rounds of a multi-round launch); the shader clock."""
    import numpy as np
    import torch
    from dw_tpu_amd import _lib, fp4_weight_to_codes
    from dw_tpu_amd.workloads import make_gmm_workload
    lib = ctypes.CDLL(os.path.join(os.path.dirname(_lib.LIB_PATH), "libdwtpu_moe_timeline.so"))
    for n, a in _lib.SIGNATURES.items():
        f = getattr(lib, n)
        f.argtypes = a
        f.restype = _lib._RESTYPES.get(n, ctypes.c_int)
    lib.dwm_timeline_set.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    st = _lib.stream_handle(dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    out_all = {}
    for name in names:
        wl = make_gmm_workload(name)
        pw = fp4_weight_to_codes(torch.from_numpy(wl.rhs_e2m1).to(dev), torch.from_numpy(wl.scale_codes).to(dev))
        lhs = torch.from_numpy(wl.lhs_bits.view(np.int16)).view(torch.bfloat16).to(dev)
        gs = torch.from_numpy(wl.group_sizes).to(dev)
        out = torch.empty((wl.M, wl.N), dtype=torch.bfloat16, device=dev)
        blocks = 16384
        buf = torch.zeros(blocks * TIMELINE_SLOTS, dtype=torch.int64, device=dev)

        def launch():
            rc = lib.dwm_gmm_fp4(P(lhs), wl.M, wl.K, P(pw.weight), P(pw.scale), P(gs), wl.E, None, wl.E, wl.N,
                                 P(out), _lib.BF16, 0, 0, st)
            if rc:
                raise RuntimeError(lib.dwm_last_error().decode())

        if lib.dwm_timeline_set(None, 0):
            raise RuntimeError(lib.dwm_last_error().decode())
        # At least 0.2 s of back-to-back launches first: after the host-side
        # input generation the power manager needs tens of ms of load to
        # bring the clock back up.
        t_end = time.time() + 0.2
        n = 0
        while n < 30 or time.time() < t_end:
            for _ in range(10):
                launch()
            n += 10
            torch.cuda.synchronize()
        if lib.dwm_timeline_set(P(buf), blocks):
            raise RuntimeError(lib.dwm_last_error().decode())
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        launch()
        e1.record()
        torch.cuda.synchronize()
        lib.dwm_timeline_set(None, 0)
        d = buf.view(blocks, TIMELINE_SLOTS).cpu().numpy().astype(np.int64)
        d = d[d[:, 0] != 0]
        rows = d[:, 3] & 0xFFFF
        narrow = (d[:, 3] >> 16) & 1
        exits = np.where(d[:, 8:20] != 0, d[:, 8:20], 0).max(axis=1)
        t0 = d[:, 0].min()
        tiles = d[rows > 0]
        tr, tn, tx = rows[rows > 0], narrow[rows > 0], exits[rows > 0]
        span = (tx - tiles[:, 0]) / 100.0
        classes = {}
        for nh in sorted(set(((tr + 15) // 16).tolist())):
            for nw in (0, 1):
                m = ((tr + 15) // 16 == nh) & (tn == nw)
                if m.any():
                    classes[f"{nh} blocks{' narrow' if nw else ''}"] = {
                        "tiles": int(m.sum()), "span_us_mean": round(float(span[m].mean()), 1),
                        "span_us_min": round(float(span[m].min()), 1), "span_us_max": round(float(span[m].max()), 1)}
        ph = lambda a, b: round(float(((tiles[:, b] - tiles[:, a]) / 100.0).mean()), 2)  # noqa: E731
        cu = (tiles[:, 1] >> 32) * 256 + ((tiles[:, 1] >> 8) & 0xFF)  # XCC_ID, then CU / SH / SE of HW_ID
        per_cu = np.unique(np.unique(cu, return_counts=True)[1], return_counts=True)
        starts = np.sort(tiles[:, 0] - t0) / 100.0
        w0 = (tiles[:, 8] > tiles[:, 0]) & (tiles[:, 20] > tiles[:, 7])
        clock = float(np.median((tiles[w0, 20] - tiles[w0, 7]) / (tiles[w0, 8] - tiles[w0, 0]) / 10.0))
        out_all[name] = {
            "event_us": round(e0.elapsed_time(e1) * 1e3, 1),
            "blocks": int(len(d)), "tile_blocks": int(len(tiles)),
            "first_entry_to_last_exit_us": round(float((exits.max() - t0) / 100.0), 1),
            "shader_clock_GHz": round(clock, 3),
            "by_row_blocks": classes,
            "phases_us_mean": {"entry_to_tile": ph(0, 2), "tile_to_first_barrier": ph(2, 4), "k_loop": ph(4, 5),
                               "epilogue_stores_issued": ph(5, 6),
                               "stores_to_last_exit": round(float(((tx - tiles[:, 6]) / 100.0).mean()), 2)},
            "tiles_per_cu": {int(k): int(v) for k, v in zip(*per_cu)},
            "tile_start_us_quantiles": [round(float(np.quantile(starts, q)), 1) for q in (0, .125, .25, .375, .5,
                                                                                           .625, .75, .875, 1)],
        }
        log(f"timeline {name}: {out_all[name]}")
        del pw, lhs, gs, out, buf
    return out_all


def probe_equal_experts(dev, kind):
    """Profiling aid (``--probe``): the grouped matmul on synthetic equal
    experts (K = 7168, N = 4096, random prepacked weights, two copies
    rotated), bf16 and MX modes, 5 rounds of 30 steps, median us per launch.

    kind "rows": 28 experts with 16 .. 96 rows each (the MFMA row blocks a
    decode tile carries); kind "cus": 28 experts x 73 rows at K = 7168 (224
    tiles, like decode_gate_up), 32 x 73 rows at K = 6272 (256 tiles holding
    the same total work: every CU busy) and 32 x 73 at K = 7168."""
    import statistics
    import torch
    from dw_tpu_amd import _lib, fp4_weight_to_codes, mx_quantize
    lib = _lib.load()
    P = ctypes.c_void_p
    st = _lib.stream_handle(dev)
    N = 4096
    shapes = ([(28, r, 7168) for r in (16, 32, 48, 64, 73, 80, 96)] if kind == "rows"
              else [(28, 73, 7168), (32, 73, 6272), (32, 73, 7168)])
    weights = {}
    cases = []
    for E, rows, K in shapes:
        if (E, K) not in weights:
            ws = []
            for _ in range(2):
                r = torch.randint(0, 256, (E, K, N // 2), dtype=torch.uint8, device=dev)
                s = torch.randint(122, 128, (E, K // 32, 1, N), dtype=torch.uint8, device=dev)
                ws.append(fp4_weight_to_codes(r, s))
                del r, s
            weights[(E, K)] = ws
        ws = weights[(E, K)]
        M = E * rows
        x = torch.randn(M, K, device=dev).to(torch.bfloat16)
        q = mx_quantize(x)
        gs = torch.full((E,), rows, dtype=torch.int32, device=dev)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        for mx in (False, True):
            def step(i, ws=ws, x=x, q=q, gs=gs, out=out, E=E, K=K, M=M, mx=mx):
                w = ws[i % 2]
                tail = (P(w.weight.data_ptr()), P(w.scale.data_ptr()), P(gs.data_ptr()), E, None, E, N,
                        P(out.data_ptr()), _lib.BF16, 0, 0, st)
                rc = (lib.dwm_gmm_fp4_mx(P(q.codes.data_ptr()), P(q.scales.data_ptr()), M, None, M, K, *tail) if mx
                      else lib.dwm_gmm_fp4(P(x.data_ptr()), M, K, *tail))
                if rc:
                    raise RuntimeError(lib.dwm_last_error().decode())
            cases.append((f"E{E}_rows{rows}_K{K}_{'mx' if mx else 'bf16'}", step, (x, q, gs, out)))
    res = {}
    for _ in range(5):
        for name, step, _keep in cases:
            res.setdefault(name, []).append(time_steps(step, 30, 10))
    return {name: round(1e3 * statistics.median(v), 2) for name, v in res.items()}


def profiled_traffic(name="gmm_fp4_decode_gate_up.md"):
    """HBM bytes per launch of the main kernel from the committed rocprofv3
    counter summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), or None."""
    import re
    try:
        text = open(os.path.join(ROOT, "profiles", name)).read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes:\s*(\d+)", text, re.M)
    return int(m.group(1)) if m else None


def cpu_workers():
    """CPU threads for the baseline: this process's cores, at most 16 (one
    GPU's share of the host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_gmm_baseline(wl, budget_s, gpu_check=None):
    """numpy oracle of the same math -- exact fp4 dequant to f32, per-expert
    f32 matmul, bf16 round -- over the non-empty experts, one expert per
    worker thread (each with a one-thread BLAS), the workers together on
    ``cpu_workers()`` cores; experts not started within ``budget_s`` are
    skipped (a bounded sample).  Plus one expert on one thread.

    gpu_check = (expert, rows as f32) of the GPU output: the oracle also
    checks those rows against its float64 product (max abs error and
    relative Frobenius error, the bf16 output rounding included)."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import fp4
    from oracle import gmm as ogmm
    from oracle.numerics import bf16_to_f32, round_bf16
    workers = cpu_workers()
    starts = np.concatenate([[0], np.cumsum(wl.group_sizes)])
    lhs = bf16_to_f32(wl.lhs_bits)
    nonempty = [e for e in range(wl.E) if wl.group_sizes[e] > 0]

    def expert_bytes(sz):
        return wl.K * wl.N // 2 + (wl.K // 32) * wl.N + sz * wl.K * 2 + sz * wl.N * 2

    def dequant(e):
        codes = fp4.e2m1_to_codes(fp4.unpack_nibbles(wl.rhs_e2m1[e]))
        return fp4.dequant_fp4_block(codes, fp4.e8m0_decode(wl.scale_codes[e]))

    def one(e):
        round_bf16(lhs[starts[e]:starts[e + 1]] @ dequant(e))

    t0 = time.perf_counter()
    deadline = t0 + budget_s

    def task(e):
        if time.perf_counter() > deadline:
            return None
        one(e)
        return e

    with threadpool_limits(limits=1):
        with ThreadPoolExecutor(workers) as ex:
            done = [e for e in ex.map(task, nonempty) if e is not None]
        dt = time.perf_counter() - t0
        e1 = nonempty[0]
        t1 = time.perf_counter()
        one(e1)
        dt1 = time.perf_counter() - t1
    bts = sum(expert_bytes(int(wl.group_sizes[e])) for e in done)
    fl = sum(2 * int(wl.group_sizes[e]) * wl.K * wl.N for e in done)
    res = {"value": round(bts / dt / 1e9, 4), "unit": "GB/s", "cores": workers, "kind": "port",
           "TFLOP_s": round(fl / dt / 1e12, 4),
           "sample": f"{len(done)} of {len(nonempty)} non-empty experts of {wl.name} (numpy oracle: exact fp4 "
                     f"dequant, f32 matmul, bf16 round; one expert per thread on {workers} threads), {dt:.1f} s",
           "value_1thread": round(expert_bytes(int(wl.group_sizes[e1])) / dt1 / 1e9, 4)}
    if gpu_check is not None:
        e, y = gpu_check
        a = lhs[starts[e]:starts[e + 1]].astype(np.float64)
        w = dequant(e).astype(np.float64)
        ref = a @ w
        err = y.astype(np.float64) - ref
        # the stated per-element tolerance (bf16 output rounding plus K * 2^-24
        # times sum_k |a_k w_k|, any order of f32 accumulation)
        bound = ogmm.error_bound(ref, np.abs(a) @ np.abs(w), wl.K, "bfloat16")
        res["parity"] = {"expert": int(e), "rows": int(ref.shape[0]),
                         "max_abs_err": float(np.abs(err).max()),
                         "rel_frobenius": float(np.linalg.norm(err) / np.linalg.norm(ref)),
                         "max_err_over_tolerance": float((np.abs(err) / bound).max()),
                         "vs": "float64 oracle product of the same bf16 lhs and exact fp4 weights"}
    return res


def cpu_mx_distance(kept, seed=20261202):
    """The MX mode's distance from the reference's arithmetic: max abs and
    relative Frobenius error of the timed MX gmm's output against the W4A16
    float64 result (bf16 lhs, exactly decoded weights) on sampled rows and
    columns -- the same oracle functions and sampling as tests/test_gpu_mx.py.
    kept: {name: (workload, device output)}."""
    import numpy as np
    import torch

    from oracle import gmm as ogmm
    res = {}
    for name, (wl, out) in kept.items():
        rows, cols = ogmm.sample_rows_cols(wl.group_sizes, wl.N, np.random.default_rng(seed))
        got = out[torch.from_numpy(rows).to(out.device)][:, torch.from_numpy(cols).to(out.device)].float().cpu()
        y64 = ogmm.w4a16_rows(wl.lhs_bits[rows], wl.rhs_e2m1, wl.scale_codes, wl.group_sizes, rows, cols)
        st = ogmm.error_stats(got.numpy(), y64)
        res[name] = {"max_abs": round(st["max_abs"], 4), "rel_fro": round(st["rel_fro"], 6),
                     "max_abs_ref": round(float(np.abs(y64).max()), 2), "rows": int(len(rows)),
                     "cols": int(len(cols)),
                     "vs": "float64 W4A16 result (bf16 lhs x exactly decoded fp4 weights), sampled rows x cols"}
    return res


def cpu_dense_baseline(m, budget_s):
    """numpy oracle of the dense W8A16 GEMM (K=7168, N=4096): e4m3 decode,
    per-128-K-block f32 dot times the block scale, f32 accumulate, on
    ``cpu_workers()`` BLAS threads; repeated within the budget."""
    from threadpoolctl import threadpool_limits

    from dw_tpu_amd.workloads import make_dense_workload
    from oracle import dense_fp8 as odf
    from oracle.numerics import bf16_to_f32
    wl = make_dense_workload(m)
    x = bf16_to_f32(wl.x_bits)
    workers = cpu_workers()
    n_runs, t0 = 0, time.perf_counter()
    with threadpool_limits(limits=workers):
        while True:
            odf.matmul_w8a16(x, wl.wq, wl.s_w8a16, accumulate="f32")
            n_runs += 1
            if time.perf_counter() - t0 > budget_s:
                break
    dt = (time.perf_counter() - t0) / n_runs
    fl = 2 * m * wl.K * wl.N
    return {"value": round(fl / dt / 1e12, 4), "unit": "TFLOP/s", "cores": workers, "kind": "port", "ms": round(dt * 1e3, 2),
            "sample": f"{n_runs} run(s) of dense W8A16 M={m}, K={wl.K}, N={wl.N} (numpy oracle, f32 "
                      f"per-K-block products on {workers} BLAS threads)"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--extra", choices=["all", "none"], default="all")
    ap.add_argument("--cpu-budget", type=float, default=15.0,
                    help="seconds of CPU-baseline work (0 skips it)")
    ap.add_argument("--probe", choices=("rows", "cus", "timeline", "gmm_steps", "dense_steps"), default=None,
                    help="profiling aid: the grouped matmul on synthetic equal experts (rows per expert, or all "
                         "CUs busy), the per-block timeline or the per-wave step accounting of the bf16 gmm on "
                         "the three workloads, or the dense FP8 kernel's per-wave step accounting at M = 128 and "
                         "1024 (the last three from the library's timeline build); prints {\"probe\": kind, "
                         "...}; not the benchmark line")
    ap.add_argument("--calib-copy", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (byte-counter calibration)")
    ap.add_argument("--only", choices=ONLY_CHOICES, default=None,
                    help="profiling aid: time one gmm workload line (name, or name_mx for the MX mode) or the "
                         "dense FP8 GEMM at one M (W8A16 then W8A8) and print it as {\"only\": name, ...}; not the "
                         "benchmark line")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the MoE hot path is built and measured on one MI355X's share of "
              "the experts; runs on more than one GPU are not measured here.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    if args.probe == "timeline":
        print(json.dumps({"probe": "timeline", "workloads": probe_timeline(dev)}), flush=True)
        return
    if args.probe == "gmm_steps":
        print(json.dumps({"probe": "gmm_steps", "workloads": probe_gmm_steps(dev)}), flush=True)
        return
    if args.probe == "dense_steps":
        print(json.dumps({"probe": "dense_steps", "cases": probe_dense_steps(dev)}), flush=True)
        return
    if args.probe:
        print(json.dumps({"probe": args.probe, "us": probe_equal_experts(dev, args.probe)}), flush=True)
        return
    if args.calib_copy:
        src = torch.empty(2 ** 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("calib copy: 3 x 1 GiB device-to-device copies done")
        return
    if args.only:
        name = args.only.rsplit("_mx", 1)[0] if "_mx" in args.only else args.only
        if args.only.startswith("dense_M"):
            r = prep_dense(dev, args.steps, args.warmup, ms_list=(int(args.only[len("dense_M"):]),))()
        elif args.only.endswith("_mx"):
            r = bench_gmm_mx(name, dev, args.steps, args.warmup)
        elif args.only.endswith("_mxfp4"):
            r = bench_gmm_mx(name, dev, args.steps, args.warmup, mode="mxfp4")
        else:
            wl1, _, ms1 = bench_gmm(name, dev, args.steps, args.warmup)
            r = gmm_result(wl1, ms1)
        print(json.dumps({"only": args.only, "result": r}), flush=True)
        return
    # The headline's inputs go to HBM first, so that its timed steps can
    # follow the other workloads with no host-side gap: after about a second
    # without GPU work the power manager lowers the clock, and a few warmup
    # launches (under 1 ms of work) run on the way back up.  Measured on this
    # workload: 170-185 us/step after an idle second, 142-155 us/step right
    # after GPU load.
    log("bench: decode_gate_up inputs")
    from dw_tpu_amd.workloads import make_gmm_workload
    wl = make_gmm_workload("decode_gate_up")
    b = GmmBench(wl, dev, copies_for(wl))
    extra = {}
    mx_out = {}  # MX outputs kept for the CPU leg's distance from the W4A16 result
    if args.extra == "all":
        # Inputs of every workload first, then every timed region back to
        # back (the GPU never waits on host-side input generation between
        # them), the headline last.
        # Compute-heavy regions first (they pull the clock down to their own
        # power-limited level), then memory-bound ones, the decode lines
        # last: the headline starts from decode-type load, not from the
        # recovery after a prefill.
        runs = []
        for name in ("prefill",):
            log(f"bench: inputs of {name} gmm, MX mode")
            # The first timed region follows seconds of host-side input
            # generation with the GPU idle: at least 60 warmup launches
            # (~0.1 s of prefill load) let the clock come back up to its
            # power-limited level first (with 5 the MX prefill measured
            # 1.65 ms against 1.55 ms after a settled clock).
            runs.append(prep_gmm_mx(name, dev, args.steps, max(args.warmup, 60), mx_out))
            log(f"bench: inputs of {name} gmm, MXFP4 lhs")
            runs.append(prep_gmm_mx(name, dev, args.steps, args.warmup, mx_out, mode="mxfp4"))
            log(f"bench: inputs of {name} gmm")
            runs.append(prep_gmm(name, dev, args.steps, args.warmup))
        for label, prep in (("moe block", prep_moe_block), ("dense fp8", prep_dense),
                            ("checkpoint formats", prep_formats), ("router", prep_routing),
                            ("dispatch / gather / combine", prep_dispatch_combine)):
            log(f"bench: inputs of {label}")
            runs.append(prep(dev, args.steps, args.warmup))
        for name in ("decode_down", "decode_gate_up"):
            log(f"bench: inputs of {name} gmm, MX mode")
            runs.append(prep_gmm_mx(name, dev, args.steps, args.warmup, mx_out))
            runs.append(prep_gmm_mx(name, dev, args.steps, args.warmup, mx_out, mode="mxfp4"))
        # The last region runs at least 200 warmup launches (~30 ms of
        # decode-type load): after memory-bound regions the power manager
        # can hold the clock low for tens of milliseconds, and a
        # compute-heavier decode started in that state runs up to 20% slow
        # (measured on this workload and decode_down).  The headline then
        # starts from a settled decode clock.
        log("bench: inputs of decode_down gmm")
        runs.append(prep_gmm("decode_down", dev, args.steps, max(args.warmup, 200)))
        log("bench: timed regions")
        for run in runs:
            extra.update(run())
    else:
        runs = []
    log("bench: decode_gate_up gmm (headline)")
    # HEADLINE_SAMPLES samples of --steps back-to-back launches, the first
    # after --warmup untimed ones; value and ms_per_step are their median (a
    # single sample has erred by 10-15% either way against the sustained
    # rate), the first sample and the spread are kept in config.
    first = time_steps(b.step, args.steps, args.warmup)
    samples = sorted([first] + [time_steps(b.step, args.steps, 0) for _ in range(HEADLINE_SAMPLES - 1)])
    ms = samples[len(samples) // 2]
    main_res = gmm_result(wl, ms)
    e_chk = int(np.flatnonzero(wl.group_sizes > 0)[0])
    r0 = int(wl.group_sizes[:e_chk].sum())
    gpu_check = (e_chk, b.out[0][r0:r0 + int(wl.group_sizes[e_chk])].float().cpu().numpy())
    del runs  # the other workloads' inputs are freed only after the headline is timed
    cpu = None
    if args.cpu_budget > 0:
        log("bench: cpu baseline")
        cpu = cpu_gmm_baseline(wl, args.cpu_budget, gpu_check)
        if mx_out:
            for key, d in cpu_mx_distance(mx_out).items():
                extra[key]["vs_w4a16"] = d
        mx_out.clear()
        if args.extra == "all":
            from dw_tpu_amd.workloads import make_gmm_workload
            cpu["other_workloads"] = {
                "prefill": cpu_gmm_baseline(make_gmm_workload("prefill"), args.cpu_budget / 2),
                "dense_w8a16_M1024": cpu_dense_baseline(1024, args.cpu_budget / 4),
            }
    line = {
        "metric": METRIC,
        "value": main_res["GB_s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_res["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded numpy PCG64: N(0,1) bf16 activations, uniform e2m1 nibbles, e8m0 exponents "
                "in [-4,2], softmax top-k routing)",
        "config": {"workload": "decode_gate_up: 32 local experts, 256 tokens x top-8 (M=2048 routed rows, 4 empty "
                               "experts), K=7168, N=4096, fp4 e2m1 weights with e8m0 block-32 scales, bf16 out",
                   "TFLOP_s": main_res["TFLOP_s"], "mfma_bf16_frac": main_res["mfma_bf16_frac"],
                   "bytes_per_step": main_res["bytes"], "flops_per_step": main_res["flops"],
                   "ms_per_step_samples": {"n": len(samples), "statistic": "median", "first": round(first, 5),
                                           "min": round(samples[0], 5), "max": round(samples[-1], 5)}},
        "roofline": {"bound": "hbm", "achieved": main_res["GB_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": main_res["hbm_frac"], "traffic": profiled_traffic()},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
