"""FP4 grouped matmul with the tokamax ``gmm_v2`` call signature.

Mirrors patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:
``needs_fp4_emulation`` (:9-14), ``e2m1_to_codes`` (:17-30), ``decode_codes``
(:33-41) and ``gmm_v2(..., rhs_fp4_codes)`` (:100-151), on MI355X.

Weights.  The reference stores fp4 expert weights as uint4 codes once at load
time so that gmm_v2 does not re-encode them per call.  Here the load-time step
is ``prepack_fp4`` (and ``fused_moe_gmm.fp4_weight_to_codes``), which also
takes the block scales and returns an ``Fp4Weight`` in the K-major layout the
gfx950 kernel streams with 16-byte loads.  ``gmm_v2`` accepts an ``Fp4Weight``
directly; a raw packed weight tensor is prepacked (a full pass over all
experts, as the reference's per-call re-encoding is) on its first call, and
the prepacked copy is reused while the raw tensors are alive and unchanged.

Tensor conventions (torch has no uint4): a 4-bit array of shape [..., N] is a
uint8 tensor [..., N/2] with element 2j in the low nibble, or a
``torch.float4_e2m1fn_x2`` tensor of the same bytes.

MX mode.  ``gmm_v2(..., lhs_quant_dtype=torch.float8_e4m3fn)`` quantizes the
lhs to e4m3 with one e8m0 scale per 32 values along K (``mx_quantize``: the
reference's power-of-two block quantizer, quantize_tensor in
patches/tpu-inference/0001-dsv4-v6e-enablement.patch:315-350, at block 32)
and contracts it with the fp4 weights on the gfx950 scaled MFMA -- the lhs
quantization tokamax performs for chips with a native low-precision matrix
path (patches/tokamax/0001-...:89-100).  An ``MxLhs`` (already quantized)
may be passed as ``lhs`` directly.  ``lhs_quant_dtype=float4_e2m1fn`` (or
``torch.float4_e2m1fn_x2``) quantizes the lhs to e2m1 instead (MXFP4, the
same block-32 power-of-two quantizer at the e2m1 range) and runs the scaled
MFMA with both operands fp4: lossier still, and also opt-in.  The default
(no lhs_quant_dtype) keeps the reference's W4A16 arithmetic: bf16 lhs,
weights decoded exactly.
"""
import collections
import ctypes
import threading
import weakref
from dataclasses import dataclass

import torch

from . import _lib

FP4_DTYPES = tuple(t for t in (getattr(torch, "float4_e2m1fn_x2", None),) if t is not None)
E4M3 = torch.float8_e4m3fn
MX_BLOCK = 32


# e2m1 magnitudes by code (bit 3 is the sign).
_E2M1_MAGS = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)
MX_FORMATS = ("e4m3", "e2m1")


@dataclass(frozen=True)
class MxLhs:
    """An lhs quantized for the MX mode: ``codes`` uint8 [rows, K] (e4m3 bit
    patterns) or, with ``fmt`` "e2m1" (MXFP4), uint8 [rows, K/2] (two e2m1
    codes per byte, element 2 j in the low nibble); ``scales`` uint8
    [rows, K/32] (e8m0 exponent codes, value 2^(code - 127))."""
    codes: torch.Tensor
    scales: torch.Tensor
    fmt: str = "e4m3"

    @property
    def shape(self):
        rows, c = self.codes.shape
        return (rows, 2 * c if self.fmt == "e2m1" else c)

    @property
    def device(self):
        return self.codes.device

    def dequantize(self) -> torch.Tensor:
        """The float32 values the codes and scales stand for (exact)."""
        rows, k = self.shape
        if self.fmt == "e2m1":
            nib = torch.stack([self.codes & 0xF, self.codes >> 4], dim=-1).reshape(rows, k).long()
            mags = torch.tensor(_E2M1_MAGS, device=self.codes.device)
            v = torch.where((nib & 8) != 0, -mags[nib & 7], mags[nib & 7])
        else:
            v = self.codes.view(E4M3).float()
        s = torch.ldexp(torch.ones((), device=self.scales.device), self.scales.to(torch.int32) - 127)
        return (v.view(rows, k // MX_BLOCK, MX_BLOCK) * s[..., None]).view(rows, k)


def mx_quantize(x: torch.Tensor, fmt: str = "e4m3") -> MxLhs:
    """bf16 [rows, K] -> ``MxLhs`` in one device pass, per 32-value block
    along K with scale 2^e (e at least -126):
    fmt "e4m3": e the smallest exponent with absmax <= 448 * 2^e, codes =
    e4m3 of x * 2^-e rounded to nearest even; a block with a NaN or infinity
    gets NaN codes and scale code 255.
    fmt "e2m1" (MXFP4): e the smallest exponent with absmax <= 6 * 2^e, codes
    = e2m1 of x * 2^-e rounded to nearest even, packed two per byte; a block
    with a NaN or infinity gets codes 0 and scale code 255."""
    if fmt not in MX_FORMATS:
        raise ValueError(f"mx_quantize: fmt must be one of {MX_FORMATS}, got {fmt!r}")
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise ValueError(f"mx_quantize: expected a 2-D bfloat16 tensor, got {x.dtype} {tuple(x.shape)}")
    rows, k = x.shape
    if k % MX_BLOCK:
        raise ValueError(f"mx_quantize: K={k} must be a multiple of {MX_BLOCK}")
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    dev = _lib.require_cuda(x)
    codes = torch.empty((rows, k // 2 if fmt == "e2m1" else k), dtype=torch.uint8, device=dev)
    scales = torch.empty((rows, k // MX_BLOCK), dtype=torch.uint8, device=dev)
    _lib.call("dwm_mx_quant_e2m1" if fmt == "e2m1" else "dwm_mx_quant_e4m3", _lib.ptr(x), rows, k, _lib.ptr(codes),
              _lib.ptr(scales), _lib.stream_handle(dev))
    return MxLhs(codes, scales, fmt)


def _mx_format(lhs_quant_dtype):
    """The MX lhs format a gmm_v2 lhs_quant_dtype names (None: no quantization)."""
    if lhs_quant_dtype is None:
        return None
    if lhs_quant_dtype in (E4M3, "float8_e4m3fn"):
        return "e4m3"
    if lhs_quant_dtype in FP4_DTYPES or lhs_quant_dtype in ("float4_e2m1fn", "float4_e2m1fn_x2"):
        return "e2m1"
    raise NotImplementedError(f"gmm_v2: lhs_quant_dtype {lhs_quant_dtype!r}: float8_e4m3fn and float4_e2m1fn "
                              "(the MX modes) are supported")


def needs_fp4_emulation(dtype) -> bool:
    """Whether an fp4 rhs must be converted before the kernel can stream it.

    The reference returns True for float4_e2m1fn on TPUs older than v7
    (:9-14).  On MI355X the converter is native, but the kernel streams the
    prepacked layout, so a float4 weight always goes through ``prepack_fp4``
    (once, at load time).
    """
    return dtype in FP4_DTYPES


def _as_bytes(t: torch.Tensor) -> torch.Tensor:
    if t.dtype in FP4_DTYPES:
        return t.view(torch.uint8)
    if t.dtype != torch.uint8:
        raise ValueError(f"expected packed 4-bit bytes (uint8 or float4_e2m1fn_x2), got {t.dtype}")
    return t


def e2m1_to_codes(rhs: torch.Tensor) -> torch.Tensor:
    """Re-encodes packed e2m1 nibbles as gmm_v2 uint4 codes (same shape, uint8).

    A code holds the int4 q = sign * (2 * exponent + mantissa); -0 becomes +0
    (:17-30).  One elementwise device pass.
    """
    src = _as_bytes(rhs).contiguous()
    _lib.require_cuda(src)
    out = torch.empty_like(src, dtype=torch.uint8)
    _lib.call("dwm_e2m1_to_codes", _lib.ptr(src), _lib.ptr(out), src.numel(), _lib.stream_handle(src.device))
    return out


def decode_fp4(packed: torch.Tensor, fmt: int, scales: torch.Tensor = None, check: bool = True) -> torch.Tensor:
    """Packed 4-bit values (``_lib.FP4_E2M1`` or ``_lib.FP4_CODES``) -> bf16
    [..., 2 * last], times the e8m0 scale of each 32-value block of the flat
    index when ``scales`` (uint8 codes) is given.  Decodes through the same
    converter as the gmm kernel."""
    src = _as_bytes(packed).contiguous()
    _lib.require_cuda(src, scales)
    n = src.numel() * 2
    if scales is not None:
        scales = scales.contiguous()
        if scales.dtype != torch.uint8 or scales.numel() * 32 < n:
            raise ValueError("scales must be uint8 e8m0 codes, one per 32 values")
    out = torch.empty(src.shape[:-1] + (src.shape[-1] * 2,), dtype=torch.bfloat16, device=src.device)
    flags = torch.zeros(1, dtype=torch.int32, device=src.device)
    _lib.call("dwm_fp4_decode", _lib.ptr(src), fmt, n, _lib.ptr(scales), _lib.ptr(out), _lib.ptr(flags),
              _lib.stream_handle(src.device))
    if check and int(flags.item()) & 1:
        raise ValueError("e8m0 scale code 255 (not a finite power of two)")
    return out


def decode_codes(codes: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    """Exactly decodes gmm_v2 uint4 codes (packed, uint8) to ``dtype`` (:33-41)."""
    return decode_fp4(codes, _lib.FP4_CODES).to(dtype)


@dataclass(frozen=True)
class Fp4Weight:
    """Prepacked fp4 expert weights [E, K, N] with e8m0 block-32 scales along K.

    ``weight`` and ``scale`` are uint8 device tensors in the kernel layout
    (documented in dw-tpu_amd/csrc/fp4.hip).  ``gate_up`` weights ([w1 | w3]
    with gate and up columns interleaved by the prepack) run only with the
    fused ``silu_and_mul_with_clamp`` activation.
    """
    weight: torch.Tensor
    scale: torch.Tensor
    num_experts: int
    k: int
    n: int
    gate_up: bool = False

    @property
    def shape(self):
        return (self.num_experts, self.k, self.n)

    @property
    def device(self):
        return self.weight.device


def prepack_fp4(rhs: torch.Tensor, rhs_scale: torch.Tensor, rhs_fp4_codes: bool = False,
                gate_up: bool = False, transpose_rhs: bool = False) -> Fp4Weight:
    """One-time relayout of packed fp4 expert weights and their scales.

    rhs: [E, K, N/2] packed bytes -- e2m1 nibbles (uint8 or
    float4_e2m1fn_x2), or gmm_v2 codes when ``rhs_fp4_codes``; with
    ``transpose_rhs`` the transposed weight [E, N, K/2] (two K values per
    byte, low nibble = even k).
    rhs_scale: [E, K/32, 1, N] or [E, K/32, N] in either case: uint8 e8m0
    codes, or f32 / bf16 powers of two (the lossless e8m0 set,
    e8m0_scale.py:25-34).
    ``gate_up``: rhs is a [w1 | w3] gate/up weight for the fused activation
    (N % 64 == 0).  Synchronises the stream once to check the scales (load time).
    """
    if rhs_fp4_codes and rhs.dtype != torch.uint8:
        raise ValueError(f"rhs_fp4_codes expects uint4 rhs, got {rhs.dtype}.")
    src = _as_bytes(rhs).contiguous()
    _lib.require_cuda(src, rhs_scale)
    if src.dim() != 3:
        raise ValueError(f"rhs must be [E, {'N, K/2' if transpose_rhs else 'K, N/2'}] packed bytes, "
                         f"got shape {tuple(src.shape)}")
    if transpose_rhs:
        e, n, half_k = src.shape
        k = 2 * half_k
    else:
        e, k, half_n = src.shape
        n = 2 * half_n
    if rhs_scale is None:
        raise ValueError("fp4 weights need block scales")
    sc = rhs_scale
    if sc.dim() == 4:
        if sc.shape[2] != 1:
            raise ValueError(f"rhs_scale must be [E, K/32, 1, N], got {tuple(sc.shape)}")
        sc = sc.reshape(sc.shape[0], sc.shape[1], sc.shape[3])
    if tuple(sc.shape) != (e, k // 32, n) or k % 32:
        raise ValueError(f"rhs_scale shape {tuple(rhs_scale.shape)} does not match rhs [E={e}, K={k}, N={n}]"
                         " with 32-element blocks along K")
    sc = sc.contiguous()
    wb = ctypes.c_int64(0)
    sb = ctypes.c_int64(0)
    _lib.call("dwm_gmm_fp4_prepack_size", e, k, n, ctypes.byref(wb), ctypes.byref(sb))
    wout = torch.empty(wb.value, dtype=torch.uint8, device=src.device)
    sout = torch.zeros(sb.value, dtype=torch.uint8, device=src.device)
    flags = torch.zeros(1, dtype=torch.int32, device=src.device)
    fmt = _lib.FP4_CODES if rhs_fp4_codes else _lib.FP4_E2M1
    if transpose_rhs:
        _lib.call("dwm_gmm_fp4_prepack_transposed", _lib.ptr(src), fmt, _lib.ptr(sc), _lib.dtype_code(sc.dtype), e,
                  k, n, 1 if gate_up else 0, _lib.ptr(wout), _lib.ptr(sout), _lib.ptr(flags),
                  _lib.stream_handle(src.device))
    else:
        entry = "dwm_gmm_fp4_prepack_gate_up" if gate_up else "dwm_gmm_fp4_prepack"
        _lib.call(entry, _lib.ptr(src), fmt, _lib.ptr(sc), _lib.dtype_code(sc.dtype), e, k, n,
                  _lib.ptr(wout), _lib.ptr(sout), _lib.ptr(flags), _lib.stream_handle(src.device))
    f = int(flags.item())
    if f & 1:
        raise ValueError("rhs_scale holds a value that is not +0.0 or a power of two in the e8m0 range "
                         "(code 255, a negative, subnormal or non-power-of-two scale)")
    if f & 2:
        raise ValueError("rhs holds uint4 code 8 (q = -8), which e2m1_to_codes never produces")
    return Fp4Weight(wout, sout, e, k, n, gate_up)


# Raw weights handed to gmm_v2 call after call (the reference's per-call
# form) are prepacked and checked once: the prepacked copy is kept while the
# raw rhs and scale tensors are alive and unmodified (the same objects with
# the same in-place version counters).  Each entry holds the prepacked bytes
# (the size of the raw weight) in device memory; clear_prepack_cache() drops
# them.
_PREPACK_CACHE_SIZE = 8
_prepack_cache = collections.OrderedDict()
_prepack_lock = threading.Lock()


def clear_prepack_cache():
    """Drop the prepacked copies gmm_v2 keeps for raw weight tensors."""
    with _prepack_lock:
        _prepack_cache.clear()


def _prepack_cached(rhs, rhs_scale, rhs_fp4_codes, gate_up, transpose_rhs=False):
    if rhs_scale is None:
        return prepack_fp4(rhs, rhs_scale, rhs_fp4_codes=rhs_fp4_codes, gate_up=gate_up, transpose_rhs=transpose_rhs)
    key = (id(rhs), id(rhs_scale), bool(rhs_fp4_codes), bool(gate_up), bool(transpose_rhs))
    with _prepack_lock:
        hit = _prepack_cache.get(key)
        if hit is not None:
            r_ref, s_ref, r_ver, s_ver, w = hit
            if r_ref() is rhs and s_ref() is rhs_scale and rhs._version == r_ver and rhs_scale._version == s_ver:
                _prepack_cache.move_to_end(key)
                return w
            del _prepack_cache[key]
    w = prepack_fp4(rhs, rhs_scale, rhs_fp4_codes=rhs_fp4_codes, gate_up=gate_up, transpose_rhs=transpose_rhs)
    with _prepack_lock:
        _prepack_cache[key] = (weakref.ref(rhs), weakref.ref(rhs_scale), rhs._version, rhs_scale._version, w)
        while len(_prepack_cache) > _PREPACK_CACHE_SIZE:
            _prepack_cache.popitem(last=False)
    return w


def gmm_v2(lhs: torch.Tensor,
           rhs,
           group_sizes: torch.Tensor,
           rhs_scale: torch.Tensor = None,
           rhs_bias: torch.Tensor = None,
           group_offset=None,
           *,
           tile_info=None,
           vmem_limit_bytes=None,
           preferred_element_type=None,
           lhs_quant_dtype=None,
           rhs_quant_dtype=None,
           zero_initialize: bool = True,
           fuse_act=None,
           transpose_rhs: bool = False,
           rhs_fp4_codes: bool = False,
           lhs_row_indices: torch.Tensor = None) -> torch.Tensor:
    """Ragged grouped matmul: out[rows of g] = lhs[rows of g] @ dequant(rhs[g - group_offset]).

    lhs: [M, K] bf16, rows sorted by group (or an ``MxLhs``: the MX mode).  rhs: ``Fp4Weight`` (prepacked)
    or packed fp4 bytes [E, K, N/2] (prepacked and checked on the first call with those rhs / rhs_scale
    tensors, which synchronises the stream once; the prepacked copy is reused while both tensors are alive
    and unmodified, see ``clear_prepack_cache``).  group_sizes:
    int32 [G] device tensor.  group_offset: None, an int, or an int32 [1]
    device tensor (first local group).  Returns [M, N] in
    ``preferred_element_type`` (bf16 default, or float32).  Rows outside the
    local groups are zero when ``zero_initialize`` and unspecified otherwise.
    ``fuse_act``: one of apply_act_fn's gated activations
    (patches/tpu-inference-experimental/fused-moe-fp4/0901-...:57-66) --
    "silu_and_mul_with_clamp" (silu(min(gate, 10)) * clip(up, -10, 10)),
    "silu", "gelu" (tanh form, jax.nn.gelu's default) or "swigluoai"
    (GPT-OSS: g = min(gate, 7), (clip(up, -7, 7) + 1) * g * sigmoid(1.702 g))
    -- with rhs a [w1 | w3] gate/up weight (an ``Fp4Weight`` prepacked with
    ``gate_up=True``, or raw bytes prepacked so per call); the result is
    [M, N/2], the activation of the f32 accumulators rounded once.
    ``rhs_bias`` ([E, N] or [E, 1, N], f32 or bf16, in the weight's column
    order) is added to the f32 accumulators of each expert's rows before the
    activation and the rounding.  Tiling / VMEM arguments of the TPU kernel
    are accepted and ignored.  ``transpose_rhs`` (raw weights only): rhs is
    stored transposed, [E, N, K/2] packed along K, and is transposed once
    when it is prepacked (``prepack_fp4``); a prepacked ``Fp4Weight``
    already carries its layout.

    ``lhs_row_indices`` (an addition; int32 [M] device tensor): row r of the
    grouped operand is ``lhs[lhs_row_indices[r]]`` (JAX gather index
    semantics), read by the kernel directly -- the dispatch row gather fused
    into the matmul.  ``lhs`` is then the source [rows, K] and the result has
    M = len(lhs_row_indices) rows.

    ``lhs_quant_dtype=torch.float8_e4m3fn`` selects the MX mode (module
    docstring): the lhs is quantized with ``mx_quantize`` (unless it is an
    ``MxLhs`` already) and each product is e4m3 x e2m1 with both block scales,
    on the scaled MFMA; ``lhs_quant_dtype`` float4_e2m1fn (or
    ``torch.float4_e2m1fn_x2``) quantizes to e2m1 (MXFP4) and each product is
    e2m1 x e2m1.  ``rhs_quant_dtype`` is accepted and ignored (the rhs is fp4
    either way).
    """
    if fuse_act not in _lib.FUSE_ACTS:
        raise NotImplementedError(f"gmm_v2: fused activation {fuse_act!r} is not supported")
    fused = fuse_act is not None
    mx_fmt = _mx_format(lhs_quant_dtype)
    if isinstance(lhs, MxLhs):
        if mx_fmt is not None and mx_fmt != lhs.fmt:
            raise ValueError(f"gmm_v2: an {lhs.fmt} MxLhs with lhs_quant_dtype {lhs_quant_dtype!r}")
        mx_fmt = lhs.fmt
    mx = mx_fmt is not None
    if isinstance(rhs, Fp4Weight):
        if rhs_scale is not None:
            raise ValueError("gmm_v2: a prepacked Fp4Weight carries its own scales; pass rhs_scale=None")
        w = rhs
    else:
        w = _prepack_cached(rhs, rhs_scale, rhs_fp4_codes, fused, transpose_rhs)
    if w.gate_up != fused:
        raise ValueError("gmm_v2: gate/up-prepacked weights run only (and always) with the fused activation"
                         if w.gate_up else "gmm_v2: the fused activation needs weights prepacked with gate_up=True")
    if isinstance(lhs, MxLhs):
        out_dtype = torch.bfloat16 if preferred_element_type is None else preferred_element_type
    else:
        if lhs.dtype != torch.bfloat16:
            raise ValueError(f"gmm_v2: lhs must be bfloat16, got {lhs.dtype}")
        out_dtype = lhs.dtype if preferred_element_type is None else preferred_element_type
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"gmm_v2: preferred_element_type must be bfloat16 or float32, got {out_dtype}")
    if len(lhs.shape) != 2 or lhs.shape[1] != w.k:
        raise ValueError(f"gmm_v2: lhs shape {tuple(lhs.shape)} does not match rhs K={w.k}")
    if group_sizes.dtype != torch.int32 or group_sizes.dim() != 1:
        raise ValueError("gmm_v2: group_sizes must be a 1-D int32 tensor")
    if mx and not isinstance(lhs, MxLhs):
        lhs = mx_quantize(lhs, mx_fmt)
    if isinstance(lhs, MxLhs):
        if lhs.codes.dtype != torch.uint8 or lhs.scales.dtype != torch.uint8 or \
                tuple(lhs.scales.shape) != (lhs.shape[0], w.k // MX_BLOCK):
            raise ValueError("gmm_v2: MxLhs needs uint8 codes [rows, K] (e2m1: [rows, K/2]) and uint8 scales "
                             "[rows, K/32]")
        dev = _lib.require_cuda(lhs.codes, lhs.scales, w.weight, group_sizes)
    else:
        dev = _lib.require_cuda(lhs, w.weight, group_sizes)
        lhs = lhs.contiguous()
        if lhs.data_ptr() % 16:
            lhs = lhs.clone()  # the kernel streams 16-byte rows
    gs = group_sizes.contiguous()
    if group_offset is None:
        go = None
    elif isinstance(group_offset, int):
        go = torch.tensor([group_offset], dtype=torch.int32, device=dev)
    else:
        go = group_offset.reshape(-1)[:1].to(device=dev, dtype=torch.int32).contiguous()
    idx = lhs_row_indices
    if idx is not None:
        if idx.dtype != torch.int32 or idx.dim() != 1:
            raise ValueError("gmm_v2: lhs_row_indices must be a 1-D int32 tensor")
        _lib.require_cuda(idx)
        idx = idx.contiguous()
    m = lhs.shape[0] if idx is None else idx.numel()
    bias = None
    if rhs_bias is not None:
        bias = rhs_bias.reshape(rhs_bias.shape[0], -1) if rhs_bias.dim() == 3 else rhs_bias
        if tuple(bias.shape) != (w.num_experts, w.n) or (rhs_bias.dim() == 3 and rhs_bias.shape[1] != 1):
            raise ValueError(f"gmm_v2: rhs_bias must be [E, N] or [E, 1, N] = [{w.num_experts}, {w.n}], "
                             f"got {tuple(rhs_bias.shape)}")
        if bias.dtype not in (torch.float32, torch.bfloat16):
            bias = bias.to(torch.float32)
        bias = bias.contiguous()
        _lib.require_cuda(bias)
    out = torch.empty((m, w.n // 2 if fused else w.n), dtype=out_dtype, device=dev)
    if mx_fmt == "e2m1":
        codes, scales = lhs.codes.contiguous(), lhs.scales.contiguous()
        _lib.call("dwm_gmm_fp4_mxfp4", _lib.ptr(codes), _lib.ptr(scales), codes.shape[0], _lib.ptr(idx), m, w.k,
                  _lib.ptr(w.weight), _lib.ptr(w.scale), _lib.ptr(bias),
                  _lib.dtype_code(bias.dtype) if bias is not None else 0, _lib.ptr(gs), gs.numel(), _lib.ptr(go),
                  w.num_experts, w.n, _lib.ptr(out), _lib.dtype_code(out_dtype), 1 if zero_initialize else 0,
                  _lib.FUSE_ACTS[fuse_act], _lib.stream_handle(dev))
        return out
    if mx:
        codes, scales = lhs.codes.contiguous(), lhs.scales.contiguous()
        desc = _lib.GmmLhs(codes.data_ptr(), scales.data_ptr(), codes.shape[0], None if idx is None else idx.data_ptr())
    else:
        desc = _lib.GmmLhs(lhs.data_ptr(), None, lhs.shape[0], None if idx is None else idx.data_ptr())
    _lib.call("dwm_gmm_fp4_ex", ctypes.byref(desc), m, w.k, _lib.ptr(w.weight), _lib.ptr(w.scale), _lib.ptr(bias),
              _lib.dtype_code(bias.dtype) if bias is not None else 0, _lib.ptr(gs), gs.numel(), _lib.ptr(go),
              w.num_experts, w.n, _lib.ptr(out), _lib.dtype_code(out_dtype), 1 if zero_initialize else 0,
              _lib.FUSE_ACTS[fuse_act], _lib.stream_handle(dev))
    return out
