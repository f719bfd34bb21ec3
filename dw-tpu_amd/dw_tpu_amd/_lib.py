"""ctypes binding of libdwtpu_moe.so (the C ABI declared in include/dwtpu_moe.h).

The library is built in-tree (``__graft_entry__.build()`` or
``make -C dw-tpu_amd/csrc``).  There is no other implementation: when the
library is missing, every entry point raises ``LibraryMissing``.
"""
import ctypes
import os
import threading

import torch

from . import _trace

LIB_NAME = "libdwtpu_moe.so"
# DWTPU_MOE_LIB names another build of the same library (the host-sanitizer
# build that the argument-check tests load); by default the in-tree one.
LIB_PATH = os.environ.get("DWTPU_MOE_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

# enum dwm_status / dwm_dtype / dwm_fp4_format / dwm_act / dwm_score
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3
BF16, F32, U8 = 0, 1, 2
FP4_E2M1, FP4_CODES = 0, 1
ACT_NONE, ACT_SILU_MUL_CLAMP, ACT_SILU_MUL, ACT_GELU_TANH_MUL, ACT_SWIGLUOAI = 0, 1, 2, 3, 4
# gmm_v2 fuse_act names (apply_act_fn) -> enum dwm_act
FUSE_ACTS = {None: ACT_NONE, "silu_and_mul_with_clamp": ACT_SILU_MUL_CLAMP, "silu": ACT_SILU_MUL,
             "gelu": ACT_GELU_TANH_MUL, "swigluoai": ACT_SWIGLUOAI}
SCORE_FNS = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}

_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_p = ctypes.c_void_p

# name -> argument types (restype is int unless listed in _RESTYPES)
SIGNATURES = {
    "dwm_version": [],
    "dwm_last_error": [],
    "dwm_e2m1_to_codes": [_p, _p, _i64, _p],
    "dwm_fp4_decode": [_p, _i32, _i64, _p, _p, _p, _p],
    "dwm_gmm_fp4_prepack_size": [_i64, _i64, _i64, _p, _p],
    "dwm_gmm_fp4_prepack": [_p, _i32, _p, _i32, _i64, _i64, _i64, _p, _p, _p, _p],
    "dwm_gmm_fp4_prepack_gate_up": [_p, _i32, _p, _i32, _i64, _i64, _i64, _p, _p, _p, _p],
    "dwm_gmm_fp4_prepack_transposed": [_p, _i32, _p, _i32, _i64, _i64, _i64, _i32, _p, _p, _p, _p],
    "dwm_gmm_fp4": [_p, _i64, _i64, _p, _p, _p, _i32, _p, _i64, _i64, _p, _i32, _i32, _i32, _p],
    "dwm_gmm_fp4_gather": [_p, _i64, _p, _i64, _i64, _p, _p, _p, _i32, _p, _i64, _i64, _p, _i32, _i32, _i32, _p],
    "dwm_gmm_fp4_ex": [_p, _i64, _i64, _p, _p, _p, _i32, _p, _i32, _p, _i64, _i64, _p, _i32, _i32, _i32, _p],
    "dwm_mx_quant_e4m3": [_p, _i64, _i64, _p, _p, _p],
    "dwm_gmm_fp4_mx": [_p, _p, _i64, _p, _i64, _i64, _p, _p, _p, _i32, _p, _i64, _i64, _p, _i32, _i32, _i32, _p],
    "dwm_mx_quant_e2m1": [_p, _i64, _i64, _p, _p, _p],
    "dwm_gmm_fp4_mxfp4": [_p, _p, _i64, _p, _i64, _i64, _p, _p, _p, _i32, _p, _i32, _p, _i64, _i64, _p, _i32, _i32,
                          _i32, _p],
    "dwm_moe_dispatch_workspace_size": [_i64, _i32, _p],
    "dwm_moe_dispatch": [_p, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _p],
    "dwm_moe_dispatch_noalloc": [_p, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p, _p],
    "dwm_row_gather": [_p, _i64, _i64, _p, _i64, _p, _p],
    "dwm_dispatch_gather": [_p, _i64, _i64, _p, _i64, _i32, _p, _p],
    "dwm_moe_combine": [_p, _i32, _i64, _i64, _p, _p, _i32, _i64, _i32, _p, _i32, _p],
    "dwm_dense_fp8_prepack": [_p, _i64, _i64, _p, _p],
    "dwm_dense_fp8_workspace_size": [_i64, _i64, _i64, _p],
    "dwm_dense_fp8_w8a16": [_p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _p],
    "dwm_dense_fp8_w8a8": [_p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _p],
    "dwm_dense_fp8_w8a16_pre": [_p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _p],
    "dwm_dense_fp8_plan": [_i64, _i64, _i64, _i32, _p],
    "dwm_dense_fp8_plan_check": [_i64, _i64, _i64, _i32, _p],
    "dwm_dense_fp8_plan_workspace_size": [_i64, _i64, _i64, _p, _p],
    "dwm_dense_fp8_w8a16_plan": [_p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _p],
    "dwm_dense_fp8_w8a8_plan": [_p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _p],
    "dwm_dense_fp8_last_plan": [_p],
    "dwm_mxfp4_requant": [_p, _p, _i64, _i64, _i64, _i32, _p, _p, _p, _p],
    "dwm_fp8_block_requant": [_p, _p, _i64, _i64, _i32, _p, _p, _p, _p],
    "dwm_route_topk": [_p, _i32, _i64, _i64, _i32, _i32, _p, _p, _i32, _p, _p, _i32, _p, _p],
    "dwm_dedupe_topk": [_p, _p, _i64, _i32, _i64, _p, _p, _p],
}
_RESTYPES = {"dwm_last_error": ctypes.c_char_p}

# enum dwm_dense_kernel
DENSE_SKINNY, DENSE_MFMA, DENSE_TILED = 1, 2, 3


class GmmLhs(ctypes.Structure):
    """struct dwm_gmm_lhs: the grouped lhs of dwm_gmm_fp4_ex."""
    _fields_ = [("data", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("rows", ctypes.c_int64),
                ("row_idx", ctypes.c_void_p)]


class DensePlan(ctypes.Structure):
    """struct dwm_dense_plan: one launch configuration of the dense GEMM."""
    _fields_ = [("kernel", ctypes.c_int32), ("tile_m", ctypes.c_int32), ("tile_n", ctypes.c_int32),
                ("ksplit", ctypes.c_int32), ("stages", ctypes.c_int32)]

    def astuple(self):
        return (self.kernel, self.tile_m, self.tile_n, self.ksplit, self.stages)


class LibraryMissing(RuntimeError):
    """libdwtpu_moe.so is not built; there is no fallback implementation."""


class Unsupported(NotImplementedError):
    """DWM_ERR_UNSUPPORTED: a valid request the kernels do not handle."""


_lock = threading.Lock()
_lib = None


def load():
    """Loads the library once (thread-safe) and declares every signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise LibraryMissing(
                    f"{LIB_PATH} is not built; run __graft_entry__.build() or "
                    "make -C dw-tpu_amd/csrc")
            lib = ctypes.CDLL(LIB_PATH)
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = lib
    return _lib


def call(name, *args):
    """Calls an entry point and maps its status to an exception (inside a
    roctx range named by the entry point when ranges are on)."""
    lib = load()
    if _trace.enabled():
        with _trace.op_range(name):
            rc = getattr(lib, name)(*args)
    else:
        rc = getattr(lib, name)(*args)
    if rc == OK:
        return
    msg = lib.dwm_last_error().decode(errors="replace")
    if rc == ERR_INVALID:
        raise ValueError(msg)
    if rc == ERR_UNSUPPORTED:
        raise Unsupported(msg)
    raise RuntimeError(msg)


def ptr(t):
    """Device (or host) address of a tensor, or None for None."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(device=None):
    """The current torch stream of ``device`` as a hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dt):
    if dt == torch.bfloat16:
        return BF16
    if dt == torch.float32:
        return F32
    if dt == torch.uint8:
        return U8
    raise ValueError(f"unsupported dtype {dt}")


def require_cuda(*tensors):
    """The kernels run on one HIP device: every tensor must live there."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"expected a device tensor, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev
