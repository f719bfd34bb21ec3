"""MoE expert block around the FP4 gmm -- numpy restatement.

Test infrastructure only (see oracle/__init__.py).

* Activation ``silu_and_mul_with_clamp`` (swiglu limit 10), applied to the
  f32 gmm1 accumulators: gate = min(acc1, 10), up = clip(acc3, -10, 10),
  silu(gate) * up
  (patches/tpu-inference-experimental/fused-moe-fp4/0901-...:60-64; the
  comment there states it equals tokamax gmm_v2's fused act).
* acc1 / acc3 are the gate / up halves of the GMM_EP weight layout
  [E, hidden, 2 * inter] = [w1 | w3] (0901-...:250-254, :500), so gmm1's columns
  [0, I) are the gate and [I, 2I) the up projection.
* The activation is rounded to the token dtype (bf16) before the down
  projection (0901-...:420-423); gmm2 accumulates in f32 and rounds once
  (0901-...:446-449), or keeps f32 (0106-...:243-250); the combine follows
  moe_fast_combine.py:44-54 (oracle/moe.py).
"""
import numpy as np

from .numerics import round_bf16

SWIGLU_LIMIT = 10.0
# |d/dx silu(x)| = |s(x) (1 + x (1 - s(x)))| <= 1.0999 for all real x
# (maximum near x = 2.4); clipping is 1-Lipschitz.
SILU_LIPSCHITZ = 1.1


def silu_and_mul_clamp(acc, limit: float = SWIGLU_LIMIT):
    """acc [M, 2I] (gmm1 accumulators, float64) -> silu(min(gate, limit)) *
    clip(up, -limit, limit) [M, I] in float64."""
    acc = np.asarray(acc, np.float64)
    i = acc.shape[-1] // 2
    gate = np.minimum(acc[..., :i], limit)
    up = np.clip(acc[..., i:], -limit, limit)
    return gate / (1.0 + np.exp(-gate)) * up


def act_error_bound(acc64, acc_err, limit: float = SWIGLU_LIMIT):
    """Bound on |act(acc) - act(acc64)| when |acc - acc64| <= acc_err
    elementwise (first-order terms plus the product of the errors), before
    the output rounding.  With g, u the clipped gate/up of acc64 and eg, eu
    their error bounds: |du * silu(g)| + |u| L eg + L eg eu."""
    acc64 = np.asarray(acc64, np.float64)
    acc_err = np.asarray(acc_err, np.float64)
    i = acc64.shape[-1] // 2
    g = np.minimum(acc64[..., :i], limit)
    u = np.clip(acc64[..., i:], -limit, limit)
    eg, eu = acc_err[..., :i], acc_err[..., i:]
    silu_g = np.abs(g / (1.0 + np.exp(-g)))
    return eu * silu_g + np.abs(u) * SILU_LIPSCHITZ * eg + SILU_LIPSCHITZ * eg * eu


def act_output_bound(act64, prop_err):
    """Stated tolerance of the fused bf16 activation output: half a bf16 ulp
    of rounding (2^-8 relative), the propagated gmm1 error, and the f32
    evaluation of silu (exp within a few f32 ulps: 2^-20 relative)."""
    a = np.abs(np.asarray(act64, np.float64))
    return 2.0 ** -8 * (a + prop_err) + prop_err + 2.0 ** -20 * a


def act_bf16(acc64, limit: float = SWIGLU_LIMIT):
    """The activation of exact accumulators rounded to bf16 (as f32 values)."""
    return round_bf16(silu_and_mul_clamp(acc64, limit).astype(np.float32))


# ---- every gated activation of apply_act_fn (0901-...:57-66), float64 ----
# act(gate, up) = f(gate) * h(up).  "gelu" is jax.nn.gelu's default tanh form;
# "swigluoai" (its body is not vendored) follows the published GPT-OSS
# definition: alpha 1.702, limit 7, (clip(up, -7, 7) + 1) * g * sigmoid(alpha g)
# with g = min(gate, 7).
GELU_C = np.sqrt(2.0 / np.pi)
OAI_ALPHA, OAI_LIMIT = 1.702, 7.0
# Lipschitz constants (L_f, L_h): |d silu| <= 1.0999; |d gelu_tanh| <= 1.1289
# (maximum near x = 1.5); g sigmoid(alpha g) = silu(alpha g) / alpha has the
# slope of silu; clipping is 1-Lipschitz.  Checked on a fine grid by the tests.
ACT_LIPSCHITZ = {"silu_and_mul_with_clamp": (SILU_LIPSCHITZ, 1.0), "silu": (SILU_LIPSCHITZ, 1.0),
                 "gelu": (1.13, 1.0), "swigluoai": (SILU_LIPSCHITZ, 1.0)}


def act_parts(gate, up, name):
    """(f(gate), h(up)) in float64 for activation ``name``."""
    g = np.asarray(gate, np.float64)
    u = np.asarray(up, np.float64)
    if name == "silu_and_mul_with_clamp":
        gc = np.minimum(g, SWIGLU_LIMIT)
        return gc / (1.0 + np.exp(-gc)), np.clip(u, -SWIGLU_LIMIT, SWIGLU_LIMIT)
    if name == "silu":
        return g / (1.0 + np.exp(-g)), u
    if name == "gelu":
        return 0.5 * g * (1.0 + np.tanh(GELU_C * (g + 0.044715 * g ** 3))), u
    if name == "swigluoai":
        gc = np.minimum(g, OAI_LIMIT)
        return gc / (1.0 + np.exp(-OAI_ALPHA * gc)), np.clip(u, -OAI_LIMIT, OAI_LIMIT) + 1.0
    raise ValueError(name)


def apply_act(acc, name):
    """acc [M, 2I] (gate | up accumulators, float64) -> act [M, I]."""
    acc = np.asarray(acc, np.float64)
    i = acc.shape[-1] // 2
    f, h = act_parts(acc[..., :i], acc[..., i:], name)
    return f * h


def act_bound(acc64, acc_err, name):
    """Stated tolerance of a fused bf16 activation output against
    apply_act(acc64): with |acc - acc64| <= acc_err elementwise, the
    propagated error p = |h| L_f eg + |f| L_h eu + L_f L_h eg eu, plus half a
    bf16 ulp of rounding (2^-8 relative of |act| + p) and the f32 evaluation
    of exp / tanh (2^-20 of |act| + |g| |h|, the absolute error tanh's
    cancellation near -1 can leave)."""
    acc64 = np.asarray(acc64, np.float64)
    acc_err = np.asarray(acc_err, np.float64)
    i = acc64.shape[-1] // 2
    f, h = act_parts(acc64[..., :i], acc64[..., i:], name)
    eg, eu = acc_err[..., :i], acc_err[..., i:]
    lf, lh = ACT_LIPSCHITZ[name]
    p = np.abs(h) * lf * eg + np.abs(f) * lh * eu + lf * lh * eg * eu
    a = np.abs(f * h)
    return 2.0 ** -8 * (a + p) + p + 2.0 ** -20 * (a + np.abs(acc64[..., :i]) * np.abs(h))
