"""Pins oracle.moe_block (the silu_and_mul_with_clamp activation and its
error bound) on the CPU against closed forms, an independent formulation,
special values and brute-force perturbation."""
import numpy as np

from oracle import moe_block as omb


def test_special_values():
    acc = np.array([[0.0, 3.0, 10.0, 25.0, -4.0, 1.0,    # gate
                     5.0, 3.0, 2.0, 2.0, 1.0, 50.0]])    # up
    out = omb.silu_and_mul_clamp(acc)[0]
    s = lambda x: x / (1 + np.exp(-x))
    assert out[0] == 0.0                                  # silu(0) = 0
    assert np.isclose(out[1], s(3.0) * 3.0, rtol=1e-15)
    assert np.isclose(out[2], s(10.0) * 2.0, rtol=1e-15)  # gate at the limit
    assert np.isclose(out[3], s(10.0) * 2.0, rtol=1e-15)  # gate clipped above only
    assert np.isclose(out[4], s(-4.0) * 1.0, rtol=1e-15)  # negative gates pass
    assert np.isclose(out[5], s(1.0) * 10.0, rtol=1e-15)  # up clipped to +10
    assert omb.silu_and_mul_clamp(np.array([[1.0, -50.0]]))[0, 0] == s(1.0) * -10.0


def test_gate_is_the_first_half():
    acc = np.concatenate([np.zeros((4, 8)), np.random.default_rng(0).normal(size=(4, 8))], axis=1)
    assert np.all(omb.silu_and_mul_clamp(acc) == 0.0)  # zero gate -> zero output for any up
    acc2 = np.concatenate([np.ones((4, 8)), np.zeros((4, 8))], axis=1)
    assert np.all(omb.silu_and_mul_clamp(acc2) == 0.0)


def test_matches_tanh_formulation():
    rng = np.random.default_rng(1)
    acc = rng.normal(scale=8, size=(64, 256))
    i = 128
    g = np.minimum(acc[:, :i], 10)
    u = np.clip(acc[:, i:], -10, 10)
    ref = g * 0.5 * (1 + np.tanh(g / 2)) * u   # sigmoid(x) = (1 + tanh(x/2)) / 2
    got = omb.silu_and_mul_clamp(acc)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-13)


def test_silu_slope_bound():
    x = np.linspace(-40, 40, 800001)
    s = 1 / (1 + np.exp(-x))
    slope = s * (1 + x * (1 - s))
    assert np.abs(slope).max() <= omb.SILU_LIPSCHITZ
    assert np.abs(slope).max() > 1.09  # the constant is tight (max ~1.0998)


def test_error_bound_covers_perturbations():
    rng = np.random.default_rng(2)
    acc = rng.normal(scale=9, size=(200, 64))
    err = np.abs(rng.normal(scale=0.05, size=acc.shape))
    bound = omb.act_error_bound(acc, err)
    base = omb.silu_and_mul_clamp(acc)
    for _ in range(50):
        delta = rng.uniform(-1, 1, size=acc.shape) * err
        assert np.all(np.abs(omb.silu_and_mul_clamp(acc + delta) - base) <= bound + 1e-12)


def test_bf16_output_bound_holds_for_rounding_alone():
    rng = np.random.default_rng(3)
    acc = rng.normal(scale=9, size=(100, 64))
    act = omb.silu_and_mul_clamp(acc)
    assert np.all(np.abs(omb.act_bf16(acc) - act) <= omb.act_output_bound(act, np.zeros_like(act)))


def test_all_activations_closed_forms_and_slopes():
    """The gated activations of apply_act_fn (0901-...:57-66) restated in
    oracle.moe_block.act_parts: special values, the clamps, jax.nn.gelu's
    tanh form (distinct from the erf form by up to ~2e-4), GPT-OSS swigluoai
    at hand-computed points, and each stated Lipschitz constant on a grid."""
    import math
    from oracle import moe_block as m
    z = np.zeros(1)
    for n in m.ACT_LIPSCHITZ:
        f, _ = m.act_parts(z, z, n)
        assert f[0] == 0.0
    # the existing clamped silu is the same function
    acc = np.random.default_rng(3).standard_normal((5, 8)) * 6
    assert np.array_equal(m.apply_act(acc, "silu_and_mul_with_clamp"), m.silu_and_mul_clamp(acc))
    # gelu: tanh form, not erf
    x = np.linspace(-6, 6, 1201)
    f, _ = m.act_parts(x, x, "gelu")
    erf_gelu = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x])
    d = np.abs(f - erf_gelu)
    assert d.max() < 5e-4 and d.max() > 1e-5
    assert abs(m.act_parts(np.array([1.0]), z, "gelu")[0][0] - 0.5 * (1 + math.tanh(math.sqrt(2 / math.pi) * 1.044715))) < 1e-15
    # swigluoai: g sigmoid(1.702 g) (clip(u, -7, 7) + 1), g clipped above at 7
    f, h = m.act_parts(np.array([2.0, 9.0, -3.0]), np.array([0.5, 100.0, -100.0]), "swigluoai")
    assert np.allclose(f, [2 / (1 + math.exp(-3.404)), 7 / (1 + math.exp(-1.702 * 7)), -3 / (1 + math.exp(5.106))], rtol=1e-15)
    assert np.array_equal(h, [1.5, 8.0, -6.0])
    # silu: no clamps
    f, h = m.act_parts(np.array([30.0]), np.array([50.0]), "silu")
    assert abs(f[0] - 30.0) < 1e-10 and h[0] == 50.0
    # slopes
    g = np.linspace(-30, 30, 600001)
    for n, (lf, _) in m.ACT_LIPSCHITZ.items():
        f, _ = m.act_parts(g, np.zeros_like(g), n)
        assert np.abs(np.diff(f) / np.diff(g)).max() <= lf


def test_act_bound_covers_perturbations():
    """act_bound against brute-force perturbations of the accumulators within
    the stated accumulator error."""
    from oracle import moe_block as m
    rng = np.random.default_rng(4)
    acc = rng.standard_normal((64, 16)) * 8
    err = np.abs(rng.standard_normal((64, 16))) * 0.05
    for n in m.ACT_LIPSCHITZ:
        want = m.apply_act(acc, n)
        for _ in range(20):
            pert = acc + err * rng.uniform(-1, 1, acc.shape)
            got = m.apply_act(pert, n)
            assert np.all(np.abs(got - want) <= m.act_bound(acc, err, n))


def test_gmm_bias_is_added_per_group():
    from oracle import gmm
    rng = np.random.default_rng(5)
    gs = np.array([2, 0, 3], np.int32)
    a = rng.standard_normal((5, 64)).astype(np.float32)
    w = rng.standard_normal((3, 64, 8)).astype(np.float32)
    b = rng.standard_normal((3, 8))
    y0, _ = gmm.gmm(a, None, None, gs, out_dtype="float64", w=w)
    y1, _ = gmm.gmm(a, None, None, gs, out_dtype="float64", w=w, bias=b)
    assert np.allclose(y1[:2] - y0[:2], b[0]) and np.allclose(y1[2:] - y0[2:], b[2])
