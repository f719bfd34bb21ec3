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
