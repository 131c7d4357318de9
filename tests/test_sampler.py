"""CPU checks of the sampler around the DiT forward (engine/src/pipeline.mm:300-316): the oracle's noise
schedule (krea_sigmas, engine/src/model.mm:594-602) against closed forms, libkh's host kh_sigmas against the
oracle bit for bit, and the oracle's Euler / guidance updates against a single rounding of the exact result."""
import math

import numpy as np
import pytest

from oracle import oracle as O


@pytest.mark.parametrize("steps", [1, 4, 28, 50])
def test_sigmas_mu0_is_linear(steps):
    # e = exp(0) = 1: 1 / (1 + 1/t - 1) = t
    s = O.sigmas(steps, 0.0)
    t = 1.0 - np.arange(steps + 1) / steps
    np.testing.assert_allclose(s, t.astype(np.float32), rtol=0, atol=1e-7)


@pytest.mark.parametrize("steps,mu", [(4, 1.15), (28, 1.15), (50, 0.5), (28, 3.0)])
def test_sigmas_logistic_shift(steps, mu):
    s = O.sigmas(steps, mu).astype(np.float64)
    assert s[0] == 1.0 and s[-1] == 0.0
    assert (np.diff(s) < 0).all()
    for i in range(1, steps):
        t = 1.0 - i / steps
        # logit(s) = mu + logit(t): the time shift of flow matching
        assert math.log(s[i] / (1 - s[i])) == pytest.approx(mu + math.log(t / (1 - t)), abs=2e-5)


def test_library_sigmas_match_oracle():
    from krea_image_amd import kh
    for steps, mu in [(1, 1.15), (4, 1.15), (28, 1.15), (50, 0.7), (1000, 2.0)]:
        np.testing.assert_array_equal(kh.sigmas(steps, mu), O.sigmas(steps, mu))
    with pytest.raises(kh.KhError):
        kh.sigmas(0)


def test_euler_oracle_single_rounding():
    rng = np.random.default_rng(1)
    z = rng.standard_normal(4097).astype(np.float32)
    v = rng.standard_normal(4097).astype(np.float32)
    dt = -0.0625  # one mantissa bit: dt v and z + dt v are exact in float64, so one rounding to f32 is the fma
    exact = z.astype(np.float64) + dt * v.astype(np.float64)
    np.testing.assert_array_equal(O.euler_step(z, v, dt), exact.astype(np.float32))
    np.testing.assert_array_equal(O.euler_step(z, v, 0.0), z)


def test_cfg_oracle_single_rounding():
    rng = np.random.default_rng(2)
    vc = rng.standard_normal(4097).astype(np.float32)
    vn = rng.standard_normal(4097).astype(np.float32)
    d = vc - vn  # f32 difference (rounded), then vc + 4.5 d exactly in float64, rounded once
    exact = vc.astype(np.float64) + 4.5 * d.astype(np.float64)
    np.testing.assert_array_equal(O.cfg_combine(vc, vn, 4.5), exact.astype(np.float32))
    np.testing.assert_array_equal(O.cfg_combine(vc, vn, 0.0), vc)
