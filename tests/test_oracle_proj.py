"""The oracle's Linear (y = x W^T, no bias): an identity weight, brute force on a tiny case, and the
stacked Q/K/V weight splitting into the three separate projections."""
import numpy as np

import pa_oracle as orc


def test_linear_identity_and_brute_force():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 5)).astype(np.float32)
    np.testing.assert_array_equal(orc.linear(x, np.eye(5, dtype=np.float32)), x.astype(np.float64))
    w = rng.standard_normal((4, 5)).astype(np.float32)
    y = orc.linear(x, w)
    for i in range(3):
        for o in range(4):
            assert abs(y[i, o] - sum(float(x[i, k]) * float(w[o, k]) for k in range(5))) < 1e-12


def test_stacked_qkv_weight_is_three_projections():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((6, 16)).astype(np.float32)
    wq, wk, wv = (rng.standard_normal((n, 16)).astype(np.float32) for n in (8, 4, 4))
    y = orc.linear(x, np.concatenate([wq, wk, wv]))
    np.testing.assert_allclose(y[:, :8], orc.linear(x, wq), rtol=0, atol=1e-12)
    np.testing.assert_allclose(y[:, 8:12], orc.linear(x, wk), rtol=0, atol=1e-12)
    np.testing.assert_allclose(y[:, 12:], orc.linear(x, wv), rtol=0, atol=1e-12)
