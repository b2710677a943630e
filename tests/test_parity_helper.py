"""The inference RGBA check itself (CPU): it accepts one fp16 ulp of RGB and
rejects two, a changed alpha bit, or a systematic shift within tolerance."""
import numpy as np
import pytest

from tests import helpers as H


def _img(seed=0):
    rng = np.random.default_rng(seed)
    return rng.uniform(0.0, 1.0, (24, 32, 4)).astype(np.float16)


def _step(a, k):
    """a moved k fp16 ulps up (k > 0) or down."""
    b = a.copy()
    for _ in range(abs(k)):
        b = np.nextafter(b, np.float16(np.inf if k > 0 else -np.inf))
    return b


def test_accepts_identical_and_one_ulp():
    w = _img()
    H.assert_infer_rgba(w.copy(), w)
    g = w.copy()
    g[3, 5, 1] = _step(g[3, 5, 1:2], 1)[0]
    g[7, 2, 0] = _step(g[7, 2, 0:1], -1)[0]
    H.assert_infer_rgba(g, w)


def test_rejects_two_ulps_alpha_and_bias():
    w = _img(1)
    g = w.copy()
    g[1, 1, 2] = _step(g[1, 1, 2:3], 2)[0]
    with pytest.raises(AssertionError):
        H.assert_infer_rgba(g, w)
    g = w.copy()
    g[4, 4, 3] = _step(g[4, 4, 3:4], 1)[0]
    with pytest.raises(AssertionError):
        H.assert_infer_rgba(g, w)
    # every RGB value one ulp up: within the per-value bound, but a mean shift
    # of about 2.4e-4 is far above what approximate shading produces
    with pytest.raises(AssertionError):
        H.assert_infer_rgba(np.concatenate([_step(w[..., :3], 1), w[..., 3:]], -1), w)
