"""CPU: pins oracle.layout (the reference's planar activation order, planes.py:43-118) by the reference's two
statements of it -- the input_index formulas (planes.py:73-85) and the reshape/transpose form of pm_x
(planes.py:96-112), restated here separately -- plus bijection and known answers read off the format comments
(planes.py:17-41)."""
import numpy as np
import pytest

from oracle import layout

QTYPES = ("IQ2_S", "IQ3_S", "IQ4_XS", "Q2_K", "Q3_K")


def _pm_x_reshape(qtype, x):
    """planes.py:96-112 as written there: reshapes and transposes."""
    n = x.shape[-1]
    lead = x.shape[:-1]
    if qtype == "IQ2_S":
        return x.reshape(lead + (n // 32, 32))
    if qtype == "IQ3_S":
        return x.reshape(lead + (n // 16, 16))
    if qtype == "IQ4_XS":
        y = np.swapaxes(x.reshape(lead + (n // 32, 2, 4, 4)), -3, -2)
        return y.reshape(lead + (n // 8, 8))
    y = np.swapaxes(x.reshape(lead + (n // 256, 2, 4, 8, 4)), -3, -2)
    return y.reshape(lead + (n // 16, 16))


@pytest.mark.parametrize("qtype", QTYPES)
def test_pm_x_is_the_reference_reshape_and_a_bijection(qtype):
    n = 3 * 256
    x = np.arange(2 * n).reshape(2, n)
    X = layout.pm_x(qtype, x)
    assert X.shape == (2, n * layout.WORDS_PER_BLOCK[qtype] // 256, layout.PLANES_PER_WORD[qtype])
    assert np.array_equal(X, _pm_x_reshape(qtype, x))
    assert np.array_equal(np.sort(X[0].reshape(-1)), np.arange(n))


def test_known_answers():
    # IQ4_XS: byte j of word w, low nibble = position 0, high = position 1 (planes.py:26-27): word 5 = sub-block 1,
    # quarter 1; c = 4 pos + j
    assert layout.input_index("IQ4_XS", 5, 4 * 1 + 2) == 32 + 16 + 4 + 2
    assert layout.input_index("IQ4_XS", 5, 2) == 32 + 4 + 2
    # K-quants: word 16 b + 8 n + q, c = 4 s + j -> 256 b + 128 n + 32 s + 4 q + j (planes.py:31-33)
    assert layout.input_index("Q2_K", 16 + 8 + 3, 4 * 2 + 1) == 256 + 128 + 64 + 12 + 1
    assert layout.input_index("IQ3_S", 7, 13) == 7 * 16 + 13
    assert layout.input_index("IQ2_S", 7, 31) == 7 * 32 + 31
