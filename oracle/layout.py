"""The reference's activation order for the planar tables (test infrastructure only).

Restates planes.py:43-118: word w of a row holds C value planes; value plane c of word w multiplies natural input
``input_index(qtype, w, c)``, and the Pallas kernel's per-word activation matrix is X[w, c] = x[input(w, c)]
(``pm_x``).  Here pm_x is a gather through input_index; the reference writes it as reshapes and transposes
(planes.py:96-112), which the tests restate separately.
"""
import numpy as np

QK = 256
WORDS_PER_BLOCK = {"IQ2_S": 8, "IQ3_S": 16, "IQ4_XS": 32, "Q2_K": 16, "Q3_K": 16}     # planes.py:43
PLANES_PER_WORD = {"IQ2_S": 32, "IQ3_S": 16, "IQ4_XS": 8, "Q2_K": 16, "Q3_K": 16}     # planes.py:44 (C)


def input_index(qtype, w, c):
    """Natural input index of value plane c of word w (planes.py:73-85)."""
    w = np.asarray(w)
    c = np.asarray(c)
    if qtype == "IQ2_S":
        return 32 * w + c                                   # c = 8 j + k
    if qtype == "IQ3_S":
        return 16 * w + c                                   # c = 4 j + k
    if qtype == "IQ4_XS":
        pos, j = c // 4, c % 4
        return 32 * (w // 4) + 16 * pos + 4 * (w % 4) + j
    if qtype in ("Q2_K", "Q3_K"):
        s, j = c // 4, c % 4
        return 256 * (w // 16) + 128 * ((w % 16) // 8) + 32 * s + 4 * (w % 8) + j
    raise ValueError(qtype)


def pm_x(qtype, x):
    """x [..., n] natural -> X [..., W, C] with X[w, c] = x[input(w, c)] (planes.py:96-112)."""
    x = np.asarray(x)
    n = x.shape[-1]
    W = n * WORDS_PER_BLOCK[qtype] // QK
    C = PLANES_PER_WORD[qtype]
    w, c = np.meshgrid(np.arange(W), np.arange(C), indexing="ij")
    return x[..., input_index(qtype, w, c)]
