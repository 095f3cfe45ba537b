"""CPU: the oracle's C++ OpenMP restatement of the decode composition (oracle/cpu_moe.cpp, the CPU baseline's second
leg) agrees with oracle.moe.decode_apply + shared_apply to f64 rounding, independently of the thread count, and
refuses expert ids outside the table."""
import numpy as np
import pytest

from oracle import cb3 as ocb3, cpu_moe, moe as omoe
from oracle.bf16 import rel_l2


def _layer(rng, E, D, I):
    mats = {}
    for name, (R, K) in (("gate", (I, D)), ("up", (I, D)), ("down", (D, I))):
        gen = [ocb3.generate(rng, R, K) for _ in range(E)]
        mats[name] = (np.stack([ocb3.pack_canonical(c) for c, _ in gen]), np.stack([cb for _, cb in gen]),
                      [ocb3.dequant(c, cb) for c, cb in gen])
    return mats


@pytest.mark.parametrize("N,k", [(1, 8), (5, 3)])
def test_cpp_decode_matches_numpy_oracle(N, k):
    rng = np.random.default_rng(11 + N)
    E, D, I, limit = 9, 512, 256, 10.0
    m = _layer(rng, E, D, I)
    idx = np.stack([rng.permutation(E - 1)[:k] for _ in range(N)]).astype(np.int32)
    w = rng.random((N, k)).astype(np.float32)
    x = ocb3.bf16_normal(rng, (N, D)) * 4
    deq = lambda name, e: m[name][2][e]
    want = omoe.decode_apply(deq, x, idx, w, limit) + omoe.shared_apply(lambda n: deq(n, E - 1), x, limit)
    got = cpu_moe.decode_cb3(m["gate"][:2], m["up"][:2], m["down"][:2], x, idx, w, limit, shared=E - 1)
    assert rel_l2(got, want) < 1e-12
    one = cpu_moe.decode_cb3(m["gate"][:2], m["up"][:2], m["down"][:2], x, idx, w, limit, shared=E - 1, threads=1)
    assert np.array_equal(one, cpu_moe.decode_cb3(m["gate"][:2], m["up"][:2], m["down"][:2], x, idx, w, limit,
                                                  shared=E - 1, threads=4))


def test_cpp_decode_rejects_bad_expert_ids():
    rng = np.random.default_rng(2)
    m = _layer(rng, 2, 256, 128)
    with pytest.raises(ValueError):
        cpu_moe.decode_cb3(m["gate"][:2], m["up"][:2], m["down"][:2], np.zeros((1, 256), np.float32),
                           np.array([[2]], np.int32), np.ones((1, 1), np.float32), 10.0)
