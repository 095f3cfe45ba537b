"""GPU parity of the grouped prefill path (resident.py:144-165): the device ragged_plan, the grouped GEMMs on
the matrix cores (CB3, IQ2_S, IQ3_S, IQ4_XS, Q2_K and Q3_K tables, gate/up and down in one format or two) and the combine, against the
CPU oracle.

Bar: the plan is bit-exact against oracle.moe.ragged_plan (pallas_moe.py:564-592 restated in numpy); prefill
outputs within rel-L2 <= 1e-3 of oracle.moe.prefill_apply, which rounds where the reference rounds (x, h and y to
bf16, the matmul combine's routing weights to bf16) and accumulates in f64.  The kernels accumulate in f32, so an h
or y element next to a bf16 rounding boundary may round the other way: the observed distance is ~1e-5.
"""
import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle.bf16 import rel_l2, round_bf16
from tests.util import Layer, softmax_topk_routing, zipf_routing

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(dtype) if dtype is not None else t


def _routing(rng, kind, T, E, k):
    if kind == "uniform":
        return (rng.integers(0, E, (T, k)).astype(np.int32),
                rng.random((T, k)).astype(np.float32))
    if kind == "one":
        return np.zeros((T, k), np.int32), rng.random((T, k)).astype(np.float32)
    if kind == "softmax":
        return softmax_topk_routing(rng, T, E, k)
    return zipf_routing(rng, T, E, k)


@pytest.mark.parametrize("T,k,E,tm,kind", [(1, 8, 64, 32, "uniform"), (512, 8, 64, 32, "uniform"),
                                           (37, 4, 12, 16, "zipf"), (300, 8, 64, 96, "zipf"),
                                           (2000, 8, 64, 32, "uniform"), (50, 2, 3, 1, "zipf"),
                                           (64, 8, 1024, 7, "uniform"), (5, 3, 5, 1000, "zipf"),
                                           (700, 3, 4, 32, "one"), (100, 4, 1, 16, "uniform"),
                                           (4096, 9, 65, 80, "zipf"), (911, 9, 257, 80, "uniform")])
def test_ragged_plan_bit_exact(pkg, gpu, T, k, E, tm, kind):
    rng = np.random.default_rng(T * 31 + E)
    idx, w = _routing(rng, kind, T, E, k)
    got = {key: v.cpu().numpy() for key, v in pkg.ragged_plan(_t(idx), _t(w), E, tm).items()}
    want = omoe.ragged_plan(idx, w, E, tm)
    for key in ("blk_expert", "n_blocks", "tok_row", "row_slot"):
        assert np.array_equal(got[key], want[key]), key
    assert np.array_equal(got["w_row"].view(np.uint32), want["w_row"].view(np.uint32))


def test_ragged_plan_invalid_ids(pkg, gpu):
    """Expert ids outside [0, E) take no row (row_slot -1); the valid slots are placed as the oracle's plan places
    them when every invalid id is renamed to an extra last expert E, whose rows and blocks come after all others."""
    T, k, E, tm = 600, 8, 64, 32
    rng = np.random.default_rng(5)
    idx, w = _routing(rng, "zipf", T, E, k)
    bad = rng.random((T, k)) < 0.1
    idx = np.where(bad, np.where(rng.random((T, k)) < 0.5, -3, E + 7), idx).astype(np.int32)
    got = {key: v.cpu().numpy() for key, v in pkg.ragged_plan(_t(idx), _t(w), E, tm).items()}
    want = omoe.ragged_plan(np.where(bad, E, idx).astype(np.int32), w, E + 1, tm)
    nb = int(got["n_blocks"][0])
    assert nb == int(want["n_blocks"][0]) - (-(-int(bad.sum()) // tm))
    assert np.array_equal(got["blk_expert"][:nb], want["blk_expert"][:nb])
    assert np.all(got["blk_expert"][nb:] == (want["blk_expert"][nb - 1] if nb else E - 1))
    assert np.array_equal(got["tok_row"][:nb * tm], want["tok_row"][:nb * tm])
    assert np.all(got["tok_row"][nb * tm:] == -1)
    assert np.array_equal(got["w_row"][:nb * tm].view(np.uint32), want["w_row"][:nb * tm].view(np.uint32))
    assert np.array_equal(got["row_slot"], np.where(bad, -1, want["row_slot"]))


def _oracle_prefill(L, x, idx, w, limit, E, shared, combine):
    if shared is not None:
        idx = np.concatenate([idx, np.full((idx.shape[0], 1), shared, np.int32)], axis=1)
        w = np.concatenate([w, np.ones((w.shape[0], 1), np.float32)], axis=1)
        E = E + 1
    return omoe.prefill_apply(L.deq, x, idx, w, limit, E, combine=combine)


SMALL = [
    (40, 4, 6, 512, 256, False, "matmul", "zipf"),
    (40, 4, 6, 512, 256, True, "gather", "zipf"),
    (200, 2, 3, 1280, 384, True, "matmul", "zipf"),       # experts with several blocks of 80 rows
    (1, 8, 16, 512, 256, False, "matmul", "softmax"),
    (97, 1, 2, 512, 256, False, "gather", "one"),         # one expert: a full block and a 17-row block
    (33, 3, 5, 768, 128, True, "matmul", "uniform"),
]
# IQ3_S: whole 256-weight blocks per row (K % 256 == 0)
SMALL_IQ3 = [
    (40, 4, 6, 512, 256, False, "matmul", "zipf"),
    (40, 4, 6, 512, 256, True, "gather", "zipf"),
    (200, 2, 3, 1024, 512, True, "matmul", "zipf"),
    (1, 8, 16, 512, 256, False, "matmul", "softmax"),
    (97, 1, 2, 512, 256, False, "gather", "one"),
    (33, 3, 5, 768, 256, True, "matmul", "uniform"),
    (81, 2, 2, 2560, 768, True, "gather", "zipf"),        # partial super tiles of 128-column tiles (K / 128 = 20, 6)
]


@pytest.mark.parametrize("qtype,T,k,E,D,I,shared,combine,kind",
                         [("CB3",) + c for c in SMALL] + [("IQ3_S",) + c for c in SMALL_IQ3] +
                         [("IQ4_XS",) + c for c in SMALL_IQ3] + [("IQ2_S",) + c for c in SMALL_IQ3] +
                         [("Q2_K",) + c for c in SMALL_IQ3] + [("Q3_K",) + c for c in SMALL_IQ3])
def test_prefill_small(pkg, gpu, qtype, T, k, E, D, I, shared, combine, kind):
    rng = np.random.default_rng(7 * T + E)
    limit = 10.0
    L = Layer(rng, qtype, E + (1 if shared else 0), D, I)
    tbs = L.tables(pkg)
    idx, w = _routing(rng, kind, T, E, k)
    x = round_bf16(rng.standard_normal((T, D)).astype(np.float32))
    se = E if shared else -1
    of, ob = pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                             shared_expert=se, combine=combine, want_bf16=True)
    want = _oracle_prefill(L, x, idx, w, limit, E, E if shared else None, combine)
    err = rel_l2(of.cpu().numpy(), want)
    assert err < TOL, err
    assert torch.equal(ob, of.to(torch.bfloat16))
    of2, _ = pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                             shared_expert=se, combine=combine)
    assert torch.equal(of, of2)                      # deterministic


@pytest.mark.parametrize("qtype", ["CB3", "IQ2_S", "IQ3_S", "IQ4_XS", "Q2_K", "Q3_K"])
def test_prefill_limit_clamps(pkg, gpu, qtype):
    """A small swiglu limit makes the clamps of model.py:119-122 active in the gate/up epilogue."""
    rng = np.random.default_rng(4)
    E, D, I, T, k, limit = 5, 512, 256, 60, 3, 0.05
    L = Layer(rng, qtype, E, D, I)
    tbs = L.tables(pkg)
    idx, w = zipf_routing(rng, T, E, k)
    x = round_bf16(rng.standard_normal((T, D)).astype(np.float32))
    of, _ = pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit)
    assert rel_l2(of.cpu().numpy(), _oracle_prefill(L, x, idx, w, limit, E, None, "matmul")) < TOL


def test_prefill_full_shape(pkg, gpu, full_cb3_layer):
    """The benchmark layer's matrix shapes (hidden 6144, intermediate 2048) with two routed experts and the shared
    expert: 200 tokens put 200 rows on each expert, three blocks of up to 96 rows each."""
    rng = np.random.default_rng(2026)
    E, D, I, T, k, limit = 2, 6144, 2048, 200, 2, 10.0
    L, tbs = full_cb3_layer
    idx = np.tile(np.array([[0, 1]], np.int32), (T, 1))
    idx[::2] = idx[::2, ::-1]
    w = rng.random((T, k)).astype(np.float32)
    x = round_bf16(rng.standard_normal((T, D)).astype(np.float32))
    of, _ = pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                            shared_expert=E)
    err = rel_l2(of.cpu().numpy(), _oracle_prefill(L, x, idx, w, limit, E, E, "matmul"))
    assert err < TOL, err


@pytest.mark.parametrize("qtype", ["CB3", "IQ2_S", "IQ3_S", "IQ4_XS", "Q2_K", "Q3_K"])
def test_resident_fetch_prefill(pkg, gpu, qtype):
    """ResidentFetch.apply with N*k > gather_max_rows takes the grouped prefill path (resident.py:104-108)."""
    rng = np.random.default_rng(8)
    E, D, I, T, k, limit = 8, 512, 256, 24, 4, 10.0
    L = Layer(rng, qtype, E, D, I)
    p = {}
    for name, key in (("gate", "gate_q"), ("up", "up_q"), ("down", "down_q")):
        p[key] = pkg.to_device_planes(L.planes(name, pkg.formats))
    fetch = pkg.ResidentFetch({0: {"gate_q": qtype, "up_q": qtype, "down_q": qtype}}, D, I)
    idx, w = zipf_routing(rng, T, E, k)
    x = round_bf16(rng.standard_normal((T, D)).astype(np.float32))
    y = fetch.apply(p, _t(x, torch.bfloat16), _t(idx), _t(w), 0, limit)
    assert y.dtype == torch.float32 and tuple(y.shape) == (T, D)
    assert rel_l2(y.cpu().numpy(), _oracle_prefill(L, x, idx, w, limit, E, None, "matmul")) < TOL


def test_prefill_full_shape_iq3s(pkg, gpu):
    """IQ3_S at the benchmark layer's matrix shapes (hidden 6144, intermediate 2048): two routed experts and the
    shared expert, 120 tokens (two blocks of 80 rows per expert)."""
    rng = np.random.default_rng(2027)
    E, D, I, T, k, limit = 2, 6144, 2048, 120, 2, 10.0
    L = Layer(rng, "IQ3_S", E + 1, D, I)
    tbs = L.tables(pkg)
    idx = np.tile(np.array([[0, 1]], np.int32), (T, 1))
    idx[::2] = idx[::2, ::-1]
    w = rng.random((T, k)).astype(np.float32)
    x = round_bf16(rng.standard_normal((T, D)).astype(np.float32))
    of, _ = pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                            shared_expert=E)
    err = rel_l2(of.cpu().numpy(), _oracle_prefill(L, x, idx, w, limit, E, E, "matmul"))
    assert err < TOL, err


@pytest.mark.parametrize("qtype,down_qtype", [("IQ3_S", "IQ4_XS"), ("CB3", "IQ4_XS"), ("IQ4_XS", "IQ3_S"),
                                              ("IQ2_S", "IQ4_XS"), ("IQ2_S", "IQ3_S"), ("Q2_K", "Q3_K"),
                                              ("Q3_K", "Q2_K")])
def test_prefill_mixed_formats(pkg, gpu, qtype, down_qtype):
    """Gate/up in one format, down in another (the reference's layers mix formats per matrix kind)."""
    rng = np.random.default_rng(61)
    E, D, I, T, k, limit = 5, 768, 512, 90, 3, 10.0
    L = Layer(rng, qtype, E + 1, D, I, down_qtype=down_qtype)
    tbs = L.tables(pkg)
    idx, w = zipf_routing(rng, T, E, k)
    x = round_bf16(rng.standard_normal((T, D)).astype(np.float32))
    of, _ = pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                            shared_expert=E, combine="gather")
    err = rel_l2(of.cpu().numpy(), _oracle_prefill(L, x, idx, w, limit, E, E, "gather"))
    assert err < TOL, err
