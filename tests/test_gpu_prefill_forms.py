"""GPU parity of the grouped prefill GEMMs in the rounding forms of the reference's other bf16 branches of
ResidentFetch.apply (mi_moe_prefill_form): the dense sweep (sweep_mode "dense", resident.py:169-187 with
pallas_moe.py:382-555), the XLA decode path (use_pallas=False, resident.py:122-135) and the XLA prefill path
(use_pallas=False, resident.py:189-210), against oracle.moe.sweep_apply / gather_apply / sweep_xla_apply.

Bar: rel-L2 <= 3e-4.  Each form's oracle lies 7e-4 .. 5e-3 from the ragged form's on these layers (each test checks
that it is more than 2x the bar away), so the bar tells the forms apart.  The kernels accumulate in f32 against the
oracle's f64, so an element next to a bf16 rounding boundary may round the other way: observed 1e-7 .. 1e-4, the
largest for the XLA forms, whose g and u are rounded too (a flipped g moves h, and y, by one bf16 step).  Routing with repeated experts per token ("uniform" over few experts, "one") exercises the sweeps'
summed routing weight.
"""
import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle.bf16 import rel_l2, round_bf16
from tests.util import Layer, zipf_routing

pytestmark = pytest.mark.gpu
TOL = 3e-4
APART = 2 * TOL


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(dtype) if dtype is not None else t


def _routing(rng, kind, T, E, k):
    if kind == "uniform":
        return rng.integers(0, E, (T, k)).astype(np.int32), rng.random((T, k)).astype(np.float32)
    if kind == "one":
        return np.zeros((T, k), np.int32), rng.random((T, k)).astype(np.float32)
    return zipf_routing(rng, T, E, k)


def _with_shared(idx, w, E, shared):
    if shared is None:
        return idx, w, E
    idx = np.concatenate([idx, np.full((idx.shape[0], 1), shared, np.int32)], axis=1)
    w = np.concatenate([w, np.ones((w.shape[0], 1), np.float32)], axis=1)
    return idx, w, E + 1


def _oracle(form, L, x, idx, w, limit, E, chunk):
    if form == "sweep":
        return omoe.sweep_apply(L.deq, x, idx, w, limit, E)
    if form == "xla_gather":
        return omoe.gather_apply(L.deq, x, idx, w, limit)
    if form == "xla_sweep":
        return omoe.sweep_xla_apply(L.deq, x, idx, w, limit, E, chunk=chunk)
    return omoe.prefill_apply(L.deq, x, idx, w, limit, E, combine=form)


# (gate/up format, down format, T, k, E, D, I, shared expert, routing)
CASES = [
    ("CB3", None, 40, 4, 6, 512, 256, False, "zipf"),
    ("CB3", None, 33, 3, 5, 768, 128, True, "uniform"),
    ("IQ3_S", None, 97, 2, 4, 512, 256, True, "uniform"),
    ("IQ3_S", None, 50, 3, 4, 512, 256, False, "one"),
    ("IQ2_S", "IQ3_S", 81, 2, 6, 512, 256, True, "zipf"),
    ("IQ4_XS", None, 20, 8, 16, 512, 256, False, "uniform"),
    ("Q3_K", "Q2_K", 64, 4, 8, 512, 256, True, "zipf"),
]


@pytest.mark.parametrize("form", ["sweep", "xla_gather", "xla_sweep"])
@pytest.mark.parametrize("qtype,down_qtype,T,k,E,D,I,shared,kind", CASES)
def test_prefill_form_matches_oracle(pkg, gpu, form, qtype, down_qtype, T, k, E, D, I, shared, kind):
    rng = np.random.default_rng(T * 7 + E + k)
    limit, chunk = 7.0, 4
    L = Layer(rng, qtype, E + 1, D, I, down_qtype=down_qtype)
    tbs = L.tables(pkg)
    idx, w = _routing(rng, kind, T, E, k)
    x = round_bf16(rng.standard_normal((T, D)).astype(np.float32))
    sh = E if shared else -1
    of, ob = pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                             shared_expert=sh, combine=form, chunk=chunk, want_bf16=True)
    oi, ow, oE = _with_shared(idx, w, E, E if shared else None)
    want = _oracle(form, L, x, oi, ow, limit, oE, chunk)
    got = of.cpu().numpy().astype(np.float64)
    d = rel_l2(got, want)
    print("%s %s rel-L2 %.2e" % (form, qtype, d))
    assert d < TOL
    # the bf16 output is the f32 output rounded once
    assert np.array_equal(ob.float().cpu().numpy(), round_bf16(of.cpu().numpy()))
    # the bar separates this form from the ragged one on the same inputs
    assert rel_l2(want, _oracle("gather", L, x, oi, ow, limit, oE, chunk)) > APART


@pytest.mark.parametrize("chunk", [1, 3, 8])
def test_xla_sweep_chunk_sizes(pkg, gpu, chunk):
    """Group sizes from one expert per group to every expert in one group (including the shared one)."""
    rng = np.random.default_rng(40 + chunk)
    E, D, I, T, k, limit = 8, 512, 256, 60, 4, 7.0
    L = Layer(rng, "IQ3_S", E + 1, D, I)
    tbs = L.tables(pkg)
    idx, w = zipf_routing(rng, T, E, k)
    x = round_bf16(rng.standard_normal((T, D)).astype(np.float32))
    of, _ = pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                            shared_expert=E, combine="xla_sweep", chunk=chunk)
    oi, ow, oE = _with_shared(idx, w, E, E)
    assert rel_l2(of.cpu().numpy(), omoe.sweep_xla_apply(L.deq, x, oi, ow, limit, oE, chunk=chunk)) < TOL


@pytest.mark.parametrize("use_pallas,sweep_mode,N,form", [(False, "ragged", 6, "xla_gather"),
                                                          (True, "dense", 40, "sweep"),
                                                          (False, "dense", 40, "xla_sweep")])
def test_resident_fetch_bf16_branches(pkg, gpu, use_pallas, sweep_mode, N, form):
    """ResidentFetch.apply with bf16 out_dtype routes the dense-sweep and XLA branches to their forms."""
    rng = np.random.default_rng(5 + N)
    E, D, I, k, limit, chunk = 8, 512, 256, 2, 7.0, 4
    L = Layer(rng, "IQ2_S", E, D, I, down_qtype="IQ3_S")
    fetch = pkg.ResidentFetch({0: {"gate_q": "IQ2_S", "up_q": "IQ2_S", "down_q": "IQ3_S"}}, D, I,
                              use_pallas=use_pallas, sweep_mode=sweep_mode, chunk=chunk, gather_max_rows=16)
    assert fetch.branch(N, k) == {"xla_gather": "gather", "sweep": "sweep", "xla_sweep": "sweep_xla"}[form]
    params = {key: pkg.to_device_planes(L.planes(name, pkg.formats))
              for name, key in (("gate", "gate_q"), ("up", "up_q"), ("down", "down_q"))}
    idx, w = _routing(rng, "uniform", N, E, k)
    x = rng.standard_normal((N, D)).astype(np.float32)
    y = fetch.apply(params, _t(x, torch.bfloat16), _t(idx), _t(w), 0, limit)
    assert y.dtype == torch.float32 and tuple(y.shape) == (N, D)
    want = _oracle(form, L, round_bf16(x), idx, w, limit, E, chunk)
    assert rel_l2(y.cpu().numpy(), want) < TOL


def test_sweep_duplicate_expert_adds_once(pkg, gpu):
    """A token naming one expert in several columns: the sweep scales h by the summed weight once
    (bf16(h * (w0 + w1))), which is not the sum of the per-column products."""
    rng = np.random.default_rng(77)
    E, D, I, T, k, limit = 3, 512, 256, 24, 3, 7.0
    L = Layer(rng, "CB3", E, D, I)
    tbs = L.tables(pkg)
    idx = np.zeros((T, k), np.int32)
    idx[:, 2] = 1
    w = rng.random((T, k)).astype(np.float32)
    x = round_bf16(rng.standard_normal((T, D)).astype(np.float32))
    of, _ = pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                            combine="sweep")
    got = of.cpu().numpy()
    assert rel_l2(got, omoe.sweep_apply(L.deq, x, idx, w, limit, E)) < TOL
    # per-column weighting (no merge) is a different result at this bar
    split = sum(omoe.sweep_apply(L.deq, x, idx[:, j:j + 1], w[:, j:j + 1], limit, E) for j in range(k))
    assert rel_l2(got, split) > 2 * TOL


def test_form_workspace_sizes(pkg, gpu):
    """The sweeps keep y in f32: their workspace is larger than the ragged forms'; an unknown form is refused."""
    rng = np.random.default_rng(3)
    L = Layer(rng, "CB3", 4, 512, 256)
    tbs = L.tables(pkg)
    n = {f: pkg.prefill_workspace_bytes(tbs["gate"], tbs["down"], 100, 4, -1, f)
         for f in ("matmul", "gather", "sweep", "xla_gather", "xla_sweep")}
    assert n["matmul"] == n["gather"] == n["xla_gather"] < n["sweep"] == n["xla_sweep"]
    with pytest.raises(ValueError):
        pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], torch.zeros((4, 512), dtype=torch.bfloat16).cuda(),
                        torch.zeros((4, 2), dtype=torch.int32).cuda(), torch.ones((4, 2)).cuda(), 7.0,
                        combine="dense")
