"""The drop-in operator's branches on the GPU (ResidentFetch.apply, resident.py:100-108,137-143): decode calls beyond
one kernel call's 16 tokens / 128 slots (chunked), f32 activations, and out_dtype float32 -- the configuration of the
reference's own CPU tests (test_resident_cpu.py:81,92,124: f32 layers, gather_max_rows 8 / 1000, IQ2_S gate/up with
IQ3_S down) -- in every branch.

Bar: rel-L2 <= 1e-5 against the f64 oracle with bf16 activations (f32 throughout); with f32 activations 5e-5: x and h
each enter the matrix cores as bf16 high part + remainder (16 mantissa bits), and a CPU model of exactly that split
gives 0.8-1.6e-5 on these layers.
"""
F32X = 5e-5
import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle.bf16 import rel_l2, round_bf16
from tests.util import Layer, zipf_routing

pytestmark = pytest.mark.gpu


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(dtype) if dtype is not None else t


def _params(pkg, L):
    return {key: pkg.to_device_planes(L.planes(name, pkg.formats))
            for name, key in (("gate", "gate_q"), ("up", "up_q"), ("down", "down_q"))}


@pytest.mark.parametrize("N,k,gmr", [(20, 2, 1000), (40, 8, 1000), (3, 8, 64)])
def test_decode_branch_beyond_one_call(pkg, gpu, N, k, gmr):
    """N*k <= gather_max_rows with more than 16 tokens or 128 slots: the decode runs in chunks, f32 out."""
    rng = np.random.default_rng(100 + N)
    E, D, I, limit = 12, 512, 256, 10.0
    L = Layer(rng, "IQ2_S", E, D, I, down_qtype="IQ3_S")
    fetch = pkg.ResidentFetch({0: {"gate_q": "IQ2_S", "up_q": "IQ2_S", "down_q": "IQ3_S"}}, D, I,
                              gather_max_rows=gmr)
    assert fetch.branch(N, k) == "kernel"
    idx, w = zipf_routing(rng, N, E, k)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    y = fetch.apply(_params(pkg, L), _t(x, torch.bfloat16), _t(idx), _t(w), 0, limit)
    assert y.dtype == torch.float32 and tuple(y.shape) == (N, D)
    assert rel_l2(y.cpu().numpy(), omoe.decode_apply(L.deq, x, idx, w, limit)) < 1e-5


@pytest.mark.parametrize("qtype", ["CB3", "IQ3_S"])
@pytest.mark.parametrize("N", [1, 7, 16])
def test_decode_f32_activations(pkg, gpu, qtype, N):
    """x f32 (not bf16 values) through mi_moe_decode_x: the reference upcasts x to f32 and keeps it (resident.py:114)."""
    rng = np.random.default_rng(200 + N)
    E, D, I, k, limit = 9, 768 if qtype == "CB3" else 512, 256, 4, 10.0
    L = Layer(rng, qtype, E + 1, D, I)
    tbs = L.tables(pkg)
    idx, w = zipf_routing(rng, N, E, k)
    x = rng.standard_normal((N, D)).astype(np.float32)
    of, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], _t(x), _t(idx), _t(w), limit, shared_expert=E)
    want = omoe.decode_apply(L.deq, x, idx, w, limit) + omoe.shared_apply(lambda m: L.deq(m, E), x, limit)
    assert rel_l2(of.cpu().numpy(), want) < F32X


@pytest.mark.parametrize("use_pallas,sweep_mode,gmr", [(True, "ragged", 8), (True, "dense", 8), (False, "ragged", 8),
                                                       (False, "ragged", 1000), (True, "ragged", 1000)])
def test_f32_out_dtype_every_branch(pkg, gpu, use_pallas, sweep_mode, gmr):
    """The reference's CPU-test layer: f32 activations, out_dtype float32, IQ2_S gate/up + IQ3_S down, 20 tokens x
    top-2 (prefill branches with gather_max_rows 8, decode branches with 1000).  Every branch is the f32
    composition (oracle.moe.prefill_apply / sweep_apply / gather_apply / sweep_xla_apply with out_dtype "f32")."""
    rng = np.random.default_rng(300)
    E, D, I, T, k, limit = 16, 256, 256, 20, 2, 10.0
    L = Layer(rng, "IQ2_S", E, D, I, down_qtype="IQ3_S")
    fetch = pkg.ResidentFetch({3: {"gate_q": "IQ2_S", "up_q": "IQ2_S", "down_q": "IQ3_S"}}, D, I,
                              out_dtype=torch.float32, gather_max_rows=gmr, chunk=4, use_pallas=use_pallas,
                              sweep_mode=sweep_mode)
    idx, w = zipf_routing(rng, T, E, k)
    x = rng.standard_normal((T, D)).astype(np.float32)
    y = fetch.apply(_params(pkg, L), _t(x), _t(idx), _t(w), 3, limit)
    br = fetch.branch(T, k)
    want = {"ragged": lambda: omoe.prefill_apply(L.deq, x, idx, w, limit, E, tm=32, out_dtype="f32"),
            "sweep": lambda: omoe.sweep_apply(L.deq, x, idx, w, limit, E, out_dtype="f32"),
            "sweep_xla": lambda: omoe.sweep_xla_apply(L.deq, x, idx, w, limit, E, chunk=4, out_dtype="f32"),
            "gather": lambda: omoe.gather_apply(L.deq, x, idx, w, limit, out_dtype="f32"),
            "kernel": lambda: omoe.decode_apply(L.deq, x, idx, w, limit)}[br]()
    assert rel_l2(y.cpu().numpy(), want) < F32X
