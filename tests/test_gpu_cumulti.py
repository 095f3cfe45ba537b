"""The CU-balanced multi-token decode launches (CB3, 2-16 tokens; cumulti.h) against the oracle: forced column
splits and row tiles in both launches, down shares run as several epochs (fewer groups staged at a time), the one-
and two-instruction forms of h (up to 8 / more than 8 tokens), duplicate experts within a token (groups keyed by
(expert, occurrence)), expert ids outside the table, the shared expert, and a repeated call on one workspace.

Bar: rel-L2 <= 1e-5 against the f64 oracle (f32 throughout, h as bf16 high part + remainder)."""

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


def _run(pkg, L, tbs, N, k, E, idx, w, limit, shared):
    x = round_bf16(np.random.default_rng(N * 13 + k).standard_normal((N, L.D)).astype(np.float32))
    plan = pkg.resident.decode_plan(tbs["gate"], tbs["down"], N, k, E if shared else -1)
    assert plan["sep_kind"] == 3, plan
    of, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                           shared_expert=E if shared else -1)
    valid = (idx >= 0) & (idx < E)
    want = omoe.decode_apply(L.deq, x, np.where(valid, idx, 0), np.where(valid, w, 0.0), limit)
    if shared:
        want = want + omoe.shared_apply(lambda m: L.deq(m, E), x, limit)
    return of, want


ENVS = [{}, {"MS1": 1, "MS2": 1}, {"MS1": 3, "MS1_RTW": 2}, {"MS2": 3, "MS2_RTW": 4, "MGMAX": 1},
        {"MS2": 1, "MGMAX": 1, "MS1_RTW": 4}]


@pytest.mark.parametrize("env", ENVS)
@pytest.mark.parametrize("N,k,E,shared", [(2, 8, 16, True), (5, 3, 7, False), (8, 8, 24, True), (9, 4, 12, True),
                                          (16, 8, 40, True), (16, 2, 3, False)])
def test_cumulti_vs_oracle(pkg, gpu, env, N, k, E, shared):
    rng = np.random.default_rng(N * 100 + k * 10 + E)
    D, I, limit = 1920, 512, 10.0
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    idx, w = zipf_routing(rng, N, E, k)
    with pkg.tuning(**env):
        of, want = _run(pkg, L, tbs, N, k, E, idx, w, limit, shared)
    assert rel_l2(of.cpu().numpy(), want) < 1e-5


@pytest.mark.parametrize("N", [3, 12])
def test_cumulti_duplicates_and_invalid_ids(pkg, gpu, N):
    """A token naming one expert in several columns forms groups (e, 0), (e, 1), ...; ids outside [0, E) add
    nothing (the reference leaves them undefined; the decode skips them)."""
    rng = np.random.default_rng(7 + N)
    E, D, I, k, limit = 5, 640, 256, 6, 10.0
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    idx = rng.integers(0, 3, (N, k)).astype(np.int32)        # many repeats of experts 0-2
    idx[0, :3] = 1
    idx[1, 0] = -1
    idx[N - 1, k - 1] = E + 7
    w = rng.random((N, k)).astype(np.float32)
    with pkg.tuning(MGMAX=1):
        of, want = _run(pkg, L, tbs, N, k, E, idx, w, limit, True)
    assert rel_l2(of.cpu().numpy(), want) < 1e-5


def test_cumulti_repeated_calls_bit_identical(pkg, gpu):
    rng = np.random.default_rng(31)
    E, D, I, N, k, limit = 20, 1280, 384, 10, 8, 10.0
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    idx, w = zipf_routing(rng, N, E, k)
    x = _t(round_bf16(rng.standard_normal((N, D)).astype(np.float32)), torch.bfloat16)
    ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], N, k, E), dtype=torch.uint8,
                     device="cuda")
    a, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], x, _t(idx), _t(w), limit, shared_expert=E, workspace=ws)
    b, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], x, _t(idx), _t(w), limit, shared_expert=E, workspace=ws)
    assert torch.equal(a, b)
