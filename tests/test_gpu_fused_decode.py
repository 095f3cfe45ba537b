"""The CB3 decode layer as one persistent launch (mi_moe_decode_fused, up to 8 tokens) and as separate launches
(mi_moe_decode; persistent gate/up and down above 8 tokens): parity with the oracle and between the two forms, the counter hand-off (counters back at zero after every call, no
wait gives up), forced launch plans that exercise the split reductions, the combine and the restaging, invalid
routing ids, graph replays and the benchmark's full shape.

Bar: rel-L2 <= 1e-5 against the f64 oracle at small shapes (f32 accumulation throughout, resident.py:114-120); the
north-star bar is 1e-3 with bf16 output.
"""

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle.bf16 import rel_l2, round_bf16
from tests.util import Layer, softmax_topk_routing, zipf_routing

pytestmark = pytest.mark.gpu


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(dtype) if dtype is not None else t


def _want(L, x, idx, w, limit, shared):
    y = omoe.decode_apply(L.deq, x, idx, w, limit)
    if shared is not None:
        y = y + omoe.shared_apply(lambda m: L.deq(m, shared), x, limit)
    return y


def _counters_clean(pkg, tbs, ws, N, k, shared):
    plan = pkg.resident.decode_plan(tbs["gate"], tbs["down"], N, k, shared)
    words = ws[:plan["ctr_bytes"]].view(torch.int32).cpu().numpy()
    assert words[plan["err_word"]] == 0, "a wait gave up"
    nz = np.flatnonzero(words)
    assert nz.size == 0, "counter words left nonzero: %s" % nz[:8]
    return plan


@pytest.mark.parametrize("N,k,E,routing,shared", [(1, 8, 16, "softmax", True), (2, 4, 9, "zipf", False),
                                                  (8, 8, 20, "zipf", True), (16, 8, 24, "zipf", True),
                                                  (11, 3, 5, "zipf", True), (16, 1, 2, "zipf", False)])
def test_fused_vs_oracle_and_separate(pkg, gpu, N, k, E, routing, shared):
    rng = np.random.default_rng(700 + 13 * N + E)
    D, I, limit = 1280, 256, 10.0
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    idx, w = (softmax_topk_routing if routing == "softmax" else zipf_routing)(rng, N, E, k)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    se = E if shared else -1
    ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], N, k, se), dtype=torch.uint8,
                     device="cuda")
    args = (tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit)
    fused = N <= 8                                      # the one launch takes up to 8 tokens per group
    of, ob = pkg.moe_decode(*args, shared_expert=se, want_bf16=True, workspace=ws, fused=fused)
    torch.cuda.synchronize()
    _counters_clean(pkg, tbs, ws, N, k, se)
    want = _want(L, x, idx, w, limit, E if shared else None)
    assert rel_l2(of.cpu().numpy(), want) < 1e-5
    assert rel_l2(ob.float().cpu().numpy(), round_bf16(want)) < 1e-3
    sep, _ = pkg.moe_decode(*args, shared_expert=se, workspace=ws)
    # both within 1e-5 of the f64 oracle; the two launch plans may split the sums differently (f32 order only)
    assert rel_l2(of.cpu().numpy(), sep.cpu().numpy()) < 1e-5
    again, _ = pkg.moe_decode(*args, shared_expert=se, workspace=ws, fused=fused)
    assert torch.equal(of, again)                      # deterministic


def test_fused_repeated_calls_one_workspace(pkg, gpu):
    """Six calls with fresh routing and activations on one workspace: every result right, counters back at zero."""
    rng = np.random.default_rng(42)
    E, D, I, N, k, limit = 12, 640, 256, 6, 4, 10.0
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], N, k, E), dtype=torch.uint8,
                     device="cuda")
    for it in range(6):
        idx, w = zipf_routing(rng, N, E, k)
        x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
        of, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                               shared_expert=E, workspace=ws, fused=True)
        torch.cuda.synchronize()
        _counters_clean(pkg, tbs, ws, N, k, E)
        assert rel_l2(of.cpu().numpy(), _want(L, x, idx, w, limit, E)) < 1e-5, "call %d" % it


def test_fused_wait_give_up_is_reported_and_the_next_call_is_clean(pkg, gpu):
    """A poll limit of 0 set from the host makes a wait give up at its first unsuccessful poll (no kernel is kept
    from exiting: the launch just ends with invalid results).  The error word reports it; the next call with the
    default limit on the same workspace -- whose counters the forced calls may have left anywhere, as the garbage it
    started with -- is correct, with a clear error word and zero counters."""
    rng = np.random.default_rng(43)
    E, D, I, N, k, limit = 12, 640, 256, 6, 4, 10.0
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    ws = torch.full((pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], N, k, E),), 0xA5,
                    dtype=torch.uint8, device="cuda")
    idx, w = zipf_routing(rng, N, E, k)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    args = (tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit)
    with pkg.tuning(SPIN_LIMIT=0):
        gave_up = 0
        for _ in range(8):
            pkg.moe_decode(*args, shared_expert=E, workspace=ws, fused=True)
            gave_up += pkg.resident.fused_error(ws, tbs["gate"], tbs["down"]) != 0
        assert gave_up > 0, "no wait had to poll in 8 forced calls"
        with pytest.raises(RuntimeError):
            for _ in range(8):                       # check_error=True raises on a call whose wait gave up
                pkg.moe_decode(*args, shared_expert=E, workspace=ws, fused=True, check_error=True)
    of, _ = pkg.moe_decode(*args, shared_expert=E, workspace=ws, fused=True, check_error=True)
    torch.cuda.synchronize()
    _counters_clean(pkg, tbs, ws, N, k, E)
    assert rel_l2(of.cpu().numpy(), _want(L, x, idx, w, limit, E)) < 1e-5


@pytest.mark.parametrize("env,Ns,fused", [
    ({"FS1": 3, "FS2": 2}, (1, 5, 8), True),
    ({"FS1": 5, "FS1_RTW": 2, "FS2": 3}, (1, 5, 8), True),
    ({"FS1": 3, "FS1_RTW": 4, "FS2": 1}, (1, 5, 8), True),
    ({"FS1": 1, "FS2": 4}, (1, 2), True),
    ({"S1": 3, "S2": 2, "S1_RTW": 2, "CUMULTI": 0}, (12, 16), False),
    ({"S1": 2, "S2": 1, "S2_RTW": 1, "CUMULTI": 0}, (9, 16), False)])
def test_forced_plans(pkg, gpu, env, Ns, fused):
    """Column splits in both phases (the one launch: the last split of a row range forms h, the last down task
    combines; the separate persistent launches: contiguous task ranges that restage when the group or split
    changes), 32 and 64 rows per wavefront, single-split phases."""
    rng = np.random.default_rng(9)
    E, D, I, limit = 10, 1920, 512, 10.0
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    with pkg.tuning(**env):
        for N in Ns:
            k = 6 if N > 1 else 8
            idx, w = zipf_routing(rng, N, E, k)
            x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
            plan = pkg.resident.decode_plan(tbs["gate"], tbs["down"], N, k, E)
            assert plan["fused"] == int(fused), plan
            if fused:
                assert plan["S1"] == min(env["FS1"], 12), plan
            else:
                assert plan["sep_S1"] == env["S1"] and plan["sep_P1"] > 0, plan
            ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], N, k, E),
                             dtype=torch.uint8, device="cuda")
            of, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w),
                                   limit, shared_expert=E, workspace=ws, fused=fused)
            torch.cuda.synchronize()
            _counters_clean(pkg, tbs, ws, N, k, E)
            assert rel_l2(of.cpu().numpy(), _want(L, x, idx, w, limit, E)) < 1e-5, (N, k, plan)


def test_fused_invalid_ids_and_empty(pkg, gpu):
    """Ids outside [0, E) contribute nothing (as in the separate launches); with no valid id and no shared expert
    the output is zero."""
    rng = np.random.default_rng(77)
    E, D, I, limit = 6, 640, 256, 10.0
    L = Layer(rng, "CB3", E, D, I)
    tbs = L.tables(pkg)
    N, k = 3, 3
    idx = np.array([[0, -1, 4], [E, 2, 2], [5, 1, E + 9]], np.int32)
    w = np.full((N, k), 1.0 / k, np.float32)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], N, k, -1), dtype=torch.uint8,
                     device="cuda")
    of, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                           workspace=ws, fused=True)
    torch.cuda.synchronize()
    _counters_clean(pkg, tbs, ws, N, k, -1)
    valid = (idx >= 0) & (idx < E)
    want = omoe.decode_apply(L.deq, x, np.where(valid, idx, 0), np.where(valid, w, 0).astype(np.float32), limit)
    assert rel_l2(of.cpu().numpy(), want) < 1e-5
    bad = np.full((N, k), -3, np.int32)
    of0, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(bad), _t(w), limit,
                            workspace=ws, fused=True)
    torch.cuda.synchronize()
    assert not of0.abs().max().item()
    _counters_clean(pkg, tbs, ws, N, k, -1)


def test_fused_graph_replays(pkg, gpu):
    """mi_moe_decode captured in a HIP graph: five replays with eager work and synchronisations between them, each
    equal to the eager result."""
    rng = np.random.default_rng(5)
    E, D, I, N, k, limit = 16, 1280, 512, 4, 8, 10.0
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    idx, w = zipf_routing(rng, N, E, k)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    xt, it, wt = _t(x, torch.bfloat16), _t(idx), _t(w)
    ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], N, k, E), dtype=torch.uint8,
                     device="cuda")
    out = torch.empty((N, D), dtype=torch.float32, device="cuda")
    eager, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], xt, it, wt, limit, shared_expert=E, workspace=ws,
                              fused=True)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g):
            pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], xt, it, wt, limit, shared_expert=E, out_f32=out,
                           workspace=ws, fused=True)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for r in range(5):
        out.fill_(float("nan"))
        scratch = torch.randn(1 << 20, device="cuda").sum()            # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), "replay %d" % r
        assert torch.isfinite(scratch)
    _counters_clean(pkg, tbs, ws, N, k, E)


def test_fused_full_shape(pkg, gpu, full_cb3_layer):
    """The benchmark's layer shape (D = 6144, I = 2048): 64 routed + 1 shared random experts (generated on the GPU),
    the one launch against the separate launches at batch 1, 8 and 16; and against the oracle at batch 2 with two
    routed experts and the shared one."""
    rng = np.random.default_rng(2)
    E, D, I, limit = 64, 6144, 2048, 10.0
    gen = torch.Generator(device="cuda")
    gen.manual_seed(31)
    tbs = {name: pkg.random_cb3_table(E + 1, R, K, gen) for name, (R, K) in
           (("gate", (I, D)), ("up", (I, D)), ("down", (D, I)))}
    for N, k in ((1, 8), (8, 8), (16, 8)):
        idx, w = (softmax_topk_routing if N == 1 else zipf_routing)(rng, N, E, k)
        xt = torch.randn((N, D), device="cuda", generator=gen).to(torch.bfloat16)
        ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], N, k, E), dtype=torch.uint8,
                         device="cuda")
        args = (tbs["gate"], tbs["up"], tbs["down"], xt, _t(idx), _t(w), limit)
        sep, _ = pkg.moe_decode(*args, shared_expert=E, workspace=ws)
        if N > 8:                                  # the separate launches only: persistent at this size (checked
                                                   # against an f64 reference in test_gpu_configs.py)
            assert pkg.resident.decode_plan(tbs["gate"], tbs["down"], N, k, E)["sep_P1"] > 0
            continue
        of, _ = pkg.moe_decode(*args, shared_expert=E, workspace=ws, fused=True)
        torch.cuda.synchronize()
        _counters_clean(pkg, tbs, ws, N, k, E)
        # the two launch plans split the K = 6144 / 2048 sums differently: f32 summation-order noise only
        assert rel_l2(of.cpu().numpy(), sep.cpu().numpy()) < 1e-5, (N, k)
    L, tbs3 = full_cb3_layer
    N, k = 2, 2
    idx = np.array([[0, 1], [1, 0]], np.int32)
    w = np.array([[0.6, 0.4], [0.3, 0.7]], np.float32)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    want = _want(L, x, idx, w, limit, 2)
    for fused in (True, False):
        of, _ = pkg.moe_decode(tbs3["gate"], tbs3["up"], tbs3["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                               shared_expert=2, fused=fused)
        assert rel_l2(of.cpu().numpy(), want) < 1e-5, fused
