"""The CB3 single-token decode's down launch doing the routing-weighted combine itself (custream.h): the last
workgroup to finish each 16-row tile sums that tile's partials in the combine launch's order.

Same arithmetic as the combine launch (the CU_COMBINE override 0 selects it), so the outputs must be equal bit for
bit, and both within rel-L2 1e-5 of the f64 oracle.  The workspace's counter block is zero again after every call.
"""
import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle.bf16 import rel_l2, round_bf16
from tests.util import Layer, softmax_topk_routing

pytestmark = pytest.mark.gpu


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(dtype) if dtype is not None else t


def _block_words(pkg, tbs, ws, k, shared):
    plan = pkg.resident.decode_plan(tbs["gate"], tbs["down"], 1, k, shared)
    torch.cuda.synchronize()
    return ws[:plan["ctr_bytes"]].view(torch.int32).cpu().numpy()


def _run(pkg, tbs, x, idx, w, limit, shared, ws, in_launch):
    with pkg.tuning(CU_COMBINE=int(in_launch)):
        plan = pkg.resident.decode_plan(tbs["gate"], tbs["down"], 1, idx.shape[1], shared)
        assert plan["sep_kind"] == 2 and plan["cu_combine"] == int(in_launch), plan
        return pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], x, idx, w, limit, shared_expert=shared,
                              want_bf16=True, workspace=ws)


@pytest.mark.parametrize("D,I,E,k,shared", [(1280, 256, 16, 8, True), (1920, 512, 9, 8, False),
                                            (640, 768, 5, 3, True), (2560, 1024, 40, 16, True)])
def test_in_launch_combine_equals_combine_launch_and_oracle(pkg, gpu, D, I, E, k, shared):
    rng = np.random.default_rng(D + I + E + k)
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    idx, w = softmax_topk_routing(rng, 1, E, k)
    x = round_bf16(rng.standard_normal((1, D)).astype(np.float32))
    se = E if shared else -1
    ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], 1, k, se), dtype=torch.uint8,
                     device="cuda")
    args = (_t(x, torch.bfloat16), _t(idx), _t(w), 10.0, se, ws)
    of, ob = _run(pkg, tbs, *args, True)
    rf, rb = _run(pkg, tbs, *args, False)
    assert torch.equal(of, rf) and torch.equal(ob, rb)
    want = omoe.decode_apply(L.deq, x, idx, w, 10.0)
    if shared:
        want = want + omoe.shared_apply(lambda m: L.deq(m, E), x, 10.0)
    assert rel_l2(of.cpu().numpy(), want) < 1e-5
    assert np.count_nonzero(_block_words(pkg, tbs, ws, k, se)) == 0


def test_in_launch_combine_full_shape_repeated_calls(pkg, gpu, full_cb3_layer):
    """The benchmark's matrices (D 6144, I 2048), several calls on one workspace with different routings: every call
    equals the combine launch's result and leaves the counter block zero."""
    L, tbs = full_cb3_layer
    rng = np.random.default_rng(5)
    ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], 1, 2, 2), dtype=torch.uint8,
                     device="cuda")
    for rep in range(4):
        idx = rng.permutation(2)[None].astype(np.int32)
        w = rng.random((1, 2)).astype(np.float32)
        x = _t(round_bf16(rng.standard_normal((1, 6144)).astype(np.float32)), torch.bfloat16)
        of, ob = _run(pkg, tbs, x, _t(idx), _t(w), 10.0, 2, ws, True)
        rf, rb = _run(pkg, tbs, x, _t(idx), _t(w), 10.0, 2, ws, False)
        assert torch.equal(of, rf) and torch.equal(ob, rb), "call %d" % rep
        assert np.count_nonzero(_block_words(pkg, tbs, ws, 2, 2)) == 0, "call %d" % rep


def test_workspace_shared_by_layer_shapes(pkg, gpu, full_cb3_layer):
    """One decode workspace used by layers of two shapes in turn (a smaller layer, then the benchmark's matrices, and
    again): the counter positions depend on the shape, so the partials of one shape must never land where the other
    keeps its counters (a fixed counter region).  Every call equals the combine launch's result on a fresh
    workspace and leaves its counters zero."""
    _, big = full_cb3_layer
    rng = np.random.default_rng(91)
    small = Layer(rng, "CB3", 41, 2560, 1024).tables(pkg)
    shapes = ((small, 2560, 40, 8, 40), (big, 6144, 2, 2, 2))
    nbytes = max(pkg.resident.decode_workspace_bytes(t["gate"], t["down"], 1, k, se) for t, _, _, k, se in shapes)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    for rep in range(4):
        tbs, D, E, k, se = shapes[rep % 2]
        idx, w = softmax_topk_routing(rng, 1, E, k)
        x = _t(round_bf16(rng.standard_normal((1, D)).astype(np.float32)), torch.bfloat16)
        of, ob = _run(pkg, tbs, x, _t(idx), _t(w), 10.0, se, ws, True)
        fresh = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
        rf, rb = _run(pkg, tbs, x, _t(idx), _t(w), 10.0, se, fresh, False)
        assert torch.equal(of, rf) and torch.equal(ob, rb), "call %d" % rep
        assert np.count_nonzero(_block_words(pkg, tbs, ws, k, se)) == 0, "call %d" % rep


def test_in_launch_combine_invalid_ids(pkg, gpu):
    """Ids outside [0, E) add nothing, as in the combine launch."""
    rng = np.random.default_rng(8)
    E, D, I, k = 6, 1280, 256, 5
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    idx = np.array([[2, -1, 4, E + 3, 2]], np.int32)
    w = rng.random((1, k)).astype(np.float32)
    x = round_bf16(rng.standard_normal((1, D)).astype(np.float32))
    ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], 1, k, E), dtype=torch.uint8,
                     device="cuda")
    args = (_t(x, torch.bfloat16), _t(idx), _t(w), 10.0, E, ws)
    of, _ = _run(pkg, tbs, *args, True)
    rf, _ = _run(pkg, tbs, *args, False)
    assert torch.equal(of, rf)
    valid = (idx >= 0) & (idx < E)
    want = omoe.decode_apply(L.deq, x, np.where(valid, idx, 0), np.where(valid, w, 0.0), 10.0)
    want = want + omoe.shared_apply(lambda m: L.deq(m, E), x, 10.0)
    assert rel_l2(of.cpu().numpy(), want) < 1e-5


def test_in_launch_combine_graph_replays(pkg, gpu):
    """The two launches captured in a HIP graph: every replay (eager work and synchronisations between them) equals
    the eager call, and the counters stay zero."""
    rng = np.random.default_rng(19)
    E, D, I, k = 10, 1920, 512, 8
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    idx, w = softmax_topk_routing(rng, 1, E, k)
    x = _t(round_bf16(rng.standard_normal((1, D)).astype(np.float32)), torch.bfloat16)
    it, wt = _t(idx), _t(w)
    ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], 1, k, E), dtype=torch.uint8,
                     device="cuda")
    ref, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], x, it, wt, 10.0, shared_expert=E, workspace=ws)
    out = torch.empty_like(ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], x, it, wt, 10.0, shared_expert=E, workspace=ws,
                       out_f32=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], x, it, wt, 10.0, shared_expert=E, workspace=ws,
                       out_f32=out)
    for rep in range(4):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), "replay %d" % rep
        _ = (x.float() * 2).sum().item()                 # eager work between replays
    assert np.count_nonzero(_block_words(pkg, tbs, ws, k, E)) == 0


@pytest.mark.parametrize("cs1", [1, 3, 4])
def test_down_forms_h_from_any_split_count(pkg, gpu, cs1):
    """The batch-1 down launch forms h from the gate/up partials of any number of column splits (summed in order
    from zero, as the SwiGLU launch sums them): bit-identical to the SwiGLU launch (CU_FORM_H override 0)."""
    rng = np.random.default_rng(60 + cs1)
    E, D, I, k = 9, 3200, 512, 8
    L = Layer(rng, "CB3", E + 1, D, I)
    tbs = L.tables(pkg)
    idx, w = softmax_topk_routing(rng, 1, E, k)
    x = _t(round_bf16(rng.standard_normal((1, D)).astype(np.float32)), torch.bfloat16)
    outs = []
    for form in (1, 0):
        with pkg.tuning(CS1=cs1, CU_FORM_H=form):
            assert pkg.resident.decode_plan(tbs["gate"], tbs["down"], 1, k, E)["sep_S1"] == cs1
            ws = torch.zeros(pkg.resident.decode_workspace_bytes(tbs["gate"], tbs["down"], 1, k, E),
                             dtype=torch.uint8, device="cuda")
            outs.append(pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], x, _t(idx), _t(w), 10.0,
                                       shared_expert=E, workspace=ws)[0])
    assert torch.equal(outs[0], outs[1])
    want = omoe.decode_apply(L.deq, x.float().cpu().numpy(), idx, w, 10.0)
    want = want + omoe.shared_apply(lambda m: L.deq(m, E), x.float().cpu().numpy(), 10.0)
    assert rel_l2(outs[0].cpu().numpy(), want) < 1e-5
