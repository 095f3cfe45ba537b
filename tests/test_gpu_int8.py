"""GPU parity of the int8 projection (quant8.py:91-99 + x @ W) against the oracle: bf16(f32(q)*s) weights, exact
bf16 products, f32 accumulation, bf16 out."""
import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import int8 as oi8
from oracle.bf16 import rel_l2, round_bf16

pytestmark = pytest.mark.gpu

CTR_BYTES = 2 * 1024 * 128      # the int8 workspace's counter blocks


@pytest.mark.parametrize("B,n_in,n_out", [(8, 512, 256), (1, 256, 16), (8, 2048, 6144), (16, 1024, 2048),
                                          (32, 512, 512), (3, 6144, 2048),
                                          (8, 6144, 6144), (8, 6144, 2048)])      # config 3: Q/K/V/O, shared gate/up
def test_int8_project(pkg, gpu, B, n_in, n_out):
    rng = np.random.default_rng(B * 1000 + n_out)
    q, s = oi8.generate(rng, n_in, n_out)
    x = round_bf16(rng.standard_normal((B, n_in)).astype(np.float32))
    qT, sv, _ = pkg.formats.int8_pack(q, s)
    yb, yf = pkg.int8_project(torch.from_numpy(x).cuda().to(torch.bfloat16), torch.from_numpy(qT).cuda(),
                              torch.from_numpy(sv).cuda(), want_f32=True)
    want = oi8.project_f32(x, q, s)
    assert rel_l2(yf.cpu().numpy(), want) < 1e-5
    assert rel_l2(yb.float().cpu().numpy(), oi8.project_bf16(x, q, s)) < 1e-3


def test_int8_golden(pkg, gpu):
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "int8.npz"))
    qT, sv, _ = pkg.formats.int8_pack(z["q"], z["s"])
    yb = pkg.int8_project(torch.from_numpy(z["x"]).cuda().to(torch.bfloat16), torch.from_numpy(qT).cuda(),
                          torch.from_numpy(sv).cuda())
    assert rel_l2(yb.float().cpu().numpy(), z["y"]) < 1e-3


def test_int8_project_many_equals_single(pkg, gpu):
    """One launch over Q, K, V-like projections (and a narrower one) gives exactly what separate calls give."""
    rng = np.random.default_rng(9)
    B, n_in = 8, 1024
    shapes = [512, 512, 256, 768]
    qs = [oi8.generate(rng, n_in, n) for n in shapes]
    x = round_bf16(rng.standard_normal((B, n_in)).astype(np.float32))
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    projs = []
    for q, s in qs:
        qT, sv, _ = pkg.formats.int8_pack(q, s)
        projs.append((torch.from_numpy(qT).cuda(), torch.from_numpy(sv).cuda()))
    many = pkg.int8_project_many(xt, projs, want_f32=True)
    for (q, s), (qT, sv), (yb, yf) in zip(qs, projs, many):
        yb1, yf1 = pkg.int8_project(xt, qT, sv, want_f32=True)
        assert rel_l2(yf.cpu().numpy(), yf1.cpu().numpy()) < 1e-6
        assert rel_l2(yf.cpu().numpy(), oi8.project_f32(x, q, s)) < 1e-5


def test_int8_split_sums_shared_lines(pkg, gpu):
    """n_out % 32 == 16 and a workspace aligned to 16 bytes only: one 128-byte line of split partials then holds
    partials of two row groups with different counters, and each row group's last workgroup must still read every
    split's stored value (device-coherent loads).  Several projections, many splits, repeated calls."""
    rng = np.random.default_rng(47)
    B, n_in = 8, 6144
    shapes = [80, 48, 112, 80]
    qs = [oi8.generate(rng, n_in, n) for n in shapes]
    x = round_bf16(rng.standard_normal((B, n_in)).astype(np.float32))
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    projs = []
    for q, s in qs:
        qT, sv, _ = pkg.formats.int8_pack(q, s)
        projs.append((torch.from_numpy(qT).cuda(), torch.from_numpy(sv).cuda()))
    L = pkg._lib.lib()
    n_outs = (ctypes.c_int32 * len(shapes))(*shapes)
    nbytes = L.mi_int8_project_many_workspace(B, n_in, n_outs, len(shapes), 1)
    raw = torch.zeros(nbytes + 256, dtype=torch.uint8, device="cuda")
    ws = raw[16:16 + nbytes]                          # 16-byte aligned, not 128
    first = None
    for rep in range(3):
        many = pkg.int8_project_many(xt, projs, want_f32=True, workspace=ws)
        for (q, s), (yb, yf) in zip(qs, many):
            assert rel_l2(yf.cpu().numpy(), oi8.project_f32(x, q, s)) < 1e-5, "call %d" % rep
        if first is None:
            first = [yf.clone() for _, yf in many]
        else:
            for a, (_, yf) in zip(first, many):
                assert torch.equal(a, yf)
    assert int(ws[:CTR_BYTES].count_nonzero()) == 0


def test_int8_split_sums_leave_counters_zero(pkg, gpu):
    """The split-K sums run in the projection launch (the last workgroup of each row group adds the partials in split
    order, counted in the workspace's first 256 KB): calls sharing one workspace -- three projections of 6144 x 6144
    at 8 tokens (3 splits), a smaller call, the MLP -- give the same bits every time and leave the counters zero."""
    rng = np.random.default_rng(31)
    B, n_in = 8, 6144
    qs = [oi8.generate(rng, n_in, 6144) for _ in range(3)]
    x = round_bf16(rng.standard_normal((B, n_in)).astype(np.float32))
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    projs = []
    for q, s in qs:
        qT, sv, _ = pkg.formats.int8_pack(q, s)
        projs.append((torch.from_numpy(qT).cuda(), torch.from_numpy(sv).cuda()))
    L = pkg._lib.lib()
    n_outs = (ctypes.c_int32 * 3)(6144, 6144, 6144)
    nbytes = max(L.mi_int8_project_many_workspace(B, n_in, n_outs, 3, 1), L.mi_int8_mlp_workspace(3, 1024, 512, 1, 0))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    first = pkg.int8_project_many(xt, projs, want_f32=True, workspace=ws)
    for (q, s), (yb, yf) in zip(qs, first):
        assert rel_l2(yf.cpu().numpy(), oi8.project_f32(x, q, s)) < 1e-5
    assert int(ws[:CTR_BYTES].count_nonzero()) == 0
    # a smaller projection, then the MLP, on the same workspace
    q2, s2 = oi8.generate(rng, 1024, 512)
    x2 = round_bf16(rng.standard_normal((3, 1024)).astype(np.float32))
    x2t = torch.from_numpy(x2).cuda().to(torch.bfloat16)
    qT2, sv2, _ = pkg.formats.int8_pack(q2, s2)
    y2 = pkg.int8_project(x2t, torch.from_numpy(qT2).cuda(), torch.from_numpy(sv2).cuda(), want_f32=True,
                          workspace=ws)[1]
    assert rel_l2(y2.cpu().numpy(), oi8.project_f32(x2, q2, s2)) < 1e-5
    gq, gs = oi8.generate(rng, 1024, 512)
    uq, us = oi8.generate(rng, 1024, 512)
    dq, ds = oi8.generate(rng, 512, 1024)
    leaves = [pkg.formats.int8_pack(q, s) for q, s in ((gq, gs), (uq, us), (dq, ds))]
    leaves = [(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), c) for a, b, c in leaves]
    m1 = pkg.int8_mlp(x2t, *leaves, 7.0, workspace=ws)
    assert int(ws[:CTR_BYTES].count_nonzero()) == 0
    m2 = pkg.int8_mlp(x2t, *leaves, 7.0, workspace=ws)
    assert torch.equal(m1, m2)
    for _ in range(2):
        again = pkg.int8_project_many(xt, projs, want_f32=True, workspace=ws)
        for (yb, yf), (yb1, yf1) in zip(first, again):
            assert torch.equal(yb, yb1) and torch.equal(yf, yf1)
    assert int(ws[:CTR_BYTES].count_nonzero()) == 0


@pytest.mark.parametrize("B,n_in,n_out", [(8, 6144, 6144), (8, 2048, 6144), (1, 512, 256), (20, 1024, 512)])
def test_int8_row_scales(pkg, gpu, B, n_in, n_out):
    """Per-row scales [in, 1], the reference's layout for row-sharded leaves (O and down projections;
    quant8.py:26-32,59-60): W = bf16(f32(q[i, o]) * s[i])."""
    rng = np.random.default_rng(B + n_in + n_out)
    q = rng.integers(-127, 128, (n_in, n_out), dtype=np.int8)
    s = rng.uniform(0.5e-3, 2e-3, (n_in, 1)).astype(np.float32)
    x = round_bf16(rng.standard_normal((B, n_in)).astype(np.float32))
    qT, sv, axis = pkg.resident.int8_leaf({"q": q, "s": s})
    assert axis == pkg._lib.MI_I8_ROW_SCALES
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    yb, yf = pkg.int8_project(xt, qT, sv, want_f32=True, scale_axis=axis)
    assert rel_l2(yf.cpu().numpy(), oi8.project_f32(x, q, s)) < 1e-5
    assert rel_l2(yb.float().cpu().numpy(), oi8.project_bf16(x, q, s)) < 1e-3
    (yb2, yf2), = pkg.int8_project_many(xt, [(qT, sv)], want_f32=True, scale_axis=axis)
    assert torch.equal(yf2, yf)


@pytest.mark.parametrize("B,n_in,n_out", [(1, 6144, 2048), (8, 4096, 1024), (32, 512, 128)])
def test_int8_lm_head_form(pkg, gpu, B, n_in, n_out):
    """The int8 lm_head (engine.py:345-351): (h @ f32(q)) * s[o] with f32 accumulation, then bf16."""
    rng = np.random.default_rng(B * 7 + n_out)
    q = rng.integers(-127, 128, (n_in, n_out), dtype=np.int8)
    s = rng.uniform(0.5e-3, 2e-3, (1, n_out)).astype(np.float32)
    x = round_bf16(rng.standard_normal((B, n_in)).astype(np.float32))
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    yb, yf = pkg.resident.int8_logits(xt, {"q": q, "s": s}, want_f32=True)
    want = oi8.project_after_f32(x, q, s)
    assert rel_l2(yf.cpu().numpy(), want) < 1e-5
    assert rel_l2(yb.float().cpu().numpy(), round_bf16(want)) < 1e-3


def _leaf(rng, n_in, n_out, axis):
    """A reference int8 leaf {"q": [in, out], "s": [1, out] (axis 1) or [in, 1] (axis 0)} of N(0, 0.05) weights."""
    q, s = oi8.quantize_array(rng.standard_normal((n_in, n_out)).astype(np.float32) * 0.05, axis)
    return {"q": q, "s": s}


@pytest.mark.parametrize("B,D,I,gu_axis,dn_axis,limit", [(1, 512, 256, 1, 1, 7.0), (8, 6144, 2048, 1, 0, 7.0),
                                                         (32, 1024, 512, 0, 0, 1.5), (40, 512, 768, 1, 0, 7.0),
                                                         (5, 2048, 1024, 1, 0, 1.5)])
def test_int8_mlp(pkg, gpu, B, D, I, gu_axis, dn_axis, limit):
    """mlp_partial over int8 leaves (model.py:125-127; the shared expert at D 6144 / I 2048): g, u, h rounded to bf16
    as the reference's bf16 matmuls and SwiGLU give them; 40 tokens run as two calls of <= 32.  Bar: the f32 output
    within rel-L2 1e-4 of oracle.int8.mlp_partial_f32 (a g, u or h element next to a bf16 rounding boundary may round
    the other way under f32 accumulation), the bf16 output that f32 output rounded once."""
    rng = np.random.default_rng(B * 7 + I)
    p = {"gate": _leaf(rng, D, I, gu_axis), "up": _leaf(rng, D, I, gu_axis), "down": _leaf(rng, I, D, dn_axis)}
    x = round_bf16(rng.standard_normal((B, D)).astype(np.float32) * 2)
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    yb, yf = pkg.int8_mlp(xt, p["gate"], p["up"], p["down"], limit, want_f32=True)
    want = oi8.mlp_partial_f32(x, (p["gate"]["q"], p["gate"]["s"]), (p["up"]["q"], p["up"]["s"]),
                               (p["down"]["q"], p["down"]["s"]), limit)
    assert rel_l2(yf.cpu().numpy(), want) < 1e-4
    assert np.array_equal(yb.float().cpu().numpy(), round_bf16(yf.cpu().numpy()))
    assert torch.equal(pkg.mlp_partial(p, xt, limit), yb)


@pytest.mark.parametrize("fuse", [0, 1, 2])
def test_int8_separate_sum_kernels_match(pkg, gpu, fuse):
    """The I8_FUSE override moves the split sums (1: projections, 2: the MLP's gate/up pair) back to the separate
    reduction and SwiGLU kernels: the same sums in the same split order, so bit-identical results."""
    rng = np.random.default_rng(53)
    B, D, I = 8, 2048, 1024
    x = round_bf16(rng.standard_normal((B, D)).astype(np.float32))
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    leaves = [pkg.formats.int8_pack(*oi8.generate(rng, a, b)) for a, b in ((D, I), (D, I), (I, D))]
    leaves = [(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), c) for a, b, c in leaves]
    proj = [(leaves[0][0], leaves[0][1]), (leaves[1][0], leaves[1][1])]
    want_p = pkg.int8_project_many(xt, proj, want_f32=True)
    want_m = pkg.int8_mlp(xt, *leaves, 7.0, want_f32=True)
    with pkg.tuning(I8_FUSE=fuse):
        got_p = pkg.int8_project_many(xt, proj, want_f32=True)
        got_m = pkg.int8_mlp(xt, *leaves, 7.0, want_f32=True)
    for (a, b), (c, d) in zip(want_p, got_p):
        assert torch.equal(a, c) and torch.equal(b, d)
    assert torch.equal(want_m[0], got_m[0]) and torch.equal(want_m[1], got_m[1])
