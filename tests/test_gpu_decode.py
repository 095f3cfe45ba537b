"""GPU parity of the fused codebook-dequant kernels against the CPU oracle (CB3, IQ2_S, IQ3_S and IQ4_XS tables).

Bar: dequantized weights bit-exact; matvec / decode outputs within rel-L2 <= 1e-3 of the f64 oracle (the
reference computes f32 end to end in decode, resident.py:114-120; the kernels reach ~1e-6 -- 1e-3 is the
north-star tolerance, tighter bounds are asserted where the arithmetic allows).
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


@pytest.mark.parametrize("qtype,R,K", [("CB3", 256, 1280), ("CB3", 512, 2048), ("CB3", 256, 384),
                                       ("IQ3_S", 256, 512), ("IQ3_S", 512, 2048), ("IQ4_XS", 256, 512),
                                       ("IQ4_XS", 512, 2048), ("IQ2_S", 256, 512), ("IQ2_S", 512, 2048),
                                       ("IQ2_S", 256, 768), ("Q2_K", 256, 512), ("Q2_K", 256, 768),
                                       ("Q3_K", 256, 512), ("Q3_K", 512, 1280)])
def test_dequant_bit_exact(pkg, gpu, qtype, R, K):
    rng = np.random.default_rng(11)
    L = Layer(rng, qtype, 3, K, R)                  # gate is R x K
    tb = L.tables(pkg)["gate"]
    for e in range(3):
        got = pkg.dequant(tb, e).cpu().numpy()
        want = L.deq("gate", e)
        diff = int((got.view(np.uint32) != want.view(np.uint32)).sum())
        assert diff == 0, "expert %d differs in %d weights" % (e, diff)


def test_dequant_real_gguf_iq3s(pkg, gpu):
    """The reference's real IQ3_S sample (blk.3.ffn_down_exps, 4 rows x 2048) tiled to 256 rows."""
    import json
    import os
    from oracle import iq3s as oiq3
    d = os.path.join(os.path.dirname(__file__), "golden", "gguf")
    s = json.load(open(os.path.join(d, "gguf_samples.json")))["IQ3_S"]
    raw = np.fromfile(os.path.join(d, s["file"]), np.uint8).reshape(s["rows"], s["ne0"] // 256, 110)
    blocks = np.tile(raw, (64, 1, 1))[None]                       # [1, 256, 8, 110]
    planes = pkg.to_device_planes(pkg.formats.iq3s_pack_planes(blocks))
    tb = pkg.ExpertTable("IQ3_S", planes, 256, s["ne0"])
    got = pkg.dequant(tb, 0).cpu().numpy()
    want = oiq3.dequant_blocks(blocks[0]).reshape(256, s["ne0"])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_real_gguf_iq4xs(pkg, gpu):
    """The reference's real IQ4_XS sample (blk.11.ffn_down_exps) tiled to 256 rows."""
    import json
    import os
    from oracle import iq4xs as oiq4
    d = os.path.join(os.path.dirname(__file__), "golden", "gguf")
    s = json.load(open(os.path.join(d, "gguf_samples.json")))["IQ4_XS"]
    raw = np.fromfile(os.path.join(d, s["file"]), np.uint8).reshape(s["rows"], s["ne0"] // 256, 136)
    reps = -(-256 // s["rows"])
    blocks = np.tile(raw, (reps, 1, 1))[:256][None]
    planes = pkg.to_device_planes(pkg.formats.iq4xs_pack_planes(blocks))
    tb = pkg.ExpertTable("IQ4_XS", planes, 256, s["ne0"])
    got = pkg.dequant(tb, 0).cpu().numpy()
    want = oiq4.dequant_blocks(blocks[0]).reshape(256, s["ne0"])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_real_gguf_iq2s(pkg, gpu):
    """The reference's real IQ2_S sample (blk.3.ffn_gate_exps, 2 rows x 4096) tiled to 256 rows."""
    import json
    import os
    from oracle import iq2s as oiq2
    d = os.path.join(os.path.dirname(__file__), "golden", "gguf")
    s = json.load(open(os.path.join(d, "gguf_samples.json")))["IQ2_S"]
    raw = np.fromfile(os.path.join(d, s["file"]), np.uint8).reshape(s["rows"], s["ne0"] // 256, 82)
    blocks = np.tile(raw, (256 // s["rows"], 1, 1))[None]
    planes = pkg.to_device_planes(pkg.formats.iq2s_pack_planes(blocks))
    tb = pkg.ExpertTable("IQ2_S", planes, 256, s["ne0"])
    got = pkg.dequant(tb, 0).cpu().numpy()
    want = oiq2.dequant_blocks(blocks[0]).reshape(256, s["ne0"])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qtype", ["CB3", "IQ2_S", "IQ3_S", "IQ4_XS", "Q2_K", "Q3_K"])
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_matvec_grouped(pkg, gpu, qtype, xdt):
    """moe_matvec semantics (pallas_moe.py:238-307): per-slot outputs, duplicate experts, an out-of-range id."""
    rng = np.random.default_rng(5)
    E, R, K = 6, 512, 1024
    L = Layer(rng, qtype, E, K, R)
    tb = L.tables(pkg)["gate"]
    idx = np.array([3, 1, 3, 0, 5, 3, 3, 2, 1, 3, 4, 3, 3, 3, 0, 3, 3, 3, 3, 3], np.int32)   # expert 3: 13 slots
    n = len(idx)
    X = rng.standard_normal((n, K)).astype(np.float32)
    if xdt == "bf16":
        X = round_bf16(X)
    Xt = _t(X, torch.bfloat16 if xdt == "bf16" else torch.float32)
    got = pkg.matvec(tb, _t(idx), Xt).cpu().numpy()
    want = np.stack([L.deq("gate", int(e)).astype(np.float64) @ X[i].astype(np.float64) for i, e in enumerate(idx)])
    assert rel_l2(got, want) < 1e-5


@pytest.mark.parametrize("qtype", ["CB3", "IQ2_S", "IQ3_S", "IQ4_XS", "Q2_K", "Q3_K"])
@pytest.mark.parametrize("N,k,E,routing", [(1, 8, 16, "softmax"), (4, 4, 12, "zipf"), (8, 8, 20, "zipf"),
                                           (16, 8, 24, "zipf"), (3, 2, 2, "zipf")])
def test_decode_small(pkg, gpu, qtype, N, k, E, routing):
    rng = np.random.default_rng(100 + N * 7 + E)
    D, I, limit = 512, 256, 10.0
    L = Layer(rng, qtype, E + 1, D, I)                 # expert E is the shared expert
    tbs = L.tables(pkg)
    if routing == "softmax":
        idx, w = softmax_topk_routing(rng, N, E, k)
    else:
        idx, w = zipf_routing(rng, N, E, k)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    xt, it, wt = _t(x, torch.bfloat16), _t(idx), _t(w)
    routed = omoe.decode_apply(L.deq, x, idx, w, limit)
    shared = omoe.shared_apply(lambda m: L.deq(m, E), x, limit)
    of, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], xt, it, wt, limit)
    assert rel_l2(of.cpu().numpy(), routed) < 1e-5
    of2, ob2 = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], xt, it, wt, limit, shared_expert=E,
                              want_bf16=True)
    want = routed + shared
    assert rel_l2(of2.cpu().numpy(), want) < 1e-5
    assert rel_l2(ob2.float().cpu().numpy(), round_bf16(want)) < TOL
    # deterministic: a second call is bit-identical
    of3, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], xt, it, wt, limit, shared_expert=E)
    assert torch.equal(of2, of3)


@pytest.mark.parametrize("N,scale,f32x", [(1, 1e6, False), (3, 3e4, False), (8, 1e9, False), (2, 1e6, True)])
def test_iq2s_large_activations(pkg, gpu, N, scale, f32x):
    """IQ2_S decodes on f16 matrix-core operands, each staged activation row at its own power of two: half of every
    row is large, the rest N(0, 1), so the row's maximum sets its scale and the small values still count.  The
    SwiGLU limit is large enough that h stays unclamped and large too."""
    rng = np.random.default_rng(17 + N)
    E, D, I, k = 6, 512, 256, 3
    L = Layer(rng, "IQ2_S", E, D, I)
    tbs = L.tables(pkg)
    idx, w = zipf_routing(rng, N, E, k)
    x = rng.standard_normal((N, D)).astype(np.float32)
    x[:, ::2] *= scale
    if not f32x:
        x = round_bf16(x)
    limit = 1e30
    want = omoe.decode_apply(L.deq, x, idx, w, limit)
    xt = _t(x) if f32x else _t(x, torch.bfloat16)
    of, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], xt, _t(idx), _t(w), limit)
    assert np.isfinite(of.cpu().numpy()).all()
    assert rel_l2(of.cpu().numpy(), want) < (5e-5 if f32x else 1e-5)


# f32 activations (and h) enter the matrix cores as a bf16 high part + remainder, 16 mantissa bits: 5e-5 there
def _tol(f32x):
    return 5e-5 if f32x else 1e-5


@pytest.mark.parametrize("f32x", [False, True])
@pytest.mark.parametrize("N", [1, 8])
@pytest.mark.parametrize("scale", [1e9, 1e-3, 1e-5, 1e-6, 1e-9, 1e-15])
def test_iq2s_decode_activation_scale(pkg, gpu, scale, N, f32x):
    """The reference decodes IQ2_S in f32 (pallas_moe.py:103-124, resident.py:114), so its result scales with the
    activations: every token's output stays within the bound of the f64 oracle whatever their scale, through the
    IQ2_S gate/up, h at the matching scale through the IQ2_S down, and the shared expert."""
    rng = np.random.default_rng(29 + N)
    E, D, I, k, limit = 6, 512, 256, 3, 1e30
    L = Layer(rng, "IQ2_S", E + 1, D, I)
    tbs = L.tables(pkg)
    idx, w = zipf_routing(rng, N, E, k)
    x = (rng.standard_normal((N, D)) * scale).astype(np.float32)
    if not f32x:
        x = round_bf16(x)
    want = omoe.decode_apply(L.deq, x, idx, w, limit) + omoe.shared_apply(lambda m: L.deq(m, E), x, limit)
    xt = _t(x) if f32x else _t(x, torch.bfloat16)
    of, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], xt, _t(idx), _t(w), limit, shared_expert=E)
    got = of.cpu().numpy()
    for n in range(N):
        assert rel_l2(got[n], want[n]) < _tol(f32x), "token %d" % n


@pytest.mark.parametrize("f32x", [False, True])
def test_iq2s_decode_mixed_token_scales(pkg, gpu, f32x):
    """Eight tokens of very different scales, routed so that they share expert groups (one workgroup stages them
    together): each staged row keeps its own scale, so a tiny token beside an O(1) one is as exact as alone."""
    rng = np.random.default_rng(41)
    E, D, I, k, limit = 4, 512, 256, 3, 1e30
    L = Layer(rng, "IQ2_S", E + 1, D, I)
    tbs = L.tables(pkg)
    scales = np.array([1.0, 1e-6, 1e-3, 1e4, 1e-9, 1.0, 1e-5, 1e2])
    N = len(scales)
    idx, w = zipf_routing(rng, N, E, k)
    x = (rng.standard_normal((N, D)) * scales[:, None]).astype(np.float32)
    if not f32x:
        x = round_bf16(x)
    want = omoe.decode_apply(L.deq, x, idx, w, limit) + omoe.shared_apply(lambda m: L.deq(m, E), x, limit)
    xt = _t(x) if f32x else _t(x, torch.bfloat16)
    of, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], xt, _t(idx), _t(w), limit, shared_expert=E)
    got = of.cpu().numpy()
    for n in range(N):
        assert rel_l2(got[n], want[n]) < _tol(f32x), "token %d (scale %g)" % (n, scales[n])


@pytest.mark.parametrize("f32x", [False, True])
def test_iq2s_matvec_row_scales(pkg, gpu, f32x):
    """moe_matvec with slots of scales 1e-30 .. 1e30, most of them on one expert (one group, one staging): every
    slot's output within the bound of the f64 product."""
    rng = np.random.default_rng(43)
    E, R, K = 3, 256, 1024
    L = Layer(rng, "IQ2_S", E, K, R)
    tb = L.tables(pkg)["gate"]
    scales = np.array([1.0, 1e-30, 1e-9, 1e6, 1e-5, 1e30, 1e-3, 1e-12, 3e-20, 1.0, 1e-6, 1e15])
    idx = np.array([0, 0, 0, 0, 0, 0, 0, 0, 1, 2, 1, 0], np.int32)
    X = (rng.standard_normal((len(idx), K)) * scales[:, None]).astype(np.float32)
    if not f32x:
        X = round_bf16(X)
    got = pkg.matvec(tb, _t(idx), _t(X) if f32x else _t(X, torch.bfloat16)).cpu().numpy()
    for i, e in enumerate(idx):
        want = L.deq("gate", int(e)).astype(np.float64) @ X[i].astype(np.float64)
        assert rel_l2(got[i], want) < _tol(f32x), "slot %d (scale %g)" % (i, scales[i])


def test_decode_limit_clamps(pkg, gpu):
    """A small swiglu limit makes the clamps of model.py:119-122 active."""
    rng = np.random.default_rng(3)
    E, D, I, N, k, limit = 6, 512, 256, 2, 3, 0.05
    L = Layer(rng, "CB3", E, D, I)
    tbs = L.tables(pkg)
    idx, w = zipf_routing(rng, N, E, k)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    of, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit)
    assert rel_l2(of.cpu().numpy(), omoe.decode_apply(L.deq, x, idx, w, limit)) < 1e-5


def test_resident_fetch_apply(pkg, gpu):
    """The drop-in operator: reference-shaped planes ([1, E*rows_p, R] u32) and the reference's apply signature."""
    rng = np.random.default_rng(21)
    E, D, I, N, k, limit = 8, 512, 256, 2, 4, 10.0
    L = Layer(rng, "IQ3_S", E, D, I)
    p = {}
    for name, key in (("gate", "gate_q"), ("up", "up_q"), ("down", "down_q")):
        p[key] = {kk: v[None] for kk, v in pkg.to_device_planes(L.planes(name, pkg.formats)).items()}
    fetch = pkg.ResidentFetch({0: {"gate_q": "IQ3_S", "up_q": "IQ3_S", "down_q": "IQ3_S"}}, D, I)
    idx, w = zipf_routing(rng, N, E, k)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    y = fetch.apply(p, _t(x, torch.bfloat16), _t(idx), _t(w), 0, limit)
    assert y.dtype == torch.float32 and tuple(y.shape) == (N, D)
    assert rel_l2(y.cpu().numpy(), omoe.decode_apply(L.deq, x, idx, w, limit)) < 1e-5


@pytest.mark.parametrize("qtype,down_qtype", [("IQ3_S", "IQ4_XS"), ("CB3", "IQ3_S"), ("IQ4_XS", "CB3"),
                                              ("IQ2_S", "IQ4_XS"), ("IQ2_S", "IQ3_S"), ("Q2_K", "Q3_K"),
                                              ("Q3_K", "Q2_K")])
@pytest.mark.parametrize("N", [1, 8, 16])
def test_decode_mixed_formats(pkg, gpu, qtype, down_qtype, N):
    """Gate/up in one format and down in another (the reference's layers mix formats per matrix kind)."""
    rng = np.random.default_rng(300 + N)
    E, D, I, k, limit = 10, 512, 256, 8, 10.0
    L = Layer(rng, qtype, E + 1, D, I, down_qtype=down_qtype)
    tbs = L.tables(pkg)
    idx, w = zipf_routing(rng, N, E, k)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    of, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                           shared_expert=E)
    want = omoe.decode_apply(L.deq, x, idx, w, limit) + omoe.shared_apply(lambda m: L.deq(m, E), x, limit)
    assert rel_l2(of.cpu().numpy(), want) < 1e-5


@pytest.mark.parametrize("qtype", ["CB3", "IQ2_S", "IQ4_XS", "Q3_K"])
def test_down_forms_h_like_the_swiglu_launch(pkg, gpu, qtype):
    """With the FUSE_SWIGLU override the down launch forms h from the gate/up partials while staging instead of a
    SwiGLU launch writing it first.  Same arithmetic: bit-identical outputs."""
    rng = np.random.default_rng(77)
    E, D, I, N, k, limit = 9, 512, 256, 4, 4, 0.5
    L = Layer(rng, qtype, E + 1, D, I)
    tbs = L.tables(pkg)
    idx, w = zipf_routing(rng, N, E, k)
    x = _t(round_bf16(rng.standard_normal((N, D)).astype(np.float32)), torch.bfloat16)
    a, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], x, _t(idx), _t(w), limit, shared_expert=E)
    with pkg.tuning(FUSE_SWIGLU=1):
        b, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], x, _t(idx), _t(w), limit, shared_expert=E)
    assert torch.equal(a, b)
