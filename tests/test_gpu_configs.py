"""Every benchmark configuration run through the HIP path and checked, at its own shapes where a reference can afford
them:

* config 0 -- one CB3 matvec, W 1024 x 2048, one slot, bf16 out with f32 accumulation: against the oracle;
* the committed golden vectors (tests/golden/cb3_mv.npz, iq3s_mv.npz) through mi_matvec, and the reference-signature
  moe_matvec (pm-ordered X, planes.py:96-112) for every reference format;
* configs 1 and 2 -- the MoE decode layer at D 6144, I 2048, 64 routed + 1 shared experts, batch 1 (softmax top-8)
  and 8 / 16 (Zipf), CB3 and IQ3_S tables generated on the GPU: against an f64 reference built from the library's
  exact dequant (mi_dequant, itself bit-exact against the oracle) with torch f64 matmuls on the GPU; batch 16 also
  against the host oracle on the session's full-size three-expert CB3 layer;
* config 4 -- the 512-token prefill chunk, top-8 of 64 (softmax routing, every expert active) + the shared expert:
  against the oracle at D 512 / I 256, through mi_moe_prefill and ResidentFetch.apply; at D 6144 / I 2048 against a
  reference built from mi_dequant with the reference's bf16 rounding points (x, tiles, h, y, the combine weights)
  and torch f32 matmuls; and beyond 8192 slots with the shared expert.
Config 3 (int8 at batch 8, 6144 x 6144 and 6144 x 2048) is in tests/test_gpu_int8.py.

Bars: decode and matvec rel-L2 <= 1e-5 (f32 throughout); prefill and bf16 outputs <= 1e-3 (the north star's bar;
measured ~1e-5: an h or y element next to a bf16 rounding boundary may round the other way under a different f32
summation order).
"""
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cb3 as ocb3, iq3s as oiq3, layout, moe as omoe
from oracle.bf16 import rel_l2, round_bf16
from tests.util import Layer, softmax_topk_routing, zipf_routing

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
D, I, E = 6144, 2048, 64


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(dtype) if dtype is not None else t


# ------------------------------------------------------------------------------------------------ config 0, golden
def test_config0_matvec(pkg, gpu):
    rng = np.random.default_rng(0)
    codes, cb = ocb3.generate(rng, 1024, 2048)
    x = ocb3.bf16_normal(rng, (1, 2048))
    planes = pkg.to_device_planes(pkg.formats.cb3_pack_planes(ocb3.pack_canonical(codes)[None], cb[None], 2048))
    tb = pkg.ExpertTable("CB3", planes, 1024, 2048)
    y = pkg.matvec(tb, _t(np.zeros(1, np.int32)), _t(x, torch.bfloat16))
    want = omoe.matvec_f64(ocb3.dequant(codes, cb), x)
    assert rel_l2(y.cpu().numpy(), want) < 1e-5
    yb = y.to(torch.bfloat16).float().cpu().numpy()                 # bf16 out, one rounding of the f32 sum
    assert rel_l2(yb, round_bf16(want)) < 1e-3
    assert np.mean(yb != round_bf16(want)) < 0.01


def test_golden_vectors_through_matvec(pkg, gpu):
    z = np.load(os.path.join(HERE, "golden", "cb3_mv.npz"))
    K = z["x"].shape[1]
    planes = pkg.to_device_planes(pkg.formats.cb3_pack_planes(z["words"][None], z["cb"][None], K))
    tb = pkg.ExpertTable("CB3", planes, z["words"].shape[0], K)
    for xd in (torch.bfloat16, torch.float32):
        y = pkg.matvec(tb, _t(np.zeros(1, np.int32)), _t(z["x"], xd))
        assert rel_l2(y.cpu().numpy(), z["y"]) < 1e-5
    z = np.load(os.path.join(HERE, "golden", "iq3s_mv.npz"))
    blocks = z["blocks"]
    tb = pkg.ExpertTable("IQ3_S", pkg.to_device_planes(pkg.formats.iq3s_pack_planes(blocks)), blocks.shape[1],
                         blocks.shape[2] * 256)
    y = pkg.matvec(tb, _t(np.zeros(1, np.int32)), _t(z["x"], torch.bfloat16))
    assert rel_l2(y.cpu().numpy(), z["y"]) < 1e-5


@pytest.mark.parametrize("qtype", ["IQ2_S", "IQ3_S", "IQ4_XS", "Q2_K", "Q3_K"])
def test_moe_matvec_reference_signature(pkg, gpu, qtype):
    """moe_matvec(planes, qtype, nblk, idx, X) with X [Nk, W, C] in the reference's planar order."""
    rng = np.random.default_rng(17)
    Ex, R, K, nk = 5, 256, 1024, 7
    L = Layer(rng, qtype, Ex, K, R)                          # gate shape: R rows x K inputs
    planes = {k: v.reshape(1, *v.shape) for k, v in pkg.to_device_planes(L.planes("gate", pkg.formats)).items()}
    idx = rng.integers(0, Ex, nk).astype(np.int32)
    idx[3] = idx[1]
    x = round_bf16(rng.standard_normal((nk, K)).astype(np.float32))
    X = layout.pm_x(qtype, x)
    y = pkg.moe_matvec(planes, qtype, K // 256, _t(idx), _t(X))
    want = np.stack([omoe.matvec_f64(L.deq("gate", int(e)), x[i:i + 1])[0] for i, e in enumerate(idx)])
    assert rel_l2(y.cpu().numpy(), want) < 1e-5


# ------------------------------------------------------------------------------------------------ configs 1, 2
@pytest.fixture(scope="module")
def full_layers(pkg, gpu):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4041)
    shapes = (("gate", (I, D)), ("up", (I, D)), ("down", (D, I)))
    return {"CB3": {n: pkg.random_cb3_table(E + 1, R, K, gen) for n, (R, K) in shapes},
            "IQ3_S": {n: pkg.random_iq3s_table(E + 1, R, K, gen) for n, (R, K) in shapes}}, gen


def _decode_f64(pkg, tbs, x, idx, w, limit, shared):
    """f64 decode composition (resident.py:110-120) from the library's exact dequant, on the GPU."""
    xd = x.double()
    idx_c, w_c = idx.cpu().numpy(), w.cpu().numpy()
    out = torch.zeros((x.shape[0], D), dtype=torch.float64, device="cuda")
    experts = sorted(set(idx_c.reshape(-1).tolist()) | {shared})
    for e in experts:
        Wg, Wu, Wd = (pkg.dequant(tbs[m], e).double() for m in ("gate", "up", "down"))
        if e == shared:
            rows, wts = np.arange(x.shape[0]), np.ones(x.shape[0])
        else:
            rows, cols = np.nonzero(idx_c == e)
            wts = w_c[rows, cols].astype(np.float64)
        xs = xd[torch.from_numpy(rows).cuda()]
        g, u = xs @ Wg.T, xs @ Wu.T
        h = F.silu(g.clamp(max=limit)) * u.clamp(-limit, limit)
        y = h @ Wd.T
        out.index_add_(0, torch.from_numpy(rows).cuda(), y * torch.from_numpy(wts).cuda()[:, None])
    return out


@pytest.mark.parametrize("qtype", ["CB3", "IQ3_S"])
@pytest.mark.parametrize("N", [1, 8, 16])
def test_config1_2_decode_full_shape(pkg, full_layers, qtype, N):
    layers, gen = full_layers
    tbs = layers[qtype]
    rng = np.random.default_rng(100 + N)
    idx, w = (softmax_topk_routing if N == 1 else zipf_routing)(rng, N, E, 8)
    x = torch.randn((N, D), device="cuda", generator=gen).to(torch.bfloat16)
    of, ob = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], x, _t(idx), _t(w), 10.0, shared_expert=E,
                            want_bf16=True)
    want = _decode_f64(pkg, tbs, x.float(), _t(idx), _t(w), 10.0, E)
    assert rel_l2(of.cpu().numpy(), want.cpu().numpy()) < 1e-5
    assert rel_l2(ob.float().cpu().numpy(), round_bf16(want.cpu().numpy())) < 1e-3     # both rounded to bf16


def test_decode_b16_full_shape_vs_oracle(pkg, gpu, full_cb3_layer):
    """16 tokens over the full-size layer's 2 routed experts + the shared one (the persistent launches at batch 16)
    against the host oracle."""
    L, tbs = full_cb3_layer
    rng = np.random.default_rng(16)
    N, k = 16, 2
    idx = np.tile(np.array([[0, 1]], np.int32), (N, 1))
    idx[::3] = idx[::3, ::-1]
    w = rng.random((N, k)).astype(np.float32)
    x = round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    assert pkg.resident.decode_plan(tbs["gate"], tbs["down"], N, k, 2)["sep_P1"] > 0      # persistent launches
    of, _ = pkg.moe_decode(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), 10.0,
                           shared_expert=2)
    want = omoe.decode_apply(L.deq, x, idx, w, 10.0) + omoe.shared_apply(lambda m: L.deq(m, 2), x, 10.0)
    assert rel_l2(of.cpu().numpy(), want) < 1e-5


# ------------------------------------------------------------------------------------------------ config 4
@pytest.mark.parametrize("qtype", ["CB3", "IQ3_S"])
def test_config4_prefill_reduced_shape(pkg, gpu, qtype):
    rng = np.random.default_rng(4)
    Dr, Ir, T, k, limit = 512, 256, 512, 8, 10.0
    L = Layer(rng, qtype, E + 1, Dr, Ir)
    tbs = L.tables(pkg)
    idx, w = softmax_topk_routing(rng, T, E, k)
    assert len(np.unique(idx)) == E
    x = round_bf16(rng.standard_normal((T, Dr)).astype(np.float32))
    of, _ = pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                            shared_expert=E)
    idx_s = np.concatenate([idx, np.full((T, 1), E, np.int32)], 1)
    w_s = np.concatenate([w, np.ones((T, 1), np.float32)], 1)
    want = omoe.prefill_apply(L.deq, x, idx_s, w_s, limit, E + 1)
    assert rel_l2(of.cpu().numpy(), want) < 1e-3
    # the drop-in: routed experts only, the prefill branch (N*k = 4096 > gather_max_rows = 64)
    p = {key: pkg.to_device_planes(L.planes(name, pkg.formats))
         for name, key in (("gate", "gate_q"), ("up", "up_q"), ("down", "down_q"))}
    fetch = pkg.ResidentFetch({0: {"gate_q": qtype, "up_q": qtype, "down_q": qtype}}, Dr, Ir)
    y = fetch.apply(p, _t(x, torch.bfloat16), _t(idx), _t(w), 0, limit)
    assert rel_l2(y.cpu().numpy(), omoe.prefill_apply(L.deq, x, idx, w, limit, E + 1)) < 1e-3


def _prefill_ref_bf16(pkg, tbs, x, idx, w, limit, shared):
    """The ragged prefill's rounding points (resident.py:144-165, pallas_moe.py:341-355,622-755) from the library's
    exact dequant: bf16 x rows and tiles, f32 dots, h = bf16(swiglu), y = bf16(h Wd^T), out = sum bf16(w) y in f32."""
    bf = lambda t: t.to(torch.bfloat16).float()
    idx_c, w_c = idx.cpu().numpy(), w.cpu().numpy()
    T = x.shape[0]
    out = torch.zeros((T, D), dtype=torch.float32, device="cuda")
    xf = bf(x.float())
    for e in sorted(set(idx_c.reshape(-1).tolist()) | {shared}):
        Wg, Wu, Wd = (bf(pkg.dequant(tbs[m], e)) for m in ("gate", "up", "down"))
        if e == shared:
            rows, wts = np.arange(T), np.ones(T, np.float32)
        else:
            rows, cols = np.nonzero(idx_c == e)
            wts = w_c[rows, cols]
        r = torch.from_numpy(rows).cuda()
        xs = xf[r]
        g, u = xs @ Wg.T, xs @ Wu.T
        h = bf(F.silu(g.clamp(max=limit)) * u.clamp(-limit, limit))
        y = bf(h @ Wd.T)
        out.index_add_(0, r, y * bf(torch.from_numpy(wts).cuda())[:, None])
    return out


@pytest.mark.parametrize("qtype", ["CB3", "IQ3_S"])
def test_config4_prefill_full_shape(pkg, full_layers, qtype):
    layers, gen = full_layers
    tbs = layers[qtype]
    rng = np.random.default_rng(512)
    T, k = 512, 8
    idx, w = softmax_topk_routing(rng, T, E, k)
    x = torch.randn((T, D), device="cuda", generator=gen).to(torch.bfloat16)
    of, _ = pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], x, _t(idx), _t(w), 10.0, shared_expert=E)
    want = _prefill_ref_bf16(pkg, tbs, x, _t(idx), _t(w), 10.0, E)
    assert rel_l2(of.cpu().numpy(), want.cpu().numpy()) < 1e-3


def test_prefill_beyond_8192_slots_with_shared(pkg, gpu):
    """1100 tokens x (8 routed + 1 shared) = 9900 slots: the plan kernel's path for more than 8192 slots inside
    mi_moe_prefill."""
    rng = np.random.default_rng(9900)
    En, Dr, Ir, T, k, limit = 16, 256, 256, 1100, 8, 10.0
    L = Layer(rng, "CB3", En + 1, Dr, Ir)
    tbs = L.tables(pkg)
    idx, w = softmax_topk_routing(rng, T, En, k)
    x = round_bf16(rng.standard_normal((T, Dr)).astype(np.float32))
    of, _ = pkg.moe_prefill(tbs["gate"], tbs["up"], tbs["down"], _t(x, torch.bfloat16), _t(idx), _t(w), limit,
                            shared_expert=En, combine="gather")
    idx_s = np.concatenate([idx, np.full((T, 1), En, np.int32)], 1)
    w_s = np.concatenate([w, np.ones((T, 1), np.float32)], 1)
    want = omoe.prefill_apply(L.deq, x, idx_s, w_s, limit, En + 1, combine="gather")
    assert rel_l2(of.cpu().numpy(), want) < 1e-3
