"""GPU parity of the bf16-weight projection and mlp_partial (model.py:125-127 over the reference's non-int8 leaves,
W bf16 [in, out]; the shared expert and dense MLPs with int8_nonexpert off, engine.py:281) against the oracle:
exact bf16 products, f32 accumulation; g, u, h rounded to bf16 as the reference's bf16 matmuls and SwiGLU give them."""
import numpy as np
import pytest
import torch

from oracle import int8 as oi8
from oracle.bf16 import rel_l2, round_bf16

pytestmark = pytest.mark.gpu


def _w(rng, n_in, n_out, scale=0.05):
    """A reference bf16 leaf W [in, out]: (bf16 values as f32 numpy, the torch.bfloat16 tensor on the GPU)."""
    W = round_bf16(rng.standard_normal((n_in, n_out)).astype(np.float32) * scale)
    return W, torch.from_numpy(W).cuda().to(torch.bfloat16)


@pytest.mark.parametrize("B,n_in,n_out", [(1, 6144, 2048), (8, 2048, 6144), (32, 512, 128), (40, 1024, 256),
                                          (5, 256, 16), (16, 6144, 6144)])
def test_bf16_project(pkg, gpu, B, n_in, n_out):
    """y = x @ W: the f32 output within rel-L2 1e-5 of the f64 product (f32 accumulation), the bf16 output that
    f32 output rounded once; a Bf16Leaf prepared once gives the same bits as the reference leaf."""
    rng = np.random.default_rng(B * 131 + n_out)
    W, Wt = _w(rng, n_in, n_out)
    x = round_bf16(rng.standard_normal((B, n_in)).astype(np.float32))
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    print("bf16_project B=%d n_in=%d n_out=%d" % (B, n_in, n_out), flush=True)
    yb, yf = pkg.bf16_project(xt, Wt, want_f32=True)
    assert rel_l2(yf.cpu().numpy(), oi8.project_w_f32(x, W)) < 1e-5
    assert np.array_equal(yb.float().cpu().numpy(), round_bf16(yf.cpu().numpy()))
    assert torch.equal(pkg.bf16_project(xt, pkg.bf16_leaf(Wt)), yb)


@pytest.mark.parametrize("B,D,I,limit", [(1, 512, 256, 7.0), (1, 6144, 2048, 7.0), (8, 6144, 2048, 7.0),
                                         (32, 1024, 512, 1.5), (40, 512, 768, 7.0), (5, 2048, 1024, 1.5)])
def test_bf16_mlp(pkg, gpu, B, D, I, limit):
    """mlp_partial over bf16 leaves (the shared expert at D 6144 / I 2048); 40 tokens run as two calls of <= 32.
    Bar: the f32 output within rel-L2 1e-4 of oracle.int8.mlp_partial_f32 on the same leaves (a g, u or h element
    next to a bf16 rounding boundary may round the other way under f32 accumulation), the bf16 output that f32
    output rounded once, and mlp_partial with the reference's leaves giving the same bits."""
    rng = np.random.default_rng(B * 7 + I + 1)
    (Wg, g), (Wu, u), (Wd, d) = _w(rng, D, I), _w(rng, D, I), _w(rng, I, D)
    x = round_bf16(rng.standard_normal((B, D)).astype(np.float32) * 2)
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    print("bf16_mlp B=%d D=%d I=%d limit=%g" % (B, D, I, limit), flush=True)
    yb, yf = pkg.bf16_mlp(xt, g, u, d, limit, want_f32=True)
    want = oi8.mlp_partial_f32(x, Wg, Wu, Wd, limit)
    assert rel_l2(yf.cpu().numpy(), want) < 1e-4
    assert np.array_equal(yb.float().cpu().numpy(), round_bf16(yf.cpu().numpy()))
    assert torch.equal(pkg.mlp_partial({"gate": g, "up": u, "down": d}, xt, limit), yb)
    leaves = [pkg.bf16_leaf(t) for t in (g, u, d)]
    assert torch.equal(pkg.mlp_partial(dict(zip(("gate", "up", "down"), leaves)), xt, limit), yb)


def test_bf16_mlp_of_dequantized_int8_matches_int8_mlp(pkg, gpu):
    """With W = bf16(f32(q) * s) the bf16 MLP and the int8 MLP contract the same bf16 weights (in other split and
    k-step groupings, so to f32 rounding and the odd g, u or h element rounding the other way)."""
    rng = np.random.default_rng(71)
    B, D, I = 8, 2048, 1024
    leaves = [oi8.quantize_array(rng.standard_normal(s).astype(np.float32) * 0.05, 1) for s in ((D, I), (D, I), (I, D))]
    x = round_bf16(rng.standard_normal((B, D)).astype(np.float32))
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    ws = [torch.from_numpy(oi8.dequant_bf16(q, s)).cuda().to(torch.bfloat16) for q, s in leaves]
    a = pkg.bf16_mlp(xt, *ws, 7.0, want_f32=True)
    b = pkg.int8_mlp(xt, *[{"q": q, "s": s} for q, s in leaves], 7.0, want_f32=True)
    assert rel_l2(a[1].cpu().numpy(), b[1].cpu().numpy()) < 1e-4
    assert rel_l2(a[1].cpu().numpy(), oi8.mlp_partial_f32(x, *leaves, 7.0)) < 1e-4


@pytest.mark.parametrize("fuse", [0, 1, 2])
def test_bf16_separate_sum_kernels_match(pkg, gpu, fuse):
    """The I8_FUSE override moves the split sums (1: projections, 2: the MLP's gate/up pair) to the separate
    reduction and SwiGLU kernels: the same sums in the same split order, so bit-identical results."""
    rng = np.random.default_rng(59)
    B, D, I = 8, 2048, 1024
    (_, g), (_, u), (_, d) = _w(rng, D, I), _w(rng, D, I), _w(rng, I, D)
    xt = torch.from_numpy(round_bf16(rng.standard_normal((B, D)).astype(np.float32))).cuda().to(torch.bfloat16)
    want_p = pkg.bf16_project(xt, g, want_f32=True)
    want_m = pkg.bf16_mlp(xt, g, u, d, 7.0, want_f32=True)
    with pkg.tuning(I8_FUSE=fuse):
        got_p = pkg.bf16_project(xt, g, want_f32=True)
        got_m = pkg.bf16_mlp(xt, g, u, d, 7.0, want_f32=True)
    assert torch.equal(want_p[0], got_p[0]) and torch.equal(want_p[1], got_p[1])
    assert torch.equal(want_m[0], got_m[0]) and torch.equal(want_m[1], got_m[1])


def test_bf16_host_errors(pkg, gpu):
    xt = torch.zeros((4, 512), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(TypeError):
        pkg.bf16_project(xt, torch.zeros((512, 64), dtype=torch.float32, device="cuda"))     # not bf16
    with pytest.raises(ValueError):
        pkg.bf16_project(xt, torch.zeros((256, 64), dtype=torch.bfloat16, device="cuda"))    # W rows != x columns
    w = torch.zeros((512, 256), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        pkg.bf16_mlp(xt, w, w, w, 7.0)                                                      # down must be [I, D]
    with pytest.raises(ValueError):
        pkg.mlp_partial({"gate": w, "up": w, "down": {"q": 0, "s": 0}}, xt, 7.0)            # mixed leaf kinds
